"""ctypes binding of libglorcq_hip.so (the C ABI declared in include/glorcq_hip.h).

The library is loaded after torch so both share one HIP runtime in the process
(torch ships libamdhip64.so.7 with the same SONAME the library links against).
Loading never touches the GPU, so symbol checks run on hosts without one.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libglorcq_hip.so"

_c_int = ctypes.c_int
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p



class MoeParams(ctypes.Structure):
    """glq_moe_params (include/glorcq_hip.h), field for field."""
    _fields_ = [
        ("tokens", _i64), ("hidden", _i64), ("experts", _i64), ("inter", _i64),
        ("top_k", _i64), ("n_clusters", _i64), ("rank", _i64), ("shared_inter", _i64),
        ("norm_topk_prob", ctypes.c_int32), ("bits", ctypes.c_int32),
        ("shared_bits", ctypes.c_int32), ("group", ctypes.c_int32),
        ("h", _vp), ("router_w", _vp), ("shared_gate_w", _vp),
        ("codes", _vp * 3), ("scales", _vp * 3), ("zeros", _vp * 3),
        ("U", _vp * 3), ("cluster_of", _vp * 3), ("SV", _vp * 3),
        ("shared_codes", _vp * 3), ("shared_scales", _vp * 3), ("shared_zeros", _vp * 3),
        ("out", _vp), ("router_logits", _vp),
        ("u_slot", _vp * 2), ("u_rows", _i64 * 3), ("residual", _vp),
    ]


class MoeShared(ctypes.Structure):
    """glq_moe_shared (include/glorcq_hip.h), field for field."""
    _fields_ = [
        ("codes", _vp * 3), ("scales", _vp * 3), ("zeros", _vp * 3), ("inter", _i64),
        ("bits", ctypes.c_int32), ("reserved", ctypes.c_int32), ("sinter", _vp), ("sy", _vp),
    ]


class TurboMat(ctypes.Structure):
    """glq_turbo_mat (include/glorcq_hip.h), field for field."""
    _fields_ = [
        ("x_rot", _vp), ("codes", _vp), ("norms", _vp), ("centroids", _vp), ("SV", _vp),
        ("parts", _vp), ("cluster", _vp), ("blocks", _i64),
    ]


# name -> (restype, argtypes); must match include/glorcq_hip.h exactly.
SIGNATURES = {
    "glq_version": (_c_int, []),
    "glq_last_error": (ctypes.c_char_p, []),
    "glq_gemv_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "glq_gemv_lora": (_c_int, [
        _vp, _i64, _i64, _i64,          # x, M, K, N
        _vp, _c_int, _vp, _vp,          # codes, bits, scales, zeros
        _i64, _c_int,                   # group, sym
        _vp, _vp, _i64, _vp,            # U, SV, rank, xU
        _vp, _vp,                       # bias, y
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
    "glq_gemv_noalloc_max_scratch_bytes": (_i64, []),
    "glq_gemv_lora_noalloc": (_c_int, [
        _vp, _i64, _i64, _i64,          # x, M, K, N
        _vp, _c_int, _vp, _vp,          # codes, bits, scales, zeros
        _i64, _c_int,                   # group, sym
        _vp, _vp, _i64, _vp,            # U, SV, rank, xU
        _vp, _vp, _vp,                  # bias, y, stream
    ]),
    "glq_gemv_lora_batched": (_c_int, [
        _i64, _vp, _i64,                # items, x, x_stride
        _i64, _i64, _i64,               # M, K, N
        _vp, _i64, _c_int,              # codes, codes_stride, bits
        _vp, _vp, _i64,                 # scales, zeros, sz_stride
        _i64, _c_int,                   # group, sym
        _vp, _i64, _vp, _i64, _i64,     # U, u_stride, SV, sv_stride, rank
        _vp, _i64,                      # xU, xu_stride
        _vp, _i64,                      # bias, bias_stride
        _vp, _i64,                      # y, y_stride
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
    "glq_gemv_lora_clustered": (_c_int, [
        _i64, _vp, _i64,                # items, x, x_stride
        _i64, _i64, _i64,               # M, K, N
        _vp, _i64, _c_int,              # codes, codes_stride, bits
        _vp, _vp, _i64,                 # scales, zeros, sz_stride
        _i64, _c_int,                   # group, sym
        _vp, _i64, _vp, _i64,           # U, u_stride, u_index, n_u
        _vp, _i64,                      # xU (per U), xu_stride
        _vp, _i64, _i64,                # SV, sv_stride, rank
        _vp, _i64,                      # bias, bias_stride
        _vp, _i64,                      # y, y_stride
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
    "glq_gemv_lora_parts": (_c_int, [
        _i64, _vp, _i64,                # items, x, x_stride
        _i64, _i64, _i64,               # M, K, N
        _vp, _i64, _c_int,              # codes, codes_stride, bits
        _vp, _vp, _i64,                 # scales, zeros, sz_stride
        _i64, _c_int,                   # group, sym
        _vp, _i64, _i64,                # SV, sv_stride, rank
        _vp, _i64, _vp, _i64,           # parts, P, u_index, n_u
        _vp, _i64,                      # bias, bias_stride
        _vp, _i64, _vp,                 # y, y_stride, stream
    ]),
    "glq_lowrank_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "glq_lowrank_xu_batched": (_c_int, [
        _i64, _vp, _i64, _i64, _i64,    # items, x, x_stride, M, K
        _vp, _i64, _i64,                # U, u_stride, rank
        _vp, _i64,                      # xu, xu_stride
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
    "glq_lowrank_xu_routed": (_c_int, [
        _i64, _vp, _i64, _vp, _i64, _i64,  # picks, x, K, U, u_rows, rank
        _vp, _i64, _vp, _vp,               # sel, experts, cluster_of, xu
        _vp, _i64, _vp,                    # workspace, bytes, stream
    ]),
    "glq_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "glq_gemm_lora": (_c_int, [
        _vp, _i64, _i64, _i64,          # x, M, K, N
        _vp, _c_int, _vp, _vp,          # codes, bits, scales, zeros
        _i64, _c_int,                   # group, sym
        _vp, _vp, _i64, _vp,            # U, SV, rank, xU
        _vp, _vp,                       # bias, y
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
    "glq_turbo_gemv_batched": (_c_int, [
        _i64, _vp, _i64, _i64, _i64, _i64,  # items, x_rot, x_stride, M, K, N
        _vp, _i64, _vp, _i64,               # codes, codes_stride, norms, norms_stride
        _vp,                                # centroids
        _vp, _i64, _vp, _i64, _i64,         # xU, xu_stride, SV, sv_stride, rank
        _vp, _i64,                          # bias, bias_stride
        _vp, _i64, _vp,                     # y, y_stride, stream
    ]),
    "glq_rht": (_c_int, [_vp, _c_int, _i64, _i64, _vp, _c_int, _vp, _c_int, _vp]),
    "glq_dequant_factor": (_c_int, [_vp, _c_int, _i64, _i64, _vp, _c_int, _c_int, _vp, _vp]),
    "glq_moe_workspace_bytes": (_i64, [ctypes.POINTER(MoeParams)]),
    "glq_moe_decode": (_c_int, [ctypes.POINTER(MoeParams), _vp, _i64, _vp]),
    "glq_moe_prefill_workspace_bytes": (_i64, [ctypes.POINTER(MoeParams)]),
    "glq_moe_prefill": (_c_int, [ctypes.POINTER(MoeParams), _vp, _i64, _vp]),
    "glq_moe_route_workspace_bytes": (_i64, [_i64, _i64]),
    "glq_moe_route": (_c_int, [
        _vp, _vp, _vp,                  # h, router_w, shared_gate_w
        _i64, _i64, _i64, _i64, _c_int,  # tokens, hidden, experts, top_k, norm
        _vp, _vp, _vp, _vp,             # sel, weights, shared_gate, logits
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
    "glq_turbo_moe_prep": (_c_int, [
        _vp, _vp, _vp, _i64, _i64, _i64, _i64,  # h, router_w, shared_gate_w, tokens, hidden, E, k
        _c_int, _vp, _vp, _vp, _vp,             # norm, sel, weights, shared_gate, logits
        _vp, _i64, _vp, _vp,                    # workspace, bytes, rht_signs, x_rot
        _vp, _i64, _i64, _vp, _vp, _vp,         # U, n_u, rank, parts, shared, stream
    ]),
    "glq_turbo_moe_down_prep": (_c_int, [
        _i64, _i64, _vp, _vp, _vp, _vp,         # picks, inter_dim, inter, Pi, rht_signs, xd
        _vp, _i64, _vp, _vp, _i64, _i64,        # U, n_clusters, cluster, sel, experts, rank
        _vp, _i64, _i64, _vp, _vp,              # parts, tokens, hidden, shared, stream
    ]),
    "glq_turbo_moe_gemv2": (_c_int, [
        _i64, _i64, _i64, _i64, _i64, _vp,      # picks, x_div, K, N, experts, sel
        _vp, _vp, _i64, _i64, _vp, _vp,         # m, up, rank, P, y, stream
    ]),
    "glq_turbo_moe_gemv": (_c_int, [
        _i64, _i64, _vp, _i64, _i64, _i64,  # picks, x_div, x_rot, K, N, experts
        _vp, _vp, _vp, _vp,                 # sel, codes, norms, centroids
        _vp, _vp, _i64, _i64,               # xU, xu_cluster, xu_tokens, xu_rows
        _vp, _i64, _vp, _vp,                # SV, rank, bias, gate
        _vp, _vp,                           # y, stream
    ]),
    "glq_moe_combine": (_c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "glq_swiglu": (_c_int, [_vp, _vp, _i64, _vp, _vp]),
    "glq_unpack_codes": (_c_int, [_vp, _i64, _i64, _c_int, _c_int, _vp, _vp]),
    "glq_dequant_weight": (_c_int, [_vp, _i64, _i64, _c_int, _vp, _vp, _i64, _c_int, _vp, _vp]),
    "glq_pack_codes": (_c_int, [_vp, _i64, _i64, _c_int, _vp, _vp]),
    "glq_rmsnorm": (_c_int, [_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp, _vp, _vp]),
    "glq_rmsnorm_xu": (_c_int, [
        _vp, _vp, _vp, _i64, _i64,      # x, residual, weight, rows, dim
        ctypes.c_float, _vp, _vp,       # eps, out, residual_out
        _vp, _i64, _i64, _i64, _vp,     # U, u_stride, n_u, rank, parts
        _vp,                            # stream
    ]),
    "glq_qk_norm_rope": (_c_int, [
        _vp, _vp, _vp, _i64,            # q, k, v, tokens
        _i64, _i64, _i64,               # q_heads, kv_heads, head_dim
        _i64, _i64, _i64,               # q_stride, q_item_rows, kv_stride
        _vp, _vp, ctypes.c_float,       # q_norm_w, k_norm_w, eps
        _vp, _vp, _i64,                 # cos, sin, cs_stride
        _vp, _vp, _vp, _i64,            # q_out, k_cache, v_cache, max_len
        _vp, _vp, _vp,                  # pos, len_out, stream
    ]),
    "glq_decode_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "glq_decode_attention": (_c_int, [
        _vp, _vp, _vp, _i64,            # q, k_cache, v_cache, tokens
        _i64, _i64, _i64, _i64,         # q_heads, kv_heads, head_dim, max_len
        _vp, ctypes.c_float, _vp,       # len, scale, advance
        _vp, _vp, _i64, _vp,            # out, workspace, bytes, stream
    ]),
    "glq_decode_attention_xu": (_c_int, [
        _vp, _vp, _vp, _i64,            # q, k_cache, v_cache, tokens
        _i64, _i64, _i64, _i64,         # q_heads, kv_heads, head_dim, max_len
        _vp, ctypes.c_float, _vp,       # len, scale, advance
        _vp, _vp, _i64, _vp,            # out, U, rank, parts
        _vp, _i64, _vp,                 # workspace, bytes, stream
    ]),
}

_lib = None
_load_error: str | None = None


def load(path: str | os.PathLike | None = None):
    """Returns the loaded library (cached); raises RuntimeError if missing."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        _load_error = f"{p} not built (run `python -m glorcq_amd.build`)"
        raise RuntimeError(_load_error)
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


def check(rc: int, what: str) -> None:
    """Raises RuntimeError with the library's message for a nonzero return."""
    if rc != 0:
        msg = _lib.glq_last_error().decode(errors="replace") if _lib else "?"
        raise RuntimeError(f"{what}: {msg} (code {rc})")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device=None) -> int:
    """hipStream_t of torch's current stream on `device`."""
    if _raw_stream is not None and isinstance(device, torch.device) and device.index is not None:
        return _raw_stream(device.index)  # (the per-call cost of the public form is ~2 us)
    return torch.cuda.current_stream(device).cuda_stream
