"""Operator boundary: Python entry points over the gfx950 HIP library.

Mirrors the reference's `inference.kernels` module (inference/kernels/
__init__.py) so host code keeps its call sites:

  is_gptq_cuda_available()            __init__.py:55
  is_cuda_available()                 __init__.py:39
  turbo_dequant_matmul_fused(...)     __init__.py:184-239  (TurboQuant codec)
  turbo_dequant_grouped_gemv_fused()  __init__.py:242-278
  gptq_dequant_matmul_fused(...)      __init__.py:284-346
  _unpack_indices_2bit(...)           __init__.py:113-118

plus the packed-format entry points this build adds:

  packed_dequant_matmul_fused(...)    fused dequant-GEMV/GEMM + low-rank + bias
  packed_dequant_matmul_batched(...)  many independent problems, one launch
  unpack_codes / dequant_weight / pack_codes_device   bit-exact codec checks
  turbo_gemv(...)                     codebook GEMV/GEMM + low-rank + bias
  rht(...)                            randomized Hadamard transform

Error contract: argument problems raise RuntimeError (the reference's
TORCH_CHECK -> RuntimeError).  Unlike the reference there is no silent
fallback: if the HIP library is missing or a launch fails the call raises, so
a result always comes from the HIP kernels.
"""

from __future__ import annotations

import logging
import weakref

import torch

from .. import _lib
from ..format import pack_codes

logger = logging.getLogger(__name__)

# workspace cache: (device index, stream handle) -> uint8 tensor.  Launches on
# one stream run in order, so one buffer per stream is enough.
_workspaces: dict = {}

# Buffers a larger one has replaced.  A graph captured earlier holds the old
# buffer's address in its kernel arguments, so the memory stays allocated for
# the life of the process (growth doubles, so these add at most the final
# size once more).
_retired_workspaces: list = []


def retire_workspace(ws) -> None:
    """Keeps a replaced workspace buffer alive (see _retired_workspaces)."""
    if ws is not None:
        _retired_workspaces.append(ws)

GEMV_MAX_M = 16


def is_gptq_cuda_available() -> bool:
    """True when the HIP library is built and a GPU is visible."""
    return _lib.available() and torch.cuda.is_available()


def is_cuda_available() -> bool:
    """True when the TurboQuant codebook kernels can run (the HIP library is
    built and a GPU is visible); the reference's flag for its turbo extension
    (inference/kernels/__init__.py:39-41)."""
    return _lib.available() and torch.cuda.is_available()


# The reference's feature flag for the grouped turbo GEMV (inference/kernels/
# __init__.py:63-66); the HIP library always has it.
_HAS_GROUPED_GEMV = True


def _require(t: torch.Tensor, name: str, dtype=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (glorcq_amd runs on the GPU only)")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise RuntimeError(f"{name} must be {dtype} (got {t.dtype})")


SYM_UNSIGNED, SYM_SIGNED, SYM_SIGNED_ZEROS = 0, 1, 2


def _sym_mode(sym) -> int:
    """Code format of the C ABI's `sym` argument: False/0 unsigned codes with
    zero-points, True/1 symmetric two's-complement codes, 2 signed codes with
    zero-points stored offset by 2^(b-1)."""
    m = int(sym)
    if m not in (SYM_UNSIGNED, SYM_SIGNED, SYM_SIGNED_ZEROS):
        raise RuntimeError(f"sym must be False/True or 0, 1, 2 (got {sym!r})")
    return m


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Scratch for the x*U partial sums, one buffer per (device, current stream),
    grown on demand (it needs no initialisation).  A replaced buffer is kept
    alive, since a captured graph may still write into it."""
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, _lib.stream_handle(dev))
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 1 << 16)
        if ws is not None:
            size = max(size, 2 * ws.numel())
        retire_workspace(ws)
        ws = torch.empty(size, dtype=torch.uint8, device=dev)
        _workspaces[key] = ws
    return ws


def _zeroed_buffer(table: dict, device: torch.device, nbytes: int,
                   stream: int | None = None) -> torch.Tensor:
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, _lib.stream_handle(dev) if stream is None else stream)
    ws = table.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 1 << 16)
        if ws is not None:
            size = max(size, 2 * ws.numel())
        retire_workspace(ws)
        ws = torch.zeros(size, dtype=torch.uint8, device=dev)
        table[key] = ws
    return ws


# GEMM and GEMV workspaces: (device index, stream handle) -> zero-filled uint8 tensor
_gemm_workspaces: dict = {}
_gemv_workspaces: dict = {}


def gemm_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Workspace of glq_gemm_lora, one per (device, current stream): its first
    4096 bytes are the x U row blocks' arrival counters, zero between calls,
    so it is allocated zero-filled and serves no other entry point.  A
    replaced buffer is kept alive (a captured graph may still use it)."""
    return _zeroed_buffer(_gemm_workspaces, device, nbytes)


def gemv_workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Workspace of the glq_gemv_lora* entry points, one per (device, current
    stream), zero-filled and for them alone: its first 69632 bytes (the
    token-tile launch's x U arrival counters, the one-row launch's x U job
    counters and K-slice sums) are zero between calls.  `stream`: the
    current stream's handle when the caller has it."""
    return _zeroed_buffer(_gemv_workspaces, device, nbytes, stream)


_gemv_ws_bytes: dict = {}


def _gemv_workspace_bytes(lib, items: int, M: int, K: int, N: int, rank: int) -> int:
    """glq_gemv_workspace_bytes, memoized (a pure function of its sizes)."""
    key = (items, M, K, N, rank)
    n = _gemv_ws_bytes.get(key)
    if n is None:
        n = _gemv_ws_bytes[key] = lib.glq_gemv_workspace_bytes(items, M, K, N, rank)
    return n


def packed_dequant_matmul_fused(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
                                zeros: torch.Tensor | None, bits: int, groupsize: int,
                                sym: bool = False, U: torch.Tensor | None = None,
                                SV: torch.Tensor | None = None,
                                precomputed_xU: torch.Tensor | None = None,
                                bias: torch.Tensor | None = None,
                                out: torch.Tensor | None = None) -> torch.Tensor:
    """y = dequant(codes) x + (x U) SV^T + bias, fp16 (M, N).

    Without `out` this is the operator glorcq_hip::packed_dequant_matmul
    (torch.library, with a fake kernel, so torch.compile traces it without a
    graph break); with `out` (a caller's buffer, e.g. under graph capture) the
    library is called directly.  Arguments as _packed_dequant_matmul_eager."""
    if out is None:
        return torch.ops.glorcq_hip.packed_dequant_matmul(
            x, codes, scales, zeros, bits, groupsize, _sym_mode(sym), U, SV, precomputed_xU, bias)
    return _packed_dequant_matmul_eager(x, codes, scales, zeros, bits, groupsize, sym, U, SV,
                                        precomputed_xU, bias, out)


def _packed_dequant_matmul_eager(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
                                 zeros: torch.Tensor | None, bits: int, groupsize: int,
                                 sym: bool = False, U: torch.Tensor | None = None,
                                 SV: torch.Tensor | None = None,
                                 precomputed_xU: torch.Tensor | None = None,
                                 bias: torch.Tensor | None = None,
                                 out: torch.Tensor | None = None) -> torch.Tensor:
    """y = dequant(codes) x + (x U) SV^T + bias, fp16 (M, N).

    M <= 16: the streaming GEMV (glq_gemv_lora); M > 16 with group 128: the
    MFMA GEMM (glq_gemm_lora); other groups: the GEMV per 16-row block.

    x (M, K) fp16; codes (N, K*bits/32) int32; scales/zeros (N, K/groupsize)
    fp16; U (K, r) fp16; SV (N, r) fp16; precomputed_xU (M, r) fp16 replaces
    x U (the cluster-shared hook of GLoRCQLinear.forward,
    inference/quantized_linear.py:286-345); bias (N,) fp16.
    """
    lib = _lib.load()
    _require(x, "x", torch.float16)
    _require(codes, "codes", torch.int32)
    _require(scales, "scales", torch.float16)
    asym = _sym_mode(sym) != SYM_SIGNED
    if asym:
        if zeros is None:
            raise RuntimeError("zeros required for asymmetric codes")
        _require(zeros, "zeros", torch.float16)
    if x.dim() != 2:
        raise RuntimeError("x must be 2-D (M, K)")
    M, K = x.shape
    N = codes.shape[0]
    if codes.shape[1] * (32 // bits) != K:
        raise RuntimeError(f"codes shape {tuple(codes.shape)} does not match K={K} at {bits} bits")
    if groupsize <= 0 or K % groupsize:
        raise RuntimeError(f"groupsize {groupsize} must divide K={K}")
    if scales.shape != (N, K // groupsize):
        raise RuntimeError(f"scales shape {tuple(scales.shape)} != ({N}, {K // groupsize})")
    if asym and zeros.shape != scales.shape:
        raise RuntimeError(f"zeros shape {tuple(zeros.shape)} != ({N}, {K // groupsize})")
    rank = 0
    if SV is not None:
        _require(SV, "SV", torch.float16)
        if SV.dim() != 2 or SV.shape[0] != N:
            raise RuntimeError("SV must be (N, r)")
        rank = SV.shape[1]
        if precomputed_xU is not None:
            _require(precomputed_xU, "precomputed_xU", torch.float16)
            if precomputed_xU.shape != (M, rank):
                raise RuntimeError("precomputed_xU must be (M, r)")
        elif U is None:
            raise RuntimeError("LoRA needs U or precomputed_xU")
        else:
            _require(U, "U", torch.float16)
            if U.shape != (K, rank):
                raise RuntimeError("U must be (K, r)")
    if bias is not None:
        _require(bias, "bias", torch.float16)
        if tuple(bias.shape) != (N,):
            raise RuntimeError(f"bias must be ({N},)")
    if out is None:
        out = torch.empty(M, N, dtype=torch.float16, device=x.device)
    else:
        _require(out, "out", torch.float16)
        if out.shape != (M, N):
            raise RuntimeError("out must be (M, N)")
    if M == 0 or N == 0:
        return out
    stream = _lib.stream_handle(x.device)
    if M > GEMV_MAX_M and groupsize == 128:
        # prefill: one MFMA GEMM over all M rows (glq_gemm_lora)
        nbytes = lib.glq_gemm_workspace_bytes(M, K, N, rank if precomputed_xU is None else 0)
        ws = gemm_workspace(x.device, nbytes)
        rc = lib.glq_gemm_lora(
            x.data_ptr(), M, K, N, codes.data_ptr(), bits, scales.data_ptr(), _lib.ptr(zeros),
            groupsize, _sym_mode(sym), _lib.ptr(U if precomputed_xU is None else None),
            _lib.ptr(SV), rank, _lib.ptr(precomputed_xU), _lib.ptr(bias), out.data_ptr(),
            ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "glq_gemm_lora")
        return out
    for m0 in range(0, M, GEMV_MAX_M):
        m1 = min(M, m0 + GEMV_MAX_M)
        mb = m1 - m0
        nbytes = _gemv_workspace_bytes(lib, 1, mb, K, N, rank if precomputed_xU is None else 0)
        ws = gemv_workspace(x.device, nbytes, stream)
        xu = None if precomputed_xU is None else precomputed_xU[m0:m1]
        rc = lib.glq_gemv_lora(
            x[m0:m1].data_ptr(), mb, K, N, codes.data_ptr(), bits, scales.data_ptr(),
            _lib.ptr(zeros), groupsize, _sym_mode(sym),
            _lib.ptr(U if precomputed_xU is None else None), _lib.ptr(SV), rank,
            _lib.ptr(xu), _lib.ptr(bias), out[m0:m1].data_ptr(),
            ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "glq_gemv_lora")
    return out


def packed_dequant_matmul_batched(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
                                  zeros: torch.Tensor | None, bits: int, groupsize: int,
                                  sym: bool = False, U: torch.Tensor | None = None,
                                  SV: torch.Tensor | None = None,
                                  bias: torch.Tensor | None = None,
                                  out: torch.Tensor | None = None,
                                  precomputed_xU: torch.Tensor | None = None,
                                  u_index: torch.Tensor | None = None) -> torch.Tensor:
    """E independent problems in one launch: x (E, M, K), codes (E, N, Kw),
    scales/zeros (E, N, G), U (E, K, r), SV (E, N, r), bias (E, N) -> (E, M, N).
    A 2-D x (M, K) is the one input of every problem (x stride 0).

    u_index (E,) int32 on the device: problem i uses U[u_index[i]] of U
    (C, K, r) (cluster-shared U, glq_gemv_lora_clustered); with u_index a
    precomputed_xU is given per U as well, (C, M, r), problem i reading
    precomputed_xU[u_index[i]].

    The packed-format counterpart of turbo_dequant_grouped_gemv_fused
    (inference/kernels/__init__.py:242-278), with the low-rank term fused.
    """
    _require(x, "x", torch.float16)
    _require(codes, "codes", torch.int32)
    _require(scales, "scales", torch.float16)
    asym = _sym_mode(sym) != SYM_SIGNED
    if asym:
        if zeros is None:
            raise RuntimeError("zeros required for codes with zero-points")
        _require(zeros, "zeros", torch.float16)
    if x.dim() == 2:  # one x for every problem
        E, (M, K), x_stride = codes.shape[0], x.shape, 0
    else:
        E, M, K = x.shape
        x_stride = M * K
    if codes.dim() != 3:
        raise RuntimeError("codes must be (E, N, K*bits/32)")
    N = codes.shape[1]
    if codes.shape[0] != E or codes.shape[2] * (32 // bits) != K:
        raise RuntimeError("codes must be (E, N, K*bits/32)")
    if M > GEMV_MAX_M:
        raise RuntimeError(f"batched GEMV takes M <= {GEMV_MAX_M}")
    if groupsize <= 0 or K % groupsize:
        raise RuntimeError(f"groupsize {groupsize} must divide K={K}")
    G = K // groupsize
    if tuple(scales.shape) != (E, N, G):
        raise RuntimeError(f"scales must be ({E}, {N}, {G})")
    if asym and tuple(zeros.shape) != (E, N, G):
        raise RuntimeError(f"zeros must be ({E}, {N}, {G})")
    rank = 0
    if SV is not None:
        _require(SV, "SV", torch.float16)
        if SV.dim() != 3 or tuple(SV.shape[:2]) != (E, N):
            raise RuntimeError(f"SV must be ({E}, {N}, r)")
        rank = SV.shape[2]
        if precomputed_xU is not None:
            _require(precomputed_xU, "precomputed_xU", torch.float16)
            if u_index is not None:
                _require(u_index, "u_index", torch.int32)
                if (precomputed_xU.dim() != 3 or precomputed_xU.shape[0] < 1
                        or tuple(precomputed_xU.shape[1:]) != (M, rank)
                        or tuple(u_index.shape) != (E,)):
                    raise RuntimeError(f"u_index must be ({E},) with precomputed_xU (C, {M}, {rank})")
            elif tuple(precomputed_xU.shape) != (E, M, rank):
                raise RuntimeError("precomputed_xU must be (E, M, r)")
        else:
            if U is None:
                raise RuntimeError("LoRA needs U or precomputed_xU")
            _require(U, "U", torch.float16)
            if u_index is not None:
                _require(u_index, "u_index", torch.int32)
                if tuple(u_index.shape) != (E,) or U.dim() != 3 or U.shape[0] < 1 \
                        or tuple(U.shape[1:]) != (K, rank):
                    raise RuntimeError(f"u_index must be ({E},) with U (C, {K}, {rank})")
            elif tuple(U.shape) != (E, K, rank):
                raise RuntimeError(f"U must be ({E}, {K}, {rank})")
    if bias is not None:
        _require(bias, "bias", torch.float16)
        if tuple(bias.shape) != (E, N):
            raise RuntimeError(f"bias must be ({E}, {N})")
    if out is None:
        out = torch.empty(E, M, N, dtype=torch.float16, device=x.device)
    else:
        _require(out, "out", torch.float16)
        if tuple(out.shape) != (E, M, N):
            raise RuntimeError(f"out must be ({E}, {M}, {N})")
    if E == 0 or M == 0 or N == 0:
        return out
    xu = precomputed_xU if SV is not None else None
    lib = _lib.load()
    stream = _lib.stream_handle(x.device)
    nbytes = _gemv_workspace_bytes(lib, E, M, K, N, rank if xu is None else 0)
    ws = gemv_workspace(x.device, nbytes, stream)
    if u_index is not None and SV is not None:
        n_u = U.shape[0] if xu is None else xu.shape[0]
        rc = lib.glq_gemv_lora_clustered(
            E, x.data_ptr(), x_stride, M, K, N, codes.data_ptr(),
            codes.shape[1] * codes.shape[2], bits, scales.data_ptr(), _lib.ptr(zeros),
            scales.shape[1] * scales.shape[2], groupsize, _sym_mode(sym),
            _lib.ptr(U if xu is None else None), K * rank, u_index.data_ptr(), n_u,
            _lib.ptr(xu), M * rank, SV.data_ptr(), N * rank, rank, _lib.ptr(bias), N,
            out.data_ptr(), M * N, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "glq_gemv_lora_clustered")
        return out
    rc = lib.glq_gemv_lora_batched(
        E, x.data_ptr(), x_stride, M, K, N, codes.data_ptr(), codes.shape[1] * codes.shape[2],
        bits, scales.data_ptr(), _lib.ptr(zeros), scales.shape[1] * scales.shape[2],
        groupsize, _sym_mode(sym), _lib.ptr(U if xu is None else None), K * rank, _lib.ptr(SV),
        N * rank, rank, _lib.ptr(xu), M * rank, _lib.ptr(bias), N, out.data_ptr(), M * N,
        ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "glq_gemv_lora_batched")
    return out


def packed_dequant_matmul_parts(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
                                zeros: torch.Tensor | None, bits: int, groupsize: int,
                                SV: torch.Tensor, parts: torch.Tensor,
                                u_index: torch.Tensor | None = None, sym: bool = False,
                                bias: torch.Tensor | None = None,
                                out: torch.Tensor | None = None) -> torch.Tensor:
    """packed_dequant_matmul_batched with a = x U given as fp32 partials
    (glq_gemv_lora_parts): parts (blocks, P, M, rpad), item i taking
    a = fp16(sum over p in order of parts[b][p]) with b = u_index[i], or i
    when u_index is None -- what rmsnorm_xu and decode_attention(U=...)
    write.  x (M, K) is every item's input; codes (E, N, K*bits/32)."""
    _require(x, "x", torch.float16)
    _require(codes, "codes", torch.int32)
    _require(scales, "scales", torch.float16)
    _require(SV, "SV", torch.float16)
    _require(parts, "parts", torch.float32)
    asym = _sym_mode(sym) != SYM_SIGNED
    if asym:
        if zeros is None:
            raise RuntimeError("zeros required for codes with zero-points")
        _require(zeros, "zeros", torch.float16)
    if x.dim() != 2 or codes.dim() != 3:
        raise RuntimeError("x must be (M, K) and codes (E, N, K*bits/32)")
    (M, K), (E, N) = x.shape, codes.shape[:2]
    if codes.shape[2] * (32 // bits) != K:
        raise RuntimeError("codes must be (E, N, K*bits/32)")
    if M > GEMV_MAX_M:
        raise RuntimeError(f"takes M <= {GEMV_MAX_M}")
    if groupsize <= 0 or K % groupsize:
        raise RuntimeError(f"groupsize {groupsize} must divide K={K}")
    G = K // groupsize
    if tuple(scales.shape) != (E, N, G) or (asym and tuple(zeros.shape) != (E, N, G)):
        raise RuntimeError(f"scales/zeros must be ({E}, {N}, {G})")
    if SV.dim() != 3 or tuple(SV.shape[:2]) != (E, N):
        raise RuntimeError(f"SV must be ({E}, {N}, r)")
    rank = SV.shape[2]
    rpad = (rank + 31) // 32 * 32
    if parts.dim() != 4 or tuple(parts.shape[2:]) != (M, rpad):
        raise RuntimeError(f"parts must be (blocks, P, {M}, {rpad})")
    nb = parts.shape[0]
    if u_index is not None:
        _require(u_index, "u_index", torch.int32)
        if tuple(u_index.shape) != (E,):
            raise RuntimeError(f"u_index must be ({E},)")
    elif nb != E:
        raise RuntimeError(f"parts must hold one block per item ({E}) without u_index")
    if bias is not None:
        _require(bias, "bias", torch.float16)
        if tuple(bias.shape) != (E, N):
            raise RuntimeError(f"bias must be ({E}, {N})")
    if out is None:
        out = torch.empty(E, M, N, dtype=torch.float16, device=x.device)
    elif tuple(out.shape) != (E, M, N) or out.dtype != torch.float16 or not out.is_contiguous():
        raise RuntimeError(f"out must be contiguous fp16 ({E}, {M}, {N})")
    if E == 0 or M == 0 or N == 0:
        return out
    lib = _lib.load()
    rc = lib.glq_gemv_lora_parts(
        E, x.data_ptr(), 0, M, K, N, codes.data_ptr(), codes.shape[1] * codes.shape[2], bits,
        scales.data_ptr(), _lib.ptr(zeros), scales.shape[1] * scales.shape[2], groupsize,
        _sym_mode(sym), SV.data_ptr(), N * rank, rank, parts.data_ptr(), parts.shape[1],
        _lib.ptr(u_index), nb, _lib.ptr(bias), N, out.data_ptr(), M * N,
        _lib.stream_handle(x.device))
    _lib.check(rc, "glq_gemv_lora_parts")
    return out


def lowrank_xu(x: torch.Tensor, U: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """a = fp16(x U): the operator glorcq_hip::lowrank_xu without `out`, else
    the library directly (see _lowrank_xu_eager)."""
    if out is None:
        return torch.ops.glorcq_hip.lowrank_xu(x, U)
    return _lowrank_xu_eager(x, U, out)


def _lowrank_xu_eager(x: torch.Tensor, U: torch.Tensor,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """a = fp16(x U) on the GPU (fp32 accumulation): x (M, K) or (E, M, K) fp16,
    U (K, r) or (E, K, r) fp16 -> (M, r) or (E, M, r).  A 2-D x with a 3-D U
    applies the one x to every U (the cluster-shared x*U of the MoE block,
    inference/moe_block.py:290-322)."""
    lib = _lib.load()
    _require(x, "x", torch.float16)
    _require(U, "U", torch.float16)
    batched = U.dim() == 3
    E = U.shape[0] if batched else 1
    K, r = U.shape[-2], U.shape[-1]
    if x.dim() == 3:
        if not batched or x.shape[0] != E:
            raise RuntimeError("x (E, M, K) needs U (E, K, r)")
        M, x_stride = x.shape[1], x.shape[1] * K
    else:
        M, x_stride = x.shape[0], 0
    if x.shape[-1] != K:
        raise RuntimeError(f"x has K={x.shape[-1]}, U has K={K}")
    shape = (E, M, r) if batched else (M, r)
    if out is None:
        out = torch.empty(shape, dtype=torch.float16, device=x.device)
    elif tuple(out.shape) != shape:
        raise RuntimeError(f"out must be {shape}")
    if M == 0 or E == 0:
        return out
    if M > GEMV_MAX_M:
        if batched:
            raise RuntimeError(f"batched x U takes M <= {GEMV_MAX_M}")
        # one x (M, K), one U: 16-row blocks as items sharing U (stride 0)
        full, tail = divmod(M, GEMV_MAX_M)
        nbytes = lib.glq_lowrank_workspace_bytes(max(full, 1), GEMV_MAX_M, K, r)
        ws = workspace(x.device, nbytes)
        stream = _lib.stream_handle(x.device)
        if full:
            _lib.check(lib.glq_lowrank_xu_batched(
                full, x.data_ptr(), GEMV_MAX_M * K, GEMV_MAX_M, K, U.data_ptr(), 0, r,
                out.data_ptr(), GEMV_MAX_M * r, ws.data_ptr(), ws.numel(), stream),
                "glq_lowrank_xu_batched")
        if tail:
            m0 = full * GEMV_MAX_M
            _lib.check(lib.glq_lowrank_xu_batched(
                1, x[m0:].data_ptr(), 0, tail, K, U.data_ptr(), 0, r, out[m0:].data_ptr(), 0,
                ws.data_ptr(), ws.numel(), stream), "glq_lowrank_xu_batched")
        return out
    nbytes = lib.glq_lowrank_workspace_bytes(E, M, K, r)
    ws = workspace(x.device, nbytes)
    _lib.check(lib.glq_lowrank_xu_batched(E, x.data_ptr(), x_stride, M, K, U.data_ptr(), K * r, r,
                                          out.data_ptr(), M * r, ws.data_ptr(), ws.numel(),
                                          _lib.stream_handle(x.device)), "glq_lowrank_xu_batched")
    return out


# Prepared codes of gptq_dequant_matmul_fused: id(qweight_int) -> (weakref to
# it, its key, code format, container bits, packed codes).  An entry lives as
# long as its tensor and is valid while the tensor's storage, shape and
# version counter are unchanged.
_gptq_prepared: dict = {}


def _tensor_version(t: torch.Tensor) -> int:
    try:
        return t._version
    except RuntimeError:  # inference tensors keep no version counter
        return -1


def _gptq_prepare(q: torch.Tensor, sym, groupsize: int, bits: int | None):
    """(code format, container bits, packed codes) of the reference's (N, K)
    integer codes, range-checked and packed once per tensor version.

    The check reads min and max back to the host (a sync), so it runs outside
    graph capture; a repeated call on the same codes reuses the result with
    no sync and no device work, as the reference's op does under capture
    (inference/quantized_linear.py:307-311 inside graph_wrapper.py:69-131)."""
    key = (q.data_ptr(), _tensor_version(q), tuple(q.shape), q.dtype, q.device, bool(sym),
           bits, groupsize)
    ent = _gptq_prepared.get(id(q))
    if ent is not None and ent[0]() is q and ent[1] == key:
        return ent[2], ent[3], ent[4]
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            "gptq_dequant_matmul_fused: these codes were not prepared before graph capture "
            "(their range check reads back to the host); call it once on them outside the "
            "capture, as a warm-up step does")
    lo, hi = (0, 0) if q.numel() == 0 else (int(v) for v in torch.aminmax(q))
    mode = None
    K = q.shape[1]
    # containers whose 16-byte pieces tile the rows and the groups
    fits = [c for c in (2, 4) if K % (128 // c) == 0 and groupsize % (128 // c) == 0] or [4]
    for b in ((bits,) if bits is not None else fits):
        h = 1 << (b - 1)
        if sym:
            if -h <= lo and hi < h:
                mode = SYM_SIGNED
        elif 0 <= lo and hi < 2 * h:
            mode = SYM_UNSIGNED
        elif -h <= lo and hi < h:
            mode = SYM_SIGNED_ZEROS
        if mode is not None:
            break
    if mode is None:
        raise RuntimeError(
            f"{'symmetric' if sym else 'asymmetric'} codes span [{lo}, {hi}], which no "
            f"{bits or 4}-bit container holds (unsigned 0..{(1 << (bits or 4)) - 1} or signed "
            f"{-(1 << ((bits or 4) - 1))}..{(1 << ((bits or 4) - 1)) - 1})")
    qi = q.to(torch.int32)
    if mode == SYM_SIGNED_ZEROS:
        qi = qi + (1 << (b - 1))  # stored offset by 2^(b-1); z is applied as given
    codes = pack_codes_device(qi.contiguous(), b)
    k = id(q)
    ref = weakref.ref(q, lambda _r, k=k: _gptq_prepared.pop(k, None))
    _gptq_prepared[k] = (ref, key, mode, b, codes)
    return mode, b, codes


def gptq_dequant_matmul_fused(x, qweight_int, scales, zeros, groupsize, sym=False,
                              lora_USV=None, bits: int | None = None):
    """Reference signature (inference/kernels/__init__.py:284): unpacked (N, K)
    integer codes, fp16 scales/zeros, optional (U, S, V) low-rank tuple ->
    fp16 (B, N).  W = q s (sym) or (q - z) s, q the codes as given (the
    reference's int8 cast, gptq_matmul.cu:15-16, 81-82).

    The reference casts the (N, K) int32 codes to int8 on every call; here
    the first call on a codes tensor range-checks them (one aminmax, a host
    sync) and packs them on the device into the narrowest container that
    holds them (2 or 4 bits, or the `bits` given): unsigned asymmetric codes
    as they are, signed ones (symmetric, or asymmetric like the reference's
    tests' codes in [-2, 2] with non-integer zero-points) offset by 2^(b-1)
    with the zero-points applied exactly.  Codes that fit no 4-bit form raise.
    Later calls on the same, unmodified tensor reuse the packed codes with no
    sync, so the op can be captured in a CUDA/HIP graph after one warm-up
    call (a call under capture on codes never seen raises).
    """
    if bits is not None and bits not in (2, 4):
        raise RuntimeError(f"{bits}-bit codes are not supported (2 or 4)")
    q = qweight_int
    if q.dim() != 2:
        raise RuntimeError("qweight_int must be (N, K)")
    mode, b, codes = _gptq_prepare(q, sym, groupsize, bits)
    xh = x.to(torch.float16).contiguous()
    U = SV = None
    if lora_USV is not None:
        U_, S_, V_ = lora_USV
        U = U_.to(torch.float16).contiguous()
        SV = (V_.float() * S_.float().unsqueeze(0)).to(torch.float16).contiguous()
    return packed_dequant_matmul_fused(xh, codes, scales.contiguous(),
                                       None if mode == SYM_SIGNED else zeros.contiguous(),
                                       b, groupsize, mode, U=U, SV=SV)


def pack_codes_device(q: torch.Tensor, bits: int) -> torch.Tensor:
    """(N, K) int32 codes on the GPU -> packed (N, K*bits/32) int32 (HIP kernel)."""
    lib = _lib.load()
    _require(q, "q", torch.int32)
    N, K = q.shape
    out = torch.empty(N, K * bits // 32, dtype=torch.int32, device=q.device)
    _lib.check(lib.glq_pack_codes(q.data_ptr(), N, K, bits, out.data_ptr(),
                                  _lib.stream_handle(q.device)), "glq_pack_codes")
    return out


def unpack_codes(codes: torch.Tensor, bits: int, K: int, sym: bool = False) -> torch.Tensor:
    """Packed (N, K*bits/32) int32 -> (N, K) int32 codes (HIP kernel)."""
    lib = _lib.load()
    _require(codes, "codes", torch.int32)
    N = codes.shape[0]
    out = torch.empty(N, K, dtype=torch.int32, device=codes.device)
    _lib.check(lib.glq_unpack_codes(codes.data_ptr(), N, K, bits, _sym_mode(sym), out.data_ptr(),
                                    _lib.stream_handle(codes.device)), "glq_unpack_codes")
    return out


def dequant_weight(codes: torch.Tensor, bits: int, K: int, scales: torch.Tensor,
                   zeros: torch.Tensor | None, groupsize: int, sym: bool = False) -> torch.Tensor:
    """fp16 W (N, K) = fp16(fp16(q - z) * s) (HIP kernel; bit-exact with the
    reference's fp16 dequant loop, inference/quantized_linear.py:271-284)."""
    lib = _lib.load()
    _require(codes, "codes", torch.int32)
    _require(scales, "scales", torch.float16)
    N = codes.shape[0]
    out = torch.empty(N, K, dtype=torch.float16, device=codes.device)
    _lib.check(lib.glq_dequant_weight(codes.data_ptr(), N, K, bits, scales.data_ptr(),
                                      _lib.ptr(zeros), groupsize, _sym_mode(sym), out.data_ptr(),
                                      _lib.stream_handle(codes.device)), "glq_dequant_weight")
    return out


def _turbo_words(packed: torch.Tensor, K: int, lead: tuple) -> torch.Tensor:
    """Indices as int32 words: (..., N, K/4) uint8 (the reference's
    packed_indices) is viewed, not copied; (..., N, K/16) int32 passes."""
    if packed.dtype == torch.uint8:
        if packed.shape[-1] * 4 != K:
            raise RuntimeError(f"packed_indices has {packed.shape[-1]} bytes per row, K={K}")
        _require(packed, "packed_indices")
        if K % 16 or packed.storage_offset() % 4:
            raise RuntimeError("packed_indices rows must hold whole 32-bit words")
        packed = packed.view(torch.int32)
    _require(packed, "packed_indices", torch.int32)
    if packed.shape[-1] * 16 != K or tuple(packed.shape[:-1]) != lead:
        raise RuntimeError(f"packed_indices shape {tuple(packed.shape)} does not match "
                           f"{lead} x K={K}")
    return packed


def turbo_gemv(x_rot: torch.Tensor, packed: torch.Tensor, norms: torch.Tensor,
               centroids: torch.Tensor, xU: torch.Tensor | None = None,
               SV: torch.Tensor | None = None, bias: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """The codebook matmul: the operator glorcq_hip::turbo_dequant_matmul
    without `out`, else the library directly (see _turbo_gemv_eager)."""
    if out is None:
        return torch.ops.glorcq_hip.turbo_dequant_matmul(x_rot, packed, norms, centroids, xU,
                                                         SV, bias)
    return _turbo_gemv_eager(x_rot, packed, norms, centroids, xU, SV, bias, out)


def _turbo_gemv_eager(x_rot: torch.Tensor, packed: torch.Tensor, norms: torch.Tensor,
                      centroids: torch.Tensor, xU: torch.Tensor | None = None,
                      SV: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """y = fp16(norms[n] * sum_k C[q(n,k)] x_rot[m,k] + (xU SV^T)[m,n] + bias[n]).

    Single problem: x_rot (M, K) fp16, packed (N, K/4) uint8 or (N, K/16)
    int32, norms (N,) fp32, centroids (4,) fp32, xU (M, r) fp16 = x U of the
    unrotated x, SV (N, r) fp16, bias (N,) fp16 -> (M, N).
    Batched: x_rot (E, M, K), packed (E, N, ...), norms (E, N), SV (E, N, r),
    xU (E, M, r), bias (E, N) -> (E, M, N), one launch (glq_turbo_gemv_batched).
    """
    lib = _lib.load()
    _require(x_rot, "x_rot", torch.float16)
    _require(norms, "norms", torch.float32)
    _require(centroids, "centroids", torch.float32)
    if centroids.numel() != 4:
        raise RuntimeError("the 2-bit codebook has 4 centroids")
    batched = x_rot.dim() == 3
    if x_rot.dim() not in (2, 3):
        raise RuntimeError("x_rot must be (M, K) or (E, M, K)")
    E = x_rot.shape[0] if batched else 1
    M, K = x_rot.shape[-2], x_rot.shape[-1]
    N = packed.shape[-2]
    lead = (E, N) if batched else (N,)
    words = _turbo_words(packed, K, lead)
    if tuple(norms.shape) != lead:
        raise RuntimeError(f"norms must be {lead}")
    rank = 0
    if SV is not None:
        _require(SV, "SV", torch.float16)
        rank = SV.shape[-1]
        if tuple(SV.shape) != lead + (rank,):
            raise RuntimeError(f"SV must be {lead + (rank,)}")
        if xU is None:
            raise RuntimeError("SV needs xU = x U")
        _require(xU, "xU", torch.float16)
        if tuple(xU.shape) != tuple(x_rot.shape[:-1]) + (rank,):
            raise RuntimeError("xU must be (..., M, r)")
    if bias is not None:
        _require(bias, "bias", torch.float16)
        if tuple(bias.shape) != lead:
            raise RuntimeError(f"bias must be {lead}")
    shape = (E, M, N) if batched else (M, N)
    if out is None:
        out = torch.empty(shape, dtype=torch.float16, device=x_rot.device)
    else:
        _require(out, "out", torch.float16)
        if tuple(out.shape) != shape:
            raise RuntimeError(f"out must be {shape}")
    if M == 0 or N == 0 or E == 0:
        return out
    rc = lib.glq_turbo_gemv_batched(
        E, x_rot.data_ptr(), M * K, M, K, N, words.data_ptr(), N * K // 16, norms.data_ptr(), N,
        centroids.data_ptr(), _lib.ptr(xU), M * rank, _lib.ptr(SV), N * rank, rank,
        _lib.ptr(bias), N, out.data_ptr(), M * N, _lib.stream_handle(x_rot.device))
    _lib.check(rc, "glq_turbo_gemv_batched")
    return out


def rht(x: torch.Tensor, signs: torch.Tensor, inverse: bool = False,
        out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Randomized Hadamard transform: the operator glorcq_hip::rht (see
    _rht_eager)."""
    od = out_dtype or x.dtype
    return torch.ops.glorcq_hip.rht(x, signs, bool(inverse), od == torch.float32)


def _rht_eager(x: torch.Tensor, signs: torch.Tensor, inverse: bool = False,
               out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Randomized Hadamard transform of the rows of x (..., d), d a power of
    two: (1/sqrt(d)) H diag(signs) x, or diag(signs) (1/sqrt(d)) H x when
    inverse.  fp16 or fp32 in and out (out_dtype defaults to x's), fp32
    arithmetic; rht(x16, signs) is the hot path's
    rht_forward(x.float(), signs).half() in one launch."""
    lib = _lib.load()
    if x.dtype not in (torch.float16, torch.float32):
        raise RuntimeError("x must be fp16 or fp32")
    _require(x, "x")
    _require(signs, "signs", torch.float32)
    d = x.shape[-1]
    if signs.numel() != d:
        raise RuntimeError(f"signs has {signs.numel()} entries, rows have {d}")
    od = out_dtype or x.dtype
    if od not in (torch.float16, torch.float32):
        raise RuntimeError("out_dtype must be fp16 or fp32")
    out = torch.empty(x.shape, dtype=od, device=x.device)
    rows = x.numel() // d if d else 0
    if rows == 0:
        return out
    rc = lib.glq_rht(x.data_ptr(), int(x.dtype == torch.float32), rows, d, signs.data_ptr(),
                     int(bool(inverse)), out.data_ptr(), int(od == torch.float32),
                     _lib.stream_handle(x.device))
    _lib.check(rc, "glq_rht")
    return out


def turbo_dequant_matmul_fused(x, packed_indices, norms, Pi, centroids, bits, dim,
                               lora_USV=None, precomputed_x_rot=None):
    """Reference signature (inference/kernels/__init__.py:184-239): x (B, K),
    packed_indices (N, K/4) uint8, norms (N,) fp32, Pi (K, K) rotation (unused
    when precomputed_x_rot is given), centroids (4,) fp32 -> fp16 (B, N).

    x_rot = fp16(x.float() @ Pi.float().T) is a plain library GEMM (torch on
    the GPU); precomputed_x_rot is used as given, rounded to fp16 (the
    reference's kernel takes fp16 x_rot).  lora_USV = (U, S, V) adds
    (x U) diag(S) V^T, fused into the turbo kernel's epilogue with one fp16
    rounding (the reference adds it in Python afterwards).  Only 2-bit codes
    have a kernel, as in the reference; other widths raise.
    """
    if bits != 2:
        raise RuntimeError(f"the TurboQuant kernel takes 2-bit codes (got bits={bits})")
    if precomputed_x_rot is not None:
        x_rot = precomputed_x_rot.to(torch.float16).contiguous()
    else:
        x_rot = (x.float() @ Pi.float().T).half()
    if x_rot.shape[-1] != dim:
        raise RuntimeError(f"x_rot has K={x_rot.shape[-1]}, dim={dim}")
    xU = SV = None
    if lora_USV is not None:
        U_, S_, V_ = lora_USV
        SV = (V_.float() * S_.float().unsqueeze(0)).to(torch.float16).contiguous()
        xU = lowrank_xu(x.to(torch.float16).contiguous(), U_.to(torch.float16).contiguous())
    return turbo_gemv(x_rot.reshape(-1, dim), packed_indices.contiguous(),
                      norms.float().contiguous(), centroids.float().contiguous(), xU=xU, SV=SV)


def turbo_dequant_grouped_gemv_fused(x_grouped, packed_cat, norms_cat, centroids, N_out):
    """Reference signature (inference/kernels/__init__.py:242-278): E experts
    with their own input row.  x_grouped (E, K) fp16, packed_cat (E*N_out, K/4)
    uint8, norms_cat (E*N_out,) fp32, centroids (4,) fp32 -> (E*N_out,) fp16,
    in one launch."""
    E, K = x_grouped.shape
    packed = packed_cat.contiguous()
    if packed.shape[0] != E * N_out:
        raise RuntimeError(f"packed_cat has {packed.shape[0]} rows, E*N_out = {E * N_out}")
    packed = packed.view(E, N_out, packed.shape[1])
    y = turbo_gemv(x_grouped.to(torch.float16).contiguous().view(E, 1, K), packed,
                   norms_cat.float().contiguous().view(E, N_out), centroids.float().contiguous())
    return y.view(E * N_out)


def _unpack_indices_2bit(packed: torch.Tensor, K: int) -> torch.Tensor:
    """Reference helper (inference/kernels/__init__.py:113-118): (N, K/4) uint8 ->
    (N, K) long, LSB-first.  Host-side format utility (not a compute path)."""
    shifts = torch.tensor([0, 2, 4, 6], device=packed.device, dtype=torch.uint8)
    return ((packed.unsqueeze(-1) >> shifts) & 0x3).reshape(packed.shape[0], -1)[:, :K].long()


__all__ = [
    "is_gptq_cuda_available", "is_cuda_available", "packed_dequant_matmul_fused",
    "packed_dequant_matmul_batched", "gptq_dequant_matmul_fused", "unpack_codes",
    "dequant_weight", "pack_codes_device", "pack_codes", "workspace", "lowrank_xu",
    "turbo_gemv", "rht", "turbo_dequant_matmul_fused", "turbo_dequant_grouped_gemv_fused",
]


# ---------------------------------------------------------------------------
# Decoder-layer pieces of the model-level decode step (no reference kernel
# counterpart: they replace transformers' Qwen3-MoE RMSNorm, q/k norm, rotary
# embedding, static-cache update and single-token attention, one launch each)
# ---------------------------------------------------------------------------
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """Qwen3MoeRMSNorm.forward on the GPU: fp16(w * fp16(y * rsqrt(mean(y^2) +
    eps))) over the last dim, y = x or, with `residual`, y = fp16(x + residual).
    Returns out, or (out, y) when a residual is given."""
    lib = _lib.load()
    _require(x, "x", torch.float16)
    _require(weight, "weight", torch.float16)
    D = x.shape[-1]
    if weight.shape != (D,):
        raise RuntimeError(f"weight must be ({D},)")
    rows = x.numel() // D if D else 0
    if out is None:
        out = torch.empty_like(x)
    res_out = None
    if residual is not None:
        _require(residual, "residual", torch.float16)
        if residual.shape != x.shape:
            raise RuntimeError("residual must match x")
        res_out = torch.empty_like(x)
    _lib.check(lib.glq_rmsnorm(x.data_ptr(), _lib.ptr(residual), weight.data_ptr(), rows, D,
                               float(eps), out.data_ptr(), _lib.ptr(res_out),
                               _lib.stream_handle(x.device)), "glq_rmsnorm")
    return out if residual is None else (out, res_out)


def rmsnorm_xu(x: torch.Tensor, weight: torch.Tensor, eps: float, U: torch.Tensor,
               residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
               parts: torch.Tensor | None = None):
    """rmsnorm of x (M <= 16 rows of dim D) and, in the same launch, the fp32
    partials of out U[u] over 256-row slices for U (n_u, D, r):
    parts (n_u, S, M, rpad), S = ceil(D / 256), rpad = r rounded up to 32
    -- the a of packed_dequant_matmul_parts (glq_rmsnorm_xu).  Returns
    (out, parts), or (out, y, parts) when a residual is given (y = fp16(x +
    residual), as rmsnorm)."""
    lib = _lib.load()
    _require(x, "x", torch.float16)
    _require(weight, "weight", torch.float16)
    _require(U, "U", torch.float16)
    D = x.shape[-1]
    if weight.shape != (D,):
        raise RuntimeError(f"weight must be ({D},)")
    if U.dim() == 2:
        U = U.unsqueeze(0)
    if U.dim() != 3 or U.shape[1] != D:
        raise RuntimeError(f"U must be (n_u, {D}, r)")
    n_u, _, r = U.shape
    rows = x.numel() // D if D else 0
    if out is None:
        out = torch.empty_like(x)
    res_out = None
    if residual is not None:
        _require(residual, "residual", torch.float16)
        if residual.shape != x.shape:
            raise RuntimeError("residual must match x")
        res_out = torch.empty_like(x)
    S, rpad = (D + 255) // 256, (r + 31) // 32 * 32
    if parts is None:
        parts = torch.empty(n_u, S, rows, rpad, dtype=torch.float32, device=x.device)
    elif tuple(parts.shape) != (n_u, S, rows, rpad) or parts.dtype != torch.float32 \
            or not parts.is_contiguous():
        raise RuntimeError(f"parts must be contiguous fp32 ({n_u}, {S}, {rows}, {rpad})")
    _lib.check(lib.glq_rmsnorm_xu(
        x.data_ptr(), _lib.ptr(residual), weight.data_ptr(), rows, D, float(eps), out.data_ptr(),
        _lib.ptr(res_out), U.data_ptr(), D * r, n_u, r, parts.data_ptr(),
        _lib.stream_handle(x.device)), "glq_rmsnorm_xu")
    return (out, parts) if residual is None else (out, res_out, parts)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_w: torch.Tensor,
                 k_norm_w: torch.Tensor, eps: float, cos: torch.Tensor, sin: torch.Tensor,
                 k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                 len_out: torch.Tensor, q_out: torch.Tensor | None = None) -> torch.Tensor:
    """One decode token per row: q (T, Hq*128) -- or item-major (n, T, R), a
    batched GEMV's output over R-row slices of the q projection -- k and v
    (T, Hk*128) fp16 -> q' (T, Hq, 128) returned; k' and v written into the
    static caches (T, Hk, max_len, 128) at position pos (device int64
    scalar); pos + 1 into len_out (device int32) for decode_attention.
    cos/sin: (T or 1, 128)."""
    lib = _lib.load()
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w"),
                 (cos, "cos"), (sin, "sin"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _require(t, n, torch.float16)
    _require(pos, "pos", torch.int64)
    _require(len_out, "len_out", torch.int32)
    T, Hk, max_len, hd = k_cache.shape
    if v_cache.shape != k_cache.shape:
        raise RuntimeError("k_cache and v_cache differ in shape")
    item_rows = 0
    if q.dim() == 3 and q.shape[1] == T and q.shape[0] > 1:  # item-major
        item_rows = q.shape[2]
        Hq = q.shape[0] * item_rows // hd
        q2 = q
    else:
        Hq = q.shape[-1] // hd
        q2 = q.reshape(-1, q.shape[-1])
    k2, v2 = k.reshape(-1, k.shape[-1]), v.reshape(-1, v.shape[-1])
    if (not item_rows and q2.shape[0] != T) or k2.shape != (T, Hk * hd) or \
            v2.shape != (T, Hk * hd):
        raise RuntimeError("q, k, v rows must match the cache's batch and heads")
    c2, s2 = cos.reshape(-1, hd), sin.reshape(-1, hd)
    if c2.shape[0] not in (1, T) or s2.shape != c2.shape:
        raise RuntimeError("cos/sin must hold 1 or T rows of head_dim")
    if q_out is None:
        q_out = torch.empty(T, Hq, hd, dtype=torch.float16, device=q.device)
    _lib.check(lib.glq_qk_norm_rope(
        q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), T, Hq, Hk, hd,
        Hq * hd if item_rows else q2.shape[1], item_rows, k2.shape[1],
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), float(eps), c2.data_ptr(), s2.data_ptr(),
        hd if c2.shape[0] > 1 else 0, q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        max_len, pos.data_ptr(), len_out.data_ptr(), _lib.stream_handle(q.device)),
        "glq_qk_norm_rope")
    return q_out


def decode_attention_workspace(q: torch.Tensor, k_cache: torch.Tensor) -> torch.Tensor:
    """A zeroed workspace for decode_attention at these shapes (keep it for
    the calls that follow: every call leaves its counters zero)."""
    lib = _lib.load()
    T, Hk, max_len, _ = k_cache.shape
    n = lib.glq_decode_attention_workspace_bytes(T, q.shape[1], Hk, max_len)
    if n < 0:
        raise RuntimeError("invalid decode attention shapes")
    return torch.zeros(max(int(n), 256), dtype=torch.uint8, device=q.device)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     length: torch.Tensor, scale: float, advance: torch.Tensor | None = None,
                     out: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None, U: torch.Tensor | None = None,
                     parts: torch.Tensor | None = None):
    """Single-query GQA attention over cache positions [0, length): q (T, Hq,
    128), caches (T, Hk, max_len, 128) -> (T, Hq*128) fp16.  `advance`
    (device int64) is incremented by one after the launch's reads.
    `workspace` from decode_attention_workspace (a fresh one when None).
    With U (Hq*128, r) the same launch also forms the fp32 partials of out U,
    one per KV group, parts (Hk, T, rpad) -- the a of
    packed_dequant_matmul_parts (glq_decode_attention_xu) -- and (out, parts)
    is returned."""
    lib = _lib.load()
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _require(t, n, torch.float16)
    _require(length, "length", torch.int32)
    if advance is not None:
        _require(advance, "advance", torch.int64)
    T, Hk, max_len, hd = k_cache.shape
    if v_cache.shape != k_cache.shape or q.shape[0] != T or q.shape[-1] != hd:
        raise RuntimeError("q (T, Hq, 128) and caches (T, Hk, max_len, 128) must agree")
    Hq = q.shape[1]
    if out is None:
        out = torch.empty(T, Hq * hd, dtype=torch.float16, device=q.device)
    if U is not None:
        _require(U, "U", torch.float16)
        if U.dim() != 2 or U.shape[0] != Hq * hd:
            raise RuntimeError(f"U must be ({Hq * hd}, r)")
        r = U.shape[1]
        rpad = (r + 31) // 32 * 32
        if parts is None:
            parts = torch.empty(Hk, T, rpad, dtype=torch.float32, device=q.device)
        elif tuple(parts.shape) != (Hk, T, rpad) or parts.dtype != torch.float32 \
                or not parts.is_contiguous():
            raise RuntimeError(f"parts must be contiguous fp32 ({Hk}, {T}, {rpad})")
        if workspace is None:
            workspace = decode_attention_workspace(q, k_cache)
        _lib.check(lib.glq_decode_attention_xu(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), T, Hq, Hk, hd, max_len,
            length.data_ptr(), float(scale), _lib.ptr(advance), out.data_ptr(), U.data_ptr(), r,
            parts.data_ptr(), workspace.data_ptr(), workspace.numel(),
            _lib.stream_handle(q.device)), "glq_decode_attention_xu")
        return out, parts
    if workspace is None:
        workspace = decode_attention_workspace(q, k_cache)
    _lib.check(lib.glq_decode_attention(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), T, Hq, Hk, hd, max_len,
        length.data_ptr(), float(scale), _lib.ptr(advance), out.data_ptr(),
        workspace.data_ptr(), workspace.numel(), _lib.stream_handle(q.device)),
        "glq_decode_attention")
    return out
