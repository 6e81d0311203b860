"""Checkpoint adapter: the reference's on-disk GLoRCQ format on the MI355X layers.

Mirrors the loader pieces of the reference's inference/model_builder.py that
sit on the hot path's data (same names and meaning):

  SharedUCache                       :27-66   shared U per (wtype, cluster), intN/int4/fp16
  _dequant_intN, _unpack_int4        :69-80   LoRA factor storage
  _build_global_u_pool               :143-173 one U pool per projection type
  _install_global_u_pool             :176-183 pool shared by every MoE layer
  _load_lora_for_module              :465-544 U + SV (int4 / fp16 / intN / old V+S)
  is_regular_expert, is_shared_expert, extract_expert_info
                                     (utils/moe_utils.py:9-36)

plus `load_glorcq_checkpoint` (the two .pt files, read with the safe loader)
and `build_glorcq_layers`, the part of `_replace_linear_layers` (:335-433)
that turns each stored module into a GLoRCQLinear, without building an HF
model around it (the reference's meta-device HF model construction targets
transformers 4.45 layouts; here the caller places the layers, e.g. into a
GraphCompatibleMoeBlock).

Differences: LoRA factors are dequantized on the GPU by the library's kernel
(glq_dequant_factor, bit-identical to the reference's fp32 arithmetic + .half()),
so `_dequant_intN` returns fp16 (every reference caller rounds to fp16). The
kernel-side global pool is a (rows, K, r) stack per projection type; the
reference's (K, rows*r) column layout is also returned for callers that use it.
"""

from __future__ import annotations

import os

import torch

from . import _lib
from .hadamard_rotation import generate_rht_signs
from .quantized_linear import GLoRCQLinear, RotationCache

__all__ = [
    "SharedUCache", "RotationCache", "_dequant_intN", "_unpack_int4", "_build_global_u_pool",
    "build_u_pool_stacks", "_install_global_u_pool",
    "_load_lora_for_module", "build_assignment_lookup", "load_glorcq_checkpoint",
    "build_glorcq_layers", "is_regular_expert", "is_shared_expert", "extract_expert_info",
]


# ---------------------------------------------------------------------------
# module-name helpers (utils/moe_utils.py:9-36)
# ---------------------------------------------------------------------------
def is_shared_expert(layer_name: str) -> bool:
    return "shared_expert" in layer_name


def _has_experts_segment(layer_name: str) -> bool:
    return ".experts." in layer_name or layer_name.startswith("experts.")


def is_regular_expert(layer_name: str) -> bool:
    return _has_experts_segment(layer_name) and not is_shared_expert(layer_name)


def extract_expert_info(layer_name: str):
    """(expert index, projection suffix) of 'x.experts.<i>.<proj>', else (None, None)."""
    if _has_experts_segment(layer_name):
        parts = layer_name.split(".")
        i = parts.index("experts") + 1
        return int(parts[i]), ".".join(parts[i + 1:])
    return None, None


_WTYPES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj",
           "w1", "w2", "w3")
_MIXTRAL = {"w1": "gate_proj", "w2": "down_proj", "w3": "up_proj"}


def module_wtype(module_name: str):
    """Projection type of a module name, Mixtral's w1/w2/w3 mapped to
    gate/down/up (model_builder.py:486-494)."""
    for wt in _WTYPES:
        if module_name == wt or module_name.endswith("." + wt):
            return _MIXTRAL.get(wt, wt)
    return None


def module_expert_index(module_name: str) -> int:
    """Expert index; -2 for the shared expert, -1 for non-expert modules
    (model_builder.py:477-483)."""
    if is_regular_expert(module_name):
        idx, _ = extract_expert_info(module_name)
        return idx if idx is not None else -3
    if is_shared_expert(module_name):
        return -2
    return -1


# ---------------------------------------------------------------------------
# LoRA factor storage
# ---------------------------------------------------------------------------
def _unpack_int4(packed: torch.Tensor, orig_rows: int) -> torch.Tensor:
    """((rows+1)//2, cols) uint8 -> (orig_rows, cols) int8 in [-7, 8]: row 2i
    in the low nibble, row 2i+1 in the high nibble, value - 7 (a format
    utility; the GPU load path fuses it into glq_dequant_factor)."""
    lo = (packed & 0xF).to(torch.int8) - 7
    hi = ((packed >> 4) & 0xF).to(torch.int8) - 7
    return torch.stack([lo, hi], dim=1).reshape(-1, packed.shape[1])[:orig_rows]


def _factor(q: torch.Tensor, scale: torch.Tensor, nbits: int, device,
            int4_rows: int | None = None) -> torch.Tensor:
    """fp16 factor from its stored codes on the GPU (glq_dequant_factor)."""
    lib = _lib.load()
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("LoRA factors are dequantized on the GPU (glorcq_amd has no CPU path)")
    q = q.to(dev).contiguous()
    scale = scale.to(dev, torch.float16).contiguous()
    cols = q.shape[1]
    rows = int4_rows if int4_rows is not None else q.shape[0]
    if int4_rows is not None:
        if q.dtype != torch.uint8 or q.shape[0] != (rows + 1) // 2:
            raise RuntimeError("int4-packed factor must be ((rows+1)//2, cols) uint8")
    elif q.dtype != torch.int8:
        raise RuntimeError(f"intN factor codes must be int8 (got {q.dtype})")
    if scale.numel() == cols and scale.shape[-1] == cols and (scale.dim() == 1 or
                                                             scale.shape[0] == 1):
        per_row = 0
    elif scale.numel() == rows and scale.shape[0] == rows:
        per_row = 1
    else:
        raise RuntimeError(f"scale {tuple(scale.shape)} is neither per column ({cols},) "
                           f"nor per row ({rows}, 1)")
    out = torch.empty(rows, cols, dtype=torch.float16, device=dev)
    rc = lib.glq_dequant_factor(q.data_ptr(), int(int4_rows is not None), rows, cols,
                                scale.data_ptr(), per_row, nbits, out.data_ptr(),
                                _lib.stream_handle(dev))
    _lib.check(rc, "glq_dequant_factor")
    return out


def _dequant_intN(q: torch.Tensor, scale: torch.Tensor, nbits: int) -> torch.Tensor:
    """fp16(q / (2^(nbits-1) - 1) * scale), fp32 arithmetic, on q's GPU
    (model_builder.py:69-72 followed by .half(), as every caller there does)."""
    return _factor(q, scale, nbits, q.device)


def dequant_int4_packed(packed: torch.Tensor, orig_rows: int, scale: torch.Tensor,
                        device="cuda") -> torch.Tensor:
    """_dequant_intN(_unpack_int4(packed, orig_rows), scale, 4).half() in one
    launch (model_builder.py:42-45, :505-509)."""
    return _factor(packed, scale, 4, device, int4_rows=orig_rows)


class SharedUCache:
    """Shared U factors per (wtype, cluster id), dequantized once at load
    (reference SharedUCache, model_builder.py:27-66).  Entries: U_fp16, or
    U_int4_packed + U_orig_rows + U_scale, or U_int8 + U_scale (u_bits); an
    old-format S is kept alongside."""

    def __init__(self, shared_matrices, uv_bits, device="cuda", u_bits=None):
        self._cache = {}
        ub = u_bits if u_bits is not None else uv_bits
        for wtype, groups in shared_matrices.items():
            for gid, data in groups.items():
                if "U_fp16" in data:
                    U = data["U_fp16"].to(device, torch.float16).contiguous()
                elif "U_int4_packed" in data:
                    U = dequant_int4_packed(data["U_int4_packed"], int(data["U_orig_rows"].item()),
                                            data["U_scale"], device)
                else:
                    U = _factor(data["U_int8"], data["U_scale"], ub, device)
                S = data["S"].to(device, torch.float16) if "S" in data else None
                self._cache[(wtype, gid)] = (U, S)

    def get(self, wtype, group_id):
        return self._cache.get((wtype, group_id), (None, None))

    def preload_for_layer(self, layer_idx, active_experts=None):
        """Interface kept from the reference (a no-op there too)."""

    def evict(self, wtype=None, group_id=None):
        """Interface kept from the reference (a no-op there too)."""


def _pool_items(u_cache):
    groups = {"gate_proj": [], "up_proj": [], "down_proj": []}
    for (wkey, gid), (U, _S) in u_cache._cache.items():
        if wkey in groups:
            groups[wkey].append((gid, U))
    for wkey in groups:
        groups[wkey].sort(key=lambda x: x[0])
    return groups


def _build_global_u_pool(u_cache):
    """Reference layout (model_builder.py:143-173): pools[proj] = (K, rows*r)
    with cluster i's U in columns [i*r, (i+1)*r); id_maps[proj][(wtype_key,
    group_id)] = i."""
    pools, id_maps = {}, {}
    for wkey, items in _pool_items(u_cache).items():
        if not items:
            continue
        proj = wkey.split("_")[0]
        pools[proj] = torch.cat([u for _, u in items], dim=1)
        id_maps[proj] = {(wkey, gid): i for i, (gid, _) in enumerate(items)}
    return pools, id_maps


def build_u_pool_stacks(u_cache):
    """Kernel layout of the same pools: stacks[proj] = (rows, K, r) fp16 and the
    same id maps; GraphCompatibleMoeBlock.set_global_pool takes these."""
    stacks, id_maps = {}, {}
    for wkey, items in _pool_items(u_cache).items():
        if not items:
            continue
        proj = wkey.split("_")[0]
        stacks[proj] = torch.stack([u.contiguous() for _, u in items]).contiguous()
        id_maps[proj] = {(wkey, gid): i for i, (gid, _) in enumerate(items)}
    return stacks, id_maps


def _install_global_u_pool(model, u_cache):
    """Installs the pool on every block of `model` that has set_global_pool
    (model_builder.py:176-183): every layer reads a cluster's U at one address."""
    stacks, id_maps = build_u_pool_stacks(u_cache)
    n = 0
    for m in model.modules():  # the model itself included
        if hasattr(m, "set_global_pool"):
            m.set_global_pool(stacks, id_maps)
            n += 1
    return n


def build_assignment_lookup(assignments):
    """(wtype, layer, expert) -> (group_id, wtype, index into per_expert_V[wtype])
    (model_builder.py:349-354)."""
    lookup = {}
    for wtype, records in assignments.items():
        for li, rec in enumerate(records):
            lookup[(wtype, rec["layer"], rec["expert"])] = (rec["group_id"], wtype, li)
    return lookup


def _load_lora_for_module(ql, layer_idx, module_name, assignment_lookup, u_cache,
                          per_expert_V, uv_bits, device, sv_bits=None):
    """Attaches U and SV to `ql` (model_builder.py:465-544): the cluster's U from
    the cache and the expert's SV stored as int4-packed, fp16, intN (sv_bits),
    or the old V (uv_bits) + shared S.  Shared experts carry no LoRA.  Tags
    ql.cluster_id = (wtype, group_id)."""
    expert_idx = module_expert_index(module_name)
    wtype = module_wtype(module_name)
    if wtype is None or expert_idx == -2:
        return
    key = (wtype, layer_idx, expert_idx)
    if key not in assignment_lookup:
        return
    group_id, wkey, local_idx = assignment_lookup[key]
    U, S_shared = u_cache.get(wkey, group_id)
    if U is None:
        return
    if wkey not in per_expert_V or per_expert_V[wkey][local_idx] is None:
        return
    v = per_expert_V[wkey][local_idx]
    if "SV_int4_packed" in v:
        SV = dequant_int4_packed(v["SV_int4_packed"], int(v["SV_orig_rows"].item()),
                                 v["SV_scale"], device)
        ql.load_sv(U, SV, device=device)
    elif "SV_fp16" in v:
        ql.load_sv(U, v["SV_fp16"].to(device, torch.float16), device=device)
    elif "SV_int8" in v:
        nb = sv_bits if sv_bits is not None else uv_bits
        ql.load_sv(U, _factor(v["SV_int8"], v["SV_scale"], nb, device), device=device)
    else:
        V = _factor(v["V_int8"], v["V_scale"], uv_bits, device)
        ql.load_lora(U, S_shared, V, device=device)
    ql.cluster_id = (wkey, group_id)


def load_glorcq_checkpoint(model_path):
    """(glorcq_model.pt dict, cross_layer_info.pt dict) from a checkpoint
    directory (model_builder.py:241-252), read with torch's safe loader
    (weights_only=True): the files hold dicts of tensors and plain values."""
    a = os.path.join(model_path, "glorcq_model.pt")
    b = os.path.join(model_path, "cross_layer_info.pt")
    if not os.path.exists(a):
        raise FileNotFoundError(f"glorcq_model.pt not found in {model_path}")
    model_data = torch.load(a, map_location="cpu", weights_only=True)
    cross = torch.load(b, map_location="cpu", weights_only=True)
    return model_data, cross


def build_glorcq_layers(model_data, cross_layer_info, device="cuda", rotation_cache=None):
    """Every stored module of a checkpoint as a GLoRCQLinear with its LoRA:
    returns ({layer_idx: {module_name: GLoRCQLinear}}, SharedUCache).  GPTQ
    modules (qweight_int) pack on the device; TurboQuant modules
    (packed_indices) need `rotation_cache` holding their codebook (and Pi for
    the QR rotation); with rotation_type 'hadamard' in the model config each
    turbo layer gets its RHT signs (model_builder.py:278-286)."""
    mc = model_data.get("model_config", {})
    layers = model_data["layers"]
    cfg = cross_layer_info.get("config", {})
    uv_bits = cfg.get("uv_bits", mc.get("uv_bits", 8))
    u_bits = cfg.get("u_bits", uv_bits)
    sv_bits = cfg.get("sv_bits", uv_bits)
    u_cache = SharedUCache(cross_layer_info["shared_matrices"], uv_bits, device=device,
                           u_bits=u_bits)
    lookup = build_assignment_lookup(cross_layer_info["assignments"])
    per_expert_V = cross_layer_info["per_expert_V"]
    hadamard = mc.get("rotation_type", "qr") == "hadamard"
    out = {}
    for layer_idx, mods in layers.items():
        out[layer_idx] = {}
        for name, packed in mods.items():
            if "qweight_int" in packed:
                n_out, n_in = packed["qweight_int"].shape
                ql = GLoRCQLinear(n_in, n_out)
                ql.load_gptq(packed, device=device)
            elif "packed_indices" in packed:
                n_out = packed["packed_indices"].shape[0]
                ql = GLoRCQLinear(int(packed["dim"]), n_out)
                if rotation_cache is None:
                    raise RuntimeError(f"layer {layer_idx} {name}: TurboQuant weights need a "
                                       f"RotationCache with their codebook")
                ql.load_turbo(packed, rotation_cache, device=device)
                if hadamard:
                    ql._rht_signs = generate_rht_signs(ql.turbo_dim, seed=ql.turbo_seed,
                                                       device=device)
            else:
                raise RuntimeError(f"layer {layer_idx} {name}: unknown stored format "
                                   f"{sorted(packed.keys())}")
            _load_lora_for_module(ql, layer_idx, name, lookup, u_cache, per_expert_V, uv_bits,
                                  device, sv_bits=sv_bits)
            out[layer_idx][name] = ql
    return out, u_cache
