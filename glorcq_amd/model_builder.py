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

plus `load_glorcq_checkpoint` (the two .pt files, read with the safe loader),
`build_glorcq_layers`, the part of `_replace_linear_layers` (:335-433) that
turns each stored module into a GLoRCQLinear, and `load_glorcq_model`
(:203-312), the one call from a checkpoint directory to a runnable causal LM:
the HF model built on the meta device from config.json, the stored modules
swapped in, every MoE block a GraphCompatibleMoeBlock over the stored experts,
the cross-layer U pool installed.

Differences: LoRA factors are dequantized on the GPU by the library's kernel
(glq_dequant_factor, bit-identical to the reference's fp32 arithmetic + .half()),
so `_dequant_intN` returns fp16 (every reference caller rounds to fp16). The
kernel-side global pool is a (rows, K, r) stack per projection type; the
reference's (K, rows*r) column layout is also returned for callers that use it.
"""

from __future__ import annotations

import glob
import os
from types import SimpleNamespace

import torch
import torch.nn as nn

from . import _lib
from .hadamard_rotation import generate_rht_signs
from .quantized_linear import GLoRCQLinear, RotationCache

__all__ = [
    "SharedUCache", "RotationCache", "_dequant_intN", "_unpack_int4", "_build_global_u_pool",
    "build_u_pool_stacks", "_install_global_u_pool",
    "_load_lora_for_module", "build_assignment_lookup", "load_glorcq_checkpoint",
    "build_glorcq_layers", "load_glorcq_model", "is_regular_expert", "is_shared_expert",
    "extract_expert_info",
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


# ---------------------------------------------------------------------------
# Model loading (model_builder.py:203-312)
# ---------------------------------------------------------------------------
def _find_linear_modules(module, prefix=""):
    """{dotted name: (parent, attribute, nn.Linear)} below `module`."""
    out = {}
    for name, child in module.named_children():
        full = f"{prefix}.{name}" if prefix else name
        if isinstance(child, nn.Linear):
            out[full] = (module, name, child)
        else:
            out.update(_find_linear_modules(child, full))
    return out


def _dense_state(model_path):
    """Tensors of any *.safetensors files in the checkpoint directory (the
    non-quantized weights under their HF names), read with the safetensors
    loader (no code runs from the file); {} when there are none."""
    files = sorted(glob.glob(os.path.join(model_path, "*.safetensors")))
    if not files:
        return {}
    from safetensors.torch import load_file

    state = {}
    for f in files:
        state.update(load_file(f, device="cpu"))
    return state


_MOE_PROJ = {"gate_proj": "gate_proj", "up_proj": "up_proj", "down_proj": "down_proj",
             "w1": "gate_proj", "w3": "up_proj", "w2": "down_proj"}


def _stored_moe(mods):
    """{block prefix: ({expert: {proj: GLoRCQLinear}}, {proj: shared GLoRCQLinear})}
    of one layer's stored modules ('mlp.experts.<e>.gate_proj', Mixtral's
    'block_sparse_moe.experts.<e>.w1', 'mlp.shared_expert.up_proj', ...)."""
    blocks = {}
    for name, ql in mods.items():
        parts = name.split(".")
        if "experts" in parts and not is_shared_expert(name):
            i = parts.index("experts")
            proj = _MOE_PROJ.get(parts[-1])
            if proj is None or len(parts) != i + 3:  # <prefix>.experts.<e>.<proj>
                continue
            prefix = ".".join(parts[:i])
            blocks.setdefault(prefix, ({}, {}))[0].setdefault(int(parts[i + 1]), {})[proj] = ql
        elif is_shared_expert(name) and parts[-1] in _MOE_PROJ:
            i = parts.index("shared_expert")
            prefix = ".".join(parts[:i])
            blocks.setdefault(prefix, ({}, {}))[1][_MOE_PROJ[parts[-1]]] = ql
    return {k: v for k, v in blocks.items() if v[0]}


def _get_submodule(root, dotted):
    m = root
    for part in dotted.split("."):
        m = getattr(m, part, None)
        if m is None:
            return None
    return m


def _dense_weight(state, key, shape, device, dtype=torch.float16):
    """The stored tensor of `key`, or zeros of `shape` when the checkpoint
    holds none (the reference zero-fills every non-quantized parameter,
    model_builder.py:416-428)."""
    t = state.get(key)
    if t is None:
        return torch.zeros(shape, dtype=dtype, device=device)
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{key}: stored shape {tuple(t.shape)} != model's {tuple(shape)}")
    return t.to(device, dtype).contiguous()


def _moe_block(config, hf_block, prefix, experts, shared, state, device):
    """A GraphCompatibleMoeBlock over a layer's stored experts (reference
    _replace_moe_blocks, model_builder.py:186-197, which wraps the HF block;
    here the HF block's experts are fused 3-D tensors in transformers 5, so
    the block is assembled from the stored GLoRCQLinear modules)."""
    from .moe_block import GraphCompatibleMoeBlock

    E = max(experts) + 1
    if sorted(experts) != list(range(E)) or any(len(v) != 3 for v in experts.values()):
        raise RuntimeError(f"{prefix}: the checkpoint must hold gate/up/down of experts 0..{E - 1}")
    H = experts[0]["gate_proj"].in_features
    top_k = int(getattr(config, "num_experts_per_tok", 2))
    norm = getattr(config, "norm_topk_prob", None)
    if norm is None:  # Mixtral renormalises its top-k weights
        norm = getattr(config, "model_type", "") == "mixtral"
    gate_key = f"{prefix}.gate.weight"
    blk = SimpleNamespace(top_k=top_k, norm_topk_prob=bool(norm), num_experts=E)
    blk.gate = SimpleNamespace(weight=_dense_weight(state, gate_key, (E, H), device))
    blk.experts = [SimpleNamespace(**experts[e]) for e in range(E)]
    if shared:
        if len(shared) != 3:
            raise RuntimeError(f"{prefix}: the shared expert needs gate/up/down")
        blk.shared_expert = SimpleNamespace(**shared)
        has_gate = _get_submodule(hf_block, "shared_expert_gate") is not None \
            or f"{prefix}.shared_expert_gate.weight" in state
        blk.shared_expert_gate = (SimpleNamespace(weight=_dense_weight(
            state, f"{prefix}.shared_expert_gate.weight", (1, H), device)) if has_gate else None)
    out = GraphCompatibleMoeBlock(blk)
    out.return_router_logits = _moe_returns_router_logits()
    return out


def _moe_returns_router_logits() -> bool:
    """transformers 4.x decoder layers unpack (states, router logits) from
    their MoE block; 5.x blocks return the states alone."""
    import transformers

    return int(transformers.__version__.split(".")[0]) < 5


def _materialize(model, config, state, device):
    """Every parameter or buffer still on the meta device gets its stored
    value from `state` (HF names) or zeros, as the reference does
    (model_builder.py:316-333, 416-428); rotary embeddings are rebuilt on the
    device from the config (zero inverse frequencies would switch rotary off)."""
    for name, mod in list(model.named_modules()):
        if type(mod).__name__.endswith("RotaryEmbedding") and any(
                b.is_meta for b in mod.buffers(recurse=False)):
            new = type(mod)(config=config).to(device)
            parent = _get_submodule(model, name.rsplit(".", 1)[0]) if "." in name else model
            setattr(parent, name.rsplit(".", 1)[-1], new)
    for name, mod in model.named_modules():
        for pname, p in list(mod.named_parameters(recurse=False)):
            if p.is_meta:
                key = f"{name}.{pname}" if name else pname
                val = _dense_weight(state, key, p.shape, device, p.dtype)
                setattr(mod, pname, nn.Parameter(val, requires_grad=False))
        for bname, b in list(mod.named_buffers(recurse=False)):
            if b.is_meta:
                key = f"{name}.{bname}" if name else bname
                mod.register_buffer(bname, _dense_weight(state, key, b.shape, device, b.dtype))


def load_glorcq_model(model_path, device="cuda:0", rotation_cache=None):
    """A GLoRCQ real-quantized checkpoint directory -> a causal LM on `device`
    whose stored projections are GLoRCQLinear layers on the gfx950 kernels
    (reference load_glorcq_model, inference/model_builder.py:203-312).

    The directory holds config.json, glorcq_model.pt and cross_layer_info.pt
    (read with torch's safe loader), and optionally *.safetensors files with
    the non-quantized weights under their HF names (embeddings, norms, router
    and shared-expert gates, attention biases, lm_head); what no file holds
    is zero-filled, as the reference does for every non-quantized parameter.
    Steps as the reference: the HF model on the meta device from the config
    (built-in architectures only: no code from the directory runs), each
    stored nn.Linear module replaced by its GLoRCQLinear with LoRA, each MoE
    block with stored experts replaced by a GraphCompatibleMoeBlock, the
    cross-layer U pool installed on every block, the rest materialised on
    `device`.  TurboQuant modules need `rotation_cache` with their codebook
    (the reference builds one from the quantizer package, absent here).
    The result runs eagerly or under GLoRCQGraphWrapper."""
    from transformers import AutoConfig, AutoModelForCausalLM

    device = torch.device(device)
    config = AutoConfig.from_pretrained(model_path)
    config.use_cache = True
    if not os.path.exists(os.path.join(model_path, "glorcq_model.pt")):
        raise FileNotFoundError(
            f"glorcq_model.pt not found in {model_path} (a fake-quant checkpoint loads with "
            f"the standard HF loader)")
    model_data, cross = load_glorcq_checkpoint(model_path)
    mc = model_data.get("model_config", {})
    if mc.get("use_turboquant", False) and rotation_cache is None:
        raise RuntimeError("this checkpoint holds TurboQuant modules: pass a RotationCache "
                           "with their codebook (and rotation)")
    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(config)
    model = model.to(torch.float16)
    model.seqlen = 4096
    layers, u_cache = build_glorcq_layers(model_data, cross, device=device,
                                          rotation_cache=rotation_cache)
    state = _dense_state(model_path)
    base = getattr(model, "model", model)
    base_prefix = "model." if base is not model else ""
    for li, layer in enumerate(base.layers):
        mods = layers.get(li, {})
        lp = f"{base_prefix}layers.{li}"
        for prefix, (experts, shared) in _stored_moe(mods).items():
            hf_block = _get_submodule(layer, prefix)
            if hf_block is None:
                raise RuntimeError(f"layer {li}: the model has no module {prefix!r}")
            blk = _moe_block(config, hf_block, f"{lp}.{prefix}", experts, shared, state, device)
            parent = _get_submodule(layer, prefix.rsplit(".", 1)[0]) if "." in prefix else layer
            setattr(parent, prefix.rsplit(".", 1)[-1], blk)
        for name, (parent, attr, lin) in _find_linear_modules(layer).items():
            ql = mods.get(name)
            if ql is None:
                continue
            if (ql.in_features, ql.out_features) != (lin.in_features, lin.out_features):
                raise RuntimeError(f"layer {li} {name}: stored ({ql.out_features}, "
                                   f"{ql.in_features}) != model's ({lin.out_features}, "
                                   f"{lin.in_features})")
            if lin.bias is not None and f"{lp}.{name}.bias" in state:
                ql.set_bias(state[f"{lp}.{name}.bias"].to(torch.float16), device=device)
            setattr(parent, attr, ql)
    _materialize(model, config, state, device)
    if getattr(config, "tie_word_embeddings", False) and hasattr(model, "lm_head"):
        model.lm_head.weight = base.embed_tokens.weight
    _install_global_u_pool(model, u_cache)
    model.eval()
    return model
