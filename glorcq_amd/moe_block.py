"""MoE block decode step on the MI355X kernels.

`GraphCompatibleMoeBlock` mirrors the reference class of the same name
(inference/moe_block.py:42-436): built from a Qwen2-MoE style block whose
expert and shared-expert projections are `GLoRCQLinear` layers, and
`forward(hidden_states) -> (final, router_logits)` with the same routing
semantics (fp32 softmax over fp16 logits, top-k, optional renormalisation,
routing weights cast to the hidden dtype, :386-392), cluster-shared x U for
gate/up (:290-322), per-expert down(act(gate) * up) with its own low-rank term,
and the sigmoid-gated shared expert (:429-433).

Differences:
* One C-ABI call (`glq_moe_decode`, four launches, five when the x U jobs are
  gated on routing) for the whole step, with
  routing kept on the device: no `.tolist()` host syncs (reference :410,454),
  no per-step weight concatenation (:509-510), and only the selected experts'
  weights are read (the reference's graph mode runs all E, :742-890).  Every
  step can be captured in a hipGraph (torch.cuda.graph) at any batch <= 64.
* The experts' packed weights are stacked expert-major once, at construction,
  and the cluster U factors form one pool per projection (the reference's
  global U pool, model_builder.py:143-183).
* Routed experts are GPTQ layers (asymmetric, group 128, 2- or 4-bit
  containers) or TurboQuant layers (the reference's 2-bit expert format).
  A TurboQuant block runs as a sequence of launches on the current stream,
  still graph-safe with routing on the device: glq_moe_route; the input
  rotation of gate/up (glq_rht, or x Pi^T as a library GEMM, as the
  reference); x U of every cluster (glq_lowrank_xu_batched); the gate, then
  the up GEMV of every pick with the SwiGLU inter formed in the up launch's
  store (glq_turbo_moe_gemv); the rotation of inter; each pick's own
  a_down = fp16(inter U_c) (glq_lowrank_xu_routed); the down GEMV of every
  pick; the shared expert (its own GLoRCQLinear projections); and the
  weighted combine with the gated shared term (glq_moe_combine).  Each step
  reads only the picked experts' weights (the reference's graph mode runs
  all E, :742-890).
"""

from __future__ import annotations

import ctypes
import os

import torch
import torch.nn as nn

from . import _lib
from .format import PROJS, MoEProblem
from .kernels import retire_workspace

_PROJ_ATTR = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}


def _stack(ts):
    return torch.stack([t.contiguous() for t in ts]).contiguous()


class GraphCompatibleMoeBlock(nn.Module):
    """Qwen2-MoE block on the gfx950 MoE kernels (reference
    inference/moe_block.py:42-436)."""

    def __init__(self, original_block=None, *, stacked: dict | None = None):
        super().__init__()
        if stacked is None:
            if original_block is None:
                raise RuntimeError("GraphCompatibleMoeBlock needs a block or stacked weights")
            stacked = self._stack_block(original_block)
        self.kind = stacked.get("kind", "gptq")
        self.num_experts = stacked["E"]
        self.top_k = stacked["top_k"]
        self.norm_topk_prob = bool(stacked["norm_topk_prob"])
        self.hidden = stacked["H"]
        self.inter = stacked["inter"]
        self.rank = stacked["rank"]
        self.n_clusters = stacked["n_clusters"]
        self.bits = stacked.get("bits", 2)
        self.shared_bits = stacked["shared_bits"]
        self.shared_inter = stacked["shared_inter"]
        self.group = 128
        self.graph_mode = True  # every step is graph-safe
        # forward returns (final, router_logits) as the reference's block does
        # (transformers 4.x decoder layers unpack the pair); False returns final
        # alone, the contract of transformers 5 sparse-MoE blocks
        self.return_router_logits = True
        self.t = stacked  # device tensors (kept alive for the kernels)
        # the prefill kernels take integer zero-points (GPTQ's are), routed and
        # shared alike; checked once here, otherwise a prefill runs as
        # consecutive decode steps
        zkeys = [f"zeros_{p}" for p in PROJS]
        zkeys += [f"szeros_{p}" for p in PROJS if f"szeros_{p}" in stacked]
        self.zeros_integral = self.kind == "gptq" and all(
            bool(torch.equal(stacked[k], stacked[k].round())) for k in zkeys)

    # ---- construction ----
    @staticmethod
    def _stack_block(blk) -> dict:
        """Stacks a block's GLoRCQLinear experts (reference constructor
        :45-77 takes the same block).  Clusters: experts whose projection
        carries the same cluster_id share one U; experts without one get
        their own."""
        experts = list(blk.experts)
        E = len(experts)
        lin0 = experts[0].gate_proj
        if lin0.quant_type == "turbo":
            return _stack_turbo_block(blk)
        dev = lin0.codes.device
        out = {"E": E, "top_k": int(blk.top_k), "norm_topk_prob": bool(blk.norm_topk_prob),
               "H": lin0.in_features, "inter": lin0.out_features,
               "bits": lin0.pack_bits, "rank": lin0.rank}
        out["router_w"] = blk.gate.weight.detach().to(dev, torch.float16).contiguous()
        n_clusters = 0
        for proj in PROJS:
            lins = [getattr(ex, _PROJ_ATTR[proj]) for ex in experts]
            for lin in lins:
                if lin.quant_type != "gptq" or lin.gptq_sym or lin.gptq_groupsize != 128:
                    raise RuntimeError("MoE kernels take asymmetric GPTQ experts, group 128")
                if lin.pack_bits != out["bits"] or lin.rank != out["rank"]:
                    raise RuntimeError("all experts need one code width and one LoRA rank")
            out[f"codes_{proj}"] = _stack([lin.codes for lin in lins])
            out[f"scales_{proj}"] = _stack([lin.scales for lin in lins])
            out[f"zeros_{proj}"] = _stack([lin.zeros for lin in lins])
            if out["rank"] > 0:
                ids, pool, cl = {}, [], []
                for e, lin in enumerate(lins):
                    key = ("c", lin.cluster_id) if lin.cluster_id is not None else ("e", e)
                    if key not in ids:
                        ids[key] = len(pool)
                        pool.append(lin.U)
                    cl.append(ids[key])
                out[f"U_{proj}"] = _stack(pool)
                out[f"urows_{proj}"] = len(pool)  # may be fewer than n_clusters
                out[f"cluster_{proj}"] = torch.tensor(cl, dtype=torch.int32, device=dev)
                out[f"ckeys_{proj}"] = list(ids.keys())  # local cluster -> key
                out[f"SV_{proj}"] = _stack([lin.SV for lin in lins])
                n_clusters = max(n_clusters, len(pool))
        out["n_clusters"] = n_clusters
        sh = getattr(blk, "shared_expert", None)
        if sh is not None:
            out["shared_bits"] = sh.gate_proj.pack_bits
            out["shared_inter"] = sh.gate_proj.out_features
            for proj in PROJS:
                lin = getattr(sh, _PROJ_ATTR[proj])
                if lin.quant_type != "gptq" or lin.gptq_sym or lin.gptq_groupsize != 128:
                    raise RuntimeError("shared expert must be asymmetric GPTQ, group 128")
                out[f"scodes_{proj}"] = lin.codes
                out[f"sscales_{proj}"] = lin.scales
                out[f"szeros_{proj}"] = lin.zeros
            g = getattr(blk, "shared_expert_gate", None)
            out["shared_gate_w"] = (None if g is None else
                                    g.weight.detach().reshape(-1).to(dev, torch.float16)
                                    .contiguous())
        else:
            out["shared_bits"], out["shared_inter"], out["shared_gate_w"] = 0, 0, None
        return out

    @classmethod
    def from_problem(cls, p: MoEProblem, device) -> "GraphCompatibleMoeBlock":
        """Block from a format.MoEProblem (synthetic configs, tests, bench)."""
        d = torch.device(device)
        if hasattr(p.experts["gate"], "centroids"):  # TurboQuant experts
            return cls(stacked=_turbo_from_problem(p, d))
        t = {"E": p.E, "top_k": p.top_k, "norm_topk_prob": p.norm_topk_prob, "H": p.H,
             "inter": p.inter, "bits": p.experts["gate"].bits, "rank": p.rank,
             "n_clusters": p.n_clusters,
             "router_w": p.router_w.to(d).contiguous()}
        for proj in PROJS:
            q = p.experts[proj]
            t[f"codes_{proj}"] = q.codes.to(d).contiguous()
            t[f"scales_{proj}"] = q.scales.to(d).contiguous()
            t[f"zeros_{proj}"] = q.zeros.to(d).contiguous()
            if p.rank > 0:
                t[f"U_{proj}"] = p.U[proj].to(d).contiguous()
                t[f"cluster_{proj}"] = p.cluster_of[proj].to(d, torch.int32).contiguous()
                t[f"SV_{proj}"] = p.SV[proj].to(d).contiguous()
        if p.shared is not None:
            t["shared_bits"] = p.shared["gate"].bits
            t["shared_inter"] = p.shared["gate"].N
            for proj in PROJS:
                s = p.shared[proj]
                t[f"scodes_{proj}"] = s.codes[0].to(d).contiguous()
                t[f"sscales_{proj}"] = s.scales[0].to(d).contiguous()
                t[f"szeros_{proj}"] = s.zeros[0].to(d).contiguous()
            t["shared_gate_w"] = p.shared_gate_w.reshape(-1).to(d).contiguous()
        else:
            t["shared_bits"], t["shared_inter"], t["shared_gate_w"] = 0, 0, None
        return cls(stacked=t)

    def set_global_pool(self, pools: dict, id_maps: dict):
        """Points the block's U factors at cross-layer pools (the reference's
        set_global_pool, inference/moe_block.py:85-99, fed by
        model_builder._install_global_u_pool): pools[proj] is a (rows, K, r)
        fp16 stack shared by every layer, id_maps[proj] maps a layer's
        cluster_id (GLoRCQLinear.cluster_id) to its row.  gate/up keep this
        block's x U per local cluster, read from the pool rows (u_slot); down
        reads the pool row of each expert's cluster.  Experts without a
        cluster_id keep their own U (a pool without their key raises)."""
        t = self.t
        if self.rank == 0:
            return
        if self.kind == "turbo":
            # the turbo step reads U by local cluster: gather the pool rows once
            for proj in PROJS:
                if proj not in pools:
                    continue
                rows = []
                for key in t[f"ckeys_{proj}"]:
                    if key[0] != "c" or key[1] not in id_maps[proj]:
                        raise RuntimeError(f"{proj}: cluster {key} is not in the pool")
                    rows.append(int(id_maps[proj][key[1]]))
                idx = torch.tensor(rows, dtype=torch.long, device=pools[proj].device)
                t[f"U_{proj}"] = pools[proj].index_select(0, idx).contiguous()
            _turbo_derived(t)
            return
        for proj in PROJS:
            if proj not in pools:
                continue
            keys = t.get(f"ckeys_{proj}")
            if keys is None:
                raise RuntimeError("set_global_pool needs a block built from GLoRCQLinear experts")
            pool = pools[proj]
            if pool.dim() != 3 or pool.shape[1:] != t[f"U_{proj}"].shape[1:]:
                raise RuntimeError(f"{proj} pool must be (rows, K, r) = (*, "
                                   f"{tuple(t[f'U_{proj}'].shape[1:])})")
            rows = []
            for key in keys:
                if key[0] != "c" or key[1] not in id_maps[proj]:
                    raise RuntimeError(f"{proj}: cluster {key} is not in the pool")
                rows.append(int(id_maps[proj][key[1]]))
            dev = pool.device
            slot = torch.tensor(rows, dtype=torch.int32, device=dev)
            t[f"U_{proj}"] = pool.contiguous()
            t[f"urows_{proj}"] = int(pool.shape[0])
            if proj == "down":  # cluster_of indexes the pool directly
                t["cluster_down"] = slot[t["cluster_down"].long()].contiguous()
            else:
                t[f"uslot_{proj}"] = slot

    # ---- the step ----
    def _op_args(self):
        """The block's tensors as the list arguments of the glorcq_hip MoE ops."""
        t = self.t
        lora = self.rank > 0
        codes = [t[f"codes_{p}"] for p in PROJS]
        scales = [t[f"scales_{p}"] for p in PROJS]
        zeros = [t[f"zeros_{p}"] for p in PROJS]
        U = [t[f"U_{p}"] for p in PROJS] if lora else []
        cl = [t[f"cluster_{p}"] for p in PROJS] if lora else []
        SV = [t[f"SV_{p}"] for p in PROJS] if lora else []
        u_slot = [t.get(f"uslot_{p}") for p in ("gate", "up")] if lora else []
        u_rows = [int(t.get(f"urows_{p}", 0)) for p in PROJS] if lora else []
        shared = self.shared_inter > 0
        sc = [t[f"scodes_{p}"] for p in PROJS] if shared else []
        ss = [t[f"sscales_{p}"] for p in PROJS] if shared else []
        sz = [t[f"szeros_{p}"] for p in PROJS] if shared else []
        return codes, scales, zeros, U, cl, SV, u_slot, u_rows, sc, ss, sz

    MAX_TOKENS = 64  # tokens per decode step (glq_moe_decode)

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor | None = None):
        """(final (b, s, H) fp16, router_logits (b*s, E) fp16), as the
        reference's forward (moe_block.py:381-436); final alone when
        return_router_logits is False.  Up to 64 tokens run as one decode step
        (glorcq_hip::moe_decode); more (a prefill) run through
        glorcq_hip::moe_prefill.
        residual (the shape of hidden_states, fp16): final becomes
        fp16(residual + fp16(block output)), the decoder layer's residual add,
        inside the step's last launch."""
        shape = hidden_states.shape
        h = hidden_states.reshape(-1, self.hidden)
        if h.dtype != torch.float16:
            h = h.half()
        h = h.contiguous()
        if not h.is_cuda:
            raise RuntimeError("hidden_states must be on the GPU")
        res = None
        if residual is not None:
            if residual.shape != hidden_states.shape or residual.dtype != torch.float16:
                raise RuntimeError("residual must match hidden_states (fp16)")
            res = residual.reshape(-1, self.hidden).contiguous()
        t = self.t
        if self.kind == "turbo":
            outs, logits = [], []
            for t0 in range(0, h.shape[0], TURBO_MAX_TOKENS):
                t1 = min(h.shape[0], t0 + TURBO_MAX_TOKENS)
                o, lg = turbo_step(self, h[t0:t1].contiguous(),
                                   None if res is None else res[t0:t1].contiguous())
                outs.append(o)
                logits.append(lg)
            out = outs[0] if len(outs) == 1 else torch.cat(outs)
            lg = logits[0] if len(logits) == 1 else torch.cat(logits)
            out = out.reshape(shape)
            return (out, lg) if self.return_router_logits else out
        codes, scales, zeros, U, cl, SV, u_slot, u_rows, sc, ss, sz = self._op_args()
        if h.shape[0] <= self.MAX_TOKENS:
            out, logits = torch.ops.glorcq_hip.moe_decode(
                h, t["router_w"], t["shared_gate_w"], codes, scales, zeros, U, cl, SV, u_slot,
                u_rows, sc, ss, sz, res, self.inter, self.top_k, self.norm_topk_prob, self.rank,
                self.n_clusters, self.bits, self.shared_bits, self.shared_inter)
        else:
            out, logits = torch.ops.glorcq_hip.moe_prefill(
                h, t["router_w"], t["shared_gate_w"], codes, scales, zeros, U, cl, SV, u_slot,
                u_rows, sc, ss, sz, res, self.inter, self.top_k, self.norm_topk_prob, self.rank,
                self.n_clusters, self.bits, self.shared_bits, self.shared_inter,
                self.zeros_integral)
        out = out.reshape(shape)
        return (out, logits) if self.return_router_logits else out

    def extra_repr(self):
        kind = "turbo" if self.kind == "turbo" else f"bits={self.bits}"
        return (f"experts={self.num_experts}, top_k={self.top_k}, hidden={self.hidden}, "
                f"inter={self.inter}, {kind}, rank={self.rank}, "
                f"clusters={self.n_clusters}, shared_inter={self.shared_inter}")


# ---------------------------------------------------------------------------
# TurboQuant routed experts
# ---------------------------------------------------------------------------
TURBO_MAX_TOKENS = 16  # tokens per turbo step (the cluster-shared x U takes <= 16 rows)
# Tokens up to which the fused turbo step runs the shared expert inside its
# launches (measured, config 2 with turbo experts: B = 1 59.3 -> 42.7 us,
# B = 4 77.6 -> 69.5 us, B = 16 128.3 -> 147.4 us)
TURBO_SHARED_LANE_MAX_B = 4


def _turbo_rotation(lins, proj):
    """(signs, Pi, centroids) of one projection's experts, which must share one
    (dim, bits, seed) configuration (the reference's rotation-cache key,
    moe_block.py:331-357)."""
    l0 = lins[0]
    key = (l0.turbo_dim, l0.turbo_bits, l0.turbo_seed)
    for lin in lins:
        if (lin.turbo_dim, lin.turbo_bits, lin.turbo_seed) != key:
            raise RuntimeError(f"{proj}: experts need one TurboQuant (dim, bits, seed)")
        if (lin._rht_signs is None) != (l0._rht_signs is None):
            raise RuntimeError(f"{proj}: experts need one rotation kind (RHT or Pi)")
    cent = l0._rotation_cache.get_centroids(*key).float().contiguous()
    if l0._rht_signs is not None:
        return l0._rht_signs.float().contiguous(), None, cent
    return None, l0._rotation_cache.get_pi(*key).contiguous(), cent


def _stack_turbo_block(blk) -> dict:
    """Stacks a block whose routed experts are TurboQuant GLoRCQLinear layers;
    the shared expert keeps its own projections (any GLoRCQLinear kind)."""
    experts = list(blk.experts)
    E = len(experts)
    lin0 = experts[0].gate_proj
    dev = lin0.turbo_words.device
    out = {"kind": "turbo", "E": E, "top_k": int(blk.top_k),
           "norm_topk_prob": bool(getattr(blk, "norm_topk_prob", False)),
           "H": lin0.in_features, "inter": lin0.out_features, "rank": lin0.rank}
    out["router_w"] = blk.gate.weight.detach().to(dev, torch.float16).contiguous()
    n_clusters = 0
    for proj in PROJS:
        lins = [getattr(ex, _PROJ_ATTR[proj]) for ex in experts]
        for lin in lins:
            if lin.quant_type != "turbo":
                raise RuntimeError("routed experts must all be TurboQuant or all GPTQ")
            if lin.rank != out["rank"]:
                raise RuntimeError("all experts need one LoRA rank")
            if getattr(lin, "bias_param", None) is not None:
                raise RuntimeError("TurboQuant MoE experts take no bias")
        out[f"words_{proj}"] = _stack([lin.turbo_words for lin in lins])
        out[f"norms_{proj}"] = _stack([lin.norms for lin in lins])
        signs, Pi, cent = _turbo_rotation(lins, proj)
        out[f"signs_{proj}"], out[f"Pi_{proj}"], out[f"cent_{proj}"] = signs, Pi, cent
        if out["rank"] > 0:
            ids, pool, cl = {}, [], []
            for e, lin in enumerate(lins):
                key = ("c", lin.cluster_id) if lin.cluster_id is not None else ("e", e)
                if key not in ids:
                    ids[key] = len(pool)
                    pool.append(lin.U)
                cl.append(ids[key])
            out[f"U_{proj}"] = _stack(pool)
            out[f"cluster_{proj}"] = torch.tensor(cl, dtype=torch.int32, device=dev)
            out[f"ckeys_{proj}"] = list(ids.keys())
            out[f"SV_{proj}"] = _stack([lin.SV for lin in lins])
            n_clusters = max(n_clusters, len(pool))
    out["n_clusters"] = n_clusters
    sh = getattr(blk, "shared_expert", None)
    if sh is not None:
        out["shared_mods"] = tuple(getattr(sh, _PROJ_ATTR[p]) for p in PROJS)
        out["shared_inter"] = out["shared_mods"][0].out_features
        g = getattr(blk, "shared_expert_gate", None)
        out["shared_gate_w"] = (None if g is None else
                                g.weight.detach().reshape(-1).to(dev, torch.float16).contiguous())
    else:
        out["shared_inter"], out["shared_gate_w"] = 0, None
    out["shared_bits"] = 0
    out["same_rot_gu"] = _same_rotation(out)
    _turbo_derived(out)
    return out


def _turbo_from_problem(p: MoEProblem, d) -> dict:
    """Turbo block tensors from a format.MoEProblem whose experts are
    format.TurboMat (the shared expert, if any, a GPTQ format.QMat)."""
    t = {"kind": "turbo", "E": p.E, "top_k": p.top_k, "norm_topk_prob": p.norm_topk_prob,
         "H": p.H, "inter": p.inter, "rank": p.rank, "n_clusters": p.n_clusters,
         "router_w": p.router_w.to(d).contiguous(), "shared_bits": 0}
    for proj in PROJS:
        q = p.experts[proj]
        t[f"words_{proj}"] = q.words().to(d).contiguous()
        t[f"norms_{proj}"] = q.norms.to(d, torch.float32).contiguous()
        t[f"cent_{proj}"] = q.centroids.to(d, torch.float32).contiguous()
        t[f"signs_{proj}"] = None if q.signs is None else q.signs.to(d, torch.float32).contiguous()
        t[f"Pi_{proj}"] = None if q.Pi is None else q.Pi.to(d, torch.float16).contiguous()
        if p.rank > 0:
            t[f"U_{proj}"] = p.U[proj].to(d).contiguous()
            t[f"cluster_{proj}"] = p.cluster_of[proj].to(d, torch.int32).contiguous()
            t[f"SV_{proj}"] = p.SV[proj].to(d).contiguous()
            t[f"ckeys_{proj}"] = [("c", c) for c in range(p.n_clusters)]
    if p.shared is not None:
        t["shared_q"] = {proj: (p.shared[proj].codes[0].to(d).contiguous(),
                                p.shared[proj].scales[0].to(d).contiguous(),
                                p.shared[proj].zeros[0].to(d).contiguous(),
                                p.shared[proj].bits) for proj in PROJS}
        t["shared_inter"] = p.shared["gate"].N
        t["shared_gate_w"] = p.shared_gate_w.reshape(-1).to(d).contiguous()
    else:
        t["shared_inter"], t["shared_gate_w"] = 0, None
    t["same_rot_gu"] = _same_rotation(t)
    _turbo_derived(t)
    return t


def _turbo_derived(t: dict) -> None:
    """Tensors the turbo step reads that follow from the block's own: Pi^T per
    QR-rotated projection (x Pi^T as one fp16 GEMM with fp32 accumulation),
    down's Pi as fp16 rows, and the gate and up U stacked (one x U launch for
    both)."""
    for proj in PROJS:
        Pi = t[f"Pi_{proj}"]
        t[f"PiT_{proj}"] = None if Pi is None else Pi.t().contiguous()
    # Pi of down as fp16 rows (output n's weights contiguous), for
    # glq_turbo_moe_down_prep
    Pd = t["Pi_down"]
    t["Pi_down_c"] = None if Pd is None else Pd.to(torch.float16).contiguous()
    if t["rank"] > 0:
        t["U_gu"] = torch.cat([t["U_gate"], t["U_up"]]).contiguous()


def _same_rotation(t: dict) -> bool:
    """gate and up rotate x alike (one x_rot serves both); checked once, at
    construction, so a step makes no host sync."""
    sg, su, pg, pu = t["signs_gate"], t["signs_up"], t["Pi_gate"], t["Pi_up"]
    if sg is not None and su is not None:
        return sg is su or bool(torch.equal(sg, su))
    if pg is not None and pu is not None:
        return pg is pu or bool(torch.equal(pg, pu))
    return False


# routing workspaces: (device index, stream handle) -> zero-filled uint8 tensor
_route_ws: dict = {}


def _rotate(x: torch.Tensor, signs, PiT) -> torch.Tensor:
    """x_rot = fp16(RHT(x)) (one glq_rht launch) or x Pi^T as one library GEMM
    of the fp16 operands with fp32 accumulation, rounded once to fp16 (the
    reference's fp16(x.float() @ Pi.float().T), moe_block.py:352-356: the
    products of fp16 values are exact in fp32 either way)."""
    from .kernels import _rht_eager
    if signs is not None:
        return _rht_eager(x, signs)
    return torch.matmul(x, PiT)


_side_streams: dict = {}


def _side_stream(dev) -> torch.cuda.Stream:
    """One side stream per device (default priority), for the shared expert."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _side_streams.get(idx)
    if st is None:
        st = torch.cuda.Stream(device=dev)
        _side_streams[idx] = st
    return st


def _turbo_shared_expert(t: dict, h: torch.Tensor, lib) -> torch.Tensor:
    """down(fp16(silu(gate(h))) * up(h)) of the shared expert on the current
    stream: its own GLoRCQLinear projections, or the problem's GPTQ weights."""
    from .kernels import _packed_dequant_matmul_eager
    if "shared_mods" in t:
        mg, mu, md = t["shared_mods"]
        sgo, suo = mg(h), mu(h)
    else:
        q = t["shared_q"]
        sgo = _packed_dequant_matmul_eager(h, q["gate"][0], q["gate"][1], q["gate"][2],
                                           q["gate"][3], 128)
        suo = _packed_dequant_matmul_eager(h, q["up"][0], q["up"][1], q["up"][2],
                                           q["up"][3], 128)
    si = torch.empty_like(sgo)
    _lib.check(lib.glq_swiglu(sgo.data_ptr(), suo.data_ptr(), si.numel(), si.data_ptr(),
                              _lib.stream_handle(h.device)), "glq_swiglu")
    if "shared_mods" in t:
        return t["shared_mods"][2](si).contiguous()
    q = t["shared_q"]
    return _packed_dequant_matmul_eager(si, q["down"][0], q["down"][1], q["down"][2],
                                        q["down"][3], 128)


def _turbo_fused_ok(blk: GraphCompatibleMoeBlock, B: int) -> bool:
    """The four-launch form of the turbo step (turbo_step_fused) takes this
    block: gate and up rotated alike (by one transform, or by one Pi), the
    down by a transform or a Pi of a 32-multiple width, a rank that is a
    multiple of 8 (or none), at most 16 tokens."""
    t = blk.t
    if os.environ.get("GLQ_TURBO_SEQ") or B > 16 or not t["same_rot_gu"]:
        return False
    if blk.rank and blk.rank % 8:
        return False
    if t["signs_down"] is None and (t["Pi_down"] is None or blk.inter % 32):
        return False
    return True


def _route_workspace(dev, stream, B, E, lib) -> torch.Tensor:
    n = lib.glq_moe_route_workspace_bytes(B, E)
    key = (dev.index, stream)
    ws = _route_ws.get(key)
    if ws is None or ws.numel() < n:
        retire_workspace(ws)  # a captured graph may still use it
        ws = torch.zeros(max(int(n), 256), dtype=torch.uint8, device=dev)  # counters start at zero
        _route_ws[key] = ws
    return ws


def _turbo_mat(x_rot, t, proj, parts, cluster, blocks) -> _lib.TurboMat:
    m = _lib.TurboMat()
    m.x_rot, m.codes = x_rot.data_ptr(), t[f"words_{proj}"].data_ptr()
    m.norms, m.centroids = t[f"norms_{proj}"].data_ptr(), t[f"cent_{proj}"].data_ptr()
    m.SV = _lib.ptr(t.get(f"SV_{proj}"))
    m.parts, m.cluster, m.blocks = parts, _lib.ptr(cluster), blocks
    return m


def _turbo_shared_weights(t: dict):
    """(codes, scales, zeros) of the shared expert's gate, up, down when they
    can ride in the fused step's launches (4-bit unsigned codes with
    zero-points, group 128, no low-rank term or bias), else None."""
    if "shared_q" in t:
        q = t["shared_q"]
        if any(q[p][3] != 4 for p in PROJS):
            return None
        return [tuple(q[p][i] for p in PROJS) for i in range(3)]
    if "shared_mods" in t:
        ms = t["shared_mods"]
        for m in ms:
            if (getattr(m, "quant_type", None) != "gptq" or m.pack_bits != 4 or m.gptq_sym
                    or m.gptq_groupsize != 128 or m.SV is not None or m.bias_param is not None
                    or m.zeros is None):
                return None
        return [tuple(m.codes for m in ms), tuple(m.scales for m in ms),
                tuple(m.zeros for m in ms)]
    return None


def turbo_step_fused(blk: GraphCompatibleMoeBlock, h: torch.Tensor, res: torch.Tensor | None):
    """turbo_step in four launches: glq_turbo_moe_prep (routing, gate/up's
    transform of h, every gate/up cluster's x U partials, the shared expert's
    gate/up rows), glq_turbo_moe_gemv2 as the gate/up pair (SwiGLU inter),
    glq_turbo_moe_down_prep (the down's input rotation, each pick's x U
    partials, the shared expert's down rows), glq_turbo_moe_gemv2 for down;
    then the combine.  The same arithmetic as turbo_step's launches except for
    the order of the Pi rotation's fp32 sums and the shared down's sums (the
    lane form's instead of the streaming kernel's).  A shared expert that
    cannot ride in the launches runs on a side stream as in turbo_step."""
    lib = _lib.load()
    t = blk.t
    dev = h.device
    B, H = h.shape
    E, k, I, r = blk.num_experts, blk.top_k, blk.inter, blk.rank
    P = B * k
    stream = _lib.stream_handle(dev)
    shared = side = sh = None
    # the shared expert in the launches' lane form up to TURBO_SHARED_LANE_MAX_B
    # tokens (each token decodes its codes again), on the side stream above
    sw = (_turbo_shared_weights(t) if 0 < blk.shared_inter and B <= TURBO_SHARED_LANE_MAX_B
          else None)
    if sw is not None:
        SI = blk.shared_inter
        sh = _lib.MoeShared()
        for i in range(3):
            sh.codes[i], sh.scales[i], sh.zeros[i] = (sw[0][i].data_ptr(), sw[1][i].data_ptr(),
                                                      sw[2][i].data_ptr())
        sh.inter, sh.bits = SI, 4
        sinter = torch.empty(B, SI, dtype=torch.float16, device=dev)
        shared = torch.empty(B, H, dtype=torch.float16, device=dev)
        sh.sinter, sh.sy = sinter.data_ptr(), shared.data_ptr()
    elif blk.shared_inter > 0:
        cur = torch.cuda.current_stream(dev)
        side = _side_stream(dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            shared = _turbo_shared_expert(t, h, lib)
    shp = ctypes.byref(sh) if sh is not None else None
    sel = torch.empty(P, dtype=torch.int32, device=dev)
    wts = torch.empty(P, dtype=torch.float16, device=dev)
    sg = torch.empty(B, dtype=torch.float16, device=dev)
    logits = torch.empty(B, E, dtype=torch.float16, device=dev)
    ws = _route_workspace(dev, stream, B, E, lib)
    signs = t["signs_gate"]
    xg = torch.empty(B, H, dtype=torch.float16, device=dev) if signs is not None \
        else _rotate(h, None, t["PiT_gate"])
    rpad = (r + 31) // 32 * 32
    S_h = (H + 255) // 256
    parts = None
    n_u = 0
    if r:
        n_u = t["U_gu"].shape[0]
        parts = torch.empty(n_u, S_h, B, rpad, dtype=torch.float32, device=dev)
    _lib.check(lib.glq_turbo_moe_prep(
        h.data_ptr(), t["router_w"].data_ptr(), _lib.ptr(t["shared_gate_w"]), B, H, E, k,
        int(blk.norm_topk_prob), sel.data_ptr(), wts.data_ptr(), sg.data_ptr(), logits.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.ptr(signs), xg.data_ptr(),
        _lib.ptr(t["U_gu"] if r else None), n_u, r, _lib.ptr(parts), shp, stream),
        "glq_turbo_moe_prep")
    cg = t["U_gate"].shape[0] if r else 0
    pp = parts.data_ptr() if r else None
    gm = _turbo_mat(xg, t, "gate", pp, t.get("cluster_gate"), max(cg, 1))
    um = _turbo_mat(xg, t, "up", pp + cg * S_h * B * rpad * 4 if r else None,
                    t.get("cluster_up"), max(n_u - cg, 1))
    inter = torch.empty(P, I, dtype=torch.float16, device=dev)
    _lib.check(lib.glq_turbo_moe_gemv2(P, k, H, I, E, sel.data_ptr(), ctypes.byref(gm),
                                       ctypes.byref(um), r, S_h, inter.data_ptr(), stream),
               "glq_turbo_moe_gemv2")
    xd = torch.empty(P, I, dtype=torch.float16, device=dev)
    S_i = (I + 255) // 256
    parts_d = torch.empty(P, S_i, 1, rpad, dtype=torch.float32, device=dev) if r else None
    Ud = t.get("U_down") if r else None
    _lib.check(lib.glq_turbo_moe_down_prep(
        P, I, inter.data_ptr(), _lib.ptr(t.get("Pi_down_c") if t["signs_down"] is None else None),
        _lib.ptr(t["signs_down"]), xd.data_ptr(), _lib.ptr(Ud), Ud.shape[0] if r else 0,
        _lib.ptr(t.get("cluster_down") if r else None), sel.data_ptr(), E, r,
        _lib.ptr(parts_d), B, H, shp, stream), "glq_turbo_moe_down_prep")
    dm = _turbo_mat(xd, t, "down", _lib.ptr(parts_d), None, P)
    yd = torch.empty(P, H, dtype=torch.float16, device=dev)
    _lib.check(lib.glq_turbo_moe_gemv2(P, 1, I, H, E, sel.data_ptr(), ctypes.byref(dm), None, r,
                                       S_i, yd.data_ptr(), stream), "glq_turbo_moe_gemv2")
    if side is not None:
        cur.wait_stream(side)
        shared.record_stream(cur)
    out = torch.empty(B, H, dtype=torch.float16, device=dev)
    _lib.check(lib.glq_moe_combine(yd.data_ptr(), wts.data_ptr(), _lib.ptr(shared), sg.data_ptr(),
                                   _lib.ptr(res), B, H, k, out.data_ptr(), stream),
               "glq_moe_combine")
    return out, logits


def turbo_step(blk: GraphCompatibleMoeBlock, h: torch.Tensor, res: torch.Tensor | None):
    """One decode step of a TurboQuant block (<= TURBO_MAX_TOKENS tokens):
    (out (B, H) fp16, router logits (B, E) fp16).  turbo_step_fused when it
    takes the block, else this launch sequence."""
    if _turbo_fused_ok(blk, h.shape[0]):
        return turbo_step_fused(blk, h, res)
    from .kernels import _lowrank_xu_eager, workspace
    lib = _lib.load()
    t = blk.t
    dev = h.device
    B, H = h.shape
    E, k, I, r = blk.num_experts, blk.top_k, blk.inter, blk.rank
    P = B * k
    stream = _lib.stream_handle(dev)
    # 0. the shared expert (routing-independent) on a side stream, overlapping
    # the routed chain (the reference's side-stream overlap, moe_block.py:
    # 661-700); the combine joins it
    shared = side = None
    if blk.shared_inter > 0:
        cur = torch.cuda.current_stream(dev)
        side = _side_stream(dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            shared = _turbo_shared_expert(t, h, lib)
    # 1. routing on the device
    sel = torch.empty(P, dtype=torch.int32, device=dev)
    wts = torch.empty(P, dtype=torch.float16, device=dev)
    sg = torch.empty(B, dtype=torch.float16, device=dev)
    logits = torch.empty(B, E, dtype=torch.float16, device=dev)
    ws = _route_workspace(dev, stream, B, E, lib)
    _lib.check(lib.glq_moe_route(h.data_ptr(), t["router_w"].data_ptr(),
                                 _lib.ptr(t["shared_gate_w"]), B, H, E, k,
                                 int(blk.norm_topk_prob), sel.data_ptr(), wts.data_ptr(),
                                 sg.data_ptr(), logits.data_ptr(), ws.data_ptr(), ws.numel(),
                                 stream), "glq_moe_route")

    def gemv(x_rot, x_div, K, N, proj, xU, xclus, xtok, xrows, gate, y):
        _lib.check(lib.glq_turbo_moe_gemv(
            P, x_div, x_rot.data_ptr(), K, N, E, sel.data_ptr(), t[f"words_{proj}"].data_ptr(),
            t[f"norms_{proj}"].data_ptr(), t[f"cent_{proj}"].data_ptr(), _lib.ptr(xU),
            _lib.ptr(xclus), xtok, xrows, _lib.ptr(t.get(f"SV_{proj}")) if r else None, r, None,
            _lib.ptr(gate), y.data_ptr(), stream), "glq_turbo_moe_gemv")

    # 2. gate and up: x rotated once per configuration, x U once per cluster
    xg = _rotate(h, t["signs_gate"], t["PiT_gate"])
    xu_ = xg if t["same_rot_gu"] else _rotate(h, t["signs_up"], t["PiT_up"])
    ag = au = None
    if r:
        agu = _lowrank_xu_eager(h, t["U_gu"])  # (Cg + Cu, B, r): gate's clusters, then up's
        cg = t["U_gate"].shape[0]
        ag, au = agu[:cg], agu[cg:]
    g = torch.empty(P, I, dtype=torch.float16, device=dev)
    gemv(xg, k, H, I, "gate", ag, t.get("cluster_gate"), B, 0 if ag is None else ag.shape[0] * B,
         None, g)
    inter = torch.empty(P, I, dtype=torch.float16, device=dev)
    gemv(xu_, k, H, I, "up", au, t.get("cluster_up"), B, 0 if au is None else au.shape[0] * B,
         g, inter)
    # 3. down: inter rotated, each pick's own a_down = fp16(inter U_c)
    xd = _rotate(inter, t["signs_down"], t["PiT_down"])
    ad = None
    if r:
        ad = torch.empty(P, r, dtype=torch.float16, device=dev)
        nb = lib.glq_lowrank_workspace_bytes(P, 1, I, r)
        wl = workspace(dev, max(int(nb), 256))
        U = t["U_down"]
        _lib.check(lib.glq_lowrank_xu_routed(P, inter.data_ptr(), I, U.data_ptr(), U.shape[0], r,
                                             sel.data_ptr(), E, t["cluster_down"].data_ptr(),
                                             ad.data_ptr(), wl.data_ptr(), wl.numel(), stream),
                   "glq_lowrank_xu_routed")
    yd = torch.empty(P, H, dtype=torch.float16, device=dev)
    gemv(xd, 1, I, H, "down", ad, None, 0, 0, None, yd)
    # 4. the combine, after the shared expert's stream has joined
    if side is not None:
        cur.wait_stream(side)
        shared.record_stream(cur)
    out = torch.empty(B, H, dtype=torch.float16, device=dev)
    _lib.check(lib.glq_moe_combine(yd.data_ptr(), wts.data_ptr(), _lib.ptr(shared), sg.data_ptr(),
                                   _lib.ptr(res), B, H, k, out.data_ptr(), stream),
               "glq_moe_combine")
    return out, logits


# ---------------------------------------------------------------------------
# Real kernels of the glorcq_hip MoE operators (glorcq_amd/ops.py)
# ---------------------------------------------------------------------------
# decode workspaces: (device index, stream handle, tokens) -> zero-filled
# uint8 tensor.  Each step leaves the router's arrival counter zero again and
# steps on one stream run in order, so every block of a model shares them.
_moe_ws: dict = {}


def _moe_params(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV, u_slot,
                u_rows, shared_codes, shared_scales, shared_zeros, residual, out, logits,
                inter, top_k, norm_topk_prob, rank, n_clusters, bits, shared_bits,
                shared_inter) -> _lib.MoeParams:
    P = _lib.MoeParams()
    P.tokens, P.hidden, P.experts, P.inter = h.shape[0], h.shape[1], router_w.shape[0], inter
    P.top_k, P.n_clusters, P.rank = top_k, n_clusters, rank
    P.shared_inter = shared_inter
    P.norm_topk_prob = int(bool(norm_topk_prob))
    P.bits, P.shared_bits, P.group = bits, shared_bits or 4, 128
    P.h, P.router_w = h.data_ptr(), router_w.data_ptr()
    P.shared_gate_w = _lib.ptr(shared_gate_w)
    if len(codes) != 3 or len(scales) != 3 or len(zeros) != 3:
        raise RuntimeError("codes, scales and zeros hold (gate, up, down)")
    for i in range(3):
        P.codes[i] = codes[i].data_ptr()
        P.scales[i] = scales[i].data_ptr()
        P.zeros[i] = zeros[i].data_ptr()
        if rank > 0:
            P.U[i] = U[i].data_ptr()
            P.cluster_of[i] = cluster_of[i].data_ptr()
            P.SV[i] = SV[i].data_ptr()
            P.u_rows[i] = u_rows[i] if u_rows else 0
            if i < 2 and u_slot:
                P.u_slot[i] = _lib.ptr(u_slot[i])
        if shared_inter > 0:
            P.shared_codes[i] = shared_codes[i].data_ptr()
            P.shared_scales[i] = shared_scales[i].data_ptr()
            P.shared_zeros[i] = shared_zeros[i].data_ptr()
    P.out = out.data_ptr()
    P.router_logits = _lib.ptr(logits)
    P.residual = _lib.ptr(residual)
    return P


def moe_decode_launch(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV,
                      u_slot, u_rows, shared_codes, shared_scales, shared_zeros, residual, inter,
                      top_k, norm_topk_prob, rank, n_clusters, bits, shared_bits, shared_inter,
                      out=None, logits=None):
    """One glq_moe_decode step (<= 64 tokens) on torch's current stream."""
    lib = _lib.load()
    if h.dim() != 2 or h.dtype != torch.float16 or not h.is_contiguous():
        raise RuntimeError("h must be contiguous fp16 (tokens, hidden)")
    if out is None:
        out = torch.empty_like(h)
    if logits is None:
        logits = torch.empty(h.shape[0], router_w.shape[0], dtype=torch.float16,
                             device=h.device)
    P = _moe_params(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV, u_slot,
                    u_rows, shared_codes, shared_scales, shared_zeros, residual, out, logits,
                    inter, top_k, norm_topk_prob, rank, n_clusters, bits, shared_bits,
                    shared_inter)
    n = lib.glq_moe_workspace_bytes(ctypes.byref(P))
    if n < 0:
        _lib.check(1, "glq_moe_workspace_bytes")
    stream = _lib.stream_handle(h.device)
    key = (h.device.index, stream, h.shape[0])
    ws = _moe_ws.get(key)
    if ws is None or ws.numel() < n:
        # zero-filled once: the router's arrival counter starts at zero and
        # every step leaves it zero; a replaced buffer stays alive for the
        # graphs captured with it
        retire_workspace(ws)
        ws = torch.zeros(max(int(n), 256), dtype=torch.uint8, device=h.device)
        _moe_ws[key] = ws
    _lib.check(lib.glq_moe_decode(ctypes.byref(P), ws.data_ptr(), ws.numel(), stream),
               "glq_moe_decode")
    return out, logits


def moe_prefill_launch(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV,
                       u_slot, u_rows, shared_codes, shared_scales, shared_zeros, residual, inter,
                       top_k, norm_topk_prob, rank, n_clusters, bits, shared_bits, shared_inter,
                       zeros_integral=True):
    """A block over many tokens: glq_moe_prefill (grouped GEMMs over each
    expert's gathered tokens); blocks whose routed zero-points are not all
    integers run consecutive 64-token decode steps instead."""
    out = torch.empty_like(h)
    logits = torch.empty(h.shape[0], router_w.shape[0], dtype=torch.float16, device=h.device)
    if not zeros_integral:
        step = GraphCompatibleMoeBlock.MAX_TOKENS
        for t0 in range(0, h.shape[0], step):
            t1 = min(h.shape[0], t0 + step)
            moe_decode_launch(h[t0:t1], router_w, shared_gate_w, codes, scales, zeros, U,
                              cluster_of, SV, u_slot, u_rows, shared_codes, shared_scales,
                              shared_zeros, None if residual is None else residual[t0:t1], inter,
                              top_k, norm_topk_prob, rank, n_clusters, bits, shared_bits,
                              shared_inter, out=out[t0:t1], logits=logits[t0:t1])
        return out, logits
    lib = _lib.load()
    if h.dim() != 2 or h.dtype != torch.float16 or not h.is_contiguous():
        raise RuntimeError("h must be contiguous fp16 (tokens, hidden)")
    P = _moe_params(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV, u_slot,
                    u_rows, shared_codes, shared_scales, shared_zeros, residual, out, logits,
                    inter, top_k, norm_topk_prob, rank, n_clusters, bits, shared_bits,
                    shared_inter)
    n = lib.glq_moe_prefill_workspace_bytes(ctypes.byref(P))
    if n < 0:
        _lib.check(1, "glq_moe_prefill_workspace_bytes")
    from .kernels import workspace
    ws = workspace(h.device, max(int(n), 256))
    _lib.check(lib.glq_moe_prefill(ctypes.byref(P), ws.data_ptr(), ws.numel(),
                                   _lib.stream_handle(h.device)), "glq_moe_prefill")
    return out, logits
