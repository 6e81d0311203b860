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
* GPTQ layers only (asymmetric, group 128, 2- or 4-bit containers).
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn

from . import _lib
from .format import PROJS, MoEProblem

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
        self.num_experts = stacked["E"]
        self.top_k = stacked["top_k"]
        self.norm_topk_prob = bool(stacked["norm_topk_prob"])
        self.hidden = stacked["H"]
        self.inter = stacked["inter"]
        self.rank = stacked["rank"]
        self.n_clusters = stacked["n_clusters"]
        self.bits = stacked["bits"]
        self.shared_bits = stacked["shared_bits"]
        self.shared_inter = stacked["shared_inter"]
        self.group = 128
        self.graph_mode = True  # every step is graph-safe
        # forward returns (final, router_logits) as the reference's block does
        # (transformers 4.x decoder layers unpack the pair); False returns final
        # alone, the contract of transformers 5 sparse-MoE blocks
        self.return_router_logits = True
        self.t = stacked  # device tensors (kept alive for the kernels)
        self._ws: dict = {}

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
    def _params(self, h, out, logits) -> _lib.MoeParams:
        t = self.t
        P = _lib.MoeParams()
        P.tokens, P.hidden, P.experts, P.inter = h.shape[0], self.hidden, self.num_experts, \
            self.inter
        P.top_k, P.n_clusters, P.rank = self.top_k, self.n_clusters, self.rank
        P.shared_inter = self.shared_inter
        P.norm_topk_prob = int(self.norm_topk_prob)
        P.bits, P.shared_bits, P.group = self.bits, self.shared_bits or 4, self.group
        P.h, P.router_w = h.data_ptr(), t["router_w"].data_ptr()
        P.shared_gate_w = _lib.ptr(t["shared_gate_w"])
        for i, proj in enumerate(PROJS):
            P.codes[i] = t[f"codes_{proj}"].data_ptr()
            P.scales[i] = t[f"scales_{proj}"].data_ptr()
            P.zeros[i] = t[f"zeros_{proj}"].data_ptr()
            if self.rank > 0:
                P.U[i] = t[f"U_{proj}"].data_ptr()
                P.cluster_of[i] = t[f"cluster_{proj}"].data_ptr()
                P.SV[i] = t[f"SV_{proj}"].data_ptr()
                P.u_rows[i] = t.get(f"urows_{proj}", 0)
                if i < 2:
                    P.u_slot[i] = _lib.ptr(t.get(f"uslot_{proj}"))
            if self.shared_inter > 0:
                P.shared_codes[i] = t[f"scodes_{proj}"].data_ptr()
                P.shared_scales[i] = t[f"sscales_{proj}"].data_ptr()
                P.shared_zeros[i] = t[f"szeros_{proj}"].data_ptr()
        P.out = out.data_ptr()
        P.router_logits = _lib.ptr(logits)
        return P

    def _workspace(self, lib, P) -> torch.Tensor:
        B = P.tokens
        ws = self._ws.get(B)
        if ws is None:
            n = lib.glq_moe_workspace_bytes(ctypes.byref(P))
            if n < 0:
                _lib.check(1, "glq_moe_workspace_bytes")
            # zero-filled once: its router arrival counter starts at zero and
            # every step leaves it zero
            ws = torch.zeros(max(int(n), 256), dtype=torch.uint8,
                             device=self.t["router_w"].device)
            self._ws[B] = ws
        return ws

    MAX_TOKENS = 64  # tokens per glq_moe_decode call

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor | None = None):
        """(final (b, s, H) fp16, router_logits (b*s, E) fp16), as the
        reference's forward (moe_block.py:381-436); final alone when
        return_router_logits is False.  Tokens are independent in the block,
        so more than 64 (a prefill) run as consecutive 64-token steps.
        residual (the shape of hidden_states, fp16): final becomes
        fp16(residual + fp16(block output)), the decoder layer's residual add,
        inside the step's last launch."""
        lib = _lib.load()
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
        out = torch.empty_like(h)
        logits = torch.empty(h.shape[0], self.num_experts, dtype=torch.float16, device=h.device)
        stream = _lib.stream_handle(h.device)
        for t0 in range(0, h.shape[0], self.MAX_TOKENS):
            t1 = min(h.shape[0], t0 + self.MAX_TOKENS)
            P = self._params(h[t0:t1], out[t0:t1], logits[t0:t1])
            P.residual = _lib.ptr(None if res is None else res[t0:t1])
            ws = self._workspace(lib, P)
            rc = lib.glq_moe_decode(ctypes.byref(P), ws.data_ptr(), ws.numel(), stream)
            _lib.check(rc, "glq_moe_decode")
        out = out.reshape(shape)
        return (out, logits) if self.return_router_logits else out

    def extra_repr(self):
        return (f"experts={self.num_experts}, top_k={self.top_k}, hidden={self.hidden}, "
                f"inter={self.inter}, bits={self.bits}, rank={self.rank}, "
                f"clusters={self.n_clusters}, shared_inter={self.shared_inter}")
