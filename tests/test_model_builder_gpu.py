"""GPU checks of the checkpoint adapter (glorcq_amd.model_builder): LoRA factor
dequantization bit-exact against the oracle, a checkpoint written in the
reference's on-disk format (cross_layer_share.py:1024-1141: glorcq_model.pt +
cross_layer_info.pt) loaded into GLoRCQLinear layers whose factors and outputs
match the oracle, and the cross-layer U pool on the MoE step (same bits with
and without the pool)."""

import numpy as np
import pytest
import torch
import torch.nn as nn

from glorcq_amd import format as fmt
from glorcq_amd import model_builder as MB
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from glorcq_amd.quantized_linear import GLoRCQLinear
from oracle import glorcq_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbits,rows,cols,rowwise,int4", [
    (8, 2048, 64, False, False), (4, 1408, 64, False, False), (2, 96, 40, False, False),
    (4, 2048, 64, False, True), (4, 63, 24, True, True), (8, 100, 32, True, False),
])
def test_dequant_factor_bit_exact(gpu, nbits, rows, cols, rowwise, int4):
    t = torch.randn(rows, cols, generator=torch.Generator().manual_seed(rows + nbits)) * 0.03
    q, s = O.quant_intN_absmax(t, nbits, rowwise)
    want = O.dequant_intN(q, s, nbits)
    if int4:
        got = MB.dequant_int4_packed(O.pack_int4(q), rows, s, gpu)
    else:
        got = MB._dequant_intN(q.to(gpu), s.to(gpu), nbits)
    torch.cuda.synchronize()
    assert got.dtype == torch.float16 and torch.equal(got.cpu(), want)


def _gptq_entry(p):
    return {"qweight_int": p.q.clone(), "scales": p.scales.clone(), "zeros": p.zeros.clone(),
            "bits": p.bits, "groupsize": p.group, "sym": False}


def _write_checkpoint(tmp_path, K=1024, N=384, r=32):
    """A two-layer checkpoint in the reference's format: experts 0/1 of layer 0
    and expert 0 of layer 1 (gate_proj) share clusters 0 and 1; a shared
    expert without LoRA; an attention projection with its own cluster.  The
    factors use every stored form the loader knows."""
    g = torch.Generator().manual_seed(3)
    probs = {(0, "mlp.experts.0.gate_proj"): fmt.make_linear(K, N, 2, rank=r, seed=1),
             (0, "mlp.experts.1.gate_proj"): fmt.make_linear(K, N, 2, rank=r, seed=2),
             (1, "mlp.experts.0.gate_proj"): fmt.make_linear(K, N, 2, rank=r, seed=3),
             (0, "mlp.shared_expert.gate_proj"): fmt.make_linear(K, N, 4, rank=r, seed=4),
             (1, "self_attn.q_proj"): fmt.make_linear(K, K, 4, rank=r, seed=5)}
    layers = {0: {}, 1: {}}
    for (li, name), p in probs.items():
        layers[li][name] = _gptq_entry(p)
    model_data = {"model_config": {"uv_bits": 8, "rotation_type": "qr", "qbit": 2},
                  "layers": layers}
    U = {gid: (torch.randn(K, r, generator=g) * 0.02) for gid in range(3)}
    Uq4, Us4 = O.quant_intN_absmax(U[0], 4)
    Uq1, Us1 = O.quant_intN_absmax(U[1], 4)  # int8 container, u_bits = 4
    shared = {"gate_proj": {0: {"U_int4_packed": O.pack_int4(Uq4),
                                "U_orig_rows": torch.tensor(K), "U_scale": Us4},
                            1: {"U_int8": Uq1, "U_scale": Us1,
                                "S": (torch.rand(r, generator=g) + 0.5).half()}},
              "q_proj": {2: {"U_fp16": U[2].half()}}}
    SV = {i: torch.randn(N if i < 3 else K, r, generator=g) * 0.02 for i in range(4)}
    s4q, s4s = O.quant_intN_absmax(SV[0], 4, rowwise=True)
    s8q, s8s = O.quant_intN_absmax(SV[3], 8)
    vq, vs = O.quant_intN_absmax(SV[2], 8)
    per_expert_V = {"gate_proj": [
        {"SV_int4_packed": O.pack_int4(s4q), "SV_orig_rows": torch.tensor(N), "SV_scale": s4s},
        {"SV_fp16": SV[1].half()},
        {"V_int8": vq, "V_scale": vs}],        # old format: V + the cluster's S
        "q_proj": [{"SV_int8": s8q, "SV_scale": s8s}]}
    assignments = {"gate_proj": [{"layer": 0, "expert": 0, "group_id": 0},
                                 {"layer": 0, "expert": 1, "group_id": 0},
                                 {"layer": 1, "expert": 0, "group_id": 1}],
                   "q_proj": [{"layer": 1, "expert": -1, "group_id": 2}]}
    cross = {"config": {"uv_bits": 8, "u_bits": 4, "sv_bits": 8}, "assignments": assignments,
             "shared_matrices": shared, "per_expert_V": per_expert_V}
    torch.save(model_data, tmp_path / "glorcq_model.pt")
    torch.save(cross, tmp_path / "cross_layer_info.pt")
    # expected fp16 factors, through the oracle
    expU = {0: O.dequant_intN(O.unpack_int4(O.pack_int4(Uq4), K), Us4, 4),
            1: O.dequant_intN(Uq1, Us1, 4), 2: U[2].half()}
    S1 = shared["gate_proj"][1]["S"]
    V2 = O.dequant_intN(vq, vs, 8)
    expSV = {(0, "mlp.experts.0.gate_proj"): O.dequant_intN(s4q, s4s, 4),
             (0, "mlp.experts.1.gate_proj"): SV[1].half(),
             (1, "mlp.experts.0.gate_proj"): (V2.float() * S1.float()[None, :]).half(),
             (1, "self_attn.q_proj"): O.dequant_intN(s8q, s8s, 8)}
    expC = {(0, "mlp.experts.0.gate_proj"): 0, (0, "mlp.experts.1.gate_proj"): 0,
            (1, "mlp.experts.0.gate_proj"): 1, (1, "self_attn.q_proj"): 2}
    return probs, expU, expSV, expC


def test_checkpoint_load(gpu, tmp_path):
    probs, expU, expSV, expC = _write_checkpoint(tmp_path)
    model_data, cross = MB.load_glorcq_checkpoint(str(tmp_path))
    layers, u_cache = MB.build_glorcq_layers(model_data, cross, device=gpu)
    torch.cuda.synchronize()
    for (li, name), p in probs.items():
        ql = layers[li][name]
        assert isinstance(ql, GLoRCQLinear) and ql.quant_type == "gptq"
        assert np.array_equal(O.unpack_codes(ql.codes.cpu().numpy(), ql.pack_bits, p.K),
                              p.q.numpy())
        if name.endswith("shared_expert.gate_proj"):
            assert ql.SV is None and ql.cluster_id is None  # shared experts carry no LoRA
            continue
        c = expC[(li, name)]
        assert torch.equal(ql.U.cpu(), expU[c]), (li, name)
        assert torch.equal(ql.SV.cpu(), expSV[(li, name)]), (li, name)
        assert ql.cluster_id[1] == c
        # the layer's forward against the oracle with these factors
        x = p.x.to(gpu)
        y = ql(x)
        ref = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, p.group, exact_weights=True,
                                    U=expU[c], SV=expSV[(li, name)])
        torch.cuda.synchronize()
        err = (y.double().cpu() - ref).abs()
        assert bool((err <= 1e-3 + 1e-2 * ref.abs()).all()), (li, name, float(err.max()))
    # one U per cluster, shared by its experts across layers
    assert layers[0]["mlp.experts.0.gate_proj"].U is layers[0]["mlp.experts.1.gate_proj"].U
    pools, ids = MB._build_global_u_pool(u_cache)
    stacks, ids2 = MB.build_u_pool_stacks(u_cache)
    assert ids == ids2
    r = stacks["gate"].shape[2]
    for (wkey, gid), i in ids["gate"].items():
        assert torch.equal(pools["gate"][:, i * r:(i + 1) * r], stacks["gate"][i])
        assert torch.equal(stacks["gate"][i].cpu(), expU[gid])


def test_moe_block_global_pool(gpu):
    """A block pointed at a cross-layer U pool (rows of other layers' clusters
    around its own, in shuffled order) gives the same bits as the block with
    its own U stack."""
    from test_moe_gpu import small

    p = small(B=5, seed=41)

    def lin(q, e, U=None, SV=None, cid=None):
        m = GLoRCQLinear(q.K, q.N)
        qi = torch.from_numpy(O.unpack_codes(q.codes[e].numpy(), q.bits, q.K))
        m.load_gptq({"qweight_int": qi, "scales": q.scales[e], "zeros": q.zeros[e],
                     "bits": q.bits, "groupsize": q.group, "sym": False}, device=gpu)
        if U is not None:
            m.load_sv(U, SV, device=gpu)
            m.cluster_id = cid
        return m

    class Expert(nn.Module):
        def __init__(self, e):
            super().__init__()
            for proj in fmt.PROJS:
                c = int(p.cluster_of[proj][e])
                setattr(self, f"{proj}_proj", lin(p.experts[proj], e, p.U[proj][c],
                                                  p.SV[proj][e], (f"{proj}_proj", c)))

    class Shared(nn.Module):
        def __init__(self):
            super().__init__()
            for proj in fmt.PROJS:
                setattr(self, f"{proj}_proj", lin(p.shared[proj], 0))

    blk = nn.Module()
    blk.num_experts, blk.top_k, blk.norm_topk_prob = p.E, p.top_k, False
    blk.gate = nn.Linear(p.H, p.E, bias=False)
    blk.gate.weight.data = p.router_w.clone()
    blk.experts = nn.ModuleList([Expert(e) for e in range(p.E)])
    blk.shared_expert = Shared()
    blk.shared_expert_gate = nn.Linear(p.H, 1, bias=False)
    blk.shared_expert_gate.weight.data = p.shared_gate_w.clone()
    own = GraphCompatibleMoeBlock(blk)
    pooled = GraphCompatibleMoeBlock(blk)
    g = torch.Generator().manual_seed(9)
    stacks, id_maps = {}, {}
    for proj in fmt.PROJS:
        C, K, r = p.U[proj].shape
        extra = 5
        rows = torch.randperm(C + extra, generator=g).tolist()
        pool = (torch.randn(C + extra, K, r, generator=g) * 0.02).half()
        id_maps[proj] = {}
        for c in range(C):
            pool[rows[c]] = p.U[proj][c]
            id_maps[proj][(f"{proj}_proj", c)] = rows[c]
        stacks[proj] = pool.to(gpu)
    pooled.set_global_pool(stacks, id_maps)
    h = p.h.reshape(1, 5, p.H).to(gpu)
    a, la = own(h)
    b, lb = pooled(h)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)
