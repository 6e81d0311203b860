"""MoE decode step with TurboQuant routed experts (the reference's 2-bit expert
format; inference/moe_block.py:331-357, 480-702) through GraphCompatibleMoeBlock
(glq_moe_route, glq_turbo_moe_gemv, glq_lowrank_xu_routed, glq_moe_combine)
against the oracle (oracle/glorcq_oracle.py: moe_forward with format.TurboMat
experts, pinned against transformers' MoE blocks in test_moe_turbo_oracle.py).

Config-2 dimensions (hidden 2048 = a power of two: gate/up rotated by an RHT;
inter 1408 is not: down rotated by a QR Pi, the two forms a real checkpoint
mixes), LoRA-heavy factors so the low-rank terms are a visible part of the
output, and routed experts alone where the shared expert's large outputs would
set the bar's row term.  Bar: test_moe_oracle.bar; routing ids and logits as in
test_moe_gpu."""

import pytest
import torch
import torch.nn as nn

from glorcq_amd import format as fmt
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from oracle import glorcq_oracle as O
from test_moe_gpu import check_routing, margin
from test_moe_oracle import bar, lora_heavy

pytestmark = pytest.mark.gpu


def problem(B, seed, shared_inter=0, E=16, top_k=4, **kw):
    p = fmt.make_turbo_moe(H=2048, E=E, inter=1408, top_k=top_k, n_clusters=4, rank=64,
                           shared_inter=shared_inter, B=B, seed=seed, **kw)
    return lora_heavy(p, 10.0)


def run(blk, p, gpu):
    out, logits = blk(p.h.reshape(1, p.B, p.H).to(gpu))
    torch.cuda.synchronize()
    return out.reshape(p.B, p.H).cpu(), logits.cpu()


@pytest.mark.parametrize("B,seed", [(1, 3), (4, 4), (16, 6), (20, 6)])
def test_turbo_routed_parity(gpu, B, seed):
    """Routed turbo experts only (20 tokens: two steps of at most 16)."""
    p = problem(B, seed)
    assert margin(p) >= 2
    print(f"turbo routed B={B} seed={seed}", flush=True)
    out, logits = run(GraphCompatibleMoeBlock.from_problem(p, gpu), p, gpu)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())
    # an oracle whose down rotation is transposed must fail the bar
    q = problem(B, seed)
    q.experts["down"].Pi = q.experts["down"].Pi.T.contiguous()
    assert not bar(out, O.moe_forward(q))


@pytest.mark.parametrize("B,seed", [(1, 7), (3, 9), (8, 8)])
def test_turbo_with_shared_expert(gpu, B, seed):
    """Config-2 semantics: turbo routed experts plus the 4-bit GPTQ shared
    expert behind its sigmoid gate, and the caller's residual folded in (1 and
    3 tokens: the shared expert inside the fused step's launches; 8: on the
    side stream)."""
    p = problem(B, seed, shared_inter=1024, E=60)
    assert margin(p) >= 2
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    h = p.h.reshape(1, p.B, p.H).to(gpu)
    r = (torch.randn(1, p.B, p.H, generator=torch.Generator().manual_seed(seed)) * 0.5).half()
    out, logits = blk(h, residual=r.to(gpu))
    torch.cuda.synchronize()
    check_routing(p, logits.cpu())
    ref = O.moe_forward(p)
    ref_r = ref.half().double() + r.reshape(p.B, p.H).double()
    assert bar(out.reshape(p.B, p.H).cpu(), ref_r)


def test_turbo_block_from_glorcq_layers(gpu):
    """A block of GLoRCQLinear experts loaded with load_turbo (the reference's
    turbo_compressed dicts and RotationCache; gate/up with RHT signs, down with
    Pi) gives the same step, bit for bit, as the block built from the problem."""
    from glorcq_amd.quantized_linear import GLoRCQLinear, RotationCache

    p = problem(5, 9, shared_inter=512, E=8, top_k=2)
    cache = RotationCache(device=gpu)
    seeds = {"gate": 11, "up": 11, "down": 12}
    for proj in ("gate", "down"):
        q = p.experts[proj]
        cache.put(q.K, 2, seeds[proj], q.Pi, q.centroids)

    def turbo_lin(proj, e):
        q = p.experts[proj]
        m = GLoRCQLinear(q.K, q.N)
        m.load_turbo({"packed_indices": q.packed[e], "norms": q.norms[e], "bits": 2,
                      "dim": q.K, "seed": seeds[proj]}, cache, device=gpu)
        if q.signs is not None:
            m._rht_signs = q.signs.to(gpu)
        c = int(p.cluster_of[proj][e])
        m.load_sv(p.U[proj][c], p.SV[proj][e], device=gpu)
        m.cluster_id = c
        return m

    def gptq_lin(q):
        m = GLoRCQLinear(q.K, q.N)
        qi = torch.from_numpy(O.unpack_codes(q.codes[0].numpy(), q.bits, q.K))
        m.load_gptq({"qweight_int": qi, "scales": q.scales[0], "zeros": q.zeros[0],
                     "bits": q.bits, "groupsize": q.group, "sym": False}, device=gpu)
        return m

    class Expert(nn.Module):
        def __init__(self, e):
            super().__init__()
            for proj in fmt.PROJS:
                setattr(self, f"{proj}_proj", turbo_lin(proj, e))

    class Shared(nn.Module):
        def __init__(self):
            super().__init__()
            for proj in fmt.PROJS:
                setattr(self, f"{proj}_proj", gptq_lin(p.shared[proj]))

    blk = nn.Module()
    blk.num_experts, blk.top_k, blk.norm_topk_prob = p.E, p.top_k, False
    blk.gate = nn.Linear(p.H, p.E, bias=False)
    blk.gate.weight.data = p.router_w.clone()
    blk.experts = nn.ModuleList([Expert(e) for e in range(p.E)])
    blk.shared_expert = Shared()
    blk.shared_expert_gate = nn.Linear(p.H, 1, bias=False)
    blk.shared_expert_gate.weight.data = p.shared_gate_w.clone()
    mine = GraphCompatibleMoeBlock(blk)
    assert mine.kind == "turbo"
    a, la = run(mine, p, gpu)
    b, lb = run(GraphCompatibleMoeBlock.from_problem(p, gpu), p, gpu)
    assert torch.equal(a, b) and torch.equal(la, lb)
    assert bar(a, O.moe_forward(p))


def test_turbo_step_in_a_hip_graph(gpu):
    """The step captured once and replayed on new inputs equals eager steps
    (routing stays on the device; eager work and syncs between replays)."""
    p = problem(4, 10, shared_inter=512, E=16)
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    hs = [torch.randn(1, 4, p.H, generator=torch.Generator().manual_seed(s)).half().to(gpu)
          for s in range(3)]
    eager = [blk(h)[0].clone() for h in hs]
    torch.cuda.synchronize()
    static_h = hs[0].clone()
    blk(static_h)  # warm-up: workspaces exist before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out, _ = blk(static_h)
    for h, ref in zip(hs, eager):
        static_h.copy_(h)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, ref)
        _ = blk(hs[0])  # eager work between replays
        torch.cuda.synchronize()


def test_turbo_block_from_checkpoint(gpu, tmp_path):
    """A checkpoint in the reference's format (glorcq_model.pt with
    packed_indices / norms / bits / dim / seed per expert module, the shared
    expert as GPTQ; cross_layer_info.pt with cluster U and per-expert SV)
    loaded by load_glorcq_checkpoint + build_glorcq_layers, placed into a block
    and run as GraphCompatibleMoeBlock, against the oracle.  Rotation 'qr':
    the RotationCache holds Pi and the codebook per (dim, bits, seed)."""
    from glorcq_amd import model_builder as MB
    from glorcq_amd.quantized_linear import RotationCache

    p = problem(3, 4, shared_inter=512, E=8, top_k=2, rot_gate_up="qr")
    assert margin(p) >= 2
    seed = 42
    layers = {0: {}}
    for e in range(p.E):
        for proj in fmt.PROJS:
            q = p.experts[proj]
            layers[0][f"mlp.experts.{e}.{proj}_proj"] = {
                "packed_indices": q.packed[e].clone(), "norms": q.norms[e].clone(),
                "bits": 2, "dim": q.K, "seed": seed}
    for proj in fmt.PROJS:
        s = p.shared[proj]
        qi = torch.from_numpy(O.unpack_codes(s.codes[0].numpy(), s.bits, s.K))
        layers[0][f"mlp.shared_expert.{proj}_proj"] = {
            "qweight_int": qi, "scales": s.scales[0].clone(), "zeros": s.zeros[0].clone(),
            "bits": s.bits, "groupsize": s.group, "sym": False}
    model_data = {"model_config": {"uv_bits": 16, "rotation_type": "qr", "qbit": 2},
                  "layers": layers}
    shared, per_expert_V, assignments = {}, {}, {}
    for proj in fmt.PROJS:
        w = f"{proj}_proj"
        shared[w] = {c: {"U_fp16": p.U[proj][c].clone()} for c in range(p.n_clusters)}
        assignments[w] = [{"layer": 0, "expert": e, "group_id": int(p.cluster_of[proj][e])}
                          for e in range(p.E)]
        per_expert_V[w] = [{"SV_fp16": p.SV[proj][e].clone()} for e in range(p.E)]
    cross = {"config": {"uv_bits": 16}, "assignments": assignments,
             "shared_matrices": shared, "per_expert_V": per_expert_V}
    torch.save(model_data, tmp_path / "glorcq_model.pt")
    torch.save(cross, tmp_path / "cross_layer_info.pt")
    cache = RotationCache(device=gpu)
    for proj in ("gate", "down"):
        q = p.experts[proj]
        cache.put(q.K, 2, seed, q.Pi, q.centroids)
    md, cl = MB.load_glorcq_checkpoint(str(tmp_path))
    built, _ = MB.build_glorcq_layers(md, cl, device=gpu, rotation_cache=cache)
    mods = built[0]

    class Proj(nn.Module):
        def __init__(self, prefix):
            super().__init__()
            for proj in fmt.PROJS:
                setattr(self, f"{proj}_proj", mods[f"{prefix}.{proj}_proj"])

    blk = nn.Module()
    blk.num_experts, blk.top_k, blk.norm_topk_prob = p.E, p.top_k, False
    blk.gate = nn.Linear(p.H, p.E, bias=False)
    blk.gate.weight.data = p.router_w.clone()
    blk.experts = nn.ModuleList([Proj(f"mlp.experts.{e}") for e in range(p.E)])
    blk.shared_expert = Proj("mlp.shared_expert")
    blk.shared_expert_gate = nn.Linear(p.H, 1, bias=False)
    blk.shared_expert_gate.weight.data = p.shared_gate_w.clone()
    mine = GraphCompatibleMoeBlock(blk)
    assert mine.kind == "turbo"
    out, logits = run(mine, p, gpu)
    check_routing(p, logits)
    assert bar(out, O.moe_forward(p))


@pytest.mark.parametrize("B,seed,inter,rot_gu,rot_down", [(1, 11, 1408, "rht", "qr"),
                                                          (4, 12, 1408, "rht", "qr"),
                                                          (3, 13, 1024, "rht", "rht"),
                                                          (2, 15, 1408, "qr", "qr"),
                                                          (16, 14, 1408, "rht", "qr")])
def test_turbo_fused_step_matches_launch_sequence(gpu, B, seed, inter, rot_gu, rot_down,
                                                  monkeypatch):
    """The four-launch turbo step (glq_turbo_moe_prep, the gate/up pair,
    glq_turbo_moe_down_prep, down) against the launch-by-launch step
    (GLQ_TURBO_SEQ=1): the same routing; with the down rotated by the
    transform the same bits end to end (with a Pi only the rotation's fp32
    sums run in another order); both within the oracle's bar."""
    p = fmt.make_turbo_moe(H=2048, E=16, inter=inter, top_k=4, n_clusters=4, rank=64,
                           shared_inter=0, B=B, seed=seed, rot_gate_up=rot_gu,
                           rot_down=rot_down)
    p = lora_heavy(p, 10.0)
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    h = p.h.reshape(1, p.B, p.H).to(gpu)
    print(f"turbo fused B={B} inter={inter} {rot_gu}/{rot_down}", flush=True)
    out_f, lg_f = blk(h)
    out_f, lg_f = out_f.clone(), lg_f.clone()
    monkeypatch.setenv("GLQ_TURBO_SEQ", "1")
    out_s, lg_s = blk(h)
    torch.cuda.synchronize()
    assert torch.equal(lg_f, lg_s)
    if rot_down == "rht":
        assert torch.equal(out_f, out_s)
    ref = O.moe_forward(p)
    for out in (out_f, out_s):
        assert bar(out.reshape(p.B, p.H).cpu(), ref)
