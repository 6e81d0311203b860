"""MoE decode step (glq_moe_decode via glorcq_amd.moe_block.GraphCompatibleMoeBlock)
against the MoE oracle (oracle/glorcq_oracle.py: route, moe_forward), which
follows GraphCompatibleMoeBlock.forward (inference/moe_block.py:381-436).

Bar: routing ids identical, routing weights equal in fp16 up to one ulp, router
logits within one fp16 ulp, block output within the composite bar of
test_moe_oracle.bar (atol 1e-3 + rtol 1e-2 |ref| + 2e-3 * row max).  Inputs
are chosen (and asserted) to have no near-tie at the top-k boundary: exact
ties have no unique answer (torch's CPU topk breaks them by its partial-sort
order, this build by lowest expert index)."""

import ctypes

import pytest
import torch

from glorcq_amd import _lib
from glorcq_amd import format as fmt
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from oracle import glorcq_oracle as O
from test_moe_oracle import bar, lora_heavy, strict_report


def margin(p):
    """Smallest gap, over tokens, between the k-th and (k+1)-th largest router
    logit, in fp16 ulps of the k-th: at >= 2 ulps a one-ulp difference in a
    logit cannot change the selection."""
    if p.top_k == p.E:
        return float("inf")
    logits, _, _ = O.route(p.h, p.router_w, p.top_k, p.norm_topk_prob, exact=True)
    s, _ = logits.float().sort(-1, descending=True)
    lk, lk1 = s[:, p.top_k - 1], s[:, p.top_k]
    return float(((lk - lk1) / logit_ulp(lk)).min())


def small(B=3, seed=5, **kw):
    args = dict(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16, shared_inter=512)
    args.update(kw)
    return fmt.make_moe(B=B, seed=seed, **args)


def params_for(p):
    """MoeParams with host-side dummy pointers (for the CPU shape checks)."""
    P = _lib.MoeParams()
    P.tokens, P.hidden, P.experts, P.inter = p.B, p.H, p.E, p.inter
    P.top_k, P.n_clusters, P.rank = p.top_k, p.n_clusters, p.rank
    P.shared_inter = p.shared["gate"].N if p.shared else 0
    P.bits, P.shared_bits, P.group = 2, 4, 128
    fake = 1 << 20  # aligned, never dereferenced by the shape checks
    P.h = P.router_w = P.shared_gate_w = P.out = fake
    for i in range(3):
        P.codes[i] = P.scales[i] = P.zeros[i] = P.U[i] = P.cluster_of[i] = P.SV[i] = fake
        P.shared_codes[i] = P.shared_scales[i] = P.shared_zeros[i] = fake
    return P


# ------------------------------------------------------------------ CPU ----
def test_workspace_and_shape_checks():
    lib = _lib.load()
    p = fmt.make_moe(B=4, seed=0)
    P = params_for(p)
    n = lib.glq_moe_workspace_bytes(ctypes.byref(P))
    assert n > 0 and n % 256 == 0
    P.tokens = 65
    assert lib.glq_moe_workspace_bytes(ctypes.byref(P)) == -1
    assert b"tokens" in lib.glq_last_error()
    P.tokens, P.group = 4, 64
    assert lib.glq_moe_workspace_bytes(ctypes.byref(P)) == -1
    P.group, P.hidden = 128, 300
    assert lib.glq_moe_workspace_bytes(ctypes.byref(P)) == -1
    P.hidden, P.rank = 2048, 12
    assert lib.glq_moe_workspace_bytes(ctypes.byref(P)) == -1
    P.rank, P.top_k = 64, 61
    assert lib.glq_moe_workspace_bytes(ctypes.byref(P)) == -1
    P.top_k = 4
    assert lib.glq_moe_decode(ctypes.byref(P), None, 0, None) == 1
    assert b"workspace" in lib.glq_last_error()


# ------------------------------------------------------------------ GPU ----
def run_block(p, gpu):
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    out, logits = blk(p.h.reshape(1, p.B, p.H).to(gpu))
    torch.cuda.synchronize()
    return blk, out.reshape(p.B, p.H).cpu(), logits.cpu()


def logit_ulp(x):
    """One fp16 ulp of x, floored at 2^-20: near zero the fp32 sums behind any
    fp16 logit (GPU, or the fp64 reference rounded once) differ by ~1e-7."""
    return torch.finfo(torch.float16).eps * x.float().abs().clamp(min=2.0**-10)


def check_routing(p, logits):
    ref_logits, _, _ = O.route(p.h, p.router_w, p.top_k, p.norm_topk_prob, exact=True)
    d = (logits.float() - ref_logits.float()).abs()
    r = d / logit_ulp(ref_logits)
    i = int(r.argmax())
    assert float(r.max()) <= 1.01, (float(r.max()), float(logits.flatten()[i]),
                                     float(ref_logits.flatten()[i]))


@pytest.mark.gpu
@pytest.mark.parametrize("B,seed", [(1, 0), (4, 1), (16, 1), (32, 6)])
def test_config2_parity(gpu, B, seed):
    """BASELINE config 2 (Qwen1.5-MoE-A2.7B block) at each batch size."""
    p = fmt.make_moe(B=B, seed=seed)
    assert margin(p) >= 2
    _, out, logits = run_block(p, gpu)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())
    strict_report(p, out, ref, f"config 2 B={B}")


@pytest.mark.gpu
@pytest.mark.parametrize("B,seed", [(1, 1), (16, 1), (32, 2), (64, 2)])
def test_config2_routed_only(gpu, B, seed):
    """Config 2's routed experts alone (no shared expert, whose large outputs
    would set the bar's row term): the output is the weighted sum of the
    selected experts, so a wrong pick or weight moves it past the bar -- an
    oracle routed with two router rows swapped (other experts picked) fails."""
    p = fmt.make_moe(B=B, seed=seed, shared_inter=0)
    assert margin(p) >= 2
    _, out, logits = run_block(p, gpu)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())
    _, _, sel = O.route(p.h, p.router_w, p.top_k, False, exact=True)
    e0 = int(sel[0, 0])
    other = next(e for e in range(p.E) if e not in sel[0].tolist())
    q = fmt.make_moe(B=B, seed=seed, shared_inter=0)
    rw = q.router_w.clone()
    rw[[e0, other]] = rw[[other, e0]]
    q.router_w = rw
    assert not bar(out, O.moe_forward(q))


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 16])
def test_config2_lora_heavy(gpu, B):
    """U and SV scaled x30 so a wrong cluster, SV row or a_down reduction
    moves the output past the bar (test_moe_oracle plants such mistakes)."""
    p = lora_heavy(fmt.make_moe(B=B, seed=1))
    assert margin(p) >= 2
    _, out, _ = run_block(p, gpu)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())
    # the low-rank terms matter at this scale: dropping them fails the bar
    q = lora_heavy(fmt.make_moe(B=B, seed=1))
    for proj in fmt.PROJS:
        q.SV[proj] = torch.zeros_like(q.SV[proj])
    assert not bar(out, O.moe_forward(q))


@pytest.mark.gpu
@pytest.mark.parametrize("kw", [
    dict(norm_topk_prob=True),
    dict(shared_inter=0),
    dict(rank=0),
    dict(bits=4),
    dict(shared_bits=2),
    dict(top_k=8, E=8),                 # every expert selected
    dict(inter=4096, rank=64),          # routed down in K parts
    dict(H=512, shared_inter=8192),     # shared down in K parts
    dict(n_clusters=1),
], ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()))
def test_variants(gpu, kw):
    B = kw.pop("B", 12)
    p = lora_heavy(small(B=B, seed=21, **kw)) if kw.get("rank", 16) else small(B=B, seed=21, **kw)
    assert margin(p) >= 2
    _, out, logits = run_block(p, gpu)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())


@pytest.mark.gpu
@pytest.mark.parametrize("B,seed", [(1, 3), (3, 6), (16, 7), (64, 14)])
def test_config4_block_gated_xu(gpu, B, seed, monkeypatch):
    """A Qwen3-30B-A3B-shaped block (128 experts, inter 768, top-8,
    norm_topk_prob, no shared expert) with 100 clusters: at B = 1 and 3 the
    clusters outnumber four times the picks, so the x U jobs run in their own
    launch and skip unpicked clusters; at 16 and 64 (the 512 picks of a
    prefill chunk, the step's maximum) they run beside the router.  LoRA
    scaled x30 (a skipped active cluster fails the bar); the forced other form
    gives the same bits."""
    p = lora_heavy(fmt.make_moe(H=2048, E=128, inter=768, top_k=8, n_clusters=100, rank=64,
                                shared_inter=0, norm_topk_prob=True, B=B, seed=seed))
    assert margin(p) >= 2
    blk, out, logits = run_block(p, gpu)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())
    monkeypatch.setenv("GLQ_MOE_XU_GATE", "0" if B < 4 else "1")
    out2, _ = blk(p.h.reshape(1, p.B, p.H).to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(out2.reshape(p.B, p.H).cpu(), out)


@pytest.mark.gpu
@pytest.mark.parametrize("B", [17, 40])
def test_skewed_routing_many_blocks(gpu, B):
    """Every token routes to expert 3 first: that expert's tokens span several
    8-token blocks; the shared expert spans several 16-token blocks."""
    p = small(B=B, seed=31, E=6, top_k=2)
    g = torch.Generator().manual_seed(5)
    v = torch.randn(p.H, generator=g)
    p.h = (v[None, :] * 2 + torch.randn(B, p.H, generator=g) * 0.5).half()
    rw = p.router_w.float()
    rw[3] = v * 0.05
    p.router_w = rw.half()
    _, _, sel = O.route(p.h, p.router_w, p.top_k, False)
    assert bool((sel[:, 0] == 3).all())
    assert margin(p) >= 2
    _, out, logits = run_block(p, gpu)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), float((out.double() - ref).abs().max())


@pytest.mark.gpu
def test_graph_capture_replays(gpu):
    """The step captured in a hipGraph (torch.cuda.CUDAGraph) replays with
    new hidden states, bit-identical to eager calls (graph_wrapper.py:69-149)."""
    p = fmt.make_moe(B=4, seed=1)
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    static_h = p.h.reshape(1, 4, p.H).to(gpu)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        for _ in range(3):
            blk(static_h)
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out, static_logits = blk(static_h)
    g = torch.Generator().manual_seed(77)
    for i in range(4):
        h = torch.randn(1, 4, p.H, generator=g).half().to(gpu)
        static_h.copy_(h)
        graph.replay()
        torch.cuda.synchronize()
        got = static_out.clone()
        want, _ = blk(h)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
    # and against the oracle for the last input
    q = fmt.make_moe(B=4, seed=1)
    q.h = h.reshape(4, p.H).cpu()
    if margin(q) >= 2:
        assert bar(got.reshape(4, p.H).cpu(), O.moe_forward(q))


@pytest.mark.gpu
def test_from_block_matches_from_problem(gpu):
    """Construction from a block of GLoRCQLinear experts (the reference's
    constructor input, moe_block.py:45-77) gives the same step."""
    import torch.nn as nn

    from glorcq_amd.quantized_linear import GLoRCQLinear

    p = small(B=5, seed=41)
    blk_ref = GraphCompatibleMoeBlock.from_problem(p, gpu)

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
                setattr(self, f"{proj}_proj",
                        lin(p.experts[proj], e, p.U[proj][c], p.SV[proj][e], c))

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
    mine = GraphCompatibleMoeBlock(blk)
    h = p.h.reshape(1, 5, p.H).to(gpu)
    a, la = mine(h)
    b, lb = blk_ref(h)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(la, lb)
