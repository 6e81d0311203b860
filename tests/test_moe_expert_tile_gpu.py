"""Routed experts of a MoE decode step in the token-tile form
(glorcq_amd/csrc/glq_moe_lane.hip: moe_lane_gu_xt_kernel and
moe_lane_down_xt_kernel over glq_tile16.h's 2-bit form): one workgroup set per
expert whose token rows are the expert's picks, so each code is decoded once
for all of them (the lane form decodes it once per pick).  The lane path takes
it when the picks are at least twice the experts (BASELINE config 3 from 8
tokens); GLQ_MOE_XT16=1 / 0 forces it on / off.

Bars as tests/test_moe_gpu.py against the MoE oracle (routing ids identical,
logits within one fp16 ulp, output within atol 1e-3 + rtol 1e-2 |ref| + 2e-3
row max), and against the same step without the tile form within the same
bar: the fp32 sums run in other orders, and the 2-bit tile form applies a
zero point with a fraction to each token's sum of x (s (sum q x - z sum x))
where the lane form rounds fp16(q - z) per code."""

import pytest
import torch

from glorcq_amd import format as fmt
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from oracle import glorcq_oracle as O
from test_moe_gpu import check_routing, margin, small
from test_moe_oracle import bar, lora_heavy

pytestmark = pytest.mark.gpu


def step(p, gpu, monkeypatch, xt):
    monkeypatch.delenv("GLQ_MOE_NO_LANE", raising=False)
    monkeypatch.setenv("GLQ_MOE_XT16", "1" if xt else "0")
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    out, logits = blk(p.h.reshape(1, p.B, p.H).to(gpu))
    torch.cuda.synchronize()
    return out.reshape(p.B, p.H).cpu(), logits.cpu()


def check(p, gpu, monkeypatch, what):
    print(what, flush=True)
    out, logits = step(p, gpu, monkeypatch, True)
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), (what, float((out.double() - ref).abs().max()))
    lane, _ = step(p, gpu, monkeypatch, False)
    assert bar(out, lane.double()), (what, "vs the lane form",
                                     float((out.double() - lane.double()).abs().max()))


def frac_zeros(p, seed):
    """Zero points with a fraction (k/4) on the routed experts."""
    g = torch.Generator().manual_seed(seed)
    for proj in fmt.PROJS:
        q = p.experts[proj]
        q.zeros = (q.zeros.float() +
                   torch.randint(0, 4, q.zeros.shape, generator=g).float() * 0.25).half()
    return p


def no_tie(make, seed):
    """The problem of the first seed from `seed` with no near-tie at the top-k
    boundary."""
    for s in range(seed, seed + 40):
        p = make(s)
        if margin(p) >= 2:
            return p
    raise AssertionError("no seed without a near-tie")


@pytest.mark.parametrize("B,seed", [(8, 4), (16, 6)])
def test_config3(gpu, monkeypatch, B, seed):
    """BASELINE config 3 (Mixtral-8x7B-shaped: H 4096, ffn 14336, 8 experts,
    top-2): gate/up rows in two K slices handed over in the launch, the down
    rows in seven K slices summed at the combine; LoRA factors x3."""
    p = no_tie(lambda s: lora_heavy(fmt.make_mixtral_layer(B=B, seed=s), f=3.0), seed)
    check(p, gpu, monkeypatch, f"config 3 B={B}")


def test_config3_fractional_zeros(gpu, monkeypatch):
    p = no_tie(lambda s: frac_zeros(lora_heavy(fmt.make_mixtral_layer(B=16, seed=s), f=3.0), 5), 9)
    check(p, gpu, monkeypatch, "config 3 B=16, zeros with fractions")


@pytest.mark.parametrize("kw", [
    dict(),                                  # H 256: one K slice of 2 groups
    dict(rank=0),
    dict(shared_inter=0),
    dict(rank=64, n_clusters=1),
    dict(top_k=8, E=8),                      # 128 picks at 16 tokens: two routing chunks
    dict(norm_topk_prob=True),
    dict(H=4096, inter=1024, E=4, shared_inter=0),  # gate/up K slices handed over
    dict(H=1024, inter=2176, rank=8),        # down rows in two K slices (17 groups)
], ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()) or "small")
@pytest.mark.parametrize("B", [1, 5, 16])
def test_forced(gpu, monkeypatch, kw, B):
    def make(s):
        p = small(B=B, seed=s, **kw)
        return lora_heavy(p) if p.rank else p
    p = no_tie(make, 31)
    check(p, gpu, monkeypatch, f"{kw} B={B}")


def test_fractional_zeros_small(gpu, monkeypatch):
    p = no_tie(lambda s: frac_zeros(lora_heavy(small(B=6, seed=s)), 3), 40)
    check(p, gpu, monkeypatch, "small B=6, zeros with fractions")


def test_graph_replay_and_workspace_reuse(gpu, monkeypatch):
    """Captured in a hipGraph the step replays bit-identical to eager calls
    (the gate/up slices' arrival counters are left zero after every step), and
    a workspace that served the lane form in between gives the same bits."""
    monkeypatch.delenv("GLQ_MOE_NO_LANE", raising=False)
    monkeypatch.setenv("GLQ_MOE_XT16", "1")
    p = lora_heavy(small(B=8, seed=3, H=4096, inter=512, E=4, shared_inter=0))
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    static_h = p.h.reshape(1, 8, p.H).to(gpu)
    first, _ = blk(static_h)
    monkeypatch.setenv("GLQ_MOE_XT16", "0")
    blk(static_h)
    monkeypatch.setenv("GLQ_MOE_XT16", "1")
    again, _ = blk(static_h)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        for _ in range(2):
            blk(static_h)
    torch.cuda.current_stream(gpu).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out, _ = blk(static_h)
    g = torch.Generator().manual_seed(78)
    for i in range(4):
        h = torch.randn(1, 8, p.H, generator=g).half().to(gpu)
        static_h.copy_(h)
        graph.replay()
        torch.cuda.synchronize()
        got = static_out.clone()
        want, _ = blk(h)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i}"
