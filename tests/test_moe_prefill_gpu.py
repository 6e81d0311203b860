"""MoE block over many tokens (glq_moe_prefill via GraphCompatibleMoeBlock with
more than 64 tokens): grouped dequant GEMMs over each active expert's gathered
tokens, the reference's _forward_sparse (inference/moe_block.py:704-740),
against the MoE oracle (oracle.moe_forward, pinned by
tests/test_moe_oracle_library.py against transformers' sparse MoE blocks).

Bars as tests/test_moe_gpu.py: routing ids identical (seeds with no near-tie
at the top-k boundary, asserted), router logits within one fp16 ulp, block
output within the MoE bar (atol 1e-3 + rtol 1e-2 |ref| + 2e-3 * row max)."""

import pytest
import torch

from glorcq_amd import format as fmt
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from oracle import glorcq_oracle as O
from test_moe_gpu import check_routing, margin
from test_moe_oracle import bar, lora_heavy

pytestmark = pytest.mark.gpu


def run(p, gpu, residual=None):
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    res = None if residual is None else residual.reshape(1, p.B, p.H).to(gpu)
    out, logits = blk(p.h.reshape(1, p.B, p.H).to(gpu), residual=res)
    torch.cuda.synchronize()
    return blk, out.reshape(p.B, p.H).cpu(), logits.cpu()


def check(p, out, logits, what):
    check_routing(p, logits)
    ref = O.moe_forward(p)
    assert bar(out, ref), (what, float((out.double() - ref).abs().max()))


def test_config3_prefill_512(gpu):
    """BASELINE config 3's prefill: a Mixtral-8x7B-shaped layer over 512 tokens
    (about 128 tokens per expert: 128-token tiles), LoRA factors x3."""
    p = lora_heavy(fmt.make_mixtral_layer(B=512, seed=42), f=3.0)
    assert margin(p) >= 2
    print("config 3 prefill T=512", flush=True)
    _, out, logits = run(p, gpu)
    check(p, out, logits, "config 3 T=512")


def test_config2_prefill(gpu):
    """A Qwen1.5-MoE-A2.7B block (60 experts, top-4, 16 clusters, 4-bit shared
    expert behind its sigmoid gate) over 80 tokens (32-token tiles)."""
    p = fmt.make_moe(B=80, seed=82)
    assert margin(p) >= 2
    _, out, logits = run(p, gpu)
    check(p, out, logits, "config 2 T=80")


@pytest.mark.parametrize("kw", [
    dict(),
    dict(norm_topk_prob=True),
    dict(rank=0),
    dict(bits=4),
    dict(shared_bits=2),
    dict(shared_inter=0),
    dict(n_clusters=1),
], ids=lambda kw: ",".join(f"{k}={v}" for k, v in kw.items()) or "base")
def test_prefill_variants(gpu, kw):
    """A small block (H 256, 8 experts, inter 384, top-2, 3 clusters, rank 16)
    over 200 tokens (64-token tiles), LoRA x30 where it has a rank."""
    args = dict(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16, shared_inter=512)
    args.update(kw)
    # the first seed from 10 whose routing has no near-tie (routing only: cheap)
    seed = next(s for s in range(10, 60) if margin(fmt.make_moe(B=200, seed=s, **args)) >= 2)
    p = fmt.make_moe(B=200, seed=seed, **args)
    if p.rank:
        p = lora_heavy(p)
    _, out, logits = run(p, gpu)
    check(p, out, logits, str(kw))


def test_prefill_residual_and_tiles(gpu, monkeypatch):
    """The residual add is fused into the combine; every token tile size gives
    the same bits (rows are independent)."""
    p = lora_heavy(fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16,
                                shared_inter=512, B=200, seed=10))
    res = (torch.randn(200, 256, generator=torch.Generator().manual_seed(3)) * 0.5).half()
    outs = []
    for tm in ("32", "64", "128"):
        monkeypatch.setenv("GLQ_PF_MOE_TM", tm)
        _, out, _ = run(p, gpu, residual=res)
        outs.append(out)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    ref = (O.moe_forward(p).half().double() + res.double())
    assert bar(outs[0], ref)


def test_prefill_matches_decode_steps(gpu):
    """The same 72 tokens as one prefill and as decode steps of 36: both within
    the bar of the oracle and of each other (different kernels, same math)."""
    p = lora_heavy(fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16,
                                shared_inter=512, B=72, seed=10))
    blk, out, logits = run(p, gpu)
    h = p.h.to(gpu)
    d0, l0 = blk(h[:36].reshape(1, 36, p.H))
    d1, l1 = blk(h[36:].reshape(1, 36, p.H))
    torch.cuda.synchronize()
    dec = torch.cat([d0.reshape(36, p.H), d1.reshape(36, p.H)]).cpu()
    assert bar(out, dec.double())
    assert torch.equal(torch.cat([l0, l1]).cpu(), logits) or \
        float((torch.cat([l0, l1]).cpu().float() - logits.float()).abs().max()) < 1e-2


def test_non_integer_zeros_use_decode_steps(gpu):
    """Zero-points that are not integers (the prefill GEMMs take integer ones)
    run as 64-token decode steps: still within the bar."""
    p = fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16, shared_inter=512,
                     B=100, seed=10)
    g = torch.Generator().manual_seed(9)
    for proj in fmt.PROJS:
        z = p.experts[proj].zeros.float()
        p.experts[proj].zeros = (z + torch.rand(z.shape, generator=g) * 0.5).half()
    assert margin(p) >= 2
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    assert not blk.zeros_integral
    out, logits = blk(p.h.reshape(1, 100, p.H).to(gpu))
    torch.cuda.synchronize()
    check(p, out.reshape(100, p.H).cpu(), logits.cpu(), "non-integer zeros")


def test_non_integer_shared_zeros_use_decode_steps(gpu):
    """Non-integer zero-points on the shared expert only (the routed ones stay
    integers): the block still takes decode steps, since the prefill GEMMs
    use round(z) for the shared expert too, and stays within the bar."""
    p = fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16, shared_inter=512,
                     B=100, seed=10)
    g = torch.Generator().manual_seed(11)
    for proj in fmt.PROJS:
        z = p.shared[proj].zeros.float()
        p.shared[proj].zeros = (z + 0.25 + torch.rand(z.shape, generator=g) * 0.5).half()
    assert margin(p) >= 2
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    assert not blk.zeros_integral
    out, logits = blk(p.h.reshape(1, 100, p.H).to(gpu))
    torch.cuda.synchronize()
    check(p, out.reshape(100, p.H).cpu(), logits.cpu(), "non-integer shared zeros")
