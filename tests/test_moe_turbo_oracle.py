"""Pins the oracle's MoE block with TurboQuant routed experts (oracle/
glorcq_oracle.py: moe_forward -> _turbo_linear, turbo_rotate) against
transformers' sparse MoE blocks, as tests/test_moe_oracle_library.py does for
GPTQ experts.

A TurboQuant expert computes y = W_t x_rot with W_t[n, k] = norm[n] C[q[n, k]]
and x_rot = R x, R the randomized Hadamard transform (1/sqrt(d)) H diag(signs)
or a QR rotation Pi (inference/moe_block.py:331-357, 480-702; quantized_linear.
py:315-349).  So the expert's dense weight is W_t R (+ SV U^T for the
low-rank term), exact in fp64; the library block run with those weights fixes
what the oracle must compute, up to the oracle's fp16 rounding points (x_rot
and a = x U in fp16, the fp16 SwiGLU product), which the MoE bar absorbs.
Planted mistakes in what the oracle is given (the RHT signs flipped, Pi
transposed, the codebook reversed, gate and up swapped) must fail the bar.
"""

import numpy as np
import pytest
import torch

from glorcq_amd import format as fmt
from oracle import glorcq_oracle as O
from test_moe_oracle import bar, lora_heavy
from test_moe_oracle_library import mixtral_block, qwen2_block, qwen3_block, run, same_routing

transformers = pytest.importorskip("transformers")


def rotation(q: fmt.TurboMat) -> torch.Tensor:
    """R (K, K) fp64 with x_rot = R x."""
    if q.signs is not None:
        K = q.K
        H = torch.from_numpy(O.hadamard_sylvester(K))
        return H * q.signs.double()[None, :] / np.sqrt(K)
    return q.Pi.double()


def turbo_weight(q: fmt.TurboMat, e: int) -> torch.Tensor:
    """W_t R in fp64: the expert's dense weight (x_rot = R x)."""
    idx = torch.from_numpy(O.unpack_indices_2bit(q.packed[e].numpy(), q.K)).long()
    Wt = q.centroids.double()[idx] * q.norms[e].double()[:, None]
    return Wt @ rotation(q)


def folded(p, proj, e):
    c = int(p.cluster_of[proj][e])
    W = turbo_weight(p.experts[proj], e)
    return W + p.SV[proj][e].double() @ p.U[proj][c].double().T


def load_turbo_experts(experts, p):
    with torch.no_grad():
        for e in range(p.E):
            experts.gate_up_proj[e].copy_(torch.cat([folded(p, "gate", e), folded(p, "up", e)]))
            experts.down_proj[e].copy_(folded(p, "down", e))


def library(p, kind):
    """The library block of `kind` with p's turbo experts loaded densely."""
    import test_moe_oracle_library as L
    saved = L.load_experts
    L.load_experts = load_turbo_experts
    try:
        return {"qwen2": qwen2_block, "qwen3": qwen3_block, "mixtral": mixtral_block}[kind](p)
    finally:
        L.load_experts = saved


def problem(B=4, seed=31, shared=0, norm=True, E=8, top_k=2, rot_gate_up="rht",
            rot_down="qr"):
    p = fmt.make_turbo_moe(H=256, E=E, inter=384, top_k=top_k, n_clusters=3, rank=16,
                           shared_inter=shared, B=B, seed=seed, norm_topk_prob=norm,
                           rot_gate_up=rot_gate_up, rot_down=rot_down)
    return lora_heavy(p)


@pytest.mark.parametrize("B,seed", [(1, 31), (6, 32)])
def test_turbo_oracle_matches_mixtral_block(B, seed):
    """Top-2 of 8, renormalised; gate/up rotated by an RHT, down by Pi."""
    p = problem(B=B, seed=seed)
    blk = library(p, "mixtral")
    assert same_routing(p, blk)
    ref = run(blk, p)
    assert bar(O.moe_forward(p, exact=True), ref)
    assert bar(O.moe_forward(p, exact=False), ref)


@pytest.mark.parametrize("rots", [("qr", "rht"), ("qr", "qr")])
def test_turbo_oracle_matches_qwen3_block_other_rotations(rots):
    """Every projection rotated by Pi, and an RHT down projection (inter 384 is
    not a power of two, so the RHT case takes inter 512)."""
    gu, dn = rots
    if dn == "rht":
        p = fmt.make_turbo_moe(H=256, E=16, inter=512, top_k=4, n_clusters=3, rank=16,
                               shared_inter=0, B=3, seed=33, norm_topk_prob=True,
                               rot_gate_up=gu, rot_down=dn)
        p = lora_heavy(p)
    else:
        p = problem(B=3, seed=33, E=16, top_k=4, rot_gate_up=gu, rot_down=dn)
    blk = library(p, "qwen3")
    assert same_routing(p, blk)
    assert bar(O.moe_forward(p, exact=True), run(blk, p))


def test_turbo_oracle_matches_qwen2_block_with_shared_expert():
    """Config-2 semantics with turbo routed experts and the 4-bit GPTQ shared
    expert behind its sigmoid gate."""
    p = problem(B=4, seed=35, shared=512, norm=False)
    blk = library(p, "qwen2")
    assert same_routing(p, blk)
    assert bar(O.moe_forward(p, exact=True), run(blk, p))


def test_turbo_planted_mistakes_fail_against_library():
    p = problem(B=6, seed=32)
    ref = run(library(p, "mixtral"), p)
    assert bar(O.moe_forward(p), ref)
    # the RHT signs of gate/up flipped on half the coordinates
    q = problem(B=6, seed=32)
    s = q.experts["gate"].signs.clone()
    s[: s.numel() // 2] *= -1
    q.experts["gate"].signs = q.experts["up"].signs = s
    assert not bar(O.moe_forward(q), ref)
    # Pi applied transposed (x Pi instead of x Pi^T)
    q = problem(B=6, seed=32)
    q.experts["down"].Pi = q.experts["down"].Pi.T.contiguous()
    assert not bar(O.moe_forward(q), ref)
    # the codebook reversed (index i -> C[3 - i])
    q = problem(B=6, seed=32)
    for proj in fmt.PROJS:
        q.experts[proj].centroids = q.experts[proj].centroids.flip(0)
    assert not bar(O.moe_forward(q), ref)
    # silu(up) * gate
    q = problem(B=6, seed=32)
    for d in (q.experts, q.SV, q.cluster_of, q.U):
        d["gate"], d["up"] = d["up"], d["gate"]
    assert not bar(O.moe_forward(q), ref)
