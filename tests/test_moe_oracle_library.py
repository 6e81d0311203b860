"""Pins the MoE block combine of the oracle (oracle/glorcq_oracle.py:
moe_forward) against a library routine: transformers' own sparse MoE blocks.

The reference's block (GraphCompatibleMoeBlock.forward, inference/moe_block.py:
381-436, and GLoRCQExperts.forward, inference/quantized_linear.py:395-428)
reproduces the semantics of the Hugging Face blocks it replaces: a softmax
router with top-k (renormalised when norm_topk_prob), SwiGLU experts
down(silu(gate(x)) * up(x)) weighted by the routing weight, and for Qwen2-MoE a
shared expert scaled by sigmoid(h . w_sg).  transformers 5.x implements each of
these as plain torch code (Qwen2MoeSparseMoeBlock: shared expert + sigmoid
gate, Qwen3MoeSparseMoeBlock: norm_topk_prob, no shared expert,
MixtralSparseMoeBlock: top-2 always renormalised = config 3), so running them in
float64 with the exact dequantized weights fixes what the oracle's combine must
compute.

The low-rank term is folded into each expert's dense weight as
W_e + SV_e U_c(e)^T (exact in fp64); the oracle keeps the reference's fp16
rounding points (a = fp16(x U), the fp16 SwiGLU product, fp16 routing weights),
which the MoE bar of test_moe_oracle.bar absorbs.  Planted mistakes in what
the oracle is given (gate and up swapped = silu(up) * gate; the shared expert
added outside its gate; renormalisation switched; the wrong cluster's U) must
fail that bar against the library block.
"""

import pytest
import torch

from glorcq_amd import format as fmt
from oracle import glorcq_oracle as O
from test_moe_oracle import bar, lora_heavy

transformers = pytest.importorskip("transformers")


def exact_weight(q: fmt.QMat, e: int) -> torch.Tensor:
    """fp64 (N, K) exact weights s * (q - z) of expert e."""
    qi = torch.from_numpy(O.unpack_codes(q.codes[e].numpy(), q.bits, q.K))
    return O.dequant_fp32(qi, q.scales[e], q.zeros[e], q.group).double()


def folded(p: fmt.MoEProblem, proj: str, e: int) -> torch.Tensor:
    """W_e + SV_e U_c^T in fp64: the expert's dense weight with its low-rank
    correction (y = x W^T + (x U) SV^T)."""
    c = int(p.cluster_of[proj][e])
    W = exact_weight(p.experts[proj], e)
    return W + p.SV[proj][e].double() @ p.U[proj][c].double().T


def load_experts(experts, p):
    with torch.no_grad():
        for e in range(p.E):
            experts.gate_up_proj[e].copy_(torch.cat([folded(p, "gate", e), folded(p, "up", e)]))
            experts.down_proj[e].copy_(folded(p, "down", e))


def qwen2_block(p: fmt.MoEProblem):
    from transformers import Qwen2MoeConfig
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeSparseMoeBlock
    cfg = Qwen2MoeConfig(hidden_size=p.H, num_experts=p.E, moe_intermediate_size=p.inter,
                         num_experts_per_tok=p.top_k, norm_topk_prob=p.norm_topk_prob,
                         shared_expert_intermediate_size=p.shared["gate"].N,
                         hidden_act="silu")
    blk = Qwen2MoeSparseMoeBlock(cfg).double()
    with torch.no_grad():
        blk.gate.weight.copy_(p.router_w.double())
        load_experts(blk.experts, p)
        blk.shared_expert.gate_proj.weight.copy_(exact_weight(p.shared["gate"], 0))
        blk.shared_expert.up_proj.weight.copy_(exact_weight(p.shared["up"], 0))
        blk.shared_expert.down_proj.weight.copy_(exact_weight(p.shared["down"], 0))
        blk.shared_expert_gate.weight.copy_(p.shared_gate_w.double())
    return blk


def qwen3_block(p: fmt.MoEProblem):
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
    cfg = Qwen3MoeConfig(hidden_size=p.H, num_experts=p.E, moe_intermediate_size=p.inter,
                         num_experts_per_tok=p.top_k, norm_topk_prob=p.norm_topk_prob,
                         hidden_act="silu")
    blk = Qwen3MoeSparseMoeBlock(cfg).double()
    with torch.no_grad():
        blk.gate.weight.copy_(p.router_w.double())
        load_experts(blk.experts, p)
    return blk


def mixtral_block(p: fmt.MoEProblem):
    from transformers import MixtralConfig
    from transformers.models.mixtral.modeling_mixtral import MixtralSparseMoeBlock
    cfg = MixtralConfig(hidden_size=p.H, num_local_experts=p.E, intermediate_size=p.inter,
                        num_experts_per_tok=p.top_k, hidden_act="silu")
    blk = MixtralSparseMoeBlock(cfg).double().eval()
    with torch.no_grad():
        blk.gate.weight.copy_(p.router_w.double())
        load_experts(blk.experts, p)
    return blk


def run(blk, p):
    with torch.no_grad():
        out = blk(p.h.double().view(1, p.B, p.H))
    if isinstance(out, tuple):
        out = out[0]
    return out.view(p.B, p.H)


def same_routing(p, blk):
    """The library router (fp64 logits) and the oracle's (fp16 logits) pick the
    same experts: the seeds below have no near-tie at the top-k boundary."""
    _, _, sel = O.route(p.h, p.router_w, p.top_k, p.norm_topk_prob, exact=True)
    with torch.no_grad():
        _, _, lib_sel = blk.gate(p.h.double())
    return torch.equal(sel.sort(-1).values, lib_sel.sort(-1).values)


def qwen2_problem(B=4, seed=21, norm=False, heavy=True):
    p = fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16,
                     shared_inter=512, B=B, seed=seed, norm_topk_prob=norm)
    return lora_heavy(p) if heavy else p


def no_shared_problem(B=4, seed=23, E=8, top_k=2, norm=True):
    p = fmt.make_moe(H=256, E=E, inter=384, top_k=top_k, n_clusters=2, rank=16,
                     shared_inter=0, B=B, seed=seed, norm_topk_prob=norm)
    return lora_heavy(p)


@pytest.mark.parametrize("B,seed", [(1, 21), (4, 22), (6, 24)])
def test_oracle_matches_qwen2_moe_block(B, seed):
    """Config-2 semantics: softmax top-k without renormalisation, cluster-shared
    low-rank experts, 4-bit shared expert behind a sigmoid gate."""
    p = qwen2_problem(B=B, seed=seed)
    blk = qwen2_block(p)
    assert same_routing(p, blk)
    assert bar(O.moe_forward(p, exact=True), run(blk, p))
    assert bar(O.moe_forward(p, exact=False), run(blk, p))


@pytest.mark.parametrize("B,seed", [(1, 23), (5, 25)])
def test_oracle_matches_qwen3_moe_block(B, seed):
    """Config-4 semantics: renormalised top-k (norm_topk_prob), no shared expert."""
    p = no_shared_problem(B=B, seed=seed, E=16, top_k=4)
    blk = qwen3_block(p)
    assert same_routing(p, blk)
    assert bar(O.moe_forward(p, exact=True), run(blk, p))


@pytest.mark.parametrize("B,seed", [(1, 27), (8, 28)])
def test_oracle_matches_mixtral_block(B, seed):
    """Config-3 semantics: top-2 of 8, weights renormalised, no shared expert."""
    p = no_shared_problem(B=B, seed=seed, E=8, top_k=2, norm=True)
    blk = mixtral_block(p)
    assert same_routing(p, blk)
    assert bar(O.moe_forward(p, exact=True), run(blk, p))


def _swap_gate_up(p):
    for d in (p.experts, p.SV, p.cluster_of, p.U):
        d["gate"], d["up"] = d["up"], d["gate"]
    return p


def test_planted_mistakes_fail_against_library():
    p = qwen2_problem(B=4, seed=22)
    ref = run(qwen2_block(p), p)
    assert bar(O.moe_forward(p), ref)
    # silu(up) * gate instead of silu(gate) * up
    assert not bar(O.moe_forward(_swap_gate_up(qwen2_problem(B=4, seed=22))), ref)
    # shared expert added outside its gate (sigmoid -> 1; a softmax over the
    # single gate logit gives the same 1)
    q = qwen2_problem(B=4, seed=22)
    q.shared_gate_w = torch.full_like(q.shared_gate_w, 60.0)
    assert not bar(O.moe_forward(q), ref)
    # renormalised top-k where the block does not renormalise
    assert not bar(O.moe_forward(qwen2_problem(B=4, seed=22, norm=True)), ref)
    # the down projection's U taken from the wrong cluster
    q = qwen2_problem(B=4, seed=22)
    q.cluster_of["down"] = (q.cluster_of["down"] + 1) % q.n_clusters
    assert not bar(O.moe_forward(q), ref)
    # Mixtral: weights not renormalised must fail too
    m = no_shared_problem(B=8, seed=28)
    mref = run(mixtral_block(m), m)
    m.norm_topk_prob = False
    assert not bar(O.moe_forward(m), mref)
