"""BASELINE config 3 on the GPU: a Mixtral-8x7B-shaped MoE layer (hidden 4096,
ffn 14336, 8 experts, top-2 renormalised, 2-bit g128 SwiGLU experts, rank-64
LoRA with U shared by 2 clusters of 4 experts, no shared expert;
glorcq_amd.format.make_mixtral_layer) against the MoE oracle
(oracle.moe_forward, which tests/test_moe_oracle_library.py pins against
transformers' MixtralSparseMoeBlock).

Decode (M = 1 and 8) runs the block's decode step (glq_moe_decode).  Bars as
tests/test_moe_gpu.py: routing ids identical, logits within one fp16 ulp,
output within the MoE bar (atol 1e-3 + rtol 1e-2 |ref| + 2e-3 row max)."""

import pytest
import torch

from glorcq_amd import format as fmt
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from oracle import glorcq_oracle as O
from test_moe_gpu import check_routing, margin
from test_moe_oracle import bar, lora_heavy, strict_report

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,seed", [(1, 3), (8, 4)])
def test_config3_decode(gpu, B, seed):
    # LoRA factors x3: the low-rank terms are about a third of the main term
    # (x30 as in the config-2 tests would overflow fp16 at K = 14336)
    p = lora_heavy(fmt.make_mixtral_layer(B=B, seed=seed), f=3.0)
    assert margin(p) >= 2
    print(f"config 3 decode B={B} seed={seed}", flush=True)
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    out, logits = blk(p.h.reshape(1, B, p.H).to(gpu))
    torch.cuda.synchronize()
    check_routing(p, logits.cpu())
    ref = O.moe_forward(p)
    got = out.reshape(B, p.H).cpu()
    assert bar(got, ref), float((got.double() - ref).abs().max())
    strict_report(p, got, ref, f"config 3 B={B}")
