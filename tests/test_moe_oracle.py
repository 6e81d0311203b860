"""Pins the MoE-block oracle (oracle/glorcq_oracle.py: route, moe_forward) on
the CPU: the reference's fp16 arithmetic against the fp64 form, the identities
the reference itself relies on, brute force for the router, and planted
mistakes the parity bar must reject."""

import hashlib
import json
import os

import pytest
import torch

from glorcq_amd import format as fmt
from oracle import glorcq_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def small(B=3, seed=5, norm=False):
    # a scaled-down block: H=256, 8 experts, inter 384, top-2, 3 clusters, r=16
    return fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16,
                        shared_inter=512, B=B, seed=seed, norm_topk_prob=norm)


def bar(y, ref, atol=1e-3, rtol=1e-2, rowtol=2e-3):
    """MoE output bar: |y - ref| <= atol + rtol |ref| + rowtol * max_row |ref|.
    The last term allows for fp16 accumulation of terms as large as the row's
    largest output (the reference sums experts and the shared expert in fp16,
    so outputs that cancel to near zero carry an error set by the row scale).
    An output whose reference overflows fp16 (|ref| > 65504) must be that inf
    (config 2's 4-bit shared expert, with zero-points in {1, 2} on codes
    0..15, drives some outputs past 65504); the row scale counts finite
    values only."""
    y = y.double()
    ref = ref.double()
    ref16 = ref.half().double()  # inf where the fp16 output overflows
    inf = ~torch.isfinite(ref16)
    if bool(inf.any()) and not torch.equal(y[inf], ref16[inf]):
        return False
    err = (y - ref).abs()
    rowmax = torch.where(inf, 0.0, ref).abs().amax(dim=-1, keepdim=True)
    ok = (err <= atol + rtol * ref.abs() + rowtol * rowmax) | inf
    return bool(ok.all())


def strict_fraction(y, ref, atol=1e-3, rtol=1e-2):
    """Fraction of outputs within the north star's bar alone, |y - ref| <=
    atol + rtol |ref| (no row term); an output whose reference overflows fp16
    counts as within when it is that inf."""
    y = y.double()
    ref = ref.double()
    ref16 = ref.half().double()
    inf = ~torch.isfinite(ref16)
    ok = (y - ref).abs() <= atol + rtol * ref.abs()
    ok = torch.where(inf, y == ref16, ok)
    return float(ok.double().mean())


def strict_report(p, out, ref, what):
    """The strict-bar fraction of a GPU output beside that of the reference's
    own fp16 CPU arithmetic (oracle.moe_forward(exact=False)) on the same
    problem; the GPU step (fp32 accumulation) must do at least as well."""
    mine = strict_fraction(out, ref)
    fp16 = strict_fraction(O.moe_forward(p, exact=False), ref)
    print(f"{what}: strict bar (atol 1e-3, rtol 1e-2) GPU {mine:.6f}, reference fp16 "
          f"arithmetic {fp16:.6f}", flush=True)
    assert mine >= fp16, (what, mine, fp16)
    return mine, fp16


def test_router_brute_force():
    p = small(B=6)
    logits, w, sel = O.route(p.h, p.router_w, p.top_k, False)
    assert logits.dtype == torch.float16 and w.dtype == torch.float16
    for t in range(6):
        probs = torch.softmax(logits[t].float(), 0)
        order = sorted(range(p.E), key=lambda e: -float(probs[e]))
        assert sel[t].tolist() == order[:p.top_k]
        assert torch.equal(w[t], probs[order[:p.top_k]].half())
    _, wn, _ = O.route(p.h, p.router_w, p.top_k, True)
    assert torch.allclose(wn.float().sum(-1), torch.ones(6), atol=2e-3)


@pytest.mark.parametrize("B", [1, 4])
def test_fp16_reference_within_bar_of_fp64(B):
    p = small(B=B, seed=B)
    assert bar(O.moe_forward(p, exact=False), O.moe_forward(p, exact=True))


def test_dense_equals_sparse():
    """Masked-dense == sparse (moe_block.py:11-13)."""
    p = small(B=2, seed=9)
    assert torch.allclose(O.moe_forward(p, dense=True), O.moe_forward(p), atol=1e-12, rtol=0)


def test_cluster_shared_xu_equals_per_expert():
    """Cluster-shared x*U == per-expert x*U (test_cluster_parallel.py:159)."""
    p = small(B=3, seed=10)
    assert torch.equal(O.moe_forward(p, cluster_shared=False), O.moe_forward(p))


def lora_heavy(q, f=30.0):
    """Scales every U and SV by f so the low-rank terms are a visible part of
    the output (with the config's N(0, 0.01) factors they are ~1e-3 of it)."""
    for proj in fmt.PROJS:
        q.U[proj] = (q.U[proj].float() * f).half()
        q.SV[proj] = (q.SV[proj].float() * f).half()
    return q


def test_planted_mistakes_fail_the_bar():
    p = small(B=4, seed=12)
    good = O.moe_forward(p)
    # shared expert gate dropped
    q = small(B=4, seed=12)
    q.shared_gate_w = torch.full_like(q.shared_gate_w, 60.0)  # sigmoid -> 1
    assert not bar(O.moe_forward(q), good)
    # wrong cluster for the down projection's U / for gate's U (LoRA-heavy)
    heavy = O.moe_forward(lora_heavy(small(B=4, seed=12)))
    for proj in ("down", "gate"):
        q = lora_heavy(small(B=4, seed=12))
        q.cluster_of[proj] = (q.cluster_of[proj] + 1) % q.n_clusters
        assert not bar(O.moe_forward(q), heavy), proj
    # renormalised top-k weights instead of raw
    q = small(B=4, seed=12, norm=True)
    assert not bar(O.moe_forward(q), good)
    # hidden state of another token
    assert not bar(O.moe_forward(p, h=p.h.roll(1, 0)), good)


def _sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def test_config2_generator_fixture():
    """The config-2 draw order (make_moe defaults, seed 0, B=1) hashes to the
    committed fixture."""
    p = fmt.make_moe(B=1, seed=0)
    got = {"router_w": _sha(p.router_w), "shared_gate_w": _sha(p.shared_gate_w),
           "gate_codes": _sha(p.experts["gate"].codes), "down_U": _sha(p.U["down"]),
           "up_SV": _sha(p.SV["up"]), "cluster_of_down": _sha(p.cluster_of["down"]),
           "shared_down_codes": _sha(p.shared["down"].codes), "h": _sha(p.h)}
    with open(os.path.join(GOLDEN, "config2_sha256.json")) as f:
        assert got == json.load(f)
