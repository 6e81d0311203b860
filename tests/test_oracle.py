"""Pins the CPU oracle (oracle/glorcq_oracle.py) without the reference.

The reference ships no golden vectors or KAT files (its kernel tests draw
unseeded random data), so each oracle function is pinned by closed forms,
brute force on tiny inputs, hand-computed words, and planted mistakes that the
parity bar must reject.  Runs on the CPU.
"""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from glorcq_amd import format as fmt
from oracle import glorcq_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- packing ----
@pytest.mark.parametrize("bits", [2, 4])
def test_pack_every_value_in_every_slot(bits):
    cpw = 32 // bits
    for slot in range(cpw):
        for v in range(1 << bits):
            q = np.zeros((1, cpw), dtype=np.int64)
            q[0, slot] = v
            w = O.pack_codes(q, bits)
            assert w.shape == (1, 1)
            assert np.uint32(w[0, 0]) == np.uint32(v << (bits * slot))
            assert np.array_equal(O.unpack_codes(w, bits, cpw), q.astype(np.int32))


def test_hand_computed_words():
    # 0x1B = 0b00011011 -> 2-bit slots (LSB first) 3, 2, 1, 0; upper bytes 0.
    w = np.array([[0x1B]], dtype=np.int32)
    assert O.unpack_codes(w, 2, 16)[0, :4].tolist() == [3, 2, 1, 0]
    assert O.unpack_codes(w, 2, 16)[0, 4:].tolist() == [0] * 12
    # 0x80000000: top 2-bit slot is 2 (0b10); top nibble is 8.
    w = np.array([[-(2**31)]], dtype=np.int32)
    assert O.unpack_codes(w, 2, 16)[0].tolist() == [0] * 15 + [2]
    assert O.unpack_codes(w, 4, 8)[0].tolist() == [0] * 7 + [8]
    # 0x76543210 -> nibbles 0..7 in order.
    w = np.array([[0x76543210]], dtype=np.int32)
    assert O.unpack_codes(w, 4, 8)[0].tolist() == list(range(8))


def test_sym_sign_extension():
    q = np.array([[-2, -1, 0, 1] * 4], dtype=np.int64)
    w = O.pack_codes(q, 2)
    assert O.unpack_codes(w, 2, 16, sym=False)[0, :4].tolist() == [2, 3, 0, 1]
    assert O.unpack_codes(w, 2, 16, sym=True)[0].tolist() == q[0].tolist()
    q4 = np.array([list(range(-8, 0))], dtype=np.int64)
    assert O.unpack_codes(O.pack_codes(q4, 4), 4, 8, sym=True)[0].tolist() == list(range(-8, 0))


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_unpack_roundtrip_random_words(bits):
    rng = np.random.default_rng(1)
    words = rng.integers(-(2**31), 2**31, size=(7, 12), dtype=np.int64).astype(np.int32)
    K = 12 * 32 // bits
    assert np.array_equal(O.pack_codes(O.unpack_codes(words, bits, K), bits), words)


@pytest.mark.parametrize("bits", [2, 4])
def test_product_pack_matches_oracle(bits):
    g = torch.Generator().manual_seed(3)
    q = torch.randint(0, 1 << bits, (33, 256), generator=g, dtype=torch.int32)
    assert np.array_equal(fmt.pack_codes(q, bits).numpy(), O.pack_codes(q.numpy(), bits))
    qs = torch.randint(-(1 << (bits - 1)), 1 << (bits - 1), (5, 128), generator=g,
                       dtype=torch.int32)
    assert np.array_equal(fmt.pack_codes(qs, bits).numpy(), O.pack_codes(qs.numpy(), bits))


# ------------------------------------------------------------- dequantize ----
@pytest.mark.parametrize("bits", [2, 4])
def test_dequant_fp16_closed_form_all_pairs(bits):
    """Integer zeros: W must be the correctly rounded fp16 of s*(q-z)."""
    levels = 1 << bits
    q = torch.arange(levels, dtype=torch.int32).repeat_interleave(levels).reshape(1, -1)
    z = torch.arange(levels, dtype=torch.int32).repeat(levels).reshape(1, -1)
    K = q.shape[1]
    g = torch.Generator().manual_seed(5)
    scales = (torch.randn(1, K, generator=g) * 0.02).abs().half()
    W = O.dequant_fp16(q, scales, z.half(), groupsize=1)
    exact = (scales.double() * (q.double() - z.double())).numpy().astype(np.float16)
    assert np.array_equal(W.numpy().view(np.uint16), exact.view(np.uint16))


def test_dequant_fp16_noninteger_zeros_two_roundings():
    """Non-integer zeros (the reference kernel tests' distribution): two fp16
    roundings, fp16(q - z) then fp16(. * s), each the correctly rounded result."""
    g = torch.Generator().manual_seed(7)
    q = torch.randint(0, 4, (16, 256), generator=g, dtype=torch.int32)
    s = (torch.randn(16, 2, generator=g).abs() * 0.1 + 0.01).half()
    z = (torch.randn(16, 2, generator=g) * 0.5).half()
    W = O.dequant_fp16(q, s, z, groupsize=128)
    zz = z.double().repeat_interleave(128, dim=1).numpy()
    ss = s.double().repeat_interleave(128, dim=1).numpy()
    t = (q.double().numpy() - zz).astype(np.float16).astype(np.float64)
    exact = (t * ss).astype(np.float16)
    assert np.array_equal(W.numpy().view(np.uint16), exact.view(np.uint16))


def test_dequant_sym():
    q = torch.tensor([[-2, -1, 0, 1]], dtype=torch.int32)
    s = torch.tensor([[0.5]], dtype=torch.float16)
    W = O.dequant_fp16(q, s, None, groupsize=4, sym=True)
    assert W.tolist() == [[-1.0, -0.5, 0.0, 0.5]]


def test_dequant_fp32_is_exact_product():
    """fp32 dequant of an 11-bit scale times a small integer is exact: compare
    with fp64 for every 4-bit (q, z) pair."""
    q = torch.arange(16, dtype=torch.int32).repeat_interleave(16).reshape(1, -1)
    z = torch.arange(16, dtype=torch.int32).repeat(16).reshape(1, -1)
    s = (torch.randn(1, 256, generator=torch.Generator().manual_seed(8)) * 0.02).abs().half()
    W = O.dequant_fp32(q, s, z.half(), groupsize=1).double()
    assert torch.equal(W, s.double() * (q.double() - z.double()))


def test_fp32_forward_within_bar_of_exact_fp64():
    for bits, K, N in [(2, 2048, 1408), (4, 2048, 2048), (4, 5632, 256)]:
        p = fmt.make_linear(K, N, bits=bits, rank=64, M=4, seed=K + N)
        y32 = O.linear_forward_fp32(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
        y64 = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV,
                                    exact_weights=True)
        assert O.parity_ok(y32, y64), (bits, K, N)


def test_dequant_fp32_matches_fp16_for_integer_zeros():
    p = fmt.make_linear(256, 40, bits=4, seed=11)
    w16 = O.dequant_fp16(p.q, p.scales, p.zeros, 128)
    w32 = O.dequant_fp32(p.q, p.scales, p.zeros, 128)
    # s*(q-z) with integer (q-z): fp32 product rounded once to fp16 == fp16 route
    assert torch.equal(w32.half(), w16)


# ---------------------------------------------------------------- forward ----
def test_fp64_matmul_orientation_bruteforce():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 8, generator=g).double()
    W = torch.randn(3, 8, generator=g).double()
    assert np.allclose((x @ W.T).numpy(), O.fp64_matvec_bruteforce(x.numpy(), W.numpy()),
                       rtol=0, atol=1e-12)


def test_config0_forward_within_bar_of_fp64():
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=0)
    y16 = O.linear_forward_fp16(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
    y64 = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
    assert y16.dtype == torch.float16 and y16.shape == (1, 1408)
    assert O.parity_ok(y16, y64)
    y32 = O.linear_forward_fp32(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
    assert O.parity_ok(y32, y64)


def test_planted_mistakes_fail_the_bar():
    """Each plausible mistake must be caught by the parity bar."""
    p = fmt.make_linear(512, 96, bits=2, rank=32, M=2, seed=4)
    args = dict(U=p.U, SV=p.SV)
    good = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, 128, **args)
    # dropped zero-point
    bad = O.linear_forward_fp64(p.x, p.q, p.scales, torch.zeros_like(p.zeros), 128, **args)
    assert not O.parity_ok(bad, good)
    # dropped low-rank term
    bad = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, 128)
    assert not O.parity_ok(bad, good)
    # wrong group index (scales of the next group)
    bad = O.linear_forward_fp64(p.x, p.q, p.scales.roll(1, dims=1), p.zeros, 128, **args)
    assert not O.parity_ok(bad, good)
    # codes read in the wrong bit order within each word
    wrong = p.q.reshape(96, -1, 16).flip(-1).reshape(96, 512)
    bad = O.linear_forward_fp64(p.x, wrong, p.scales, p.zeros, 128, **args)
    assert not O.parity_ok(bad, good)
    # wrong sign of the low-rank term
    bad = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=-p.SV)
    assert not O.parity_ok(bad, good)


def test_precomputed_xu_equals_inline():
    p = fmt.make_linear(256, 64, bits=4, rank=32, M=3, seed=9)
    a = p.x @ p.U
    y1 = O.linear_forward_fp16(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
    y2 = O.linear_forward_fp16(p.x, p.q, p.scales, p.zeros, 128, SV=p.SV, precomputed_xU=a)
    assert torch.equal(y1, y2)


# ------------------------------------------------------- golden fixtures ----
def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def test_config0_generator_fixture():
    """The seeded config-0 draw order is part of the oracle: its tensors must
    hash to the committed fixture (tests/golden/make_golden.py wrote it)."""
    with open(os.path.join(GOLDEN, "config0_sha256.json")) as f:
        want = json.load(f)
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=0)
    got = {"codes": _sha(p.codes), "scales": _sha(p.scales), "zeros": _sha(p.zeros),
           "U": _sha(p.U), "SV": _sha(p.SV), "x": _sha(p.x)}
    assert got == want


def test_small_forward_fixture():
    """Committed small vectors: inputs regenerate from the seed; the expected
    fp64 output is stored, and the oracle must meet the bar against it."""
    d = np.load(os.path.join(GOLDEN, "small_linear.npz"))
    p = fmt.make_linear(int(d["K"]), int(d["N"]), bits=int(d["bits"]), rank=int(d["rank"]),
                        M=int(d["M"]), seed=int(d["seed"]))
    assert np.array_equal(p.codes.numpy(), d["codes"])
    y64 = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
    assert np.allclose(y64.numpy(), d["y64"], rtol=0, atol=1e-9)
    y16 = O.linear_forward_fp16(p.x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)
    assert O.parity_ok(y16, torch.from_numpy(d["y64"]))
