"""Pins the TurboQuant / RHT functions of the CPU oracle (no GPU), and the
host-side checks of the turbo and RHT C entry points.

The reference's turbo kernel test (inference/kernels/test_kernels.py) draws
unseeded random data and holds no vectors, so the oracle is pinned by what
the mathematics fixes: brute-force loops over the packed bytes, closed forms
(constant codes), the equivalence with the GPTQ container and oracle when the
codebook is (0, 1, 2, 3), and for the Hadamard transform scipy.linalg.hadamard,
orthogonality and the inverse."""

import numpy as np
import pytest
import scipy.linalg
import torch

from glorcq_amd import _lib
from glorcq_amd import format as fmt
from glorcq_amd import hadamard_rotation as HR
from oracle import glorcq_oracle as O


def test_unpack_indices_every_value_every_slot():
    # byte j*64 + v*... : put value v in slot s of byte b, zeros elsewhere
    for s in range(4):
        for v in range(4):
            packed = np.zeros((1, 3), dtype=np.uint8)
            packed[0, 1] = v << (2 * s)
            idx = O.unpack_indices_2bit(packed, 12)
            want = np.zeros(12, dtype=np.int64)
            want[4 + s] = v
            assert np.array_equal(idx[0], want)


def test_unpack_indices_match_int32_container():
    """The same bytes read as little-endian int32 words are the 2-bit packed
    container of the GPTQ path: both unpackers agree code for code."""
    g = np.random.default_rng(0)
    packed = g.integers(0, 256, (5, 64), dtype=np.uint8)
    words = packed.view(np.int32)
    a = O.unpack_indices_2bit(packed, 256)
    b = O.unpack_codes(words, 2, 256)
    assert np.array_equal(a, b)
    p = fmt.make_turbo(256, 5, seed=1)
    assert np.array_equal(p.words()[0].numpy(), p.packed[0].numpy().view(np.int32))


def test_turbo_matmul_bruteforce_tiny():
    p = fmt.make_turbo(32, 6, M=3, seed=2, dist="randn")
    y32 = O.turbo_matmul_fp32(p.x_rot[0], p.packed[0].numpy(), p.norms[0], p.centroids)
    y64 = O.turbo_matmul_fp64(p.x_rot[0], p.packed[0].numpy(), p.norms[0], p.centroids)
    yb = O.turbo_bruteforce(p.x_rot[0].float().numpy(), p.packed[0].numpy(),
                            p.norms[0].numpy(), p.centroids.numpy())
    assert np.allclose(y64.numpy(), yb, rtol=1e-12, atol=1e-12)
    assert np.allclose(y32.numpy(), yb, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("c", range(4))
def test_turbo_matmul_constant_codes_closed_form(c):
    K, N = 128, 3
    byte = c | (c << 2) | (c << 4) | (c << 6)
    packed = np.full((N, K // 4), byte, dtype=np.uint8)
    g = torch.Generator().manual_seed(c)
    x = torch.randn(2, K, generator=g).half()
    norms = torch.tensor([0.5, 1.0, 2.0])
    cent = torch.tensor([-1.25, -0.5, 0.375, 1.5])
    y = O.turbo_matmul_fp64(x, packed, norms, cent)
    want = norms.double()[None, :] * float(cent[c]) * x.double().sum(1, keepdim=True)
    assert torch.allclose(y, want, rtol=1e-12, atol=1e-12)


def test_turbo_matmul_equals_gptq_with_identity_codebook():
    """C = (0,1,2,3), norm 1: the turbo product is x q^T, the GPTQ oracle's
    product with s = 1, z = 0."""
    K, N = 256, 7
    p = fmt.make_turbo(K, N, M=2, seed=3)
    q = torch.from_numpy(O.unpack_indices_2bit(p.packed[0].numpy(), K)).to(torch.int32)
    y = O.turbo_matmul_fp64(p.x_rot[0], p.packed[0].numpy(), torch.ones(N),
                            torch.tensor([0.0, 1.0, 2.0, 3.0]))
    ones = torch.ones(N, K // 128, dtype=torch.float16)
    zeros = torch.zeros(N, K // 128, dtype=torch.float16)
    yg = O.linear_forward_fp64(p.x_rot[0], q, ones, zeros, 128, exact_weights=True)
    assert torch.allclose(y, yg.double(), rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("d", [2, 16, 256])
def test_hadamard_matches_scipy(d):
    assert np.array_equal(O.hadamard_sylvester(d), scipy.linalg.hadamard(d))


def test_rht_forward_properties():
    d = 64
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, d, generator=g)
    signs = O.generate_rht_signs(d, seed=7)
    y = O.rht_forward(x, signs)
    H = torch.from_numpy(scipy.linalg.hadamard(d)).double()
    assert torch.allclose(y, (x.double() * signs.double()) @ H / d ** 0.5, atol=1e-12)
    assert torch.allclose(y.norm(dim=1), x.double().norm(dim=1), rtol=1e-12)
    assert torch.allclose(O.rht_backward(y, signs), x.double(), atol=1e-12)
    e0 = torch.zeros(1, d)
    e0[0, 0] = 1.0
    assert torch.allclose(O.rht_forward(e0, torch.ones(d)),
                          torch.full((1, d), d ** -0.5, dtype=torch.float64))


def test_rht_signs_host_mirror():
    s = O.generate_rht_signs(2048, seed=42)
    h = HR.generate_rht_signs(2048, seed=42, device="cpu")
    assert torch.equal(s, h)
    assert set(s.unique().tolist()) == {-1.0, 1.0}
    assert not torch.equal(s, O.generate_rht_signs(2048, seed=43))


def test_turbo_entry_point_checks():
    """Bad shapes come back as errors on the host, before any launch."""
    lib = _lib.load()
    P = 1 << 12
    rc = lib.glq_turbo_gemv_batched(1, P, 0, 1, 100, 64, P, 0, P, 0, P, None, 0, None, 0, 0,
                                    None, 0, P, 0, None)
    assert rc == 1 and b"multiple of 64" in lib.glq_last_error()
    rc = lib.glq_turbo_gemv_batched(1, P + 2, 0, 1, 128, 64, P, 0, P, 0, P, None, 0, None, 0, 0,
                                    None, 0, P, 0, None)
    assert rc == 1 and b"aligned" in lib.glq_last_error()
    rc = lib.glq_turbo_gemv_batched(1, P, 0, 1, 128, 64, P, 0, P, 0, P, None, 0, P, 0, 12,
                                    None, 0, P, 0, None)
    assert rc == 1 and b"rank" in lib.glq_last_error()
    rc = lib.glq_turbo_gemv_batched(1, P, 0, 1, 128, 64, P, 0, P, 0, P, None, 0, P, 0, 16,
                                    None, 0, P, 0, None)
    assert rc == 1 and b"xU" in lib.glq_last_error()
    # empty work is a no-op (turbo_matmul.cu:287-289)
    assert lib.glq_turbo_gemv_batched(1, None, 0, 0, 128, 64, None, 0, None, 0, None, None, 0,
                                      None, 0, 0, None, 0, None, 0, None) == 0
    rc = lib.glq_rht(P, 0, 2, 48, P, 0, P + 4096, 0, None)
    assert rc == 1 and b"power of two" in lib.glq_last_error()
    rc = lib.glq_rht(P, 0, 2, 64, P, 0, P, 0, None)
    assert rc == 1 and b"alias" in lib.glq_last_error()
    assert lib.glq_rht(None, 0, 0, 64, None, 0, None, 0, None) == 0


def test_turbo_bytes():
    assert fmt.turbo_bytes(1, 2048, 1408) == 1408 * 512 + 4 * 1408 + 2 * (2048 + 1408)
