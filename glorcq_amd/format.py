"""Host-side helpers for the packed GLoRCQ weight format and seeded synthetic
problems of the benchmark configurations.

Packed format (load-time, device-independent): b-bit codes, b in {2, 4}, packed
LSB-first along K into int32 words, code k of a row at bit b*(k % (32/b)) of
word k // (32/b).  This is the reference's LSB-first sub-byte convention
(inference/kernels/__init__.py:113-118, inference/quantized_linear.py:115-146)
read as little-endian 32-bit words.  Symmetric codes are b-bit two's
complement (the reference's `two_compl`, quantizer/quantizer.py:145-146).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


def codes_per_word(bits: int) -> int:
    if bits not in (2, 4):
        raise ValueError(f"bits must be 2 or 4 (got {bits})")
    return 32 // bits


def pack_codes(q: torch.Tensor, bits: int) -> torch.Tensor:
    """(N, K) integer codes -> (N, K*bits/32) int32, on q's device (CPU or GPU).

    Values are masked to `bits` bits, so signed symmetric codes pack as two's
    complement.
    """
    cpw = codes_per_word(bits)
    N, K = q.shape
    if K % cpw:
        raise ValueError(f"K={K} must be a multiple of {cpw}")
    mask = (1 << bits) - 1
    v = (q.to(torch.int64) & mask).reshape(N, K // cpw, cpw)
    shifts = torch.arange(cpw, device=q.device, dtype=torch.int64) * bits
    words = (v << shifts).sum(dim=-1)  # < 2^32, fits int64
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32).contiguous()


@dataclass
class LinearProblem:
    """One GLoRCQ linear layer plus its activation, all on the CPU."""

    q: torch.Tensor        # (N, K) int32 codes (unsigned, or signed if sym)
    codes: torch.Tensor    # (N, K*bits/32) int32 packed
    scales: torch.Tensor   # (N, G) fp16
    zeros: torch.Tensor    # (N, G) fp16
    U: torch.Tensor        # (K, r) fp16, input-side factor (reference `U`)
    SV: torch.Tensor       # (N, r) fp16, output-side factor (reference `SV`)
    x: torch.Tensor        # (M, K) fp16
    bits: int
    group: int
    sym: bool = False

    @property
    def N(self) -> int:
        return self.q.shape[0]

    @property
    def K(self) -> int:
        return self.q.shape[1]

    @property
    def rank(self) -> int:
        return self.U.shape[1]


def make_linear(K: int, N: int, bits: int = 2, group: int = 128, rank: int = 64,
                M: int = 1, seed: int = 0, sym: bool = False,
                generator: torch.Generator | None = None) -> LinearProblem:
    """Seeded problem in the benchmark configurations' draw order.

    Draw order (one CPU generator, fp32 samples rounded to fp16):
      codes (N,K) uniform {0..2^b-1}; scale (N,G) = |N(0,0.02)|;
      zero (N,G) uniform {1,2}; V (r,K) = N(0,0.01) (the input-side factor,
      stored as U = V^T); U_out (N,r) = N(0,0.01) (stored as SV); x (M,K) =
      N(0,1).  sym=True draws signed codes in [-2^(b-1), 2^(b-1)-1] instead
      and the zero draw is kept (unused) so later draws do not shift.
    """
    g = generator if generator is not None else torch.Generator().manual_seed(seed)
    G = K // group
    if sym:
        h = 1 << (bits - 1)
        q = torch.randint(-h, h, (N, K), generator=g, dtype=torch.int32)
    else:
        q = torch.randint(0, 1 << bits, (N, K), generator=g, dtype=torch.int32)
    scales = (torch.randn(N, G, generator=g) * 0.02).abs().half()
    zeros = torch.randint(1, 3, (N, G), generator=g, dtype=torch.int32).half()
    V = (torch.randn(rank, K, generator=g) * 0.01).half()
    U_out = (torch.randn(N, rank, generator=g) * 0.01).half()
    x = torch.randn(M, K, generator=g).half()
    return LinearProblem(q=q, codes=pack_codes(q, bits), scales=scales, zeros=zeros,
                         U=V.t().contiguous(), SV=U_out, x=x, bits=bits, group=group,
                         sym=sym)


def algorithmic_bytes(M: int, K: int, N: int, bits: int, group: int, rank: int) -> int:
    """HBM bytes one fused call must move at minimum: packed codes, fp16 scale and
    zero per group, fp16 U (K x r) and SV (N x r), fp16 x in and y out."""
    G = K // group
    return N * K * bits // 8 + 4 * N * G + 2 * rank * (K + N) + 2 * M * (K + N)


def algorithmic_flops(M: int, K: int, N: int, rank: int) -> int:
    return 2 * M * (N * K + rank * (K + N))
