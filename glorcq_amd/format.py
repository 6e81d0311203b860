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


# ---------------------------------------------------------------------------
# MoE block (BASELINE config 2 shape: Qwen1.5-MoE-A2.7B decode)
# ---------------------------------------------------------------------------
PROJS = ("gate", "up", "down")


@dataclass
class QMat:
    """Packed group-quantized weights of E (or 1) matrices (N, K)."""

    codes: torch.Tensor    # (E, N, K*bits/32) int32
    scales: torch.Tensor   # (E, N, G) fp16
    zeros: torch.Tensor    # (E, N, G) fp16
    bits: int
    group: int

    @property
    def N(self) -> int:
        return self.codes.shape[1]

    @property
    def K(self) -> int:
        return self.codes.shape[2] * (32 // self.bits)


@dataclass
class MoEProblem:
    """One Qwen2-MoE style block: router, E routed SwiGLU experts with
    cluster-shared LoRA U (input side) and per-expert SV, a 4-bit shared expert
    (no LoRA) with a sigmoid gate, and B tokens of hidden state."""

    H: int
    E: int
    inter: int
    top_k: int
    norm_topk_prob: bool
    rank: int
    n_clusters: int
    router_w: torch.Tensor         # (E, H) fp16
    shared_gate_w: torch.Tensor    # (1, H) fp16
    experts: dict                  # proj -> QMat (E, N, .)
    SV: dict                       # proj -> (E, N, r) fp16
    cluster_of: dict               # proj -> (E,) int64
    U: dict                        # proj -> (C, K, r) fp16
    shared: dict | None            # proj -> QMat (1, N, .); None: no shared expert
    h: torch.Tensor                # (B, H) fp16

    @property
    def B(self) -> int:
        return self.h.shape[0]


def _rand_qmat(g, E, N, K, bits, group) -> QMat:
    """Uniform codes drawn as random packed words (every code uniform over
    0..2^b-1), |N(0,0.02)| fp16 scales, zero-points uniform over {1, 2}."""
    G = K // group
    words = torch.randint(-(2**31), 2**31 - 1, (E, N, K * bits // 32), generator=g,
                          dtype=torch.int64).to(torch.int32)
    scales = (torch.randn(E, N, G, generator=g) * 0.02).abs().half()
    zeros = torch.randint(1, 3, (E, N, G), generator=g, dtype=torch.int32).half()
    return QMat(codes=words, scales=scales, zeros=zeros, bits=bits, group=group)


def make_moe(H=2048, E=60, inter=1408, top_k=4, n_clusters=16, rank=64, shared_inter=5632,
             B=1, bits=2, shared_bits=4, group=128, norm_topk_prob=False,
             seed=0, balanced_clusters=False) -> MoEProblem:
    """Seeded MoE block in a fixed draw order (one CPU generator):
    router W (E,H) N(0,0.02); shared-expert gate w (1,H) N(0,0.02); then for
    proj in (gate, up, down): cluster assignment randint(0, C, (E,)), U (C,K,r)
    N(0,0.01), expert weights (codes, scales, zeros as in make_linear), SV
    (E,N,r) N(0,0.01); then the shared expert's gate, up, down weights
    (shared_bits, no LoRA; skipped when shared_inter = 0); then h (B,H) N(0,1).  All fp32 draws rounded to fp16.
    balanced_clusters: the cluster assignment is randperm(E) % C instead (clusters
    of E/C experts each).
    Defaults are BASELINE config 2 (Qwen1.5-MoE-A2.7B)."""
    g = torch.Generator().manual_seed(seed)
    router_w = (torch.randn(E, H, generator=g) * 0.02).half()
    shared_gate_w = (torch.randn(1, H, generator=g) * 0.02).half()
    dims = {"gate": (H, inter), "up": (H, inter), "down": (inter, H)}
    experts, SV, cluster_of, U = {}, {}, {}, {}
    for proj in PROJS:
        K, N = dims[proj]
        if balanced_clusters:
            cluster_of[proj] = torch.randperm(E, generator=g) % n_clusters
        else:
            cluster_of[proj] = torch.randint(0, n_clusters, (E,), generator=g)
        U[proj] = (torch.randn(n_clusters, K, rank, generator=g) * 0.01).half()
        experts[proj] = _rand_qmat(g, E, N, K, bits, group)
        SV[proj] = (torch.randn(E, N, rank, generator=g) * 0.01).half()
    sdims = {"gate": (H, shared_inter), "up": (H, shared_inter), "down": (shared_inter, H)}
    shared = None if shared_inter == 0 else {
        proj: _rand_qmat(g, 1, sdims[proj][1], sdims[proj][0], shared_bits, group)
        for proj in PROJS}
    h = torch.randn(B, H, generator=g).half()
    return MoEProblem(H=H, E=E, inter=inter, top_k=top_k, norm_topk_prob=norm_topk_prob,
                      rank=rank, n_clusters=n_clusters, router_w=router_w,
                      shared_gate_w=shared_gate_w, experts=experts, SV=SV,
                      cluster_of=cluster_of, U=U, shared=shared, h=h)


def make_mixtral_layer(B=1, seed=0, **kw) -> MoEProblem:
    """a Mixtral-8x7B-shaped MoE layer -- hidden 4096, ffn
    14336, 8 experts, top-2 with the weights renormalised (Mixtral's router),
    SwiGLU experts with 2-bit g128 codes, rank-64 LoRA whose U is shared by 2
    random clusters of 4 experts per projection, no shared expert."""
    args = dict(H=4096, E=8, inter=14336, top_k=2, n_clusters=2, rank=64, shared_inter=0,
                norm_topk_prob=True, balanced_clusters=True)
    args.update(kw)
    return make_moe(B=B, seed=seed, **args)


def moe_step_bytes(p: MoEProblem, active_experts: int, active_clusters: dict) -> int:
    """Algorithmic HBM bytes of one decode step: the active experts' three
    projections (codes, scales+zeros, SV), the active clusters' U, the shared
    expert, the router and shared-gate weights, hidden state in and out."""
    total = 0
    for proj in PROJS:
        q = p.experts[proj]
        per = q.N * q.K * q.bits // 8 + 4 * q.N * (q.K // q.group) + 2 * q.N * p.rank
        total += active_experts * per
        total += active_clusters[proj] * 2 * q.K * p.rank
        if p.shared is not None:
            s = p.shared[proj]
            total += s.N * s.K * s.bits // 8 + 4 * s.N * (s.K // s.group)
    total += 2 * (p.E + (1 if p.shared is not None else 0)) * p.H
    total += 2 * 2 * p.B * p.H
    return total


# ---------------------------------------------------------------------------
# TurboQuant codec (the reference's 2-bit expert format)
# ---------------------------------------------------------------------------
# Lloyd-Max quantizer of N(0, 1) at 4 levels; TurboQuant's 2-bit codebook for
# unit rows of dimension d is this scaled by 1/sqrt(d) (turbo_weight_quantizer.py
# draws it from the external turboquant package; only its shape matters here).
LLOYD_MAX_2BIT = (-1.5104, -0.4528, 0.4528, 1.5104)


@dataclass
class TurboProblem:
    """`items` TurboQuant layers of one shape plus their inputs, on the CPU."""

    packed: torch.Tensor     # (items, N, K/4) uint8: 4 indices per byte, LSB-first
    norms: torch.Tensor      # (items, N) fp32
    centroids: torch.Tensor  # (4,) fp32
    x: torch.Tensor          # (items, M, K) fp16, the unrotated input
    x_rot: torch.Tensor      # (items, M, K) fp16, the rotated input
    U: torch.Tensor | None   # (K, r) fp16 (shared by the items)
    SV: torch.Tensor | None  # (items, N, r) fp16
    bias: torch.Tensor | None  # (items, N) fp16

    @property
    def items(self) -> int:
        return self.packed.shape[0]

    @property
    def N(self) -> int:
        return self.packed.shape[1]

    @property
    def K(self) -> int:
        return self.packed.shape[2] * 4

    @property
    def M(self) -> int:
        return self.x.shape[1]

    def words(self) -> torch.Tensor:
        """The packed bytes as (items, N, K/16) int32 words (no copy of bits)."""
        return self.packed.contiguous().view(torch.int32)


def make_turbo(K: int, N: int, M: int = 1, items: int = 1, seed: int = 0, rank: int = 0,
               bias: bool = False, dist: str = "lloyd") -> TurboProblem:
    """Seeded TurboQuant problem.  Draw order (one CPU generator): packed bytes
    (items,N,K/4) uniform; norms (items,N) = |N(0,1)| + 0.1; centroids; x
    (items,M,K) = N(0,1); x_rot = N(0,1) (an orthogonal rotation of Gaussian x
    is Gaussian); then U, SV (N(0,0.01)) and bias (N(0,0.1)) when asked.
    dist='lloyd': centroids = LLOYD_MAX_2BIT / sqrt(K) (realistic scale);
    dist='randn': centroids = N(0,1), the reference's kernel test data
    (inference/kernels/test_kernels.py:48-80)."""
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (items, N, K // 4), generator=g, dtype=torch.int32)
    packed = packed.to(torch.uint8)
    norms = torch.randn(items, N, generator=g).abs() + 0.1
    if dist == "lloyd":
        cent = torch.tensor(LLOYD_MAX_2BIT, dtype=torch.float32) / K ** 0.5
    elif dist == "randn":
        cent = torch.randn(4, generator=g)
    else:
        raise ValueError(dist)
    x = torch.randn(items, M, K, generator=g).half()
    x_rot = torch.randn(items, M, K, generator=g).half()
    U = SV = b = None
    if rank:
        U = (torch.randn(K, rank, generator=g) * 0.01).half()
        SV = (torch.randn(items, N, rank, generator=g) * 0.01).half()
    if bias:
        b = (torch.randn(items, N, generator=g) * 0.1).half()
    return TurboProblem(packed=packed, norms=norms, centroids=cent, x=x, x_rot=x_rot, U=U,
                        SV=SV, bias=b)


def turbo_bytes(M: int, K: int, N: int, items: int = 1, rank: int = 0) -> int:
    """HBM bytes one turbo call must move at minimum: 2-bit indices, fp32 norm
    per row, fp16 x_rot in and y out (+ fp16 SV rows and x U when rank > 0)."""
    per = N * K // 4 + 4 * N + 2 * M * (K + N) + 2 * rank * (N + M)
    return items * per


@dataclass
class TurboMat:
    """TurboQuant weights of E matrices (N, K) sharing one rotation and
    codebook (one (dim, bits, seed) configuration, the reference's
    RotationCache key): y = norm[n] * sum_k C[q[n,k]] x_rot[k], x_rot the
    randomized Hadamard transform of x (signs) or x Pi^T (Pi)."""

    packed: torch.Tensor     # (E, N, K/4) uint8: 4 indices per byte, LSB-first
    norms: torch.Tensor      # (E, N) fp32
    centroids: torch.Tensor  # (4,) fp32
    signs: torch.Tensor | None  # (K,) fp32 +-1: RHT rotation, or None
    Pi: torch.Tensor | None     # (K, K) fp16 QR rotation when signs is None
    bits: int = 2

    @property
    def N(self) -> int:
        return self.packed.shape[1]

    @property
    def K(self) -> int:
        return self.packed.shape[2] * 4

    def words(self) -> torch.Tensor:
        """(E, N, K/16) int32 view of the packed bytes."""
        return self.packed.contiguous().view(torch.int32)


def random_orthogonal(K: int, g: torch.Generator) -> torch.Tensor:
    """Pi = Q of the QR factorisation of a Gaussian (K, K) matrix, signs fixed
    by diag(R) > 0 (how TurboQuant draws its rotation), rounded to fp16."""
    A = torch.randn(K, K, generator=g, dtype=torch.float64)
    Q, R = torch.linalg.qr(A)
    Q = Q * torch.sign(torch.diagonal(R))[None, :]
    return Q.half()


def _rand_turbo(g, E, N, K, rotation: str) -> TurboMat:
    packed = torch.randint(0, 256, (E, N, K // 4), generator=g, dtype=torch.int32).to(torch.uint8)
    norms = torch.randn(E, N, generator=g).abs() * 0.5 + 0.5
    cent = torch.tensor(LLOYD_MAX_2BIT, dtype=torch.float32) / K ** 0.5
    if rotation == "rht":
        signs = (torch.randint(0, 2, (K,), generator=g) * 2 - 1).float()
        return TurboMat(packed=packed, norms=norms, centroids=cent, signs=signs, Pi=None)
    if rotation == "qr":
        return TurboMat(packed=packed, norms=norms, centroids=cent, signs=None,
                        Pi=random_orthogonal(K, g))
    raise ValueError(rotation)


def make_turbo_moe(H=2048, E=60, inter=1408, top_k=4, n_clusters=16, rank=64,
                   shared_inter=5632, B=1, shared_bits=4, group=128, norm_topk_prob=False,
                   seed=0, rot_gate_up="rht", rot_down="qr") -> MoEProblem:
    """make_moe's block with TurboQuant routed experts (the reference's 2-bit
    expert format): same draw order, with each projection's GPTQ weights
    replaced by a TurboMat (indices uniform, norms |N(0,0.5)| + 0.5, the
    Lloyd-Max codebook / sqrt(K); gate and up share one rotation, by default an
    RHT -- H is a power of two -- and down a QR Pi, since config 2's inter 1408
    is not).  The shared expert stays GPTQ (shared_bits)."""
    g = torch.Generator().manual_seed(seed)
    router_w = (torch.randn(E, H, generator=g) * 0.02).half()
    shared_gate_w = (torch.randn(1, H, generator=g) * 0.02).half()
    dims = {"gate": (H, inter), "up": (H, inter), "down": (inter, H)}
    rots = {"gate": rot_gate_up, "up": rot_gate_up, "down": rot_down}
    experts, SV, cluster_of, U = {}, {}, {}, {}
    for proj in PROJS:
        K, N = dims[proj]
        cluster_of[proj] = torch.randint(0, n_clusters, (E,), generator=g)
        U[proj] = (torch.randn(n_clusters, K, rank, generator=g) * 0.01).half()
        experts[proj] = _rand_turbo(g, E, N, K, rots[proj])
        SV[proj] = (torch.randn(E, N, rank, generator=g) * 0.01).half()
    # gate and up share one (dim, bits, seed) configuration, as in a real model
    experts["up"].signs = experts["gate"].signs
    experts["up"].Pi = experts["gate"].Pi
    experts["up"].centroids = experts["gate"].centroids
    sdims = {"gate": (H, shared_inter), "up": (H, shared_inter), "down": (shared_inter, H)}
    shared = None if shared_inter == 0 else {
        proj: _rand_qmat(g, 1, sdims[proj][1], sdims[proj][0], shared_bits, group)
        for proj in PROJS}
    h = torch.randn(B, H, generator=g).half()
    return MoEProblem(H=H, E=E, inter=inter, top_k=top_k, norm_topk_prob=norm_topk_prob,
                      rank=rank, n_clusters=n_clusters, router_w=router_w,
                      shared_gate_w=shared_gate_w, experts=experts, SV=SV,
                      cluster_of=cluster_of, U=U, shared=shared, h=h)
