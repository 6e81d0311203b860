"""GPU parity of the fused dequant-GEMV + low-rank kernels against the CPU oracle.

Bars (north star): unpacked codes and dequantized fp16 weights bit-exact;
outputs |y - y_ref| <= 1e-3 + 1e-2 |y_ref| (fp16 out, fp32 accumulate) against
  * the reference fallback of the op the kernel replaces, restated in
    oracle.linear_forward_fp32 (gptq_dequant_matmul_fused's
    _gptq_pytorch_fallback + lora_out, inference/kernels/__init__.py:149-178,
    284-346) — the primary oracle;
  * the exact-weight fp64 sum (oracle.linear_forward_fp64(exact_weights=True));
  * for 2-bit codes also GLoRCQLinear's fp16 CPU fallback
    (oracle.linear_forward_fp16, quantized_linear.py:271-355).  For 2-bit the
    fp16 dequant is exact (|q - z| <= 3), so both fallbacks share W; for 4-bit
    the fp16 route rounds s*(q - z) (15 significant bits) to 11 and the two
    fallbacks themselves differ by more than the bar, so it is not used there.
Every call goes through the C ABI (libglorcq_hip.so) via glorcq_amd.kernels.
"""

import dataclasses

import numpy as np
import pytest
import torch

from glorcq_amd import format as fmt
from glorcq_amd import kernels as K_
from oracle import glorcq_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def to(p, dev):
    return {k: getattr(p, k).to(dev) for k in ("codes", "scales", "zeros", "U", "SV", "x")}


class Refs:
    """The oracle outputs one GPU result is held to."""

    def __init__(self, p, lora=True, xu=None, bias=None, SV=None):
        SV = p.SV if SV is None else SV
        kw = dict(U=p.U if lora else None, SV=SV if lora else None, precomputed_xU=xu,
                  bias=bias)
        self.fp32 = O.linear_forward_fp32(p.x, p.q, p.scales, p.zeros, p.group, p.sym, **kw)
        self.fp64 = O.linear_forward_fp64(p.x, p.q, p.scales, p.zeros, p.group, p.sym,
                                          exact_weights=True, **kw)
        self.fp16 = None
        if p.bits == 2:
            self.fp16 = O.linear_forward_fp16(p.x, p.q, p.scales, p.zeros, p.group, p.sym, **kw)


def oracle_y(p, lora=True, xu=None, bias=None, SV=None):
    return Refs(p, lora, xu, bias, SV)


def _check(y, ref, what):
    y = y.float().cpu().double()
    ref = ref.double().cpu()
    err = (y - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {bad.numel()} outside bar, "
                                 f"max err {err.max().item():.3e}")


def assert_parity(y, refs, what):
    _check(y, refs.fp32, f"{what} vs fp32 fallback")
    _check(y, refs.fp64, f"{what} vs exact fp64")
    if refs.fp16 is not None:
        _check(y, refs.fp16, f"{what} vs fp16 CPU fallback")


# ----------------------------------------------------------- codec (exact) --
@pytest.mark.parametrize("bits,sym", [(2, False), (4, False), (2, True), (4, True)])
def test_unpack_bit_exact(gpu, bits, sym):
    g = torch.Generator().manual_seed(bits * 10 + sym)
    words = torch.randint(-(2**31), 2**31 - 1, (257, 96), generator=g, dtype=torch.int64)
    words = words.to(torch.int32)
    K = 96 * 32 // bits
    got = K_.unpack_codes(words.to(gpu), bits, K, sym).cpu().numpy()
    assert np.array_equal(got, O.unpack_codes(words.numpy(), bits, K, sym))


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_device_matches_oracle(gpu, bits):
    g = torch.Generator().manual_seed(21)
    q = torch.randint(-(1 << (bits - 1)), 1 << bits, (64, 512), generator=g, dtype=torch.int32)
    got = K_.pack_codes_device(q.to(gpu), bits).cpu().numpy()
    assert np.array_equal(got, O.pack_codes(q.numpy(), bits))


@pytest.mark.parametrize("bits,sym,intz", [(2, False, True), (4, False, True), (2, True, True),
                                           (4, True, True), (2, False, False), (4, False, False)])
def test_dequant_bit_exact(gpu, bits, sym, intz):
    p = fmt.make_linear(1024, 160, bits=bits, group=128, seed=31 + bits, sym=sym)
    zeros = p.zeros
    if not intz:  # the reference kernel tests' non-integer zero-points
        g = torch.Generator().manual_seed(77)
        zeros = (torch.randn(p.zeros.shape, generator=g) * 0.5).half()
    W = K_.dequant_weight(p.codes.to(gpu), bits, 1024, p.scales.to(gpu),
                          None if sym else zeros.to(gpu), 128, sym).cpu()
    ref = O.dequant_fp16(p.q, p.scales, zeros, 128, sym)
    assert np.array_equal(W.numpy().view(np.uint16), ref.numpy().view(np.uint16))


# ------------------------------------------------------ fused GEMV + LoRA ---
def test_config0_exact_inputs(gpu):
    """K=2048, N=1408, 2-bit, g=128, r=64, M=1, seed 0."""
    p = fmt.make_linear(2048, 1408, bits=2, group=128, rank=64, M=1, seed=0)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"])
    torch.cuda.synchronize()
    assert y.shape == (1, 1408) and y.dtype == torch.float16
    assert_parity(y, oracle_y(p), "config0")


SHAPES = [  # (name, K, N, bits) — Qwen1.5-MoE-A2.7B projections (config 1) + more
    ("expert gate/up 2b", 2048, 1408, 2),
    ("expert down 2b", 1408, 2048, 2),
    ("attn q/k/v/o 4b", 2048, 2048, 4),
    ("shared gate/up 4b", 2048, 5632, 4),
    ("shared down 4b", 5632, 2048, 4),
]


@pytest.mark.parametrize("name,K,N,bits", SHAPES)
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_shapes_batch_sweep(gpu, name, K, N, bits, M):
    p = fmt.make_linear(K, N, bits=bits, group=128, rank=64, M=M, seed=K + N + M)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"{name} M={M}")


@pytest.mark.parametrize("bits", [2, 4])
def test_no_lora_and_bias(gpu, bits):
    p = fmt.make_linear(1024, 320, bits=bits, rank=64, M=3, seed=5)
    d = to(p, gpu)
    bias = (torch.randn(320, generator=torch.Generator().manual_seed(1)) * 0.1).half()
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       bias=bias.to(gpu))
    assert_parity(y, oracle_y(p, lora=False, bias=bias), "no-lora+bias")
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"], bias=bias.to(gpu))
    assert_parity(y, oracle_y(p, bias=bias), "lora+bias")


def test_precomputed_xu(gpu):
    """Cluster-shared x*U hook (quantized_linear.py:286-345)."""
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=4, seed=8)
    d = to(p, gpu)
    xu = (p.x @ p.U)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       SV=d["SV"], precomputed_xU=xu.to(gpu))
    assert_parity(y, oracle_y(p, xu=xu), "precomputed xU")


@pytest.mark.parametrize("bits", [2, 4])
def test_sym(gpu, bits):
    p = fmt.make_linear(2048, 512, bits=bits, rank=64, M=1, seed=12, sym=True)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], None, bits, 128,
                                       sym=True, U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), "sym")


def test_noninteger_zeros(gpu):
    p = fmt.make_linear(2048, 256, bits=2, rank=64, M=2, seed=13)
    p.zeros = (torch.randn(p.zeros.shape, generator=torch.Generator().manual_seed(3)) * 0.5).half()
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), "non-integer zeros")


@pytest.mark.parametrize("K,N,M,group,rank", [
    (128, 16, 1, 128, 8),      # smallest legal problem
    (256, 1000, 5, 256, 40),   # ragged N, group 256, rank not a multiple of 32
    (14336, 4096, 1, 128, 64),  # Mixtral down_proj K (the reference's smem overflow case)
    (14336, 512, 2, 128, 64),
    (4096, 14336, 1, 128, 128),
    (2048, 64, 16, 128, 512),  # max rank
])
def test_edge_shapes(gpu, K, N, M, group, rank):
    p = fmt.make_linear(K, N, bits=2, group=group, rank=rank, M=M, seed=K + N)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, group,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"K={K} N={N} M={M}")


def test_empty_batch(gpu):
    """B=0 returns shape (0, N) (test_kernels_qwen.py:151-154)."""
    p = fmt.make_linear(2048, 1408, bits=2, M=1, seed=0)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"][:0], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"])
    assert y.shape == (0, 1408)
    torch.zeros(1, device=gpu)
    torch.cuda.synchronize()


def test_m_above_16_blocks(gpu):
    p = fmt.make_linear(1024, 256, bits=4, rank=64, M=40, seed=14)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 4, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), "M=40")


def test_repeat_calls_reuse_workspace(gpu):
    """Counters self-reset: consecutive launches on one stream agree exactly."""
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=0)
    d = to(p, gpu)
    ys = [K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                         U=d["U"], SV=d["SV"]) for _ in range(5)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


@pytest.mark.parametrize("bits", [2, 4])
def test_batched_items(gpu, bits):
    E, M, K, N, r = 6, 2, 2048, 1408, 64
    ps = [fmt.make_linear(K, N, bits=bits, rank=r, M=M, seed=100 + e) for e in range(E)]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    y = K_.packed_dequant_matmul_batched(st("x"), st("codes"), st("scales"), st("zeros"), bits,
                                         128, U=st("U"), SV=st("SV"))
    for e, p in enumerate(ps):
        assert_parity(y[e], oracle_y(p), f"item {e}")


def test_reference_signature_unpacked_codes(gpu):
    """gptq_dequant_matmul_fused with the reference's (N, K) int32 codes and an
    (U, S, V) low-rank tuple."""
    p = fmt.make_linear(2048, 512, bits=2, rank=64, M=1, seed=15)
    g = torch.Generator().manual_seed(2)
    S = torch.rand(64, generator=g).half()
    V = p.SV  # (N, r)
    y = K_.gptq_dequant_matmul_fused(p.x.to(gpu), p.q.to(gpu), p.scales.to(gpu),
                                     p.zeros.to(gpu), 128, False,
                                     lora_USV=(p.U.to(gpu), S.to(gpu), V.to(gpu)))
    SV = (V.float() * S.float()[None]).half()
    assert_parity(y, oracle_y(p, SV=SV), "reference signature")


def test_graph_capture_replays(gpu):
    """The fused call captured in a HIP graph: every replay, with eager work
    between replays, matches the eager result."""
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=0)
    d = to(p, gpu)
    out = torch.empty(1, 1408, dtype=torch.float16, device=gpu)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"], out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"], out=out)
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        _ = (d["x"].float() * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("K,N,M,bits", [(2048, 1408, 1, 2), (1408, 2048, 4, 2), (2048, 2048, 16, 4),
                                        (2048, 512, 12, 2)])
def test_ksplit_fallback_path(gpu, monkeypatch, K, N, M, bits):
    """The K-split kernel (used when the streaming kernel's conditions fail:
    group != 128, odd N, rank > 128, or x too large for LDS) forced on shapes
    the streaming kernel would otherwise take."""
    monkeypatch.setenv("GLQ_GEMV_NO_STREAM", "1")
    p = fmt.make_linear(K, N, bits=bits, rank=64, M=M, seed=K + M)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"k-split K={K} N={N} M={M}")


@pytest.mark.parametrize("bits,K,N,rank,sym,ipw", [
    (2, 2048, 1408, 64, False, None),   # config 0 shape: 32 lanes per row, 2 rows per step
    (2, 1408, 1462, 40, False, 12),    # 22 of 32 lanes live, ragged N, rank 40; waves of 12
                                       # iterations start and end inside 32-iteration units
    (4, 2048, 2048, 64, True, 96),     # 64 lanes per row, symmetric codes, 1.5 units a wave
    (4, 1408, 200, 128, False, None),  # 44 of 64 lanes live, rank 128 (an SV dword a lane)
    (2, 2048, 320, 128, False, 20),    # rank 128 over 32-lane groups: 2 SV dwords per lane
    (2, 512, 130, 16, True, 48),       # 4 rows per step (16-lane groups), run past N
    (2, 4096, 448, 0, False, 8),       # 64 lanes per row at 2 bits, no low-rank term
    (2, 1024, 640, 128, False, None),  # 16-lane groups with 4 SV dwords per lane
    (2, 2048, 512, 8, False, None),    # rank 8: one U column block, x U split over codes
    (4, 1024, 300, 48, False, 8),      # rank 48 (6 column blocks), waves past the last round
])
def test_lane_path_m1(gpu, monkeypatch, bits, K, N, rank, sym, ipw):
    """The one-token-row kernel (glq_lane.h) on the shapes it takes: live and
    idle lanes, 1/2/4 rows per step, 1/2/4 SV dwords per lane, bias,
    symmetric codes, waves covering parts of units and several units
    (GLQ_LANE_RPW), no LoRA; against the oracle and against the streaming
    kernel forced on the same inputs."""
    if ipw:
        monkeypatch.setenv("GLQ_LANE_RPW", str(ipw // 4))
    p = fmt.make_linear(K, N, bits=bits, rank=max(rank, 8), M=1, seed=K + N + bits, sym=sym)
    d = to(p, gpu)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(N)) * 0.1).half()
    kw = dict(U=d["U"], SV=d["SV"]) if rank else {}
    zeros = None if sym else d["zeros"]
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], zeros, bits, 128,
                                       sym=sym, bias=bias.to(gpu), **kw)
    assert_parity(y, oracle_y(p, lora=rank > 0, bias=bias), f"lane K={K} N={N}")
    if rank:  # a = x U formed in the launch vs by the separate partial-sum launch
        monkeypatch.setenv("GLQ_LANE_NO_XU", "1")
        y1 = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], zeros, bits, 128,
                                            sym=sym, bias=bias.to(gpu), **kw)
        monkeypatch.delenv("GLQ_LANE_NO_XU")
        assert_parity(y1, oracle_y(p, bias=bias), "lane, separate x U launch")
        # the two differ only in the fp32 summation order of a = x U
        assert bool(((y.float() - y1.float()).abs() <= 1e-4 + 2e-3 * y1.float().abs()).all())
    xu = (p.x.double() @ p.U.double()).half()
    if rank:  # the precomputed a = x U hook
        y2 = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], zeros, bits, 128,
                                            sym=sym, SV=d["SV"], precomputed_xU=xu.to(gpu),
                                            bias=bias.to(gpu))
        assert_parity(y2, oracle_y(p, xu=xu, bias=bias), "lane precomputed xU")
    monkeypatch.setenv("GLQ_GEMV_NO_LANE", "1")
    ys = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], zeros, bits, 128,
                                        sym=sym, bias=bias.to(gpu), **kw)
    assert_parity(ys, oracle_y(p, lora=rank > 0, bias=bias), "stream kernel, same inputs")


def test_lane_path_batched_items(gpu, monkeypatch):
    """Many items of one token row in one launch, waves of 44 iterations (a
    unit and 3/8 of the next)."""
    monkeypatch.setenv("GLQ_LANE_RPW", "11")
    E, K, N, r = 9, 2048, 1408, 64
    ps = [fmt.make_linear(K, N, bits=2, rank=r, M=1, seed=300 + e) for e in range(E)]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    y = K_.packed_dequant_matmul_batched(st("x"), st("codes"), st("scales"), st("zeros"), 2,
                                         128, U=st("U"), SV=st("SV"))
    for e, p in enumerate(ps):
        assert_parity(y[e], oracle_y(p), f"item {e}")


@pytest.mark.parametrize("bits,K,N,rank,items", [
    (2, 2048, 1408, 64, 1),   # config 0: 8 K slices
    (2, 1408, 1462, 40, 1),   # a last slice of 128 rows, rank 40
    (4, 4096, 448, 128, 1),   # 16 slices, rank 128
    (2, 512, 130, 8, 1),      # 2 slices, rank 8
    (2, 2048, 1408, 64, 9),   # 9 items: 72 jobs, one counter an item
])
def test_lane_xu_jobs(gpu, monkeypatch, bits, K, N, rank, items):
    """a = x U of the one-token-row launch formed by job workgroups in front
    of the grid (one 256-row K slice each, handed over) and summed in slice
    order by every row workgroup: against the oracle; against the launch
    whose row workgroups each form a over the whole row (GLQ_LANE_XJ=0,
    another fp32 order); bit-equal to row workgroups whose wait is bounded
    at zero ticks (GLQ_LANE_SPIN_TICKS=0: the slices formed locally in the
    same order) and to calls after those (the counters left zero)."""
    ps = [fmt.make_linear(K, N, bits=bits, rank=rank, M=1, seed=K + N + rank + e)
          for e in range(items)]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    args = (st("x"), st("codes"), st("scales"), st("zeros"), bits, 128)

    def call():
        y = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"))
        torch.cuda.synchronize()
        return y

    for v in ("GLQ_LANE_XJ", "GLQ_LANE_SPIN_TICKS", "GLQ_LANE_NO_XU"):
        monkeypatch.delenv(v, raising=False)
    y = call()
    for e, p in enumerate(ps):
        assert_parity(y[e], oracle_y(p), f"x U jobs item {e}")
    monkeypatch.setenv("GLQ_LANE_SPIN_TICKS", "0")
    y0 = call()
    monkeypatch.delenv("GLQ_LANE_SPIN_TICKS")
    assert torch.equal(y, y0), "zero-tick wait"
    monkeypatch.setenv("GLQ_LANE_XJ", "0")
    yw = call()
    monkeypatch.delenv("GLQ_LANE_XJ")
    assert torch.equal(y, call()), "x U jobs after the local runs"
    # the two differ only in the fp32 summation order of a = x U
    assert bool(((y.float() - yw.float()).abs() <= 1e-4 + 2e-3 * yw.float().abs()).all())


def test_lane_xu_jobs_graph_replays(gpu):
    """The one-token-row call with x U jobs captured in a HIP graph on a side
    stream (its own zero-filled workspace): replays with eager calls on the
    capture stream between them all match the eager result."""
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=5)
    d = to(p, gpu)
    out = torch.empty(1, 1408, dtype=torch.float16, device=gpu)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def call(o):
        K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"], out=o)

    with torch.cuda.stream(s):
        call(out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _ in range(3):
            call(out)
    for i in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        with torch.cuda.stream(s):
            other = torch.empty_like(out)
            call(other)
        s.synchronize()
        assert torch.equal(other, eager), f"eager call after replay {i}"


@pytest.mark.parametrize("bits,K,N,rank,sym", [
    (4, 4096, 2048, 64, False),   # config-4 o projection: 128 pieces, two a lane
    (2, 8192, 512, 128, True),    # 2-bit rows of 128 pieces, rank 128, symmetric codes
    (4, 2560, 320, 64, False),    # 80 pieces: the second piece live on 16 of 64 lanes
])
def test_lane_two_pieces_a_lane(gpu, monkeypatch, bits, K, N, rank, sym):
    """Code rows of 65..128 16-byte pieces on the one-token-row kernel, two
    pieces a lane (NP = 2), with a = x U formed in the launch; against the
    oracle and the streaming kernel forced on the same inputs."""
    p = fmt.make_linear(K, N, bits=bits, rank=rank, M=1, seed=K + 7 * N + bits, sym=sym)
    d = to(p, gpu)
    zeros = None if sym else d["zeros"]
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], zeros, bits, 128,
                                       sym=sym, U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"two pieces a lane K={K} N={N}")
    monkeypatch.setenv("GLQ_GEMV_NO_LANE", "1")
    ys = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], zeros, bits, 128,
                                        sym=sym, U=d["U"], SV=d["SV"])
    assert_parity(ys, oracle_y(p), "stream kernel, same inputs")


@pytest.mark.parametrize("M", [1, 4])
def test_clustered_u_index(gpu, M):
    """q, k and v of one layer as ten items sharing x (glq_gemv_lora_clustered):
    items 0..7 name U 0, items 8 and 9 name U 1 and 2.  The same bits as the
    batched call with each item's U copied out, and parity per item."""
    K, N, r, bits = 2048, 512, 64, 4
    ps = [fmt.make_linear(K, N, bits=bits, rank=r, M=M, seed=900 + i) for i in range(10)]
    x = ps[0].x
    Us = torch.stack([ps[0].U, ps[8].U, ps[9].U])
    uidx = [0] * 8 + [1, 2]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    args = (x.to(gpu), st("codes"), st("scales"), st("zeros"), bits, 128)
    y = K_.packed_dequant_matmul_batched(*args, U=Us.to(gpu), SV=st("SV"),
                                         u_index=torch.tensor(uidx, dtype=torch.int32,
                                                              device=gpu))
    ycopy = K_.packed_dequant_matmul_batched(*args, U=Us[uidx].contiguous().to(gpu),
                                             SV=st("SV"))
    torch.cuda.synchronize()
    assert torch.equal(y, ycopy)
    for i, p in enumerate(ps):
        q = dataclasses.replace(p, x=x, U=Us[uidx[i]])
        assert_parity(y[i], oracle_y(q), f"item {i}")
    # a given per U (C, M, r), item i reading row block u_index[i]: the same
    # bits as the batched call with each item's a copied out
    a = K_.lowrank_xu(x.to(gpu), Us.to(gpu))  # (3, M, r)
    ya = K_.packed_dequant_matmul_batched(*args, SV=st("SV"), precomputed_xU=a,
                                          u_index=torch.tensor(uidx, dtype=torch.int32,
                                                               device=gpu))
    yacopy = K_.packed_dequant_matmul_batched(*args, SV=st("SV"),
                                              precomputed_xU=a[uidx].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(ya, yacopy)
    for i, p in enumerate(ps):
        q = dataclasses.replace(p, x=x, U=Us[uidx[i]])
        assert_parity(ya[i], oracle_y(q), f"item {i}, a per U")


@pytest.mark.parametrize("M,bits,nb,uidx", [(1, 4, 3, [0] * 8 + [1, 2]), (3, 4, 2, [1, 0, 1]),
                                             (5, 4, 1, [0, 0]), (16, 4, 2, None),
                                             (1, 2, 2, None), (2, 2, 4, [3, 1])])
def test_parts_entry_point(gpu, M, bits, nb, uidx):
    """glq_gemv_lora_parts: a given as fp32 partials (blocks, P, M, rpad),
    item i summing block u_index[i] in order -- the same bits as the batched
    GEMV given a = fp16 of that sum (sequential fp32 adds, the kernels'
    order) for each item, and parity with the oracle.  M = 1 takes the lane
    kernel, 3 the streaming kernel, 5 and 16 the token-tile form."""
    K, N, r, P = 2048, 512, 64, 8
    E = len(uidx) if uidx is not None else nb
    ps = [fmt.make_linear(K, N, bits=bits, rank=r, M=M, seed=700 + i) for i in range(E)]
    x = ps[0].x.to(gpu)
    gen = torch.Generator().manual_seed(M + 10 * bits)
    parts = (torch.randn(nb, P, M, r, generator=gen) * 0.3).float().to(gpu)
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    ui = torch.tensor(uidx, dtype=torch.int32, device=gpu) if uidx is not None else None
    y = K_.packed_dequant_matmul_parts(x, st("codes"), st("scales"), st("zeros"), bits, 128,
                                       st("SV"), parts, u_index=ui)
    acc = torch.zeros(nb, M, r, dtype=torch.float32, device=gpu)
    for p in range(P):  # the kernels' order
        acc = acc + parts[:, p]
    a = acc.half()
    blocks = uidx if uidx is not None else list(range(nb))
    ya = K_.packed_dequant_matmul_batched(x, st("codes"), st("scales"), st("zeros"), bits, 128,
                                          SV=st("SV"), precomputed_xU=a[blocks].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(y, ya)
    for i, p in enumerate(ps):
        assert_parity(y[i], oracle_y(dataclasses.replace(p, x=ps[0].x), xu=a[blocks[i]].cpu()),
                      f"item {i}")


@pytest.mark.parametrize("bits", [2, 4])
def test_stream_bias_odd_tiles_sym(gpu, bits):
    """Streaming kernel with bias, a partial last 16-row tile (N = 16k + 6),
    a K tail that ends half-way into a 2-bit step (K = 1408) and symmetric codes."""
    for sym in (False, True):
        p = fmt.make_linear(1408, 1462, bits=bits, rank=40, M=3, seed=77 + sym, sym=sym)
        d = to(p, gpu)
        bias = (torch.randn(1462, generator=torch.Generator().manual_seed(9)) * 0.1).half()
        y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"],
                                           None if sym else d["zeros"], bits, 128, sym=sym,
                                           U=d["U"], SV=d["SV"], bias=bias.to(gpu))
        assert_parity(y, oracle_y(p, bias=bias), f"stream bias sym={sym}")


@pytest.mark.parametrize("E,M,K,r,shared_x", [(1, 1, 2048, 64, False), (5, 3, 1408, 64, False),
                                              (16, 4, 2048, 64, True), (3, 16, 5632, 128, False),
                                              (2, 2, 256, 8, True), (7, 1, 1408, 8, False),
                                              (3, 1, 1408, 16, True), (2, 1, 384, 128, False),
                                              (3, 1, 2048, 40, False)])
def test_lowrank_xu(gpu, E, M, K, r, shared_x):
    """a = fp16(x U) with fp32 accumulation (reference `x @ U`,
    inference/quantized_linear.py:344; cluster-shared form with one x,
    inference/moe_block.py:290-322) against the fp64 product."""
    g = torch.Generator().manual_seed(E * 100 + K)
    U = (torch.randn(E, K, r, generator=g) * 0.01).half()
    x = torch.randn(M, K, generator=g).half() if shared_x else torch.randn(E, M, K, generator=g).half()
    a = K_.lowrank_xu(x.to(gpu), U.to(gpu)).cpu()
    xd = x.double() if not shared_x else x.double().unsqueeze(0).expand(E, M, K)
    ref = xd @ U.double()
    # one fp16 rounding of an fp32 sum: |err| <= 2^-11 |a| + tiny
    assert a.shape == (E, M, r)
    err = (a.double() - ref).abs()
    assert bool((err <= 1e-3 * ref.abs() + 1e-4).all()), float(err.max())


@pytest.mark.parametrize("bits", [2, 4])
def test_batched_precomputed_xu(gpu, bits):
    """Batched GEMV fed a = lowrank_xu(x, U) equals the oracle with that a."""
    E, M, K, N, r = 4, 2, 2048, 1408, 64
    ps = [fmt.make_linear(K, N, bits=bits, rank=r, M=M, seed=300 + e) for e in range(E)]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    xu = K_.lowrank_xu(st("x"), st("U"))
    y = K_.packed_dequant_matmul_batched(st("x"), st("codes"), st("scales"), st("zeros"), bits,
                                         128, SV=st("SV"), precomputed_xU=xu)
    for e, p in enumerate(ps):
        assert_parity(y[e], oracle_y(p, xu=xu[e].cpu()), f"item {e}")


@pytest.mark.parametrize("ks", ["0", "1"])
@pytest.mark.parametrize("K,N,bits,M,items,bias", [
    (4096, 2048, 4, 1, 1, False),    # the Qwen3 o projection at one token
    (4096, 2048, 4, 16, 1, True),
    (2048, 1408, 2, 8, 1, False),
    (2048, 1462, 2, 12, 3, True),    # ragged N, several items
    (5632, 2048, 4, 4, 1, False),
])
def test_stream_forms(gpu, monkeypatch, ks, K, N, bits, M, items, bias):
    """The streaming GEMV in both forms (GLQ_STREAM_KS: one wave per tile, or
    the K-split form with a tile's chunks dealt over the four waves and the
    partial tiles summed in a fixed order) against the oracle; the lane path
    is switched off so M = 1 streams too."""
    monkeypatch.setenv("GLQ_STREAM_KS", ks)
    monkeypatch.setenv("GLQ_GEMV_NO_LANE", "1")
    ps = [fmt.make_linear(K, N, bits=bits, rank=64, M=M, seed=7 * K + N + M + e)
          for e in range(items)]
    g = torch.Generator().manual_seed(N)
    bs = [(torch.randn(N, generator=g) * 0.1).half() if bias else None for _ in range(items)]
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    B = torch.stack(bs).to(gpu) if bias else None
    y = K_.packed_dequant_matmul_batched(st("x"), st("codes"), st("scales"), st("zeros"), bits,
                                         128, U=st("U"), SV=st("SV"), bias=B)
    again = K_.packed_dequant_matmul_batched(st("x"), st("codes"), st("scales"), st("zeros"),
                                             bits, 128, U=st("U"), SV=st("SV"), bias=B)
    torch.cuda.synchronize()
    assert torch.equal(y, again)
    for e, p in enumerate(ps):
        assert_parity(y[e], oracle_y(p, bias=bs[e]), f"ks={ks} item {e}")


@pytest.mark.parametrize("K,N,M,items", [(2048, 4096, 16, 1), (2048, 512, 8, 3), (4096, 2048, 16, 1),
                                         (1024, 1408, 4, 2), (2048, 1400, 5, 1), (768, 2048, 6, 1)])
def test_token_tile_path(gpu, monkeypatch, K, N, M, items):
    """4-bit asymmetric codes at 4..16 token rows take the token-tile MFMA form
    (glq_tile16.h via gemv_t16_kernel: each code decoded once for every row;
    1, 2 or 4 groups a wave for K up to 1024, 2048, 4096; N = 1400 leaves a
    ragged row block, K = 768 idle waves): against the oracle, with LoRA from
    U (x U formed in the same launch) and bias, with a precomputed xU, and
    against the streaming kernel forced on the same inputs (GLQ_GEMV_NO_T16)."""
    ps = [fmt.make_linear(K, N, bits=4, group=128, rank=64, M=M, seed=K + N + M + e)
          for e in range(items)]
    bias = (torch.randn(items, N, generator=torch.Generator().manual_seed(3)) * 0.1).half()
    st = lambda k: torch.stack([getattr(p, k) for p in ps]).to(gpu)  # noqa: E731
    args = (st("x"), st("codes"), st("scales"), st("zeros"), 4, 128)
    monkeypatch.delenv("GLQ_GEMV_NO_T16", raising=False)
    y = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"), bias=bias.to(gpu))
    y2 = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"), bias=bias.to(gpu))
    assert torch.equal(y, y2)
    for e, p in enumerate(ps):
        assert_parity(y[e], oracle_y(p, bias=bias[e]), f"tile form item {e}")
    xu = torch.stack([p.x @ p.U for p in ps])
    yx = K_.packed_dequant_matmul_batched(*args, SV=st("SV"), precomputed_xU=xu.half().to(gpu))
    for e, p in enumerate(ps):
        assert_parity(yx[e], oracle_y(p, xu=xu[e].half().float()), f"tile form xU item {e}")
    # x U formed in the tile form's own launch (its first workgroups, handed
    # over) against the separate partial-sum launch (GLQ_T16_XU2) and against
    # row blocks whose wait is bounded at zero ticks (GLQ_T16_SPIN_TICKS=0:
    # a formed in the waiting workgroup): the same sums in the same order
    monkeypatch.setenv("GLQ_T16_XU2", "1")
    y3 = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"), bias=bias.to(gpu))
    monkeypatch.delenv("GLQ_T16_XU2")
    monkeypatch.setenv("GLQ_T16_SPIN_TICKS", "0")
    y4 = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"), bias=bias.to(gpu))
    monkeypatch.delenv("GLQ_T16_SPIN_TICKS")
    y5 = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"), bias=bias.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(y, y3), "in-launch x U vs the separate launch"
    assert torch.equal(y, y4), "zero-tick wait"
    assert torch.equal(y, y5), "in-launch x U after the local runs"
    monkeypatch.setenv("GLQ_GEMV_NO_T16", "1")
    ys = K_.packed_dequant_matmul_batched(*args, U=st("U"), SV=st("SV"), bias=bias.to(gpu))
    _check(y, ys.float(), "tile form vs streaming kernel")
