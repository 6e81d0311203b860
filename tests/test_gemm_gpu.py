"""GPU parity of the prefill MFMA GEMM (glq_gemm_lora, M > 16) against the CPU
oracle, at the bars of test_gemv_gpu (fp32 reference fallback, exact fp64 sum,
and for 2-bit the fp16 CPU fallback): |y - y_ref| <= 1e-3 + 1e-2 |y_ref|.
The reference's M > 4 path is gptq_dequant_gemm_kernel
(inference/kernels/gptq_matmul.cu:111-213); its fallback is the same
_gptq_pytorch_fallback as the GEMV's."""

import ctypes

import pytest
import torch

from glorcq_amd import _lib
from glorcq_amd import format as fmt
from glorcq_amd import kernels as K_
from test_gemv_gpu import assert_parity, oracle_y, to


def test_gemm_workspace_sizes():
    lib = _lib.load()
    n0 = lib.glq_gemm_workspace_bytes(512, 2048, 1408, 0)  # split-K tiles, if any
    n = lib.glq_gemm_workspace_bytes(512, 2048, 1408, 64)  # + a = x U
    assert n0 >= 0 and n0 % 256 == 0
    assert n >= n0 + 512 * 64 * 2 and n % 256 == 0
    assert lib.glq_gemm_workspace_bytes(0, 2048, 1408, 64) == 0
    # argument errors come back before any launch
    rc = lib.glq_gemm_lora(None, 64, 2048, 64, None, 2, None, None, 64, 0, None, None, 0, None,
                           None, None, None, 0, None)
    assert rc == 1 and b"group" in lib.glq_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("name,K,N,bits,M", [
    ("expert gate/up 2b", 2048, 1408, 2, 128),
    ("expert gate/up 2b", 2048, 1408, 2, 512),
    ("expert down 2b", 1408, 2048, 2, 128),
    ("attn q/k/v/o 4b", 2048, 2048, 4, 128),
    ("attn q/k/v/o 4b", 2048, 2048, 4, 512),
])
def test_config1_prefill(gpu, name, K, N, bits, M):
    """BASELINE config 1's GEMM batch sizes."""
    p = fmt.make_linear(K, N, bits=bits, group=128, rank=64, M=M, seed=K + N + M + bits)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"{name} M={M}")


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,bits,rank", [
    (384, 200, 17, 2, 16),     # odd group count, N and M tails
    (1408, 70, 65, 4, 40),     # rank not a multiple of 32
    (256, 64, 130, 2, 64),     # one chunk
    (1024, 130, 300, 4, 8),
])
def test_edge_shapes(gpu, K, N, M, bits, rank):
    p = fmt.make_linear(K, N, bits=bits, group=128, rank=rank, M=M, seed=K * 7 + M)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"K={K} N={N} M={M} b={bits} r={rank}")


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 4])
def test_sym_bias_nolora(gpu, bits):
    g = torch.Generator().manual_seed(3)
    for sym in (True, False):
        p = fmt.make_linear(1024, 192, bits=bits, rank=32, M=48, seed=30 + bits + sym, sym=sym)
        d = to(p, gpu)
        bias = (torch.randn(192, generator=g) * 0.1).half()
        y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"],
                                           None if sym else d["zeros"], bits, 128, sym=sym,
                                           bias=bias.to(gpu))
        assert_parity(y, oracle_y(p, lora=False, bias=bias), f"sym={sym} b={bits} no-lora+bias")


@pytest.mark.gpu
def test_precomputed_xu(gpu):
    p = fmt.make_linear(2048, 256, bits=2, rank=64, M=96, seed=41)
    d = to(p, gpu)
    xu = (p.x.float() @ p.U.float()).half()
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       SV=d["SV"], precomputed_xU=xu.to(gpu))
    assert_parity(y, oracle_y(p, xu=xu), "precomputed xU")


@pytest.mark.gpu
def test_precomputed_xu_exact_workspace(gpu):
    """With a = x U given the workspace is the rank-0 size, exactly: the call
    takes a buffer of glq_gemm_workspace_bytes(M, K, N, 0) bytes and no more."""
    lib = _lib.load()
    M, K, N = 512, 2048, 1408
    p = fmt.make_linear(K, N, bits=2, rank=64, M=M, seed=44)
    d = to(p, gpu)
    xu = (p.x.float() @ p.U.float()).half()
    xg = xu.to(gpu)
    need = lib.glq_gemm_workspace_bytes(M, K, N, 0)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=gpu)  # (a buffer even at 0)
    y = torch.empty(M, N, dtype=torch.float16, device=gpu)
    rc = lib.glq_gemm_lora(d["x"].data_ptr(), M, K, N, d["codes"].data_ptr(), 2,
                           d["scales"].data_ptr(), d["zeros"].data_ptr(), 128, 0, None,
                           d["SV"].data_ptr(), 64, xg.data_ptr(), None, y.data_ptr(),
                           ws.data_ptr(), need, _lib.stream_handle(gpu))
    _lib.check(rc, "glq_gemm_lora")
    torch.cuda.synchronize()
    assert_parity(y, oracle_y(p, xu=xu), "precomputed xU, exact workspace")


@pytest.mark.gpu
def test_gemm_matches_gemv_blocks(gpu):
    """The GEMM and the 16-row GEMV blocks compute the same function: both
    within the bar of the oracle, and close to each other."""
    p = fmt.make_linear(2048, 512, bits=2, rank=64, M=64, seed=43)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"])
    blocks = torch.cat([K_.packed_dequant_matmul_fused(d["x"][i:i + 16], d["codes"], d["scales"],
                                                       d["zeros"], 2, 128, U=d["U"], SV=d["SV"])
                        for i in range(0, 64, 16)])
    torch.cuda.synchronize()
    diff = (y.float() - blocks.float()).abs()
    assert float(diff.max()) <= 2e-3 + 1e-2 * float(blocks.float().abs().max())
    assert_parity(y, oracle_y(p), "GEMM M=64")


@pytest.mark.gpu
@pytest.mark.parametrize("ks", [1, 3, 8])
@pytest.mark.parametrize("K,N,M,bits,rank", [
    (2048, 1408, 128, 2, 64),   # config 1 gate/up
    (1408, 330, 70, 4, 128),    # 6 chunks, rank 128 (two rank tiles per wave in the x U jobs)
    (1024, 200, 40, 2, 192),    # rank above the in-launch x U limit: low-rank launches
])
def test_split_k_variants(gpu, monkeypatch, ks, K, N, M, bits, rank):
    """K splits forced (GLQ_PF_KS; capped at the group count): each tile's
    last-arriving split sums the partial tiles in split order and runs the
    epilogue; rank 192 takes the low-rank entry point first."""
    monkeypatch.setenv("GLQ_PF_KS", str(ks))
    p = fmt.make_linear(K, N, bits=bits, group=128, rank=rank, M=M, seed=K + N + ks)
    d = to(p, gpu)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(ks)) * 0.1).half()
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"], bias=bias.to(gpu))
    assert_parity(y, oracle_y(p, bias=bias), f"ks={ks} K={K} N={N} M={M}")
    y2 = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                        U=d["U"], SV=d["SV"], bias=bias.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(y, y2)  # fixed summation order: the same bits every call


def test_gemm_requires_workspace():
    """The prefill path takes a workspace (split-K tiles, a = x U): a missing
    or short one is an argument error, raised before any launch."""
    lib = _lib.load()
    fake = 1 << 20  # never dereferenced: the checks run first
    args = [fake, 80, 2048, 320, fake, 2, fake, fake, 128, 0, None, fake, 64, fake, None, fake]
    assert lib.glq_gemm_lora(*args, None, 0, None) == 1
    assert b"workspace" in lib.glq_last_error()
    need = lib.glq_gemm_workspace_bytes(80, 2048, 320, 0)
    assert lib.glq_gemm_lora(*args, fake, need - 256, None) == 1
    assert b"workspace" in lib.glq_last_error()


@pytest.mark.gpu
def test_config1_down_m512(gpu):
    """The config-1 down projection (1408 -> 2048) at the prefill size M=512."""
    p = fmt.make_linear(1408, 2048, bits=2, group=128, rank=64, M=512, seed=1408 + 512)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], 2, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), "expert down 2b M=512")


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 4])
def test_large_prefill_tiles(gpu, bits):
    """M = 1024 over K = 4096 (128-token tiles for 2-bit, one K split)."""
    p = fmt.make_linear(4096, 1024, bits=bits, group=128, rank=64, M=1024, seed=77 + bits)
    d = to(p, gpu)
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"])
    assert_parity(y, oracle_y(p), f"M=1024 K=4096 b={bits}")


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", ["16,1,1", "16,2,1", "32,1,1", "32,2,1", "64,2,1", "64,2,0",
                                 "128,2,0", "32,4,0"])
@pytest.mark.parametrize("bits", [2, 4])
def test_tile_configs(gpu, monkeypatch, cfg, bits):
    """Every token tile x weight-row tile x ring depth the dense launch can take
    (GLQ_PF_CFG "tm,rt,deep"), on ragged M and N, rank 40, a bias, and
    zero-points half integral and half not (the in-kernel sum of x that
    non-integer zero-points need): the same bar against the oracle."""
    monkeypatch.setenv("GLQ_PF_CFG", cfg)
    p = fmt.make_linear(1408, 330, bits=bits, group=128, rank=40, M=70, seed=bits * 31)
    z = p.zeros.float()
    frac = torch.rand(z.shape, generator=torch.Generator().manual_seed(bits)) * 0.5
    rows = torch.arange(z.shape[0]).unsqueeze(1) % 2 == 1  # odd rows: non-integer
    p.zeros = torch.where(rows, z + frac, z).half()
    d = to(p, gpu)
    bias = (torch.randn(330, generator=torch.Generator().manual_seed(5)) * 0.1).half()
    y = K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits, 128,
                                       U=d["U"], SV=d["SV"], bias=bias.to(gpu))
    assert_parity(y, oracle_y(p, bias=bias), f"cfg {cfg} bits {bits}")
    # symmetric codes on the same tile
    ps = fmt.make_linear(1024, 200, bits=bits, group=128, rank=16, M=40, seed=bits + 7, sym=True)
    ds = to(ps, gpu)
    ys = K_.packed_dequant_matmul_fused(ds["x"], ds["codes"], ds["scales"], None, bits, 128,
                                        sym=True, U=ds["U"], SV=ds["SV"])
    assert_parity(ys, oracle_y(ps), f"cfg {cfg} bits {bits} sym")


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,bits", [(128, 2048, 1408, 2), (77, 2048, 512, 4),
                                        (512, 1408, 2048, 2), (4100, 1024, 256, 4)])
def test_one_launch_xu(gpu, monkeypatch, M, K, N, bits):
    """a = x U of the prefill formed in the GEMM's own launch (16-row blocks
    over K slices in the first grid rows, the block's last arriving slice sums
    them; the GEMM's epilogue waits for its rows' blocks): parity, the same
    bits on repeated calls and graph replays (the arrival counters are left at
    zero), with every epilogue wait bounded at zero ticks (GLQ_PF_SPIN_TICKS=0:
    a block not yet ready is formed in the waiting workgroup, in the same
    order) and from the separate one-launch x U (GLQ_PF_XU1); the two-launch
    form (GLQ_PF_XU2) within the parity bar."""
    p = fmt.make_linear(K, N, bits=bits, rank=64, M=M, seed=M + K)
    d = to(p, gpu)
    print(f"one-launch x U M={M} K={K} N={N} bits={bits}", flush=True)

    def call(out=None):
        return K_.packed_dequant_matmul_fused(d["x"], d["codes"], d["scales"], d["zeros"], bits,
                                              128, U=d["U"], SV=d["SV"], out=out)

    y = call()
    torch.cuda.synchronize()
    assert_parity(y, oracle_y(p), f"M={M}")
    for i in range(2):
        assert torch.equal(call(), y), f"repeat {i}"
    out = torch.empty_like(y)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call(out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(out)
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y), f"replay {i}"
        _ = (d["x"].float() * 2).sum().item()  # eager work between replays
    monkeypatch.setenv("GLQ_PF_SPIN_TICKS", "0")
    for i in range(2):
        assert torch.equal(call(), y), f"zero-tick wait {i}"
    monkeypatch.delenv("GLQ_PF_SPIN_TICKS")
    monkeypatch.setenv("GLQ_PF_XU1", "1")
    assert torch.equal(call(), y), "separate one-launch x U"
    monkeypatch.delenv("GLQ_PF_XU1")
    assert torch.equal(call(), y), "fused again"
    monkeypatch.setenv("GLQ_PF_XU2", "1")
    y2 = call()
    torch.cuda.synchronize()
    assert_parity(y2, oracle_y(p), f"two-launch x U M={M}")
