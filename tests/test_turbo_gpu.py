"""GPU parity of the TurboQuant codebook kernel and the RHT kernel against the
CPU oracle.

Bar (north star): |y - y_ref| <= 1e-3 + 1e-2 |y_ref| (fp16 out, fp32
accumulation), y_ref the fp64 sum norm[n] * sum_k C[q] x_rot (the reference
kernel, turbo_matmul.cu:80-137, accumulates in fp32 and scales last).  The
reference's own test bar, max |y - y_fp32| < 0.01 against its fp32 PyTorch
path (inference/kernels/test_kernels.py:24-41, :105), is checked as well
where |y| keeps fp16's rounding below it.  Shapes follow that test (Mixtral
N=14336 x K=4096 and transposed, B in {1, 4, 16, 32}, 64 x 64) plus the
Qwen expert shapes and the edge cases of the host code (tails, K=14336 with 16
tokens, empty input).  RHT: fp16 output within one fp16 rounding of the fp64
transform.
"""

import numpy as np
import pytest
import torch

from glorcq_amd import format as fmt
from glorcq_amd import hadamard_rotation as HR
from glorcq_amd import kernels as K_
from glorcq_amd.quantized_linear import GLoRCQLinear, RotationCache
from oracle import glorcq_oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def check(y, ref, what, rtol=RTOL, atol=ATOL):
    y = y.float().cpu().double()
    ref = ref.double().cpu()
    assert y.shape == ref.shape, (what, tuple(y.shape), tuple(ref.shape))
    err = (y - ref).abs()
    bad = err > atol + rtol * ref.abs()
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {bad.numel()} outside bar, "
                                 f"max err {err.max().item():.3e}")


def refs(p, i=0, lora=False, bias=False, x_rot=None):
    """fp64 oracle output of item i (+ the fp16 low-rank factor and bias)."""
    xr = p.x_rot[i] if x_rot is None else x_rot
    y = O.turbo_matmul_fp64(xr, p.packed[i].numpy(), p.norms[i], p.centroids)
    if lora:
        a = (p.x[i].double() @ p.U.double()).half()
        y = y + a.double() @ p.SV[i].double().T
    if bias:
        y = y + p.bias[i].double()[None, :]
    return y


def run(p, dev, lora=False, bias=False):
    words = p.words().to(dev)
    xU = None
    if lora:
        xU = K_.lowrank_xu(p.x.to(dev).reshape(-1, p.K), p.U.to(dev)).reshape(p.items, p.M, -1)
    y = K_.turbo_gemv(p.x_rot.to(dev), words, p.norms.to(dev), p.centroids.to(dev),
                      xU=xU, SV=None if not lora else p.SV.to(dev),
                      bias=None if not bias else p.bias.to(dev))
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("K,N,M", [
    (2048, 1408, 1), (2048, 1408, 4), (1408, 2048, 1), (1408, 2048, 16),
    (64, 64, 1), (64, 64, 5), (4096, 14336, 1), (4096, 14336, 4), (14336, 4096, 16),
    (14336, 4096, 32), (4096, 14336, 32), (192, 40, 17), (320, 7, 33),
])
def test_turbo_gemv_shapes(gpu, K, N, M):
    print(f"turbo K={K} N={N} M={M}", flush=True)
    p = fmt.make_turbo(K, N, M=M, seed=K + N + M)
    y = run(p, gpu)[0]
    check(y, refs(p), f"K={K} N={N} M={M}")
    y32 = O.turbo_matmul_fp32(p.x_rot[0], p.packed[0].numpy(), p.norms[0], p.centroids)
    assert float((y.float().cpu() - y32).abs().max()) < 0.01  # the reference test's bar


@pytest.mark.parametrize("K,N,M", [(4096, 512, 1), (1024, 256, 32), (64, 64, 4)])
def test_turbo_gemv_reference_test_data(gpu, K, N, M):
    """The reference test's distributions (randn codebook, |randn|+0.1 norms):
    |y| reaches hundreds, so only the relative bar applies."""
    p = fmt.make_turbo(K, N, M=M, seed=5 + M, dist="randn")
    check(run(p, gpu)[0], refs(p), f"randn K={K} N={N} M={M}")


@pytest.mark.parametrize("M", [1, 3, 16, 20])
def test_turbo_lora_bias(gpu, M):
    p = fmt.make_turbo(2048, 1408, M=M, seed=30 + M, rank=64, bias=True)
    y = run(p, gpu, lora=True, bias=True)[0]
    check(y, refs(p, lora=True, bias=True), f"lora+bias M={M}")


@pytest.mark.parametrize("K,N,M,items,rank,bias", [
    (2048, 40000 - 6, 1, 1, 0, False),   # many rows of one matrix, N tail
    (1408, 2048, 1, 60, 0, False),       # grouped down over 60 experts
    (1408, 2048, 16, 16, 32, True),      # 16 tokens, low-rank term, bias
    (4096, 32768, 1, 1, 0, False),       # two prefetch rounds per tile
    (1152, 40000, 3, 1, 64, True),       # partial last step, idle prefetch slots
])
def test_turbo_streaming_form(gpu, K, N, M, items, rank, bias):
    """Problems of >= 2048 tiles take the streaming kernel (waves walk tiles)."""
    print(f"turbo stream K={K} N={N} M={M} items={items} r={rank}", flush=True)
    p = fmt.make_turbo(K, N, M=M, items=items, seed=K + N + items, rank=rank, bias=bias)
    y = run(p, gpu, lora=rank > 0, bias=bias)
    for i in range(items):
        check(y[i], refs(p, i, lora=rank > 0, bias=bias), f"stream item {i}")


def test_turbo_rank_not_multiple_of_32(gpu):
    p = fmt.make_turbo(1408, 300, M=2, seed=8, rank=40)
    check(run(p, gpu, lora=True)[0], refs(p, lora=True), "rank 40")


def test_turbo_batched_items(gpu):
    p = fmt.make_turbo(1408, 256, M=2, items=5, seed=9, rank=32, bias=True)
    y = run(p, gpu, lora=True, bias=True)
    for i in range(p.items):
        check(y[i], refs(p, i, lora=True, bias=True), f"item {i}")


def test_grouped_gemv_reference_signature(gpu):
    """turbo_dequant_grouped_gemv_fused (inference/kernels/__init__.py:242-278):
    E experts, each with its own input row, outputs concatenated."""
    E, K, N = 6, 1408, 2048
    p = fmt.make_turbo(K, N, M=1, items=E, seed=10)
    packed_cat = p.packed.reshape(E * N, K // 4).to(gpu)
    y = K_.turbo_dequant_grouped_gemv_fused(p.x_rot[:, 0].to(gpu), packed_cat,
                                            p.norms.reshape(-1).to(gpu), p.centroids.to(gpu), N)
    torch.cuda.synchronize()
    assert y.shape == (E * N,) and y.dtype == torch.float16
    for e in range(E):
        check(y[e * N:(e + 1) * N][None], refs(p, e), f"expert {e}")


def test_matmul_fused_with_pi_and_lora(gpu):
    """turbo_dequant_matmul_fused (inference/kernels/__init__.py:184-239) with a
    QR rotation and lora_USV."""
    K, N, M, r = 512, 384, 3, 32
    p = fmt.make_turbo(K, N, M=M, seed=11)
    g = torch.Generator().manual_seed(12)
    Pi, _ = torch.linalg.qr(torch.randn(K, K, generator=g))
    U = (torch.randn(K, r, generator=g) * 0.05).half()
    S = (torch.rand(r, generator=g) + 0.5).half()
    V = (torch.randn(N, r, generator=g) * 0.05).half()
    x = p.x[0]
    y = K_.turbo_dequant_matmul_fused(x.to(gpu), p.packed[0].to(gpu), p.norms[0].to(gpu),
                                      Pi.half().to(gpu), p.centroids.to(gpu), 2, K,
                                      lora_USV=(U.to(gpu), S.to(gpu), V.to(gpu)))
    torch.cuda.synchronize()
    x_rot = O.rotate_qr(x, Pi.half())
    ref = O.turbo_matmul_fp64(x_rot, p.packed[0].numpy(), p.norms[0], p.centroids)
    SV = (V.float() * S.float()[None, :]).half()
    a = (x.double() @ U.double()).half()
    check(y, ref + a.double() @ SV.double().T, "fused Pi + lora")
    with pytest.raises(RuntimeError, match="2-bit"):
        K_.turbo_dequant_matmul_fused(x.to(gpu), p.packed[0].to(gpu), p.norms[0].to(gpu),
                                      Pi.half().to(gpu), p.centroids.to(gpu), 4, K)


def test_empty_batch(gpu):
    p = fmt.make_turbo(256, 64, M=1, seed=13)
    y = K_.turbo_gemv(torch.empty(0, 256, dtype=torch.float16, device=gpu), p.words()[0].to(gpu),
                      p.norms[0].to(gpu), p.centroids.to(gpu))
    assert y.shape == (0, 64)


def fp16_ulp(v):
    e = torch.floor(torch.log2(v.abs().clamp_min(2.0 ** -14)))
    return 2.0 ** (e - 10)


@pytest.mark.parametrize("d,rows", [(2, 3), (64, 5), (2048, 7), (16384, 2)])
def test_rht_forward_fp16(gpu, d, rows):
    g = torch.Generator().manual_seed(d)
    x = torch.randn(rows, d, generator=g).half()
    signs = O.generate_rht_signs(d, seed=42)
    y = HR.rht_rotate_half(x.to(gpu), signs.to(gpu))
    torch.cuda.synchronize()
    ref = O.rht_forward(x, signs)
    err = (y.double().cpu() - ref).abs()
    assert bool((err <= fp16_ulp(ref) * 0.5 + 1e-6 * ref.abs().max()).all()), float(err.max())


def test_rht_fp32_and_inverse(gpu):
    d = 1024
    g = torch.Generator().manual_seed(14)
    x = torch.randn(4, d, generator=g)
    signs = HR.generate_rht_signs(d, seed=3, device=gpu)
    y = HR.rht_forward(x.to(gpu), signs)
    z = HR.rht_backward(y, signs)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    ref = O.rht_forward(x, signs.cpu())
    assert torch.allclose(y.double().cpu(), ref, atol=1e-5, rtol=1e-5)
    assert torch.allclose(z.double().cpu(), x.double(), atol=1e-5, rtol=1e-5)


def _turbo_layer(p, dev, rank=0, bias=False, rht=False):
    lin = GLoRCQLinear(p.K, p.N).to(dev)
    cache = RotationCache(device=dev)
    g = torch.Generator().manual_seed(15)
    Pi = None if rht else torch.linalg.qr(torch.randn(p.K, p.K, generator=g))[0].half()
    cache.put(p.K, 2, 42, Pi, p.centroids)
    lin.load_turbo({"packed_indices": p.packed[0], "norms": p.norms[0], "bits": 2,
                    "dim": p.K, "seed": 42}, cache, device=dev)
    if rank:
        lin.load_sv(p.U, p.SV[0], device=dev)
    if bias:
        lin.set_bias(p.bias[0], device=dev)
    if rht:
        lin._rht_signs = HR.generate_rht_signs(p.K, seed=42, device=dev)
    return lin, Pi


@pytest.mark.parametrize("rht", [False, True])
def test_glorcq_linear_turbo_forward(gpu, rht):
    p = fmt.make_turbo(1024, 512, M=4, seed=16, rank=32, bias=True)
    lin, Pi = _turbo_layer(p, gpu, rank=32, bias=True, rht=rht)
    y = lin(p.x[0].to(gpu))
    torch.cuda.synchronize()
    if rht:
        x_rot = O.rht_forward(p.x[0], O.generate_rht_signs(p.K, seed=42)).half()
    else:
        x_rot = O.rotate_qr(p.x[0], Pi)
    check(y, refs(p, lora=True, bias=True, x_rot=x_rot), f"GLoRCQLinear turbo rht={rht}")
    # precomputed rotation and x U (the MoE block's hooks)
    xu = (p.x[0].double() @ p.U.double()).half()
    y2 = lin(p.x[0].to(gpu), precomputed_xU=xu.to(gpu), precomputed_x_rot=p.x_rot[0].to(gpu))
    torch.cuda.synchronize()
    check(y2, refs(p, lora=True, bias=True), "precomputed x_rot + xU")
