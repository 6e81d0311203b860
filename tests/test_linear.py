"""GLoRCQLinear / GLoRCQExperts host layer (glorcq_amd/quantized_linear.py),
loaded from the reference's on-disk dict format (joint_optim.py:320-327):
CPU checks of the loaders, GPU parity of forward against the oracle."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from glorcq_amd import format as fmt
from glorcq_amd.quantized_linear import GLoRCQExperts, GLoRCQLinear, container_bits
from oracle import glorcq_oracle as O

RTOL, ATOL = 1e-2, 1e-3


def gptq_dict(p, bits=None):
    return {"qweight_int": p.q.clone(), "scales": p.scales.clone(), "zeros": p.zeros.clone(),
            "bits": bits or p.bits, "groupsize": p.group, "sym": p.sym}


def close(y, ref):
    y = y.double().cpu()
    ref = ref.double().cpu()
    err = (y - ref).abs()
    assert bool((err <= ATOL + RTOL * ref.abs()).all()), float(err.max())


# ------------------------------------------------------------------ CPU ----
def test_container_bits():
    assert container_bits(2) == 2 and container_bits(3) == 4 and container_bits(4) == 4
    with pytest.raises(RuntimeError):
        container_bits(8)


def test_load_gptq_packs_like_oracle_on_cpu():
    p = fmt.make_linear(256, 48, bits=2, rank=16, seed=1)
    lin = GLoRCQLinear(256, 48)
    lin.load_gptq(gptq_dict(p), device="cpu")
    assert np.array_equal(lin.codes.numpy(), O.pack_codes(p.q.numpy(), 2))
    assert lin.pack_bits == 2 and lin.gptq_groupsize == 128 and not lin.gptq_sym
    # 3-bit checkpoint codes go to the 4-bit container unchanged
    g = torch.Generator().manual_seed(2)
    q3 = torch.randint(0, 8, (48, 256), generator=g, dtype=torch.int32)
    d = gptq_dict(p, bits=3)
    d["qweight_int"] = q3
    lin.load_gptq(d, device="cpu")
    assert lin.pack_bits == 4
    assert np.array_equal(O.unpack_codes(lin.codes.numpy(), 4, 256), q3.numpy())


def test_load_checks_and_lora_fusion():
    p = fmt.make_linear(256, 48, bits=4, rank=16, seed=3)
    lin = GLoRCQLinear(256, 64)
    with pytest.raises(RuntimeError, match="shape"):
        lin.load_gptq(gptq_dict(p), device="cpu")
    # turbo loader checks: code width, shape, and a rotation cache that was
    # never given the rotation/codebook (the turboquant package is absent)
    from glorcq_amd.quantized_linear import RotationCache
    tp = fmt.make_turbo(256, 64, seed=5)
    td = {"packed_indices": tp.packed[0], "norms": tp.norms[0], "bits": 3, "dim": 256}
    with pytest.raises(RuntimeError, match="3-bit"):
        lin.load_turbo(td, RotationCache("cpu"), device="cpu")
    td["bits"] = 2
    with pytest.raises(RuntimeError, match="turboquant"):
        lin.load_turbo(td, RotationCache("cpu"), device="cpu")
    with pytest.raises(RuntimeError, match="shape"):
        GLoRCQLinear(256, 48).load_turbo(td, RotationCache("cpu"), device="cpu")
    cache = RotationCache("cpu")
    cache.put(256, 2, 42, None, tp.centroids)
    lin.load_turbo(td, cache, device="cpu")
    assert lin.quant_type == "turbo" and lin.turbo_words.shape == (64, 16)
    assert torch.equal(lin.turbo_words, tp.words()[0])
    lin = GLoRCQLinear(256, 48)
    S = torch.rand(16, generator=torch.Generator().manual_seed(4)) + 0.5
    lin.load_lora(p.U, S, p.SV, device="cpu")
    assert torch.equal(lin.SV, (p.SV.float() * S[None]).half())
    assert lin.rank == 16
    assert "lora_rank=16" in lin.extra_repr()


def test_forward_without_load_raises():
    with pytest.raises(RuntimeError):
        GLoRCQLinear(128, 16)(torch.zeros(1, 128, dtype=torch.float16))


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
@pytest.mark.parametrize("bits,sym", [(2, False), (4, False), (2, True), (4, True)])
def test_forward_parity(gpu, bits, sym):
    p = fmt.make_linear(2048, 1408, bits=bits, rank=64, M=3, seed=40 + bits + sym, sym=sym)
    lin = GLoRCQLinear(2048, 1408)
    lin.load_gptq(gptq_dict(p), device=gpu)
    lin.load_sv(p.U, p.SV, device=gpu)
    x3 = p.x.reshape(1, 3, 2048)  # (batch, seq, K) like an HF hidden state
    y = lin(x3.to(gpu))
    assert y.shape == (1, 3, 1408) and y.dtype == torch.float16
    ref = O.linear_forward_fp32(p.x, p.q, p.scales, p.zeros, 128, sym, U=p.U, SV=p.SV)
    close(y.reshape(3, 1408), ref)
    W = lin._dequant_gptq().cpu()
    assert torch.equal(W, O.dequant_fp16(p.q, p.scales, p.zeros, 128, sym))


@pytest.mark.gpu
def test_forward_3bit_bias_precomputed_xu(gpu):
    g = torch.Generator().manual_seed(7)
    p = fmt.make_linear(1024, 512, bits=4, rank=32, M=2, seed=8)
    q3 = torch.randint(0, 8, (512, 1024), generator=g, dtype=torch.int32)
    d = gptq_dict(p, bits=3)
    d["qweight_int"] = q3
    lin = GLoRCQLinear(1024, 512)
    lin.load_gptq(d, device=gpu)
    lin.load_sv(p.U, p.SV, device=gpu)
    bias = (torch.randn(512, generator=g) * 0.1).half()
    lin.set_bias(bias, device=gpu)
    xu = (p.x.float() @ p.U.float()).half()
    y = lin(p.x.to(gpu), precomputed_xU=xu.to(gpu))
    ref = O.linear_forward_fp32(p.x, q3, p.scales, p.zeros, 128, U=p.U, SV=p.SV,
                                precomputed_xU=xu, bias=bias)
    close(y, ref)


@pytest.mark.gpu
def test_experts_container(gpu):
    """GLoRCQExperts against the reference dispatch semantics computed with the
    oracle per expert (inference/quantized_linear.py:395-428)."""
    E, H, I, T, topk = 4, 256, 384, 5, 2
    gen = torch.Generator().manual_seed(11)
    ex = GLoRCQExperts(E, H, I, F.silu)
    probs = {}
    for e in range(E):
        for name, (k, n) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
            p = fmt.make_linear(k, n, bits=2, rank=16, seed=1000 + 10 * e + len(name))
            probs[(name, e)] = p
            mod = getattr(ex, f"{name}_experts")[e]
            mod.load_gptq(gptq_dict(p), device=gpu)
            mod.load_sv(p.U, p.SV, device=gpu)
    h = torch.randn(T, H, generator=gen).half()
    logits = torch.randn(T, E, generator=gen)
    w, idx = torch.topk(torch.softmax(logits, -1), topk, dim=-1)
    w = w.half()
    out = ex(h.to(gpu), idx.to(gpu), w.to(gpu)).cpu()

    def lin(name, e, x):
        p = probs[(name, e)]
        return O.linear_forward_fp32(x, p.q, p.scales, p.zeros, 128, U=p.U, SV=p.SV)

    ref = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for k in range(topk):
            e = int(idx[t, k])
            x = h[t:t + 1]
            inter = (F.silu(lin("gate", e, x).float()) * lin("up", e, x).float()).half()
            ref[t] += float(w[t, k]) * lin("down", e, inter).double()[0]
    err = (out.double() - ref).abs()
    assert bool((err <= 2e-3 + 2e-2 * ref.abs()).all()), float(err.max())
