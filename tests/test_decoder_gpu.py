"""Decoder-layer kernels of the model-level decode step (glq_rmsnorm,
glq_qk_norm_rope, glq_decode_attention via glorcq_amd.kernels) against the
transformers Qwen3-MoE ops they replace (run on the GPU in fp16: the same
rounding points) and fp32 references, and the fused decoder layers against
transformers' own layer code around the same GLoRCQ projections and MoE
blocks.

Bars: the rounding points are the framework's, but the fp32 sum order and
rsqrt may differ by an fp32 ulp, which can move the first fp16 rounding by
one ulp; the weight product after it scales that (weights here lie in
[0.5, 1.5]) -- so RMSNorm within 2 fp16 ulps of the framework op, and the
rotary output (a sum of two rounded products, which may cancel) within
3 eps (|x_i| + |x_partner|) of it, x the normed head; residual sums and cache
copies bit-exact; attention within atol 2e-3 + rtol
1e-2 of an fp32 softmax(q K^T s) V; the fused model's logits within 1 % of
their range of the framework-layer model's, with the same greedy tokens.
"""

import pytest
import torch

from glorcq_amd import kernels

pytestmark = pytest.mark.gpu


def ulps(a, b):
    """Distance in fp16 ulps of b (floored at the smallest normal's ulp)."""
    d = (a.float() - b.float()).abs()
    u = torch.finfo(torch.float16).eps * b.float().abs().clamp(min=2.0**-14)
    return float((d / u).max())


def _hf_norm(dim, eps, dev, seed):
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRMSNorm

    m = Qwen3MoeRMSNorm(dim, eps=eps).to(dev).half().requires_grad_(False)
    g = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        m.weight.copy_((0.5 + torch.rand(dim, generator=g, device=dev)).half())
    return m


@pytest.mark.parametrize("rows,dim", [(1, 2048), (16, 2048), (37, 4096), (5, 8192), (3, 136)])
def test_rmsnorm_matches_framework(gpu, rows, dim):
    m = _hf_norm(dim, 1e-6, gpu, rows)
    g = torch.Generator(device=gpu).manual_seed(dim)
    x = (torch.randn(rows, dim, generator=g, device=gpu) * 3).half()
    r = torch.randn(rows, dim, generator=g, device=gpu).half()
    with torch.no_grad():
        out = kernels.rmsnorm(x, m.weight, 1e-6)
        ref = m(x)
        assert ulps(out, ref) <= 2.0
        out2, y = kernels.rmsnorm(x, m.weight, 1e-6, residual=r)
        assert torch.equal(y, x + r)
        assert ulps(out2, m(x + r)) <= 2.0
    # fp64 restatement: a dropped weight or eps would fail this
    xd = (x.double() + r.double()).half().double()
    ref64 = (xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)).half().double() \
        * m.weight.double()
    assert float((out2.double() - ref64).abs().max()) <= 4e-3 * float(ref64.abs().max())


def _xu_bar(xu, ref):
    """x U as fp32 partials summed, against the fp32 product of the fp16 rows:
    the sum orders differ (relative 2^-16 of the row's terms) -- within
    2^-12 |ref| + 1e-4 of the row's largest magnitude."""
    err = (xu.float() - ref).abs()
    tol = 2.0 ** -12 * ref.abs() + 1e-4 * ref.abs().amax(-1, keepdim=True) + 1e-5
    return bool((err <= tol).all()), float(err.max())


@pytest.mark.parametrize("rows,dim,n_u,rank", [(1, 2048, 3, 64), (2, 2048, 3, 64),
                                               (3, 2048, 1, 96), (16, 2048, 2, 32),
                                               (1, 4096, 1, 128), (5, 136, 2, 64)])
def test_rmsnorm_xu(gpu, rows, dim, n_u, rank):
    """glq_rmsnorm_xu: the normalized rows (and the fused residual sum) carry
    the bits of glq_rmsnorm; the slice partials summed give out U[u] within
    fp32 rounding of the fp32 product (columns past rank zero); a second call
    gives the same bits; a planted wrong U (the stack's order reversed) fails
    the bar."""
    m = _hf_norm(dim, 1e-6, gpu, rows + 7)
    g = torch.Generator(device=gpu).manual_seed(dim + rows)
    x = (torch.randn(rows, dim, generator=g, device=gpu) * 3).half()
    r = torch.randn(rows, dim, generator=g, device=gpu).half()
    U = (torch.randn(n_u, dim, rank, generator=g, device=gpu) * 0.05).half()
    S, rpad = (dim + 255) // 256, (rank + 31) // 32 * 32
    with torch.no_grad():
        out, parts = kernels.rmsnorm_xu(x, m.weight, 1e-6, U)
        assert torch.equal(out, kernels.rmsnorm(x, m.weight, 1e-6))
        out2, y, parts2 = kernels.rmsnorm_xu(x, m.weight, 1e-6, U, residual=r)
        ref_out, ref_y = kernels.rmsnorm(x, m.weight, 1e-6, residual=r)
        assert torch.equal(out2, ref_out) and torch.equal(y, ref_y)
        again = kernels.rmsnorm_xu(x, m.weight, 1e-6, U, residual=r)[2]
    torch.cuda.synchronize()
    assert tuple(parts.shape) == (n_u, S, rows, rpad)
    assert torch.equal(parts2, again)
    assert not bool(parts[..., rank:].any())
    for o, pt in ((out, parts), (out2, parts2)):
        ref = torch.matmul(o.float().unsqueeze(0), U.float())  # (n_u, rows, rank)
        ok, worst = _xu_bar(pt.sum(1)[..., :rank], ref)
        assert ok, worst
    if n_u > 1:
        wrong = torch.matmul(out.float().unsqueeze(0), U.flip(0).float())
        assert not _xu_bar(parts.sum(1)[..., :rank], wrong)[0]


def _rope(dev, positions):
    from glorcq_amd.synthetic_model import qwen3_moe_config
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeRotaryEmbedding

    cfg = qwen3_moe_config(num_hidden_layers=1, vocab_size=64)
    rot = Qwen3MoeRotaryEmbedding(config=cfg).to(dev)
    x = torch.zeros(1, 1, 2048, dtype=torch.float16, device=dev)
    return rot(x, torch.tensor([positions], device=dev))


@pytest.mark.parametrize("B,pos,shared_rows", [(1, 0, True), (1, 511, True), (4, 37, True),
                                               (3, 100, False)])
def test_qk_norm_rope_matches_framework(gpu, B, pos, shared_rows):
    from transformers.models.qwen3_moe.modeling_qwen3_moe import apply_rotary_pos_emb

    Hq, Hk, hd, L = 32, 4, 128, 640
    g = torch.Generator(device=gpu).manual_seed(pos + B)
    q = torch.randn(B, Hq * hd, generator=g, device=gpu).half()
    k = torch.randn(B, Hk * hd, generator=g, device=gpu).half()
    v = torch.randn(B, Hk * hd, generator=g, device=gpu).half()
    qn, kn = _hf_norm(hd, 1e-6, gpu, 1), _hf_norm(hd, 1e-6, gpu, 2)
    cos, sin = _rope(gpu, [pos])
    if not shared_rows:  # one row per token (same position), cs_stride = 128
        cos, sin = cos.expand(B, 1, hd).contiguous(), sin.expand(B, 1, hd).contiguous()
    kc = torch.zeros(B, Hk, L, hd, dtype=torch.float16, device=gpu)
    vc = torch.zeros_like(kc)
    p = torch.tensor(pos, dtype=torch.int64, device=gpu)
    ln = torch.zeros(1, dtype=torch.int32, device=gpu)
    with torch.no_grad():
        qo = kernels.qk_norm_rope(q, k, v, qn.weight, kn.weight, 1e-6, cos, sin, kc, vc, p, ln)
        rq = qn(q.view(B, 1, Hq, hd)).transpose(1, 2)
        rk = kn(k.view(B, 1, Hk, hd)).transpose(1, 2)
        rq, rk = apply_rotary_pos_emb(rq, rk, cos, sin)
        # q item-major (a batched GEMV's output over 512-row slices): same bits
        kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
        q_im = q.view(B, Hq * hd // 512, 512).transpose(0, 1).contiguous()
        qo2 = kernels.qk_norm_rope(q_im, k, v, qn.weight, kn.weight, 1e-6, cos, sin, kc2, vc2, p,
                                   ln)
    torch.cuda.synchronize()
    assert torch.equal(qo2, qo) and torch.equal(kc2, kc) and torch.equal(vc2, vc)
    assert int(ln) == pos + 1
    eps = torch.finfo(torch.float16).eps
    for got, ref, nrm in ((qo, rq[:, :, 0], qn(q.view(B, Hq, hd))),
                          (kc[:, :, pos], rk[:, :, 0], kn(k.view(B, Hk, hd)))):
        a = nrm.float().abs()
        bound = 3 * eps * (a + torch.cat([a[..., 64:], a[..., :64]], dim=-1)) + 2.0**-24
        assert bool(((got.float() - ref.float()).abs() <= bound).all())
    assert torch.equal(vc[:, :, pos], v.view(B, Hk, hd))
    mask = torch.ones(L, dtype=torch.bool)
    mask[pos] = False
    assert not kc[:, :, mask].any() and not vc[:, :, mask].any()
    # rotary convention pinned independently: pairs (i, i + 64) rotate by the
    # position's angle, so norms of each pair are kept (to fp16 rounding)
    n = qn(q.view(B, Hq, hd)).float()
    pair = lambda t: (t[..., :64].pow(2) + t[..., 64:].pow(2)).sqrt()  # noqa: E731
    assert torch.allclose(pair(qo.float()), pair(n), rtol=2e-3, atol=2e-3)


def test_qk_norm_rope_out_of_range_position_writes_nothing(gpu):
    """A position past the static cache writes no cache row and turns q' into
    NaN, so the step's attention output shows the overflow."""
    B, Hq, Hk, hd, L = 1, 32, 4, 128, 64
    q = torch.randn(B, Hq * hd, device=gpu).half()
    k, v = torch.randn(B, Hk * hd, device=gpu).half(), torch.randn(B, Hk * hd, device=gpu).half()
    w = torch.ones(hd, dtype=torch.float16, device=gpu)
    cos, sin = _rope(gpu, [3])
    kc = torch.zeros(B, Hk, L, hd, dtype=torch.float16, device=gpu)
    vc = torch.zeros_like(kc)
    ln = torch.zeros(1, dtype=torch.int32, device=gpu)
    qo = kernels.qk_norm_rope(q, k, v, w, w, 1e-6, cos, sin, kc, vc,
                              torch.tensor(L, dtype=torch.int64, device=gpu), ln)
    torch.cuda.synchronize()
    assert not kc.any() and not vc.any() and int(ln) == L + 1
    assert torch.isnan(qo.float()).all()


@pytest.mark.parametrize("B,Hq,Hk,L,maxlen", [(1, 32, 4, 1, 640), (1, 32, 4, 513, 640),
                                              (16, 32, 4, 600, 640), (2, 8, 8, 1000, 1024),
                                              (3, 16, 2, 4096, 4096), (1, 32, 4, 128, 130),
                                              (2, 24, 4, 129, 129)])
def test_decode_attention_matches_fp32(gpu, B, Hq, Hk, L, maxlen):
    hd = 128
    g = torch.Generator(device=gpu).manual_seed(L + B)
    q = torch.randn(B, Hq, hd, generator=g, device=gpu).half()
    kc = torch.randn(B, Hk, maxlen, hd, generator=g, device=gpu).half()
    vc = torch.randn(B, Hk, maxlen, hd, generator=g, device=gpu).half()
    kc[:, :, L:] = 60.0  # positions past L would dominate every softmax if read
    vc[:, :, L:] = 1000.0
    ln = torch.tensor([L], dtype=torch.int32, device=gpu)
    adv = torch.tensor(L - 1, dtype=torch.int64, device=gpu)
    scale = hd ** -0.5
    ws = kernels.decode_attention_workspace(q, kc)
    out = kernels.decode_attention(q, kc, vc, ln, scale, advance=adv, workspace=ws)
    again = kernels.decode_attention(q, kc, vc, ln, scale, workspace=ws)  # counters reset
    torch.cuda.synchronize()
    assert int(adv) == L
    assert torch.equal(out, again)
    rep = Hq // Hk
    K = kc[:, :, :L].float().repeat_interleave(rep, dim=1)
    V = vc[:, :, :L].float().repeat_interleave(rep, dim=1)
    Kt = K.transpose(-1, -2).contiguous()
    s = torch.matmul(q.float().unsqueeze(2), Kt).squeeze(2) * scale
    ref = torch.matmul(torch.softmax(s, dim=-1).unsqueeze(2), V).squeeze(2).reshape(B, Hq * hd)
    err = (out.float() - ref).abs()
    assert bool((err <= 2e-3 + 1e-2 * ref.abs()).all()), float(err.max())


@pytest.mark.parametrize("B,Hq,Hk,L,maxlen,rank", [(1, 32, 4, 600, 640, 64),
                                                    (2, 32, 4, 1, 640, 64),
                                                    (3, 16, 4, 300, 512, 32),
                                                    (1, 8, 8, 129, 256, 128)])
def test_decode_attention_xu(gpu, B, Hq, Hk, L, maxlen, rank):
    """glq_decode_attention_xu: out carries the bits of glq_decode_attention
    and the KV groups' partials summed give out U within fp32 rounding of the
    fp32 product; repeated calls give the same bits and advance the fill
    counter once each; a planted wrong row order of U fails the bar."""
    hd = 128
    g = torch.Generator(device=gpu).manual_seed(L + 3 * B)
    q = torch.randn(B, Hq, hd, generator=g, device=gpu).half()
    kc = torch.randn(B, Hk, maxlen, hd, generator=g, device=gpu).half()
    vc = torch.randn(B, Hk, maxlen, hd, generator=g, device=gpu).half()
    U = (torch.randn(Hq * hd, rank, generator=g, device=gpu) * 0.05).half()
    ln = torch.tensor([L], dtype=torch.int32, device=gpu)
    adv = torch.tensor(0, dtype=torch.int64, device=gpu)
    scale = hd ** -0.5
    ref_out = kernels.decode_attention(q, kc, vc, ln, scale)
    ws = kernels.decode_attention_workspace(q, kc)
    out, parts = kernels.decode_attention(q, kc, vc, ln, scale, advance=adv, workspace=ws, U=U)
    out2, parts2 = kernels.decode_attention(q, kc, vc, ln, scale, advance=adv, workspace=ws,
                                            U=U)
    torch.cuda.synchronize()
    assert int(adv) == 2
    assert torch.equal(out, ref_out) and torch.equal(out2, out) and torch.equal(parts2, parts)
    assert tuple(parts.shape) == (Hk, B, (rank + 31) // 32 * 32)
    xu = parts.sum(0)[:, :rank]
    ok, worst = _xu_bar(xu, out.float() @ U.float())
    assert ok, worst
    wrong = out.float() @ U.roll(Hq // Hk * hd, dims=0).float()
    assert not _xu_bar(xu, wrong)[0]


def _models(dev, layers=2):
    from glorcq_amd.synthetic_model import build_qwen3_moe, qwen3_moe_config

    cfg = qwen3_moe_config(num_hidden_layers=layers, vocab_size=2048,
                           max_position_embeddings=256)
    fused, _ = build_qwen3_moe(cfg, dev, seed=4, fused=True)
    plain, _ = build_qwen3_moe(cfg, dev, seed=4, fused=False)
    return cfg, fused, plain


@torch.no_grad()
@pytest.mark.parametrize("B,producer", [(1, False), (1, True), (2, True), (12, False)])
def test_fused_layers_match_framework_layers(gpu, monkeypatch, B, producer):
    """The same weights (same seed) with the fused decoder layers and with
    transformers' layer code: a 20-token prefill and 8 decode steps through
    static caches give logits within 1 % of the range and the same greedy
    tokens where the margin allows; the caches agree within fp16 rounding.
    B = 1 takes x U in the projections' own one-row launches (x U jobs in
    front of the row workgroups) and, forced, from the launches that produce
    the projections' inputs (glq_rmsnorm_xu for q/k/v,
    glq_decode_attention_xu for o), as B = 2 does; B = 12 the token-tile
    forms with x U in their own launches."""
    from glorcq_amd import decoder
    from glorcq_amd.graph_wrapper import _static_cache

    if producer:
        monkeypatch.setattr(decoder.GLoRCQQwen3Attention, "XU_PRODUCER_MIN_M", 1)
    assert decoder.GLoRCQQwen3Attention.xu_by_producer(B) == producer

    cfg, fused, plain = _models(gpu)
    assert type(fused.model.layers[0]).__name__ == "GLoRCQQwen3DecoderLayer"
    ids = torch.randint(0, cfg.vocab_size, (B, 20), generator=torch.Generator().manual_seed(1))
    ids = ids.to(gpu)
    caches = [_static_cache(m, B, 64, gpu, torch.float16) for m in (fused, plain)]
    outs = [m(input_ids=ids, past_key_values=c, use_cache=True, return_dict=False)[0]
            for m, c in zip((fused, plain), caches)]
    checked = 0
    for step in range(8):
        a, b = outs[0][:, -1].float(), outs[1][:, -1].float()
        span = float(b.abs().max())
        assert float((a - b).abs().max()) <= 0.01 * span, (step, float((a - b).abs().max()))
        top2 = torch.topk(b, 2, dim=-1).values
        ok = (top2[:, 0] - top2[:, 1]) > 0.01 * span
        assert bool((a.argmax(-1) == b.argmax(-1))[ok].all()), step
        checked += int(ok.sum())
        t = b.argmax(-1, keepdim=True)
        outs = [m(input_ids=t, past_key_values=c, use_cache=True, return_dict=False)[0]
                for m, c in zip((fused, plain), caches)]
    assert checked >= min(8, 4 * B)  # (8 steps: B = 1 offers 8 comparisons in all)
    for la, lb in zip(caches[0].layers, caches[1].layers):
        assert int(la.cumulative_length) == int(lb.cumulative_length) == 28
        n = 28
        kd = (la.keys[:, :, :n].float() - lb.keys[:, :, :n].float()).abs().max()
        assert float(kd) <= 0.02 * float(lb.keys[:, :, :n].float().abs().max())
        assert torch.equal(la.keys[:, :, n:], lb.keys[:, :, n:])
