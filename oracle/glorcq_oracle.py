"""CPU oracle for the GLoRCQ hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or, in the bench, as the timed CPU
baseline).  The product path (glorcq_amd) never imports it.

Each function restates, in plain PyTorch-on-CPU / numpy, the reference
algorithm it cites (nicyyyy/GLoRCQ).  How each one is pinned (golden vectors,
closed forms, brute force) is written in its docstring; the checks live in
tests/test_oracle.py.

Reference rounding points of the CPU fallback GLoRCQLinear.forward
(inference/quantized_linear.py:286-355, no extension present):
  W  = fp16 dequant, group by group: fp16(fp16(q - z) * s)       (:271-284)
  y  = fp16(x @ W.T)                                             (:313-314)
  a  = fp16(x @ U)   (or the caller's precomputed_xU)            (:340-344)
  y  = fp16(y + fp16(a @ SV.T))                                  (:345)
  y  = fp16(y + bias)                                            (:348-349)
"""

from __future__ import annotations

import numpy as np
import torch


# ---------------------------------------------------------------------------
# Bit packing (format)
# ---------------------------------------------------------------------------
def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """(N, K) codes -> (N, K*bits/32) int32, built byte by byte.

    Follows the reference's LSB-first sub-byte order (turbo packing read by
    _unpack_indices_2bit, inference/kernels/__init__.py:113-118, and
    _unpack_indices, inference/quantized_linear.py:115-146: value j of a byte
    sits at bits [b*j, b*j+b)); four such bytes read as one little-endian
    int32 word form the packed container.  Signed codes are masked to b bits
    (two's complement, quantizer/quantizer.py:145-146).
    Pinned by: brute force over every value in every slot of one word, and
    pack(unpack(w)) == w over random words (tests/test_oracle.py).
    """
    q = np.asarray(q, dtype=np.int64)
    N, K = q.shape
    per_byte = 8 // bits
    assert K % (32 // bits) == 0
    v = (q & ((1 << bits) - 1)).astype(np.uint8).reshape(N, K // per_byte, per_byte)
    byte = np.zeros((N, K // per_byte), dtype=np.uint8)
    for j in range(per_byte):
        byte |= (v[:, :, j] << (bits * j)).astype(np.uint8)
    return byte.view("<i4").reshape(N, K * bits // 32).copy()


def unpack_codes(packed: np.ndarray, bits: int, K: int, sym: bool = False) -> np.ndarray:
    """(N, K*bits/32) int32 -> (N, K) int32 codes.

    The int32 words are viewed as little-endian bytes and unpacked exactly as
    the reference's _unpack_indices does (inference/quantized_linear.py:132-146):
    unpacked = (byte >> (b*j)) & (2^b - 1), j = 0..8/b-1, then trimmed to K.
    sym: sign-extend the b-bit two's complement value.
    """
    packed = np.ascontiguousarray(packed, dtype="<i4")
    N = packed.shape[0]
    per_byte = 8 // bits
    byte = packed.view(np.uint8).reshape(N, -1)
    shifts = np.arange(per_byte, dtype=np.uint8) * bits
    out = ((byte[:, :, None] >> shifts) & ((1 << bits) - 1)).reshape(N, -1)[:, :K]
    out = out.astype(np.int32)
    if sym:
        out = np.where(out >= (1 << (bits - 1)), out - (1 << bits), out).astype(np.int32)
    return out


# ---------------------------------------------------------------------------
# Dequantization
# ---------------------------------------------------------------------------
def dequant_fp16(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None,
                 groupsize: int, sym: bool = False) -> torch.Tensor:
    """GLoRCQLinear._dequant_gptq (inference/quantized_linear.py:271-284): fp16
    W, group by group, W = (q.half() - z) * s in fp16 arithmetic (sym: q * s).

    Pinned by the closed form: (q - z) is a small integer (exact in fp16) when
    z is integer-valued, and an IEEE fp16 multiply is correctly rounded, so W
    must equal fp16(fp32(s) * fp32(q - z)) bit for bit; checked against an
    fp64 route over every (q, z) pair and random scales.
    """
    q = torch.as_tensor(q)
    N, K = q.shape
    W = torch.zeros(N, K, dtype=torch.float16)
    n_groups = scales.shape[1]
    for gi in range(n_groups):
        c0 = gi * groupsize
        c1 = min(c0 + groupsize, K)
        qs = q[:, c0:c1].half()
        if sym:
            W[:, c0:c1] = qs * scales[:, gi:gi + 1]
        else:
            W[:, c0:c1] = (qs - zeros[:, gi:gi + 1]) * scales[:, gi:gi + 1]
    return W


def dequant_fp32(q: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor | None,
                 groupsize: int, sym: bool = False) -> torch.Tensor:
    """_gptq_pytorch_fallback's weight (inference/kernels/__init__.py:149-178):
    W = (q - z) * s computed in fp32."""
    q = torch.as_tensor(q)
    N, K = q.shape
    W = torch.zeros(N, K, dtype=torch.float32)
    for gi in range(scales.shape[1]):
        c0 = gi * groupsize
        c1 = min(c0 + groupsize, K)
        qs = q[:, c0:c1].float()
        if sym:
            W[:, c0:c1] = qs * scales[:, gi:gi + 1].float()
        else:
            W[:, c0:c1] = (qs - zeros[:, gi:gi + 1].float()) * scales[:, gi:gi + 1].float()
    return W


# ---------------------------------------------------------------------------
# GLoRCQLinear forward
# ---------------------------------------------------------------------------
def linear_forward_fp16(x: torch.Tensor, q: torch.Tensor, scales: torch.Tensor,
                        zeros: torch.Tensor | None, groupsize: int, sym: bool = False,
                        U: torch.Tensor | None = None, SV: torch.Tensor | None = None,
                        precomputed_xU: torch.Tensor | None = None,
                        bias: torch.Tensor | None = None) -> torch.Tensor:
    """The reference CPU fallback of GLoRCQLinear.forward (quantized_linear.py:
    286-355 with _HAS_GPTQ_FUSED_KERNEL False): fp16 dequant loop, fp16
    `x @ W.T`, fp16 LoRA `y + (x @ U) @ SV.T`, fp16 bias.  All arithmetic is
    torch-on-CPU in fp16, as the reference runs it.
    Pinned by: tolerance against linear_forward_fp64 (the exact sum of the
    exactly dequantized weights), which a wrong term, sign, index or transposed
    operand fails.
    """
    orig = x.shape
    x = x.reshape(-1, orig[-1]).half()
    W = dequant_fp16(q, scales, zeros, groupsize, sym)
    y = x @ W.T
    if SV is not None:
        a = precomputed_xU.half() if precomputed_xU is not None else x @ U.half()
        y = y + a @ SV.half().T
    if bias is not None:
        y = y + bias.half()
    return y.reshape(*orig[:-1], y.shape[-1])


def linear_forward_fp32(x, q, scales, zeros, groupsize, sym=False, U=None, SV=None,
                        bias=None, precomputed_xU=None) -> torch.Tensor:
    """The fallback of the op the fused kernel replaces: gptq_dequant_matmul_fused
    (inference/kernels/__init__.py:284-346) when its extension raises —
    _gptq_pytorch_fallback (:149-178: W = (q - z) * s in fp32, y = x_fp32 @ W.T)
    plus the fp32 lora_out (:311-315), cast to fp16 once (:346).  The
    reference's own kernel tests use the same oracle (reference_gptq_dequant_
    matmul, inference/kernels/test_gptq_kernel.py:17-53).
    Pinned by: tolerance against linear_forward_fp64(exact_weights=True), and
    W = dequant_fp32 equals the exact product s*(q - z) (tests/test_oracle.py).
    """
    xf = x.float()
    y = xf @ dequant_fp32(q, scales, zeros, groupsize, sym).T
    if SV is not None:
        a = precomputed_xU.float() if precomputed_xU is not None else xf @ U.float()
        y = y + a @ SV.float().T
    if bias is not None:
        y = y + bias.float()
    return y.half()


def linear_forward_fp64(x, q, scales, zeros, groupsize, sym=False, U=None, SV=None,
                        precomputed_xU=None, bias=None, exact_weights=False) -> torch.Tensor:
    """Reference-of-reference: fp64 sum of the dequantized weights times x, plus
    (x U) SV^T (or precomputed_xU SV^T) + bias.  Weights are the fp16-rounded
    ones of dequant_fp16, or with exact_weights the exact s*(q - z) (what
    dequant_fp32 computes: an 11-bit scale times a small integer is exact in
    fp32)."""
    xd = x.double()
    if exact_weights:
        W = dequant_fp32(q, scales, zeros, groupsize, sym).double()
    else:
        W = dequant_fp16(q, scales, zeros, groupsize, sym).double()
    y = xd @ W.T
    if SV is not None:
        a = precomputed_xU.double() if precomputed_xU is not None else xd @ U.double()
        y = y + a @ SV.double().T
    if bias is not None:
        y = y + bias.double()
    return y


def fp64_matvec_bruteforce(x: np.ndarray, W: np.ndarray) -> np.ndarray:
    """Explicit double loop y[m, n] = sum_k x[m,k] W[n,k] (pure Python; tiny
    inputs only) — pins the torch matmul orientation used above."""
    M, K = x.shape
    N = W.shape[0]
    y = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += float(x[m, k]) * float(W[n, k])
            y[m, n] = s
    return y


def parity_ok(y: torch.Tensor, ref: torch.Tensor, rtol: float = 1e-2, atol: float = 1e-3) -> bool:
    """The north star's output bar: |y - ref| <= atol + rtol*|ref| elementwise."""
    y = y.double().cpu()
    ref = ref.double().cpu()
    return bool(((y - ref).abs() <= atol + rtol * ref.abs()).all())


# ---------------------------------------------------------------------------
# MoE block (GraphCompatibleMoeBlock.forward, inference/moe_block.py:381-436,
# with the sparse dispatch of _forward_sparse :704-740 / the HF-style
# GLoRCQExperts.forward, inference/quantized_linear.py:395-428)
# ---------------------------------------------------------------------------
def route(h: torch.Tensor, router_w: torch.Tensor, top_k: int, norm_topk_prob: bool,
          exact: bool = False):
    """Router (moe_block.py:386-392): logits = gate(h) in fp16, softmax in fp32,
    torch.topk, optional renormalisation, cast to fp16.
    exact=True rounds the fp64 sum of each logit to fp16 once (what the
    reference's fp16 nn.Linear does on the GPU: fp32 accumulation, one
    rounding); exact=False uses torch's CPU fp16 matmul, whose blocked kernel
    (from about 16 rows up) can land a few fp16 ulps away from that.
    Returns (fp16 logits (B,E), fp16 weights (B,k), int64 experts (B,k))."""
    if exact:
        logits = (h.double() @ router_w.double().T).half()
    else:
        logits = h.half() @ router_w.half().T
    rw = torch.softmax(logits.float(), dim=1)
    w, sel = torch.topk(rw, top_k, dim=-1)
    if norm_topk_prob:
        w = w / w.sum(dim=-1, keepdim=True)
    return logits, w.half(), sel


def turbo_rotate(x: torch.Tensor, q, exact: bool) -> torch.Tensor:
    """x_rot of a format.TurboMat's configuration, rounded to fp16 as the
    reference's rotation cache does: fp16(rht_forward(x.float(), signs))
    (inference/moe_block.py:349-351) or fp16(x.float() @ Pi.float().T) (:352-356).
    exact=True takes both in fp64 before the rounding (the package and torch
    compute them in fp32)."""
    if q.signs is not None:
        return rht_forward(x.float(), q.signs).half()
    if exact:
        return (x.double() @ q.Pi.double().T).half()
    return rotate_qr(x, q.Pi)


def _turbo_linear(x, q, e, exact, U=None, SV=None, a=None):
    """TurboQuant expert e of a format.TurboMat as the MoE block calls it
    (GLoRCQLinear's turbo forward with a precomputed x_rot, inference/
    quantized_linear.py:315-349; moe_block.py:480-702): x_rot = turbo_rotate(x);
    y = norm * C[q] x_rot (+ a @ SV_e^T, a = fp16(x @ U) of the unrotated x
    unless given).  exact=True: fp64 sums; else the reference's fp32 fallback
    rounded to fp16 and fp16 low-rank matmuls."""
    xr = turbo_rotate(x, q, exact)
    packed = q.packed[e].numpy()
    if exact:
        y = turbo_matmul_fp64(xr, packed, q.norms[e], q.centroids)
        if SV is not None:
            if a is None:
                a = (x.double() @ U.double()).half()
            y = y + a.double() @ SV.double().T
        return y
    y = turbo_matmul_fp32(xr, packed, q.norms[e], q.centroids).half()
    if SV is not None:
        if a is None:
            a = x.half() @ U.half()
        y = y + a.half() @ SV.half().T
    return y


def _qmat_linear(x, q, e, exact, U=None, SV=None, a=None, memo=None):
    """y = x @ W_e^T (+ a @ SV_e^T, a = fp16(x @ U) unless given) for expert e of
    a format.QMat (a format.TurboMat goes to _turbo_linear).  exact=False: the reference's fp16 CPU fallback (fp16 dequant,
    fp16 matmuls, quantized_linear.py:286-355); exact=True: fp64 sums of the
    exact weights s*(q - z), with a rounded to fp16 as the reference does.
    memo (exact only): a dict that keeps each expert's exact weights across
    calls, for callers whose weights do not change (multi-step decoding)."""
    if hasattr(q, "centroids"):
        return _turbo_linear(x, q, e, exact, U=U, SV=SV, a=a)
    if exact and memo is not None and (id(q), e) in memo:
        W = memo[(id(q), e)].double()
    elif exact:
        qi = torch.from_numpy(unpack_codes(q.codes[e].numpy(), q.bits, q.K))
        W32 = dequant_fp32(qi, q.scales[e], q.zeros[e], q.group)  # exact in fp32
        if memo is not None:
            memo[(id(q), e)] = W32
        W = W32.double()
    if exact:
        y = x.double() @ W.T
        if SV is not None:
            if a is None:
                a = (x.double() @ U.double()).half()
            y = y + a.double() @ SV.double().T
        return y
    qi = torch.from_numpy(unpack_codes(q.codes[e].numpy(), q.bits, q.K))
    W = dequant_fp16(qi, q.scales[e], q.zeros[e], q.group)
    y = x.half() @ W.T
    if SV is not None:
        if a is None:
            a = x.half() @ U.half()
        y = y + a.half() @ SV.half().T
    return y


def moe_forward(p, exact: bool = True, h: torch.Tensor | None = None, dense: bool = False,
                cluster_shared: bool = True, memo: dict | None = None):
    """MoE block output (B, H) for format.MoEProblem p.

    Rounding points kept from the reference in both modes: routing weights,
    the cluster-shared a = fp16(h @ U_c) (_precompute_xU_for_experts,
    moe_block.py:290-322), inter = fp16(silu(gate) * up) (act_fn on fp16,
    :465-468), the down projection's own a = fp16(inter @ U_down), the shared
    gate fp16(sigmoid(h @ w_sg)) (:429-433).  exact=True sums in fp64;
    exact=False reproduces the reference's fp16 CPU arithmetic, including the
    fp16 index_add accumulation in expert order.
    dense=True evaluates every expert with weight 0 for the unselected ones (the
    graph-mode identity the reference relies on, moe_block.py:11-13).
    cluster_shared=False computes x @ U per expert instead of per cluster
    (test_cluster_parallel.py:159 asserts the two agree).
    memo: see _qmat_linear (routed experts, exact mode)."""
    h = p.h if h is None else h
    B, H = h.shape
    _, w, sel = route(h, p.router_w, p.top_k, p.norm_topk_prob, exact=exact)
    acc_dtype = torch.float64 if exact else torch.float16
    final = torch.zeros(B, H, dtype=acc_dtype)
    xu = {}
    for proj in ("gate", "up"):
        for c in range(p.n_clusters):
            xu[(proj, c)] = (h.double() @ p.U[proj][c].double()).half() if exact \
                else h.half() @ p.U[proj][c].half()
    experts = range(p.E) if dense else sorted(set(sel.flatten().tolist()))
    for e in experts:
        tok_pos = [(t, k) for t in range(B) for k in range(p.top_k) if int(sel[t, k]) == e]
        toks = [t for t, _ in tok_pos] if tok_pos else []
        if dense:
            toks = list(range(B))
        if not toks:
            continue
        x = h[toks]
        outs = {}
        for proj in ("gate", "up"):
            c = int(p.cluster_of[proj][e])
            a = xu[(proj, c)][toks] if cluster_shared else None
            outs[proj] = _qmat_linear(x, p.experts[proj], e, exact, U=p.U[proj][c],
                                      SV=p.SV[proj][e], a=a, memo=memo)
        g, u = outs["gate"], outs["up"]
        if exact:
            inter = (torch.nn.functional.silu(g.half().float()).half().double() *
                     u.half().double()).half()
        else:
            inter = torch.nn.functional.silu(g.half()) * u.half()
        cd = int(p.cluster_of["down"][e])
        y = _qmat_linear(inter, p.experts["down"], e, exact, U=p.U["down"][cd],
                         SV=p.SV["down"][e], memo=memo)
        wt = torch.zeros(len(toks), dtype=torch.float16)
        for i, t in enumerate(toks):
            for k in range(p.top_k):
                if int(sel[t, k]) == e:
                    wt[i] = w[t, k]
        if exact:
            final.index_add_(0, torch.tensor(toks), y * wt.double()[:, None])
        else:
            final.index_add_(0, torch.tensor(toks), (y.half() * wt[:, None]).half())
    if p.shared is None:  # a block without a shared expert (Mixtral-style)
        return final
    # shared expert (4-bit, no LoRA) with the sigmoid gate
    if exact:
        sgl = (h.double() @ p.shared_gate_w.double().T).half()
    else:
        sgl = h.half() @ p.shared_gate_w.half().T
    sg = torch.sigmoid(sgl.float()).half()
    sgu = {proj: _qmat_linear(h, p.shared[proj], 0, exact) for proj in ("gate", "up")}
    if exact:
        sinter = (torch.nn.functional.silu(sgu["gate"].half().float()).half().double() *
                  sgu["up"].half().double()).half()
        sd = _qmat_linear(sinter, p.shared["down"], 0, exact)
        return final + sd.half().double() * sg.double()
    sinter = torch.nn.functional.silu(sgu["gate"].half()) * sgu["up"].half()
    sd = _qmat_linear(sinter, p.shared["down"], 0, exact).half()
    return final + (sg * sd).half()


# ---------------------------------------------------------------------------
# TurboQuant codec (the reference's 2-bit expert format): codebook GEMV and
# the input rotations
# ---------------------------------------------------------------------------
def unpack_indices_2bit(packed: np.ndarray, K: int) -> np.ndarray:
    """(N, K/4) uint8 -> (N, K) int64 codebook indices, value j of a byte at
    bits [2j, 2j+2) (_unpack_indices_2bit, inference/kernels/__init__.py:
    113-118).  Pinned by: brute force over every value in every slot, and
    equality with unpack_codes of the same bytes read as little-endian int32
    words (tests/test_turbo_oracle.py)."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 4), dtype=np.int64)
    for j in range(4):
        out[:, j::4] = (p >> (2 * j)) & 3
    return out[:, :K]


def turbo_matmul_fp32(x_rot: torch.Tensor, packed: np.ndarray, norms: torch.Tensor,
                      centroids: torch.Tensor) -> torch.Tensor:
    """The reference's pure-PyTorch path (_pytorch_fallback, inference/
    kernels/__init__.py:121-146, and reference_turbo_matmul of
    inference/kernels/test_kernels.py:24-41): W = C[idx] * norm[:, None] in
    fp32, y = x_rot.float() @ W.T in fp32 (the kernels round y to fp16).
    Pinned by: brute-force loops on tiny inputs, the closed form y = norm *
    C[c] * sum(x) for constant codes, and equality with the GPTQ oracle when
    C = (0, 1, 2, 3), norm = 1 (tests/test_turbo_oracle.py)."""
    K = x_rot.shape[1]
    idx = torch.from_numpy(unpack_indices_2bit(packed, K))
    W = centroids.float()[idx] * norms.float()[:, None]
    return x_rot.float() @ W.T


def turbo_matmul_fp64(x_rot: torch.Tensor, packed: np.ndarray, norms: torch.Tensor,
                      centroids: torch.Tensor) -> torch.Tensor:
    """y = norm[n] * sum_k C[q(n,k)] x_rot[m,k] with fp64 sums of the exact fp32
    codebook/norm values (the bar's reference; the CUDA kernel,
    turbo_matmul.cu:80-137, accumulates in fp32 and multiplies by the norm
    last).  Pinned as turbo_matmul_fp32."""
    K = x_rot.shape[1]
    idx = torch.from_numpy(unpack_indices_2bit(packed, K))
    S = x_rot.double() @ centroids.double()[idx].T
    return S * norms.double()[None, :]


def turbo_bruteforce(x_rot: np.ndarray, packed: np.ndarray, norms: np.ndarray,
                     centroids: np.ndarray) -> np.ndarray:
    """Pure-Python loops over bytes and bit slots (tiny inputs only):
    y[m, n] = norms[n] * sum_k centroids[(byte(n, k/4) >> 2(k%4)) & 3] x[m, k]."""
    M, K = x_rot.shape
    N = packed.shape[0]
    y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                q = (int(packed[n, k // 4]) >> (2 * (k % 4))) & 3
                s += float(centroids[q]) * float(x_rot[m, k])
            y[m, n] = float(norms[n]) * s
    return y


def hadamard_sylvester(d: int) -> np.ndarray:
    """H_d by the Sylvester recursion H_2n = [[H, H], [H, -H]] (the ordering
    fast-hadamard-transform applies); equals scipy.linalg.hadamard(d)."""
    H = np.ones((1, 1))
    while H.shape[0] < d:
        H = np.block([[H, H], [H, -H]])
    return H


def rht_forward(x: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """y = (1/sqrt(d)) H diag(signs) x in fp64 (hadamard_rotation.py:52-67;
    the external package computes it in fp32).  Pinned by: scipy.linalg.
    hadamard, norm preservation, rht_backward(rht_forward(x)) == x, and H e_0
    = all-ones (tests/test_turbo_oracle.py)."""
    d = x.shape[-1]
    H = torch.from_numpy(hadamard_sylvester(d))
    return (x.double() * signs.double()) @ H.T / np.sqrt(d)


def rht_backward(y: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """x = diag(signs) (1/sqrt(d)) H y in fp64 (hadamard_rotation.py:70-86)."""
    d = y.shape[-1]
    H = torch.from_numpy(hadamard_sylvester(d))
    return (y.double() @ H.T / np.sqrt(d)) * signs.double()


def generate_rht_signs(d: int, seed: int = 42) -> torch.Tensor:
    """(d,) fp32 of +-1 from torch's CPU generator (hadamard_rotation.py:32-49):
    randint(0, 2) * 2 - 1 under manual_seed(seed)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return (torch.randint(0, 2, (d,), generator=g) * 2 - 1).float()


def rotate_qr(x: torch.Tensor, Pi: torch.Tensor) -> torch.Tensor:
    """x_rot = fp16(x.float() @ Pi.float().T) (turbo_dequant_matmul_fused,
    inference/kernels/__init__.py:209-212)."""
    return (x.float() @ Pi.float().T).half()


# ---------------------------------------------------------------------------
# LoRA factor storage (load time): intN per-column / per-row absmax codes,
# int4 row-pair nibble packing
# ---------------------------------------------------------------------------
def quant_intN_absmax(t: torch.Tensor, nbits: int, rowwise: bool = False):
    """Symmetric absmax quantization to [-maxval, maxval], maxval =
    2^(nbits-1) - 1, stored as int8, scale fp16 per column (cols,) or per row
    (rows, 1) (cross_layer_share.py:584-595 and :604-614).  Test-data
    generator; pinned by the round-trip bound |dequant(q) - t| <= scale /
    (2 maxval) + fp16 rounding (tests/test_factor_oracle.py)."""
    maxval = 2 ** (nbits - 1) - 1
    if rowwise:
        scale = t.float().abs().max(dim=1, keepdim=True).values.clamp(min=1e-8)
    else:
        scale = t.float().abs().max(dim=0).values.clamp(min=1e-8)
    q = (t.float() / scale * maxval).round().clamp(-maxval, maxval).to(torch.int8)
    return q, scale.half()


def dequant_intN(q: torch.Tensor, scale: torch.Tensor, nbits: int) -> torch.Tensor:
    """fp16(q.float() / maxval * scale.float()) in fp32 (_dequant_intN,
    inference/model_builder.py:69-72, then the callers' .half(), :46-50,
    :510-527).  Pinned by: q = +-maxval gives +-scale exactly, q = 0 gives 0,
    and an explicit per-element loop for both scale layouts."""
    maxval = 2 ** (nbits - 1) - 1
    return (q.float() / maxval * scale.float()).half()


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """(rows, cols) int8 in [-7, 7] -> ((rows+1)//2, cols) uint8: row 2i in the
    low nibble, row 2i+1 in the high nibble, each as value + 7
    (cross_layer_share.py:619-634).  Pinned by unpack_int4 brute force."""
    rows, cols = q.shape
    u = (q.to(torch.int16) + 7).to(torch.uint8)
    if rows % 2:
        u = torch.cat([u, torch.zeros(1, cols, dtype=torch.uint8)], dim=0)
    return (u[0::2] | (u[1::2] << 4)).to(torch.uint8)


def unpack_int4(packed: torch.Tensor, orig_rows: int) -> torch.Tensor:
    """Inverse of pack_int4 (_unpack_int4, inference/model_builder.py:75-80):
    element (r, c) = ((byte(r//2, c) >> 4*(r%2)) & 15) - 7.  Pinned by every
    nibble value in both positions and pack/unpack round trips over odd and
    even row counts."""
    rows = orig_rows
    out = torch.empty(rows, packed.shape[1], dtype=torch.int8)
    p = packed.to(torch.int16)
    for r in range(rows):
        out[r] = ((p[r // 2] >> (4 * (r % 2))) & 15) - 7
    return out
