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
