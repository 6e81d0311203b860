"""torch.library operators over the HIP library (namespace `glorcq_hip`).

The reference registers its CUDA kernels as custom ops with fake (meta)
kernels so Dynamo can trace them (inference/kernels/__init__.py:63-107:
`glorcq::turbo_dequant_matmul`, `glorcq::gptq_dequant_matmul`).  This module
does the same for the gfx950 library, in its own namespace so it never
collides with the reference's:

  glorcq_hip::packed_dequant_matmul  fused dequant-GEMV/GEMM + low-rank + bias
                                     (GLoRCQLinear.forward's GPTQ path)
  glorcq_hip::turbo_dequant_matmul   TurboQuant codebook matmul + low-rank + bias
  glorcq_hip::lowrank_xu             a = fp16(x U)
  glorcq_hip::rht                    randomized Hadamard transform
  glorcq_hip::moe_decode             one MoE block step (<= 64 tokens)
  glorcq_hip::moe_prefill            one MoE block over many tokens

Each real kernel calls the C ABI on torch's current stream (inputs on any
other device raise RuntimeError: there is no CPU path); each fake kernel
returns an empty tensor of the output's shape and dtype after the same shape
checks, so torch.compile(fullgraph=True) traces a GLoRCQ layer or MoE block
into one graph without running it.  The ops allocate their outputs through
torch's caching allocator (the reference's ops do the same).
"""

from __future__ import annotations

from typing import List, Optional

import torch
from torch import Tensor

from . import kernels as _k

_NS = "glorcq_hip"


def _fail(msg: str):
    raise RuntimeError(msg)


# ---------------------------------------------------------------------------
# packed_dequant_matmul
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::packed_dequant_matmul", mutates_args=())
def packed_dequant_matmul(x: Tensor, codes: Tensor, scales: Tensor, zeros: Optional[Tensor],
                          bits: int, groupsize: int, sym: int, U: Optional[Tensor],
                          SV: Optional[Tensor], precomputed_xU: Optional[Tensor],
                          bias: Optional[Tensor]) -> Tensor:
    return _k._packed_dequant_matmul_eager(x, codes, scales, zeros, bits, groupsize, sym, U, SV,
                                           precomputed_xU, bias)


@packed_dequant_matmul.register_fake
def _(x, codes, scales, zeros, bits, groupsize, sym, U, SV, precomputed_xU, bias):
    if x.dim() != 2 or codes.dim() != 2:
        _fail("x must be (M, K) and codes (N, K*bits/32)")
    if bits not in (2, 4) or codes.shape[1] * (32 // bits) != x.shape[1]:
        _fail(f"codes shape {tuple(codes.shape)} does not match K={x.shape[1]} at {bits} bits")
    if x.dtype != torch.float16 or codes.dtype != torch.int32:
        _fail("x must be fp16 and codes int32")
    return x.new_empty((x.shape[0], codes.shape[0]), dtype=torch.float16)


# ---------------------------------------------------------------------------
# turbo_dequant_matmul
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::turbo_dequant_matmul", mutates_args=())
def turbo_dequant_matmul(x_rot: Tensor, packed_indices: Tensor, norms: Tensor,
                         centroids: Tensor, xU: Optional[Tensor], SV: Optional[Tensor],
                         bias: Optional[Tensor]) -> Tensor:
    return _k._turbo_gemv_eager(x_rot, packed_indices, norms, centroids, xU, SV, bias)


@turbo_dequant_matmul.register_fake
def _(x_rot, packed_indices, norms, centroids, xU, SV, bias):
    if x_rot.dim() not in (2, 3) or x_rot.dtype != torch.float16:
        _fail("x_rot must be fp16 (M, K) or (E, M, K)")
    N = packed_indices.shape[-2]
    return x_rot.new_empty((*x_rot.shape[:-1], N), dtype=torch.float16)


# ---------------------------------------------------------------------------
# lowrank_xu
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::lowrank_xu", mutates_args=())
def lowrank_xu(x: Tensor, U: Tensor) -> Tensor:
    return _k._lowrank_xu_eager(x, U)


@lowrank_xu.register_fake
def _(x, U):
    if x.shape[-1] != U.shape[-2]:
        _fail(f"x has K={x.shape[-1]}, U has K={U.shape[-2]}")
    r = U.shape[-1]
    if U.dim() == 3:
        M = x.shape[-2]
        return x.new_empty((U.shape[0], M, r), dtype=torch.float16)
    return x.new_empty((x.shape[0], r), dtype=torch.float16)


# ---------------------------------------------------------------------------
# rht
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::rht", mutates_args=())
def rht(x: Tensor, signs: Tensor, inverse: bool, out_fp32: bool) -> Tensor:
    return _k._rht_eager(x, signs, inverse, torch.float32 if out_fp32 else torch.float16)


@rht.register_fake
def _(x, signs, inverse, out_fp32):
    if signs.numel() != x.shape[-1]:
        _fail(f"signs has {signs.numel()} entries, rows have {x.shape[-1]}")
    return x.new_empty(x.shape, dtype=torch.float32 if out_fp32 else torch.float16)


# ---------------------------------------------------------------------------
# MoE block: decode step and prefill
# ---------------------------------------------------------------------------
# The decode step's workspace (routing tables, partial sums, the router's
# arrival counter) is kept by the real kernel per (device, stream, tokens):
# steps on one stream run in order and each leaves the counter zero, so the
# operator has no mutable argument.
@torch.library.custom_op(f"{_NS}::moe_decode", mutates_args=())
def moe_decode(h: Tensor, router_w: Tensor, shared_gate_w: Optional[Tensor],
               codes: List[Tensor], scales: List[Tensor], zeros: List[Tensor],
               U: List[Tensor], cluster_of: List[Tensor], SV: List[Tensor],
               u_slot: List[Optional[Tensor]], u_rows: List[int],
               shared_codes: List[Tensor], shared_scales: List[Tensor],
               shared_zeros: List[Tensor], residual: Optional[Tensor],
               inter: int, top_k: int, norm_topk_prob: bool, rank: int, n_clusters: int,
               bits: int, shared_bits: int, shared_inter: int) -> List[Tensor]:
    from .moe_block import moe_decode_launch
    return list(moe_decode_launch(h, router_w, shared_gate_w, codes, scales, zeros, U,
                                  cluster_of, SV, u_slot, u_rows, shared_codes, shared_scales,
                                  shared_zeros, residual, inter, top_k, norm_topk_prob, rank,
                                  n_clusters, bits, shared_bits, shared_inter))


@moe_decode.register_fake
def _(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV, u_slot, u_rows,
      shared_codes, shared_scales, shared_zeros, residual, inter, top_k,
      norm_topk_prob, rank, n_clusters, bits, shared_bits, shared_inter):
    if h.dim() != 2 or h.shape[1] != router_w.shape[1]:
        _fail("h must be (tokens, hidden) with hidden = router_w's columns")
    if h.shape[0] > 64:
        _fail("moe_decode takes at most 64 tokens")
    return [torch.empty_like(h), h.new_empty((h.shape[0], router_w.shape[0]))]


@torch.library.custom_op(f"{_NS}::moe_prefill", mutates_args=())
def moe_prefill(h: Tensor, router_w: Tensor, shared_gate_w: Optional[Tensor],
                codes: List[Tensor], scales: List[Tensor], zeros: List[Tensor],
                U: List[Tensor], cluster_of: List[Tensor], SV: List[Tensor],
                u_slot: List[Optional[Tensor]], u_rows: List[int], shared_codes: List[Tensor],
                shared_scales: List[Tensor], shared_zeros: List[Tensor],
                residual: Optional[Tensor], inter: int, top_k: int, norm_topk_prob: bool,
                rank: int, n_clusters: int, bits: int, shared_bits: int,
                shared_inter: int, zeros_integral: bool) -> List[Tensor]:
    from .moe_block import moe_prefill_launch
    return list(moe_prefill_launch(h, router_w, shared_gate_w, codes, scales, zeros, U,
                                   cluster_of, SV, u_slot, u_rows, shared_codes, shared_scales,
                                   shared_zeros, residual, inter, top_k, norm_topk_prob, rank,
                                   n_clusters, bits, shared_bits, shared_inter, zeros_integral))


@moe_prefill.register_fake
def _(h, router_w, shared_gate_w, codes, scales, zeros, U, cluster_of, SV, u_slot, u_rows,
      shared_codes, shared_scales, shared_zeros, residual, inter, top_k, norm_topk_prob, rank,
      n_clusters, bits, shared_bits, shared_inter, zeros_integral):
    if h.dim() != 2 or h.shape[1] != router_w.shape[1]:
        _fail("h must be (tokens, hidden) with hidden = router_w's columns")
    return [torch.empty_like(h), h.new_empty((h.shape[0], router_w.shape[0]))]
