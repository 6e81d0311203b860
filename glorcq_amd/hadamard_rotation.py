"""Randomized Hadamard transform (RHT) for TurboQuant inputs, on the GPU.

Mirrors the reference's hadamard_rotation.py (same names and meaning):

  is_hadamard_available()          :25-27
  generate_rht_signs(d, seed, dev) :32-49   (same torch CPU draw, so the
                                             signs match the quantizer's)
  rht_forward(x, signs)            :52-67   y = (1/sqrt(d)) H diag(signs) x
  rht_backward(y, signs)           :70-86   x = diag(signs) (1/sqrt(d)) H y

The reference needs the external fast-hadamard-transform package for H; here
the transform is the library's own kernel (glq_rht), fp32 arithmetic, fp16 or
fp32 in and out (the output keeps the input dtype, as the package does).
"""

from __future__ import annotations

import torch

from . import kernels


def is_hadamard_available() -> bool:
    """True when the RHT kernel can run (library built, GPU visible)."""
    return kernels.is_cuda_available()


def generate_rht_signs(d: int, seed: int = 42, device="cuda") -> torch.Tensor:
    """(d,) fp32 of +-1: torch.randint(0, 2) * 2 - 1 from a CPU generator under
    manual_seed(seed), then moved to `device`."""
    rng = torch.Generator(device="cpu")
    rng.manual_seed(seed)
    signs = torch.randint(0, 2, (d,), generator=rng) * 2 - 1
    return signs.float().to(device)


def rht_forward(x: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """y = (1/sqrt(d)) H diag(signs) x over the last dimension (a power of two)."""
    return kernels.rht(x.contiguous(), signs.float().contiguous())


def rht_backward(y: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """x = diag(signs) (1/sqrt(d)) H y, the inverse of rht_forward."""
    return kernels.rht(y.contiguous(), signs.float().contiguous(), inverse=True)


def rht_rotate_half(x: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """The hot-path rotation rht_forward(x.float(), signs).half()
    (inference/moe_block.py:351,525,649,840) for fp16 x, in one launch."""
    return kernels.rht(x.to(torch.float16).contiguous(), signs.float().contiguous(),
                       out_dtype=torch.float16)
