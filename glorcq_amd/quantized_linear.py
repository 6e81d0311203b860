"""GLoRCQLinear on the MI355X kernels.

Mirrors the reference's quantized linear layer (inference/quantized_linear.py:
152-362) — same class name, loaders, attributes and forward signature — so
host code that builds and calls it keeps its call sites.  Differences:

* `load_gptq` packs the (N, K) integer codes into the int32 container once, on
  the device (the reference keeps them unpacked and casts them to int8 on
  every call, inference/kernels/__init__.py:305-309).  Widths 2 and 4 use
  their own container; 3-bit codes use the 4-bit container.
* `forward` is one fused call: dequant-GEMV (M <= 16, or per 16-row block),
  a = x U (or the caller's precomputed_xU), y += a SV^T, + bias.  No silent
  CPU fallback: a missing HIP library raises.
* TurboQuant layers (`load_turbo`, 2-bit) run the codebook kernel
  (glq_turbo_gemv_batched) with the low-rank term and bias fused into its
  epilogue.  The input rotation is the layer's RHT when `_rht_signs` is set
  (the model builder's hadamard mode, inference/model_builder.py:278-286),
  else x Pi^T with Pi from the rotation cache, unless precomputed_x_rot is
  given.  Widths other than 2 raise (the reference runs them in pure PyTorch,
  inference/quantized_linear.py:331-334).  `load_turbo_predequant` needs the
  external TurboQuant quantizer and is not provided.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import kernels
from .format import pack_codes
from .hadamard_rotation import rht_rotate_half

SUPPORTED_BITS = (2, 3, 4)


def container_bits(bits: int) -> int:
    """Packed container width for b-bit codes."""
    if bits not in SUPPORTED_BITS:
        raise RuntimeError(f"{bits}-bit GPTQ codes are not supported (2, 3 or 4)")
    return 2 if bits == 2 else 4


class RotationCache:
    """TurboQuant rotations and codebooks per (dim, bits, seed), shared by all
    layers of that configuration (reference RotationCache, inference/
    model_builder.py:86-137).  The reference generates them with the external
    turboquant package (TurboQuantMSE), which is not available here: `put`
    supplies them, and `register` of a key never put raises."""

    def __init__(self, device="cuda"):
        self._device = device
        self._pi = {}          # (dim, bits, seed) -> Pi (dim, dim) fp16
        self._centroids = {}   # (dim, bits, seed) -> centroids (2^bits,) fp32

    def put(self, dim, bits, seed, Pi, centroids):
        key = (dim, bits, seed)
        self._pi[key] = None if Pi is None else Pi.to(self._device, torch.float16).contiguous()
        self._centroids[key] = centroids.to(self._device, torch.float32).contiguous()

    def register(self, dim, bits, seed=42):
        if (dim, bits, seed) not in self._centroids:
            raise RuntimeError(
                f"no rotation/codebook for dim={dim} bits={bits} seed={seed}: the turboquant "
                f"package that generates them is not available; supply them with put()")

    def get_pi(self, dim, bits, seed=42):
        return self._pi[(dim, bits, seed)]

    def get_centroids(self, dim, bits, seed=42):
        return self._centroids[(dim, bits, seed)]


class GLoRCQLinear(nn.Module):
    """Quantized linear layer: y = dequant(W_q) x + (x U) SV^T + bias.

    Reference: inference/quantized_linear.py:152-362 (GLoRCQLinear).
    """

    def __init__(self, in_features, out_features, bias=False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.quant_type = None       # "gptq" or "turbo"
        # GPTQ state (packed)
        self.codes = None            # (out, in*b/32) int32, LSB-first
        self.scales = None           # (out, n_groups) fp16
        self.zeros = None            # (out, n_groups) fp16
        self.gptq_bits = None        # code width of the checkpoint
        self.pack_bits = None        # container width (2 or 4)
        self.gptq_groupsize = None
        self.gptq_sym = False
        # TurboQuant state
        self.packed_indices = None   # (out, in/4) uint8, 4 indices per byte LSB-first
        self.turbo_words = None      # the same bytes as (out, in/16) int32 words
        self.norms = None            # (out,) fp32 per-row norms
        self.turbo_bits = None
        self.turbo_dim = None
        self.turbo_seed = 42
        self._rotation_cache = None  # RotationCache (Pi and centroids)
        self._rht_signs = None       # (in,) fp32 +-1: RHT rotation instead of Pi
        # LoRA compensation
        self.U = None                # (in, rank) fp16, shared across a cluster
        self.SV = None               # (out, rank) fp16, S fused into V
        self.cluster_id = None       # set by the model builder for cluster-shared x*U
        self.bias_param = None       # (out,) fp16

    # ---- loaders (reference :195-269) ----
    def load_gptq(self, packed_data, device="cuda"):
        """Loads the reference's `gptq_packed` dict (joint_optim.py:320-327):
        qweight_int (out, in) int codes, scales/zeros (out, G) fp16, bits,
        groupsize, sym; packs the codes on the device."""
        self.quant_type = "gptq"
        self.gptq_bits = int(packed_data["bits"])
        self.pack_bits = container_bits(self.gptq_bits)
        self.gptq_groupsize = int(packed_data["groupsize"])
        self.gptq_sym = bool(packed_data.get("sym", False))
        q = torch.as_tensor(packed_data["qweight_int"]).to(torch.int32)
        if q.shape != (self.out_features, self.in_features):
            raise RuntimeError(f"qweight_int shape {tuple(q.shape)} != "
                               f"({self.out_features}, {self.in_features})")
        q = q.to(device)
        if q.is_cuda:
            self.codes = kernels.pack_codes_device(q.contiguous(), self.pack_bits)
        else:
            self.codes = pack_codes(q, self.pack_bits)
        self.scales = packed_data["scales"].to(device=device, dtype=torch.float16).contiguous()
        z = packed_data.get("zeros")
        self.zeros = None if z is None else z.to(device=device,
                                                 dtype=torch.float16).contiguous()

    def load_turbo(self, compressed_data, rotation_cache, device="cuda"):
        """Loads the reference's `turbo_compressed` dict (packed_indices (out,
        in/4) uint8, norms (out,), bits, dim, seed; reference :205-227).  The
        indices stay packed; the kernel reads them as int32 words."""
        self.quant_type = "turbo"
        self.turbo_bits = int(compressed_data["bits"])
        self.turbo_dim = int(compressed_data["dim"])
        self.turbo_seed = int(compressed_data.get("seed", 42))
        if self.turbo_bits != 2:
            raise RuntimeError(f"{self.turbo_bits}-bit TurboQuant layers are not supported "
                               f"(the codebook kernel takes 2-bit indices)")
        if self.turbo_dim != self.in_features:
            raise RuntimeError(f"turbo dim {self.turbo_dim} != in_features {self.in_features}")
        packed = torch.as_tensor(compressed_data["packed_indices"]).to(device=device,
                                                                       dtype=torch.uint8)
        if packed.shape != (self.out_features, self.in_features // 4):
            raise RuntimeError(f"packed_indices shape {tuple(packed.shape)} != "
                               f"({self.out_features}, {self.in_features // 4})")
        self.packed_indices = packed.contiguous()
        self.turbo_words = self.packed_indices.view(torch.int32)
        self.norms = torch.as_tensor(compressed_data["norms"]).to(
            device=device, dtype=torch.float32).contiguous()
        self._rotation_cache = rotation_cache
        rotation_cache.register(self.turbo_dim, self.turbo_bits, self.turbo_seed)

    def load_lora(self, U, S, V, device="cuda"):
        """SV = V * S[None, :] fused at load time (reference :249-259)."""
        if U is not None:
            self.U = U.to(device=device, dtype=torch.float16).contiguous()
            self.SV = (V.float() * S.float().unsqueeze(0)).to(device=device,
                                                              dtype=torch.float16).contiguous()

    def load_sv(self, U, SV, device="cuda"):
        """Pre-fused SV (reference :261-269)."""
        if U is not None:
            self.U = U.to(device=device, dtype=torch.float16).contiguous()
            self.SV = SV.to(device=device, dtype=torch.float16).contiguous()

    def set_bias(self, bias, device="cuda"):
        self.bias_param = None if bias is None else bias.to(device=device,
                                                            dtype=torch.float16).contiguous()

    # ---- dequant (reference :271-284) ----
    def _dequant_gptq(self):
        """fp16 W (out, in), bit-exact with the reference's fp16 dequant loop."""
        return kernels.dequant_weight(self.codes, self.pack_bits, self.in_features, self.scales,
                                      None if self.gptq_sym else self.zeros,
                                      self.gptq_groupsize, self.gptq_sym)

    @property
    def rank(self):
        return 0 if self.SV is None else self.SV.shape[1]

    # ---- forward (reference :286-355) ----
    def _forward_turbo(self, x2, xu, precomputed_x_rot):
        """y = fp16(norm * C[q] x_rot + a SV^T + bias) (reference :315-349)."""
        key = (self.turbo_dim, self.turbo_bits, self.turbo_seed)
        cache = self._rotation_cache
        centroids = cache.get_centroids(*key)
        if precomputed_x_rot is not None:
            x_rot = precomputed_x_rot.reshape(-1, self.in_features).to(torch.float16).contiguous()
        elif self._rht_signs is not None:
            x_rot = rht_rotate_half(x2, self._rht_signs)
        else:
            Pi = cache.get_pi(*key)
            x_rot = (x2.float() @ Pi.float().T).half()
        if self.SV is not None and xu is None:
            xu = kernels.lowrank_xu(x2, self.U)
        return kernels.turbo_gemv(x_rot, self.turbo_words, self.norms, centroids,
                                  xU=xu if self.SV is not None else None, SV=self.SV,
                                  bias=self.bias_param)

    def forward(self, x, precomputed_xU=None, precomputed_x_rot=None):
        if self.quant_type not in ("gptq", "turbo"):
            raise RuntimeError(f"Unknown quant_type: {self.quant_type}")
        if precomputed_x_rot is not None and self.quant_type != "turbo":
            raise RuntimeError("precomputed_x_rot applies to TurboQuant layers only")
        orig_shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.float16:
            x2 = x2.half()
        x2 = x2.contiguous()
        xu = None
        if self.SV is not None and precomputed_xU is not None:
            xu = precomputed_xU.reshape(-1, self.rank).to(torch.float16).contiguous()
        if self.quant_type == "turbo":
            y = self._forward_turbo(x2, xu, precomputed_x_rot)
            return y.reshape(*orig_shape[:-1], self.out_features)
        y = kernels.packed_dequant_matmul_fused(
            x2, self.codes, self.scales, None if self.gptq_sym else self.zeros, self.pack_bits,
            self.gptq_groupsize, sym=self.gptq_sym,
            U=self.U if xu is None else None, SV=self.SV, precomputed_xU=xu,
            bias=self.bias_param)
        return y.reshape(*orig_shape[:-1], self.out_features)

    def extra_repr(self):
        s = f"in_features={self.in_features}, out_features={self.out_features}"
        s += f", quant_type={self.quant_type}"
        if self.quant_type == "turbo":
            s += f", turbo_bits={self.turbo_bits}"
        if self.gptq_bits is not None:
            s += f", bits={self.gptq_bits}, groupsize={self.gptq_groupsize}"
        if self.SV is not None:
            s += f", lora_rank={self.rank}"
        return s


class GLoRCQExperts(nn.Module):
    """Quantized MoE experts with the HF-5 `XxxExperts` call shape
    (reference inference/quantized_linear.py:368-428): per-expert gate, up and
    down GLoRCQLinear lists; forward(hidden, top_k_index, top_k_weights)."""

    def __init__(self, num_experts, hidden_dim, intermediate_dim, act_fn):
        super().__init__()
        self.num_experts = num_experts
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.gate_experts = nn.ModuleList([GLoRCQLinear(hidden_dim, intermediate_dim)
                                           for _ in range(num_experts)])
        self.up_experts = nn.ModuleList([GLoRCQLinear(hidden_dim, intermediate_dim)
                                         for _ in range(num_experts)])
        self.down_experts = nn.ModuleList([GLoRCQLinear(intermediate_dim, hidden_dim)
                                           for _ in range(num_experts)])
        self.act_fn = act_fn

    def forward(self, hidden_states, top_k_index, top_k_weights):
        """Same dispatch semantics as the reference (:395-428): for each hit
        expert, gather its tokens, down(act(gate) * up), scale by the routing
        weight and index_add into the output."""
        final = torch.zeros_like(hidden_states)
        with torch.no_grad():
            mask = torch.nn.functional.one_hot(top_k_index, num_classes=self.num_experts)
            mask = mask.permute(2, 1, 0)
            hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
        for e in hit.flatten().tolist():
            pos, tok = torch.where(mask[e])
            h = hidden_states[tok]
            inter = self.act_fn(self.gate_experts[e](h)) * self.up_experts[e](h)
            out = self.down_experts[e](inter)
            out = out * top_k_weights[tok, pos, None]
            final.index_add_(0, tok, out.to(final.dtype))
        return final
