"""Decoder layer of the model-level decode step on the MI355X kernels.

The reference's model path runs everything around its quantized projections
and MoE blocks as framework ops (its graph wrapper captures them as they are,
inference/graph_wrapper.py:69-149).  For the Qwen3-MoE-shaped model that is
~60 small kernels per layer per decode token (RMSNorm alone is 7), which at
decode sizes cost more than the projections.  These modules replace them
with one launch each, keeping the framework's fp16 rounding points:

* `FusedRMSNorm` -- Qwen3MoeRMSNorm (glq_rmsnorm);
* `GLoRCQQwen3Attention` -- Qwen3MoeAttention for one decode token against a
  static cache: GLoRCQLinear q/k/v projections, then q/k head RMSNorm +
  rotary embedding + cache write (glq_qk_norm_rope), single-query GQA
  attention (glq_decode_attention), GLoRCQLinear o projection.  Prefill (more
  than one token) and a cache that is not static or not yet allocated take
  the wrapped module's own forward;
* `GLoRCQQwen3DecoderLayer` -- Qwen3MoeDecoderLayer with the residual add
  after attention fused into the post-attention RMSNorm.

The cache semantics are those of transformers' StaticLayer: the token is
written at the layer's `cumulative_length` (a device counter), attention
covers positions [0, cumulative_length], and the counter then advances by
one -- all on the device, so the step can be captured in a graph.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import kernels
from .moe_block import GraphCompatibleMoeBlock


class FusedRMSNorm(nn.Module):
    """Qwen3MoeRMSNorm in one launch (same weight parameter)."""

    def __init__(self, norm):
        super().__init__()
        self.weight = norm.weight
        self.variance_epsilon = norm.variance_epsilon

    def forward(self, hidden_states):
        return kernels.rmsnorm(hidden_states.contiguous(), self.weight, self.variance_epsilon)


def _static_layer(past_key_values, idx, batch):
    """The layer's StaticLayer when its buffers exist and match the batch."""
    layers = getattr(past_key_values, "layers", None)
    if layers is None or idx >= len(layers):
        return None
    lay = layers[idx]
    cum = getattr(lay, "cumulative_length", None)
    if not getattr(lay, "is_initialized", False) or not torch.is_tensor(cum):
        return None
    keys = getattr(lay, "keys", None)
    if keys is None or keys.dim() != 4 or keys.shape[0] != batch or keys.dtype != torch.float16:
        return None
    return lay


class GLoRCQQwen3Attention(nn.Module):
    """Qwen3MoeAttention with a fused single-token decode path."""

    def __init__(self, attn):
        super().__init__()
        self.inner = attn
        self.layer_idx = attn.layer_idx
        self.head_dim = attn.head_dim
        self.scaling = attn.scaling
        if attn.q_norm.variance_epsilon != attn.k_norm.variance_epsilon:
            raise RuntimeError("q_norm and k_norm must share eps")
        # q/k/v share their input: their U factors side by side, so one
        # launch forms all three x U products
        self._U_qkv = None
        lins = (attn.q_proj, attn.k_proj, attn.v_proj)
        Us = [getattr(m, "U", None) for m in lins]
        if all(u is not None and getattr(m, "quant_type", None) == "gptq" for u, m in zip(Us, lins)) \
                and len({tuple(u.shape) for u in Us}) == 1 and Us[0].is_cuda:
            self._U_qkv = torch.stack(Us).contiguous()
            for i, m in enumerate(lins):
                m.U = self._U_qkv[i]  # the same values, now views of the stack
        # Decode tokens (up to 16): q, k and v as ONE batched GEMV launch
        # (plus, from 2 tokens, its x U partials) over items of kv_out rows --
        # q's rows as q_out/kv_out items, then k, then v -- with the three
        # layers' codes, scales, zero-points and SV laid end to end (the layers
        # keep views of them) and each item naming its U in the (3, K, r)
        # stack (q's items share one, so one token forms x U_q once); q comes
        # out item-major, which the norm/rotary kernel reads as it is.
        self._qkv = None
        q, k, v = lins
        nkv = k.out_features
        if (self._U_qkv is not None and v.out_features == nkv and q.out_features % nkv == 0
                and all(m.bias_param is None and not m.gptq_sym and m.zeros is not None
                        and m.pack_bits == q.pack_bits and m.gptq_groupsize == q.gptq_groupsize
                        for m in lins)):
            nq = q.out_features // nkv
            cat = {}
            for name in ("codes", "scales", "zeros", "SV"):
                full = torch.cat([getattr(m, name) for m in lins]).contiguous()
                cat[name] = full.view(nq + 2, nkv, *full.shape[1:])
                setattr(q, name, full[:q.out_features])
                setattr(k, name, full[q.out_features:q.out_features + nkv])
                setattr(v, name, full[q.out_features + nkv:])
            cat["U"] = self._U_qkv
            cat["u_index"] = torch.tensor([0] * nq + [1, 2], dtype=torch.int32,
                                          device=self._U_qkv.device)
            self._qkv = cat
        # The o projection's x U formed by the attention launch itself (its
        # merging blocks, glq_decode_attention_xu) at XU_PRODUCER_MIN_M ..
        # XU_PRODUCER_MAX_M tokens, as partials that the projection sums as
        # its a (glq_gemv_lora_parts).
        o = attn.o_proj
        self._o_xu = (getattr(o, "quant_type", None) == "gptq" and getattr(o, "U", None) is not None
                      and getattr(o, "SV", None) is not None and o.U.is_cuda
                      and o.U.shape[1] % 8 == 0 and o.bias_param is None)
        self._len = None  # device int32: positions the step attends to
        self._ws = None   # decode attention workspace (counters stay zero between calls)
        self._ws_key = None

    # At this many tokens the decode step forms the projections' x U in the
    # launches that produce their inputs (the input RMSNorm for q/k/v, the
    # attention for o).  At one token the projections' own one-row launches
    # form it (x U jobs in front of the row workgroups: about 2.8 us a layer
    # less than the producers' partials); from 4 tokens the token-tile GEMV
    # forms it in its own launch.
    XU_PRODUCER_MIN_M = 2
    XU_PRODUCER_MAX_M = 3

    @classmethod
    def xu_by_producer(cls, B):
        return cls.XU_PRODUCER_MIN_M <= B <= cls.XU_PRODUCER_MAX_M

    def qkv_u(self, B):
        """The (3, K, r) stack of the q/k/v U factors when a decode step of B
        tokens takes its x U partials from the input RMSNorm's launch
        (rmsnorm_xu), else None."""
        if self._qkv is not None and self.xu_by_producer(B) and self._U_qkv.shape[2] % 8 == 0:
            return self._U_qkv
        return None

    def forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None,
                qkv_xu=None, **kwargs):
        """qkv_xu: x U partials of the q/k/v stack (3, S, B, rpad) for this
        step's normalized hidden states, formed by their RMSNorm launch
        (qkv_u, rmsnorm_xu)."""
        B, S, H = hidden_states.shape
        lay = _static_layer(past_key_values, self.layer_idx, B) if S == 1 else None
        if lay is None or self.head_dim != 128:
            return self.inner(hidden_states, position_embeddings, attention_mask,
                              past_key_values=past_key_values, **kwargs)
        inner = self.inner
        x = hidden_states.reshape(B, H)
        if self._qkv is not None and B <= kernels.GEMV_MAX_M:
            c = self._qkv
            if qkv_xu is not None:  # partials per U, item i summing qkv_xu[u_index[i]]
                y = kernels.packed_dequant_matmul_parts(
                    x.contiguous(), c["codes"], c["scales"], c["zeros"], inner.q_proj.pack_bits,
                    inner.q_proj.gptq_groupsize, c["SV"], qkv_xu, u_index=c["u_index"])
            else:
                y = kernels.packed_dequant_matmul_batched(
                    x.contiguous(), c["codes"], c["scales"], c["zeros"], inner.q_proj.pack_bits,
                    inner.q_proj.gptq_groupsize, U=c["U"], SV=c["SV"],
                    u_index=c["u_index"])  # (items, B, kv rows)
            n = y.shape[0] - 2
            q, k, v = y[:n], y[n], y[n + 1]  # q item-major: the norm/rotary kernel reads it so
        elif self._U_qkv is not None and B <= kernels.GEMV_MAX_M:
            xu = kernels.lowrank_xu(x.contiguous(), self._U_qkv)  # (3, B, r)
            q = inner.q_proj(x, precomputed_xU=xu[0])
            k = inner.k_proj(x, precomputed_xU=xu[1])
            v = inner.v_proj(x, precomputed_xU=xu[2])
        else:
            q = inner.q_proj(x)
            k = inner.k_proj(x)
            v = inner.v_proj(x)
        cos, sin = position_embeddings
        if self._len is None or self._len.device != x.device:
            self._len = torch.zeros(1, dtype=torch.int32, device=x.device)
        qr = kernels.qk_norm_rope(q, k, v, inner.q_norm.weight, inner.k_norm.weight,
                                  inner.q_norm.variance_epsilon, cos.contiguous(),
                                  sin.contiguous(), lay.keys, lay.values, lay.cumulative_length,
                                  self._len)
        if self._ws is None or self._ws_key != (tuple(lay.keys.shape), x.device):
            kernels.retire_workspace(self._ws)  # a captured graph may still use it
            self._ws = kernels.decode_attention_workspace(qr, lay.keys)
            self._ws_key = (tuple(lay.keys.shape), x.device)
        if self._o_xu and self.xu_by_producer(B):
            o = inner.o_proj
            a, parts = kernels.decode_attention(qr, lay.keys, lay.values, self._len, self.scaling,
                                                advance=lay.cumulative_length, workspace=self._ws,
                                                U=o.U)
            y = kernels.packed_dequant_matmul_parts(
                a, o.codes.unsqueeze(0), o.scales.unsqueeze(0),
                None if o.gptq_sym else o.zeros.unsqueeze(0), o.pack_bits, o.gptq_groupsize,
                o.SV.unsqueeze(0), parts.unsqueeze(0), sym=o.gptq_sym)
            return y.reshape(B, 1, -1), None
        a = kernels.decode_attention(qr, lay.keys, lay.values, self._len, self.scaling,
                                     advance=lay.cumulative_length, workspace=self._ws)
        return inner.o_proj(a).reshape(B, 1, -1), None


class GLoRCQQwen3DecoderLayer(nn.Module):
    """Qwen3MoeDecoderLayer: fused RMSNorms, the post-attention one taking the
    residual add with it, the GLoRCQ attention above, the layer's MoE block."""

    def __init__(self, layer):
        super().__init__()
        self.self_attn = GLoRCQQwen3Attention(layer.self_attn)
        self.mlp = layer.mlp
        self.input_layernorm = layer.input_layernorm
        self.post_attention_layernorm = layer.post_attention_layernorm
        self.hidden_size = layer.hidden_size

    def forward(self, hidden_states, attention_mask=None, position_ids=None,
                past_key_values=None, use_cache=False, position_embeddings=None, **kwargs):
        ln1, ln2 = self.input_layernorm, self.post_attention_layernorm
        x = hidden_states.contiguous()
        B, S = x.shape[0], x.shape[1]
        Uq = self.self_attn.qkv_u(B) if S == 1 else None
        if Uq is not None:  # the q/k/v x U in the norm's launch
            h, xu = kernels.rmsnorm_xu(x, ln1.weight, ln1.variance_epsilon, Uq)
            kwargs["qkv_xu"] = xu
        else:
            h = kernels.rmsnorm(x, ln1.weight, ln1.variance_epsilon)
        a, _ = self.self_attn(hidden_states=h, position_embeddings=position_embeddings,
                              attention_mask=attention_mask, past_key_values=past_key_values,
                              position_ids=position_ids, use_cache=use_cache, **kwargs)
        h2, res = kernels.rmsnorm(a.contiguous(), ln2.weight, ln2.variance_epsilon, residual=x)
        if isinstance(self.mlp, GraphCompatibleMoeBlock):
            y = self.mlp(h2, residual=res)  # the residual add inside the MoE step
            return y[0] if isinstance(y, tuple) else y
        return res + self.mlp(h2)


def fuse_decoder_layers(model):
    """Swaps every decoder layer of a Qwen3-MoE causal LM for
    GLoRCQQwen3DecoderLayer and the final norm for FusedRMSNorm (in place);
    returns the model."""
    inner = model.model
    for i, layer in enumerate(inner.layers):
        if not isinstance(layer, GLoRCQQwen3DecoderLayer):
            inner.layers[i] = GLoRCQQwen3DecoderLayer(layer)
    if not isinstance(inner.norm, FusedRMSNorm):
        inner.norm = FusedRMSNorm(inner.norm)
    return model
