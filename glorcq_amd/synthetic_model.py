"""Random-init Qwen3-MoE-shaped decoder on the MI355X layers (the model-level
benchmark shape: a Qwen3-30B-A3B-shaped model, greedy decode under a graph).

The reference has no Qwen3 inference path; its loader swaps each
`Qwen2MoeSparseMoeBlock` for `GraphCompatibleMoeBlock` and each quantized
projection for `GLoRCQLinear` (inference/model_builder.py:186-197,465-544).
This builder does the same to transformers' own Qwen3-MoE modeling code:

* every attention projection (q, k, v, o) is a `GLoRCQLinear` with GPTQ codes
  (4-bit by default, group 128) and its own rank-r low-rank factors;
* every sparse MoE block is a `GraphCompatibleMoeBlock` with b-bit routed
  experts (2-bit by default) whose gate/up/down U factors are rows of one
  cross-layer pool per projection: `n_clusters` clusters, each (layer,
  expert, projection) assigned one at random -- the reference's global U
  pool (model_builder.py:143-183), with the same cluster's U at one address
  for every layer that uses it;
* embeddings, norms and lm_head stay fp16 (the reference keeps them dense).

All weights are drawn on the device (a 48-layer model is ~10 GB of packed
weights and factors): codes uniform over every b-bit value (random packed
words), scales |N(0, 0.02)| fp16, low-rank factors N(0, 0.01) fp16, router
N(0, 0.02) fp16, embeddings and lm_head N(0, 0.02) fp16, norms 1.  Expert
zero-points are uniform over {1, 2} (2-bit codes centred, as in the kernel
benchmarks); attention zero-points sit at the middle of the code range
(uniform over {2^(b-1) - 1, 2^(b-1)}), so the projections stay zero-mean and
48 residual additions stay far inside fp16's range.
"""

from __future__ import annotations

import torch

from .format import PROJS
from .moe_block import GraphCompatibleMoeBlock
from .quantized_linear import GLoRCQLinear

GROUP = 128


def qwen3_moe_config(num_hidden_layers: int = 48, vocab_size: int = 151936,
                     max_position_embeddings: int = 4096):
    """Qwen3-30B-A3B dimensions: hidden 2048, 32 query / 4 KV heads of 128,
    128 experts of intermediate 768, top-8 with renormalised weights, every
    layer sparse."""
    from transformers import Qwen3MoeConfig

    return Qwen3MoeConfig(vocab_size=vocab_size, hidden_size=2048, intermediate_size=6144,
                          num_hidden_layers=num_hidden_layers, num_attention_heads=32,
                          num_key_value_heads=4, head_dim=128, moe_intermediate_size=768,
                          num_experts=128, num_experts_per_tok=8, norm_topk_prob=True,
                          decoder_sparse_step=1, mlp_only_layers=[], rms_norm_eps=1e-6,
                          max_position_embeddings=max_position_embeddings,
                          tie_word_embeddings=False, attention_bias=False)


def _words(shape, gen, dev):
    """Random packed code words: every code of every width uniform."""
    return torch.randint(-(2**31), 2**31 - 1, shape, generator=gen, device=dev,
                         dtype=torch.int64).to(torch.int32)


def _normal(shape, std, gen, dev):
    return (torch.randn(shape, generator=gen, device=dev) * std).half()


def _attn_linear(K, N, bits, rank, gen, dev) -> GLoRCQLinear:
    lin = GLoRCQLinear(K, N)
    mid = 1 << (bits - 1)
    q = torch.randint(0, 1 << bits, (N, K), generator=gen, device=dev, dtype=torch.int32)
    scales = (torch.randn(N, K // GROUP, generator=gen, device=dev) * 0.02).abs().half()
    zeros = torch.randint(mid - 1, mid + 1, (N, K // GROUP), generator=gen, device=dev,
                          dtype=torch.int32).half()
    lin.load_gptq({"qweight_int": q, "scales": scales, "zeros": zeros, "bits": bits,
                   "groupsize": GROUP, "sym": False}, device=dev)
    if rank > 0:
        lin.load_sv(_normal((K, rank), 0.01, gen, dev), _normal((N, rank), 0.01, gen, dev),
                    device=dev)
    return lin


def _moe_block(cfg, pools, ids, bits, rank, gen, dev) -> GraphCompatibleMoeBlock:
    """One layer's block: stacked random experts; ids[proj] holds each
    expert's pool row.  Gate/up form x U per local cluster (the distinct rows,
    reached through u_slot); down reads U at each expert's pool row."""
    E, H, I = cfg.num_experts, cfg.hidden_size, cfg.moe_intermediate_size
    t = {"E": E, "top_k": cfg.num_experts_per_tok, "norm_topk_prob": cfg.norm_topk_prob,
         "H": H, "inter": I, "bits": bits, "rank": rank, "shared_bits": 0, "shared_inter": 0,
         "shared_gate_w": None, "router_w": _normal((E, H), 0.02, gen, dev)}
    dims = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    C = 1
    for proj in PROJS:
        N, K = dims[proj]
        t[f"codes_{proj}"] = _words((E, N, K * bits // 32), gen, dev)
        t[f"scales_{proj}"] = (torch.randn(E, N, K // GROUP, generator=gen, device=dev)
                               * 0.02).abs().half()
        t[f"zeros_{proj}"] = torch.randint(1, 3, (E, N, K // GROUP), generator=gen, device=dev,
                                           dtype=torch.int32).half()
        if rank > 0:
            t[f"SV_{proj}"] = _normal((E, N, rank), 0.01, gen, dev)
            t[f"U_{proj}"] = pools[proj]
            t[f"urows_{proj}"] = int(pools[proj].shape[0])
            if proj == "down":
                t["cluster_down"] = ids[proj].to(torch.int32).contiguous()
            else:
                uniq, local = torch.unique(ids[proj], return_inverse=True)
                t[f"cluster_{proj}"] = local.to(torch.int32).contiguous()
                t[f"uslot_{proj}"] = uniq.to(torch.int32).contiguous()
                C = max(C, int(uniq.numel()))
    t["n_clusters"] = C
    blk = GraphCompatibleMoeBlock(stacked=t)
    blk.return_router_logits = False  # transformers 5 sparse blocks return the states alone
    return blk


@torch.no_grad()
def build_qwen3_moe(config, device, seed: int = 0, attn_bits: int = 4, expert_bits: int = 2,
                    rank: int = 64, n_clusters: int = 128, fused: bool = True):
    """Qwen3MoeForCausalLM(config) in fp16 on `device` with GLoRCQ layers and
    random weights.  Returns (model, info); info["pools"][proj] is the
    (n_clusters, K, rank) U pool and info["cluster_ids"][proj] the (layers,
    experts) pool row of every expert.  fused: decoder layers and the final
    norm on this build's kernels (glorcq_amd.decoder); False keeps
    transformers' own layer code around the GLoRCQ projections and MoE blocks."""
    from transformers import Qwen3MoeForCausalLM

    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    with torch.device("meta"):
        model = Qwen3MoeForCausalLM(config)
    L, E, H, I = (config.num_hidden_layers, config.num_experts, config.hidden_size,
                  config.moe_intermediate_size)
    pools, cids = {}, {}
    if rank > 0:
        for proj, K in (("gate", H), ("up", H), ("down", I)):
            pools[proj] = _normal((n_clusters, K, rank), 0.01, gen, dev).contiguous()
            cids[proj] = torch.randint(0, n_clusters, (L, E), generator=gen, device=dev)
    for li, layer in enumerate(model.model.layers):
        attn = layer.self_attn
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin = getattr(attn, name)
            setattr(attn, name, _attn_linear(lin.in_features, lin.out_features, attn_bits, rank,
                                             gen, dev))
        layer.mlp = _moe_block(config, pools, {p: cids[p][li] for p in cids}, expert_bits, rank,
                               gen, dev)
    # the dense remainder: embeddings, norms, lm_head (the GLoRCQ layers hold
    # plain tensors, not parameters, so to_empty leaves them alone)
    model = model.to_empty(device=dev).half()
    for name, prm in model.named_parameters():
        if name.endswith("norm.weight"):
            prm.fill_(1.0)
        else:
            prm.copy_(_normal(prm.shape, 0.02, gen, dev))
    # rotary tables are buffers computed at construction (empty after
    # to_empty): rebuild them on the device, in fp32
    rot = model.model.rotary_emb
    model.model.rotary_emb = type(rot)(config=config).to(dev)
    if fused:
        from .decoder import fuse_decoder_layers

        fuse_decoder_layers(model)
    model.eval()
    return model, {"pools": pools, "cluster_ids": cids}
