"""load_glorcq_model (the reference's one-call loader, inference/model_builder.py:
203-312) on a checkpoint directory written in the reference's on-disk format:
config.json, glorcq_model.pt (GPTQ codes of every expert, shared-expert and
attention projection), cross_layer_info.pt (cluster-shared U per projection
type and layer-spanning cluster ids, per-expert SV), plus a safetensors file
with the non-quantized weights (embeddings, norms, router and shared-expert
gates, q/k/v biases, lm_head).

The loaded model runs greedy decode under GLoRCQGraphWrapper and must give
the eager model's tokens exactly, and the tokens of a CPU twin built from the
SOURCE data (not from the loaded model: exact dense weights for the
attention, the MoE oracle for the blocks) wherever the twin's top-2 margin
exceeds 2 % of its logit range, with the prompt's logits within that 2 %."""

import copy

import pytest
import torch

from glorcq_amd import format as fmt
from glorcq_amd import model_builder as MB
from glorcq_amd.graph_wrapper import GLoRCQGraphWrapper
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from glorcq_amd.quantized_linear import GLoRCQLinear
from oracle import glorcq_oracle as O
from test_graph_wrapper_gpu import (E, H, INTER, RANK, SHARED, TOPK, VOCAB, DenseTwinLinear,
                                    OracleMoe, _config, _eager_greedy, _twin_greedy)

pytestmark = pytest.mark.gpu


def _gptq(codes, scales, zeros, bits, K):
    qi = torch.from_numpy(O.unpack_codes(codes.numpy(), bits, K)).to(torch.int32)
    return {"qweight_int": qi, "scales": scales.clone(), "zeros": zeros.clone(), "bits": bits,
            "groupsize": 128, "sym": False}


def _write(tmp_path):
    from safetensors.torch import save_file
    from transformers import Qwen2MoeForCausalLM

    cfg = _config()
    torch.manual_seed(0)
    base = Qwen2MoeForCausalLM(cfg).eval()
    with torch.no_grad():
        base.lm_head.weight.mul_(4.0)
    twin = copy.deepcopy(base).float().eval()
    dense = {k: v.half().contiguous() for k, v in base.state_dict().items()
             if ".experts." not in k and not k.endswith("_proj.weight")
             and "rotary" not in k}
    layers, shared_m, per_v, assign = {}, {}, {}, {}

    def lora(wt, li, e, gid, U, SV):
        shared_m.setdefault(wt, {}).setdefault(gid, {"U_fp16": U.clone()})
        per_v.setdefault(wt, []).append({"SV_fp16": SV.clone()})
        assign.setdefault(wt, []).append({"layer": li, "expert": e, "group_id": gid})

    g = torch.Generator().manual_seed(5)
    for li in range(cfg.num_hidden_layers):
        p = fmt.make_moe(H=H, E=E, inter=INTER, top_k=TOPK, n_clusters=3, rank=RANK,
                         shared_inter=SHARED, B=1, seed=100 + li)
        twin.model.layers[li].mlp = OracleMoe(p)
        mods = {}
        for proj in fmt.PROJS:
            wt, q, s = f"{proj}_proj", p.experts[proj], p.shared[proj]
            for e in range(E):
                mods[f"mlp.experts.{e}.{wt}"] = _gptq(q.codes[e], q.scales[e], q.zeros[e],
                                                      q.bits, q.K)
                c = int(p.cluster_of[proj][e])
                lora(wt, li, e, 10 * li + c, p.U[proj][c], p.SV[proj][e])
            mods[f"mlp.shared_expert.{wt}"] = _gptq(s.codes[0], s.scales[0], s.zeros[0],
                                                    s.bits, s.K)
        dense[f"model.layers.{li}.mlp.gate.weight"] = p.router_w.clone()
        dense[f"model.layers.{li}.mlp.shared_expert_gate.weight"] = p.shared_gate_w.clone()
        attn, tattn = base.model.layers[li].self_attn, twin.model.layers[li].self_attn
        for j, name in enumerate(("q_proj", "k_proj", "v_proj", "o_proj")):
            lin = getattr(attn, name)
            lp = fmt.make_linear(lin.in_features, lin.out_features, bits=4, group=128, rank=RANK,
                                 seed=1000 * li + j)
            bias = (torch.randn(lin.out_features, generator=g) * 0.02).half() \
                if lin.bias is not None else None
            mods[f"self_attn.{name}"] = _gptq(lp.codes, lp.scales, lp.zeros, 4, lp.K)
            lora(name, li, -1, 1000 + 4 * li + j, lp.U, lp.SV)
            if bias is not None:
                dense[f"model.layers.{li}.self_attn.{name}.bias"] = bias
            setattr(tattn, name, DenseTwinLinear(lp, bias))
        layers[li] = mods
    cfg.save_pretrained(tmp_path)
    save_file(dense, str(tmp_path / "model.safetensors"))
    torch.save({"model_config": {"uv_bits": 16, "rotation_type": "qr", "qbit": 2},
                "layers": layers}, tmp_path / "glorcq_model.pt")
    torch.save({"config": {"uv_bits": 16}, "assignments": assign, "shared_matrices": shared_m,
                "per_expert_V": per_v}, tmp_path / "cross_layer_info.pt")
    return twin


@torch.no_grad()
def test_load_glorcq_model_decodes_like_twin(gpu, tmp_path):
    twin = _write(tmp_path)
    print("checkpoint written; loading", flush=True)
    model = MB.load_glorcq_model(str(tmp_path), device=gpu)
    torch.cuda.synchronize()
    for li, layer in enumerate(model.model.layers):
        assert isinstance(layer.mlp, GraphCompatibleMoeBlock), li
        assert layer.mlp.num_experts == E and layer.mlp.top_k == TOPK
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            ql = getattr(layer.self_attn, name)
            assert isinstance(ql, GLoRCQLinear) and ql.SV is not None, (li, name)
    assert not any(p.is_meta for p in model.parameters())
    prompt = torch.randint(0, VOCAB, (1, 12), generator=torch.Generator().manual_seed(3))
    n = 12
    wrapper = GLoRCQGraphWrapper(model, max_batch_size=1, max_seq_len=128)
    out, _ = wrapper.generate(prompt.to(gpu), max_new_tokens=n)
    torch.cuda.synchronize()
    graph_toks = out[0, prompt.shape[1]:].tolist()
    eager_toks, eager_first, _ = _eager_greedy(model, prompt, n, gpu, 128)
    assert graph_toks == eager_toks, (graph_toks, eager_toks)
    twin_toks, margins, twin_first = _twin_greedy(twin, prompt, n)
    span = float(twin_first.abs().max())
    err = float((eager_first - twin_first.float()).abs().max())
    assert err <= 0.02 * span, (err, span)
    for i, (a, b, m) in enumerate(zip(graph_toks, twin_toks, margins)):
        if a != b:
            assert m < 0.02 * span, f"step {i}: token {a} vs twin {b}, margin {m:.4f}"
            break
    matched = sum(1 for a, b in zip(graph_toks, twin_toks) if a == b)
    print(f"loaded model: {graph_toks}\ntwin:         {twin_toks}\nmatched {matched}/{n}, "
          f"prompt logits max err {err:.4f} of {span:.3f}", flush=True)
