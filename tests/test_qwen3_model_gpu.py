"""Model-level greedy decode of the Qwen3-MoE-shaped model that the model
benchmark runs (glorcq_amd.synthetic_model: transformers' Qwen3-MoE modeling
code, 4-bit GLoRCQLinear attention projections, GraphCompatibleMoeBlock with
2-bit routed experts and cross-layer U pools), at full width -- hidden 2048,
32/4 heads of 128, 128 experts of 768, top-8 renormalised, rank 64 -- with 2
layers and a 1024-token vocabulary so that a CPU twin stays small.

The twin is built from the GPU model's own tensors (packed codes unpacked by
the oracle, exact weights s (q - z) in fp32, the MoE oracle over each layer's
experts with their pool rows as clusters), so the builder's wiring -- pool
rows through u_slot for gate/up, pool rows directly for down -- is checked
along with the kernels.

Checks (as for the Qwen2-MoE model, the graph wrapper's contract and the
north star's greedy-token criterion):
  * graph replays give exactly the eager model's tokens;
  * tokens match the twin wherever the twin's top-2 margin exceeds the fp16
    pipeline's error, and the prompt's logits agree within 2 % of their range;
  * a teacher-forced continuation: every replayed position's logits within 2 %
    of the twin's range, the same argmax where the margin allows.
"""

import copy

import pytest
import torch
import torch.nn as nn

from glorcq_amd import format as fmt
from glorcq_amd.graph_wrapper import GLoRCQGraphWrapper
from glorcq_amd.synthetic_model import build_qwen3_moe, qwen3_moe_config
from oracle import glorcq_oracle as O
from test_graph_wrapper_gpu import DenseTwinLinear, _eager_greedy, _twin_greedy

pytestmark = pytest.mark.gpu

VOCAB = 1024


class _Lin:
    """The fields DenseTwinLinear reads, from a GPU GLoRCQLinear."""

    def __init__(self, lin):
        K = lin.in_features
        self.q = torch.from_numpy(O.unpack_codes(lin.codes.cpu().numpy(), lin.pack_bits, K))
        self.scales, self.zeros = lin.scales.cpu(), lin.zeros.cpu()
        self.group = lin.gptq_groupsize
        self.U, self.SV = lin.U.cpu(), lin.SV.cpu()


def _problem(blk) -> fmt.MoEProblem:
    """The block's weights as an oracle problem: each expert's cluster is its
    pool row (gate/up: the local cluster's u_slot entry; down: as stored)."""
    t = blk.t
    experts, SV, U, cl = {}, {}, {}, {}
    for proj in fmt.PROJS:
        experts[proj] = fmt.QMat(codes=t[f"codes_{proj}"].cpu(), scales=t[f"scales_{proj}"].cpu(),
                                 zeros=t[f"zeros_{proj}"].cpu(), bits=blk.bits, group=128)
        SV[proj] = t[f"SV_{proj}"].cpu()
        U[proj] = t[f"U_{proj}"].cpu()
        c = t[f"cluster_{proj}"].long()
        cl[proj] = (c if proj == "down" else t[f"uslot_{proj}"].long()[c]).cpu()
    rows = int(U["gate"].shape[0])
    return fmt.MoEProblem(H=blk.hidden, E=blk.num_experts, inter=blk.inter, top_k=blk.top_k,
                          norm_topk_prob=blk.norm_topk_prob, rank=blk.rank, n_clusters=rows,
                          router_w=t["router_w"].cpu(), shared_gate_w=None, experts=experts,
                          SV=SV, cluster_of=cl, U=U, shared=None,
                          h=torch.zeros(1, blk.hidden, dtype=torch.float16))


class OracleMoe(nn.Module):
    def __init__(self, p):
        super().__init__()
        self.p = p
        self.memo = {}  # the experts' exact weights, formed once

    def forward(self, hidden_states):
        shape = hidden_states.shape
        y = O.moe_forward(self.p, exact=True, h=hidden_states.reshape(-1, self.p.H).half(),
                          memo=self.memo)
        return y.float().reshape(shape)


_CACHE = {}


def _build(dev):
    if "m" in _CACHE:
        return _CACHE["m"]
    from transformers import Qwen3MoeForCausalLM

    cfg = qwen3_moe_config(num_hidden_layers=2, vocab_size=VOCAB, max_position_embeddings=512)
    model, _ = build_qwen3_moe(cfg, dev, seed=0)
    with torch.no_grad():  # a sharper head, so greedy margins stand clear of fp16 noise
        model.lm_head.weight.mul_(4.0)
    with torch.device("meta"):
        twin = Qwen3MoeForCausalLM(copy.deepcopy(cfg))
    for li, layer in enumerate(twin.model.layers):
        src = model.model.layers[li]
        sattn = getattr(src.self_attn, "inner", src.self_attn)  # the fused layer wraps it
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(layer.self_attn, name, DenseTwinLinear(_Lin(getattr(sattn, name)), None))
        layer.mlp = OracleMoe(_problem(src.mlp))
    twin = twin.to_empty(device="cpu").float()
    sd = {k.replace(".self_attn.inner.", ".self_attn."): v.float().cpu()
          for k, v in model.state_dict().items() if "rotary_emb" not in k}
    missing, unexpected = twin.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary_emb" in k for k in missing), (missing, unexpected)
    twin.model.rotary_emb = type(twin.model.rotary_emb)(config=cfg)
    twin.eval()
    _CACHE["m"] = (model, twin)
    return model, twin


def test_builder_wiring(gpu):
    """Pool rows: every expert's gate/up cluster maps back to its drawn pool
    row, all layers share one pool tensor per projection."""
    cfg = qwen3_moe_config(num_hidden_layers=2, vocab_size=VOCAB, max_position_embeddings=512)
    model, info = build_qwen3_moe(cfg, gpu, seed=1)
    for li, layer in enumerate(model.model.layers):
        t = layer.mlp.t
        for proj in ("gate", "up"):
            rows = t[f"uslot_{proj}"].long()[t[f"cluster_{proj}"].long()]
            assert torch.equal(rows, info["cluster_ids"][proj][li])
            assert t[f"U_{proj}"].data_ptr() == info["pools"][proj].data_ptr()
        assert torch.equal(t["cluster_down"].long(), info["cluster_ids"]["down"][li])
        assert layer.mlp.n_clusters == max(int(t["uslot_gate"].numel()),
                                           int(t["uslot_up"].numel()))


@torch.no_grad()
def test_graph_decode_matches_eager_and_twin(gpu):
    model, twin = _build(gpu)
    prompt = torch.randint(0, VOCAB, (1, 12), generator=torch.Generator().manual_seed(3))
    n = 16
    wrapper = GLoRCQGraphWrapper(model, max_batch_size=1, max_seq_len=128)
    out, secs = wrapper.generate(prompt.to(gpu), max_new_tokens=n)
    torch.cuda.synchronize()
    graph_toks = out[0, prompt.shape[1]:].tolist()
    assert len(graph_toks) == n and secs > 0
    eager_toks, eager_first, _ = _eager_greedy(model, prompt, n, gpu, 128)
    torch.cuda.synchronize()
    assert graph_toks == eager_toks, (graph_toks, eager_toks)
    twin_toks, margins, twin_first = _twin_greedy(twin, prompt, n)
    err = (eager_first - twin_first.float()).abs().max()
    span = twin_first.abs().max()
    assert float(err) <= 0.02 * float(span), (float(err), float(span))
    for i, (a, b, m) in enumerate(zip(graph_toks, twin_toks, margins)):
        if a != b:
            assert m < 0.02 * float(span), f"step {i}: token {a} vs twin {b}, margin {m:.4f}"
            break  # below the fp16 pipeline's resolution; later tokens follow other prefixes
    matched = sum(1 for a, b in zip(graph_toks, twin_toks) if a == b)
    print(f"graph decode: {graph_toks}\ntwin:         {twin_toks}\nmatched {matched}/{n}, "
          f"prompt logits max err {float(err):.4f} of {float(span):.3f}", flush=True)


@torch.no_grad()
def test_teacher_forced_steps_match_twin(gpu):
    from transformers import DynamicCache

    model, twin = _build(gpu)
    g = torch.Generator().manual_seed(11)
    prompt = torch.randint(0, VOCAB, (1, 10), generator=g)
    cont = torch.randint(0, VOCAB, (12,), generator=g).tolist()
    wrapper = GLoRCQGraphWrapper(model, max_batch_size=1, max_seq_len=64)
    wrapper.capture_graph()
    wrapper.static_cache.reset()
    model(input_ids=prompt.to(gpu), cache_position=torch.arange(10, device=gpu),
          past_key_values=wrapper.static_cache, use_cache=True, return_dict=False)
    cache = DynamicCache()
    twin(input_ids=prompt, past_key_values=cache, use_cache=True, return_dict=False)
    checked = 0
    for i, t in enumerate(cont):
        mine = wrapper.replay(torch.tensor([[t]], device=gpu), 10 + i)[0, -1].float().cpu()
        ref = twin(input_ids=torch.tensor([[t]]), past_key_values=cache, use_cache=True,
                   return_dict=False)[0][0, -1].float()
        span = float(ref.abs().max())
        err = float((mine - ref).abs().max())
        assert err <= 0.02 * span, (i, err, span)
        top2 = torch.topk(ref, 2).values
        if float(top2[0] - top2[1]) > 0.02 * span:
            assert int(torch.argmax(mine)) == int(torch.argmax(ref)), i
            checked += 1
    assert checked >= len(cont) // 2, checked


@torch.no_grad()
def test_batched_graph_decode_matches_eager(gpu):
    """Batch 4 under the graph: each row's tokens equal the eager model's run
    of the same batch (the step at B > 1 takes the MoE grouped path)."""
    model, _ = _build(gpu)
    B, n = 4, 8
    prompt = torch.randint(0, VOCAB, (B, 9), generator=torch.Generator().manual_seed(7)).to(gpu)
    wrapper = GLoRCQGraphWrapper(model, max_batch_size=B, max_seq_len=64)
    out, _ = wrapper.generate(prompt, max_new_tokens=n)
    from glorcq_amd.graph_wrapper import _static_cache

    cache = _static_cache(model, B, 64, gpu, torch.float16)
    logits = model(input_ids=prompt, cache_position=torch.arange(9, device=gpu),
                   past_key_values=cache, use_cache=True, return_dict=False)[0]
    toks = []
    for i in range(n):
        t = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
        toks.append(t)
        if i + 1 < n:
            logits = model(input_ids=t, cache_position=torch.tensor([9 + i], device=gpu),
                           past_key_values=cache, use_cache=True, return_dict=False)[0]
    eager = torch.cat(toks, dim=1)
    torch.cuda.synchronize()
    assert torch.equal(out[:, 9:], eager), (out[:, 9:].tolist(), eager.tolist())


def _twin_greedy_batch(twin, prompt, n):
    """Greedy decode of every row of `prompt` (B, T) through the CPU twin:
    (n lists of B tokens, n lists of B top-2 margins, the prompt's logits)."""
    from transformers import DynamicCache

    cache = DynamicCache()
    logits = twin(input_ids=prompt, past_key_values=cache, use_cache=True, return_dict=False)[0]
    first = logits.clone()
    toks, margins = [], []
    for i in range(n):
        last = logits[:, -1]
        top2 = torch.topk(last, 2, dim=-1).values
        margins.append((top2[:, 0] - top2[:, 1]).tolist())
        t = torch.argmax(last, dim=-1, keepdim=True)
        toks.append(t[:, 0].tolist())
        if i + 1 < n:
            logits = twin(input_ids=t, past_key_values=cache, use_cache=True,
                          return_dict=False)[0]
    return toks, margins, first


def _check_rows_against_twin(graph, twin_toks, margins, span, what):
    """Row by row: the graph's tokens equal the twin's up to the first step
    whose twin margin is below the fp16 pipeline's resolution (2 % of the
    logit range); later tokens follow another prefix."""
    matched = 0
    for b in range(graph.shape[0]):
        for i in range(graph.shape[1]):
            if int(graph[b, i]) != twin_toks[i][b]:
                assert margins[i][b] < 0.02 * span, \
                    f"{what} row {b} step {i}: {int(graph[b, i])} vs twin {twin_toks[i][b]}, " \
                    f"margin {margins[i][b]:.4f}"
                break
            matched += 1
    return matched


@torch.no_grad()
def test_b16_graph_decode_matches_twin(gpu):
    """BASELINE config 4's batch 16: sixteen prompts decoded together under
    the graph (the MoE step's 16-token path, the token-tile attention
    projections) against the twin decoding the same batch; the 16 x 12-token
    prompt (192 tokens) runs the MoE prefill and the prefill GEMM."""
    from glorcq_amd.graph_wrapper import _static_cache

    model, twin = _build(gpu)
    B, T, n = 16, 12, 8
    prompt = torch.randint(0, VOCAB, (B, T), generator=torch.Generator().manual_seed(17))
    wrapper = GLoRCQGraphWrapper(model, max_batch_size=B, max_seq_len=64)
    out, _ = wrapper.generate(prompt.to(gpu), max_new_tokens=n)
    graph = out[:, T:].cpu()
    cache = _static_cache(model, B, 64, gpu, torch.float16)
    first = model(input_ids=prompt.to(gpu), cache_position=torch.arange(T, device=gpu),
                  past_key_values=cache, use_cache=True, return_dict=False)[0].float().cpu()
    torch.cuda.synchronize()
    print("B=16 graph decode done; running the twin", flush=True)
    twin_toks, margins, twin_first = _twin_greedy_batch(twin, prompt, n)
    span = float(twin_first.abs().max())
    err = float((first - twin_first.float()).abs().max())
    assert err <= 0.02 * span, (err, span)
    matched = _check_rows_against_twin(graph, twin_toks, margins, span, "B=16")
    print(f"B=16: {matched}/{B * n} tokens matched before any low-margin step; prompt "
          f"logits max err {err:.4f} of {span:.3f}", flush=True)


@torch.no_grad()
def test_long_prompt_prefill_matches_twin(gpu):
    """A 128-token prompt (BASELINE config 4's workload is a 512-token prompt):
    the prefill runs the MoE block's grouped-GEMM path (glq_moe_prefill, more
    than 64 tokens) and the attention projections' prefill GEMM (glq_gemm_lora,
    more than 16 rows).  Every prompt position's logits within 2 % of the
    twin's range, then greedy tokens under the graph equal the eager model's
    and the twin's where the margin allows."""
    model, twin = _build(gpu)
    T, n = 128, 8
    prompt = torch.randint(0, VOCAB, (1, T), generator=torch.Generator().manual_seed(19))
    wrapper = GLoRCQGraphWrapper(model, max_batch_size=1, max_seq_len=256)
    out, _ = wrapper.generate(prompt.to(gpu), max_new_tokens=n)
    torch.cuda.synchronize()
    graph_toks = out[0, T:].tolist()
    eager_toks, eager_first, _ = _eager_greedy(model, prompt, n, gpu, 256)
    torch.cuda.synchronize()
    assert graph_toks == eager_toks, (graph_toks, eager_toks)
    print("T=128 prefill + decode done; running the twin", flush=True)
    twin_toks, margins, twin_first = _twin_greedy(twin, prompt, n)
    span = float(twin_first.abs().max())
    err = (eager_first - twin_first.float()).abs()
    assert float(err.max()) <= 0.02 * span, (float(err.max()), span)
    worst = int(err.amax(dim=-1).argmax())
    matched = _check_rows_against_twin(torch.tensor([graph_toks]),
                                       [[t] for t in twin_toks], [[m] for m in margins],
                                       span, "T=128")
    print(f"T=128: prompt logits max err {float(err.max()):.4f} of {span:.3f} (position "
          f"{worst}); {matched}/{n} tokens matched", flush=True)
