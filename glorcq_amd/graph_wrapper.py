"""hipGraph-captured greedy decode for models built on the MI355X layers.

Mirrors the reference's GLoRCQGraphWrapper (inference/graph_wrapper.py:21-212):
same constructor, `capture_graph`, `replay` and `generate`, same phases —
prefill as an ordinary forward into a static KV cache, then every decode
token as one replay of a graph captured over a fixed (batch, 1) step.  On
ROCm `torch.cuda.CUDAGraph` records a hipGraph; every entry point of the
library is capture-safe (no allocation, no host sync), and the MoE step keeps
its routing on the device, so the captured step reads only the selected
experts' weights (the reference's graph mode computes all of them).

Differences: the static KV cache is built for the installed transformers
(`StaticCache(config, max_cache_len)` in 5.x; the 4.x signature with batch,
device and dtype is used when that is what the class takes); `generate`
captures (if needed) before its prefill, so capture's own warm-up steps never
land in the prompt's cache; the capture stream keeps the default priority.
"""

from __future__ import annotations

import gc
import inspect
import time

import torch


def _static_cache(model, max_batch_size, max_seq_len, device, dtype):
    from transformers import StaticCache

    params = inspect.signature(StaticCache.__init__).parameters
    if "max_batch_size" in params:  # transformers 4.x
        return StaticCache(config=model.config, max_batch_size=max_batch_size,
                           max_cache_len=max_seq_len, device=device, dtype=dtype)
    return StaticCache(config=model.config, max_cache_len=max_seq_len)


class GLoRCQGraphWrapper:
    """Graph-captured decode (reference inference/graph_wrapper.py:21-212).

    Usage:
        wrapper = GLoRCQGraphWrapper(model, max_batch_size=1, max_seq_len=4096)
        output_ids, duration = wrapper.generate(input_ids, max_new_tokens=128)
    """

    def __init__(self, model, max_batch_size=1, max_seq_len=4096):
        self.model = model
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        p = next(model.parameters())
        self.device, self.dtype = p.device, p.dtype
        self.static_cache = _static_cache(model, max_batch_size, max_seq_len, self.device,
                                          self.dtype)
        self.static_input_ids = torch.zeros((max_batch_size, 1), dtype=torch.long,
                                            device=self.device)
        self.static_cache_position = torch.zeros((1,), dtype=torch.long, device=self.device)
        self.static_logits = None
        self.graph = None
        self.graph_stream = torch.cuda.Stream(device=self.device)
        self.last_timing = {}

    def _set_moe_graph_mode(self, mode: bool):
        """Sets graph_mode on every MoE block (the reference toggles its blocks
        between the eager and the all-experts graph path; this build's blocks
        run one graph-safe path either way)."""
        for module in self.model.modules():
            if hasattr(module, "graph_mode"):
                module.graph_mode = mode

    def _step(self):
        return self.model(input_ids=self.static_input_ids,
                          cache_position=self.static_cache_position,
                          past_key_values=self.static_cache, use_cache=True, return_dict=False)

    @torch.no_grad()
    def capture_graph(self):
        """Step 0 allocates (the cache's lazy buffers), 3 warm-up steps run on a
        side stream, then one decode step is captured (reference :69-131)."""
        self.model.eval()
        self._set_moe_graph_mode(True)
        self.static_input_ids.fill_(1)
        self.static_cache_position.fill_(0)
        self._step()
        torch.cuda.synchronize(self.device)
        gc.collect()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(3):
                self.static_input_ids.fill_(1)
                self.static_cache_position.fill_(10)
                self._step()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        gc.collect()
        self.graph = torch.cuda.CUDAGraph()
        self.static_input_ids.fill_(1)
        self.static_cache_position.fill_(0)
        with torch.cuda.graph(self.graph, stream=self.graph_stream):
            self.static_logits = self._step()[0]

    @torch.no_grad()
    def replay(self, input_ids, cache_position_val):
        """One decode step: (batch, 1) ids at sequence position
        cache_position_val -> the captured logits buffer (reference :134-149)."""
        if input_ids.shape[0] != self.max_batch_size:
            raise RuntimeError(f"input batch {input_ids.shape[0]} != graph batch "
                               f"{self.max_batch_size}")
        self.static_input_ids.copy_(input_ids)
        self.static_cache_position.fill_(cache_position_val)
        self.graph.replay()
        return self.static_logits

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens=100):
        """Greedy generation: prefill forward, then graph replays; returns
        (prompt + generated ids, seconds) as the reference (:151-212).  The
        prefill and decode times are kept in `last_timing`."""
        batch, seq_len = input_ids.shape
        if batch != self.max_batch_size:
            raise RuntimeError(f"input batch {batch} != max_batch_size {self.max_batch_size}")
        if self.graph is None:
            # captured before the prefill: capture's own steps write the cache,
            # which the reset below clears (the reference captures after its
            # prefill, over positions 0 and 10 of the prompt's cache)
            self.capture_graph()
        t0 = time.time()
        output_ids = input_ids.clone()
        self._set_moe_graph_mode(False)
        self.static_cache.reset()
        cache_position = torch.arange(seq_len, device=self.device)
        logits = self.model(input_ids=input_ids, cache_position=cache_position,
                            past_key_values=self.static_cache, use_cache=True,
                            return_dict=False)[0]
        next_token = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
        output_ids = torch.cat([output_ids, next_token], dim=1)
        torch.cuda.synchronize(self.device)
        t1 = time.time()
        self._set_moe_graph_mode(True)
        for i in range(max_new_tokens - 1):
            pos = seq_len + i
            if pos >= self.max_seq_len:
                break
            logits = self.replay(next_token, pos)
            next_token = torch.argmax(logits[:, -1, :], dim=-1, keepdim=True)
            output_ids = torch.cat([output_ids, next_token], dim=1)
        torch.cuda.synchronize(self.device)
        t2 = time.time()
        self.last_timing = {"prefill_s": t1 - t0, "decode_s": t2 - t1,
                            "decode_tokens": output_ids.shape[1] - seq_len - 1}
        return output_ids, t2 - t0
