"""Graph capture of the boundary's entry points.

* The reference-signature op gptq_dequant_matmul_fused (inference/kernels/
  __init__.py:284-346) runs inside the reference's CUDA-graph capture
  (GLoRCQLinear.forward, inference/quantized_linear.py:307-311, under
  graph_wrapper.py:69-131).  After one warm-up call on the same codes it does
  no host sync and no repack, so it captures; every replay must equal the
  eager result bit for bit (same kernels, same inputs).
* A workspace replaced by a larger one stays allocated: a graph captured with
  the old buffer still writes into it, and memory allocated after the
  replacement must not be overwritten by its replays.

Each replay is separated by eager work and a synchronization, and checked.
"""

import pytest
import torch

from glorcq_amd import kernels as K_
from test_gptq_gpu import gptq_data, lora

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,N,K,usv", [(1, 1408, 2048, False), (4, 2048, 1408, True),
                                       (32, 1408, 2048, True)])
def test_gptq_signature_captures_after_warmup(gpu, B, N, K, usv):
    x, q, s, z = gptq_data(B, N, K, seed=B)
    x, q, s, z = x.to(gpu), q.to(gpu), s.to(gpu), z.to(gpu)
    lu = tuple(t.to(gpu) for t in lora(K, N)) if usv else None
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        eager = K_.gptq_dequant_matmul_fused(x, q, s, z, 128, False, lora_USV=lu)  # warm-up
        eager = eager.clone()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = K_.gptq_dequant_matmul_fused(x, q, s, z, 128, False, lora_USV=lu)
    torch.cuda.synchronize()
    for i in range(3):
        y.fill_(float("nan"))
        _ = (x * 2).sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {i}"
    # the prepared codes are reused only while the tensor is unchanged
    q.add_(0)
    y2 = K_.gptq_dequant_matmul_fused(x, q, s, z, 128, False, lora_USV=lu)
    assert torch.equal(y2, eager)


def test_replaced_workspace_survives_for_captured_graph(gpu):
    """Capture a multi-row GEMV (x U partials in the per-stream workspace),
    then grow that stream's workspace with a larger eager call; replays still
    give the eager result and leave later allocations alone."""
    from glorcq_amd import format as fmt

    small = fmt.make_linear(512, 256, bits=4, group=128, rank=64, M=4, seed=3)
    # K = 8192 at 16 rows and rank 128: 32 K-slices x 16 x 128 x 4 B = 256 KiB of
    # partials, past the first buffer's 64 KiB
    big = fmt.make_linear(8192, 512, bits=4, group=128, rank=128, M=16, seed=4)
    d = lambda t: t.to(gpu)  # noqa: E731
    args = (d(small.x), d(small.codes), d(small.scales), d(small.zeros), 4, 128)
    kw = dict(U=d(small.U), SV=d(small.SV))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        eager = K_.packed_dequant_matmul_fused(*args, **kw).clone()
        ws0 = K_.gemv_workspace(gpu, 1)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y = K_.packed_dequant_matmul_fused(*args, **kw)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        K_.packed_dequant_matmul_fused(d(big.x), d(big.codes), d(big.scales), d(big.zeros), 4,
                                       128, U=d(big.U), SV=d(big.SV))
        ws1 = K_.gemv_workspace(gpu, 1)
    torch.cuda.synchronize()
    assert ws1.data_ptr() != ws0.data_ptr(), "the large call should have grown the workspace"
    del ws0
    sentinels = [torch.full((1 << 16,), 7, dtype=torch.uint8, device=gpu) for _ in range(16)]
    for i in range(3):
        y.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {i}"
        assert all(bool((t == 7).all()) for t in sentinels), f"replay {i} wrote into new memory"
