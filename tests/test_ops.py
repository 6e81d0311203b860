"""The torch.library operator layer (glorcq_amd.ops, namespace glorcq_hip): the
counterpart of the reference's custom ops with fake kernels
(inference/kernels/__init__.py:63-107).

CPU: every operator is registered, its fake kernel gives the real kernel's
output shape and dtype on meta tensors, torch.library.opcheck passes its schema,
fake-tensor and AOT-dispatch checks there, and Dynamo traces a GLoRCQLinear
and a MoE block into one graph (fullgraph) under fake tensors.
GPU (tests marked gpu): opcheck on device tensors (fake vs real outputs), and
torch.compile(fullgraph=True) of GLoRCQLinear.forward and of the MoE block
equals eager, bit for bit."""

import pytest
import torch
from torch.library import opcheck

import glorcq_amd  # noqa: F401  (registers the operators)
from glorcq_amd import format as fmt
from glorcq_amd.moe_block import GraphCompatibleMoeBlock
from glorcq_amd.quantized_linear import GLoRCQLinear

OPS = ["packed_dequant_matmul", "turbo_dequant_matmul", "lowrank_xu", "rht", "moe_decode",
       "moe_prefill"]


def meta(*shape, dtype=torch.float16):
    return torch.empty(*shape, dtype=dtype, device="meta")


def gptq_args(M=4, K=2048, N=1408, r=64, dev="meta"):
    mk = (lambda *s, dtype=torch.float16: torch.empty(*s, dtype=dtype, device=dev))
    return (mk(M, K), mk(N, K // 16, dtype=torch.int32), mk(N, K // 128), mk(N, K // 128), 2,
            128, False, mk(K, r), mk(N, r), None, None)


def test_operators_registered():
    for name in OPS:
        assert hasattr(torch.ops.glorcq_hip, name), name


def test_fake_kernels_on_meta():
    y = torch.ops.glorcq_hip.packed_dequant_matmul(*gptq_args())
    assert y.shape == (4, 1408) and y.dtype == torch.float16
    t = torch.ops.glorcq_hip.turbo_dequant_matmul(meta(3, 1024), meta(512, 256, dtype=torch.uint8),
                                                  meta(512, dtype=torch.float32),
                                                  meta(4, dtype=torch.float32), None, None, None)
    assert t.shape == (3, 512)
    a = torch.ops.glorcq_hip.lowrank_xu(meta(5, 2048), meta(3, 2048, 64))
    assert a.shape == (3, 5, 64)
    r = torch.ops.glorcq_hip.rht(meta(2, 256), meta(256, dtype=torch.float32), False, True)
    assert r.shape == (2, 256) and r.dtype == torch.float32
    with pytest.raises(RuntimeError, match="does not match K"):
        torch.ops.glorcq_hip.packed_dequant_matmul(meta(4, 1024), *gptq_args()[1:])


def test_opcheck_on_meta():
    r = opcheck(torch.ops.glorcq_hip.packed_dequant_matmul.default, gptq_args())
    assert all(v == "SUCCESS" for v in r.values()), r
    r = opcheck(torch.ops.glorcq_hip.lowrank_xu.default, (meta(5, 2048), meta(2048, 64)))
    assert all(v == "SUCCESS" for v in r.values()), r


def linear(dev, M=3, seed=11):
    p = fmt.make_linear(2048, 1408, bits=2, rank=64, M=M, seed=seed)
    from oracle import glorcq_oracle as O
    lin = GLoRCQLinear(2048, 1408)
    lin.load_gptq({"qweight_int": torch.from_numpy(O.unpack_codes(p.codes.numpy(), 2, 2048)),
                   "scales": p.scales, "zeros": p.zeros, "bits": 2, "groupsize": 128},
                  device=dev)
    lin.load_sv(p.U, p.SV, device=dev)
    return lin, p.x.to(dev)


def test_dynamo_traces_linear_fullgraph_on_fake_tensors():
    """Dynamo + AOT (aot_eager) trace GLoRCQLinear.forward into one graph with
    the fake kernel standing in (no device code runs: the weights are CPU
    tensors faked as their GPU shapes by the traced op)."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    lin, x = linear("cpu")
    with FakeTensorMode(allow_non_fake_inputs=True) as mode:
        fx = mode.from_tensor(x)
        lin.codes, lin.scales, lin.zeros, lin.U, lin.SV = (
            mode.from_tensor(t) for t in (lin.codes, lin.scales, lin.zeros, lin.U, lin.SV))
        gm, guards = torch._dynamo.export(lin.forward)(fx)
    names = [n.target for n in gm.graph.nodes if n.op == "call_function"]
    assert torch.ops.glorcq_hip.packed_dequant_matmul.default in names or \
        torch.ops.glorcq_hip.packed_dequant_matmul in names, names


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_opcheck_real_vs_fake(gpu):
    lin, x = linear(gpu)
    args = (x, lin.codes, lin.scales, lin.zeros, 2, 128, False, lin.U, lin.SV, None, None)
    r = opcheck(torch.ops.glorcq_hip.packed_dequant_matmul.default, args)
    assert all(v == "SUCCESS" for v in r.values()), r


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 5, 40])
def test_compile_linear_fullgraph_equals_eager(gpu, M):
    lin, x = linear(gpu, M=M, seed=12 + M)
    eager = lin(x)
    torch._dynamo.reset()
    compiled = torch.compile(lin.forward, fullgraph=True, backend="aot_eager")
    got = compiled(x)
    torch.cuda.synchronize()
    assert torch.equal(got, eager)


@pytest.mark.gpu
def test_compile_moe_block_fullgraph_equals_eager(gpu):
    p = fmt.make_moe(H=256, E=8, inter=384, top_k=2, n_clusters=3, rank=16, shared_inter=512,
                     B=4, seed=5)
    blk = GraphCompatibleMoeBlock.from_problem(p, gpu)
    h = p.h.reshape(1, 4, p.H).to(gpu)
    eager, el = blk(h)
    torch._dynamo.reset()
    compiled = torch.compile(blk.forward, fullgraph=True, backend="aot_eager")
    got, gl = compiled(h)
    torch.cuda.synchronize()
    assert torch.equal(got, eager) and torch.equal(gl, el)
