"""The C ABI library loads and exports every symbol include/glorcq_hip.h declares
(no compute calls: runs without a GPU), and the host-side checks of the
boundary behave like the reference's TORCH_CHECK contract."""

import ctypes
import os
import re
import subprocess

import pytest

from glorcq_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "glorcq_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(glq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_entry_points():
    syms = declared_symbols()
    for need in ["glq_gemv_lora", "glq_gemv_lora_batched", "glq_unpack_codes",
                 "glq_dequant_weight", "glq_pack_codes", "glq_last_error"]:
        assert need in syms


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} declared but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_exported_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (glq_\w+)$", out, flags=re.M))
    assert set(declared_symbols()) <= exported


def test_version_and_workspace_sizes(lib):
    assert lib.glq_version() >= 100
    a = lib.glq_gemv_workspace_bytes(1, 1, 2048, 1408, 64)
    b = lib.glq_gemv_workspace_bytes(4, 1, 2048, 1408, 64)
    assert 0 < a < b
    assert lib.glq_gemv_workspace_bytes(1, 1, 2048, 1408, 0) < a
    assert lib.glq_gemv_workspace_bytes(-1, 1, 1, 1, 1) == -1


def test_argument_checks_raise_before_any_launch(lib):
    """Invalid arguments are rejected on the host (no device pointer is
    touched), mirroring gptq_matmul.cu:232-267; empty work is a no-op
    (gptq_matmul.cu:271-276)."""
    nul = None
    # bits
    rc = lib.glq_gemv_lora(1 << 12, 1, 2048, 1408, 1 << 12, 3, 1 << 12, 1 << 12, 128, 0,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"bits" in lib.glq_last_error()
    # M > 16
    rc = lib.glq_gemv_lora(1 << 12, 17, 2048, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 128, 0,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"M" in lib.glq_last_error()
    # group 64 on a row too long for the lane kernel (the one kernel that takes
    # groups below 128 codes)
    rc = lib.glq_gemv_lora(1 << 12, 1, 16384, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 64, 0,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"group" in lib.glq_last_error()
    # group not a whole number of 16-byte pieces (64 codes at 2 bits)
    rc = lib.glq_gemv_lora(1 << 12, 1, 2048, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 32, 0,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"group" in lib.glq_last_error()
    # K not a whole number of pieces (4-bit: 32 codes)
    rc = lib.glq_gemv_lora(1 << 12, 1, 80, 64, 1 << 12, 4, 1 << 12, 1 << 12, 16, 0,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"K=80" in lib.glq_last_error()
    # code format
    rc = lib.glq_gemv_lora(1 << 12, 1, 2048, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 128, 3,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"sym" in lib.glq_last_error()
    rc = lib.glq_gemm_lora(1 << 12, 64, 2048, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 128, 3,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"sym" in lib.glq_last_error()
    # signed codes with zero-points need the zero-points
    rc = lib.glq_gemv_lora(1 << 12, 1, 2048, 1408, 1 << 12, 2, 1 << 12, nul, 128, 2,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"null" in lib.glq_last_error()
    # workspace too small (two token rows: the x U partials need one; one row
    # forms x U inside its launch)
    rc = lib.glq_gemv_lora(1 << 12, 2, 2048, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 128, 0,
                           1 << 12, 1 << 12, 64, nul, nul, 1 << 12, 1 << 12, 16, nul)
    assert rc == 1 and b"workspace" in lib.glq_last_error()
    # misaligned x
    rc = lib.glq_gemv_lora((1 << 12) + 2, 1, 2048, 1408, 1 << 12, 2, 1 << 12, 1 << 12, 128, 0,
                           nul, nul, 0, nul, nul, 1 << 12, 1 << 12, 1 << 20, nul)
    assert rc == 1 and b"aligned" in lib.glq_last_error()
    # empty work: success, nothing launched
    assert lib.glq_gemv_lora(nul, 0, 2048, 1408, nul, 2, nul, nul, 128, 0, nul, nul, 0, nul,
                             nul, nul, nul, 0, nul) == 0
    assert lib.glq_unpack_codes(nul, 0, 64, 2, 0, nul, nul) == 0
    assert lib.glq_unpack_codes(nul, 4, 63, 2, 0, nul, nul) == 1


def test_decoder_entry_points_check_arguments(lib):
    """The decoder-layer entry points reject bad shapes on the host; empty
    work is a no-op."""
    nul, p = None, 1 << 12
    assert lib.glq_rmsnorm(p, nul, p, 4, 2050, 1e-6, p, nul, nul) == 1
    assert b"multiple of 8" in lib.glq_last_error()
    assert lib.glq_rmsnorm(p, nul, p, 4, 16384, 1e-6, p, nul, nul) == 1
    assert lib.glq_rmsnorm(p + 2, nul, p, 4, 2048, 1e-6, p, nul, nul) == 1
    assert b"aligned" in lib.glq_last_error()
    assert lib.glq_rmsnorm(p, p, p, 4, 2048, 1e-6, p, nul, nul) == 1  # residual_out missing
    assert lib.glq_rmsnorm(nul, nul, nul, 0, 2048, 1e-6, nul, nul, nul) == 0
    args = [p, p, p, 1, 32, 4, 128, 4096, 0, 512, p, p, 1e-6, p, p, 0, p, p, p, 640, p, p, nul]
    bad = list(args); bad[6] = 64                       # head_dim
    assert lib.glq_qk_norm_rope(*bad) == 1 and b"head_dim" in lib.glq_last_error()
    bad = list(args); bad[5] = 5                        # 32 % 5
    assert lib.glq_qk_norm_rope(*bad) == 1
    bad = list(args); bad[7] = 2048                     # q_stride < heads * 128
    assert lib.glq_qk_norm_rope(*bad) == 1
    bad = list(args); bad[8] = 384                      # item rows not dividing 4096
    assert lib.glq_qk_norm_rope(*bad) == 1 and b"q_item_rows" in lib.glq_last_error()
    bad = list(args); bad[3] = 0
    assert lib.glq_qk_norm_rope(*bad) == 0
    n = lib.glq_decode_attention_workspace_bytes(2, 32, 4, 640)
    assert n == 4 * 2 * 32 * 5 * 132 + 256  # (m, l, pad, o) per split, then the counters
    aargs = [p, p, p, 2, 32, 4, 128, 640, p, 0.088, nul, p, 1 << 16, n, nul]
    bad = list(aargs); bad[5] = 2                       # 16 q heads per KV head
    assert lib.glq_decode_attention(*bad) == 1 and b"q heads" in lib.glq_last_error()
    bad = list(aargs); bad[13] = n - 1                  # workspace too small
    assert lib.glq_decode_attention(*bad) == 1 and b"workspace" in lib.glq_last_error()
    bad = list(aargs); bad[0] = p + 8                   # q not 16-byte aligned
    assert lib.glq_decode_attention(*bad) == 1
    bad = list(aargs); bad[3] = 0
    assert lib.glq_decode_attention(*bad) == 0


def test_turbo_moe_entry_points_check_arguments(lib):
    """The pieces of a TurboQuant-expert MoE step reject bad shapes on the
    host, before any launch; empty work is a no-op."""
    nul, p = None, 1 << 12
    n = lib.glq_moe_route_workspace_bytes(4, 60)
    assert n == 4 * 64 + 2 * 4 * 61
    assert lib.glq_moe_route_workspace_bytes(0, 60) == -1
    rargs = [p, p, nul, 4, 2048, 60, 4, 0, p, p, p, nul, p, n, nul]
    bad = list(rargs); bad[6] = 0                        # top_k
    assert lib.glq_moe_route(*bad) == 1 and b"top_k" in lib.glq_last_error()
    bad = list(rargs); bad[4] = 8192                     # hidden past the router's 4096
    assert lib.glq_moe_route(*bad) == 1 and b"hidden" in lib.glq_last_error()
    bad = list(rargs); bad[5] = 300                      # experts
    assert lib.glq_moe_route(*bad) == 1
    bad = list(rargs); bad[13] = n - 1                   # workspace too small
    assert lib.glq_moe_route(*bad) == 1 and b"workspace" in lib.glq_last_error()
    bad = list(rargs); bad[0] = p + 2                    # h not 16-byte aligned
    assert lib.glq_moe_route(*bad) == 1
    targs = [16, 4, p, 2048, 1408, 60, p, p, p, p, p, p, 4, 16, p, 64, nul, nul, p, nul]
    bad = list(targs); bad[3] = 2000                     # K not a multiple of 64
    assert lib.glq_turbo_moe_gemv(*bad) == 1 and b"multiple of 64" in lib.glq_last_error()
    bad = list(targs); bad[15] = 60                      # rank not a multiple of 8
    assert lib.glq_turbo_moe_gemv(*bad) == 1 and b"rank" in lib.glq_last_error()
    bad = list(targs); bad[10] = nul                     # SV without xU
    assert lib.glq_turbo_moe_gemv(*bad) == 1
    bad = list(targs); bad[12] = 0                       # a cluster table without its rows
    assert lib.glq_turbo_moe_gemv(*bad) == 1
    bad = list(targs); bad[1] = 0                        # x_div
    assert lib.glq_turbo_moe_gemv(*bad) == 1
    bad = list(targs); bad[0] = 0
    assert lib.glq_turbo_moe_gemv(*bad) == 0
    largs = [16, p, 1408, p, 4, 64, p, 60, p, p, p, 1 << 20, nul]
    bad = list(largs); bad[5] = 60                       # rank
    assert lib.glq_lowrank_xu_routed(*bad) == 1 and b"rank" in lib.glq_last_error()
    bad = list(largs); bad[11] = 16                      # workspace too small
    assert lib.glq_lowrank_xu_routed(*bad) == 1 and b"workspace" in lib.glq_last_error()
    bad = list(largs); bad[8] = nul                      # no cluster table
    assert lib.glq_lowrank_xu_routed(*bad) == 1
    bad = list(largs); bad[0] = 0
    assert lib.glq_lowrank_xu_routed(*bad) == 0
    assert lib.glq_moe_combine(p, p, nul, nul, nul, 4, 2048, 17, p, nul) == 1  # top_k
    assert lib.glq_moe_combine(p, p, p, nul, nul, 4, 2048, 4, p, nul) == 1  # shared, no gate
    assert lib.glq_moe_combine(nul, nul, nul, nul, nul, 0, 2048, 4, nul, nul) == 0
    assert lib.glq_swiglu(nul, p, 16, p, nul) == 1
    assert lib.glq_swiglu(nul, nul, 0, nul, nul) == 0


def test_python_boundary_rejects_cpu_tensors():
    import torch

    from glorcq_amd import kernels

    x = torch.zeros(1, 128, dtype=torch.float16)
    codes = torch.zeros(16, 8, dtype=torch.int32)
    s = torch.zeros(16, 1, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU"):
        kernels.packed_dequant_matmul_fused(x, codes, s, s, 2, 128)
    assert kernels.is_cuda_available() is False


def test_gptq_signature_range_checks_codes():
    """gptq_dequant_matmul_fused takes the reference's (N, K) integer codes;
    codes no 4-bit container holds raise before any device work (the
    reference would wrap them in its int8 cast)."""
    import torch

    from glorcq_amd import kernels

    x = torch.zeros(1, 128, dtype=torch.float32)
    s = torch.ones(16, 1, dtype=torch.float16)
    q = torch.zeros(16, 128, dtype=torch.int32)
    q[3, 5] = 16                                   # asymmetric: above 0..15
    with pytest.raises(RuntimeError, match=r"span \[0, 16\]"):
        kernels.gptq_dequant_matmul_fused(x, q, s, s, 128, False)
    q[3, 5] = -9                                   # signed: below -8
    with pytest.raises(RuntimeError, match="span"):
        kernels.gptq_dequant_matmul_fused(x, q, s, s, 128, False)
    q[3, 5] = 8                                    # symmetric: above 7
    with pytest.raises(RuntimeError, match="symmetric codes span"):
        kernels.gptq_dequant_matmul_fused(x, q, s, None, 128, True)
    q[3, 5] = 2                                    # a 2-bit container asked for [-2, 2]
    q[4, 5] = -2
    with pytest.raises(RuntimeError, match="2-bit"):
        kernels.gptq_dequant_matmul_fused(x, q, s, s, 128, False, bits=2)
    with pytest.raises(RuntimeError, match="2 or 4"):
        kernels.gptq_dequant_matmul_fused(x, q, s, s, 128, False, bits=3)
    # in range: the pack is the first device step
    with pytest.raises(RuntimeError, match="GPU"):
        kernels.gptq_dequant_matmul_fused(x, q, s, s, 128, False)
    with pytest.raises(RuntimeError, match="sym must be"):
        kernels._sym_mode(3)


def test_batched_checks_zeros_shape_for_signed_codes_with_zeros(monkeypatch):
    """Code format sym=2 (signed codes with zero-points) reads the zero-points,
    so packed_dequant_matmul_batched checks their shape as for unsigned codes,
    before any library call."""
    import torch

    from glorcq_amd import kernels

    def dtype_only(t, name, dtype=None):
        if dtype is not None and t.dtype != dtype:
            raise RuntimeError(f"{name} must be {dtype}")

    def no_library():
        raise AssertionError("the library was reached")

    monkeypatch.setattr(kernels, "_require", dtype_only)
    monkeypatch.setattr(kernels._lib, "load", no_library)
    E, M, K, N = 2, 1, 256, 16
    x = torch.zeros(E, M, K, dtype=torch.float16)
    codes = torch.zeros(E, N, K * 2 // 32, dtype=torch.int32)
    s = torch.ones(E, N, K // 128, dtype=torch.float16)
    bad = torch.zeros(E, N, 1, dtype=torch.float16)
    for sym in (0, 2):
        with pytest.raises(RuntimeError, match="zeros must be"):
            kernels.packed_dequant_matmul_batched(x, codes, s, bad, 2, 128, sym=sym)
        with pytest.raises(RuntimeError, match="zeros required"):
            kernels.packed_dequant_matmul_batched(x, codes, s, None, 2, 128, sym=sym)


def test_gptq_signature_refuses_unprepared_codes_under_capture(monkeypatch):
    """Under graph capture the reference-signature op cannot range-check codes
    it has not seen (that reads back to the host): it raises a clear error
    before any device work instead of failing inside the capture."""
    import torch

    from glorcq_amd import kernels

    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    x = torch.zeros(1, 128, dtype=torch.float16)
    s = torch.ones(16, 1, dtype=torch.float16)
    q = torch.zeros(16, 128, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="not prepared before graph capture"):
        kernels.gptq_dequant_matmul_fused(x, q, s, s, 128, False)
