"""The allocation-free GEMV entry point (glq_gemv_lora_noalloc, C ABI) gives the
same bits as glq_gemv_lora with a caller workspace, on calls in a row (the
second a smaller multi-row input whose x*U partials reuse the scratch, so a
stale first-call scratch would show), and it rejects sizes beyond its static
scratch on the host."""

import pytest
import torch

from glorcq_amd import _lib
from glorcq_amd import format as fmt

pytestmark = pytest.mark.gpu


def _call_pair(lib, dev, p, stream):
    d = {k: getattr(p, k).to(dev) for k in ("codes", "scales", "zeros", "U", "SV", "x")}
    M, K, N, r = p.x.shape[0], p.K, p.N, p.rank
    y_ref = torch.empty(M, N, dtype=torch.float16, device=dev)
    y_new = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    nbytes = lib.glq_gemv_workspace_bytes(1, M, K, N, r)
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)  # counter words at zero
    args = (d["x"].data_ptr(), M, K, N, d["codes"].data_ptr(), p.bits, d["scales"].data_ptr(),
            d["zeros"].data_ptr(), p.group, 0, d["U"].data_ptr(), d["SV"].data_ptr(), r, None,
            None)
    _lib.check(lib.glq_gemv_lora(*args, y_ref.data_ptr(), ws.data_ptr(), ws.numel(), stream),
               "glq_gemv_lora")
    _lib.check(lib.glq_gemv_lora_noalloc(*args, y_new.data_ptr(), stream),
               "glq_gemv_lora_noalloc")
    torch.cuda.synchronize()
    return y_ref, y_new


def test_noalloc_matches_workspace_entry_point(gpu):
    lib = _lib.load()
    stream = _lib.stream_handle(gpu)
    # first call: config-1 down projection (K=1408) at M=8, rank 128, whose
    # x*U partials fill the static scratch; second: a smaller multi-row
    # problem (M=4, K=512, rank 64) whose partials reuse the same scratch
    # (a stale first-call partial would change its bits), in the token-tile
    # form whose in-launch x*U counters sit in the scratch's header, twice
    # (the first call must leave them zero); last: one token row twice and a
    # config-0 row, whose x*U jobs keep their counters and K-slice words in
    # the scratch's header (each call must leave them zero, or the next one
    # reads stale words)
    big = fmt.make_linear(1408, 2048, bits=2, rank=128, M=8, seed=71)
    small = fmt.make_linear(512, 640, bits=4, rank=64, M=4, seed=72)
    single = fmt.make_linear(512, 640, bits=4, rank=64, M=1, seed=73)
    config0 = fmt.make_linear(2048, 1408, bits=2, rank=64, M=1, seed=74)
    for p in (big, small, small, single, single, config0):
        print(f"noalloc case K={p.K} N={p.N} M={p.x.shape[0]} bits={p.bits} r={p.rank}",
              flush=True)
        y_ref, y_new = _call_pair(lib, gpu, p, stream)
        assert torch.equal(y_ref, y_new), f"K={p.K}: allocation-free output differs"


def test_noalloc_rejects_oversized_scratch(gpu):
    lib = _lib.load()
    cap = lib.glq_gemv_noalloc_max_scratch_bytes()
    assert cap == 4 << 20
    # M=16, rank 512 and K=65536 need 256 K-slices x 16 x 512 x 4 B = 8 MiB
    K, N, M, r = 65536, 64, 16, 512
    assert lib.glq_gemv_workspace_bytes(1, M, K, N, r) > cap
    fake = 1 << 20  # never dereferenced: the size check runs first
    rc = lib.glq_gemv_lora_noalloc(fake, M, K, N, fake, 2, fake, fake, 128, 0, fake, fake, r,
                                   None, None, fake, None)
    assert rc == 1 and b"static scratch" in lib.glq_last_error()
