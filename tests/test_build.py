"""The build's packed-fp32 guard: a kernel compiled without the flag that
forbids packed fp32 VALU ops holds one (hipcc -O3 pairs two fp32 FMAs of a
float2), and check_no_packed_fp32 must reject it; the same kernel with the
build's flags must pass."""

import shutil
import subprocess
from pathlib import Path

import pytest

from glorcq_amd import build

KERNEL = r'''
#include <hip/hip_runtime.h>
__global__ void pk(const float2* __restrict__ a, const float2* __restrict__ b,
                   float2* __restrict__ c, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    float2 x = a[i], y = b[i];
    c[i] = make_float2(x.x * y.x + x.x, x.y * y.y + x.y);
  }
}
'''


@pytest.mark.skipif(not (shutil.which("hipcc") or Path("/opt/rocm/bin/hipcc").exists()),
                    reason="hipcc not installed")
def test_packed_fp32_guard(tmp_path):
    src = tmp_path / "pk.hip"
    src.write_text(KERNEL)
    cc = build.hipcc()
    plain = tmp_path / "plain.o"
    subprocess.run([cc, f"--offload-arch={build.ARCH}", "-O3", "-c", str(src), "-o", str(plain)],
                   check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    with pytest.raises(RuntimeError, match="packed fp32"):
        build.check_no_packed_fp32([plain], verbose=False)
    guarded = tmp_path / "guarded.o"
    subprocess.run([cc, *build.HIPCC_FLAGS, "-c", str(src), "-o", str(guarded)], check=True,
                   stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    build.check_no_packed_fp32([guarded], verbose=False)
