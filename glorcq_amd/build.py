"""Builds libglorcq_hip.so (all HIP sources under csrc/) for gfx950 with hipcc.

Usage: python -m glorcq_amd.build   (or glorcq_amd.build.build_library()).
The library is written in-tree (glorcq_amd/lib/) so it travels with the source
tree to the GPU host; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libglorcq_hip.so"
ARCH = os.environ.get("GLQ_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: the device pass may not emit packed fp32 VALU ops
# (v_pk_add/mul/fma_f32).  hipcc hands the flag to the host pass too, which
# warns that x86 has no such feature; the device pass honours it, and
# check_no_packed_fp32() verifies every built code object after the link.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (need ROCm)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build_library(verbose: bool = True, jobs: int = 8) -> Path:
    """Compiles every csrc/*.hip to an object, then links the shared library."""
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objs = []
    for src in sources():
        obj = obj_dir / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print("[glorcq_amd.build]", " ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        if len(procs) >= jobs:
            _drain(procs)
    _drain(procs)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print("[glorcq_amd.build]", " ".join(cmd), flush=True)
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"link failed:\n{out.stdout}")
    os.replace(tmp, LIB_PATH)
    check_no_packed_fp32(objs, verbose=verbose)
    return LIB_PATH


PACKED_FP32 = ("v_pk_add_f32", "v_pk_mul_f32", "v_pk_fma_f32")


def check_no_packed_fp32(objs, verbose: bool = True) -> None:
    """Disassembles the gfx950 code object of each built object file and
    fails the build if it holds a packed fp32 VALU instruction."""
    llvm = Path("/opt/rocm/llvm/bin")
    tools = [llvm / t for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")]
    if not all(t.exists() for t in tools):
        print("[glorcq_amd.build] LLVM tools missing: packed-fp32 check skipped", flush=True)
        return
    objcopy, bundler, objdump = map(str, tools)
    found = []
    checked = 0
    with tempfile.TemporaryDirectory() as tmpd:
        for obj in objs:
            fat = Path(tmpd) / (obj.stem + ".fatbin")
            co = Path(tmpd) / (obj.stem + ".co")
            dump = subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", str(obj),
                                   str(Path(tmpd) / "discard.o")], stdout=subprocess.PIPE,
                                  stderr=subprocess.STDOUT, text=True)
            if dump.returncode != 0:
                if "not found" in dump.stdout:
                    continue  # host code only
                raise RuntimeError(f"{obj.name}: {dump.stdout}")
            checked += 1
            subprocess.run([bundler, "--unbundle", "--type=o", f"--input={fat}",
                            f"--targets=hipv4-amdgcn-amd-amdhsa--{ARCH}", f"--output={co}"],
                           check=True)
            dis = subprocess.run([objdump, "-d", str(co)], check=True, stdout=subprocess.PIPE,
                                 text=True).stdout
            n = sum(dis.count(op) for op in PACKED_FP32)
            if n:
                found.append(f"{obj.name}: {n}")
    if found:
        raise RuntimeError("packed fp32 VALU instructions in the device code: " + ", ".join(found))
    if verbose:
        print(f"[glorcq_amd.build] no packed fp32 VALU instructions in {checked} code objects",
              flush=True)


def _drain(procs):
    errs = []
    for src, p in procs:
        out, _ = p.communicate()
        text = out.decode(errors="replace")
        if p.returncode != 0:
            errs.append(f"{src.name}:\n{text}")
        elif text.strip():
            print(text, flush=True)
    procs.clear()
    if errs:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errs))


if __name__ == "__main__":
    path = build_library()
    print(path)
    sys.exit(0)
