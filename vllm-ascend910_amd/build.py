"""Build recipe for the gfx950 HIP library behind the C ABI (include/w4a8_amd.h).

Compiles every ``csrc/*.hip`` with hipcc for gfx950 only and links them into
``_lib/libw4a8_amd.so`` inside this package, so the built library travels with
the source tree.  Every call recompiles (kernel headers are real dependencies;
a stale library is never reused).

    python vllm-ascend910_amd/build.py        # or __graft_entry__.build()
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "_lib"
LIBNAME = "libw4a8_amd.so"
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for all device code on this platform;
# hipcc's host pass warns that it does not know the feature, which is harmless.
# MFMA results stay in ordinary VGPRs: the folds read every accumulator with
# VALU instructions, which cannot address AGPRs (each element would first need
# a v_accvgpr_read).
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-amdgpu-mfma-vgpr-form=1"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
                "-Wno-unused-function", "-Wno-unused-variable"]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise FileNotFoundError("hipcc not found; the W4A8 library needs ROCm's hipcc")
    return exe


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # Filter the known host-pass warning about the packed-fp32 feature.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile and link the library; returns its path."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        list(ex.map(lambda so: _compile(*so), zip(srcs, objs)))
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    # A kernel whose host launch stub the compiler dropped links fine and
    # fails only when the library is loaded: refuse such a build here.
    nm = shutil.which("nm")
    if nm:
        syms = subprocess.run([nm, "-D", "--undefined-only", str(tmp)], capture_output=True, text=True).stdout
        missing = [l.split()[-1] for l in syms.splitlines() if "__device_stub__" in l]
        if missing:
            raise RuntimeError(f"undefined kernel launch stubs in {tmp.name}: {missing[:4]}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
