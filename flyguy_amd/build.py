"""Build the flyguy MI355X library (flyguy_amd/libflyguy_core.so) with hipcc for gfx950.

    python -m flyguy_amd.build

The library is plain HIP C++ behind a C ABI (include/flyguy_core.h, include/flyguy_train.h); it links only the HIP
runtime, so ctypes loads it next to PyTorch in the same process and GPU context.  The teaching trainer's executable
(flyguy_amd/flyguy_train) is a one-line main over the library's ft_main, found next to it at run time.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "libflyguy_core.so"
EXE = PKG / "flyguy_train"
CPU_LIB = PKG / "libfly_infer.so"          # decisions on the host CPU (include/fly_infer.h): no HIP
SOURCES = [PKG / "csrc" / n for n in ("kernels.hip", "core.hip", "core16.hip", "readout.hip", "hop_api.hip", "half.hip", "train.hip", "probe.hip")]
HEADERS = [PKG / "csrc" / n for n in ("common.h", "kernels.h", "device.h", "core.h", "half.h")] + \
    [ROOT / "include" / "flyguy_core.h", ROOT / "include" / "flyguy_train.h", ROOT / "include" / "fly_infer.h"]
ARCH = os.environ.get("FLYGUY_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the flyguy library)")


def build(verbose: bool = False) -> Path:
    """Compile every source (always: the build check is that this succeeds) and link the shared library."""
    out_dir = PKG / "_build"
    out_dir.mkdir(exist_ok=True)
    flags = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-result",
             # packed fp32 instructions are left to nothing: code generation of ordinary float code only
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", str(ROOT / "include")]
    objs = []
    procs = []
    for src in SOURCES:
        obj = out_dir / (src.stem + ".o")
        cmd = [hipcc(), *flags, "-c", str(src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    for cmd, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{text}")
        if verbose and text.strip():
            print(text)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    tmp = EXE.with_suffix(".tmp")
    cmd = ["g++", "-O2", "-std=c++17", str(PKG / "csrc" / "flyguy_train_main.cpp"), "-o", str(tmp), f"-L{PKG}",
           "-lflyguy_core", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, EXE)
    tmp = CPU_LIB.with_suffix(".so.tmp")
    # float32 sums as written: no multiply-add contraction
    cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-pthread", "-Wall", "-ffp-contract=off",
           str(PKG / "csrc" / "infer_cpu.cpp"),
           "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CPU_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
