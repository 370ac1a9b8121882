"""Ahead-of-time build of libaetherkv.so for gfx950 (hipcc, in-tree).

Every source under ``csrc/`` is compiled in parallel with hipcc ``--offload-arch=gfx950`` and linked
into ``aetherkv/libaetherkv.so`` next to this file, so the library travels with the source tree.

Flags that matter for parity:
  -ffp-contract=off                              no silent FMA contraction (bit-exact codec)
  -fhip-fp32-correctly-rounded-divide-sqrt       IEEE division, as torch's fp32 `/`
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-fp32 VALU ops
  -mllvm -amdgpu-mfma-vgpr-form                  matrix-instruction results in ordinary VGPRs: otherwise
                                                 the compiler keeps some accumulators in AGPRs and copies
                                                 every result to VGPRs for the VALU that consumes it

Beside it, gcc builds ``aetherkv/_fastcall*.so`` from ``aetherkv/_fastcall.c``: CPython fast-call
functions over the same C ABI for the entry points called once per token (linked against
libaetherkv.so through $ORIGIN, so both share one loaded library), and hipcc builds
``aetherkv/libaetherkv_probe.so`` from ``probe/stream_probe.hip``: bench.py's streaming probe, kept
out of the product library.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent                      # deepseek-v4-codebase_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB = PKG / "libaetherkv.so"
OBJ_DIR = ROOT / "_build"

ARCH = os.environ.get("AETHERKV_ARCH", "gfx950")
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libaetherkv)")


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


# Per-source flags.  quant_attn_mfma.hip, sink_attention_mfma.hip: the split combines' scalar
# arguments arrive in registers at dispatch (their one memory round then does not wait for the
# argument block; byval struct arguments, as the other kernels there take, are not preloaded).
# Measured per kernel: it helps the combine (HCA decode) and left the codec kernels within noise or
# up to 1.7% slower, so it is not applied library-wide.
_PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
SOURCE_FLAGS = {
    "quant_attn_mfma.hip": _PRELOAD,
    "sink_attention_mfma.hip": _PRELOAD,
}


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.name + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, jobs: int = 8) -> Path:
    """Compile every HIP source and link libaetherkv.so (always rebuilds)."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(jobs, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libaetherkv.so", *map(str, objs), "-o",
           str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_fastcall()
    build_probe()
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


PROBE_SRC = ROOT / "probe" / "stream_probe.hip"
PROBE_LIB = PKG / "libaetherkv_probe.so"


def build_probe() -> Path:
    """hipcc the measurement probe into its own library (bench.py loads it; the product does not)."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *COMMON_FLAGS, "-shared", "-x", "hip", str(PROBE_SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


FASTCALL_SRC = PKG / "_fastcall.c"
FASTCALL_LIB = PKG / ("_fastcall" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))


def build_fastcall() -> Path:
    """gcc the CPython fast-call module over libaetherkv.so (next to it)."""
    tmp = FASTCALL_LIB.with_name(FASTCALL_LIB.name + ".tmp")
    cmd = ["gcc", "-shared", "-fPIC", "-O2", "-Wall", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
           str(FASTCALL_SRC), f"-L{PKG}", "-laetherkv", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"fast-call module build failed:\n{res.stderr}")
    os.replace(tmp, FASTCALL_LIB)
    return FASTCALL_LIB


if __name__ == "__main__":
    build(verbose=True)
