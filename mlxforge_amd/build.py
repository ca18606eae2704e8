"""Build recipe for the HIP sampler library (gfx950).

Produces ``mlxforge_amd/libmlxf_sampler.so`` in-tree from
``mlxforge_amd/csrc/sampler.hip`` (host side), ``sampler_{f32,bf16,f16}.hip``
(one logits dtype's kernels each), ``penalties.hip``, ``uniforms.hip``,
``mask.hip`` and ``filter.hip``, compiled in parallel
with hipcc, and the C++
known-answer test
driver ``mlxforge_amd/sampler_kat`` (tests/cpp/sampler_kat.cpp) that exercises
the C++ host wrapper (mlxforge_amd/include/mlxforge_amd/sampler.hpp).

Flags:
  -ffp-contract=off   every fp32 operation stays IEEE-rounded, so
                      z' = round(z / T) is bit-identical to the CPU oracle;
                      division stays correctly rounded (HIP's default
                      -fhip-fp32-correctly-rounded-divide-sqrt).
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed-fp32 instructions are generated.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SRCS = [os.path.join(CSRC, f) for f in ("sampler.hip", "sampler_f32.hip", "sampler_bf16.hip", "sampler_f16.hip",
                                         "penalties.hip", "uniforms.hip", "mask.hip", "filter.hip")]
LIB = os.path.join(HERE, "libmlxf_sampler.so")
KAT_SRC = os.path.join(ROOT, "tests", "cpp", "sampler_kat.cpp")
KAT_BIN = os.path.join(HERE, "sampler_kat")
ARCH = os.environ.get("MLXF_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    _report(cmd, proc)


def _report(cmd, proc):
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line.
    noise = [l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l]
    if proc.returncode != 0:
        raise RuntimeError("build failed:\n" + " ".join(cmd) + "\n" + "\n".join(noise))
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build_lib() -> str:
    import tempfile
    objs, procs = [], []
    with tempfile.TemporaryDirectory() as tmpd:
        for src in SRCS:
            obj = os.path.join(tmpd, os.path.basename(src) + ".o")
            cmd = [hipcc(), *HIP_FLAGS, "-c", "-I", os.path.join(ROOT, "include"), "-o", obj, src]
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
            objs.append(obj)
        for cmd, pr in procs:
            out, err = pr.communicate()
            _report(cmd, subprocess.CompletedProcess(cmd, pr.returncode, out, err))
        tmp = LIB + ".tmp"
        _run([hipcc(), *HIP_FLAGS, "-shared", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_kat() -> str:
    """C++ known-answer driver over the C++ wrapper; links the built library."""
    # Host code only (no kernels): the system C++ compiler against the HIP
    # runtime headers and library.
    tmp = KAT_BIN + ".tmp"
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    _run([shutil.which("g++") or "g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(rocm, "include"), "-I", os.path.join(ROOT, "include"),
          "-I", os.path.join(HERE, "include"), "-o", tmp, KAT_SRC, LIB,
          "-L", os.path.join(rocm, "lib"), "-lamdhip64",
          f"-Wl,-rpath,{HERE}", f"-Wl,-rpath,{os.path.join(rocm, 'lib')}"])
    os.replace(tmp, KAT_BIN)
    return KAT_BIN


def build_all() -> None:
    build_lib()
    if os.path.exists(KAT_SRC):
        build_kat()


if __name__ == "__main__":
    build_all()
    print(LIB)
