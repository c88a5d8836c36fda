"""Build the gfx950 HIP library ``libtierkv_hip.so`` in-tree.

``python -m paged_tierkv_amd.build`` (or ``__graft_entry__.build()``)
compiles every HIP source for gfx950 with hipcc and the host-only C++ with
g++, then links one shared library next to this file.  Objects go to
``paged_tierkv_amd/_build``.  The library exports only the C ABI declared in
``include/tierkv_hip.h``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libtierkv_hip.so"
# bench.py's HBM ceiling measurement (its own library, outside the C ABI).
CEILING_LIB = PKG / "libtierkv_ceiling.so"
ARCH = os.environ.get("TIERKV_OFFLOAD_ARCH", "gfx950")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", os.path.join(ROCM, "bin", "hipcc"))

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed fp32 VALU ops are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
]

# Per-source extra flags: the codecs must not contract mul+add into FMA.
HIP_SOURCES = {
    # The tier branches of the tile loader store to different elements of the
    # same register arrays; LLVM's common-store sinking would merge them into
    # one dynamically indexed store and push the tiles to scratch memory.
    # The decode kernel's leading scalar arguments (table row pointers, query,
    # geometry) are preloaded into SGPRs at wave launch, saving a kernarg
    # round trip before the table row can be read.  The atomic optimizer is
    # off: the kernel's atomics are already issued by one lane (tile hand-out,
    # arrival) or are rare (error bits), and its wave-reduction wrapper added
    # about ten instructions to every tile hand-out.
    "decode_attention.hip": ["-mllvm", "-simplifycfg-sink-common=false",
                             "-mllvm", "-amdgpu-kernarg-preload-count=9",
                             "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
    "quantize.hip": ["-ffp-contract=off"],
    "block_score.hip": ["-ffp-contract=off"],
    # The append kernel's leading arguments are preloaded (as the decode
    # kernel's); the other runtime kernels take a parameter block first.
    "runtime.hip": ["-ffp-contract=off", "-mllvm", "-amdgpu-kernarg-preload-count=8"],
    # MFMA accumulators in ordinary VGPRs: the logits are consumed by VALU
    # code right away, and accumulators in AGPRs cost a copy per element.
    "prefill_score.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}
CXX_SOURCES = ["block_manager.cpp"]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")
    return proc.stdout


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    include = ["-I", str(PKG.parent / "include")]
    procs = []
    objs = []
    for src, extra in HIP_SOURCES.items():
        obj = BUILD / (src + ".o")
        cmd = [HIPCC, *HIP_FLAGS, *extra, *include, "-c", str(CSRC / src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    for src in CXX_SOURCES:
        obj = BUILD / (src + ".o")
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", *include,
               "-c", str(CSRC / src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    errors = []
    for cmd, proc in procs:
        out, _ = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"$ {' '.join(cmd)}\n{out}")
        elif verbose and out.strip():
            print(out)
    if errors:
        raise RuntimeError("HIP build failed:\n" + "\n".join(errors))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    tmp = CEILING_LIB.with_suffix(".so.tmp")
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", str(tmp), str(CSRC / "ceiling.hip")])
    os.replace(tmp, CEILING_LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
