"""Build libschedpd.so (the HIP kernels + C ABI) for gfx950, in-tree.

    python sched-pass_amd/build_lib.py        # or build() from Python

Each .hip translation unit compiles in its own hipcc process (in parallel),
then hipcc links the shared library next to this file. Packed-FP32 VALU
instructions are disabled for all device code.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libschedpd.so")
SOURCES = ["sched_rt.hip", "paged_decode.hip", "probe.hip", "kv_append.hip", "staging.hip",
           # the decode kernels, one instantiation group per unit (kernel_set.h)
           "kernels_bf16_page16.hip", "kernels_bf16_pageblocks.hip", "kernels_fp8.hip", "kernels_fp8_tokmajor.hip",
           "kernels_f16.hip", "kernels_f16_pageblocks.hip", "kernels_valu.hip",
           "kernels_wave.hip", "kernels_wave_groups.hip"]
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the online-softmax rescale multiplies them
    # on the VALU, which otherwise copies them out of AGPRs every page.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(ROOT, "include"),
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise.
    err = "\n".join(l for l in r.stderr.splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = False) -> str:
    """Compile every source and link libschedpd.so; returns its path."""
    os.makedirs(OBJ, exist_ok=True)
    jobs = []
    for src in SOURCES:
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        jobs.append((obj, [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]))
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        list(ex.map(lambda j: (_run(j[1]), verbose and print(" ".join(j[1]))), jobs))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
          *[o for o, _ in jobs]])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
