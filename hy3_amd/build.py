"""Build libhy3x.so (HIP, gfx950) in-tree with hipcc.

    python -m hy3_amd.build        # or hy3_amd.build.build()

Every .hip under hy3_amd/csrc is compiled for gfx950 and linked into
hy3_amd/libhy3x.so. Flags:
  -fhip-fp32-correctly-rounded-divide-sqrt  the routing contract needs IEEE
                                            fp32 division and sqrt;
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                            no packed-fp32 instructions are
                                            generated (they are unreliable on
                                            the target machines);
  -mllvm -amdgpu-mfma-vgpr-form             MFMA accumulators in VGPRs (no
                                            copies between accumulation and
                                            vector registers around the
                                            per-block scale FMAs).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libhy3x.so")
BUILD = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


# Per-source additions: the narrow and wide MFMA tile kernels and the
# single-token router launch schedule with LLVM's iterative-ILP strategy
# (measured: 512 tokens gate/up 350.1 -> 347.6 us, down 200.6 -> 198.3; 32
# tokens 164.1 -> 163.1 and 95.5 -> 94.7; decode 29.30 -> 29.06 us with the
# router launch alone). The 128-token tiles, the decode expert kernels and
# the multi-token router measured slower with it (1250 -> 1336 us; 29.3 ->
# 30.4 us; router stage at 512 tokens 42.8 -> 45.3 us), so they keep the
# default scheduler.
# The decode expert kernels (hy3x_gemv.hip) schedule with the AMDGPU
# register-pressure trackers (decode 29.41 -> 29.26 us; other scheduler
# strategies, larger memory clauses and wave priorities measured slower).
ILP = ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]
FILE_FLAGS = {
    "hy3x_mfma.hip": ILP,
    "hy3x_mfma_wide.hip": ILP,
    "hy3x_route_decode.hip": ILP,
    "hy3x_gemv.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers"],
}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", OUT + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(OUT + ".tmp", OUT)
    if verbose:
        print("built", OUT)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
