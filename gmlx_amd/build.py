"""Build libgmlx_amd.so (gfx950) in-tree with hipcc.

    python -m gmlx_amd.build            # compile every csrc/*.hip, link the .so
    python -m gmlx_amd.build --check    # also print the kernels' VGPR / scratch use

Each translation unit is compiled to an object in parallel, then linked into
gmlx_amd/libgmlx_amd.so, which travels with the source tree.  All device code
is compiled without floating-point contraction (the bit-exact dequant relies
on it) and without packed-fp32 instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgmlx_amd.so")
ARCH = os.environ.get("GMLX_AMD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src, extra=()):
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name: harmless
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, err


def build(verbose=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def resource_usage():
    """VGPR / AGPR / scratch / LDS per kernel, from the compiler's remarks."""
    out = {}
    for src in sources():
        r = subprocess.run([HIPCC, *FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src,
                            "-o", os.devnull, "--offload-device-only"],
                           capture_output=True, text=True)
        cur = None
        for line in r.stderr.splitlines():
            if "Function Name:" in line:
                cur = line.split("Function Name:")[1].strip()
                out[cur] = {}
            elif cur and "remark:" in line and ":" in line.split("remark:")[1]:
                k, v = line.split("remark:")[1].rsplit(":", 1)
                out[cur][k.strip()] = v.strip()
    return out


if __name__ == "__main__":
    print(build(verbose=True))
    if "--check" in sys.argv:
        for name, info in resource_usage().items():
            print(name[:90], {k: info.get(k) for k in ("VGPRs", "AGPRs", "ScratchSize [bytes/lane]",
                                                      "Occupancy [waves/SIMD]", "LDS Size [bytes/block]")})
