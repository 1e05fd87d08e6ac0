"""Build libdsv41.so (all HIP kernels + the C ABI) for gfx950 with hipcc.

    python deepseek-v41-mlx_amd/build.py            # -> deepseek-v41-mlx_amd/dsv41/libdsv41.so

Each .hip source compiles to an object in parallel, then one shared library is linked.
Packed-fp32 instructions are disabled for every device compile.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "dsv41", "libdsv41.so")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


# -packed-fp32-ops: no v_pk_*_f32 generation. -amdgpu-mfma-vgpr-form: MFMA accumulators in
# VGPRs -- with a one-workgroup-per-CU LDS footprint the default heuristic parks them in AGPRs
# and copies them around every VALU use.
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-mfma-vgpr-form"]


def _compile(src: str, obj: str) -> None:
    cmd = [hipcc(), *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")


def build(verbose: bool = True) -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with tempfile.TemporaryDirectory(prefix="dsv41_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            list(ex.map(_compile, srcs, objs))
        tmp_out = OUT + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        os.replace(tmp_out, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
