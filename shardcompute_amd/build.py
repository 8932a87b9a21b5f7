"""Builds libshardcompute_hip.so in-tree with hipcc for gfx950.

    python -m shardcompute_amd.build            # compile (always)

The library is a plain C-ABI shared object (no torch or Python headers), so it
can be bound from ctypes, cgo, JNI or N-API alike.  Object files are built in
parallel and linked into ``shardcompute_amd/libshardcompute_hip.so``.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD_DIR = os.path.join(PKG, "_build")
LIB_PATH = os.path.join(PKG, "libshardcompute_hip.so")
ARCH = os.environ.get("SC_OFFLOAD_ARCH", "gfx950")

SOURCES = ["abi.hip", "qgemv_dma.hip", "qgemv_m1.hip", "qgemv16.hip", "qgemv.hip", "qgemm.hip", "qgemm_band.hip", "gather.hip", "quant.hip", "decode.hip", "attn_prefill.hip", "decode_step.hip", "act.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # packed-fp32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]

# per-source additions: the prefill attention kernel keeps its MFMA accumulators in
# VGPRs (it rescales them in place every few blocks; in AGPRs each block would copy
# them to VGPRs and back)
EXTRA_FLAGS = {
    "attn_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")
    return path


def _compile(src):
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj, r.stderr


def build(verbose=False):
    os.makedirs(BUILD_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        results = list(ex.map(_compile, SOURCES))
    objs = [o for o, _ in results]
    if verbose:
        for _, err in results:
            warn = "\n".join(l for l in err.splitlines() if "packed-fp32-ops" not in l)
            if warn.strip():
                print(warn, file=sys.stderr)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
