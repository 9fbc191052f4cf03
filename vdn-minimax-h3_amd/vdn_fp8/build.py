"""Builds libvdnfp8.so (the HIP kernels and their C ABI) for gfx950 with hipcc.

    python vdn-minimax-h3_amd/vdn_fp8/build.py        # or vdn_fp8.build.build()

Objects are compiled in a temporary directory (in parallel) and only the shared
library lands next to this file, where the ctypes loader looks for it.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)                      # vdn-minimax-h3_amd/
_CSRC = os.path.join(_ROOT, "csrc")
_INCLUDE = os.path.join(os.path.dirname(_ROOT), "include")
LIB_NAME = "libvdnfp8.so"
LIB_PATH = os.path.join(_PKG, LIB_NAME)

SOURCES = ["capi.hip", "quantize.hip", "lora_requant.hip", "gemm.hip", "qk_prep.hip", "block_ops.hip"]

# -ffp-contract=off: the quantizers' binary32 arithmetic is bit-exact only as
# written (explicit fma where one is meant). Packed fp32 instructions are kept
# out of the device code. No fast-math: the row scale needs IEEE division.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# Per-source additions. The LoRA kernels read every MFMA result with VALU code:
# accumulating in VGPRs (rather than AGPRs) saves one copy per element.
EXTRA_FLAGS = {"lora_requant.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the fp8 library needs ROCm's hipcc to build")


def build(verbose=False):
    """Compile every source for gfx950 and link libvdnfp8.so. Returns its path."""
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="vdnfp8_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.splitext(src)[0] + ".o")
            cmd = [cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-I", _INCLUDE, "-I", _CSRC, "-c",
                   os.path.join(_CSRC, src), "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
            if verbose and r.stderr:
                print(r.stderr, file=sys.stderr)
            return obj

        workers = min(len(SOURCES), max(1, (os.cpu_count() or 1)))
        with concurrent.futures.ThreadPoolExecutor(workers) as ex:
            objs = list(ex.map(compile_one, SOURCES))
        tmp_lib = os.path.join(tmp, LIB_NAME)
        r = subprocess.run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp_lib, *objs],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"linking {LIB_NAME} failed:\n{r.stderr}")
        # Copy next to the target, then rename: a process that already mapped
        # the old library keeps a consistent file.
        shutil.copyfile(tmp_lib, LIB_PATH + ".tmp")
        os.replace(LIB_PATH + ".tmp", LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
