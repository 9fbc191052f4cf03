"""Builds libvdnfp8.so (the HIP kernels and their C ABI) for gfx950 with hipcc.

    python vdn-minimax-h3_amd/vdn_fp8/build.py        # or vdn_fp8.build.build()

Objects are compiled in a temporary directory (in parallel) and only the shared
library lands next to this file, where the ctypes loader looks for it.

The library carries the sha256 of every source it was built from (and of the flags, and
the compiler's identity), returned by vdn_fp8_build_info(); the loader compares it with
the sources on disk (and the installed hipcc, where there is one) and refuses a library
built from other sources or by another compiler, so a stale build cannot stand in for
the current kernels.
"""
import concurrent.futures
import hashlib
import json
import os
import shutil
import subprocess
import sys
import tempfile

_PKG = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_PKG)                      # vdn-minimax-h3_amd/
CSRC = os.path.join(_ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(_ROOT), "include")
LIB_NAME = "libvdnfp8.so"
LIB_PATH = os.path.join(_PKG, LIB_NAME)
# The measurement probes bench.py sets the kernels' rates against -- a bare read +
# write stream for the row kernels, a bare fp8 MFMA loop for the GEMM -- (not part of
# the C ABI; built alongside, loaded by bench.py only).
PROBE_SOURCES = ["stream_probe.hip", "mfma_probe.hip"]
PROBE_PATH = os.path.join(_PKG, "libvdnprobe.so")

SOURCES = ["capi.hip", "quantize.hip", "lora_requant.hip", "gemm.hip", "qk_prep.hip", "block_ops.hip"]
HEADERS = ["vdn_common.h"]             # in csrc/
PUBLIC_HEADERS = ["vdn_fp8.h"]         # in include/

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


def _sha256(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


_compiler_id = None


def compiler_id():
    """The compiler's identity, the "HIP version" and "clang version" lines of
    `hipcc --version` (the kernels' exact wait counts and schedules depend on its
    output), or None when no hipcc is installed."""
    global _compiler_id
    if _compiler_id is None:
        try:
            r = subprocess.run([hipcc(), "--version"], capture_output=True, text=True, timeout=60)
        except (RuntimeError, OSError, subprocess.SubprocessError):
            return None
        lines = [ln.strip() for ln in r.stdout.splitlines() if "HIP version" in ln or "clang version" in ln]
        _compiler_id = " | ".join(lines) if r.returncode == 0 and lines else "unknown"
    return _compiler_id


def source_manifest(csrc=CSRC, include=INCLUDE, compiler=None):
    """{"sources": {file: sha256}, "flags": sha256, "compiler": str, "digest": sha256 of
    all of it}: what a library built from these files, with these flags and this
    compiler (compiler_id() unless given), carries. Raises FileNotFoundError if a file
    is missing."""
    files = {name: _sha256(os.path.join(csrc, name)) for name in SOURCES + HEADERS}
    files.update({name: _sha256(os.path.join(include, name)) for name in PUBLIC_HEADERS})
    flags = hashlib.sha256(json.dumps([HIPCC_FLAGS, EXTRA_FLAGS], sort_keys=True).encode()).hexdigest()
    compiler = compiler if compiler is not None else (compiler_id() or "unknown")
    body = json.dumps({"sources": files, "flags": flags, "compiler": compiler}, sort_keys=True)
    return {"sources": files, "flags": flags, "compiler": compiler,
            "digest": hashlib.sha256(body.encode()).hexdigest()}


# The files that make each kernel family (its source plus the shared headers).
KERNEL_FILES = {
    "gemm": ["gemm.hip", "vdn_common.h", "vdn_fp8.h"],
    "quantize": ["quantize.hip", "vdn_common.h", "vdn_fp8.h"],
    "lora_requant": ["lora_requant.hip", "quantize.hip", "vdn_common.h", "vdn_fp8.h"],
}


def kernel_digest(manifest, family):
    """sha256 over the hashes of one kernel family's files (KERNEL_FILES) and of the
    flags in a manifest: identifies the code of that kernel, e.g. for profiles keyed to
    it."""
    files = KERNEL_FILES[family]
    return hashlib.sha256(json.dumps([manifest["sources"][f] for f in files] + [manifest["flags"]]).encode()
                          ).hexdigest()


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the fp8 library needs ROCm's hipcc to build")


def build(verbose=False, csrc=CSRC, include=INCLUDE, out=LIB_PATH):
    """Compile every source for gfx950 and link libvdnfp8.so. Returns its path."""
    cc = hipcc()
    manifest = source_manifest(csrc, include)
    with tempfile.TemporaryDirectory(prefix="vdnfp8_build_") as tmp:
        info_h = os.path.join(tmp, "vdn_build_info.h")
        with open(info_h, "w") as f:
            f.write("#define VDN_FP8_BUILD_INFO %s\n" % json.dumps(json.dumps(manifest, sort_keys=True)))

        def compile_one(src):
            obj = os.path.join(tmp, os.path.splitext(src)[0] + ".o")
            extra = ["-include", info_h] if src == "capi.hip" else []
            cmd = [cc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), *extra, "-I", include, "-I", csrc, "-c",
                   os.path.join(csrc, src), "-o", obj]
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
        shutil.copyfile(tmp_lib, out + ".tmp")
        os.replace(out + ".tmp", out)
    if out == LIB_PATH:
        build_probe()
    return out


def build_probe(csrc=CSRC, out=PROBE_PATH):
    """Compile the measurement probes into libvdnprobe.so. Returns its path."""
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="vdnprobe_build_") as tmp:
        tmp_lib = os.path.join(tmp, os.path.basename(out))
        r = subprocess.run([cc, *HIPCC_FLAGS, "-shared", *(os.path.join(csrc, f) for f in PROBE_SOURCES),
                            "-o", tmp_lib], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {', '.join(PROBE_SOURCES)}:\n{r.stderr}")
        shutil.copyfile(tmp_lib, out + ".tmp")
        os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
