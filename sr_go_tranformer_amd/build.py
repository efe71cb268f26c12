"""Build the gfx950 library in place: sr_go_tranformer_amd/libsrq.so.

Each HIP source compiles separately with hipcc for gfx950 (in parallel),
then one shared library is linked.  Flags:
  -ffp-contract=off     every fused multiply-add in the kernels is explicit
  -packed-fp32-ops off  no packed FP32 VALU instructions are generated
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsrq.so")
SOURCES = ["pack.hip", "gemv.hip", "gemv_q8.hip", "gemv_q4.hip", "gemv_f32.hip", "gemm.hip", "glue.hip", "attention.hip", "sample.hip", "api.cpp", "safetensors.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH, "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument"]


def _compile(src):
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, "-x", "hip", "-c"] + FLAGS + ["-I", os.path.join(HERE, "..", "include"),
                                                  os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = [ln for ln in (r.stderr or "").splitlines()
             if "packed-fp32-ops" not in ln and "not a recognized feature" not in ln and ln.strip()]
    if r.returncode != 0:
        raise RuntimeError("hipcc failed for %s:\n%s" % (src, "\n".join(noise)))
    return out, noise


def build(jobs=None):
    """Compile every HIP source for gfx950 and link libsrq.so (always rebuilds)."""
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, noise in results:
        for ln in noise:
            if "warning" in ln:
                print(ln, file=sys.stderr)
    tmp = LIB + ".tmp%d" % os.getpid()
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    return LIB


# Host-sanitized build for the CPU tests: the host code of every source with
# AddressSanitizer and UndefinedBehaviorSanitizer (the device code as in the
# product build, unsanitized), linked as _build/asan/libsrq_asan.so.  The CPU
# tests load it through SRQ_LIB under the sanitizer runtime to check the host
# paths they reach: the archive and config checks and the ABI.
ASAN_DIR = os.path.join(OBJ, "asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libsrq_asan.so")
ASAN_FLAGS = ["-O1", "-g", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH, "-ffp-contract=off",
              "-Xarch_device", "-O0",  # device code is never launched from this build: compile it quickly
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Xarch_host", "-fsanitize=address,undefined", "-Xarch_host", "-fno-omit-frame-pointer",
              "-Xarch_host", "-fno-sanitize-recover=undefined", "-Wno-unused-command-line-argument"]


def _compile_asan(src):
    out = os.path.join(ASAN_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, "-x", "hip", "-c"] + ASAN_FLAGS + ["-I", os.path.join(HERE, "..", "include"),
                                                       os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("sanitized hipcc failed for %s:\n%s" % (src, r.stderr))
    return out


def build_sanitized(jobs=None):
    """Compile every source for the host with ASan + UBSan and link
    libsrq_asan.so (always rebuilds)."""
    os.makedirs(ASAN_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile_asan, SOURCES))
    tmp = ASAN_LIB + ".tmp%d" % os.getpid()
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-Xarch_host", "-fsanitize=address,undefined",
           "-shared-libsan", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("sanitized link failed:\n" + r.stderr)
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


if __name__ == "__main__":
    print(build())
