"""Build the gfx950 HIP library ``ascend_rsfa/lib/librsfa.so``.

Every ``csrc/*.hip`` translation unit is compiled with hipcc for gfx950 in
parallel and linked into one shared library exporting the C ABI declared in
``include/rsfa.h``.  Usage::

    python ascend-rsfa_amd/build_native.py [-j JOBS]
"""
import argparse
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
LIB_DIR = os.path.join(PKG_ROOT, "ascend_rsfa", "lib")
LIB_NAME = "librsfa.so"
OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{fma,mul,add}_f32 in device code.  The host pass
# warns that it does not know the feature; that warning is expected.
# amdgpu-atomic-optimizer-strategy=None: the task queue's ticket atomic stays a
# plain returning atomic whose result is waited for where it is used (the
# optimizer's wave-aggregated form consumes it at once, exposing its latency at
# the start of every task).
HIPCC_FLAGS = [
    "--offload-arch=" + OFFLOAD_ARCH,
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(REPO_ROOT, "include"),
]

# Per-file flags.  kern_d256.hip: MFMAs in the VGPR form (accumulators in
# VGPRs) for its one-wave-per-SIMD float8-V tile, which has 512 registers:
# left to choose, the compiler gives every MFMA an AGPR accumulator and the
# softmax then copies each score out of the AGPRs.  The kernels built for two
# waves per SIMD use no AGPRs either way and compile to the same code.
FILE_FLAGS = {"kern_d256.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build librsfa.so")
    return path


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and "is not a recognized feature" not in line
    )
    return proc.returncode, out


def build(jobs=None, verbose=False):
    """Compile all sources and link the library; returns the library path."""
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    obj_dir = os.path.join(PKG_ROOT, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    cc = hipcc()
    t0 = time.time()

    def compile_one(src):
        obj = os.path.join(obj_dir, src[:-4] + ".o")
        rc, out = _run([cc] + HIPCC_FLAGS + FILE_FLAGS.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj])
        return src, obj, rc, out

    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(compile_one, srcs))
    failed = [(s, out) for s, _, rc, out in results if rc != 0]
    for s, _, rc, out in results:
        if out.strip() and (verbose or rc != 0):
            print(f"--- {s}\n{out}", file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed for: " + ", ".join(s for s, _ in failed))
    lib = os.path.join(LIB_DIR, LIB_NAME)
    tmp = lib + ".tmp"
    rc, out = _run([cc, "--offload-arch=" + OFFLOAD_ARCH, "-shared", "-fPIC", "-o", tmp]
                   + [o for _, o, _, _ in results])
    if rc != 0:
        raise RuntimeError("link failed:\n" + out)
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} in {time.time() - t0:.1f}s", file=sys.stderr)
    return lib


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
