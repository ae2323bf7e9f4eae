"""Builds lib/libcheddar_amd.so (HIP kernels for gfx950 + C++ host + C-ABI).

Usage: python cheddar-fhe_amd/build.py [--jobs N] [--phase-timestamps DIR]
                                        [--host-asan DIR]
Compiles every source each time it is called (hipcc, no cache).
--phase-timestamps builds an instrumented copy into DIR instead (the forward
NTT records per-wave phase timestamps; tests/cpp/ntt_phase_timeline.cpp reads
them). --host-asan builds a copy into DIR whose host code runs under
AddressSanitizer (device code as in the product; tests/cpp's `asan` target
links the C++ API test against it).
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
OUT_DIR = os.path.join(PKG, "lib")
OBJ_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(OUT_DIR, "libcheddar_amd.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + os.path.join(PKG, "csrc"),
    "-I" + os.path.join(PKG, "host"),
]
# device code: gfx950 only, packed-fp32 instruction selection disabled
DEVICE = ["-x", "hip", "--offload-arch=" + ARCH,
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

# BConv's MFMA results go straight to VGPRs (no accumulator-register copies)
MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]

SOURCES = [
    ("csrc/ntt.hip", True, []),
    ("csrc/bconv.hip", True, MFMA_VGPR),
    ("csrc/elementwise.hip", True, []),
    ("csrc/hmult_noalloc.hip", True, []),
    ("host/device_tables.cpp", False, []),
    ("host/memory_pool.cpp", False, []),
    ("host/cheddar.cpp", False, []),
    ("host/encoder.cpp", False, []),
    ("host/param_json.cpp", False, []),
    ("host/context_ops.cpp", False, []),
    ("host/capi.cpp", False, []),
]


def compile_one(rel, device, extra, obj_dir=OBJ_DIR):
    src = os.path.join(PKG, rel)
    obj = os.path.join(obj_dir, rel.replace("/", "_") + ".o")
    if device:
        cmd = [HIPCC] + COMMON + DEVICE + extra + ["-c", src, "-o", obj]
    else:
        cmd = [HIPCC] + COMMON + extra + ["-D__HIP_PLATFORM_AMD__", "-c",
                                          src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s\n%s" %
                           (" ".join(cmd), res.stdout, res.stderr))
    return obj


# host code only: each option preceded by -Xarch_host, so no device code
# is built with the sanitizer
HOST_ASAN = ["-Xarch_host", "-fsanitize=address",
             "-Xarch_host", "-fno-omit-frame-pointer"]


def build(jobs=8, phase_timestamps=None, host_asan=None):
    """phase_timestamps: a directory for an instrumented copy of the library
    (the forward NTT's per-wave phase timestamps, for measurement only);
    host_asan: a directory for a copy whose host code is built with
    AddressSanitizer (for testing only); the product library is not touched
    by either"""
    out_dir, obj_dir, lib = OUT_DIR, OBJ_DIR, LIB
    dev_extra, host_extra, link_extra = [], [], []
    if phase_timestamps or host_asan:
        out_dir = os.path.abspath(phase_timestamps or host_asan)
        obj_dir = os.path.join(out_dir, "_build")
        lib = os.path.join(out_dir, "libcheddar_amd.so")
    if phase_timestamps:
        dev_extra = ["-DCHD_PHASE_TIMESTAMPS"]
    if host_asan:
        dev_extra = host_extra = link_extra = HOST_ASAN
    os.makedirs(out_dir, exist_ok=True)
    os.makedirs(obj_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(
            lambda s: compile_one(s[0], s[1],
                                  s[2] + (dev_extra if s[1] else host_extra),
                                  obj_dir), SOURCES))
    tmp = lib + ".tmp"
    cmd = ([HIPCC, "-shared", "--offload-arch=" + ARCH] + link_extra +
           ["-o", tmp] + objs)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed: %s\n%s" % (res.stdout, res.stderr))
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--phase-timestamps", metavar="DIR",
                    help="build an instrumented copy into DIR instead")
    ap.add_argument("--host-asan", metavar="DIR",
                    help="build a copy with host-side AddressSanitizer into "
                         "DIR instead")
    a = ap.parse_args()
    if a.phase_timestamps and a.host_asan:
        ap.error("--phase-timestamps and --host-asan are separate builds")
    print(build(a.jobs, a.phase_timestamps, a.host_asan))
    sys.exit(0)
