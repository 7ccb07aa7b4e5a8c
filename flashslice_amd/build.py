"""Build the HIP library ``flashslice_amd/_lib/libflashslice_hip.so`` in-tree.

    python -m flashslice_amd.build            # compile for gfx950
    python -m flashslice_amd.build --verbose  # also print register usage

Every translation unit under ``csrc/`` is compiled by ``hipcc`` for gfx950
in parallel and linked into one shared library with the C ABI declared in
``include/flashslice_hip.h``. Packed-fp32 VALU instructions are disabled
(``-packed-fp32-ops``): the kernels' fp32 arithmetic is scalar per lane.
"""

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "libflashslice_hip.so"
LIB_PATH = os.path.join(OUT_DIR, LIB_NAME)
BUILD_DIR = os.path.join(os.path.dirname(HERE), "_build")

ARCH = "gfx950"
SOURCES = ("fs_fused.hip", "fs_blocked.hip", "fs_coop.hip", "fs_reduce.hip", "fs_layernorm.hip",
           "fs_abi.cpp")
# explicit instances of fused_launch<K, T, DK> (fs_fused_kernels.h), one
# generated translation unit each so that they compile in parallel
_FUSED_TYPES = (("float", (0,)), ("__bf16", (0, 1, 2)), ("_Float16", (0, 1, 2)))
FUSED_INSTANCES = tuple((k, t, dk) for k in range(5) for t, dks in _FUSED_TYPES for dk in dks)
# and of blocked_launch<K, T, DK> (fs_blocked_kernels.h)
BLOCKED_INSTANCES = tuple((k, t, dk) for k in range(8) for t, dks in _FUSED_TYPES for dk in dks)
FLAGS = [
    "--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _generated_sources():
    """Write the per-instance translation units; returns their paths."""
    gen = os.path.join(BUILD_DIR, "gen")
    os.makedirs(gen, exist_ok=True)
    out = []
    units = [("fused", "fs_fused_kernels.h", "fused_launch", i) for i in FUSED_INSTANCES]
    units += [("blocked", "fs_blocked_kernels.h", "blocked_launch", i) for i in BLOCKED_INSTANCES]
    for fam, header, fn, (k, t, dk) in units:
        name = "%s_k%d_%s_dk%d.hip" % (fam, k, t.strip("_"), dk)
        text = ('#include "%s"\nnamespace fs {\ntemplate hipError_t %s<%d, %s, %d>'
                '(const Args&, hipStream_t);\n}\n' % (os.path.join(CSRC, header), fn, k, t, dk))
        path = os.path.join(gen, name)
        if not os.path.exists(path) or open(path).read() != text:
            with open(path, "w") as f:
                f.write(text)
        out.append(path)
    return out


def _compile(src, verbose):
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    path = src if os.path.isabs(src) else os.path.join(CSRC, src)
    cmd = [_hipcc(), *FLAGS, "-x", "hip", "-c", path, "-o", obj]
    if verbose:
        cmd += ["-Rpass-analysis=kernel-resource-usage"]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("compiling %s failed:\n%s" % (src, r.stderr[-8000:]))
    return obj, time.time() - t0, r.stderr


def build(verbose=False, jobs=None):
    """Compile every source and link the library. Returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    sources = list(SOURCES) + _generated_sources()
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    t0 = time.time()
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        res = list(ex.map(lambda s: _compile(s, verbose), sources))
    for (obj, dt, err), src in zip(res, sources):
        if verbose and err:
            print(err)
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + [o for o, _, _ in res]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("linking failed:\n" + r.stderr[-4000:])
    os.replace(tmp, LIB_PATH)
    print("[build] wrote %s (%d units, %.0f s)" % (LIB_PATH, len(sources), time.time() - t0),
          flush=True)
    _build_abi_smoke()
    return LIB_PATH


ROOT = os.path.dirname(HERE)
ABI_SMOKE_SRC = os.path.join(ROOT, "tests", "abi_smoke.cpp")
ABI_SMOKE_BIN = os.path.join(ROOT, "tests", "_bin", "fs_abi_smoke")


def _build_abi_smoke():
    """The torch-free C ABI check (tests/abi_smoke.cpp): a host-only program
    linked against the library, run by tests/test_abi_gpu.py."""
    if not os.path.exists(ABI_SMOKE_SRC):
        return
    os.makedirs(os.path.dirname(ABI_SMOKE_BIN), exist_ok=True)
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = ["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(rocm, "include"),
           ABI_SMOKE_SRC, "-o", ABI_SMOKE_BIN, "-L" + OUT_DIR, "-lflashslice_hip",
           "-L" + os.path.join(rocm, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../flashslice_amd/_lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        # a test helper: the library itself is built; tests/test_abi_gpu.py
        # reports the missing program
        print("[build] WARNING: the C ABI check (tests/abi_smoke.cpp) did not build:\n"
              + r.stderr[-2000:], flush=True)
        return
    print("[build] wrote %s" % ABI_SMOKE_BIN, flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args(argv)
    build(verbose=a.verbose)


if __name__ == "__main__":
    sys.exit(main())
