"""Build the gfx950 library: every HIP/C++ source under csrc/ -> kernels/gfx950/libcolabfold_gfx950.so.

  python colabfold-legacy-kernels_amd/build.py [--jobs N] [--verbose]

hipcc cross-compiles for gfx950 without a GPU. Objects go to _build/ at the repository root;
the library goes in-tree, where the locator (colabfold_legacy_kernels.library_path) finds it.
The XLA FFI handlers (csrc/xla_ffi.cc) are part of the same library: they are written against
the XLA FFI C API structures declared in csrc/xla_ffi_api.h, so no jax headers are needed.
"""
import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "colabfold_legacy_kernels", "kernels", "gfx950")
LIB_NAME = "libcolabfold_gfx950.so"
BUILD_DIR = os.path.join(ROOT, "_build")
ARCH = "gfx950"

# Packed fp32 VALU forms are kept out of the generated code (no v_pk_{add,mul,fma}_f32).
# MFMA results stay in VGPRs (no v_accvgpr_read per use of an accumulator).
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=" + ARCH,
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-mllvm", "-amdgpu-mfma-vgpr-form",
             "-Wall", "-Wno-unused-result", "-Wno-unused-function"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cc")))


def compile_one(cc, src, verbose):
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    # every source is compiled as HIP: the .cc files hold host code only, but share the headers
    cmd = [cc, "-x", "hip"] + HIP_FLAGS + ["-I", INCLUDE, "-I", CSRC, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = (r.stdout + r.stderr).strip()
    # hipcc's host pass does not know the packed-fp32-ops feature; that warning is expected
    lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l]
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s" % (src, "\n".join(lines)))
    if verbose and lines:
        print("\n".join(lines))
    return obj


def build(jobs=None, verbose=False):
    cc = hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1), 16)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(cc, s, verbose), srcs))
    lib = os.path.join(OUT_DIR, LIB_NAME)
    tmp = lib + ".tmp"
    # libstdc++ and libgcc are linked statically, as the reference links its libraries
    # (its CI audits for them): the library then needs the HIP runtime and the C library only,
    # whatever C++ runtime the host process (jaxlib, torch) brings
    cmd = [cc, "-shared", "-fPIC", "--offload-arch=" + ARCH, "-o", tmp] + objs + \
          ["-static-libstdc++", "-static-libgcc", "-Wl,--no-undefined", "-Wl,-soname," + LIB_NAME,
           "-Wl,--exclude-libs,ALL", "-Wl,--version-script=" + os.path.join(HERE, "exports.map")]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))
    sys.exit(0)
