"""Build recipe for libattn_flash.so (gfx950 HIP kernels + C host layer).

    python -m transfer_station_amd.build          # or __graft_entry__.build()

Compiles in-tree into transfer_station_amd/lib/. HIP sources go through hipcc for
gfx950 only; the C host layer through gcc against the HIP runtime API headers; the
link through g++ against libamdhip64 (and libgomp for the synthetic-data generator).
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(PKG, "_build")
LIBNAME = "libattn_flash.so"
# The same library with the persistent prefill's phase stamps compiled in (ATTN_PHASE_STAMPS=1),
# for transfer_station_amd/phases.py only; nothing else loads it.
STAMPS_LIBNAME = "libattn_flash_stamps.so"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["attn_kernels.hip"]
# Standalone roofline microbenchmark (MFMA peak, HBM copy/read), built next to the library.
TOOL_SOURCES = {"roofline_bench": "roofline_bench.hip"}
C_SOURCES = ["attn_flash.c", "attn_devutil.c", "attn_synth.c"]

# Packed fp32 VALU forms are disabled for all device code on this platform.
# IEEE mode off (with NaNs not honoured): fmaxf lowers to a bare v_max/v_max3 instead of
# canonicalising each MFMA result first. A NaN input still reaches O through the products.
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Wall",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-mno-amdgpu-ieee", "-fno-honor-nans",
               "-I" + INCLUDE]
CC_FLAGS = ["-O2", "-fPIC", "-std=c11", "-Wall", "-Wextra", "-fopenmp",
            "-I" + INCLUDE, "-I" + os.path.join(ROCM, "include")]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s%s" % (" ".join(cmd), r.stdout, r.stderr))
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    return out.strip()


def lib_path():
    return os.path.join(LIBDIR, LIBNAME)


def stamps_lib_path():
    return os.path.join(LIBDIR, STAMPS_LIBNAME)


def tool_path(name):
    return os.path.join(LIBDIR, name)


def build(verbose=False, jobs=8):
    """Compile every source and link the shared library; returns its path."""
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    cmds = []
    objs = []
    stamp_objs = []
    for s in HIP_SOURCES:
        o = os.path.join(OBJDIR, s + ".o")
        cmds.append([hipcc] + HIPCC_FLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
        objs.append(o)
        o = os.path.join(OBJDIR, s + ".stamps.o")
        cmds.append([hipcc] + HIPCC_FLAGS + ["-DATTN_PHASE_STAMPS=1", "-c", os.path.join(CSRC, s),
                                             "-o", o])
        stamp_objs.append(o)
    for s in C_SOURCES:
        o = os.path.join(OBJDIR, s + ".o")
        cmds.append(["gcc"] + CC_FLAGS + ["-c", os.path.join(CSRC, s), "-o", o])
        objs.append(o)
        stamp_objs.append(o)
    for exe, src in TOOL_SOURCES.items():
        cmds.append([hipcc] + HIPCC_FLAGS + [os.path.join(CSRC, src), "-o",
                                             os.path.join(LIBDIR, exe)])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, cmds):
            if out and verbose:
                print(out)
    for path, parts in ((lib_path(), objs), (stamps_lib_path(), stamp_objs)):
        tmp = path + ".tmp"
        _run(["g++", "-shared", "-o", tmp] + parts +
             ["-L" + os.path.join(ROCM, "lib"), "-lamdhip64", "-fopenmp", "-lm",
              "-Wl,-rpath," + os.path.join(ROCM, "lib")])
        os.replace(tmp, path)
    return lib_path()


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
