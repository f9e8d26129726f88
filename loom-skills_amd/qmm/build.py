"""Builds libqmm.so in-tree: every csrc/*.hip compiled for gfx950 with hipcc, linked into one shared library.

    python loom-skills_amd/qmm/build.py        (or qmm.build.build())

The library lands next to this file (loom-skills_amd/qmm/libqmm.so) so that it travels with the source tree.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(HERE, "libqmm.so")
ARCH = os.environ.get("QMM_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# Packed-FP32 instructions stay off: the compiler would otherwise form v_pk_{add,mul,fma}_f32 from float code.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src, obj_dir=OBJ, defines=()):
    obj = os.path.join(obj_dir, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, *[f"-D{d}" for d in defines], "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose=False, lib=LIB, defines=()):
    """Compiles every HIP source (in parallel) and links the library (libqmm.so next to this file unless `lib`
    names another path; `defines` are extra -D macros, e.g. a kernel's tuning knob); returns the library path."""
    obj_dir = OBJ if lib == LIB else lib + ".objs"
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir, defines), srcs))
    LIB_ = lib
    tmp = LIB_ + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_)
    if verbose:
        print(f"built {LIB_} from {len(srcs)} sources")
    return LIB_


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
