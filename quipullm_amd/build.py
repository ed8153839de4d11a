"""Builds the native parts in-tree (quipullm_amd/lib/):

* quipu_kernels.hsaco -- the gfx950 kernels (hipcc --genco), loaded at run time with hipModuleLoad;
* libquipu.so         -- the C ABI of include/quipu.h (HIP runtime, op table);
* quipu_napi.node     -- the Node.js (N-API) addon over libquipu.so, for the JavaScript host.

Every call recompiles (it is the "does it build" check); nothing is downloaded.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
NODE_INC = "/usr/include/node"

HSACO = os.path.join(LIB, "quipu_kernels.hsaco")
SO = os.path.join(LIB, "libquipu.so")
NAPI = os.path.join(LIB, "quipu_napi.node")

# hipcc flags for device code: gfx950 only; packed-fp32 instructions disabled.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"build of {what} failed: {' '.join(cmd)}")
    return r


def _atomic(out, build):
    """Builds into a temporary name and renames, so a half-written file is never loaded."""
    tmp = out + ".tmp%d" % os.getpid()
    try:
        build(tmp)
        os.replace(tmp, out)
    finally:
        if os.path.exists(tmp):
            os.remove(tmp)


# The timeline build (profiling only): the same sources with -DQP_TIMELINE, in lib/timeline/.  Its kernels record
# per-workgroup start / end times of the launches captured in a graph; select it with QP_ADDON (Node.js) or
# QP_LIB (Python) and name the output with QP_TIMELINE_OUT; `python -m quipullm_amd.timeline` summarizes it.
TIMELINE_LIB = os.path.join(LIB, "timeline")


def build_kernels(lib=LIB, defs=()):
    src = os.path.join(CSRC, "kernels", "qp_kernels.hip")
    out = os.path.join(lib, "quipu_kernels.hsaco")
    _atomic(out, lambda o: _run([HIPCC, "--genco", *HIP_FLAGS, *defs, "-o", o, src], "kernels"))
    return out


def build_lib(lib=LIB, defs=()):
    src = os.path.join(CSRC, "quipu.cpp")
    # the scratch array of qp_dispatch_noalloc: a device array, so its file goes through hipcc (device code for
    # gfx950 embedded in the object) and is linked into the library
    scratch = os.path.join(CSRC, "qp_scratch.hip")
    obj = os.path.join(lib, "qp_scratch.o")
    _atomic(obj, lambda o: _run([HIPCC, "-c", "-fPIC", *HIP_FLAGS, "-o", o, scratch], "scratch array"))
    out = os.path.join(lib, "libquipu.so")
    cmd = lambda o: ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wno-unused-parameter",
                     "-D__HIP_PLATFORM_AMD__", *defs, f"-I{ROCM}/include", "-o", o, src, obj, f"-L{ROCM}/lib",
                     "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-Wl,-soname,libquipu.so"]
    _atomic(out, lambda o: _run(cmd(o), "libquipu"))
    return out


def build_napi(lib=LIB):
    if not os.path.isdir(NODE_INC):
        return None
    src = os.path.join(CSRC, "napi", "quipu_napi.cpp")
    out = os.path.join(lib, "quipu_napi.node")
    cmd = lambda o: ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wno-unused-parameter",
                     f"-I{NODE_INC}", f"-I{os.path.join(ROOT, 'include')}", "-o", o, src, f"-L{lib}", "-lquipu",
                     "-Wl,-rpath,$ORIGIN"]
    _atomic(out, lambda o: _run(cmd(o), "N-API addon"))
    return out


def build_timeline():
    """The profiling build of the kernels, library and addon into lib/timeline/ (not part of build_all)."""
    os.makedirs(TIMELINE_LIB, exist_ok=True)
    defs = ("-DQP_TIMELINE",)
    out = [build_kernels(TIMELINE_LIB, defs), build_lib(TIMELINE_LIB, defs), build_napi(TIMELINE_LIB)]
    return [o for o in out if o]


def build_oracle():
    """The CPU checker (test infrastructure; not part of the product)."""
    _run(["make", "-s", "-B", "-C", os.path.join(ROOT, "oracle")], "oracle")


def build_all(oracle=True):
    os.makedirs(LIB, exist_ok=True)
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        raise RuntimeError("hipcc not found")
    out = [build_kernels(), build_lib(), build_napi()]
    if oracle:
        build_oracle()
    return [o for o in out if o]


def built() -> bool:
    return all(os.path.exists(p) for p in (HSACO, SO))


if __name__ == "__main__":
    for p in (build_timeline() if "--timeline" in sys.argv[1:] else build_all()):
        print(p)
