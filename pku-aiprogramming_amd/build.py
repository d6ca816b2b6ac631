"""Build the MI355X TinyTensor extension in-tree.

Replaces the reference's two torch ``CUDAExtension`` setups
(Task3/Tinytensor/setup.py:15-23 ``myTensor``, :42-53 ``myLayer``) with:

* ``libtt_hip.so`` -- every HIP source under ``csrc/`` compiled by ``hipcc``
  for ``--offload-arch=gfx950`` and linked into one shared library that
  exports the C-ABI of ``include/tt_attn.h``;
* ``myTensor`` and ``myLayer`` -- pybind11 modules built by ``g++`` from the
  host-only C++ sources; they call the C-ABI and link ``libtt_hip.so`` by
  ``$ORIGIN`` rpath.

Everything lands next to this file, so the directory is the import root
(``import myTensor, myLayer``) and the ``.so`` files travel with the tree.
Run ``python build.py`` or call ``build()``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")

HIP_SOURCES = ["tt_runtime.hip", "attn_fwd.hip", "attn_bwd.hip", "attn_bwd_w64.hip", "attn_decode.hip", "softmax.hip",
               "gemm.hip", "staging.hip", "conv.hip"]
# Per-file extra flags.  attn_bwd_w64.hip keeps its dK / dV accumulators in
# AGPRs by inline asm and needs its builtin MFMAs (scores) to write VGPRs.
HIP_FILE_FLAGS = {"attn_bwd_w64.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
# Host-only C++ linked into libtt_hip.so (the staged transfers' copy loops).
LIB_HOST_SOURCES = ["host_copy.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-FP32 instructions are kept out of every kernel; the host pass warns
# that it does not know the feature, which is harmless.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-command-line-argument",
]
CXX = os.environ.get("CXX", "g++")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _jobs():
    n = os.cpu_count() or 4
    return max(1, min(n, 16))


def ext_suffix():
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def built_paths():
    """Paths of the three build products."""
    suf = ext_suffix()
    return {
        "libtt_hip": os.path.join(HERE, "libtt_hip.so"),
        "myTensor": os.path.join(HERE, "myTensor" + suf),
        "myLayer": os.path.join(HERE, "myLayer" + suf),
    }


def build(verbose: bool = False) -> dict:
    """Compile everything (always; no up-to-date check) and return the paths."""
    import pybind11

    os.makedirs(OBJ, exist_ok=True)
    paths = built_paths()

    def hip_obj(src):
        obj = os.path.join(OBJ, src.replace(".hip", ".o"))
        _run([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(src, []), "-I", INCLUDE, "-c", os.path.join(CSRC, src), "-o", obj],
             verbose)
        return obj

    py_inc = sysconfig.get_paths()["include"]
    cxx_flags = ["-O2", "-fPIC", "-std=c++17", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
                 "-I", pybind11.get_include(), "-I", py_inc, "-I", INCLUDE, "-I", CSRC]

    def cxx_obj(src):
        obj = os.path.join(OBJ, src.replace(".cpp", ".o"))
        _run([CXX, *cxx_flags, "-c", os.path.join(CSRC, src), "-o", obj], verbose)
        return obj

    def lib_obj(src):
        obj = os.path.join(OBJ, src.replace(".cpp", ".o"))
        _run([CXX, "-O3", "-fPIC", "-std=c++17", "-Wall", "-c", os.path.join(CSRC, src), "-o", obj], verbose)
        return obj

    host_sources = ["tinytensor.cpp", "layers.cpp", "bind_tensor.cpp", "bind_layer.cpp"]
    with ThreadPoolExecutor(max_workers=_jobs()) as ex:
        hip_futs = [ex.submit(hip_obj, s) for s in HIP_SOURCES]
        lib_futs = [ex.submit(lib_obj, s) for s in LIB_HOST_SOURCES]
        cxx_futs = {s: ex.submit(cxx_obj, s) for s in host_sources}
        hip_objs = [f.result() for f in hip_futs] + [f.result() for f in lib_futs]
        cxx_objs = {s: f.result() for s, f in cxx_futs.items()}

    tmp = paths["libtt_hip"] + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *hip_objs,
          "-Wl,-rpath,/opt/rocm/lib", "-Wl,-soname,libtt_hip.so"], verbose)
    os.replace(tmp, paths["libtt_hip"])

    link = ["-shared", "-L", HERE, "-ltt_hip", "-Wl,-rpath,$ORIGIN"]
    for mod, objs in (("myTensor", ["tinytensor.cpp", "bind_tensor.cpp"]),
                      ("myLayer", ["tinytensor.cpp", "layers.cpp", "bind_layer.cpp"])):
        tmp = paths[mod] + ".tmp"
        _run([CXX, "-o", tmp, *[cxx_objs[s] for s in objs], *link], verbose)
        os.replace(tmp, paths[mod])
    return paths


def clean():
    shutil.rmtree(OBJ, ignore_errors=True)
    for p in built_paths().values():
        if os.path.exists(p):
            os.remove(p)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    for k, v in build(verbose="-v" in sys.argv).items():
        print(f"{k}: {v}")
