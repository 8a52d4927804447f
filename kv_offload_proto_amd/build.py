"""Build the native parts of kv_offload_proto_amd in-tree.

* ``kvops_ext/libkvx.so`` -- the gfx950 kernels and the C ABI (include/kvx/kvx.h),
  compiled by hipcc for ``--offload-arch=gfx950``.
* ``kvops_ext/_kvops*.so`` -- the pybind11 module with the reference's
  ``kvops_ext._kvops`` surface, linked against libkvx.so (rpath $ORIGIN).

Run ``python kv_offload_proto_amd/build.py`` (as a script: importing the package
needs what this builds), or call :func:`build`.
"""
import os
import subprocess
import sys
import sysconfig
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "kvops_ext")
INCLUDE = os.path.join(ROOT, "include")

HIP_SOURCES = ["sieve.hip", "sieve_fast.hip", "sieve_wave.hip", "sieve_batch.hip", "sieve_table.hip", "rows.hip",
               "kvx_host.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # hand-packed FP32 forms are not used anywhere; keep the compiler from
    # forming them either
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# flags of one source only
HIP_SOURCE_FLAGS = {
    # the parallel SIEVE kernel is a chain of dependent LDS steps at a fixed
    # four waves per SIMD; the scheduler that groups memory operations into
    # clauses gives it ~1% (same-box A/B against the default scheduler)
    "sieve_fast.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
}


# extra hipcc flags for every source (profiling builds, e.g. -DKVX_BATCH_STAMPS)
EXTRA_FLAGS = os.environ.get("KVX_EXTRA_HIPFLAGS", "").split()


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def lib_path():
    return os.path.join(OUT, "libkvx.so")


def ext_path():
    return os.path.join(OUT, "_kvops" + sysconfig.get_config_var("EXT_SUFFIX"))


def build(verbose=False):
    """Compile libkvx.so (gfx950) and the _kvops module.  Always recompiles.

    Each source compiles to an object of its own (in parallel, in a
    temporary folder), so that a source can carry flags of its own."""
    os.makedirs(OUT, exist_ok=True)
    lib = lib_path()
    tmp = lib + ".tmp"
    with tempfile.TemporaryDirectory(prefix="kvx_build_") as bdir:
        def compile_one(src):
            obj = os.path.join(bdir, src + ".o")
            cmd = [HIPCC] + HIP_FLAGS + HIP_SOURCE_FLAGS.get(src, []) + EXTRA_FLAGS
            cmd += ["-c", "-I", INCLUDE, "-I", CSRC, "-o", obj, os.path.join(CSRC, src)]
            _run(cmd, verbose)
            return obj

        with ThreadPoolExecutor(max_workers=max(1, min(len(HIP_SOURCES), os.cpu_count() or 1))) as pool:
            objs = list(pool.map(compile_one, HIP_SOURCES))
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, lib)

    import pybind11

    ext = ext_path()
    tmp = ext + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        "-I", pybind11.get_include(), "-I", sysconfig.get_paths()["include"], "-I", INCLUDE,
        "-o", tmp, os.path.join(CSRC, "kvops_pybind.cpp"),
        "-L", OUT, "-lkvx", "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd, verbose)
    os.replace(tmp, ext)
    return lib, ext


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
