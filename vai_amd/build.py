"""Builds libvai_amd.so in-tree for gfx950 with hipcc (no JIT, no torch).

    python -m vai_amd.build            # kernels + C ABI + C++ engine
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ENGINE = os.path.join(HERE, "engine")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libvai_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++20", f"--offload-arch={ARCH}", "-I", os.path.join(ROOT, "include"),
          "-I", HERE, "-Wno-pass-failed"]
# The streaming GEMV takes the pointers and sizes its first loads need as
# leading scalar arguments, which gfx950 can preload into SGPRs at launch (a
# struct argument is not preloaded): about 0.06 us of a 6.5 us step at M = 1.
# (The packed MFMA GEMV measured no difference.) The 3x3 and pointwise conv
# kernels do the same with their pointers and sizes: about 0.02-0.03 us.
FILE_FLAGS = {"slab.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"],
              "conv.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"]}


PYMOD_SRC = os.path.join(ENGINE, "pyvai.cpp")
# C++ programs that use the engine the way a model does; the GPU tests run them.
CPP_TESTS = os.path.join(ROOT, "tests", "cpp")
CPP_TEST_BIN = os.path.join(CPP_TESTS, "_bin")


def _sources():
    srcs = []
    for d in (CSRC, ENGINE):
        if os.path.isdir(d):
            for f in sorted(os.listdir(d)):
                if f.endswith((".hip", ".cpp")) and os.path.join(d, f) != PYMOD_SRC:
                    srcs.append(os.path.join(d, f))
    return srcs


def _build_pymodule():
    """pybind11 module _pyvai (the engine's Python surface), linked to libvai_amd.so."""
    import sysconfig
    import pybind11
    ext = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(HERE, "_pyvai" + ext)
    obj = os.path.join(BUILD, "pyvai.o")
    inc = ["-I", pybind11.get_include(), "-I", sysconfig.get_paths()["include"]]
    cmd = [HIPCC, "-x", "hip", "-O2", "-fPIC", "-std=c++20", f"--offload-arch={ARCH}"] + DEVICE_FLAGS + ["-I",
           os.path.join(ROOT, "include"), "-I", HERE] + inc + ["-c", PYMOD_SRC, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("pyvai compile failed:\n" + r.stderr)
    tmp = out + ".tmp"
    cmd = [HIPCC, "-shared", "-o", tmp, obj, "-L", HERE, "-lvai_amd", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("pyvai link failed:\n" + r.stderr)
    os.replace(tmp, out)
    return out


def _local_headers(src, seen=None):
    """The quoted #include files src pulls in, transitively."""
    import re
    seen = set() if seen is None else seen
    with open(src) as f:
        for inc in re.findall(r'^\s*#include\s+"([^"]+)"', f.read(), re.M):
            h = os.path.normpath(os.path.join(os.path.dirname(src), inc))
            if os.path.exists(h) and h not in seen:
                seen.add(h)
                _local_headers(h, seen)
    return seen


def _stale(src, obj):
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(f) > t for f in [src, *_local_headers(src)])


def _compile(src, only_stale=False):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if only_stale and not _stale(src, obj):
        return obj
    cmd = [HIPCC] + COMMON + DEVICE_FLAGS + FILE_FLAGS.get(os.path.basename(src), []) + ["-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC] + COMMON + ["-x", "hip", "-c", src, "-o", obj] + DEVICE_FLAGS
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{errs}")
    return obj


def build(jobs=None, only_stale=False):
    """Compiles every source (only_stale: only those older than their object
    or its local headers -- a development shortcut; the default rebuilds all)."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)), 16)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, only_stale), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp] + objs + ["-Wl,-soname,libvai_amd.so"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    _build_probe()
    _build_pymodule()
    _build_cpp_programs()
    return LIB


PROBE_SRC = os.path.join(HERE, "probe", "read_ceiling.hip")
PROBE_LIB = os.path.join(HERE, "libvai_probe.so")


MFMA_RATE_SRC = os.path.join(HERE, "probe", "mfma_rate.cpp")
MFMA_RATE_BIN = os.path.join(HERE, "probe", "_bin", "mfma_rate")


def _build_probe():
    """libvai_probe.so: bench.py's measurement kernels (the plain-read ceiling),
    and the mfma_rate program (the matrix-core ceiling behind the roofline
    notes), kept out of the product library."""
    tmp = PROBE_LIB + ".tmp"
    cmd = [HIPCC] + COMMON + DEVICE_FLAGS + ["-shared", PROBE_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("probe build failed:\n" + r.stderr)
    os.replace(tmp, PROBE_LIB)
    os.makedirs(os.path.dirname(MFMA_RATE_BIN), exist_ok=True)
    cmd = [HIPCC, "-x", "hip", "-O3", "-std=c++20", f"--offload-arch={ARCH}"] + DEVICE_FLAGS + [
        MFMA_RATE_SRC, "-o", MFMA_RATE_BIN + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("mfma_rate build failed:\n" + r.stderr)
    os.replace(MFMA_RATE_BIN + ".tmp", MFMA_RATE_BIN)


def _build_cpp_programs():
    """tests/cpp/*.cpp -> tests/cpp/_bin/<name>, linked to libvai_amd.so."""
    if not os.path.isdir(CPP_TESTS):
        return
    os.makedirs(CPP_TEST_BIN, exist_ok=True)
    for f in sorted(os.listdir(CPP_TESTS)):
        if not f.endswith(".cpp"):
            continue
        out = os.path.join(CPP_TEST_BIN, f[:-4])
        cmd = [HIPCC, "-x", "hip", "-O2", "-std=c++20", f"--offload-arch={ARCH}"] + DEVICE_FLAGS + ["-I", os.path.join(ROOT, "include"),
               "-I", ENGINE, os.path.join(CPP_TESTS, f), "-o", out + ".tmp", "-L", HERE, "-lvai_amd",
               "-Wl,-rpath," + os.path.relpath(HERE, CPP_TEST_BIN).join(["$ORIGIN/", ""])]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"C++ program {f} failed to build:\n" + r.stderr)
        os.replace(out + ".tmp", out)


if __name__ == "__main__":
    print(build(only_stale="--changed" in sys.argv))
    sys.exit(0)
