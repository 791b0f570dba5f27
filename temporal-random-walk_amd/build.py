"""Build the engine in-tree.

Produces, inside ``temporal-random-walk_amd/temporal_random_walk/``:

* ``libtrw_engine.so`` -- the HIP engine (gfx950 code objects) behind the
  C ABI of ``include/trw_engine.h``;
* ``_temporal_random_walk*.so`` -- the pybind11 module that mirrors the
  reference's Python surface on top of the C++ ``TemporalRandomWalk`` class,
  which calls the C ABI;

and ``temporal-random-walk_amd/probe/libtrw_probe.so``, bench.py's
random-gather probe (a measurement aid outside the engine).

Run ``python temporal-random-walk_amd/build.py`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
HOST = os.path.join(PKG_ROOT, "host")
OUT_DIR = os.path.join(PKG_ROOT, "temporal_random_walk")
BUILD_DIR = os.path.join(PKG_ROOT, "_build")
INCLUDE = os.path.join(REPO, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("TRW_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # a*b+c stays two roundings, as on the reference's x86-64 host path
    "-ffp-contract=off",
    # no packed-FP32 instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
]

HIP_SOURCES = ["primitives.hip", "build.hip", "walk.hip", "handoff.hip", "pickers.hip", "capi.hip"]
PROBE_DIR = os.path.join(PKG_ROOT, "probe")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{out}")
    return out


def build_engine() -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=min(6, len(HIP_SOURCES))) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    lib = os.path.join(OUT_DIR, "libtrw_engine.so")
    tmp = lib + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", *objs, "-o", tmp])
    os.replace(tmp, lib)
    return lib


def build_python_module() -> str:
    import pybind11

    suffix = sysconfig.get_config_var("EXT_SUFFIX")
    target = os.path.join(OUT_DIR, "_temporal_random_walk" + suffix)
    tmp = target + ".tmp"
    py_inc = sysconfig.get_paths()["include"]
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        f"-I{INCLUDE}", f"-I{HOST}", f"-I{pybind11.get_include()}", f"-I{py_inc}",
        os.path.join(HOST, "TemporalRandomWalk.cpp"),
        os.path.join(HOST, "RandomPicker.cpp"),
        os.path.join(HOST, "py_module.cpp"),
        f"-L{OUT_DIR}", "-ltrw_engine", "-Wl,-rpath,$ORIGIN",
        "-o", tmp,
    ]
    _run(cmd)
    os.replace(tmp, target)
    return target


def build_probe() -> str:
    """bench.py's random-gather probe: its own library beside probe.hip, not
    part of the engine."""
    lib = os.path.join(PROBE_DIR, "libtrw_probe.so")
    tmp = lib + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", os.path.join(PROBE_DIR, "probe.hip"), "-o", tmp])
    os.replace(tmp, lib)
    return lib


def build_all() -> None:
    build_engine()
    build_python_module()
    build_probe()


if __name__ == "__main__":
    build_all()
    print("built", OUT_DIR, file=sys.stderr)
