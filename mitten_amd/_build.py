"""Builds libmitten_kv.so (hipcc, gfx950) and libmitten_kvhost.so (g++) in-tree.

The libraries land in mitten_amd/lib/, next to the sources, so they travel with
the repository snapshot. RPATH lists torch's lib directory before /opt/rocm so
that, inside a process that also runs PyTorch, both use one HIP runtime.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
REPO = os.path.dirname(PKG)
INCLUDE = os.path.join(REPO, "include")

DEVICE_LIB = os.path.join(LIBDIR, "libmitten_kv.so")
HOST_LIB = os.path.join(LIBDIR, "libmitten_kvhost.so")

DEVICE_SOURCES = ["mkv_pool.hip", "mkv_attention.hip", "mkv_prep.hip", "mkv_wire.hip"]
HOST_SOURCES = ["host/kv_host.cpp"]

ARCH = "gfx950"


def _rocm() -> str:
    return os.environ.get("ROCM_PATH", "/opt/rocm")


def _torch_libdir() -> str | None:
    try:
        import importlib.util

        spec = importlib.util.find_spec("torch")
        if spec is None or not spec.origin:
            return None
        d = os.path.join(os.path.dirname(spec.origin), "lib")
        return d if os.path.isdir(d) else None
    except Exception:
        return None


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def _hipcc() -> str:
    return shutil.which("hipcc") or os.path.join(_rocm(), "bin", "hipcc")


# Packed FP32 (v_pk_*_f32) stays off for all device code.
_DEVICE_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall",
                 "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def device_obj_cmd(src: str, obj: str, extra: list[str] | None = None) -> list[str]:
    """One translation unit of the device library -> object (host code plus
    its embedded gfx950 code object)."""
    return ([_hipcc(), f"--offload-arch={ARCH}"] + _DEVICE_FLAGS + [f"-I{INCLUDE}"] + (extra or []) +
            ["-c", os.path.join(CSRC, src), "-o", obj])


def device_link_cmd(objs: list[str], out: str = DEVICE_LIB) -> list[str]:
    rpaths = [p for p in (_torch_libdir(), os.path.join(_rocm(), "lib")) if p]
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC"]
    cmd += [f"-Wl,-rpath,{p}" for p in rpaths]
    return cmd + objs + ["-o", out]


def host_cmd(out: str = HOST_LIB, extra: list[str] | None = None) -> list[str]:
    cxx = os.environ.get("CXX", "g++")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", "-Wall", "-Wextra",
           f"-I{INCLUDE}"]
    cmd += extra or []
    cmd += [os.path.join(CSRC, s) for s in HOST_SOURCES] + ["-o", out]
    return cmd


def build(verbose: bool = False) -> None:
    """Compile both libraries (always recompiles). The device sources compile
    in parallel, one hipcc per file, and are linked into one library."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(LIBDIR, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="mkv_build_") as tmp:
        objs = [os.path.join(tmp, os.path.splitext(os.path.basename(s))[0] + ".o") for s in DEVICE_SOURCES]
        cmds = [device_obj_cmd(s, o) for s, o in zip(DEVICE_SOURCES, objs)]
        have_host = all(os.path.exists(os.path.join(CSRC, s)) for s in HOST_SOURCES)
        if have_host:
            cmds.append(host_cmd(HOST_LIB + ".tmp"))
        with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            for f in [ex.submit(_run, c, verbose) for c in cmds]:
                f.result()
        _run(device_link_cmd(objs, DEVICE_LIB + ".tmp"), verbose)
    os.replace(DEVICE_LIB + ".tmp", DEVICE_LIB)
    if have_host:
        os.replace(HOST_LIB + ".tmp", HOST_LIB)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(DEVICE_LIB)
    print(HOST_LIB)
