"""Build libmvlm_hip.so (gfx950) in-tree with hipcc.

    python -m mvlm_amd.build            # compile every source, link the library
    python -m mvlm_amd.build --check    # also list the exported mvlm_* symbols
    python -m mvlm_amd.build --incremental   # recompile only sources newer than their object

The library lands in mvlm_amd/lib/ so it travels with the source tree; the
object files go to mvlm_amd/_build/.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
ENGINE = os.path.join(PKG, "engine")
OBJ = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libmvlm_hip.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Packed fp32 VALU forms are switched off for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-command-line-argument",
          f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", f"-I{ENGINE}"]


def sources():
    srcs = []
    for d in (CSRC, ENGINE):
        for f in sorted(os.listdir(d)):
            if f.endswith((".hip", ".cpp")):
                srcs.append(os.path.join(d, f))
    return srcs


def _stack_kernels(remarks: str) -> list:
    """Kernels whose private (scratch) memory is more than their register
    spills explain, from the compiler's kernel-resource-usage remarks: an
    array the compiler could not keep in registers (a dynamically indexed
    one) lands in scratch memory and costs every access a memory round trip."""
    bad = []
    for block in remarks.split("Function Name: ")[1:]:
        name = block.split()[0]
        def val(key):
            m = re.search(re.escape(key) + r": (\d+)", block)
            return int(m.group(1)) if m else 0
        scratch = val("ScratchSize [bytes/lane]")
        spills = val("VGPRs Spill") + val("SGPRs Spill")
        if scratch > 4 * spills + 16:
            bad.append(f"{name}: {scratch} bytes of scratch per lane, {spills} spilled registers")
    return bad


def _compile(src: str) -> str:
    obj = _object(src)
    cmd = [HIPCC, f"--offload-arch={ARCH}", *COMMON]
    if src.endswith(".hip"):
        cmd += ["-x", "hip", *DEVICE_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"]
    cmd += ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = r.stdout + r.stderr
    msgs = "\n".join(l for l in out.splitlines()
                     if "packed-fp32-ops' is not a recognized feature" not in l and "remark:" not in l
                     and "-Rpass-analysis=kernel-resource-usage" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    bad = _stack_kernels("\n".join(l.split("remark: ", 1)[1] for l in out.splitlines() if "remark: " in l))
    if bad:
        os.remove(obj)
        raise RuntimeError(f"{src}: kernels with scratch memory beyond their register spills:\n  " + "\n  ".join(bad))
    return obj


def _object(src: str) -> str:
    return os.path.join(OBJ, os.path.relpath(src, PKG).replace(os.sep, "_") + ".o")


def _stale(src: str, newest_header: float) -> bool:
    obj = _object(src)
    return not os.path.exists(obj) or os.path.getmtime(obj) < max(os.path.getmtime(src), newest_header)


def build(jobs: int = 8, verbose: bool = True, incremental: bool = False) -> str:
    """Compile every source (or, with incremental, those newer than their
    object file or than any header) and link the library."""
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    todo = srcs
    if incremental:
        headers = [os.path.join(d, f) for d in (CSRC, ENGINE, os.path.join(ROOT, "include"))
                   for f in os.listdir(d) if f.endswith(".h")]
        newest = max(os.path.getmtime(h) for h in headers)
        todo = [s for s in srcs if _stale(s, newest)]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, max(1, len(todo))))) as ex:
        list(ex.map(_compile, todo))
    objs = [_object(s) for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-Wl,-rpath,/opt/rocm/lib", "-Wl,--no-undefined"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    build_engine_test()
    if verbose:
        print(f"built {LIB} and {ENGINE_TEST}")
    return LIB


ENGINE_TEST = os.path.join(LIBDIR, "test_engine")


def build_engine_test() -> str:
    """The C++ test of the mgpu:: drop-in (tests/cpp/test_engine.cpp): plain C++
    over the C ABI, linked against the library next to it."""
    src = os.path.join(ROOT, "tests", "cpp", "test_engine.cpp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", f"-I{os.path.join(ROOT, 'include')}",
           f"-I{ENGINE}", src, "-o", ENGINE_TEST + ".tmp", f"-L{LIBDIR}", "-lmvlm_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"engine test build failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(ENGINE_TEST + ".tmp", ENGINE_TEST)
    return ENGINE_TEST


def exported_symbols(path: str = LIB):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return sorted({l.split()[-1] for l in out.splitlines() if l.split() and l.split()[-1].startswith("mvlm_")})


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=8)
    ap.add_argument("--incremental", action="store_true")
    a = ap.parse_args()
    build(a.jobs, incremental=a.incremental)
    if a.check:
        print("\n".join(exported_symbols()))
