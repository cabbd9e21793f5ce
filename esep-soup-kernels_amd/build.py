"""Ahead-of-time build of libesep_body.so (the HIP kernels and their C ABI) for gfx950.

    python esep-soup-kernels_amd/build.py            # compile every source, link the library

Each csrc/*.hip file is compiled to an object under _build/ (in parallel), then linked into
solution/body/libesep_body.so next to the ctypes loader that opens it. The bench's streaming
probes (benchlib/probe.hip) go into their own benchlib/libesep_probe.so. Both libraries are
always rebuilt from source; nothing is cached between calls.
"""

import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
OBJDIR = REPO / "_build"
LIB = PKG / "solution" / "body" / "libesep_body.so"
# measurement kernels of bench.py, kept out of the product library
PROBE_SRC = PKG / "benchlib" / "probe.hip"
PROBE_LIB = PKG / "benchlib" / "libesep_probe.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from forming packed fp32 arithmetic (v_pk_* fp32 forms).
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{CSRC}", f"-I{PKG / 'benchlib'}",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src):
    obj = OBJDIR / (("bench_" if src == PROBE_SRC else "") + src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def _link(objs, out):
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {out.name} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def build(verbose=True):
    """Compile all kernels for gfx950 and link libesep_body.so, and the bench's streaming probes
    into benchlib/libesep_probe.so. Returns the product library's path."""
    OBJDIR.mkdir(exist_ok=True)
    srcs = sources() + [PROBE_SRC]
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs[:-1], LIB)
    _link(objs[-1:], PROBE_LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size // 1024} KiB) from {len(srcs) - 1} sources, "
              f"{PROBE_LIB.name} for the bench")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
