"""Build libkvssd_hip.so for gfx950 with hipcc (no CMake, no torch extension).

    python kvssd-attention_amd/csrc/build.py [--jobs N] [--verbose]

Each .hip file compiles to an object in csrc/_build/, then the objects link into
kvssd-attention_amd/kvssd/libkvssd_hip.so, which the kvssd package loads with
ctypes after ``import torch`` so it shares torch's HIP runtime
(libamdhip64.so.7).  fastcall.c (a CPython module that calls one entry point
of that library without ctypes' per-argument conversions) compiles with the
host C compiler into kvssd/_fastcall<EXT_SUFFIX>.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import re
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent / "kvssd"
OUT = PKG / "libkvssd_hip.so"
TIMELINE_OUT = PKG / "libkvssd_hip_timeline.so"
FASTCALL_SRC = HERE / "fastcall.c"
FASTCALL_OUT = PKG / ("_fastcall" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
BUILD = HERE / "_build"
SOURCES = ["abi.hip", "decode_general.hip", "decode_mfma.hip", "decode_staged.hip", "merge.hip", "codec.hip", "records.hip", "vllm_codec.hip"]
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-mcode-object-version=5",
    # packed fp32 VALU forms stay off: hipcc may not emit v_pk_{add,mul,fma}_f32
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # scalar kernel arguments (up to 16 dwords, up to the first struct passed
    # by value) arrive preloaded in SGPRs at wave launch instead of through a
    # load from the kernel-argument segment
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-result",
]


HEADER = HERE.parent.parent / "include" / "kvssd_hip.h"
BUILD_ID_MARK = b"kvssd-build-id:"


def source_hash() -> str:
    """Hash of everything the library is built from: every HIP source and
    header here, the CPython module's source, the public header and the
    compile flags (16 hex digits)."""
    h = hashlib.sha256()
    files = sorted(p for p in HERE.iterdir() if p.suffix in (".hip", ".hpp", ".c")) + [HEADER]
    for f in files:
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    h.update(" ".join(COMMON + SOURCES).encode())
    return h.hexdigest()[:16]


def built_id(path: Path = OUT) -> str | None:
    """The build id stored in a built library (read from the file, without
    loading it), or None when the file is absent or carries none."""
    try:
        data = path.read_bytes()
    except OSError:
        return None
    m = re.search(re.escape(BUILD_ID_MARK) + rb"([0-9a-z]+)\0", data)
    return m.group(1).decode() if m else None


def is_stale(path: Path = OUT) -> bool:
    """True when the library is absent or was built from other sources (or,
    for the in-tree library, the CPython module built with it is absent or
    was built from other sources)."""
    tree = source_hash()
    return built_id(path) != tree or (path == OUT and built_id(FASTCALL_OUT) != tree)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; install ROCm or put /opt/rocm/bin on PATH")
    return path


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build_fastcall(verbose: bool = False) -> Path:
    """The CPython module, with the host C compiler against this interpreter's headers."""
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no host C compiler (gcc) found")
    include = sysconfig.get_paths()["include"]
    tmp = FASTCALL_OUT.with_name(FASTCALL_OUT.name + ".tmp")
    _run([cc, "-O2", "-shared", "-fPIC", "-Wall", "-Werror", f'-DKVSSD_BUILD_ID="{source_hash()}"', f"-I{include}",
          str(FASTCALL_SRC), "-o", str(tmp)], verbose)
    os.replace(tmp, FASTCALL_OUT)
    return FASTCALL_OUT


def build(jobs: int = 0, verbose: bool = False, timeline: bool = False) -> Path:
    """Compile every source and link the library.  ``timeline`` builds the
    instrumented variant (per-workgroup phase stamps, csrc/timeline.hpp) to
    kvssd/libkvssd_hip_timeline.so instead; the product never loads it."""
    out = TIMELINE_OUT if timeline else OUT
    build_dir = BUILD / "timeline" if timeline else BUILD
    build_dir.mkdir(parents=True, exist_ok=True)
    cc = hipcc()
    flags = [*COMMON, f'-DKVSSD_BUILD_ID="{source_hash()}"']
    if timeline:
        flags.append("-DKVSSD_TIMELINE")
    objs = [build_dir / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[cc, *flags, "-c", str(HERE / s), "-o", str(o)] for s, o in zip(SOURCES, objs)]
    workers = jobs or min(len(cmds), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, out)
    if not timeline:
        build_fastcall(verbose)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=0)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--timeline", action="store_true", help="build the instrumented library (phase stamps)")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.timeline))


if __name__ == "__main__":
    main()
