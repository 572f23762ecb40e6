"""Build ``libtritium_hip.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Usage: ``python -m helion_amd._build [--jobs N]``.  Objects are compiled in
parallel into ``helion_amd/_build/`` and linked into
``helion_amd/libtritium_hip.so`` (in-tree, so it travels with the source tree
to the GPU machine).

Flags worth knowing:
* ``--offload-arch=gfx950`` only: MI355X (CDNA4) is the single target;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the compiler
  from emitting packed-fp32 VALU ops (v_pk_*_f32);
* ``-mcode-object-version=5`` is understood by both ROCm 7.0 (torch's bundled
  runtime) and ROCm 7.2.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_DIR = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libtritium_hip.so")
# measurement-only probes (HBM streaming ceilings), loaded by bench.py alone
PROBE_SRC = os.path.join(PKG_DIR, "probe", "stream_probe.hip")
PROBE_PATH = os.path.join(PKG_DIR, "libtritium_probe.so")

HIPCC = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

COMPILE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
    f"-I{os.path.join(REPO_DIR, 'include')}",
]


def sources() -> list[str]:
    return sorted(
        os.path.join(SRC_DIR, f) for f in os.listdir(SRC_DIR) if f.endswith(".hip")
    )


def _compile(src: str, obj_dir: str = OBJ_DIR, defines: tuple[str, ...] = ()) -> tuple[str, str]:
    obj = os.path.join(obj_dir, os.path.basename(src)[: -len(".hip")] + ".o")
    cmd = [HIPCC, *COMPILE_FLAGS, *(f"-D{d}" for d in defines), "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{log}")
    return obj, log


def build(jobs: int | None = None, verbose: bool = False, out: str = LIB_PATH,
          defines: tuple[str, ...] = ()) -> str:
    """Compile every csrc/*.hip and link the shared library; return its path.

    ``out`` and ``defines`` (``-D`` macros) build variant libraries, e.g. a
    different GEMM tile configuration, next to the default one."""
    obj_dir = OBJ_DIR if out == LIB_PATH else out + ".objs"
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda s: _compile(s, obj_dir, tuple(defines)), srcs))
    for obj, log in results:
        if log.strip() and verbose:
            print(f"[{os.path.basename(obj)}]\n{log}", file=sys.stderr)
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp,
           *[obj for obj, _ in results]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, out)
    return out


def build_probe() -> str:
    """Compile the streaming probes into their own library (not the product's)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    obj_dir = os.path.join(OBJ_DIR, "probe")
    os.makedirs(obj_dir, exist_ok=True)
    obj, _ = _compile(PROBE_SRC, obj_dir)
    tmp = PROBE_PATH + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, PROBE_PATH)
    return PROBE_PATH


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--out", default=LIB_PATH, help="library path (default: in-tree)")
    ap.add_argument("-D", dest="defines", action="append", default=[], help="preprocessor macro")
    args = ap.parse_args(argv)
    print(build(args.jobs, args.verbose, args.out, tuple(args.defines)))
    if args.out == LIB_PATH:
        print(build_probe())
    return 0


if __name__ == "__main__":
    sys.exit(main())
