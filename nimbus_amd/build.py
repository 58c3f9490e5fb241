"""Builds libnimbus_attn.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m nimbus_amd.build            # compile
    python -m nimbus_amd.build --verbose  # also print register/LDS usage

The library goes next to this file so it travels with the source tree.
It links the HIP runtime by its soname (libamdhip64.so.7); loaded after
`import torch`, the dynamic loader resolves that soname to the runtime torch
already mapped, so the kernels and torch share one HIP runtime (streams and
graph capture work across the boundary).
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libnimbus_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["write_kv.hip", "paged_decode.hip", "paged_prefill.hip", "paged_general.hip", "rmsnorm.hip",
           "int8_matmul.hip", "elementwise.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-mcode-object-version=5",
        # Packed fp32 VALU forms stay off: the compiler must not emit them.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE,
        "-I", CSRC,
    ]


def _run(cmd: list[str], verbose: bool) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}")
    if verbose:
        sys.stdout.write(res.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compiles every source into LIB_PATH (always recompiles): one object per
    source, compiled in parallel, then one link. Returns the path."""
    cc = hipcc()
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    extra = ["-Rpass-analysis=kernel-resource-usage"] if verbose else []
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[cc, *extra, *flags(), "-c", "-o", o, os.path.join(CSRC, s)] for s, o in zip(SOURCES, objs)]
    workers = jobs or min(len(cmds), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    tmp = LIB_PATH + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose=False)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    print(build(verbose=args.verbose))


if __name__ == "__main__":
    main()
