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

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libnimbus_attn.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["write_kv.hip", "paged_decode.hip", "paged_prefill.hip", "rmsnorm.hip", "int8_matmul.hip",
           "elementwise.hip"]
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


def build(verbose: bool = False) -> str:
    """Compiles every source into LIB_PATH (always recompiles). Returns the path."""
    cc = hipcc()
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, *flags(), "-shared", "-o", tmp, *[os.path.join(CSRC, s) for s in SOURCES]]
    if verbose:
        cmd.insert(1, "-Rpass-analysis=kernel-resource-usage")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}")
    if verbose:
        sys.stdout.write(res.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    print(build(verbose=args.verbose))


if __name__ == "__main__":
    main()
