"""Builds ``libgdn.so``: every HIP source under ``csrc/`` compiled for gfx950
by hipcc into one shared library exporting the C ABI of ``include/gdn.h``."""

from __future__ import annotations

import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_PATH = os.path.join(HERE, "libgdn.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    # Packed float32 VALU ops are disabled for every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def build(verbose: bool = False) -> str:
    """Compile all kernels into ``libgdn.so`` (always recompiles): one hipcc
    process per source file, run in parallel, then one link."""

    import concurrent.futures
    import tempfile

    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="gdn_build_") as tmpdir:
        jobs = []
        for src in sources():
            obj = os.path.join(tmpdir, os.path.basename(src) + ".o")
            jobs.append(([hipcc, *compile_flags, "-c", src, "-o", obj], obj))
        workers = min(len(jobs), max(1, min(os.cpu_count() or 1, 8)))

        def run(cmd):
            if verbose:
                print(" ".join(cmd), flush=True)
            subprocess.run(cmd, check=True)

        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            for f in [pool.submit(run, cmd) for cmd, _ in jobs]:
                f.result()
        tmp = LIB_PATH + f".tmp{os.getpid()}"
        run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *[o for _, o in jobs], "-o", tmp])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
