"""Builds sapphire_amd/libsapphire_hip.so with hipcc for gfx950.

    python -m sapphire_amd.build            # compile (always recompiles)
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libsapphire_hip.so")
SOURCES = ["runtime.cpp", "tensor.cpp", "dispatch.cpp", "decoder.cpp", "gemv.hip", "gemv_mfma.hip", "gemm_mfma.hip",
           "ops.hip", "sample.hip", "decode.hip",
           "decode_persist.hip", "quantize.hip", "gemm_bf16.hip", "noalloc.cpp", "transformer.cpp"]
ARCH = os.environ.get("SAPPHIRE_OFFLOAD_ARCH", "gfx950")

COMMON = [
    "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
    # contraction only where the source writes an explicit fmaf
    "-ffp-contract=off",
    # packed fp32 instructions are not used on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-D__HIP_PLATFORM_AMD__",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compiles every source (in parallel, `jobs` at a time; 0 = one per CPU up to 8) and links."""
    cc = hipcc()
    jobs = jobs or max(1, min(8, os.cpu_count() or 1))
    with tempfile.TemporaryDirectory(prefix="sapphire_build_") as tmp:
        cmds, objs = [], []
        for src in SOURCES:
            path = os.path.join(CSRC, src)
            if not os.path.exists(path):
                continue
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [cc, f"--offload-arch={ARCH}", *COMMON, "-c", path, "-o", obj]
            if src.endswith(".cpp"):
                cmd.insert(1, "-x")
                cmd.insert(2, "hip")
            if verbose:
                print(" ".join(cmd), flush=True)
            cmds.append(cmd)
            objs.append(obj)
        with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
            for f in [pool.submit(subprocess.run, c, check=True) for c in cmds]:
                f.result()
        tmp_out = OUT + ".tmp"
        # -Bsymbolic-functions: the library's calls to its own exported API bind inside it, never to
        # an engine's same-named functions loaded earlier
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-Bsymbolic-functions", "-o", tmp_out, *objs,
               "-lpthread", "-ldl"]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp_out, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
