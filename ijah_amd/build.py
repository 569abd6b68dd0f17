"""Builds the EXL3 HIP library (ijah_amd/_lib/libijah_exl3.so) for gfx950 with hipcc; no CMake, no JIT cache.

    python -m ijah_amd.build          # or: from ijah_amd.build import build; build()
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OUT = PKG / "_lib"
LIB = OUT / "libijah_exl3.so"
PROBES = OUT / "libijah_probes.so"  # the measurement probes (bench.py --probe), kept out of the product library
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("IJAH_ARCH", "gfx950")

SOURCES = ["exl3_kernels.hip", "moe_fused.hip", "moe_batch.hip", "noalloc.hip", "moe_q8.hip", "exl3_host.cpp", "capi.cpp", "json.cpp", "pack_align.cpp"]
# -ffp-contract=off: the prepared input must round exactly as the reference's f32 arithmetic (no fused x*suh + y).
# -packed-fp32-ops off: packed FP32 VALU forms are not used on this pool.
COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
          f"-I{PKG.parent / 'include'}"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]


def _compile(src):
    obj = OUT / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE, "-x", "hip", "-c", str(SRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
    return obj, r.stderr


def build(verbose=False):
    """Compiles every source and links the shared library. Returns its path."""
    OUT.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        results = list(ex.map(_compile, SOURCES + ["probes.hip"]))
    objs = [str(o) for o, _ in results[:-1]]
    probe_obj = results[-1][0]
    if verbose:
        for _, err in results:
            if err.strip():
                print(err, file=sys.stderr)
    for out, files in ((LIB, objs), (PROBES, [str(probe_obj)])):
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out), *files]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link of {out.name} failed:\n{r.stderr[-4000:]}")
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
