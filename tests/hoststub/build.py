"""Builds the library's host code (exl3_host.cpp, capi.cpp, json.cpp, pack_align.cpp) against the host-only HIP
stand-in (hip_stub.cpp) with g++: tests/hoststub/_build/libijah_hoststub.so, for CPU tests of the capture and
lifetime invariants. TEST INFRASTRUCTURE ONLY."""
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "_build" / "libijah_hoststub.so"
SOURCES = [ROOT / "ijah_amd" / "csrc" / f for f in ("exl3_host.cpp", "capi.cpp", "json.cpp", "pack_align.cpp")] + \
          [HERE / "hip_stub.cpp"]


def build():
    """Compiles when a source is newer than the library; returns its path."""
    if OUT.exists() and all(s.stat().st_mtime < OUT.stat().st_mtime for s in SOURCES):
        return OUT
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", "-Wno-format-truncation",
           "-I/opt/rocm/include", f"-I{ROOT / 'include'}", *map(str, SOURCES), "-o", str(OUT)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return OUT


if __name__ == "__main__":
    print(build())
