"""ijah_amd: EXL3 trellis-decode MoE / trunk linears for MI355X (gfx950), behind the reference's C API.

The compute path is the HIP library ijah_amd/_lib/libijah_exl3.so (built by ijah_amd.build); there is no CPU
fallback: loading fails loudly when the library is missing.
"""
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libijah_exl3.so"


def load_engine():
    """The ctypes Engine over the built library, or the one NE_LIB names (raises if it is not built)."""
    from .engine import Engine, LIB
    if not LIB.exists():
        raise RuntimeError(f"{LIB} is not built: run python -m ijah_amd.build")
    return Engine(LIB)
