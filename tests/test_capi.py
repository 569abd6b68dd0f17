"""C-ABI checks that need no GPU: the library loads, exports every NE_API symbol the headers declare, keeps the
reference's error convention (0/-1 or NULL + ne_last_error) and reads safetensors packs (no compute calls)."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from ijah_amd import synth
from ijah_amd.engine import SIGNATURES

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        names |= set(re.findall(r"NE_API\s+[^;(]*?\b(ne_\w+)\s*\(", h.read_text()))
    return names


def test_headers_declare_entry_points():
    names = declared_symbols()
    assert {"ne_abi_version", "ne_run_kernel", "ne_pack_open", "ne_moe_run", "ne_exl3_lin_run"} <= names


def test_library_exports_every_declared_symbol(eng):
    missing = [n for n in sorted(declared_symbols()) if not eng.has(n)]
    assert not missing, missing
    assert not eng.missing, eng.missing
    assert set(SIGNATURES) == declared_symbols()


def test_abi_and_dtypes(eng):
    assert eng.abi_version() == 1
    L = eng.lib
    for i, (n, s) in enumerate([("F32", 4), ("F16", 2), ("BF16", 2), ("U8", 1), ("U16", 2), ("U32", 4),
                                ("I32", 4), ("I64", 8), ("I8", 1), ("I16", 2), ("U64", 8), ("F64", 8),
                                ("BOOL", 1)]):
        assert L.ne_dtype_name(i).decode() == n and L.ne_dtype_size(i) == s
    assert L.ne_dtype_name(99).decode() == "?" and L.ne_dtype_size(99) == 0


def test_error_convention(eng, tmp_path):
    L = eng.lib
    assert L.ne_pack_open(str(tmp_path / "nope").encode()) is None
    assert "no such directory" in eng.last_error()
    assert L.ne_pack_open(str(tmp_path).encode()) is None
    assert "no .safetensors" in eng.last_error()
    assert L.ne_tensor_info(None, b"x", None) == -1
    assert L.ne_upload(None, 0, None, 0) == -1 and "out of range" in eng.last_error()
    assert L.ne_run_kernel(b"no_such_kernel", None, 0, None, 0, (C.c_uint32 * 3)(1, 1, 1), (C.c_uint32 * 3)(64, 1, 1),
                           0, 1, None, None) == -1
    assert "no kernel" in eng.last_error()
    assert eng.kernel_exists("moe_gateup") and eng.kernel_exists("exl3_decode") and not eng.kernel_exists("zz")
    assert L.ne_moe_create(None) is None and "null" in eng.last_error()


def test_pack_reader(eng, tmp_path):
    w = synth.moe_layer(1, hid=256, inter=128, ne=4, topk=2, K=5, shared=True, Ks=6, sgate=True)
    prefix = synth.write_moe_pack(tmp_path, w, layer=3, shards=2)
    p = eng.pack_open(tmp_path)
    names = p.names()
    assert names == sorted(names) and len(names) == 2 + 18
    assert p.config()["expert_quant"]["window"] == 15
    t = p.info(prefix + "switch_mlp.down_proj.trellis")
    assert t.dtype == "U16" and t.shape == (4, 8, 16, 80)
    assert np.array_equal(t.host, w["down.trellis"])
    r = p.info(prefix + "gate.weight")
    assert r.dtype == "BF16" and np.array_equal(r.host, w["router"])
    su = p.info(prefix + "shared_expert.gate_proj.suh")
    assert su.dtype == "F16" and np.array_equal(su.host, w["sgate_proj.suh"])
    with pytest.raises(Exception, match="no tensor"):
        p.info("missing.tensor")


def test_pack_odd_header_alignment(eng, tmp_path):
    """Shards whose data start at odd offsets (the reference's misaligned K5 shards) still read byte-exact."""
    rng = np.random.default_rng(2)
    a = rng.integers(0, 1 << 16, (3, 5), dtype=np.uint16)
    synth.write_safetensors(tmp_path / "m.safetensors", {"a": a}, pad_header_to=None)
    p = eng.pack_open(tmp_path)
    assert np.array_equal(p.info("a").host, a)


def test_moe_load_rejects_wrong_shapes(eng, tmp_path):
    w = synth.moe_layer(2, hid=256, inter=128, ne=4, topk=2, K=5, shared=False)
    w["up.trellis"] = w["up.trellis"][:, :, :4]  # wrong out/16
    prefix = synth.write_moe_pack(tmp_path, w)
    p = eng.pack_open(tmp_path)
    assert eng.lib.ne_moe_load(p.ptr, prefix.encode(), 2) is None
    assert "up_proj.trellis has shape" in eng.last_error()


@pytest.mark.parametrize("case", ["q8_group64", "bf16_dense", "unknown_part", "gate_without_expert"])
def test_moe_load_refuses_unsupported_shared_expert(eng, tmp_path, case):
    """A shared expert in a form the layer does not take is refused with a message, never silently dropped."""
    kind = "q8" if case in ("q8_group64",) else False
    w = synth.moe_layer(3, hid=256, inter=128, ne=4, topk=2, K=5, shared=kind, sgate=True)
    pre = "language_model.model.layers.0.mlp."
    extra = {}
    if case == "q8_group64":  # scales / biases of 64-wide groups (the reference's fn_moe takes g128 only)
        rng = np.random.default_rng(1)
        for p, i, o in (("gate", 256, 128), ("up", 256, 128), ("down", 128, 256)):
            wq, sc, bi = synth.q8_linear(rng, i, o, group=64)
            w[f"sq8_{p}.weight"], w[f"sq8_{p}.scales"], w[f"sq8_{p}.biases"] = wq, sc, bi
    elif case == "bf16_dense":
        extra[pre + "shared_expert.gate_proj.weight"] = np.zeros((128, 256), np.uint16)
    elif case == "unknown_part":
        extra[pre + "shared_expert.gate_proj.qweight"] = np.zeros((128, 64), np.uint32)
    prefix = synth.write_moe_pack(tmp_path, w, extra=extra)
    assert prefix == pre
    p = eng.pack_open(tmp_path)
    assert eng.lib.ne_moe_load(p.ptr, prefix.encode(), 2) is None
    msg = eng.last_error()
    assert {"q8_group64": "group 64", "bf16_dense": "weight", "unknown_part": "shared expert in a form",
            "gate_without_expert": "without a shared expert"}[case] in msg, msg
