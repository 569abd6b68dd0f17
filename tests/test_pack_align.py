"""ne_pack_align (reference core/pack_align.h:1-25, `align-pack`): no GPU needed. The copy is checked against the
source arrays themselves and a header parse of its own (not the library's): every tensor's data starts aligned,
the bytes, dtypes, shapes and metadata are the source's, aligned shards and other files are links, a rerun keeps
what is done, a dry run only counts, and the library's pack reader reads the copy."""
import json
import os
import struct

import numpy as np
import pytest

from ijah_amd import synth


def header(path):
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        h = json.loads(f.read(n))
    return 8 + n, h


def tensors(path):
    data0, h = header(path)
    raw = open(path, "rb").read()
    out = {}
    for k, v in h.items():
        if k == "__metadata__":
            continue
        a, b = v["data_offsets"]
        out[k] = (v["dtype"], v["shape"], data0 + a, raw[data0 + a:data0 + b])
    return out


def write_with_meta(path, arrays, meta):
    """a safetensors file with __metadata__ and the data area at an odd offset"""
    hdr, off, blobs = {"__metadata__": meta}, 0, []
    for name in sorted(arrays):
        a = np.ascontiguousarray(arrays[name])
        dt = {np.dtype(np.uint16): "U16", np.dtype(np.uint8): "U8", np.dtype(np.float32): "F32"}[a.dtype]
        hdr[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    h = json.dumps(hdr, separators=(",", ":")).encode()
    if (8 + len(h)) % 2 == 0:
        h += b" "
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


@pytest.fixture
def src(tmp_path):
    rng = np.random.default_rng(7)
    d = tmp_path / "src"
    d.mkdir()
    mis = {"a.trellis": rng.integers(0, 1 << 16, (3, 5), dtype=np.uint16),   # 30 B
           "b.bytes": rng.integers(0, 256, (7,), dtype=np.uint8),             # 7 B
           "c.f32": rng.standard_normal((4, 4)).astype(np.float32),            # 64 B
           "d.suh": rng.integers(0, 1 << 16, (5,), dtype=np.uint16)}          # 10 B
    write_with_meta(d / "model-00001-of-00002.safetensors", mis, {"format": "pt", "note": "odd \"quoted\" text"})
    ok = {"e.w": rng.integers(0, 1 << 16, (64,), dtype=np.uint16)}        # 128 B, placed aligned below
    synth.write_safetensors(d / "model-00002-of-00002.safetensors", ok, pad_header_to=64)
    (d / "config.json").write_text('{"hidden_size": 256}')
    (d / "tokenizer.txt").write_text("x")
    return d, {**mis, **ok}


def expected_misaligned(d, align):
    n = nb = 0
    for f in sorted(d.glob("*.safetensors")):
        for dt, shp, start, raw in tensors(f).values():
            n += start % align != 0
            nb += len(raw) if start % align else 0
    return n, nb


def test_align_copies_every_tensor_aligned(eng, src):
    d, arrays = src
    dst = d.parent / "dst"
    n_mis, b_mis = expected_misaligned(d, 64)
    assert n_mis >= 3  # the fixture really is misaligned
    st = eng.pack_align(d, dst, 64)
    assert st["tensors"] == 5 and st["misaligned_tensors"] == n_mis and st["misaligned_bytes"] == b_mis
    assert st["files_rewritten"] == 1 and st["files_linked"] == 1 and st["files_kept"] == 0
    s1 = dst / "model-00001-of-00002.safetensors"
    assert not s1.is_symlink() and st["bytes_written"] == s1.stat().st_size
    for name in ("model-00002-of-00002.safetensors", "config.json", "tokenizer.txt"):
        assert (dst / name).is_symlink() and os.path.realpath(dst / name) == os.path.realpath(d / name)
    got = {}
    for f in sorted(dst.glob("*.safetensors")):
        got.update(tensors(f))
    assert sorted(got) == sorted(arrays)
    for name, a in arrays.items():
        dt, shp, start, raw = got[name]
        assert start % 64 == 0, name
        assert shp == list(a.shape) and raw == a.tobytes(), name
    assert header(s1)[1]["__metadata__"] == {"format": "pt", "note": "odd \"quoted\" text"}
    assert header(s1)[0] % 64 == 0
    assert dst.joinpath("model-00001-of-00002.safetensors.part").exists() is False
    # the library's own reader sees the same tensors
    p = eng.pack_open(dst)
    assert p.names() == sorted(arrays)
    assert np.array_equal(p.info("a.trellis").host, arrays["a.trellis"])
    assert np.array_equal(p.info("c.f32").host, arrays["c.f32"])


def test_align_rerun_keeps_the_copy(eng, src):
    d, _ = src
    dst = d.parent / "dst"
    eng.pack_align(d, dst, 64)
    s1 = dst / "model-00001-of-00002.safetensors"
    before = (s1.stat().st_ino, s1.stat().st_mtime_ns)
    st = eng.pack_align(d, dst, 64)
    assert st["files_kept"] == 1 and st["files_rewritten"] == 0 and st["bytes_written"] == 0
    assert (s1.stat().st_ino, s1.stat().st_mtime_ns) == before
    # a damaged copy is rewritten
    raw = bytearray(s1.read_bytes())
    raw[-1] ^= 0xFF
    s1.write_bytes(bytes(raw))
    st = eng.pack_align(d, dst, 64)
    assert st["files_rewritten"] == 1
    assert tensors(s1)["d.suh"][3] == tensors(d / "model-00001-of-00002.safetensors")["d.suh"][3]


def test_align_other_alignments_and_dry_run(eng, src):
    d, arrays = src
    st = eng.pack_align(d, d.parent / "never", 16, dry_run=True)
    assert (st["misaligned_tensors"], st["misaligned_bytes"]) == expected_misaligned(d, 16)
    assert st["files_rewritten"] == 0 and not (d.parent / "never").exists()
    dst = d.parent / "a4k"
    eng.pack_align(d, dst, 4096)
    for f in dst.glob("*.safetensors"):
        for name, (dt, shp, start, raw) in tensors(f).items():
            assert start % 4096 == 0 and raw == arrays[name].tobytes()


def test_align_errors(eng, src, tmp_path):
    d, _ = src
    L = eng.lib
    assert L.ne_pack_align(str(d).encode(), str(tmp_path / "x").encode(), 0, 0, None) == -1
    assert "alignment" in eng.last_error()
    assert L.ne_pack_align(str(tmp_path / "none").encode(), str(tmp_path / "x").encode(), 64, 0, None) == -1
    assert "no such directory" in eng.last_error()
    assert L.ne_pack_align(str(d).encode(), str(d).encode(), 64, 0, None) == -1
    assert "same directory" in eng.last_error()
    (tmp_path / "blocked").mkdir()
    (tmp_path / "blocked" / "config.json").write_text("{}")  # a regular file where a link would go
    assert L.ne_pack_align(str(d).encode(), str(tmp_path / "blocked").encode(), 64, 0, None) == -1
    assert "not a link" in eng.last_error()
