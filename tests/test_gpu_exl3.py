"""GPU parity of the EXL3 decode and linear (trunk) kernels against the CPU oracle, through the C ABI.

Decoded weights must be bit-exact; linear outputs within rel-L2 5e-5 of the oracle's kernel arithmetic (the
reference's own kernel tolerance, tests/trunk6/check_kernels.py:105) and within 1e-2 of the exact f64 product.
"""
import numpy as np
import pytest

from ijah_amd import synth

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("K", range(2, 9))
@pytest.mark.parametrize("inp,out", [(128, 96), (256, 48), (64, 32)])
def test_decode_bit_exact(eng, oracle, K, inp, out):
    print(f"decode K{K} {inp}x{out}", flush=True)
    rng = np.random.default_rng(K * 1000 + inp + out)
    t, su, sv = synth.linear(rng, inp, out, K)
    lin = eng.exl3_linear(t, su, sv)
    got = lin.decode().view(np.uint16)
    want = oracle.decode(t).view(np.uint16)
    assert np.array_equal(got, want)


def test_decode_config1(eng, oracle):
    """Config 1: 2048 -> 512, K5 (the single-linear CPU case): every decoded weight bit-exact."""
    rng = np.random.default_rng(2048)
    t, su, sv = synth.linear(rng, 2048, 512, 5)
    got = eng.exl3_linear(t, su, sv).decode().view(np.uint16)
    assert np.array_equal(got, oracle.decode(t).view(np.uint16))


@pytest.mark.parametrize("R", [1, 2, 3, 4, 8])
def test_linear_config1(eng, oracle, R):
    print(f"linear 2048x512 K5 R{R}", flush=True)
    rng = np.random.default_rng(77 + R)
    t, su, sv = synth.linear(rng, 2048, 512, 5)
    x = synth.bf16_values(rng, R, 2048)
    lin = eng.exl3_linear(t, su, sv)
    y = lin.run(x)
    assert rel(y, oracle.exl3_linear(x, t, su, sv)) < 5e-5
    assert rel(y, oracle.exl3_linear(x, t, su, sv, exact=True)) < 1e-2
    assert np.array_equal(y, lin.run(x))  # deterministic


@pytest.mark.parametrize("inp,out,K,R", [(2048, 4096, 6, 1), (2048, 512, 6, 1), (4096, 2048, 6, 1),
                                         (2048, 512, 6, 4), (320, 640, 7, 2), (48, 96, 8, 1), (96, 48, 4, 8),
                                         (2048, 1024, 8, 1)])
def test_linear_trunk_shapes(eng, oracle, inp, out, K, R):
    """Config 3's trunk shapes (q / k / v / o at K6) and odd Hadamard sizes (64, 32, 16)."""
    print(f"linear {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp * 7 + out + K)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    y = eng.exl3_linear(t, su, sv).run(x)
    assert rel(y, oracle.exl3_linear(x, t, su, sv)) < 5e-5
    assert rel(y, oracle.exl3_linear(x, t, su, sv, exact=True)) < 1e-2


@pytest.mark.parametrize("inp,out,K,R", [(2048, 512, 5, 9), (2048, 512, 5, 16), (2048, 512, 5, 32),
                                         (2048, 4096, 6, 16), (4096, 2048, 6, 16), (320, 640, 7, 12), (96, 48, 4, 12),
                                         (2048, 1024, 8, 16), (2048, 640, 3, 20), (2048, 512, 2, 10), (48, 96, 8, 12)])
def test_linear_matrix_cores(eng, oracle, inp, out, K, R):
    """9..32 rows take the grouped matrix-core GEMM (lin_mm; 48 inputs = 3 k tiles, odd, run as groups of 8 rows on
    the GEMV): same tolerances as the GEMV rows."""
    print(f"linear mfma {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp * 5 + out + K + R)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    lin = eng.exl3_linear(t, su, sv)
    y = lin.run(x)
    assert rel(y, oracle.exl3_linear(x, t, su, sv)) < 5e-5
    assert rel(y, oracle.exl3_linear(x, t, su, sv, exact=True)) < 1e-2
    assert np.array_equal(y, lin.run(x))  # deterministic
    y1 = lin.run(x[:1])  # the GEMV path on the first row agrees with the matrix-core row
    assert rel(y1, y[:1]) < 5e-5


@pytest.mark.parametrize("inp,out,K,R", [(2048, 512, 5, 1), (2048, 4096, 6, 3), (320, 640, 7, 8), (96, 48, 4, 2)])
def test_linear_one_launch_matches_staged(eng, oracle, inp, out, K, R, monkeypatch):
    """The one-launch linear (in-workgroup prep, last-arriver finish) against the three-launch path: bit-identical
    (same per-element arithmetic and split order), over repeated runs (the block counters reset themselves)."""
    print(f"linear one-launch vs staged {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp + out + K + R)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    one = eng.exl3_linear(t, su, sv)
    monkeypatch.setenv("IJAH_LIN_PATH", "staged")
    staged = eng.exl3_linear(t, su, sv)
    want = staged.run(x)
    for _ in range(3):
        assert np.array_equal(one.run(x), want)
    assert rel(want, oracle.exl3_linear(x, t, su, sv)) < 5e-5


def test_lm_head_k8_column_blocks(eng, oracle):
    """Config 3's lm_head 2048 -> 151936 at K8 (311 MB of trellis). H_out is block-diagonal over 128 columns, so
    any 128-column block of y equals the oracle run on that block's trellis columns alone."""
    print("lm_head 2048x151936 K8", flush=True)
    rng = np.random.default_rng(151936)
    inp, out, K = 2048, 151936, 8
    t = rng.integers(0, 1 << 16, (inp // 16, out // 16, 16 * K), dtype=np.uint16)
    su, sv = synth.scales(rng, inp), synth.scales(rng, out)
    x = synth.bf16_values(rng, 1, inp)
    y = eng.exl3_linear(t, su, sv).run(x)
    assert np.isfinite(y).all()
    for blk in (0, 1, 517, out // 128 - 1):
        cols = slice(blk * 128, blk * 128 + 128)
        tb = np.ascontiguousarray(t[:, blk * 8:blk * 8 + 8])
        want = oracle.exl3_linear(x, tb, su, sv[cols])
        assert rel(y[:, cols], want) < 5e-5, blk


def test_run_kernel_decode_by_name(eng, oracle):
    """ne_run_kernel drives a registered kernel by name with function constants (reference tools/engine.py)."""
    K, inp, out = 5, 64, 64
    rng = np.random.default_rng(9)
    t, _, _ = synth.linear(rng, inp, out, K)
    # re-lay the tiles as the library stores them: [out/32 pairs][in/16][2]
    IT, OT = inp // 16, out // 16
    rel_t = np.zeros((OT // 2, IT, 2, 16 * K), np.uint16)
    for tk in range(IT):
        for tn in range(OT):
            rel_t[tn // 2, tk, tn % 2] = t[tk, tn]
    tiles = eng.from_numpy(rel_t)
    w = eng.alloc(inp * out * 2)
    eng.run_kernel("exl3_decode", [tiles, np.int32(IT), np.int32(OT), w], grid=((IT * OT + 3) // 4, 1, 1),
                   tg=(256, 1, 1), fconsts=[(10, "u32", K)])
    assert np.array_equal(w.download(np.uint16, (inp, out)), oracle.decode(t).view(np.uint16))
