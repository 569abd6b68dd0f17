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


@pytest.mark.parametrize("inp,out,K,R", [(2560, 10240, 6, 1), (2560, 12288, 6, 1), (2560, 640, 6, 1), (320, 10240, 8, 1),
                                         (2560, 12288, 6, 4), (2560, 640, 6, 16), (320, 10240, 8, 8)])
def test_linear_reference_trunk_shapes(eng, oracle, inp, out, K, R):
    """The reference's own trunk shapes, whose published timings BASELINE.md quotes (docs/trunk6.md:93-100): 2560 ->
    10240 and 2560 -> 12288 at K6, 2560 -> 640 at K6, 320 -> 10240 at K8; against the oracle, and rows bit-identical
    to the one-row run."""
    print(f"linear reference shape {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp + out * 3 + K + R)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    lin = eng.exl3_linear(t, su, sv)
    y = lin.run(x)
    assert rel(y, oracle.exl3_linear(x, t, su, sv)) < 5e-5
    assert rel(y, oracle.exl3_linear(x, t, su, sv, exact=True)) < 1e-2
    if R > 1:
        for i in (0, R - 1):
            assert np.array_equal(lin.run(x[i:i + 1])[0], y[i])


@pytest.mark.parametrize("inp,out,K,R", [(2048, 512, 5, 9), (2048, 512, 5, 16), (2048, 512, 5, 32),
                                         (2048, 4096, 6, 16), (4096, 2048, 6, 16), (320, 640, 7, 12), (96, 48, 4, 12),
                                         (2048, 1024, 8, 16), (2048, 640, 3, 20), (2048, 512, 2, 10), (48, 96, 8, 12),
                                         (64, 256, 5, 12), (32, 128, 6, 16), (288, 640, 5, 12), (576, 640, 6, 16),
                                         (352, 640, 5, 16), (144, 272, 4, 24)])
def test_linear_rows_bit_identical(eng, oracle, inp, out, K, R):
    """Many rows on the matrix cores, every row bit-identical to that row run alone (the k chunk / k group order is
    fixed by the shape, not by R), and within the oracle's tolerances. The shapes cover partial k chunks (48, 144,
    352 inputs), partial k groups (288, 320, 576) and single-chunk linears (32, 64)."""
    print(f"linear rows {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp * 5 + out + K + R)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    lin = eng.exl3_linear(t, su, sv)
    y = lin.run(x)
    assert rel(y, oracle.exl3_linear(x, t, su, sv)) < 5e-5
    assert rel(y, oracle.exl3_linear(x, t, su, sv, exact=True)) < 1e-2
    assert np.array_equal(y, lin.run(x))  # deterministic
    for r in sorted({0, 1, R // 2, R - 1}):
        assert np.array_equal(lin.run(x[r:r + 1])[0], y[r]), r
    assert np.array_equal(lin.run(x[:3]), y[:3])


@pytest.mark.parametrize("R", [1, 4, 16])
def test_linear_multi_launch_matches_single(eng, oracle, R):
    """q, k and v of config 3 (2048 -> 4096 / 512 / 512, K6) and a K5 linear recorded together
    (ne_exl3_lin_run_multi; reference trunk6.h:78 record_multi): each output bit-identical to the linear run alone
    (the K5 one in a launch of its own), each on its own input rows."""
    print(f"linear multi q/k/v R{R}", flush=True)
    rng = np.random.default_rng(300 + R)
    shapes = [(2048, 4096, 6), (2048, 512, 6), (2048, 512, 6), (1024, 256, 5)]
    lins, xs = [], []
    for inp, out, K in shapes:
        lins.append(eng.exl3_linear(*synth.linear(rng, inp, out, K)))
        xs.append(synth.bf16_values(rng, R, inp))
    ys = eng.lin_run_multi(lins, xs)
    for lin, x, y in zip(lins, xs, ys):
        assert np.array_equal(y, lin.run(x))
    assert np.array_equal(eng.lin_run_multi(lins, xs)[1], ys[1])  # again: the counters reset themselves


@pytest.mark.parametrize("inp,out,K,R", [(2048, 512, 5, 1), (2048, 4096, 6, 3), (320, 640, 7, 8), (96, 48, 4, 2)])
def test_linear_one_launch_matches_staged(eng, oracle, inp, out, K, R):
    """The one-launch linear (in-workgroup prep, last-arriver finish) against the three-launch path (prep launch, GEMM,
    finish launch): bit-identical, over repeated runs (the block counters reset themselves)."""
    print(f"linear one-launch vs staged {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp + out + K + R)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    one = eng.exl3_linear(t, su, sv)
    staged = eng.exl3_linear(t, su, sv).configure("staged", 1)
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


@pytest.mark.parametrize("inp,out,K,R", [(576, 65536 + 96, 5, 16), (2048, 65536, 8, 9), (512, 65536 + 256, 4, 32),
                                         (1024, 65536, 6, 5)])
def test_wide_linear_rows_bit_identical(eng, oracle, inp, out, K, R):
    """Linears of >= 2048 tile pairs (vocabulary heads) at 5..32 rows take the wide form (8 tile pairs per
    workgroup, one k group each, a k chunk's rows staged once for the 8 waves): every row bit-identical to that row
    run alone (the one-row k-loop form) and to the first rows run as a batch of 3; sampled column blocks (the output
    Hadamard's width) within the oracle's tolerance. The shapes cover a partial last k group (576 inputs: one 4-tile chunk), a last workgroup
    with 3 of its 8 tile pairs (65632 outputs), and a last workgroup with one full block of its two (65792)."""
    print(f"wide linear {inp}x{out} K{K} R{R}", flush=True)
    rng = np.random.default_rng(inp + out + K + R)
    t = rng.integers(0, 1 << 16, (inp // 16, out // 16, 16 * K), dtype=np.uint16)
    su, sv = synth.scales(rng, inp), synth.scales(rng, out)
    x = synth.bf16_values(rng, R, inp)
    lin = eng.exl3_linear(t, su, sv)
    y = lin.run(x)
    assert np.isfinite(y).all()
    assert np.array_equal(y, lin.run(x))  # deterministic; the block counters reset themselves
    for r in sorted({0, 1, R // 2, R - 1}):
        assert np.array_equal(lin.run(x[r:r + 1])[0], y[r]), r
    assert np.array_equal(lin.run(x[:3]), y[:3])
    W = oracle.had_size(out)  # H_out is block-diagonal over W columns: a W-column slice is a linear of its own
    assert out % W == 0 and oracle.had_size(W) == W
    for blk in (0, 1, 2 * out // W // 3, out // W - 1):
        cols = slice(blk * W, blk * W + W)
        tb = np.ascontiguousarray(t[:, blk * W // 16:(blk + 1) * W // 16])
        assert rel(y[:, cols], oracle.exl3_linear(x, tb, su, sv[cols])) < 5e-5, blk


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


# ------------------------------------------------------------------------------------------------ fused epilogues
def epi_case(eng, oracle, kind, inp, out, K, R, refr=True, ldy=0, yoff=0, seed=0):
    """The linear with epilogue `kind` (reference kernels/trunk6/trunk6.metal:129-197) against the oracle's epilogue
    applied to the same launch's plain output v (the GPU's v is deterministic): returns (got, want) pairs."""
    rng = np.random.default_rng(9000 + 31 * kind + inp + out + K + R + seed)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, R, inp)
    lin = eng.exl3_linear(t, su, sv)
    v = lin.run(x)
    ld = ldy or out  # y rows of ld floats, the epilogue's columns at [yoff, yoff + out) (reference gb [R][96])
    assert yoff + out <= ld
    base = rng.standard_normal((R, ld)).astype(np.float32)  # columns outside the epilogue's must survive
    yb = eng.from_numpy(base)
    e0 = e1 = e2 = None
    hc, T = 4, 0
    if kind == 1:
        e0 = rng.standard_normal((R, hc, out)).astype(np.float32)
        e1 = rng.standard_normal((R, 8)).astype(np.float32)
        e2 = np.zeros((R, hc, out), np.float32)
    elif kind == 6:
        e0 = synth.bf16(rng.standard_normal(out).astype(np.float32))
        e1 = synth.bf16(rng.standard_normal(out).astype(np.float32))
    elif kind == 7:
        T = 3
        e0 = np.full((T + R + 2, 128), -1.0, np.float32)
        e1 = np.array([T], np.uint32)
    bufs = [None if a is None else eng.from_numpy(a) for a in (e0, e1, e2)]
    lin.run_epi(R, eng.from_numpy(x), yb, kind, y_off=4 * yoff, refr=refr, hc=hc, ldy=ldy, e0=bufs[0], e1=bufs[1],
                e2=bufs[2])
    got = yb.download(np.float32, (R, ld))
    want_y = base.copy()
    e0w = None if e0 is None else e0.copy()
    e2w = None if e2 is None else e2.copy()
    want_y[:, yoff:yoff + out] = oracle.lin_epi(v, kind, refr=refr, hc=hc, e0=e0w, e1=e1, e2=e2w)
    pairs = [(got, want_y)]
    if kind == 1:
        pairs.append((bufs[2].download(np.float32, e2.shape), e2w))
    if kind == 7:
        pairs.append((bufs[0].download(np.float32, e0.shape), e0w))
    ref_full = oracle.lin_epi(oracle.exl3_linear(x, t, su, sv), kind, refr=refr, hc=hc, e0=None if e0 is None else
                              e0.copy(), e1=e1, e2=None if e2 is None else e2.copy())
    return pairs, got[:, yoff:yoff + out], ref_full


@pytest.mark.parametrize("kind,inp,out,K,R,refr,ldy,yoff", [
    (0, 2048, 512, 5, 1, True, 0, 0), (3, 2048, 512, 5, 2, True, 0, 0), (3, 2048, 512, 5, 12, True, 0, 0),
    (2, 2048, 1024, 6, 1, True, 0, 0), (2, 2048, 1024, 6, 16, True, 0, 0), (2, 2048, 1024, 6, 3, False, 0, 0),
    (1, 2048, 512, 6, 1, True, 0, 0), (1, 2048, 512, 6, 4, True, 0, 0), (1, 2048, 512, 6, 16, True, 0, 0),
    (1, 48, 96, 8, 12, True, 0, 0), (1, 2048, 512, 6, 2, False, 0, 0),
    (5, 2048, 48, 6, 1, True, 96, 48), (5, 2048, 48, 6, 10, True, 96, 48),
    (6, 2048, 48, 6, 1, True, 96, 0), (6, 2048, 48, 6, 10, True, 96, 0), (6, 2048, 48, 6, 2, False, 96, 0),
    (7, 2048, 640, 6, 1, True, 0, 0), (7, 2048, 640, 6, 16, True, 0, 0), (7, 48, 640, 5, 12, True, 0, 0),
    (3, 512, 65536, 4, 8, True, 0, 0), (2, 512, 65536, 4, 16, True, 0, 0)])  # the wide form (>= 2048 pairs)
def test_linear_fused_epilogues(eng, oracle, kind, inp, out, K, R, refr, ldy, yoff):
    print(f"linear epilogue {kind} {inp}x{out} K{K} R{R} refr {refr} ldy {ldy} y_off {yoff}", flush=True)
    pairs, y, ref_full = epi_case(eng, oracle, kind, inp, out, K, R, refr, ldy, yoff)
    transcendental = kind in (2, 5, 6)
    for g, w in pairs:
        if not transcendental and (refr or kind != 1):
            assert np.array_equal(g, w)  # adds, products and bf16 rounding only
            continue
        d = np.abs(g.astype(np.float64) - w)
        step = np.maximum(np.abs(g), np.abs(w)) * 2.0 ** -7 + 1e-30
        if refr and kind == 6:
            # unrounded exp output; an interior rounding (u, softplus) may flip one step at a boundary, rarely
            assert (d <= 4e-6 * np.abs(w) + 1e-30).mean() > 0.98
        elif refr:
            # GPU expf / logf vs the host's can straddle a bf16 rounding boundary: at most one step, rarely
            assert (d / step).max() <= 1.0 + 1e-6 and (d == 0).mean() > 0.98
        else:
            assert np.allclose(g, w, rtol=1e-5, atol=1e-7)
    assert rel(y, ref_full) < 1e-2  # end to end against the oracle linear + epilogue


def test_linear_epilogue_rejects(eng, oracle):
    rng = np.random.default_rng(3)
    t, su, sv = synth.linear(rng, 256, 48, 5)
    lin = eng.exl3_linear(t, su, sv)
    x = eng.from_numpy(synth.bf16_values(rng, 2, 256))
    y = eng.alloc(2 * 96 * 4)
    for kind, kw, msg in [(4, {}, "not supported"), (8, {}, "not supported"), (6, {}, "e0 (A_log) missing"),
                          (1, {"hc": 4}, "e0 (h) missing"), (0, {"ldy": 40}, "ldy 40 below out"),
                          (7, {}, "e0 (key cache) missing")]:
        with pytest.raises(RuntimeError, match=msg.replace("(", r"\(").replace(")", r"\)")):
            lin.run_epi(2, x, y, kind, **kw)
    with pytest.raises(RuntimeError, match="y buffer too small"):
        lin.run_epi(2, x, y, 5, y_off=4 * 49, ldy=96)


# ------------------------------------------------------------------------------------------------ HC read
def bf_steps(a, b):
    return np.abs(a.astype(np.float64) - b) / (np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + 1e-30)


@pytest.mark.parametrize("hid,lr,K,R", [(2560, 320, 6, 1), (2560, 320, 6, 4), (2560, 320, 6, 16), (128, 64, 5, 3)])
def test_hc_read(eng, oracle, hid, lr, K, R):
    """ne_hc_read (reference models/flash_next/layer_t6.mm:89-133 with kernels/trunk6/t6_epi.metal:16-97) against the
    oracle read on the same inputs: 1/rms bit-close, mix / out / gates within bf16 flips where the GPU's f32 sums and
    the oracle's straddle a rounding boundary; rounding off, rel-L2 within the linears' own bar."""
    print(f"hc read hid {hid} lr {lr} K{K} R{R}", flush=True)
    rng = np.random.default_rng(hid + lr + K + R)
    h = (rng.standard_normal((R, 4, hid)) * np.array([0.5, 1, 2, 4])[None, :, None]).astype(np.float32)
    nw = synth.bf16((1 + 0.1 * rng.standard_normal(4 * hid)).astype(np.float32))
    iw = synth.bf16((rng.standard_normal((4, 4 * hid)) / np.sqrt(4 * hid)).astype(np.float32))
    down, up = synth.linear(rng, 4 * hid, lr, K), synth.linear(rng, lr, 4 * hid, K)
    ld, lu = eng.exl3_linear(*down), eng.exl3_linear(*up)
    hb, nb, ib = eng.from_numpy(h), eng.from_numpy(nw), eng.from_numpy(iw)
    mb, jb, ob = eng.alloc(R * lr * 4), eng.alloc(R * 32), eng.alloc(R * hid * 4)
    from ijah_amd.engine import hc_read
    for refr in (True, False):
        hc_read(ld, lu, R, hb, nb, ib, mb, jb, ob, refr=refr)
        mix, inj, out = mb.download(np.float32, (R, lr)), jb.download(np.float32, (R, 8)), ob.download(np.float32,
                                                                                                     (R, hid))
        want_mix, want_inj, want_out = oracle.hc_read(h, nw, iw, down, up, refr=refr)
        assert np.allclose(inj[:, 4:], want_inj[:, 4:], rtol=2e-6)
        if refr:
            # the inner rounding rr(v) before silu / sigmoid may flip one step where the GPU's and the oracle's f32
            # sums straddle a boundary (the activation can then move the output by many steps: silu(t) ~ t e^t for
            # t << 0): each value is the activation of the oracle's rr(v) or of one of its bf16 neighbours
            xn, ip, _ = oracle.hc_prep(h, nw, iw)
            v = oracle.exl3_linear(xn, *down)
            assert act_of_neighbour(mix, v, lambda c: c / 4 / (1 + np.exp(-c / 4)))
            assert act_of_neighbour(inj[:, :4], ip.astype(np.float64).sum(axis=1), lambda c: 2 / (1 + np.exp(-c / 4)))
            assert (mix == want_mix).mean() > 0.97
            assert (out == want_out).mean() > 0.95 and rel(out, want_out) < 3e-3
        else:
            # out is a mean over streams whose normed terms often cancel: the up linear's own error (5e-5) grows
            assert rel(mix, want_mix) < 1e-4 and rel(out, want_out) < 1e-3
            assert np.allclose(inj[:, :4], want_inj[:, :4], rtol=1e-5)
    hc_read(ld, lu, R, hb, nb, ib, mb, jb, ob, refr=True)
    assert np.array_equal(ob.download(np.float32, (R, hid)), hc_read_again(ld, lu, R, hb, nb, ib, eng, lr, hid))


@pytest.mark.parametrize("hid,lr,K", [(2560, 320, 6), (512, 64, 5)])
def test_hc_read_one_row_matches_rows(eng, oracle, hid, lr, K):
    """At one row the HC read's input step (1/rms, the normed input, the inject partials) runs inside the down
    linear's workgroups instead of its own launch: each row read alone gives the bits of that row of a 4-row read,
    which takes the separate step."""
    print(f"hc read one row vs rows hid {hid} lr {lr} K{K}", flush=True)
    rng = np.random.default_rng(hid + 7)
    R = 4
    h = (rng.standard_normal((R, 4, hid)) * np.array([0.5, 1, 2, 4])[None, :, None]).astype(np.float32)
    nw = synth.bf16((1 + 0.1 * rng.standard_normal(4 * hid)).astype(np.float32))
    iw = synth.bf16((rng.standard_normal((4, 4 * hid)) / np.sqrt(4 * hid)).astype(np.float32))
    ld, lu = eng.exl3_linear(*synth.linear(rng, 4 * hid, lr, K)), eng.exl3_linear(*synth.linear(rng, lr, 4 * hid, K))
    nb, ib = eng.from_numpy(nw), eng.from_numpy(iw)
    from ijah_amd.engine import hc_read
    for refr in (True, False):
        mb, jb, ob = eng.alloc(R * lr * 4), eng.alloc(R * 32), eng.alloc(R * hid * 4)
        hc_read(ld, lu, R, eng.from_numpy(h), nb, ib, mb, jb, ob, refr=refr)
        mix, inj, out = mb.download(np.float32, (R, lr)), jb.download(np.float32, (R, 8)), ob.download(np.float32,
                                                                                                     (R, hid))
        for r in range(R):
            m1, j1, o1 = eng.alloc(lr * 4), eng.alloc(32), eng.alloc(hid * 4)
            hc_read(ld, lu, 1, eng.from_numpy(np.ascontiguousarray(h[r:r + 1])), nb, ib, m1, j1, o1, refr=refr)
            assert np.array_equal(m1.download(np.float32, (1, lr))[0], mix[r])
            assert np.array_equal(j1.download(np.float32, (1, 8))[0], inj[r])
            assert np.array_equal(o1.download(np.float32, (1, hid))[0], out[r])


def act_of_neighbour(got, v, act):
    """got == rr(act(c)) within one bf16 step, for c = rr(v) or a bf16 neighbour of it"""
    b = oracle_bf16(v)
    u = b.view(np.uint32)
    ok = np.zeros(got.shape, bool)
    for d in (-1, 0, 1):
        c = ((u.astype(np.int64) >> 16) + d).astype(np.uint32) << 16
        cand = oracle_bf16(act(c.view(np.float32).astype(np.float64)))
        ok |= bf_steps(got, cand) <= 1.0 + 1e-6
    return bool(ok.all())


def oracle_bf16(x):
    u = np.asarray(x, np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def hc_read_again(ld, lu, R, hb, nb, ib, eng, lr, hid):
    from ijah_amd.engine import hc_read
    mb, jb, ob = eng.alloc(R * lr * 4), eng.alloc(R * 32), eng.alloc(R * hid * 4)
    hc_read(ld, lu, R, hb, nb, ib, mb, jb, ob, refr=True)
    return ob.download(np.float32, (R, hid))  # deterministic across runs and output buffers


def test_hc_read_rejects(eng, oracle):
    rng = np.random.default_rng(4)
    from ijah_amd.engine import hc_read
    ld, lu = eng.exl3_linear(*synth.linear(rng, 512, 64, 5)), eng.exl3_linear(*synth.linear(rng, 64, 256, 5))
    b = eng.alloc(1 << 16)
    with pytest.raises(RuntimeError, match="must be 4 hid -> lr -> 4 hid"):
        hc_read(ld, lu, 1, b, b, b, b, b, b)
    lu = eng.exl3_linear(*synth.linear(rng, 64, 512, 5))
    with pytest.raises(RuntimeError, match="h buffer too small"):
        hc_read(ld, lu, 1, eng.alloc(16), b, b, b, b, b)
