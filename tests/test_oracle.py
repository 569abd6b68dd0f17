"""Pins the CPU oracle (oracle/exl3_oracle.c) before it is trusted as the parity reference.

The reference ships no golden vectors for this path and its CPU decoder (exl3_codec) is external. Each oracle
function is checked here against something it does not share code with: numpy's IEEE fp16 arithmetic, the textbook
Sylvester Hadamard matrix, a pure-Python walk over the tail-biting ring, the reference's two other trellis readers
(restated in the oracle from kernels/ne_common.h and kernels/trunk6/trunk6.metal), hand-computed known answers,
numpy's stable argsort, and an explicit-matrix numpy restatement of the EXL3 linear and the MoE layer.
"""
import numpy as np
import pytest

from ijah_amd import synth


# ------------------------------------------------------------------------------------------------ number formats
def test_f16_conversion_matches_numpy(oracle):
    L = oracle.lib()
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
                           np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 6.1e-5, -7.0],
                                    np.float32)])
    vals = vals.astype(np.float32)
    got = np.array([L.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([L.orc_f16_to_f32(int(h)) for h in want], np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


def test_bf16_round_known_answers(oracle):
    L = oracle.lib()
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even -> 1.0; 1 + 3*2^-8 ties up to 1 + 2^-6 (even mantissa)
    assert L.orc_bf16r(1.0 + 2 ** -8) == 1.0
    assert L.orc_bf16r(1.0 + 3 * 2 ** -8) == 1.0 + 2 ** -6
    assert L.orc_bf16r(1.0 + 2 ** -8 + 2 ** -20) == 1.0 + 2 ** -7
    assert L.orc_bf16r(-3.0) == -3.0


# ------------------------------------------------------------------------------------------------ codebook
def test_mcg_known_answers(oracle):
    # cw 0: r = 0x3B603B60, both halves 0x3B60 = 0.921875 -> 1.84375 = fp16 0x3F60
    assert oracle.mcg(0) == 0x3F60
    # bit 15 is ignored (window 15)
    assert oracle.mcg(0x8000) == oracle.mcg(0)
    # cw 1: r = 0xCBAC1FED & 0x8FFF8FFF ^ 0x3B603B60 = 0xB0CC348D -> fp16(0x348D) + fp16(0xB0CC)
    r = (0xCBAC1FED & 0x8FFF8FFF) ^ 0x3B603B60
    assert r == 0xB0CC348D
    lo = np.array([0x348D], np.uint16).view(np.float16)[0]
    hi = np.array([0xB0CC], np.uint16).view(np.float16)[0]
    assert oracle.mcg(1) == np.array([np.float16(lo + hi)]).view(np.uint16)[0]


def test_mcg_table_vs_numpy(oracle):
    """All 2^15 codewords against numpy's uint32 wrap-around multiply and fp16 add."""
    cw = np.arange(1 << 15, dtype=np.uint32)
    r = ((cw * np.uint32(0xCBAC1FED)) & np.uint32(0x8FFF8FFF)) ^ np.uint32(0x3B603B60)
    h = r.view(np.uint16).reshape(-1, 2).view(np.float16)
    want = (h[:, 0] + h[:, 1]).astype(np.float16).view(np.uint16)
    got = oracle.mcg_table()
    assert np.array_equal(got, want)
    v = got.view(np.float16).astype(np.float64)
    # both halves lie in +-[2^-3, 2^1): every value is finite and below 4 in magnitude
    assert np.isfinite(v).all() and np.abs(v).max() < 4.0
    # the codebook is a zero-mean, unit-scale Gaussian proxy
    assert abs(v.mean()) < 0.05 and 0.8 < v.std() < 1.3


# ------------------------------------------------------------------------------------------------ trellis readers
def py_ring_codewords(tile, K):
    """Pure-Python walk over the ring (the definition, independent of the C code)."""
    words = [int(tile[2 * w]) | (int(tile[2 * w + 1]) << 16) for w in range(8 * K)]
    bits = []
    for w in words:
        bits.extend((w >> (31 - b)) & 1 for b in range(32))
    tot = 256 * K
    out = []
    for i in range(256):
        end = (i + 1) * K
        v = 0
        for p in range(end - 15, end):
            v = (v << 1) | bits[p % tot]
        out.append(v)
    return np.array(out, np.uint16)


@pytest.mark.parametrize("K", range(1, 9))
def test_readers_agree(oracle, K):
    rng = np.random.default_rng(100 + K)
    for t in range(25):
        tile = rng.integers(0, 1 << 16, 16 * K, dtype=np.uint16)
        ring = oracle.tile_cw(tile, K, "ring") & 0x7FFF
        assert np.array_equal(ring, oracle.tile_cw(tile, K, "t6") & 0x7FFF)
        if 4 <= K <= 6:
            assert np.array_equal(ring, oracle.tile_cw(tile, K, "lane") & 0x7FFF)
        if t < 2:
            assert np.array_equal(ring, py_ring_codewords(tile, K))


@pytest.mark.parametrize("K", [4, 5, 8])
def test_constant_tiles(oracle, K):
    zeros = np.zeros(16 * K, np.uint16)
    ones = np.full(16 * K, 0xFFFF, np.uint16)
    assert (oracle.tile_cw(zeros, K) & 0x7FFF == 0).all()
    assert (oracle.tile_cw(ones, K) & 0x7FFF == 0x7FFF).all()
    w = oracle.decode(zeros.reshape(1, 1, -1))
    assert (w.view(np.uint16) == 0x3F60).all()


def test_single_bit_moves_expected_codewords(oracle):
    """A single set bit at ring position p appears in exactly the codewords whose 15-bit window covers p."""
    K = 5
    for p in (0, 7, 31, 32, 639, 1279):
        tile = np.zeros(16 * K, np.uint16)
        w, b = divmod(p, 32)
        word = 1 << (31 - b)
        tile[2 * w] = word & 0xFFFF
        tile[2 * w + 1] = word >> 16
        cw = oracle.tile_cw(tile, K) & 0x7FFF
        for i in range(256):
            end = (i + 1) * K
            covered = [(end - 15 + t) % (256 * K) for t in range(15)]
            want = (1 << (14 - covered.index(p))) if p in covered else 0
            assert cw[i] == want, (p, i)


def test_slot_map_is_a_bijection_with_reference_rows(oracle):
    seen = set()
    for s in range(256):
        r, c = oracle.slot_rc(s)
        l, j = s >> 3, s & 7
        q = l & 3
        assert r == [2 * q, 2 * q + 1, 2 * q + 8, 2 * q + 9][j & 3]
        assert c == (l >> 2) + 8 * (j >> 2)
        seen.add((r, c))
    assert len(seen) == 256


def test_decode_matrix_tiles(oracle):
    rng = np.random.default_rng(3)
    K = 6
    t = rng.integers(0, 1 << 16, (3, 2, 16 * K), dtype=np.uint16)
    w = oracle.decode(t).view(np.uint16)
    table = oracle.mcg_table()
    for tk in range(3):
        for tn in range(2):
            cw = py_ring_codewords(t[tk, tn], K)
            for s in range(0, 256, 37):
                r, c = oracle.slot_rc(s)
                assert w[16 * tk + r, 16 * tn + c] == table[cw[s]]


# ------------------------------------------------------------------------------------------------ Hadamard
def sylvester(n):
    i = np.arange(n)
    x = i[:, None] & i[None, :]
    pc = np.zeros((n, n), np.int64)
    while x.any():
        pc += x & 1
        x = x >> 1
    return np.where(pc % 2 == 0, 1.0, -1.0) / np.sqrt(n)


@pytest.mark.parametrize("n,had", [(128, 128), (512, 128), (320, 64), (48, 16), (96, 32)])
def test_fwht_matches_sylvester(oracle, n, had):
    assert oracle.had_size(n) == had
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n)
    H = sylvester(had)
    want = (v.reshape(-1, had) @ H).reshape(-1)
    assert np.allclose(oracle.fwht(v, had, f64=True), want, rtol=0, atol=1e-12)
    assert np.allclose(oracle.fwht(v.astype(np.float32), had), want, rtol=0, atol=1e-5)


# ------------------------------------------------------------------------------------------------ linear
def np_linear_exact(oracle, x, t, suh, svh):
    """x @ (diag(suh) H_in W' H_out diag(svh)) with explicit matrices (tools/convert_trunk_enc.py:125-128)."""
    w = oracle.decode(t).astype(np.float64)
    k, m = w.shape
    hk, hm = oracle.had_size(k), oracle.had_size(m)
    Hk = np.kron(np.eye(k // hk), sylvester(hk))
    Hm = np.kron(np.eye(m // hm), sylvester(hm))
    W = np.diag(suh.astype(np.float64)) @ Hk @ w @ Hm @ np.diag(svh.astype(np.float64))
    return x.astype(np.float64) @ W


@pytest.mark.parametrize("inp,out,K", [(256, 128, 5), (128, 320, 6), (512, 256, 8), (128, 128, 4)])
def test_linear_vs_explicit_matrices(oracle, inp, out, K):
    rng = np.random.default_rng(inp + out + K)
    t, su, sv = synth.linear(rng, inp, out, K)
    x = synth.bf16_values(rng, 3, inp)
    want = np_linear_exact(oracle, x, t, su, sv)
    exact = oracle.exl3_linear(x, t, su, sv, exact=True)
    assert np.allclose(exact, want, rtol=1e-12, atol=1e-9)
    emul = oracle.exl3_linear(x, t, su, sv)
    rel = np.linalg.norm(emul - want) / np.linalg.norm(want)
    assert rel < 2e-3  # the fp16 input preparation (reference docs/trunk6.md:74-84: ~3e-4)


# ------------------------------------------------------------------------------------------------ router
def test_route_ties_and_order(oracle):
    rng = np.random.default_rng(5)
    for trial in range(50):
        lg = (np.round(rng.standard_normal(64) * 4) / 4).astype(np.float32)  # many ties
        ids, w = oracle.route(lg, 10)
        want = np.argsort(-lg, kind="stable")[:10]
        assert np.array_equal(ids, want)
        top = lg[want]
        e = np.exp((top - top[0]).astype(np.float32))
        assert np.allclose(w, e / e.sum(), rtol=1e-6)
        assert abs(w.sum() - 1) < 1e-5


def test_router_logits(oracle):
    rng = np.random.default_rng(6)
    x = synth.bf16_values(rng, 256)
    rw = synth.bf16(rng.standard_normal((32, 256)).astype(np.float32) / 16)
    lg = oracle.router_logits(x, rw)
    want = x.astype(np.float64) @ ((rw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)).T
    assert np.allclose(lg, want, rtol=1e-2, atol=1e-6)
    assert np.array_equal(synth.bf16(lg), (lg.view(np.uint32) >> 16).astype(np.uint16))  # bf16-representable


# ------------------------------------------------------------------------------------------------ MoE layer
def np_moe_exact(oracle, W, x, route, sg):
    """Explicit-matrix restatement of one MoE row set: tools/opref.py:417-435 (+ the shared expert)."""
    hid, inter, topk = W.d["hid"], W.d["inter"], W.d["topk"]

    def mat(t, su, sv):
        w = oracle.decode(t).astype(np.float64)
        k, m = w.shape
        Hk = np.kron(np.eye(k // oracle.had_size(k)), sylvester(oracle.had_size(k)))
        Hm = np.kron(np.eye(m // oracle.had_size(m)), sylvester(oracle.had_size(m)))
        return np.diag(su.astype(np.float64)) @ Hk @ w @ Hm @ np.diag(sv.astype(np.float64))

    def expert(mats, xr):
        g, u = xr @ mats[0], xr @ mats[1]
        return (g / (1 + np.exp(-g)) * u) @ mats[2]

    d = W.d
    y = np.zeros((x.shape[0], hid))
    for r in range(x.shape[0]):
        xr = x[r].astype(np.float64)
        for k in range(topk):
            e = int(route[r, k])
            wk = route[r, topk + k:topk + k + 1].view(np.float32)[0]
            mats = [mat(d[f"{p}.trellis"][e], d[f"{p}.suh"][e], d[f"{p}.svh"][e]) for p in ("gate", "up", "down")]
            y[r] += wk * expert(mats, xr)
        if "sgate_proj.trellis" in d:
            mats = [mat(d[f"{p}.trellis"], d[f"{p}.suh"], d[f"{p}.svh"]) for p in ("sgate_proj", "sup_proj",
                                                                                    "sdown_proj")]
            y[r] += (1.0 if sg is None else sg[r]) * expert(mats, xr)
    return y


@pytest.mark.parametrize("shared,sgate", [(True, False), (False, False), (True, True)])
def test_moe_layer_vs_explicit(oracle, shared, sgate):
    w = synth.moe_layer(11, hid=256, inter=128, ne=16, topk=4, K=5, shared=shared, Ks=6, sgate=sgate)
    W = oracle.MoeWeights(w)
    rng = np.random.default_rng(12)
    x = synth.bf16_values(rng, 2, 256)
    y, lg, rt = oracle.moe_layer(W, x)
    for r in range(2):
        ids, wt = oracle.route(lg[r], 4)
        assert np.array_equal(rt[r, :4], ids)
        assert np.array_equal(rt[r, 4:].view(np.float32), wt)
    sg = None
    if sgate:
        l = np.array([oracle.router_logits(x[r], w["sgate"][None]) for r in range(2)]).reshape(-1)
        sg = 1 / (1 + np.exp(-l.astype(np.float32)))
    want = np_moe_exact(oracle, W, x, rt, sg)
    exact = oracle.moe_experts(W, x, rt, sg=sg, exact=True)
    assert np.allclose(exact, want, rtol=1e-9, atol=1e-9 * np.abs(want).max())
    rel = np.linalg.norm(y - want) / np.linalg.norm(want)
    assert rel < 5e-3
    fast, used = oracle.moe_experts(W, x, rt, sg=sg, fast_threads=2)
    assert used >= 1
    assert np.linalg.norm(fast - y) / np.linalg.norm(y) < 1e-5


# ------------------------------------------------------------------------------------------------ linear epilogues
def bfr(x):
    """f64 -> f32 -> bf16 round to nearest even (independent of the oracle's own rounding)"""
    u = np.asarray(x, np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def np_epi(v, kind, refr, hc=4, e0=None, e1=None, T=0):
    """closed forms of kernels/trunk6/trunk6.metal:129-197 in f64 with the rounding points written out"""
    q = bfr if refr else (lambda a: np.asarray(a, np.float64))
    v = v.astype(np.float64)
    R, out = v.shape
    if kind == 1:
        b = q(v)
        h = e0.astype(np.float64).reshape(R, hc, out)
        inj = e1.astype(np.float64).reshape(R, 8)[:, :hc]
        return b, q(h + q(b[:, None, :] * inj[:, :, None]))
    if kind == 2:
        t = q(v) / 4
        return q(t / (1 + np.exp(-t))), None
    if kind == 3:
        return q(v), None
    if kind == 5:
        return q(1 / (1 + np.exp(-q(v)))), None
    if kind == 6:
        A = (e0.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        dt = (e1.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        u = q(q(v) + dt)
        sp = q(np.where(u > 20, u, np.log1p(np.exp(np.minimum(u, 20)))))
        return np.exp(-np.exp(A) * sp), None
    raise ValueError(kind)


def bf_steps(a, b):
    """distance in bf16 steps of the larger magnitude"""
    step = np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -7 + 1e-30
    return np.abs(a - b) / step


@pytest.mark.parametrize("kind", [1, 2, 3, 5, 6])
@pytest.mark.parametrize("refr", [True, False])
def test_lin_epi_closed_forms(oracle, kind, refr):
    rng = np.random.default_rng(40 + kind)
    R, out, hc = 5, 384, 4
    v = (rng.standard_normal((R, out)) * 3).astype(np.float32)
    e0 = e1 = e2 = None
    if kind == 1:
        e0 = rng.standard_normal((R, hc, out)).astype(np.float32)
        e1 = rng.standard_normal((R, 8)).astype(np.float32)
        e2 = np.zeros_like(e0)
    if kind == 6:
        e0 = synth.bf16(rng.standard_normal(out).astype(np.float32))
        e1 = synth.bf16(rng.standard_normal(out).astype(np.float32))
        v[0, :8] = [0, 30, -30, 19.9, 20.5, 1e-3, -5, 5]  # both softplus branches
    y = oracle.lin_epi(v, kind, refr=refr, hc=hc, e0=e0, e1=e1, e2=e2)
    want, want2 = np_epi(v, kind, refr, hc, e0, e1)
    got = [(y, want)] + ([(e2, want2)] if kind == 1 else [])
    for g, w in got:
        g = g.astype(np.float64).reshape(w.shape)
        if refr and kind != 6:
            assert np.array_equal(bfr(g), g)  # the result is a bf16 value
            assert bf_steps(g, w).max() <= 1.0
            assert (g == w).mean() > 0.98  # f32 vs f64 transcendental boundaries only
        elif refr:
            assert np.allclose(g, w, rtol=2e-2, atol=1e-6)  # one interior rounding may flip a step
            assert (np.abs(g - w) <= 1e-5 * np.abs(w) + 1e-7).mean() > 0.98
        else:
            assert np.allclose(g, w, rtol=2e-5, atol=1e-7)


def test_lin_epi_known_answers(oracle):
    v = np.zeros((1, 2), np.float32)
    assert np.array_equal(oracle.lin_epi(v, 2), [[0, 0]])            # silu(0) = 0
    assert np.array_equal(oracle.lin_epi(v, 5), [[0.5, 0.5]])        # sigmoid(0) = 1/2
    e0 = synth.bf16(np.zeros(2, np.float32))                           # A_log 0: exp = 1; dt_bias 0
    y = oracle.lin_epi(v, 6, e0=e0, e1=e0.copy())
    sp = bfr(np.log(2.0))                                              # rr(softplus(0)) = rr(ln 2) = 0.69140625
    assert sp == 0.69140625 and np.allclose(y, np.exp(-sp), rtol=1e-6)
    y = oracle.lin_epi(np.array([[30.0, 1.0]], np.float32), 6, e0=e0, e1=e0.copy())
    assert np.isclose(y[0, 0], np.exp(-30.0), rtol=1e-5)              # u > 20: softplus(u) = u
    assert np.array_equal(oracle.lin_epi(np.array([[1.00390625, -2.5]], np.float32), 3), [[1.0, -2.5]])  # tie


def test_lin_epi_stride_and_cache(oracle):
    rng = np.random.default_rng(47)
    R, out = 3, 640
    v = rng.standard_normal((R, out)).astype(np.float32)
    base = np.full((R, 700), 7.0, np.float32)
    y = oracle.lin_epi(v, 0, ldy=700, y=base)
    assert np.array_equal(y[:, :out], v) and np.all(y[:, out:] == 7.0)
    cache = np.full((8, 128), -1.0, np.float32)
    y = oracle.lin_epi(v, 7, e0=cache, e1=np.array([4], np.uint32))
    assert np.array_equal(y, v)
    assert np.all(cache[:4] == -1.0)                                   # rows before T untouched
    assert np.array_equal(cache[4:7], v[:, 512:])                      # rows T..T+R-1 = the key columns
    assert np.all(cache[7] == -1.0)
    cache = np.full((5, 128), -1.0, np.float32)                        # capacity bound: row 5 and 6 dropped
    oracle.lin_epi(v, 7, e0=cache, e1=np.array([4], np.uint32))
    assert np.array_equal(cache[4], v[0, 512:]) and np.all(cache[:4] == -1.0)


# ------------------------------------------------------------------------------------------------ MoE HC write
def bf32(x):
    """f32 -> bf16 round to nearest even, in f32"""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("refr", [True, False])
def test_hc_write_closed_form(oracle, refr):
    rng = np.random.default_rng(60)
    R, hid, hc = 3, 256, 4
    s, t = (rng.standard_normal((R, hid)).astype(np.float32) for _ in range(2))
    h = rng.standard_normal((R, hc, hid)).astype(np.float32)
    inj = rng.standard_normal((R, 8)).astype(np.float32)
    q = bf32 if refr else (lambda a: np.asarray(a, np.float32))
    br = q(q(s) + q(t))                                                     # f32 adds and products, as in C
    want_h = q(h + q(br[:, None, :] * inj[:, :hc, None]))
    y, hout = oracle.hc_write(s, t, h, inj, refr=refr)
    assert np.array_equal(y, br) and np.array_equal(hout, want_h)
    y0, _ = oracle.hc_write(s, None, h, inj, refr=refr)                     # no shared expert: t = 0
    assert np.array_equal(y0, q(q(s)))


def test_moe_layer_hc_matches_plain_layer(oracle):
    """rounding off: the branch is the plain layer's slot-order sum bit for bit (the shared gate unrounded);
    rounding on: the branch is bf16-valued and within a few bf16 steps of the plain layer"""
    w = synth.moe_layer(13, hid=256, inter=128, ne=16, topk=4, K=5, shared=True, Ks=6, sgate=True)
    W = oracle.MoeWeights(w)
    rng = np.random.default_rng(14)
    R, hc = 2, 4
    x = synth.bf16_values(rng, R, 256)
    h = rng.standard_normal((R, hc, 256)).astype(np.float32)
    inj = rng.standard_normal((R, 8)).astype(np.float32)
    y_plain, _, _ = oracle.moe_layer(W, x)
    y, hout = oracle.moe_layer_hc(W, x, h, inj, refr=False)
    assert np.array_equal(y, y_plain)
    assert np.array_equal(hout, h + y[:, None, :] * inj[:, :hc, None])
    y1, hout1 = oracle.moe_layer_hc(W, x, h, inj, refr=True)
    assert np.array_equal(bf32(y1), y1) and np.array_equal(bf32(hout1), hout1)
    step = np.abs(y_plain) * 2.0 ** -7 + 1e-3 * np.abs(y_plain).max()
    assert np.all(np.abs(y1 - y_plain) <= 4 * step)


# ------------------------------------------------------------------------------------------------ HC read
def hc_case(seed, R=2, hid=128, lr=64, K=5):
    rng = np.random.default_rng(seed)
    h = (rng.standard_normal((R, 4, hid)) * np.array([0.5, 1, 2, 4])[None, :, None]).astype(np.float32)
    nw = synth.bf16((1 + 0.1 * rng.standard_normal(4 * hid)).astype(np.float32))
    iw = synth.bf16((rng.standard_normal((4, 4 * hid)) / np.sqrt(4 * hid)).astype(np.float32))
    down = synth.linear(rng, 4 * hid, lr, K)
    up = synth.linear(rng, lr, 4 * hid, K)
    return h, nw, iw, down, up


def np_hc_prep(h, nw, iw):
    R, _, hid = h.shape
    w = bf16_f64(nw).reshape(4, hid)
    inv = 1 / np.sqrt((h.astype(np.float64) ** 2).mean(axis=2) + 1e-6)         # [R, 4]
    xw = h.astype(np.float64) * w[None]
    xn = (xw * inv[:, :, None]).reshape(R, 4 * hid)
    ip = np.einsum("rsi,jsi->rsj", xw, bf16_f64(iw).reshape(4, 4, hid)) * inv[:, :, None]
    return xn, ip, inv


def bf16_f64(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_hc_prep_closed_form(oracle):
    h, nw, iw, _, _ = hc_case(90)
    xn, ip, inj = oracle.hc_prep(h, nw, iw)
    want_xn, want_ip, inv = np_hc_prep(h, nw, iw)
    assert np.allclose(inj[:, 4:], inv, rtol=1e-6) and np.all(inj[:, :4] == 0)
    assert np.allclose(xn, want_xn, rtol=2e-6, atol=1e-7)
    assert np.allclose(ip, want_ip, rtol=1e-5, atol=1e-6)
    # scale invariance: 1/rms cancels a scale of h (up to the 1e-6 epsilon: ~4e-6 relative at rms 0.5)
    xn2, _, inj2 = oracle.hc_prep(h * np.float32(8.0), nw, iw)
    assert np.allclose(xn2, xn, rtol=2e-5, atol=1e-7) and np.allclose(inj2[:, 4:] * 8, inj[:, 4:], rtol=2e-5)


@pytest.mark.parametrize("refr", [True, False])
def test_hc_out_closed_form(oracle, refr):
    rng = np.random.default_rng(91)
    h, nw, iw, _, _ = hc_case(92)
    R, _, hid = h.shape
    _, ip, inj = oracle.hc_prep(h, nw, iw)
    u = (rng.standard_normal((R, 4 * hid)) * 2).astype(np.float32)
    out, inj2 = oracle.hc_out(u, h, nw, ip, inj, refr=refr)
    q = bfr if refr else (lambda a: np.asarray(a, np.float64))
    inv = inj[:, 4:].astype(np.float64)
    sg = q(1 / (1 + np.exp(-q(u.reshape(R, 4, hid)))))
    v = q(sg * q(h * inv[:, :, None] * bf16_f64(nw).reshape(1, 4, hid)))
    want = q(((v[:, 0] + v[:, 1]) + (v[:, 2] + v[:, 3])) * 0.25)
    gates = q(2 / (1 + np.exp(-q(ip.astype(np.float64).sum(axis=1)) * 0.25)))
    if refr:
        assert bf_steps(out, want).max() <= 1.0 and (out == want).mean() > 0.97
        assert bf_steps(inj2[:, :4], gates).max() <= 1.0
    else:
        assert np.allclose(out, want, rtol=1e-5, atol=1e-7) and np.allclose(inj2[:, :4], gates, rtol=1e-6)
    assert np.array_equal(inj2[:, 4:], inj[:, 4:])


def test_hc_read_vs_f64(oracle):
    """the whole read (prep, down linear + silu(/4), up linear, sigmoid-weighted stream mean, gates) against f64
    numpy with explicit decoded matrices and no rounding: within the fp16 input preparation of the two linears"""
    h, nw, iw, down, up = hc_case(93)
    R, _, hid = h.shape
    mix, inj, out = oracle.hc_read(h, nw, iw, down, up, refr=False)
    xn, ip, inv = np_hc_prep(h, nw, iw)
    d = np_linear_exact(oracle, xn, *down) / 4
    want_mix = d / (1 + np.exp(-d))
    u = np_linear_exact(oracle, want_mix, *up).reshape(R, 4, hid)
    normed = h * inv[:, :, None] * bf16_f64(nw).reshape(1, 4, hid)
    want_out = (normed / (1 + np.exp(-u))).mean(axis=1)
    assert np.linalg.norm(mix - want_mix) / np.linalg.norm(want_mix) < 3e-3
    assert np.linalg.norm(out - want_out) / np.linalg.norm(want_out) < 3e-3
    assert np.allclose(inj[:, :4], 2 / (1 + np.exp(-ip.sum(axis=1) / 4)), rtol=1e-5)
    assert np.allclose(inj[:, 4:], inv, rtol=1e-6)


# ---------------------------------------------------------------------------------------------- 8-bit shared expert
def _bf(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32).astype(np.float64)


def _dequant(w_u32, sc, bi, group=128):
    """the explicit matrix W[o][i] = scale[o][i / group] q[o][i] + bias[o][i / group] (MLX affine, f64)"""
    q = np.ascontiguousarray(w_u32).view(np.uint8).astype(np.float64)
    return q * np.repeat(_bf(sc), group, axis=1) + np.repeat(_bf(bi), group, axis=1)


def _rr(v):
    """round f32 values to bf16 (RNE) and back"""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) & np.uint32(0xFFFF0000)).view(np.float32)


@pytest.mark.parametrize("inp,out", [(256, 64), (2048, 32), (640, 16)])
def test_q8_linear_vs_dequantized_matrix(oracle, inp, out):
    """orc_q8_linear against x @ W^T with W dequantized explicitly; a dropped bias or a scale on the wrong group fails"""
    from ijah_amd import synth
    rng = np.random.default_rng(inp + out)
    w, sc, bi = synth.q8_linear(rng, inp, out)
    x = rng.standard_normal((3, inp)).astype(np.float32)
    W = _dequant(w, sc, bi)
    want = x.astype(np.float64) @ W.T
    got = oracle.q8_linear(x, w, sc, bi)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    # mutations the check must catch: no bias; each group's scale and bias taken from the next group
    assert np.abs(x.astype(np.float64) @ (W - np.repeat(_bf(bi), 128, axis=1)).T - got).max() > 1e-3 * np.abs(got).max()
    if inp > 128:
        Ws = _dequant(w, np.roll(sc, 1, axis=1), np.roll(bi, 1, axis=1))
        assert np.abs(x.astype(np.float64) @ Ws.T - got).max() > 1e-3 * np.abs(got).max()


def test_q8_shared_closed_form(oracle):
    """the layer's 8-bit shared expert: g, u, h, o with the reference's bf16 rounding points (kernels/fn_moe.metal:47,
    268, 288), against numpy on the dequantized matrices; with the rounding off it is the plain f64 SwiGLU"""
    from ijah_amd import synth
    w = synth.moe_layer(71, hid=1024, inter=256, ne=4, topk=2, K=5, shared="q8")
    W = oracle.MoeWeights(w)
    x = synth.bf16_values(np.random.default_rng(72), 1, 1024)[0]
    Wg, Wu, Wd = (_dequant(w[f"sq8_{p}.weight"], w[f"sq8_{p}.scales"], w[f"sq8_{p}.biases"]) for p in
                  ("gate", "up", "down"))
    g, u = Wg @ x, Wu @ x
    h = g / (1 + np.exp(-g)) * u
    plain = Wd @ h
    assert np.abs(oracle.q8_shared(W, x, refr=False) - plain).max() <= 1e-5 * np.abs(plain).max()
    g, u = _rr(g), _rr(u)
    h = _rr((g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).astype(np.float32))
    o = _rr((Wd @ h).astype(np.float32))
    got = oracle.q8_shared(W, x, refr=True)
    assert np.mean(got == o) > 0.97 and np.all(np.abs(got - o) <= np.abs(o) * 2 ** -7 + 1e-7)
    assert np.array_equal(got, _rr(got))  # bf16-valued
    # the rounding points matter: without them the result differs
    assert np.mean(oracle.q8_shared(W, x, refr=False) == got) < 0.5


def test_moe_layer_q8_shared_term(oracle):
    """the layer with an 8-bit shared expert = the routed slots in slot order + sg * o (o = the shared expert)"""
    from ijah_amd import synth
    w = synth.moe_layer(73, hid=512, inter=128, ne=8, topk=3, K=5, shared="q8", sgate=True)
    W = oracle.MoeWeights(w)
    routed = dict(w)
    for k in [k for k in w if k.startswith("sq8_")]:
        del routed[k]
    Wr = oracle.MoeWeights(routed)
    x = synth.bf16_values(np.random.default_rng(74), 2, 512)
    y, lg, rt = oracle.moe_layer(W, x)
    sg = np.array([1 / (1 + np.exp(-np.float32(oracle.router_logits(x[r], w["sgate"][None])[0]))) for r in range(2)],
                  np.float32)
    s = oracle.moe_experts(Wr, x, rt, sg=sg)
    for r in range(2):
        want = s[r] + sg[r] * oracle.q8_shared(W, x[r])
        assert np.allclose(y[r], want, rtol=1e-6, atol=1e-7)
