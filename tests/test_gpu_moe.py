"""GPU parity of the fused MoE layer (router, top-k, routed + shared EXL3 experts, combine) against the CPU oracle.

Checks, per the reference's layer tests (tests/test_fn_layer.py:86-126,271-312; tools/compare.py:22-36, tie-aware
top-k at :94): logits within one bf16 step; the route bit-exact given the GPU's logits (ids) and within 1e-6 (weights);
the layer output within rel-L2 1e-4 of the oracle's kernel arithmetic on that route and within 1e-2 of the exact f64
layer; decoded expert weights bit-exact through the re-laid HBM blocks.
"""
import numpy as np
import pytest

from ijah_amd import synth

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def check_layer(eng, oracle, moe, W, x, tol=1e-4, exact=True):
    R = x.shape[0]
    y = moe.run(x)
    lg, rt, sg = moe.read("logits", R), moe.read("route", R), moe.read("shared_gate", R)
    topk = W.d["topk"]
    for r in range(R):
        want_lg = oracle.router_logits(x[r], W.d["router"])
        assert np.all(np.abs(lg[r] - want_lg) <= np.abs(want_lg) * 2 ** -7 + 1e-6)
        ids, w = oracle.route(lg[r], topk)
        assert np.array_equal(rt[r, :topk], ids)
        assert np.allclose(rt[r, topk:].view(np.float32), w, rtol=1e-6, atol=0)
    if W.d.get("sgate") is not None:
        for r in range(R):
            l = oracle.router_logits(x[r], W.d["sgate"][None])[0]
            # the gate logit, like the others, may round to the neighbouring bf16 value (sigmoid' <= 1/4)
            assert abs(sg[r] - 1 / (1 + np.exp(-np.float64(l)))) < 0.25 * abs(l) * 2 ** -7 + 1e-6
    else:
        assert np.all(sg == 1.0)
    sgv = sg if W.d.get("sgate") is not None else None
    want = oracle.moe_experts(W, x, rt, sg=sgv)
    assert rel(y, want) < tol
    if exact:
        assert rel(y, oracle.moe_experts(W, x, rt, sg=sgv, exact=True)) < 1e-2
    assert np.array_equal(moe.read("mlp_out", R), y)
    return y, rt


@pytest.mark.parametrize("R,shared,sgate", [(1, True, False), (1, False, False), (3, True, True)])
def test_moe_small(eng, oracle, R, shared, sgate):
    print(f"moe ne64 R{R} shared={shared} sgate={sgate}", flush=True)
    w = synth.moe_layer(21 + R, hid=2048, inter=512, ne=64, topk=10, K=5, shared=shared, Ks=5, sgate=sgate)
    W = oracle.MoeWeights(w)
    moe = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(5 + R), R, 2048)
    y, _ = check_layer(eng, oracle, moe, W, x)
    assert np.array_equal(y, moe.run(x))  # deterministic


def test_moe_mixed_bits(eng, oracle):
    """K4 routed experts (the MTP head's) with a K6 shared expert in one launch (per-slot K)."""
    print("moe K4 + shared K6", flush=True)
    w = synth.moe_layer(31, hid=1024, inter=256, ne=32, topk=8, K=4, shared=True, Ks=6)
    W = oracle.MoeWeights(w)
    x = synth.bf16_values(np.random.default_rng(32), 2, 1024)
    check_layer(eng, oracle, eng.moe_create(w), W, x)


def test_moe_config2_full(eng, oracle):
    """Config 2 at full size: 512 experts (1 GB of K5 trellis), hidden 2048, inter 512, top-10 + shared."""
    print("moe config2 ne512", flush=True)
    w = synth.moe_layer(2, hid=2048, inter=512, ne=512, topk=10, K=5, shared=True, Ks=5)
    W = oracle.MoeWeights(w)
    moe = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(3), 1, 2048)
    check_layer(eng, oracle, moe, W, x)
    for e in (int(moe.read("route")[0, 0]), 0, 511):
        for proj, key in ((0, "gate"), (1, "up"), (2, "down")):
            got = moe.decode(e, proj).view(np.uint16)
            assert np.array_equal(got, oracle.decode(w[f"{key}.trellis"][e]).view(np.uint16)), (e, proj)
    assert np.array_equal(moe.decode(512, 2).view(np.uint16), oracle.decode(w["sdown_proj.trellis"]).view(np.uint16))


def test_moe_zero_input_ties(eng, oracle):
    """x = 0: every logit ties at 0, so the route is experts 0..9 (lower index first) with weight 1/10, and y = 0."""
    w = synth.moe_layer(41, hid=1024, inter=256, ne=32, topk=10, K=5, shared=True)
    moe = eng.moe_create(w)
    y = moe.run(np.zeros((1, 1024), np.float32))
    rt = moe.read("route")
    assert np.array_equal(rt[0, :10], np.arange(10))
    assert np.allclose(rt[0, 10:].view(np.float32), 0.1, rtol=1e-6)
    assert np.all(y == 0)


def test_moe_pack_loader_matches_arrays(eng, oracle, tmp_path):
    """ne_moe_load (safetensors pack, 2 shards, re-laid on load) gives bit-identical output to ne_moe_create."""
    w = synth.moe_layer(51, hid=1024, inter=256, ne=16, topk=4, K=5, shared=True, Ks=6, sgate=True)
    prefix = synth.write_moe_pack(tmp_path, w, layer=7, shards=2)
    p = eng.pack_open(tmp_path)
    a, b = eng.moe_load(p, prefix, 4), eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(52), 2, 1024)
    ya = a.run(x)
    assert np.array_equal(ya, b.run(x))
    check_layer(eng, oracle, a, oracle.MoeWeights(w), x)


def test_moe_graph_replay_matches_eager(eng):
    """The timed path (HIP graph of a layer chain, replayed) computes what the eager call does, on every replay."""
    layers = [eng.moe_synth(1024, 256, 64, 8, 5, True, 5, seed=s) for s in (1, 2)]
    x = synth.bf16_values(np.random.default_rng(1), 1, 1024)
    xb = eng.from_numpy(x)
    eager = [m.run(x) for m in layers]
    for _ in range(3):
        us = eng.moe_time(layers, 1, xb, warmup=1, reps=2)
        assert us > 0
        for m, e in zip(layers, eager):
            assert np.array_equal(m.run(x), e)


def test_moe_synth_full_properties(eng):
    """Config 2 at full size on device-generated weights: route validity, finiteness, determinism, byte count."""
    m = eng.moe_synth(2048, 512, 512, 10, 5, True, 5, seed=7)
    x = synth.bf16_values(np.random.default_rng(8), 1, 2048)
    y = m.run(x)
    assert np.isfinite(y).all() and np.abs(y).max() > 0
    rt = m.read("route")
    ids, wt = rt[0, :10], rt[0, 10:].view(np.float32)
    lg = m.read("logits")[0]
    assert len(set(ids.tolist())) == 10 and ids.max() < 512
    assert np.all(np.diff(lg[ids]) <= 0) and abs(wt.sum() - 1) < 1e-5 and np.all(np.diff(wt) <= 0)
    assert np.array_equal(y, m.run(x))
    per_expert = 3 * 2048 * 512 * 5 // 8 + 2 * 3 * (2048 + 512)
    assert m.bytes(1) == 11 * per_expert + 512 * 2048 * 2


def test_moe_fused_and_staged_paths_agree(eng, oracle):
    """The persistent fused launch and the four staged launches compute the same layer (same decode, prep and combine
    arithmetic; the f32 k-accumulation order differs), and each is deterministic; the inner outputs agree too."""
    w = synth.moe_layer(61, hid=2048, inter=512, ne=64, topk=10, K=5, shared=True, Ks=6, sgate=True)
    x = synth.bf16_values(np.random.default_rng(62), 1, 2048)  # the fused step serves one row
    st = eng.moe_create(w).configure("staged", 1)
    ys = st.run(x)
    m = eng.moe_create(w)
    yf = m.run(x)
    assert rel(yf, ys) < 1e-5
    for name in ("experts_gu", "experts_dn"):
        assert rel(m.read(name), st.read(name)) < 1e-5, name
    for _ in range(3):  # counters reset between launches
        assert np.array_equal(m.run(x), yf)
    check_layer(eng, oracle, m, oracle.MoeWeights(w), x)


@pytest.mark.parametrize("Ks", [4, 5, 6])
def test_moe_m1_k4_mtp_head(eng, oracle, Ks):
    """The MTP head's MoE at M=1: K4 routed experts (reference core/main_test.mm:371, mtp_k = 4) at the config-2
    shape, with a K4 / K5 / K6 shared expert, on the fused single-row kernel (moe_step<4, Ks>); against the oracle
    and the staged kernels."""
    print(f"moe M=1 K4 shared K{Ks}", flush=True)
    w = synth.moe_layer(110 + Ks, hid=2048, inter=512, ne=64, topk=10, K=4, shared=True, Ks=Ks, sgate=True)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(111 + Ks), 1, 2048)
    y, _ = check_layer(eng, oracle, m, W, x)
    assert np.array_equal(m.run(x), y)
    assert rel(eng.moe_create(w).configure("staged", 1).run(x), y) < 5e-5  # same arithmetic, other f32 accumulation orders


@pytest.mark.parametrize("R", [1, 4])
def test_moe_reference_shape_2560(eng, oracle, R):
    """The reference's own layer shape (hidden 2560, intermediate 640: kernels/fn_moe.metal:16), top-10 + shared,
    K5 routed and K6 shared; one row (staged kernels) and four rows (the grouped matrix-core path)."""
    print(f"moe 2560x640 R{R}", flush=True)
    w = synth.moe_layer(120 + R, hid=2560, inter=640, ne=64, topk=10, K=5, shared=True, Ks=6, sgate=True)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(121 + R), R, 2560)
    y, _ = check_layer(eng, oracle, m, W, x)
    assert np.array_equal(m.run(x), y)


# ---------------------------------------------------------------------------------------------- batched path (R >= 2)
@pytest.mark.parametrize("R", [16, 200, 640])
def test_moe_batch_chunks(eng, oracle, R):
    """R rows through the grouped matrix-core path: experts with more than one 128-row chunk (the shared expert at
    R = 200, ~50 rows per routed expert), ties and order checked against the oracle on the GPU's route. R = 640 takes
    the many-row router."""
    print(f"moe batch R{R}", flush=True)
    w = synth.moe_layer(70 + R, hid=1024, inter=256, ne=16, topk=4, K=5, shared=True, Ks=6, sgate=True)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(71), R, 1024)
    y, _ = check_layer(eng, oracle, m, W, x, exact=R <= 16)
    assert np.array_equal(m.run(x), y)  # deterministic despite the unordered placement inside an expert


@pytest.mark.parametrize("R", [32, 33])
def test_moe_batch_row_block_forms(eng, oracle, R):
    """64 experts, top-10 + shared: at 32 rows the GEMMs take their one-row-block form and the shared expert fills a
    whole 32-row chunk; at 33 rows the 128-row form (both row-major: few rows per routed expert)."""
    print(f"moe batch forms R{R}", flush=True)
    w = synth.moe_layer(90 + R, hid=1024, inter=256, ne=64, topk=10, K=5, shared=True, Ks=5, sgate=True)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(91), R, 1024)
    y, _ = check_layer(eng, oracle, m, W, x, exact=False)
    assert np.array_equal(m.run(x), y)


def test_moe_batch_matches_staged(eng, oracle):
    """The grouped path and the staged kernels compute the same layer for several rows."""
    w = synth.moe_layer(81, hid=2048, inter=512, ne=64, topk=10, K=5, shared=True, Ks=5, sgate=False)
    x = synth.bf16_values(np.random.default_rng(82), 5, 2048)
    ys = eng.moe_create(w).configure("staged", 1).run(x)
    yb = eng.moe_create(w).run(x)
    assert rel(yb, ys) < 1e-4  # matrix-core vs lane accumulation order; fp16 rounding of h may flip


def test_moe_verify_config4(eng, oracle):
    """Config 4: 16 rows of the config-2 layer (512 experts, top-10, K5 + shared K5), independent routing per row."""
    print("moe verify R16 ne512", flush=True)
    w = synth.moe_layer(4, hid=2048, inter=512, ne=512, topk=10, K=5, shared=True, Ks=5)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(44), 16, 2048)
    check_layer(eng, oracle, m, W, x, exact=False)


def test_moe_verify_config4_k4(eng, oracle):
    """Config 4's K4 variant at full size: 16 rows of a 512-expert layer, top-10, K4 routed + K4 shared."""
    print("moe verify R16 ne512 K4", flush=True)
    w = synth.moe_layer(44, hid=2048, inter=512, ne=512, topk=10, K=4, shared=True, Ks=4)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(45), 16, 2048)
    check_layer(eng, oracle, m, W, x, exact=False)


def _rows_match_one_row(m, x, R):
    """every row of an R-row batch equals the one-row step on that row, bit for bit: logits, route, shared gate,
    layer output"""
    y = m.run(x)
    lg, rt, sg = m.read("logits", R), m.read("route", R), m.read("shared_gate", R)
    for i in range(R):
        y1 = m.run(x[i:i + 1])
        assert np.array_equal(m.read("logits", 1)[0], lg[i]), ("logits", i)
        assert np.array_equal(m.read("route", 1)[0], rt[i]), ("route", i)
        assert np.array_equal(m.read("shared_gate", 1)[0], sg[i]), ("shared gate", i)
        assert np.array_equal(y1[0], y[i]), ("output", i, rel(y1[0], y[i]))
    return y


@pytest.mark.parametrize("ne,K,Ks,sgate", [(64, 5, 5, True), (64, 4, 6, False), (64, 6, 6, True)])
def test_moe_verify_rows_bit_identical_to_one_row(eng, ne, K, Ks, sgate):
    """Speculative verify (16 rows through the grouped matrix-core kernels) against the fused one-row step: the same
    router arithmetic, prepared input and k-chunk fold order, so each row is bit-identical to that row run alone."""
    print(f"moe verify rows vs one row ne{ne} K{K}/{Ks} sgate={sgate}", flush=True)
    w = synth.moe_layer(130 + K + Ks, hid=2048, inter=512, ne=ne, topk=10, K=K, shared=True, Ks=Ks, sgate=sgate)
    m = eng.moe_create(w)
    _rows_match_one_row(m, synth.bf16_values(np.random.default_rng(131 + K), 16, 2048), 16)


def test_moe_verify_config4_rows_bit_identical(eng):
    """Config 4 at full size (512 experts, top-10 + shared, K5, device-generated): every one of the 16 verify rows
    equals the fused one-row step on that row, bit for bit."""
    print("moe verify config4 rows vs one row", flush=True)
    m = eng.moe_synth(2048, 512, 512, 10, 5, True, 5, seed=4)
    _rows_match_one_row(m, synth.bf16_values(np.random.default_rng(46), 16, 2048), 16)


def test_moe_verify_32_rows_small_shape_bit_identical(eng):
    """The largest verify batch (32 rows) at hidden 1024 / inter 256 (two k groups per column), no shared expert."""
    print("moe verify R32 1024x256 rows vs one row", flush=True)
    w = synth.moe_layer(140, hid=1024, inter=256, ne=32, topk=8, K=5, shared=False)
    m = eng.moe_create(w)
    _rows_match_one_row(m, synth.bf16_values(np.random.default_rng(141), 32, 1024), 32)


def test_moe_prefill_config5_rows_vs_oracle(eng, oracle):
    """Config 5 at full size with host weights (4096 rows, 512 experts, top-10 + shared, K5): sampled rows of the
    grouped layer against the oracle directly (logits within one bf16 step, the route on the GPU's logits, the
    row's output at rel-L2 1e-4 of the oracle's kernel arithmetic)."""
    print("moe config5 R4096 sampled rows vs oracle", flush=True)
    w = synth.moe_layer(5, hid=2048, inter=512, ne=512, topk=10, K=5, shared=True, Ks=5)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(6), 4096, 2048)
    y = m.run(x)
    assert np.isfinite(y).all()
    lg, rt = m.read("logits", 4096), m.read("route", 4096)
    for i in (0, 1, 777, 2048, 3001, 4095):
        want_lg = oracle.router_logits(x[i], W.d["router"])
        assert np.all(np.abs(lg[i] - want_lg) <= np.abs(want_lg) * 2 ** -7 + 1e-6), i
        ids, wt = oracle.route(lg[i], 10)
        assert np.array_equal(rt[i, :10], ids), i
        assert np.allclose(rt[i, 10:].view(np.float32), wt, rtol=1e-6, atol=0), i
        want = oracle.moe_experts(W, x[i:i + 1], rt[i:i + 1])
        assert rel(y[i:i + 1], want) < 1e-4, i


def test_moe_prefill_config5_rows_match_single_row(eng):
    """Config 5 at full size (4096 rows, 512 experts, top-10 + shared, K5, device-generated weights): every sampled
    row of the grouped matrix-core layer equals the fused single-row layer on that row (rows are independent; only
    the f32 accumulation order differs), with the same route, and the batched output is deterministic."""
    print("moe config5 R4096 rows vs single row", flush=True)
    m = eng.moe_synth(2048, 512, 512, 10, 5, True, 5, seed=5)
    x = synth.bf16_values(np.random.default_rng(6), 4096, 2048)
    y = m.run(x)
    assert np.isfinite(y).all()
    rt, lg = m.read("route", 4096), m.read("logits", 4096)
    assert np.array_equal(y, m.run(x))
    same = 0
    for i in (0, 1, 777, 2048, 4095):
        y1 = m.run(x[i:i + 1])
        r1, l1 = m.read("route", 1)[0], m.read("logits", 1)[0]
        # the two router kernels sum in different orders: a logit may round to the neighbouring bf16 value
        assert np.all(np.abs(l1[:512] - lg[i, :512]) <= np.abs(lg[i, :512]) * 2.0 ** -7 + 1e-6), i
        if not np.array_equal(r1[:10], rt[i, :10]):
            continue  # such a logit changed the ranking: the rows legitimately route differently
        assert rel(y1[0], y[i]) < 1e-4, i
        same += 1
    assert same >= 3


# ------------------------------------------------------------------------------------------------ HC write
@pytest.mark.parametrize("R,path,dims", [
    (1, "fused", (2048, 512, 64, 10)), (1, "staged", (2048, 512, 64, 10)), (3, "staged", (1024, 256, 16, 4)),
    (3, "batched", (1024, 256, 16, 4)), (16, "batched", (1024, 256, 16, 4)), (40, "batched", (1024, 256, 16, 4))])
def test_moe_hc_write(eng, oracle, R, path, dims):
    """ne_moe_run_hc, the hyper-connection write fused into the combine (reference kernels/fn_moe.metal:437-448), on
    the fused single-row kernel, the staged kernels and the batched GEMM forms (16 rows: the one-row-block form, 40
    rows x 4 slots over 16 experts: the transposed form). Rounding off: the branch is the plain run's output bit for
    bit and hout = h + branch * inj exactly. Rounding on: against the oracle layer with the write, within bf16 flips
    where the GPU's and the oracle's f32 sums straddle a rounding boundary."""
    hid, inter, ne, topk = dims
    print(f"moe hc write R{R} {path} hid {hid} ne {ne}", flush=True)
    w = synth.moe_layer(70 + R, hid=hid, inter=inter, ne=ne, topk=topk, K=5, shared=True, Ks=6, sgate=True)
    W = oracle.MoeWeights(w)
    moe = eng.moe_create(w)
    if path == "staged":
        moe.configure("staged", 1)
    rng = np.random.default_rng(80 + R)
    x = synth.bf16_values(rng, R, hid)
    hc = 4
    h = rng.standard_normal((R, hc, hid)).astype(np.float32)
    inj = rng.standard_normal((R, 8)).astype(np.float32)
    xb, hb, ib = eng.from_numpy(x), eng.from_numpy(h), eng.from_numpy(inj)
    y_plain = moe.run(x)
    yb, ob = eng.alloc(R * hid * 4), eng.alloc(h.nbytes)
    moe.run_hc(R, xb, yb, hb, ib, ob, hc=hc, refr=False)
    y0, o0 = yb.download(np.float32, (R, hid)), ob.download(np.float32, h.shape)
    assert np.array_equal(y0, y_plain)
    assert np.array_equal(o0, h + y0[:, None, :] * inj[:, :hc, None])
    moe.run_hc(R, xb, yb, hb, ib, ob, hc=hc, refr=True)
    y1, o1 = yb.download(np.float32, (R, hid)), ob.download(np.float32, h.shape)
    want_y, want_o = oracle.moe_layer_hc(W, x, h, inj, refr=True)
    for g, wv in ((y1, want_y), (o1, want_o)):
        assert np.array_equal((g.view(np.uint32) & 0xFFFF), np.zeros(g.shape, np.uint32))  # bf16 values
        assert (g == wv).mean() > 0.97
        assert rel(g, wv) < 3e-3
    assert np.array_equal(moe.read("mlp_out", R), y1)
    moe.run_hc(R, xb, yb, hb, ib, hb, hc=hc, refr=True)  # in place (hout = h)
    assert np.array_equal(hb.download(np.float32, h.shape), o1)
    assert np.array_equal(moe.run(x), y_plain)  # the plain run after the write is unchanged


def test_moe_hc_rejects(eng, oracle):
    w = synth.moe_layer(5, hid=1024, inter=256, ne=16, topk=4, K=5, shared=True, Ks=6, sgate=True)
    moe = eng.moe_create(w)
    x = eng.from_numpy(np.zeros((2, 1024), np.float32))
    y, h, inj = eng.alloc(2 * 1024 * 4), eng.alloc(2 * 4 * 1024 * 4), eng.alloc(2 * 8 * 4)
    with pytest.raises(RuntimeError, match="hc 0"):
        moe.run_hc(2, x, y, h, inj, h, hc=0)
    with pytest.raises(RuntimeError, match="h missing or under"):
        moe.run_hc(2, x, y, h, inj, h, hc=5)
    with pytest.raises(RuntimeError, match="inj missing or under"):
        moe.run_hc(2, x, y, h, eng.alloc(16), h, hc=4)


def test_hc_read_then_moe_hc_write(eng, oracle):
    """The reference's MLP block order (models/flash_next/layer_t6.mm:141-144, then kernels/fn_moe.metal:437-448): the
    HC read's out and inj buffers feed ne_moe_run_hc directly. Against the oracle layer with the write run on the
    GPU read's own outputs (the read itself is checked against the oracle in test_hc_read)."""
    from ijah_amd.engine import hc_read
    print("hc read -> moe hc write, hid 1024", flush=True)
    hid, R = 1024, 3
    rng = np.random.default_rng(97)
    w = synth.moe_layer(97, hid=hid, inter=256, ne=16, topk=4, K=5, shared=True, Ks=6, sgate=True)
    W = oracle.MoeWeights(w)
    moe = eng.moe_create(w)
    h = (rng.standard_normal((R, 4, hid)) * np.array([0.5, 1, 2, 4])[None, :, None]).astype(np.float32)
    nw = synth.bf16((1 + 0.1 * rng.standard_normal(4 * hid)).astype(np.float32))
    iw = synth.bf16((rng.standard_normal((4, 4 * hid)) / np.sqrt(4 * hid)).astype(np.float32))
    ld, lu = eng.exl3_linear(*synth.linear(rng, 4 * hid, 128, 6)), eng.exl3_linear(*synth.linear(rng, 128, 4 * hid, 6))
    hb = eng.from_numpy(h)
    mb, jb, xb = eng.alloc(R * 128 * 4), eng.alloc(R * 32), eng.alloc(R * hid * 4)
    hc_read(ld, lu, R, hb, eng.from_numpy(nw), eng.from_numpy(iw), mb, jb, xb)
    yb, ob = eng.alloc(R * hid * 4), eng.alloc(h.nbytes)
    moe.run_hc(R, xb, yb, hb, jb, ob, hc=4)
    x, inj = xb.download(np.float32, (R, hid)), jb.download(np.float32, (R, 8))
    y, hout = yb.download(np.float32, (R, hid)), ob.download(np.float32, h.shape)
    want_y, want_o = oracle.moe_layer_hc(W, x, h, inj, refr=True)
    for g, wv in ((y, want_y), (hout, want_o)):
        assert (g == wv).mean() > 0.97 and rel(g, wv) < 3e-3
    assert np.all(np.abs(inj[:, :4]) <= 2) and np.all(inj[:, 4:] > 0)  # gates 2 sigmoid, 1/rms


# ---------------------------------------------------------------------------------------------- 8-bit shared expert
def check_q8_layer(eng, oracle, moe, W, x, sgate):
    """The layer with the reference's 8-bit affine shared expert (kernels/fn_moe.metal:40-46, :264-290): the shared
    output o = rr(down . rr(silu(rr g) rr u)) within one bf16 step of the oracle's (the GPU's f32 sums and the
    oracle's f64 ones may round to neighbouring bf16 values; near zero, within 2^-12 of the row's rms), >= 95% of it
    bit-exact; the layer within rel-L2 1e-3 of
    the oracle's kernel arithmetic on the GPU's route and within 1e-2 of the f64 layer."""
    R = x.shape[0]
    y = moe.run(x)
    rt, sg = moe.read("route", R), moe.read("shared_gate", R)
    o = moe.read("shared_q8", R)
    y_all = y
    if R > 40:  # many rows: sampled rows against the oracle (its layer costs ~1 s a row)
        rows = [0, 1, R // 2, R - 1]
        x, y, rt, sg, o = x[rows], y[rows], rt[rows], sg[rows], o[rows]
        R = len(rows)
    for r in range(R):
        want = oracle.q8_shared(W, x[r])
        assert np.mean(o[r] == want) > 0.95, (r, np.mean(o[r] == want))
        # one bf16 step of the value, or (an output near zero, where the sums cancel) a small part of the row's scale
        scale = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
        assert np.all(np.abs(o[r] - want) <= np.abs(want) * 2 ** -6 + scale * 2 ** -12), r
    sgv = sg if sgate else None
    assert rel(y, oracle.moe_experts(W, x, rt, sg=sgv)) < 1e-3
    assert rel(y, oracle.moe_experts(W, x, rt, sg=sgv, exact=True)) < 1e-2
    return y_all


@pytest.mark.parametrize("R", [1, 3, 16, 40, 200])
def test_moe_q8_shared_expert(eng, oracle, R):
    """R = 1 runs the fused one-row step, 3 and 16 the few-row kernels, 40 and 200 the many-row ones (the shared
    expert on the matrix cores: bf16 weights, x split into bf16 hi + lo); each with the 8-bit shared expert and its
    gate."""
    print(f"moe q8 shared R{R}", flush=True)
    w = synth.moe_layer(150 + R, hid=2048, inter=512, ne=64, topk=10, K=5, shared="q8", sgate=True)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(151 + R), R, 2048)
    y = check_q8_layer(eng, oracle, m, oracle.MoeWeights(w), x, True)
    assert np.array_equal(y, m.run(x))


@pytest.mark.parametrize("R", [1, 4])
def test_moe_q8_reference_shape(eng, oracle, R):
    """The reference's own shape (hidden 2560, inter 640; kernels/fn_moe.metal:16) with its 8-bit shared expert."""
    print(f"moe q8 shared 2560x640 R{R}", flush=True)
    w = synth.moe_layer(160 + R, hid=2560, inter=640, ne=32, topk=10, K=5, shared="q8", sgate=True)
    m = eng.moe_create(w)
    check_q8_layer(eng, oracle, m, oracle.MoeWeights(w), synth.bf16_values(np.random.default_rng(161), R, 2560), True)


def test_moe_q8_verify_rows_bit_identical_to_one_row(eng):
    """With the 8-bit shared expert, every row of a 16-row verify batch equals the fused one-row step on that row,
    bit for bit (the shared rows' dot is the same function in both paths)."""
    print("moe q8 verify rows vs one row", flush=True)
    w = synth.moe_layer(170, hid=2048, inter=512, ne=64, topk=10, K=5, shared="q8", sgate=True)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(171), 16, 2048)
    _rows_match_one_row(m, x, 16)
    m.run(x)
    o16 = m.read("shared_q8", 16)
    for i in (0, 7, 15):
        m.run(x[i:i + 1])
        assert np.array_equal(m.read("shared_q8", 1)[0], o16[i]), i


def test_moe_q8_pack_loader(eng, oracle, tmp_path):
    """A pack whose shared expert is 8-bit (.weight U32 / .scales / .biases BF16, g128, the reference's real layout)
    loads through ne_moe_load and gives the same output as the arrays."""
    w = synth.moe_layer(180, hid=1024, inter=256, ne=16, topk=4, K=5, shared="q8", sgate=True)
    prefix = synth.write_moe_pack(tmp_path, w, layer=2)
    a, b = eng.moe_load(eng.pack_open(tmp_path), prefix, 4), eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(181), 2, 1024)
    assert np.array_equal(a.run(x), b.run(x))
    assert np.array_equal(a.run(x[:1]), b.run(x[:1]))
    check_q8_layer(eng, oracle, a, oracle.MoeWeights(w), x, True)


def test_moe_q8_hc_write(eng, oracle):
    """The hyper-connection write with the 8-bit shared expert, rounding on: the branch and the streams against the
    oracle layer with the write (rr(sigmoid) gate, rr(gate * o))."""
    print("moe q8 hc write", flush=True)
    w = synth.moe_layer(190, hid=2048, inter=512, ne=64, topk=10, K=5, shared="q8", sgate=True)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    rng = np.random.default_rng(191)
    for R in (1, 4):
        x = synth.bf16_values(rng, R, 2048)
        h = rng.standard_normal((R, 4, 2048)).astype(np.float32)
        inj = rng.standard_normal((R, 8)).astype(np.float32)
        xb, yb, hb, ib, ob = (eng.from_numpy(x), eng.alloc(R * 2048 * 4), eng.from_numpy(h), eng.from_numpy(inj),
                              eng.alloc(h.nbytes))
        m.run_hc(R, xb, yb, hb, ib, ob, hc=4, refr=True)
        y, hout = yb.download(np.float32, (R, 2048)), ob.download(np.float32, h.shape)
        wy, whout = oracle.moe_layer_hc(W, x, h, inj, refr=True)
        assert np.mean(y == wy) > 0.9 and rel(y, wy) < 3e-3, (R, np.mean(y == wy), rel(y, wy))
        assert rel(hout, whout) < 3e-3


def test_few_row_pool_shared_by_layers(eng):
    """Two layers of one shape share the few-row kernels' scratch pool: layer A at 4 rows, then B at 32 rows (the
    pool grows), then A at 4 rows again gives A's first output (A takes the pool's current arrays)."""
    print("moe few-row pool shared by layers", flush=True)
    a = eng.moe_synth(1024, 256, 64, 8, 5, True, 5, seed=21)
    b = eng.moe_synth(1024, 256, 64, 8, 5, True, 5, seed=22)
    rng = np.random.default_rng(23)
    x4, x32 = synth.bf16_values(rng, 4, 1024), synth.bf16_values(rng, 32, 1024)
    y4 = a.run(x4)
    yb = b.run(x32)
    assert np.array_equal(a.run(x4), y4)
    assert np.array_equal(b.run(x32), yb)
    assert np.array_equal(a.run(x4), y4)


@pytest.mark.parametrize("R", [2, 4, 6, 8])
def test_moe_verify_draft_sizes_bit_identical(eng, R):
    """The reference's draft sizes (grouped verify at R = 2 .. 8, docs/mtp.md:987-993), config 2's layer at full size
    (512 experts, top-10 + shared, K5): every row equals the fused one-row step on that row, bit for bit."""
    print(f"moe verify R{R} rows vs one row", flush=True)
    m = eng.moe_synth(2048, 512, 512, 10, 5, True, 5, seed=50 + R)
    _rows_match_one_row(m, synth.bf16_values(np.random.default_rng(51 + R), R, 2048), R)


@pytest.mark.parametrize("shared,K,Ks", [(True, 5, 5), (True, 5, 6), (True, 4, 4), ("q8", 5, 5), ("q8", 6, 6)])
def test_moe_fused_reference_shape(eng, oracle, shared, K, Ks):
    """The fused one-row step at the reference's own shape (hidden 2560, inter 640: kernels/fn_moe.metal:16), where a
    workgroup's units outnumber its LDS slots and some down units take a finished gate/up chunk's slot: the step is
    the fused launch (its kernel timed by ne_moe_time_kernels), against the oracle, and bit-identical to itself."""
    print(f"moe fused 2560x640 shared={shared} K{K}/{Ks}", flush=True)
    w = synth.moe_layer(200 + K + Ks, hid=2560, inter=640, ne=64, topk=10, K=K, shared=shared, Ks=Ks, sgate=True)
    W = oracle.MoeWeights(w)
    m = eng.moe_create(w)
    x = synth.bf16_values(np.random.default_rng(201 + K), 1, 2560)
    assert "fused" in eng.moe_time_kernels([m], 1, eng.from_numpy(x), reps=1)
    y = check_q8_layer(eng, oracle, m, W, x, True) if shared == "q8" else check_layer(eng, oracle, m, W, x)[0]
    for _ in range(2):
        assert np.array_equal(m.run(x), y)
    if shared is True:  # the verify rows of this shape agree with the fused step, bit for bit
        _rows_match_one_row(m, synth.bf16_values(np.random.default_rng(202), 4, 2560), 4)
