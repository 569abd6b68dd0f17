"""The allocation-free linear (ne_exl3_lin_run_noalloc) through the C ABI against ne_exl3_lin_run on the same linear
and input: bit-identical outputs (the same kernels over the same partials, only their memory differs), on two calls in
a row with the second smaller, with the input prepared inside the GEMM and by a prep launch (many tile pairs times
many rows); and a run needing more scratch than the fixed per-GPU array is rejected with an error."""
import numpy as np
import pytest

from ijah_amd import synth
from ijah_amd.engine import EngineError

pytestmark = pytest.mark.gpu


def run_noalloc(eng, lin, x):
    R = x.shape[0]
    xb, yb = eng.from_numpy(np.ascontiguousarray(x, np.float32)), eng.alloc(R * lin.out * 4)
    eng._ok(eng.lib.ne_exl3_lin_run_noalloc(lin.ptr, R, xb.ptr, 0, yb.ptr, 0), "ne_exl3_lin_run_noalloc")
    return yb.download(np.float32, (R, lin.out))


@pytest.mark.parametrize("inp,out,K,rows", [
    (2048, 512, 5, (8, 3)),     # one launch, completion counters, the input prepared inside the GEMM
    (2048, 4096, 6, (32, 9)),   # 32 rows: a prep launch first; then 9 rows prepared inside the GEMM
    (144, 272, 4, (20, 5)),     # a partial k chunk
])
def test_noalloc_matches_run(eng, inp, out, K, rows):
    print(f"noalloc linear {inp}x{out} K{K} rows {rows}", flush=True)
    rng = np.random.default_rng(inp + out + K)
    t, su, sv = synth.linear(rng, inp, out, K)
    lin = eng.exl3_linear(t, su, sv)
    for R in rows:  # the second call smaller: it finds the first call's scratch contents
        x = synth.bf16_values(rng, R, inp)
        want = lin.run(x)
        got = run_noalloc(eng, lin, x)
        assert np.array_equal(got, want), (R, float(np.abs(got - want).max()))
        assert np.array_equal(run_noalloc(eng, lin, x), want), R  # again, with this call's contents left behind


def test_noalloc_rejects_oversize(eng):
    print("noalloc linear oversize", flush=True)
    rng = np.random.default_rng(9)
    t, su, sv = synth.linear(rng, 256, 262144, 2)
    lin = eng.exl3_linear(t, su, sv)
    x = synth.bf16_values(rng, 32, 256)
    with pytest.raises(EngineError, match="maximum"):
        run_noalloc(eng, lin, x)  # 32 rows of 262144 partials: 32 MiB of them alone
    assert np.array_equal(run_noalloc(eng, lin, x[:1]), lin.run(x[:1]))  # one row fits
