"""The allocation-free linear (ne_exl3_lin_run_noalloc) through the C ABI against ne_exl3_lin_run on the same linear
and input: bit-identical outputs (the same kernels over the same partials, only their memory differs), on two calls in
a row with the second smaller, with the input prepared inside the GEMM and by a prep launch (many tile pairs times
many rows) and for a vocabulary-wide linear (the looped k groups); captured into a HIP graph on the library's stream
(ne_stream) and replayed with other calls of it in between; and a run needing more scratch than the fixed per-GPU
array is rejected with an error."""
import ctypes as C
import os

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
    (512, 65536, 4, (8, 3)),    # a vocabulary-wide linear: the wide form at 8 rows, the looped one at 3
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


def hip_runtime():
    """the HIP runtime the library already uses (loaded with it), for the graph calls"""
    h = C.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD | os.RTLD_GLOBAL)
    vp = C.c_void_p
    for name, args in (("hipStreamBeginCapture", [vp, C.c_int]), ("hipStreamEndCapture", [vp, C.POINTER(vp)]),
                       ("hipGraphInstantiate", [C.POINTER(vp), vp, vp, C.c_char_p, C.c_size_t]),
                       ("hipGraphLaunch", [vp, vp]), ("hipStreamSynchronize", [vp]),
                       ("hipGraphExecDestroy", [vp]), ("hipGraphDestroy", [vp])):
        f = getattr(h, name)
        f.restype, f.argtypes = C.c_int, args
    return h


@pytest.mark.parametrize("inp,out,K,R", [(2048, 512, 5, 8), (2048, 4096, 6, 32)])
def test_noalloc_graph_replay(eng, inp, out, K, R):
    """a call captured on the library's stream replays to the captured input's result every time, with eager calls of
    the same entry point on another input (which leave their partials and counters in the shared array) between the
    replays: the zero-fill kernel, not a memset, clears what must start at zero"""
    print(f"noalloc graph replay {inp}x{out} K{K} R{R}", flush=True)
    hip = hip_runtime()
    rng = np.random.default_rng(inp + out + 7)
    t, su, sv = synth.linear(rng, inp, out, K)
    lin = eng.exl3_linear(t, su, sv)
    x1, x2 = synth.bf16_values(rng, R, inp), synth.bf16_values(rng, R, inp)
    want1, want2 = lin.run(x1), lin.run(x2)
    assert np.array_equal(run_noalloc(eng, lin, x2), want2)
    s = eng.lib.ne_stream()
    assert s, eng.last_error()
    xb, yb = eng.from_numpy(np.ascontiguousarray(x1, np.float32)), eng.alloc(R * out * 4)
    eng.sync()
    g, ex = C.c_void_p(), C.c_void_p()
    assert hip.hipStreamBeginCapture(s, 1) == 0  # thread-local capture mode
    rc = eng.lib.ne_exl3_lin_run_noalloc(lin.ptr, R, xb.ptr, 0, yb.ptr, 0)
    assert hip.hipStreamEndCapture(s, C.byref(g)) == 0
    assert rc == 0, eng.last_error()
    try:
        assert hip.hipGraphInstantiate(C.byref(ex), g, None, None, 0) == 0
        for i in range(3):
            assert np.array_equal(run_noalloc(eng, lin, x2), want2), i
            assert hip.hipGraphLaunch(ex, s) == 0
            assert hip.hipStreamSynchronize(s) == 0
            got = yb.download(np.float32, (R, out))
            assert np.array_equal(got, want1), (i, float(np.abs(got - want1).max()))
    finally:
        if ex.value:
            hip.hipGraphExecDestroy(ex)
        hip.hipGraphDestroy(g)
