"""CPU tests of the library's stream-capture and buffer-lifetime invariants, on its host code built against a host-only
HIP stand-in (tests/hoststub: device memory is host memory; every allocation, free, memset, attribute change, capture,
graph and launch is tracked, and every kernel launcher records the buffers its arguments point to).

Checked for the timing entry points that capture HIP graphs and replay them (ne_exl3_lin_time, ne_exl3_lin_time_multi,
ne_moe_time) and for the allocation-free linear under a capture:
  - no allocation, free, memset, copy, stream wait or kernel-attribute change happens while a stream is capturing;
  - every buffer a captured launch references is still allocated at every replay and when its graph is destroyed;
  - every replay has been waited for before its graph exec is destroyed;
  - nothing is left capturing and no graph is left alive afterwards.
The instrumentation itself is checked by making it see each kind of violation (a capture around an allocation, a
buffer freed under a live graph exec)."""
import ctypes as C

import numpy as np
import pytest

from ijah_amd import synth


@pytest.fixture(scope="module")
def host():
    import importlib.util
    from pathlib import Path

    from ijah_amd.engine import Engine
    spec = importlib.util.spec_from_file_location("hoststub_build", Path(__file__).parent / "hoststub" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    build = mod.build
    eng = Engine(build())
    L = eng.lib
    L.hipstub_violations.restype, L.hipstub_violations.argtypes = C.c_int, [C.c_char_p, C.c_int]
    for f in ("hipstub_graph_launches", "hipstub_live_graphs", "hipstub_capturing", "hipstub_begin_capture",
              "hipstub_end_capture"):
        getattr(L, f).restype = C.c_int
    return eng


def violations(eng):
    buf = C.create_string_buffer(1 << 16)
    n = eng.lib.hipstub_violations(buf, len(buf))
    return n, buf.value.decode()


def clean(eng):
    n, msg = violations(eng)
    assert n == 0, msg
    assert eng.lib.hipstub_capturing() == 0
    assert eng.lib.hipstub_live_graphs() == 0


def linears(eng, shapes, seed=1):
    rng = np.random.default_rng(seed)
    return [eng.exl3_linear(*synth.linear(rng, i, o, k)) for i, o, k in shapes]


CONFIG3 = [(2048, 4096, 6), (2048, 512, 6), (2048, 512, 6), (4096, 2048, 6)]


def test_lin_time_capture_invariants(host):
    """the trunk timing sequence of bench.py (config 3 at 1 and 16 rows, then 32: the k-group partials grow between
    captures, never inside one)"""
    eng = host
    eng.lib.hipstub_reset()
    lins = linears(eng, CONFIG3 + [(2048, 151936 // 16 * 16 // 8, 8)])
    x = eng.alloc(32 * 4096 * 4)
    for R in (1, 16, 32, 4):
        for lin in lins:
            assert eng.lin_time([lin], R, x, warmup=2, reps=3) > 0
        assert eng.lin_time(lins, R, x, warmup=1, reps=2) > 0
        clean(eng)
    assert eng.lib.hipstub_graph_launches() > 0


@pytest.mark.parametrize("group", [2, 4])
def test_lin_time_multi_capture_invariants(host, group):
    eng = host
    eng.lib.hipstub_reset()
    lins = linears(eng, CONFIG3, seed=group)
    x = eng.alloc(16 * 4096 * 4)
    for R in (1, 16):
        assert eng.lin_time_multi(lins[:3], R, x, group, warmup=1, reps=2) > 0
        clean(eng)


def test_moe_time_capture_invariants(host):
    """the MoE chain timing (layers of a shape, their scratch grown for R before the capture)"""
    eng = host
    eng.lib.hipstub_reset()
    layers = [eng.moe_synth(1024, 256, 16, 4, 5, True, 5, seed=s) for s in (1, 2)]
    x = eng.alloc(16 * 1024 * 4)
    for R in (1, 4, 16):
        assert eng.moe_time(layers, R, x, warmup=1, reps=2) > 0
        clean(eng)


def test_noalloc_linear_under_capture(host):
    """the allocation-free linear is for callers that capture: inside a capture it allocates, frees and sets nothing
    (its scratch is the fixed per-GPU array, cleared by a kernel)"""
    eng = host
    eng.lib.hipstub_reset()
    lin = linears(eng, [(2048, 512, 5)])[0]
    x, y = eng.alloc(8 * 2048 * 4), eng.alloc(8 * 512 * 4)
    for R in (8, 1):
        assert eng.lib.hipstub_begin_capture() == 0
        rc = eng.lib.ne_exl3_lin_run_noalloc(lin.ptr, R, x.ptr, 0, y.ptr, 0)
        assert eng.lib.hipstub_end_capture() == 0
        assert rc == 0, eng.last_error()
        clean(eng)


def test_linear_refuses_growth_under_capture(host):
    """a run that would grow a linear's partials while the stream captures is refused (the old buffer would stay in
    the graph), and nothing was freed"""
    eng = host
    eng.lib.hipstub_reset()
    lin = linears(eng, [(2048, 4096, 6)], seed=9)[0]
    x, y = eng.alloc(32 * 2048 * 4), eng.alloc(32 * 4096 * 4)
    lin.run_bufs(1, x, y)
    assert eng.lib.hipstub_begin_capture() == 0
    rc = eng.lib.ne_exl3_lin_run(lin.ptr, 32, x.ptr, 0, y.ptr, 0, None)
    err = eng.last_error()
    assert eng.lib.hipstub_end_capture() == 0
    assert rc != 0 and "before a stream capture" in err
    clean(eng)


def test_instrumentation_sees_violations(host):
    """the stand-in reports an allocation inside a capture and a buffer freed while a live graph exec uses it"""
    eng = host
    eng.lib.hipstub_reset()
    assert eng.lib.hipstub_begin_capture() == 0
    b = eng.alloc(1024)
    assert eng.lib.hipstub_end_capture() == 0
    n, msg = violations(eng)
    assert n >= 1 and "hipMalloc while a stream is capturing" in msg
    b.free()
    eng.lib.hipstub_reset()
    # a captured linear whose input is freed before the graph exec is destroyed
    lin = linears(eng, [(256, 128, 5)])[0]
    x, y = eng.alloc(256 * 4), eng.alloc(128 * 4)
    lin.run_bufs(1, x, y)
    L = eng.lib
    assert L.hipstub_begin_capture() == 0
    assert L.ne_exl3_lin_run(lin.ptr, 1, x.ptr, 0, y.ptr, 0, None) == 0
    # end the capture through the runtime itself and keep its graph: instantiate, free x, replay
    L.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    L.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    L.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    L.hipGraphExecDestroy.argtypes = [C.c_void_p]
    L.hipGraphDestroy.argtypes = [C.c_void_p]
    L.hipstub_library_stream.restype = C.c_void_p
    g, ge = C.c_void_p(), C.c_void_p()
    stream = C.c_void_p(L.hipstub_library_stream())
    assert L.hipStreamEndCapture(stream, C.byref(g)) == 0
    assert L.hipGraphInstantiate(C.byref(ge), g, None, None, 0) == 0
    x.free()
    assert L.hipGraphLaunch(ge, stream) == 0
    n, msg = violations(eng)
    assert "a live graph exec uses it" in msg and "references freed memory" in msg, msg
    L.hipGraphExecDestroy(ge)
    L.hipGraphDestroy(g)
    eng.lib.hipstub_reset()
