"""Buffer semantics of the C ABI on a discrete GPU (reference include/engine.h:6-7 and tools/engine.py:97-103: the
reference's buffers are unified memory, so a caller writes inputs through Buf.numpy() and runs).

Here the bytes live in HBM and ne_buf_contents() hands out a host mirror refreshed at that call. Before any library
call uses the buffer (a kernel run, a hot-path run, an upload or download), the bytes the caller changed in the mirror
since its last refresh go to the device - and only those, so a mirror the caller did not touch never overwrites
newer device data."""
import numpy as np
import pytest

from ijah_amd import synth

pytestmark = pytest.mark.gpu


def test_mirror_writes_reach_the_device_before_use(eng):
    print("buffers: mirror write-through", flush=True)
    n = 4096
    b = eng.alloc(n * 4)
    b.upload(np.zeros(n, np.float32))
    a = b.numpy()
    a[10:20] = 7.0
    got = b.download(np.float32)  # a library call on b: the pending mirror writes go first
    assert np.all(got[10:20] == 7.0) and not got[:10].any() and not got[20:].any()
    # the device changes behind the mirror; the untouched mirror must not overwrite it
    ref = np.arange(n, dtype=np.float32)
    b.upload(ref)
    assert np.array_equal(b.download(np.float32), ref)
    # a write through the now-stale mirror reaches the device for the changed element only
    a[5] = -1.0
    want = ref.copy()
    want[5] = -1.0
    assert np.array_equal(b.download(np.float32), want)
    # a fresh mirror sees the device
    assert np.array_equal(b.numpy(), want)


def test_reference_pattern_numpy_write_then_run_kernel(eng, oracle):
    """Buf.numpy() writes, then ne_run_kernel on the buffer (the reference's tools/engine.py usage), then the output
    read back through numpy(): the trellis tiles written through the mirror are decoded by a kernel run by name."""
    print("buffers: numpy write then run_kernel", flush=True)
    from ijah_amd import synth
    K, inp, out = 5, 64, 96
    t, _, _ = synth.linear(np.random.default_rng(12), inp, out, K)
    IT, OT = inp // 16, out // 16
    rel_t = np.zeros((OT // 2, IT, 2, 16 * K), np.uint16)  # the library's tile order: [out/32 pairs][in/16][2]
    for tk in range(IT):
        for tn in range(OT):
            rel_t[tn // 2, tk, tn % 2] = t[tk, tn]
    tiles, w = eng.alloc(rel_t.nbytes), eng.alloc(inp * out * 2)
    tiles.numpy(np.uint16)[:] = rel_t.reshape(-1)
    w0 = w.numpy(np.uint16)  # a mirror of w taken before the kernel writes it
    assert not w0.any()
    run = lambda: eng.run_kernel("exl3_decode", [tiles, np.int32(IT), np.int32(OT), w], grid=((IT * OT + 3) // 4, 1, 1),
                                 tg=(256, 1, 1), fconsts=[(10, "u32", K)])
    run()
    want = oracle.decode(t).view(np.uint16).reshape(-1)
    assert np.array_equal(w.numpy(np.uint16), want)
    # the stale mirror w0 was not touched: using w again does not put its old zeros back
    run()
    assert np.array_equal(w.download(np.uint16), want)


def test_reference_pattern_numpy_write_then_linear(eng, oracle):
    """The input row written through numpy() and the output read through numpy() around ne_exl3_lin_run."""
    print("buffers: numpy write then linear", flush=True)
    rng = np.random.default_rng(3)
    t, su, sv = synth.linear(rng, 256, 128, 5)
    lin = eng.exl3_linear(t, su, sv)
    x = synth.bf16_values(rng, 2, 256)
    xb, yb = eng.alloc(x.nbytes), eng.alloc(2 * 128 * 4)
    xb.numpy()[:] = x.reshape(-1)
    yb.numpy()  # a mirror of y before the run
    lin.run_bufs(2, xb, yb)
    assert np.array_equal(yb.numpy().reshape(2, 128), lin.run(x))
