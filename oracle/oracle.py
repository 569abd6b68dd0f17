"""numpy front end of the C oracle (oracle/exl3_oracle.c). TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product package (ijah_amd/).

Every function restates the reference (publicExcess/ijah) algorithm; the C source cites file:line for each.
"""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


def build(force=False):
    """Compile the oracle with its Makefile (gcc)."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-C", str(HERE), "-B" if force else "all"], check=True, capture_output=True)
    return LIB_PATH


class _Moe(C.Structure):
    _fields_ = [("hid", C.c_int), ("inter", C.c_int), ("ne", C.c_int), ("topk", C.c_int), ("K", C.c_int),
                ("router", C.c_void_p), ("sgate", C.c_void_p),
                ("gt", C.c_void_p), ("ut", C.c_void_p), ("dt", C.c_void_p), ("gsu", C.c_void_p),
                ("gsv", C.c_void_p), ("usu", C.c_void_p), ("usv", C.c_void_p), ("dsu", C.c_void_p),
                ("dsv", C.c_void_p), ("Ks", C.c_int),
                ("sgt", C.c_void_p), ("sut", C.c_void_p), ("sdt", C.c_void_p), ("sgsu", C.c_void_p),
                ("sgsv", C.c_void_p), ("susu", C.c_void_p), ("susv", C.c_void_p), ("sdsu", C.c_void_p),
                ("sdsv", C.c_void_p), ("qgroup", C.c_int)] + \
               [(n, C.c_void_p) for n in ("qgw", "quw", "qdw", "qgs", "qgb", "qus", "qub", "qds", "qdb")]


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(str(LIB_PATH))
        L.orc_f32_to_f16.restype, L.orc_f32_to_f16.argtypes = C.c_uint16, [C.c_float]
        L.orc_f16_to_f32.restype, L.orc_f16_to_f32.argtypes = C.c_float, [C.c_uint16]
        L.orc_bf16r.restype, L.orc_bf16r.argtypes = C.c_float, [C.c_float]
        L.orc_mcg.restype, L.orc_mcg.argtypes = C.c_uint16, [C.c_uint32]
        L.orc_slot_rc.restype, L.orc_slot_rc.argtypes = None, [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        for n in ("orc_tile_cw_ring", "orc_tile_cw_lane", "orc_tile_cw_t6"):
            f = getattr(L, n)
            f.restype, f.argtypes = (None if n.endswith("ring") else C.c_int), [_u16p, C.c_int, _u16p]
        L.orc_decode.restype, L.orc_decode.argtypes = None, [_u16p, C.c_int, C.c_int, C.c_int, _u16p]
        L.orc_had_size.restype, L.orc_had_size.argtypes = C.c_int, [C.c_int]
        L.orc_fwht_f32.restype, L.orc_fwht_f32.argtypes = None, [_f32p, C.c_int, C.c_int]
        L.orc_fwht_f64.restype, L.orc_fwht_f64.argtypes = None, [_f64p, C.c_int, C.c_int]
        L.orc_exl3_linear.restype = None
        L.orc_exl3_linear.argtypes = [_f32p, C.c_int, _u16p, _u16p, _u16p, C.c_int, C.c_int, C.c_int, _f32p]
        L.orc_exl3_linear_exact.restype = None
        L.orc_exl3_linear_exact.argtypes = [_f32p, C.c_int, _u16p, _u16p, _u16p, C.c_int, C.c_int, C.c_int, _f64p]
        L.orc_lin_epi.restype = C.c_int
        L.orc_lin_epi.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, C.c_void_p,
                                  C.c_void_p, C.c_void_p, C.c_long]
        L.orc_hc_prep.restype = None
        L.orc_hc_prep.argtypes = [_f32p, _u16p, _u16p, C.c_int, C.c_int, _f32p, _f32p, _f32p]
        L.orc_hc_out.restype = None
        L.orc_hc_out.argtypes = [_f32p, _f32p, _u16p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
        L.orc_hc_write.restype = None
        L.orc_hc_write.argtypes = [_f32p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, _f32p, _f32p, _f32p]
        L.orc_moe_layer_hc.restype = C.c_int
        L.orc_moe_layer_hc.argtypes = [C.POINTER(_Moe), _f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p, _f32p, _f32p]
        L.orc_router_logits.restype = None
        L.orc_router_logits.argtypes = [_f32p, _u16p, C.c_int, C.c_int, C.c_int, _f32p]
        L.orc_route.restype, L.orc_route.argtypes = None, [_f32p, C.c_int, C.c_int, _u32p, _f32p]
        L.orc_moe_layer.restype = C.c_int
        L.orc_moe_layer.argtypes = [C.POINTER(_Moe), _f32p, C.c_int, _f32p, _f32p, _u32p]
        L.orc_moe_experts.restype = C.c_int
        L.orc_moe_experts.argtypes = [C.POINTER(_Moe), _f32p, C.c_int, _u32p, C.c_void_p, _f32p]
        L.orc_moe_experts_exact.restype = C.c_int
        L.orc_moe_experts_exact.argtypes = [C.POINTER(_Moe), _f32p, C.c_int, _u32p, C.c_void_p, _f64p]
        L.orc_q8_linear.restype = None
        L.orc_q8_linear.argtypes = [_f32p, C.c_int, np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS"), _u16p,
                                    _u16p, C.c_int, C.c_int, C.c_int, _f32p]
        L.orc_q8_shared.restype = None
        L.orc_q8_shared.argtypes = [C.POINTER(_Moe), _f32p, C.c_int, _f32p]
        L.orc_moe_experts_fast.restype = C.c_int
        L.orc_moe_experts_fast.argtypes = [C.POINTER(_Moe), _f32p, C.c_int, _u32p, C.c_void_p, _f32p, C.c_int]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def mcg(cw):
    return int(lib().orc_mcg(int(cw)))


def mcg_table():
    """fp16 bits of all 2^15 window-15 codewords."""
    L = lib()
    return np.array([L.orc_mcg(c) for c in range(1 << 15)], np.uint16)


def slot_rc(s):
    r, c = C.c_int(), C.c_int()
    lib().orc_slot_rc(int(s), C.byref(r), C.byref(c))
    return r.value, c.value


def tile_cw(tile, K, reader="ring"):
    out = np.zeros(256, np.uint16)
    rc = getattr(lib(), f"orc_tile_cw_{reader}")(_c(tile, np.uint16), int(K), out)
    if rc not in (None, 0):
        raise ValueError(f"reader {reader} does not support K={K}")
    return out


def decode(trellis, K=None):
    """trellis U16 [in/16, out/16, 16K] -> W' fp16 [in, out]"""
    t = _c(trellis, np.uint16)
    it, ot, n = t.shape
    K = K or n // 16
    w = np.zeros((it * 16, ot * 16), np.uint16)
    lib().orc_decode(t, it * 16, ot * 16, K, w)
    return w.view(np.float16)


def had_size(d):
    return lib().orc_had_size(int(d))


def fwht(v, had=None, f64=False):
    v = np.array(v, np.float64 if f64 else np.float32, copy=True).reshape(-1)
    had = had or had_size(v.size)
    (lib().orc_fwht_f64 if f64 else lib().orc_fwht_f32)(v, v.size, had)
    return v


def exl3_linear(x, trellis, suh, svh, exact=False):
    """x f32 [R, in] -> y [R, out] (kernel arithmetic; exact=True: f64, no fp16 input rounding)"""
    x = _c(np.atleast_2d(x), np.float32)
    t = _c(trellis, np.uint16)
    it, ot, n = t.shape
    R, din = x.shape
    assert din == it * 16
    y = np.zeros((R, ot * 16), np.float64 if exact else np.float32)
    f = lib().orc_exl3_linear_exact if exact else lib().orc_exl3_linear
    f(x, R, t, _c(suh, np.float16).view(np.uint16), _c(svh, np.float16).view(np.uint16), it * 16, ot * 16, n // 16, y)
    return y


def lin_epi(v, kind, refr=True, hc=4, ldy=None, y=None, e0=None, e1=None, e2=None):
    """the fused epilogue of a finished linear output v f32 [R, out] (kernels/trunk6/trunk6.metal:129-197).
    Returns y [R, ldy] (columns beyond out keep y's values); e0..e2 numpy arrays are updated in place."""
    v = _c(np.atleast_2d(v), np.float32)
    R, out = v.shape
    ldy = ldy or out
    y = np.zeros((R, ldy), np.float32) if y is None else _c(y, np.float32).copy()
    assert y.shape == (R, ldy)
    ptr = lambda a: None if a is None else a.ctypes.data
    for a in (e0, e1, e2):
        assert a is None or a.flags.c_contiguous
    cap = e0.nbytes // 512 if (kind == 7 and e0 is not None) else 0
    rc = lib().orc_lin_epi(v, R, out, kind, int(bool(refr)), hc, ldy, y, ptr(e0), ptr(e1), ptr(e2), cap)
    assert rc == 0, f"epilogue {kind} not covered"
    return y


def router_logits(x, rw_bf16, round_bf16=True):
    x = _c(x, np.float32).reshape(-1)
    rw = _c(rw_bf16, np.uint16)
    out = np.zeros(rw.shape[0], np.float32)
    lib().orc_router_logits(x, rw, rw.shape[0], rw.shape[1], int(round_bf16), out)
    return out


def route(logits, topk):
    lg = _c(logits, np.float32).reshape(-1)
    ids = np.zeros(topk, np.uint32)
    w = np.zeros(topk, np.float32)
    lib().orc_route(lg, lg.size, topk, ids, w)
    return ids, w


class MoeWeights:
    """Holds numpy arrays of one synthetic / pack MoE layer and the C struct pointing into them."""

    def __init__(self, d):
        self.d = {k: (np.ascontiguousarray(v) if isinstance(v, np.ndarray) else v) for k, v in d.items()}
        g = self.d
        m = _Moe()
        m.hid, m.inter, m.ne, m.topk, m.K = g["hid"], g["inter"], g["ne"], g["topk"], g["K"]

        def p(key):
            a = g.get(key)
            return None if a is None else a.ctypes.data

        m.router, m.sgate = p("router"), p("sgate")
        m.gt, m.ut, m.dt = p("gate.trellis"), p("up.trellis"), p("down.trellis")
        m.gsu, m.gsv, m.usu, m.usv = p("gate.suh"), p("gate.svh"), p("up.suh"), p("up.svh")
        m.dsu, m.dsv = p("down.suh"), p("down.svh")
        m.Ks = g.get("Ks", g["K"])
        m.sgt, m.sut, m.sdt = p("sgate_proj.trellis"), p("sup_proj.trellis"), p("sdown_proj.trellis")
        m.sgsu, m.sgsv, m.susu, m.susv = (p("sgate_proj.suh"), p("sgate_proj.svh"), p("sup_proj.suh"),
                                          p("sup_proj.svh"))
        m.sdsu, m.sdsv = p("sdown_proj.suh"), p("sdown_proj.svh")
        if g.get("sq8_gate.weight") is not None:  # the 8-bit affine shared expert (bytes of the U32 weights)
            m.qgroup = g.get("qgroup", 128)
            m.qgw, m.quw, m.qdw = p("sq8_gate.weight"), p("sq8_up.weight"), p("sq8_down.weight")
            m.qgs, m.qgb, m.qus, m.qub = (p("sq8_gate.scales"), p("sq8_gate.biases"), p("sq8_up.scales"),
                                          p("sq8_up.biases"))
            m.qds, m.qdb = p("sq8_down.scales"), p("sq8_down.biases")
        self.m = m


def q8_linear(x, w_u32, scales, biases, group=128):
    """8-bit affine linear (kernels/ne_common.h:33-88): x f32 [R, in], weight U32 [out, in/4] (bytes), scales /
    biases bf16 bits [out, in/group] -> y f32 [R, out]"""
    x = _c(np.atleast_2d(x), np.float32)
    w = _c(w_u32, np.uint32)
    out, inp = w.shape[0], w.shape[1] * 4
    y = np.zeros((x.shape[0], out), np.float32)
    lib().orc_q8_linear(x, x.shape[0], w.view(np.uint8), _c(scales, np.uint16), _c(biases, np.uint16), inp, out,
                        group, y)
    return y


def q8_shared(W, x, refr=True):
    """the layer's 8-bit shared expert on one row x [hid] -> o [hid] (rr'd when refr)"""
    o = np.zeros(W.m.hid, np.float32)
    lib().orc_q8_shared(C.byref(W.m), _c(x, np.float32).reshape(-1), int(bool(refr)), o)
    return o


def moe_layer(W, x):
    """Full layer (router + top-k + experts): returns y [R, hid], logits [R, ne], route u32 [R, 2 topk]."""
    x = _c(np.atleast_2d(x), np.float32)
    R = x.shape[0]
    m = W.m
    y = np.zeros((R, m.hid), np.float32)
    lg = np.zeros((R, m.ne), np.float32)
    rt = np.zeros((R, 2 * m.topk), np.uint32)
    lib().orc_moe_layer(C.byref(m), x, R, y, lg, rt)
    return y, lg, rt


def hc_prep(h, nw, iw):
    """h f32 [R, 4, hid], hc_norm bf16 bits [4 hid], inject bf16 bits [4, 4 hid] -> xn [R, 4 hid], ip [R, 4, 4],
    inj [R, 8] (inv_s filled, gates 0)"""
    h = _c(h, np.float32)
    R, _, hid = h.shape
    xn, ip, inj = np.zeros((R, 4 * hid), np.float32), np.zeros((R, 4, 4), np.float32), np.zeros((R, 8), np.float32)
    lib().orc_hc_prep(h, _c(nw, np.uint16), _c(iw, np.uint16), R, hid, xn, ip, inj)
    return xn, ip, inj


def hc_out(u, h, nw, ip, inj, refr=True):
    """u [R, 4 hid] (the up linear's output) -> out [R, hid]; inj [R, 8] gets its gates (a copy is returned)"""
    h = _c(h, np.float32)
    R, _, hid = h.shape
    inj = _c(inj, np.float32).copy()
    out = np.zeros((R, hid), np.float32)
    lib().orc_hc_out(_c(u, np.float32), h, _c(nw, np.uint16), _c(ip, np.float32), R, hid, int(bool(refr)), inj, out)
    return out, inj


def hc_read(h, nw, iw, down, up, refr=True):
    """the HC read on EXL3 mixes (models/flash_next/layer_t6.mm:89-133): down / up = (trellis, suh, svh) of the
    4 hid -> lr and lr -> 4 hid linears. Returns mix [R, lr], inj [R, 8], out [R, hid]."""
    xn, ip, inj = hc_prep(h, nw, iw)
    mix = lin_epi(exl3_linear(xn, *down), 2, refr=refr)
    u = exl3_linear(mix, *up)
    out, inj = hc_out(u, h, nw, ip, inj, refr=refr)
    return mix, inj, out


def hc_write(s, t, h, inj, refr=True):
    """the MoE finisher's hyper-connection write (kernels/fn_moe.metal:437-448): s, t [R, hid] (t may be None),
    h [R, hc, hid], inj [R, 8] -> (branch y [R, hid], hout [R, hc, hid])"""
    s = _c(np.atleast_2d(s), np.float32)
    R, hid = s.shape
    h = _c(h, np.float32)
    hc = h.shape[1]
    t = None if t is None else _c(t, np.float32).reshape(R, hid)
    y, hout = np.zeros((R, hid), np.float32), np.zeros_like(h)
    lib().orc_hc_write(s, None if t is None else t.ctypes.data, R, hid, hc, int(bool(refr)), h,
                       _c(inj, np.float32), y, hout)
    return y, hout


def moe_layer_hc(W, x, h, inj, refr=True):
    """the layer with the hyper-connection write: (branch y [R, hid], hout [R, hc, hid])"""
    x = _c(np.atleast_2d(x), np.float32)
    R = x.shape[0]
    h = _c(h, np.float32)
    y, hout = np.zeros((R, W.m.hid), np.float32), np.zeros_like(h)
    lib().orc_moe_layer_hc(C.byref(W.m), x, R, h.shape[1], int(bool(refr)), h, _c(inj, np.float32), y, hout)
    return y, hout


def moe_experts(W, x, route_u32, sg=None, exact=False, fast_threads=None):
    """Expert part of the layer for a given route [R, 2 topk] (ids, f32 weight bits) and shared gate sg [R]."""
    x = _c(np.atleast_2d(x), np.float32)
    R = x.shape[0]
    m = W.m
    rt = _c(route_u32, np.uint32)
    sgp = None
    if sg is not None:
        sg = _c(sg, np.float32)
        sgp = sg.ctypes.data
    if exact:
        y = np.zeros((R, m.hid), np.float64)
        lib().orc_moe_experts_exact(C.byref(m), x, R, rt, sgp, y)
        return y
    y = np.zeros((R, m.hid), np.float32)
    if fast_threads is not None:
        used = lib().orc_moe_experts_fast(C.byref(m), x, R, rt, sgp, y, int(fast_threads))
        return y, used
    lib().orc_moe_experts(C.byref(m), x, R, rt, sgp, y)
    return y
