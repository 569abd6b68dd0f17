"""Python front end of the library's C ABI (include/engine.h + include/ijah_exl3.h, ijah_amd/_lib/libijah_exl3.so).

The public names are the reference binding's (tools/engine.py:150-613: Engine, Buf, TensorDesc, Pack and
Engine.run_kernel, with the same arguments and errors), so code written against it runs here unchanged; the EXL3
hot-path objects (Exl3Linear, MoeLayer) sit beside them. The ctypes structure layouts and the symbol table below are
the C interface itself and must match the headers byte for byte; everything else is this module's own design: every
native object is a _Handle that owns one pointer and its release function, and arguments are marshalled by type
through one dispatch table. numpy only.

    from ijah_amd.engine import Engine
    eng = Engine()
    b = eng.from_numpy(np.arange(16, dtype=np.float32)); b.download(np.float32, (16,))
    p = eng.pack_open(path); t = p.info("model.layers.0.mlp.gate.weight")
    moe = eng.moe_load(p, "model.layers.0.mlp.", topk=10); y = moe.run(x)
"""
import ctypes as C
import json
import os
import struct
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB = Path(os.environ.get("NE_LIB", PKG / "_lib" / "libijah_exl3.so"))
MAX_DIMS = 8
# ne_dtype codes (include/engine.h) and their numpy storage types (BF16 kept as raw uint16 bits)
DTYPES = {0: "F32", 1: "F16", 2: "BF16", 3: "U8", 4: "U16", 5: "U32", 6: "I32", 7: "I64", 8: "I8", 9: "I16",
          10: "U64", 11: "F64", 12: "BOOL"}
NP = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "U8": np.uint8, "U16": np.uint16, "U32": np.uint32,
      "I32": np.int32, "I64": np.int64, "I8": np.int8, "I16": np.int16, "U64": np.uint64, "F64": np.float64,
      "BOOL": np.uint8}
FC_TYPES = {"u32": 0, "i32": 1, "f32": 2, "bool": 3, "u16": 4, "i16": 5}


# ---------------------------------------------------------------------------------------------- C structures
class DeviceInfo(C.Structure):  # ne_device_info
    _fields_ = [("name", C.c_char * 64), ("has_nax", C.c_int), ("has_metal4", C.c_int),
                ("max_buffer_length", C.c_uint64), ("recommended_working_set", C.c_uint64),
                ("max_threadgroup_memory", C.c_uint64), ("backend", C.c_char * 16)]


class TensorDescC(C.Structure):  # ne_tensor_desc
    _fields_ = [("dtype", C.c_int), ("ndim", C.c_int), ("shape", C.c_int64 * MAX_DIMS), ("nbytes", C.c_uint64),
                ("file", C.c_char_p), ("file_offset", C.c_uint64), ("host", C.c_void_p), ("buf", C.c_void_p),
                ("buf_offset", C.c_uint64)]


class FConst(C.Structure):  # ne_fconst
    _fields_ = [("index", C.c_uint32), ("type", C.c_uint32), ("bits", C.c_uint32)]


class ArgC(C.Structure):  # ne_arg
    _fields_ = [("buf", C.c_void_p), ("offset", C.c_uint64), ("bytes", C.c_void_p), ("nbytes", C.c_uint32)]


_MOE_INTS = ("hid", "inter", "ne", "topk", "K", "Ks")
_MOE_EXL3 = ("router", "sgate", "gt", "ut", "dt", "gsu", "gsv", "usu", "usv", "dsu", "dsv", "sgt", "sut", "sdt",
             "sgsu", "sgsv", "susu", "susv", "sdsu", "sdsv")
_MOE_Q8 = ("qgw", "quw", "qdw", "qgs", "qgb", "qus", "qub", "qds", "qdb")


class MoeDesc(C.Structure):  # ne_moe_desc
    _fields_ = ([(n, C.c_int) for n in _MOE_INTS] + [(n, C.c_void_p) for n in _MOE_EXL3] + [("qgroup", C.c_int)] +
                [(n, C.c_void_p) for n in _MOE_Q8])


class PackAlignStats(C.Structure):  # ne_pack_align_stats
    _fields_ = [(n, C.c_uint64) for n in ("tensors", "misaligned_tensors", "misaligned_bytes", "files_rewritten",
                                          "files_linked", "files_kept", "bytes_written")]


class Exl3Epi(C.Structure):  # ne_exl3_epi: kind, rounding switch, streams, y row stride, extra buffers
    _fields_ = [("kind", C.c_int), ("refr", C.c_int), ("hc", C.c_int), ("ldy", C.c_int),
                ("e0", C.c_void_p), ("e1", C.c_void_p), ("e2", C.c_void_p)]


class MoeHc(C.Structure):  # ne_moe_hc: the hyper-connection write fused into the MoE combine
    _fields_ = [("hc", C.c_int), ("refr", C.c_int), ("h", C.c_void_p), ("inj", C.c_void_p), ("hout", C.c_void_p)]


class EngineError(RuntimeError):
    pass


# ---------------------------------------------------------------------------------------------- symbol table
_vp, _u64, _i, _i64, _s = C.c_void_p, C.c_uint64, C.c_int, C.c_int64, C.c_char_p
_dp, _ip = C.POINTER(C.c_double), C.POINTER(C.c_int)
_U3 = C.POINTER(C.c_uint32 * 3)
SIGNATURES = {
    # include/engine.h (the reference's core ABI, its tools/engine.py:278-300)
    "ne_abi_version": (_i, []), "ne_last_error": (_s, []), "ne_dtype_name": (_s, [_i]), "ne_dtype_size": (_i, [_i]),
    "ne_device_query": (_i, [C.POINTER(DeviceInfo)]),
    "ne_alloc": (_vp, [_u64]), "ne_free": (None, [_vp]), "ne_buf_size": (_u64, [_vp]),
    "ne_buf_contents": (_vp, [_vp]), "ne_buf_gpu_address": (_u64, [_vp]),
    "ne_upload": (_i, [_vp, _u64, _vp, _u64]), "ne_download": (_i, [_vp, _u64, _vp, _u64]),
    "ne_pack_open": (_vp, [_s]), "ne_pack_close": (None, [_vp]), "ne_pack_config_json": (_s, [_vp]),
    "ne_pack_num_tensors": (_i64, [_vp]), "ne_pack_tensor_name": (_s, [_vp, _i64]),
    "ne_tensor_info": (_i, [_vp, _s, C.POINTER(TensorDescC)]),
    "ne_pack_view_rows": (_vp, [_vp, _s, _i64, _i64, C.POINTER(_u64)]),
    "ne_kernel_exists": (_i, [_s]),
    "ne_run_kernel": (_i, [_s, C.POINTER(FConst), _i, C.POINTER(ArgC), _i, _U3, _U3, C.c_uint32, _i, _s, _dp]),
    # include/ijah_exl3.h
    "ne_buf_flush": (_i, [_vp]), "ne_sync": (_i, []), "ne_stream": (_vp, []),
    "ne_pack_align": (_i, [_s, _s, _u64, _i, _vp]),
    "ne_exl3_lin_load": (_vp, [_vp, _s]), "ne_exl3_lin_create": (_vp, [_vp, _vp, _vp, _i, _i, _i]),
    "ne_exl3_lin_free": (None, [_vp]), "ne_exl3_lin_info": (_i, [_vp, _ip, _ip, _ip]),
    "ne_exl3_lin_run": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _dp]),
    "ne_exl3_lin_run_noalloc": (_i, [_vp, _i, _vp, _u64, _vp, _u64]),
    "ne_exl3_lin_run_epi": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _vp, _dp]),
    "ne_hc_read": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _dp]),
    "ne_exl3_lin_time": (_i, [C.POINTER(_vp), _i, _i, _vp, _i, _i, _dp]),
    "ne_exl3_lin_time_multi": (_i, [_vp, _i, _i, _i, _vp, _i, _i, _dp]),
    "ne_exl3_lin_run_multi": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _dp]),
    "ne_exl3_lin_decode": (_i, [_vp, _vp, _dp]),
    "ne_moe_create": (_vp, [C.POINTER(MoeDesc)]), "ne_moe_load": (_vp, [_vp, _s, _i]),
    "ne_moe_synth": (_vp, [_i, _i, _i, _i, _i, _i, _i, _u64]), "ne_moe_free": (None, [_vp]),
    "ne_moe_run": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _dp]),
    "ne_moe_run_hc": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _vp, _dp]),
    "ne_moe_read": (_i, [_vp, _s, _vp, _u64]), "ne_moe_decode": (_i, [_vp, _i, _i, _vp, _dp]),
    "ne_moe_configure": (_i, [_vp, _s, _i]), "ne_exl3_lin_configure": (_i, [_vp, _s, _i]),
    "ne_moe_info": (_i, [_vp] + [_ip] * 6), "ne_moe_bytes": (_i, [_vp, _i, C.POINTER(_u64)]),
    "ne_moe_time": (_i, [C.POINTER(_vp), _i, _i, _vp, _i, _i, _dp]),
    "ne_moe_time_kernels": (_i, [C.POINTER(_vp), _i, _i, _vp, _i, _vp, _dp, _ip]),
}


def bf16_to_f32(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


def _host_array(addr, dtype, count):
    """numpy array over `count` elements of dtype at a host address (no copy)"""
    dtype = np.dtype(dtype)
    if count == 0:
        return np.empty(0, dtype)
    raw = np.ctypeslib.as_array(C.cast(C.c_void_p(addr), C.POINTER(C.c_uint8)), shape=(count * dtype.itemsize,))
    return raw.view(dtype)


def _ptrs(objs):
    """a C array of the handles' pointers"""
    return (C.c_void_p * len(objs))(*[o.ptr for o in objs])


class _Handle:
    """One native object: its pointer, the engine, and the symbol that releases it (None: not ours to release)."""
    _release = None

    def __init__(self, eng, ptr, owned=True):
        self.eng, self.ptr, self.owned = eng, ptr, owned

    def free(self):
        p, self.ptr = self.ptr, None
        if p and self.owned and self._release:
            getattr(self.eng.lib, self._release)(p)

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def _call(self, name, *args):
        """the symbol with this handle as its first argument; non-zero rc raises"""
        self.eng._ok(getattr(self.eng.lib, name)(self.ptr, *args), name)


# ---------------------------------------------------------------------------------------------- buffers, packs
class Buf(_Handle):
    """A device buffer (ne_buf). owned=False for pack-owned ones, which the pack releases."""
    _release = "ne_free"

    @property
    def size(self):
        return self.eng.lib.ne_buf_size(self.ptr)

    def contents(self):
        return self.eng.lib.ne_buf_contents(self.ptr)

    def gpu_address(self):
        return self.eng.lib.ne_buf_gpu_address(self.ptr)

    def _count(self, dtype, shape, offset):
        return (self.size - offset) // dtype.itemsize if shape is None else int(np.prod(shape))

    def upload(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        self._call("ne_upload", offset, a.ctypes.data, a.nbytes)

    def download(self, dtype=np.float32, shape=None, offset=0):
        dtype = np.dtype(dtype)
        out = np.empty(self._count(dtype, shape, offset), dtype)
        self._call("ne_download", offset, out.ctypes.data, out.nbytes)
        return out if shape is None else out.reshape(shape)

    def numpy(self, dtype=np.float32, shape=None, offset=0):
        """The buffer's host mirror (refreshed from the device now). Bytes changed through it reach the device before
        the next library call that uses the buffer; flush() pushes the whole mirror at once."""
        dtype = np.dtype(dtype)
        base = self.contents()
        if not base:
            raise EngineError(f"ne_buf_contents: {self.eng.last_error()}")
        a = _host_array(base + offset, dtype, self._count(dtype, shape, offset))
        return a if shape is None else a.reshape(shape)

    def flush(self):
        self._call("ne_buf_flush")


class TensorDesc:
    """A pack tensor's descriptor: dtype name, shape, bytes, file placement, host view and device copy."""

    def __init__(self, eng, name, d):
        self.name, self.nbytes = name, d.nbytes
        self.dtype = DTYPES.get(d.dtype, str(d.dtype))
        self.shape = tuple(d.shape[:d.ndim])
        self.file = d.file.decode() if d.file else None
        self.file_offset, self.buf_offset, self._host = d.file_offset, d.buf_offset, d.host
        self.buf = Buf(eng, d.buf, owned=False) if d.buf else None

    @property
    def host(self):
        """read-only numpy view of the mapped bytes (BF16 as its uint16 bits)"""
        dt = np.dtype(NP[self.dtype])
        a = _host_array(self._host, dt, self.nbytes // dt.itemsize).reshape(self.shape)
        a.flags.writeable = False
        return a

    def f32(self):
        return bf16_to_f32(self.host) if self.dtype == "BF16" else self.host.astype(np.float32)

    def arg(self):
        return (self.buf, self.buf_offset)

    def __repr__(self):
        return f"TensorDesc({self.name}, {self.dtype}, {self.shape})"


class Pack(_Handle):
    """A pack directory (safetensors shards + config.json), opened read-only."""
    _release = "ne_pack_close"

    def __init__(self, eng, path):
        self.path = str(Path(path).expanduser())
        super().__init__(eng, eng.lib.ne_pack_open(self.path.encode()))
        if not self.ptr:
            raise EngineError(f"ne_pack_open({self.path}): {eng.last_error()}")

    def config(self):
        return json.loads(self.eng.lib.ne_pack_config_json(self.ptr).decode())

    def names(self):
        L = self.eng.lib
        return [L.ne_pack_tensor_name(self.ptr, i).decode() for i in range(L.ne_pack_num_tensors(self.ptr))]

    def info(self, name):
        d = TensorDescC()
        self._call("ne_tensor_info", name.encode(), C.byref(d))
        return TensorDesc(self.eng, name, d)

    def view_rows(self, name, row0, nrows):
        off = C.c_uint64(0)
        p = self.eng.lib.ne_pack_view_rows(self.ptr, name.encode(), row0, nrows, C.byref(off))
        if not p:
            raise EngineError(f"ne_pack_view_rows({name}): {self.eng.last_error()}")
        return Buf(self.eng, p), off.value


# ---------------------------------------------------------------------------------------------- EXL3 objects
def _ms_arg(timed, box):
    return C.byref(box) if timed else None


class Exl3Linear(_Handle):
    """y[R, out] = x[R, in] @ W for one EXL3 linear resident in HBM (ne_exl3_lin_*)."""
    _release = "ne_exl3_lin_free"

    def __init__(self, eng, ptr, keep=()):
        super().__init__(eng, ptr)
        self._keep = keep
        dims = [C.c_int() for _ in range(3)]
        self._call("ne_exl3_lin_info", *map(C.byref, dims))
        self.inp, self.out, self.K = (d.value for d in dims)

    def run_bufs(self, R, x, y, x_off=0, y_off=0, timed=False):
        ms = C.c_double(0)
        self._call("ne_exl3_lin_run", R, x.ptr, x_off, y.ptr, y_off, _ms_arg(timed, ms))
        return ms.value

    def run_epi(self, R, x, y, kind, x_off=0, y_off=0, refr=True, hc=4, ldy=0, e0=None, e1=None, e2=None,
                timed=False):
        """ne_exl3_lin_run_epi; e0..e2 are device buffers (or None)"""
        d = Exl3Epi(kind, int(bool(refr)), hc, ldy, *(b.ptr if b is not None else None for b in (e0, e1, e2)))
        ms = C.c_double(0)
        self._call("ne_exl3_lin_run_epi", R, x.ptr, x_off, y.ptr, y_off, C.byref(d), _ms_arg(timed, ms))
        return ms.value

    def run(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        xb, yb = self.eng.from_numpy(x), self.eng.alloc(x.shape[0] * self.out * 4)
        self.run_bufs(x.shape[0], xb, yb)
        return yb.download(np.float32, (x.shape[0], self.out))

    def configure(self, key, value):
        """ne_exl3_lin_configure ("staged": 1 = three launches)"""
        self._call("ne_exl3_lin_configure", key.encode(), int(value))
        return self

    def decode(self):
        w = self.eng.alloc(self.inp * self.out * 2)
        self._call("ne_exl3_lin_decode", w.ptr, None)
        return w.download(np.uint16, (self.inp, self.out)).view(np.float16)


def hc_read(down, up, R, h, hc_norm, inject, mix, inj, out, refr=True, timed=False):
    """ne_hc_read: the hyper-connection read through two Exl3Linear mixes (device buffers throughout)"""
    ms = C.c_double(0)
    down._call("ne_hc_read", up.ptr, R, *(b.ptr for b in (h, hc_norm, inject, mix, inj, out)), int(bool(refr)),
               _ms_arg(timed, ms))
    return ms.value


class MoeLayer(_Handle):
    """The MoE layer (router, top-k, routed EXL3 experts, shared expert, combine) resident in HBM (ne_moe_*)."""
    _release = "ne_moe_free"
    _READS = {"logits": ("ne", np.float32), "route": ("route", np.uint32), "shared_gate": ("row", np.float32),
              "experts_gu": ("gu", np.float32), "experts_dn": ("dn", np.float32), "mlp_out": ("hid", np.float32),
              "shared_q8": ("hid", np.float32)}

    def __init__(self, eng, ptr, keep=()):
        super().__init__(eng, ptr)
        self._keep = keep
        dims = [C.c_int() for _ in range(6)]
        self._call("ne_moe_info", *map(C.byref, dims))
        self.hid, self.inter, self.ne, self.topk, self.K, self.slots = (d.value for d in dims)

    def run_bufs(self, R, x, y, x_off=0, y_off=0, timed=False):
        ms = C.c_double(0)
        self._call("ne_moe_run", R, x.ptr, x_off, y.ptr, y_off, _ms_arg(timed, ms))
        return ms.value

    def run_hc(self, R, x, y, h, inj, hout, hc=4, refr=True, x_off=0, y_off=0, timed=False):
        """ne_moe_run_hc: y = the branch, hout = h + branch * inj per stream (device buffers)"""
        d = MoeHc(hc, int(bool(refr)), h.ptr, inj.ptr, hout.ptr)
        ms = C.c_double(0)
        self._call("ne_moe_run_hc", R, x.ptr, x_off, y.ptr, y_off, C.byref(d), _ms_arg(timed, ms))
        return ms.value

    def run(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        self._R = x.shape[0]
        self._io = (self.eng.from_numpy(x), self.eng.alloc(self._R * self.hid * 4))  # "mlp_out" reads the output
        self.run_bufs(self._R, *self._io)
        return self._io[1].download(np.float32, (self._R, self.hid))

    def read(self, name, R=None):
        R = R or getattr(self, "_R", 1)
        kind, dt = self._READS[name]
        shape = {"ne": (R, self.ne), "route": (R, 2 * self.topk), "row": (R,), "hid": (R, self.hid),
                 "gu": (R, self.slots, 2, self.inter), "dn": (R, self.slots, self.hid)}[kind]
        out = np.zeros(shape, dt)
        self._call("ne_moe_read", name.encode(), out.ctypes.data, out.nbytes)
        return out

    def configure(self, key, value):
        """ne_moe_configure ("staged": 1 = the four staged launches at every row count; "trace": 1 = per-wave stamps
        of the fused step)"""
        self._call("ne_moe_configure", key.encode(), int(value))
        return self

    def decode(self, e, proj):
        inp, out = (self.inter, self.hid) if proj == 2 else (self.hid, self.inter)
        w = self.eng.alloc(inp * out * 2)
        self._call("ne_moe_decode", e, proj, w.ptr, None)
        return w.download(np.uint16, (inp, out)).view(np.float16)

    def bytes(self, R=1):
        b = C.c_uint64(0)
        self._call("ne_moe_bytes", R, C.byref(b))
        return b.value


# ---------------------------------------------------------------------------------------------- kernel arguments
def _arg_buf(a):
    return ArgC(a.ptr, 0, None, 0), None


def _arg_buf_at(a):
    return ArgC(a[0].ptr, int(a[1]), None, 0), None


def _arg_inline(a):
    raw = bytes(a) if isinstance(a, (bytes, bytearray)) else np.ascontiguousarray(a).tobytes()
    cb = C.create_string_buffer(raw, len(raw))
    return ArgC(None, 0, C.cast(cb, C.c_void_p), len(raw)), cb


def _marshal(a):
    """one kernel argument -> (ne_arg, an object to keep alive until the call returns)"""
    if isinstance(a, TensorDesc):
        a = a.arg()
    if isinstance(a, Buf):
        return _arg_buf(a)
    if isinstance(a, tuple) and a and isinstance(a[0], Buf):
        return _arg_buf_at(a)
    return _arg_inline(a)


def _fconst(idx, ty, val):
    bits = struct.unpack("<I", struct.pack("<f", float(val)))[0] if ty == "f32" else int(val) & 0xFFFFFFFF
    return FConst(idx, FC_TYPES[ty], bits)


# ---------------------------------------------------------------------------------------------- the engine
class Engine:
    """The loaded library: every declared symbol bound (absent ones listed in .missing), plus object factories."""

    def __init__(self, lib=None):
        path = Path(lib or LIB)
        if not path.exists():
            raise EngineError(f"{path} not built (python -m ijah_amd.build)")
        self.lib = C.CDLL(str(path))
        self.missing = [n for n, sig in SIGNATURES.items() if not self._bind(n, *sig)]

    def _bind(self, name, restype, argtypes):
        f = getattr(self.lib, name, None)
        if f is None:
            return False
        f.restype, f.argtypes = restype, argtypes
        return True

    def has(self, name):
        return getattr(self.lib, name, None) is not None

    def fn(self, name, restype, argtypes):
        """any other exported symbol, bound with the given types"""
        if not self._bind(name, restype, argtypes):
            raise AttributeError(name)
        return getattr(self.lib, name)

    def last_error(self):
        e = self.lib.ne_last_error()
        return e.decode() if e else ""

    def _ok(self, rc, what):
        if rc != 0:
            raise EngineError(f"{what}: {self.last_error()}")

    def _made(self, p, what):
        if not p:
            raise EngineError(f"{what}: {self.last_error()}")
        return p

    def abi_version(self):
        return self.lib.ne_abi_version()

    def device(self):
        d = DeviceInfo()
        self._ok(self.lib.ne_device_query(C.byref(d)), "ne_device_query")
        info = {k: getattr(d, k) for k, _ in DeviceInfo._fields_}
        for k in ("name", "backend"):
            info[k] = info[k].decode()
        for k in ("has_nax", "has_metal4"):
            info[k] = bool(info[k])
        return info

    def sync(self):
        self._ok(self.lib.ne_sync(), "ne_sync")

    # ---- buffers and packs
    def alloc(self, nbytes):
        return Buf(self, self._made(self.lib.ne_alloc(int(nbytes)), f"ne_alloc({nbytes})"))

    def from_numpy(self, arr):
        a = np.ascontiguousarray(arr)
        b = self.alloc(max(a.nbytes, 1))
        b.upload(a)
        return b

    def pack_open(self, path):
        return Pack(self, path)

    def pack_align(self, src, dst, align=64, dry_run=False):
        """a copy of the pack in src under dst whose every tensor's data is align-byte aligned in its shard
        (reference core/pack_align.h align_pack); returns the counts"""
        st = PackAlignStats()
        self._ok(self.lib.ne_pack_align(str(src).encode(), str(dst).encode(), align, int(dry_run), C.byref(st)),
                 "ne_pack_align")
        return {n: getattr(st, n) for n, _ in PackAlignStats._fields_}

    # ---- kernels by name
    def kernel_exists(self, fn):
        return self.lib.ne_kernel_exists(fn.encode()) == 1

    def run_kernel(self, fn, args, grid, tg, fconsts=(), tg_mem=0, reps=1, backend=None):
        """Runs a library kernel by name and waits (the reference's ne_run_kernel): args are Buf, (Buf, offset),
        TensorDesc, bytes or numpy values (passed inline); fconsts (index, type, value). Returns GPU ms."""
        packed = [_marshal(a) for a in args]
        ca = (ArgC * max(len(packed), 1))(*[p for p, _ in packed])
        fc = (FConst * max(len(fconsts), 1))(*[_fconst(*f) for f in fconsts])
        ms = C.c_double(0)
        rc = self.lib.ne_run_kernel(fn.encode(), fc, len(fconsts), ca, len(packed), C.byref((C.c_uint32 * 3)(*grid)),
                                    C.byref((C.c_uint32 * 3)(*tg)), tg_mem, reps,
                                    backend.encode() if backend else None, C.byref(ms))
        self._ok(rc, f"ne_run_kernel({fn})")
        return ms.value

    # ---- EXL3 linears
    def exl3_linear(self, trellis, suh, svh):
        t = np.ascontiguousarray(trellis, np.uint16)
        su, sv = (np.ascontiguousarray(v, np.float16).view(np.uint16) for v in (suh, svh))
        it, ot, n = t.shape
        p = self.lib.ne_exl3_lin_create(t.ctypes.data, su.ctypes.data, sv.ctypes.data, it * 16, ot * 16, n // 16)
        return Exl3Linear(self, self._made(p, "ne_exl3_lin_create"))

    def exl3_linear_load(self, pack, prefix):
        p = self.lib.ne_exl3_lin_load(pack.ptr, prefix.encode())
        return Exl3Linear(self, self._made(p, f"ne_exl3_lin_load({prefix})"), keep=(pack,))

    def lin_time(self, lins, R, x, warmup=3, reps=20):
        """GPU microseconds per linear over a graph of the given linears at R rows (ne_exl3_lin_time)"""
        us = C.c_double(0)
        self._ok(self.lib.ne_exl3_lin_time(_ptrs(lins), len(lins), R, x.ptr, warmup, reps, C.byref(us)),
                 "ne_exl3_lin_time")
        return us.value

    def lin_time_multi(self, lins, R, x, group, warmup=3, reps=20):
        """GPU microseconds per replay of the linears recorded together, `group` per launch"""
        us = C.c_double(0)
        self._ok(self.lib.ne_exl3_lin_time_multi(_ptrs(lins), len(lins), group, R, x.ptr, warmup, reps, C.byref(us)),
                 "ne_exl3_lin_time_multi")
        return us.value

    def lin_run_multi(self, lins, xs):
        """ne_exl3_lin_run_multi: linear i on rows xs[i] (f32 [R][in_i], one R for all); returns the outputs"""
        R, n = np.atleast_2d(xs[0]).shape[0], len(lins)
        xb = [self.from_numpy(np.ascontiguousarray(np.atleast_2d(x), np.float32)) for x in xs]
        yb = [self.alloc(R * m.out * 4) for m in lins]
        self._ok(self.lib.ne_exl3_lin_run_multi(_ptrs(lins), n, R, _ptrs(xb), (C.c_uint64 * n)(), _ptrs(yb),
                                                (C.c_uint64 * n)(), None), "ne_exl3_lin_run_multi")
        return [b.download(np.float32, (R, m.out)) for b, m in zip(yb, lins)]

    # ---- MoE layers
    # host-array keys of a layer dict (ijah_amd.synth.moe_layer) -> (descriptor field, storage dtype)
    _MOE_ARRAYS = {"router": ("router", np.uint16), "sgate": ("sgate", np.uint16)}
    for _k, _f in (("gate", "g"), ("up", "u"), ("down", "d")):
        _MOE_ARRAYS[f"{_k}.trellis"] = (f"{_f}t", np.uint16)
        _MOE_ARRAYS[f"{_k}.suh"] = (f"{_f}su", np.float16)
        _MOE_ARRAYS[f"{_k}.svh"] = (f"{_f}sv", np.float16)
        _MOE_ARRAYS[f"s{_k}_proj.trellis"] = (f"s{_f}t", np.uint16)
        _MOE_ARRAYS[f"s{_k}_proj.suh"] = (f"s{_f}su", np.float16)
        _MOE_ARRAYS[f"s{_k}_proj.svh"] = (f"s{_f}sv", np.float16)
        _MOE_ARRAYS[f"sq8_{_k}.weight"] = (f"q{_f}w", np.uint32)
        _MOE_ARRAYS[f"sq8_{_k}.scales"] = (f"q{_f}s", np.uint16)
        _MOE_ARRAYS[f"sq8_{_k}.biases"] = (f"q{_f}b", np.uint16)
    del _k, _f

    def moe_create(self, w):
        """w: dict of numpy arrays in the pack layout (ijah_amd.synth.moe_layer)."""
        d, keep = MoeDesc(), []
        for n in _MOE_INTS:
            setattr(d, n, int(w.get(n) or 0))
        d.qgroup = int(w.get("qgroup", 128)) if w.get("sq8_gate.weight") is not None else 0
        for key, (field, dt) in self._MOE_ARRAYS.items():
            a = w.get(key)
            if a is None:
                continue
            a = np.ascontiguousarray(a, dt)
            keep.append(a)
            setattr(d, field, a.ctypes.data)
        return MoeLayer(self, self._made(self.lib.ne_moe_create(C.byref(d)), "ne_moe_create"))

    def moe_load(self, pack, prefix, topk):
        p = self.lib.ne_moe_load(pack.ptr, prefix.encode(), topk)
        return MoeLayer(self, self._made(p, f"ne_moe_load({prefix})"), keep=(pack,))

    def moe_synth(self, hid, inter, ne, topk, K, has_shared=True, Ks=None, seed=0):
        """has_shared: False / True (an EXL3 shared expert of Ks bits) / "q8" (the 8-bit affine one)"""
        sh = 2 if has_shared == "q8" else int(bool(has_shared))
        p = self.lib.ne_moe_synth(hid, inter, ne, topk, K, sh, Ks or K, seed)
        return MoeLayer(self, self._made(p, "ne_moe_synth"))

    def moe_time(self, layers, R, x, warmup=3, reps=20):
        us = C.c_double(0)
        self._ok(self.lib.ne_moe_time(_ptrs(layers), len(layers), R, x.ptr, warmup, reps, C.byref(us)), "ne_moe_time")
        return us.value

    def moe_time_kernels(self, layers, R, x, reps=5):
        names, us, n = (C.c_char * 16 * 8)(), (C.c_double * 8)(), C.c_int(8)
        self._ok(self.lib.ne_moe_time_kernels(_ptrs(layers), len(layers), R, x.ptr, reps, names, us, C.byref(n)),
                 "ne_moe_time_kernels")
        return {names[i].value.decode(): us[i] for i in range(n.value)}
