"""ctypes binding of include/engine.h + include/ijah_exl3.h (ijah_amd/_lib/libijah_exl3.so).

Mirrors the reference's host binding (tools/engine.py:150-613: Engine, Buf, TensorDesc, Pack, run_kernel) so code
written against it runs here; adds the EXL3 hot-path objects (Exl3Linear, MoeLayer). numpy only.

    from ijah_amd.engine import Engine
    eng = Engine()
    b = eng.from_numpy(np.arange(16, dtype=np.float32)); b.download(np.float32, (16,))
    p = eng.pack_open(path); t = p.info("model.layers.0.mlp.gate.weight")
    moe = eng.moe_load(p, "model.layers.0.mlp.", topk=10); y = moe.run(x)
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB = Path(os.environ.get("NE_LIB", PKG / "_lib" / "libijah_exl3.so"))
MAX_DIMS = 8
DTYPES = {0: "F32", 1: "F16", 2: "BF16", 3: "U8", 4: "U16", 5: "U32", 6: "I32", 7: "I64", 8: "I8", 9: "I16",
          10: "U64", 11: "F64", 12: "BOOL"}
NP = {"F32": np.float32, "F16": np.float16, "BF16": np.uint16, "U8": np.uint8, "U16": np.uint16, "U32": np.uint32,
      "I32": np.int32, "I64": np.int64, "I8": np.int8, "I16": np.int16, "U64": np.uint64, "F64": np.float64,
      "BOOL": np.uint8}
FC_TYPES = {"u32": 0, "i32": 1, "f32": 2, "bool": 3, "u16": 4, "i16": 5}


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("has_nax", C.c_int), ("has_metal4", C.c_int),
                ("max_buffer_length", C.c_uint64), ("recommended_working_set", C.c_uint64),
                ("max_threadgroup_memory", C.c_uint64), ("backend", C.c_char * 16)]


class TensorDescC(C.Structure):
    _fields_ = [("dtype", C.c_int), ("ndim", C.c_int), ("shape", C.c_int64 * MAX_DIMS), ("nbytes", C.c_uint64),
                ("file", C.c_char_p), ("file_offset", C.c_uint64), ("host", C.c_void_p), ("buf", C.c_void_p),
                ("buf_offset", C.c_uint64)]


class FConst(C.Structure):
    _fields_ = [("index", C.c_uint32), ("type", C.c_uint32), ("bits", C.c_uint32)]


class ArgC(C.Structure):
    _fields_ = [("buf", C.c_void_p), ("offset", C.c_uint64), ("bytes", C.c_void_p), ("nbytes", C.c_uint32)]


class MoeDesc(C.Structure):
    """ne_moe_desc (include/ijah_exl3.h)"""
    _fields_ = [(n, C.c_int) for n in ("hid", "inter", "ne", "topk", "K", "Ks")] + \
               [(n, C.c_void_p) for n in ("router", "sgate", "gt", "ut", "dt", "gsu", "gsv", "usu", "usv", "dsu",
                                          "dsv", "sgt", "sut", "sdt", "sgsu", "sgsv", "susu", "susv", "sdsu",
                                          "sdsv")]


class EngineError(RuntimeError):
    pass


_vp, _u64, _i, _i64 = C.c_void_p, C.c_uint64, C.c_int, C.c_int64
_dp = C.POINTER(C.c_double)
SIGNATURES = {
    # include/engine.h (reference include/engine.h; tools/engine.py:278-300)
    "ne_abi_version": (_i, []), "ne_last_error": (C.c_char_p, []),
    "ne_dtype_name": (C.c_char_p, [_i]), "ne_dtype_size": (_i, [_i]),
    "ne_device_query": (_i, [C.POINTER(DeviceInfo)]),
    "ne_alloc": (_vp, [_u64]), "ne_free": (None, [_vp]),
    "ne_buf_size": (_u64, [_vp]), "ne_buf_contents": (_vp, [_vp]), "ne_buf_gpu_address": (_u64, [_vp]),
    "ne_upload": (_i, [_vp, _u64, _vp, _u64]), "ne_download": (_i, [_vp, _u64, _vp, _u64]),
    "ne_pack_open": (_vp, [C.c_char_p]), "ne_pack_close": (None, [_vp]),
    "ne_pack_config_json": (C.c_char_p, [_vp]), "ne_pack_num_tensors": (_i64, [_vp]),
    "ne_pack_tensor_name": (C.c_char_p, [_vp, _i64]),
    "ne_tensor_info": (_i, [_vp, C.c_char_p, C.POINTER(TensorDescC)]),
    "ne_pack_view_rows": (_vp, [_vp, C.c_char_p, _i64, _i64, C.POINTER(_u64)]),
    "ne_kernel_exists": (_i, [C.c_char_p]),
    "ne_run_kernel": (_i, [C.c_char_p, C.POINTER(FConst), _i, C.POINTER(ArgC), _i, C.POINTER(C.c_uint32 * 3),
                           C.POINTER(C.c_uint32 * 3), C.c_uint32, _i, C.c_char_p, _dp]),
    # include/ijah_exl3.h
    "ne_buf_flush": (_i, [_vp]), "ne_sync": (_i, []),
    "ne_exl3_lin_load": (_vp, [_vp, C.c_char_p]),
    "ne_exl3_lin_create": (_vp, [_vp, _vp, _vp, _i, _i, _i]),
    "ne_exl3_lin_free": (None, [_vp]),
    "ne_exl3_lin_info": (_i, [_vp, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i)]),
    "ne_exl3_lin_run": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _dp]),
    "ne_exl3_lin_run_noalloc": (_i, [_vp, _i, _vp, _u64, _vp, _u64]),
    "ne_exl3_lin_run_multi": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _dp]),
    "ne_exl3_lin_time_multi": (_i, [_vp, _i, _i, _i, _vp, _i, _i, _dp]),
    "ne_exl3_lin_run_epi": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _vp, _dp]),
    "ne_hc_read": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _dp]),
    "ne_exl3_lin_decode": (_i, [_vp, _vp, _dp]),
    "ne_moe_create": (_vp, [C.POINTER(MoeDesc)]),
    "ne_moe_load": (_vp, [_vp, C.c_char_p, _i]),
    "ne_moe_synth": (_vp, [_i, _i, _i, _i, _i, _i, _i, _u64]),
    "ne_moe_free": (None, [_vp]),
    "ne_moe_run": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _dp]),
    "ne_moe_run_hc": (_i, [_vp, _i, _vp, _u64, _vp, _u64, _vp, _dp]),
    "ne_moe_read": (_i, [_vp, C.c_char_p, _vp, _u64]),
    "ne_moe_decode": (_i, [_vp, _i, _i, _vp, _dp]),
    "ne_moe_info": (_i, [_vp] + [C.POINTER(_i)] * 6),
    "ne_moe_bytes": (_i, [_vp, _i, C.POINTER(_u64)]),
    "ne_moe_time": (_i, [C.POINTER(_vp), _i, _i, _vp, _i, _i, _dp]),
    "ne_exl3_lin_time": (_i, [C.POINTER(_vp), _i, _i, _vp, _i, _i, _dp]),
    "ne_moe_time_kernels": (_i, [C.POINTER(_vp), _i, _i, _vp, _i, C.c_void_p, _dp, C.POINTER(_i)]),
    "ne_pack_align": (_i, [C.c_char_p, C.c_char_p, _u64, _i, C.c_void_p]),
}


class PackAlignStats(C.Structure):
    """include/ijah_exl3.h ne_pack_align_stats"""
    _fields_ = [(n, C.c_uint64) for n in ("tensors", "misaligned_tensors", "misaligned_bytes", "files_rewritten",
                                          "files_linked", "files_kept", "bytes_written")]


class Exl3Epi(C.Structure):
    """include/ijah_exl3.h ne_exl3_epi: a linear's fused epilogue (kind 0/1/2/3/5/6/7, bf16 rounding switch, streams,
    y row stride in floats, extra buffers)"""
    _fields_ = [("kind", C.c_int), ("refr", C.c_int), ("hc", C.c_int), ("ldy", C.c_int),
                ("e0", C.c_void_p), ("e1", C.c_void_p), ("e2", C.c_void_p)]


class MoeHc(C.Structure):
    """include/ijah_exl3.h ne_moe_hc: the hyper-connection write fused into the MoE combine"""
    _fields_ = [("hc", C.c_int), ("refr", C.c_int), ("h", C.c_void_p), ("inj", C.c_void_p), ("hout", C.c_void_p)]


def bf16_to_f32(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


class Buf:
    """An ne_buf handle (HBM). owned=False for pack-owned copies (never freed)."""

    def __init__(self, eng, ptr, owned=True):
        self.eng, self.ptr, self.owned = eng, ptr, owned

    @property
    def size(self):
        return self.eng.lib.ne_buf_size(self.ptr)

    def contents(self):
        return self.eng.lib.ne_buf_contents(self.ptr)

    def gpu_address(self):
        return self.eng.lib.ne_buf_gpu_address(self.ptr)

    def upload(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        self.eng._ok(self.eng.lib.ne_upload(self.ptr, offset, a.ctypes.data, a.nbytes), "ne_upload")

    def download(self, dtype=np.float32, shape=None, offset=0):
        dtype = np.dtype(dtype)
        n = (self.size - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        out = np.empty(n, dtype)
        self.eng._ok(self.eng.lib.ne_download(self.ptr, offset, out.ctypes.data, out.nbytes), "ne_download")
        return out.reshape(shape) if shape is not None else out

    def numpy(self, dtype=np.float32, shape=None, offset=0):
        """Host mirror refreshed from the device now (a copy on a discrete GPU). Bytes changed through it reach the
        device before the next library call that uses this buffer; flush() pushes the whole mirror."""
        dtype = np.dtype(dtype)
        n = (self.size - offset) // dtype.itemsize if shape is None else int(np.prod(shape))
        addr = self.contents()
        if not addr:
            raise EngineError(f"ne_buf_contents: {self.eng.last_error()}")
        raw = (C.c_char * (n * dtype.itemsize)).from_address(addr + offset)
        a = np.frombuffer(raw, dtype, n)
        return a.reshape(shape) if shape is not None else a

    def flush(self):
        self.eng._ok(self.eng.lib.ne_buf_flush(self.ptr), "ne_buf_flush")

    def free(self):
        if self.ptr and self.owned:
            self.eng.lib.ne_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class TensorDesc:
    def __init__(self, eng, name, d):
        self.name = name
        self.dtype = DTYPES.get(d.dtype, str(d.dtype))
        self.shape = tuple(d.shape[i] for i in range(d.ndim))
        self.nbytes = d.nbytes
        self.file = d.file.decode() if d.file else None
        self.file_offset = d.file_offset
        self._host = d.host
        self.buf = Buf(eng, d.buf, owned=False) if d.buf else None
        self.buf_offset = d.buf_offset

    @property
    def host(self):
        dt = np.dtype(NP[self.dtype])
        raw = (C.c_char * self.nbytes).from_address(self._host)
        a = np.frombuffer(raw, dt, self.nbytes // dt.itemsize).reshape(self.shape)
        a.flags.writeable = False
        return a

    def f32(self):
        h = self.host
        return bf16_to_f32(h) if self.dtype == "BF16" else h.astype(np.float32)

    def arg(self):
        return (self.buf, self.buf_offset)

    def __repr__(self):
        return f"TensorDesc({self.name}, {self.dtype}, {self.shape})"


class Pack:
    """reference tools/engine.py Pack: names, config, tensor descriptors."""

    def __init__(self, eng, path):
        self.eng = eng
        self.path = str(Path(path).expanduser())
        self.ptr = eng.lib.ne_pack_open(self.path.encode())
        if not self.ptr:
            raise EngineError(f"ne_pack_open({self.path}): {eng.last_error()}")

    def config(self):
        import json
        return json.loads(self.eng.lib.ne_pack_config_json(self.ptr).decode())

    def names(self):
        n = self.eng.lib.ne_pack_num_tensors(self.ptr)
        return [self.eng.lib.ne_pack_tensor_name(self.ptr, i).decode() for i in range(n)]

    def info(self, name):
        d = TensorDescC()
        self.eng._ok(self.eng.lib.ne_tensor_info(self.ptr, name.encode(), C.byref(d)), f"ne_tensor_info({name})")
        return TensorDesc(self.eng, name, d)

    def view_rows(self, name, row0, nrows):
        off = C.c_uint64(0)
        p = self.eng.lib.ne_pack_view_rows(self.ptr, name.encode(), row0, nrows, C.byref(off))
        if not p:
            raise EngineError(f"ne_pack_view_rows({name}): {self.eng.last_error()}")
        return Buf(self.eng, p), off.value

    def close(self):
        if self.ptr:
            self.eng.lib.ne_pack_close(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _ptr(a):
    return None if a is None else a.ctypes.data


class Exl3Linear:
    """y[R, out] = x[R, in] @ W for one EXL3 linear resident in HBM (ne_exl3_lin_*)."""

    def __init__(self, eng, ptr, keep=()):
        self.eng, self.ptr, self._keep = eng, ptr, keep
        i, o, k = C.c_int(), C.c_int(), C.c_int()
        eng._ok(eng.lib.ne_exl3_lin_info(ptr, C.byref(i), C.byref(o), C.byref(k)), "ne_exl3_lin_info")
        self.inp, self.out, self.K = i.value, o.value, k.value

    def run_bufs(self, R, x, y, x_off=0, y_off=0, timed=False):
        ms = C.c_double(0)
        self.eng._ok(self.eng.lib.ne_exl3_lin_run(self.ptr, R, x.ptr, x_off, y.ptr, y_off,
                                                  C.byref(ms) if timed else None), "ne_exl3_lin_run")
        return ms.value

    def run_epi(self, R, x, y, kind, x_off=0, y_off=0, refr=True, hc=4, ldy=0, e0=None, e1=None, e2=None,
                timed=False):
        """ne_exl3_lin_run_epi; e0..e2 are device buffers (or None)"""
        d = Exl3Epi(kind, int(bool(refr)), hc, ldy, *(None if b is None else b.ptr for b in (e0, e1, e2)))
        ms = C.c_double(0)
        self.eng._ok(self.eng.lib.ne_exl3_lin_run_epi(self.ptr, R, x.ptr, x_off, y.ptr, y_off, C.byref(d),
                                                      C.byref(ms) if timed else None), "ne_exl3_lin_run_epi")
        return ms.value

    def run(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        R = x.shape[0]
        xb, yb = self.eng.from_numpy(x), self.eng.alloc(R * self.out * 4)
        self.run_bufs(R, xb, yb)
        return yb.download(np.float32, (R, self.out))

    def decode(self):
        w = self.eng.alloc(self.inp * self.out * 2)
        self.eng._ok(self.eng.lib.ne_exl3_lin_decode(self.ptr, w.ptr, None), "ne_exl3_lin_decode")
        return w.download(np.uint16, (self.inp, self.out)).view(np.float16)

    def free(self):
        if self.ptr:
            self.eng.lib.ne_exl3_lin_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def hc_read(down, up, R, h, hc_norm, inject, mix, inj, out, refr=True, timed=False):
    """ne_hc_read: the hyper-connection read through two Exl3Linear mixes (device buffers throughout)"""
    eng = down.eng
    ms = C.c_double(0)
    eng._ok(eng.lib.ne_hc_read(down.ptr, up.ptr, R, h.ptr, hc_norm.ptr, inject.ptr, mix.ptr, inj.ptr, out.ptr,
                               int(bool(refr)), C.byref(ms) if timed else None), "ne_hc_read")
    return ms.value


class MoeLayer:
    """The fused MoE layer (router, top-k, routed + shared EXL3 experts, combine) resident in HBM (ne_moe_*)."""

    def __init__(self, eng, ptr, keep=()):
        self.eng, self.ptr, self._keep = eng, ptr, keep
        v = [C.c_int() for _ in range(6)]
        eng._ok(eng.lib.ne_moe_info(ptr, *[C.byref(x) for x in v]), "ne_moe_info")
        self.hid, self.inter, self.ne, self.topk, self.K, self.slots = (x.value for x in v)

    def run_bufs(self, R, x, y, x_off=0, y_off=0, timed=False):
        ms = C.c_double(0)
        self.eng._ok(self.eng.lib.ne_moe_run(self.ptr, R, x.ptr, x_off, y.ptr, y_off,
                                             C.byref(ms) if timed else None), "ne_moe_run")
        return ms.value

    def run_hc(self, R, x, y, h, inj, hout, hc=4, refr=True, x_off=0, y_off=0, timed=False):
        """ne_moe_run_hc: y = the branch, hout = h + branch * inj per stream (device buffers)"""
        d = MoeHc(hc, int(bool(refr)), h.ptr, inj.ptr, hout.ptr)
        ms = C.c_double(0)
        self.eng._ok(self.eng.lib.ne_moe_run_hc(self.ptr, R, x.ptr, x_off, y.ptr, y_off, C.byref(d),
                                                C.byref(ms) if timed else None), "ne_moe_run_hc")
        return ms.value

    def run(self, x):
        x = np.ascontiguousarray(np.atleast_2d(x), np.float32)
        R = x.shape[0]
        xb, yb = self.eng.from_numpy(x), self.eng.alloc(R * self.hid * 4)
        self.run_bufs(R, xb, yb)
        self._R = R
        self._io = (xb, yb)  # "mlp_out" reads the last output buffer: keep it alive
        return yb.download(np.float32, (R, self.hid))

    def read(self, name, R=None):
        R = R or getattr(self, "_R", 1)
        shapes = {"logits": ((R, self.ne), np.float32), "route": ((R, 2 * self.topk), np.uint32),
                  "shared_gate": ((R,), np.float32), "experts_gu": ((R, self.slots, 2, self.inter), np.float32),
                  "experts_dn": ((R, self.slots, self.hid), np.float32), "mlp_out": ((R, self.hid), np.float32)}
        shape, dt = shapes[name]
        out = np.zeros(shape, dt)
        self.eng._ok(self.eng.lib.ne_moe_read(self.ptr, name.encode(), out.ctypes.data, out.nbytes),
                     f"ne_moe_read({name})")
        return out

    def decode(self, e, proj):
        inp, out = (self.inter, self.hid) if proj == 2 else (self.hid, self.inter)
        w = self.eng.alloc(inp * out * 2)
        self.eng._ok(self.eng.lib.ne_moe_decode(self.ptr, e, proj, w.ptr, None), "ne_moe_decode")
        return w.download(np.uint16, (inp, out)).view(np.float16)

    def bytes(self, R=1):
        b = C.c_uint64(0)
        self.eng._ok(self.eng.lib.ne_moe_bytes(self.ptr, R, C.byref(b)), "ne_moe_bytes")
        return b.value

    def free(self):
        if self.ptr:
            self.eng.lib.ne_moe_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Engine:
    def __init__(self, lib=None):
        path = Path(lib or LIB)
        if not path.exists():
            raise EngineError(f"{path} not built (python -m ijah_amd.build)")
        self.lib = C.CDLL(str(path))
        self.missing = []
        for name, (res, args) in SIGNATURES.items():
            try:
                f = getattr(self.lib, name)
            except AttributeError:
                self.missing.append(name)
                continue
            f.restype, f.argtypes = res, args

    def has(self, name):
        try:
            getattr(self.lib, name)
            return True
        except AttributeError:
            return False

    def fn(self, name, restype, argtypes):
        f = getattr(self.lib, name)
        f.restype, f.argtypes = restype, argtypes
        return f

    def last_error(self):
        e = self.lib.ne_last_error()
        return e.decode() if e else ""

    def _ok(self, rc, what):
        if rc != 0:
            raise EngineError(f"{what}: {self.last_error()}")

    def abi_version(self):
        return self.lib.ne_abi_version()

    def device(self):
        d = DeviceInfo()
        self._ok(self.lib.ne_device_query(C.byref(d)), "ne_device_query")
        return {"name": d.name.decode(), "has_nax": bool(d.has_nax), "has_metal4": bool(d.has_metal4),
                "max_buffer_length": d.max_buffer_length, "recommended_working_set": d.recommended_working_set,
                "max_threadgroup_memory": d.max_threadgroup_memory, "backend": d.backend.decode()}

    def sync(self):
        self._ok(self.lib.ne_sync(), "ne_sync")

    def alloc(self, nbytes):
        p = self.lib.ne_alloc(int(nbytes))
        if not p:
            raise EngineError(f"ne_alloc({nbytes}): {self.last_error()}")
        return Buf(self, p)

    def from_numpy(self, arr):
        a = np.ascontiguousarray(arr)
        b = self.alloc(max(a.nbytes, 1))
        b.upload(a)
        return b

    def pack_open(self, path):
        return Pack(self, path)

    def pack_align(self, src, dst, align=64, dry_run=False):
        """reference core/pack_align.h align_pack: a copy of the pack in src under dst whose every tensor's data
        is align-byte aligned in its shard; returns the counts as a dict."""
        st = PackAlignStats()
        self._ok(self.lib.ne_pack_align(str(src).encode(), str(dst).encode(), align, int(dry_run), C.byref(st)),
                 "ne_pack_align")
        return {n: getattr(st, n) for n, _ in PackAlignStats._fields_}

    def kernel_exists(self, fn):
        return self.lib.ne_kernel_exists(fn.encode()) == 1

    def run_kernel(self, fn, args, grid, tg, fconsts=(), tg_mem=0, reps=1, backend=None):
        """reference tools/engine.py run_kernel: args Buf | (Buf, offset) | TensorDesc | bytes | numpy (inline)."""
        keep = []
        ca = (ArgC * max(len(args), 1))()
        for i, a in enumerate(args):
            if isinstance(a, TensorDesc):
                a = a.arg()
            if isinstance(a, Buf):
                ca[i] = ArgC(a.ptr, 0, None, 0)
            elif isinstance(a, tuple) and isinstance(a[0], Buf):
                ca[i] = ArgC(a[0].ptr, int(a[1]), None, 0)
            else:
                raw = a if isinstance(a, (bytes, bytearray)) else np.ascontiguousarray(a).tobytes()
                cb = C.create_string_buffer(bytes(raw), len(raw))
                keep.append(cb)
                ca[i] = ArgC(None, 0, C.cast(cb, C.c_void_p), len(raw))
        fc = (FConst * max(len(fconsts), 1))()
        for i, (idx, ty, val) in enumerate(fconsts):
            bits = int(np.float32(val).view(np.uint32)) if ty == "f32" else int(val) & 0xFFFFFFFF
            fc[i] = FConst(idx, FC_TYPES[ty], bits)
        g = (C.c_uint32 * 3)(*grid)
        t3 = (C.c_uint32 * 3)(*tg)
        ms = C.c_double(0)
        rc = self.lib.ne_run_kernel(fn.encode(), fc, len(fconsts), ca, len(args), C.byref(g), C.byref(t3), tg_mem,
                                    reps, backend.encode() if backend else None, C.byref(ms))
        self._ok(rc, f"ne_run_kernel({fn})")
        return ms.value

    # ---- EXL3 hot path
    def exl3_linear(self, trellis, suh, svh):
        t = np.ascontiguousarray(trellis, np.uint16)
        su = np.ascontiguousarray(suh, np.float16).view(np.uint16)
        sv = np.ascontiguousarray(svh, np.float16).view(np.uint16)
        it, ot, n = t.shape
        p = self.lib.ne_exl3_lin_create(t.ctypes.data, su.ctypes.data, sv.ctypes.data, it * 16, ot * 16, n // 16)
        if not p:
            raise EngineError(f"ne_exl3_lin_create: {self.last_error()}")
        return Exl3Linear(self, p)

    def exl3_linear_load(self, pack, prefix):
        p = self.lib.ne_exl3_lin_load(pack.ptr, prefix.encode())
        if not p:
            raise EngineError(f"ne_exl3_lin_load({prefix}): {self.last_error()}")
        return Exl3Linear(self, p, keep=(pack,))

    def moe_create(self, w):
        """w: dict of numpy arrays in the pack layout (ijah_amd.synth.moe_layer)."""
        d = MoeDesc()
        d.hid, d.inter, d.ne, d.topk, d.K = w["hid"], w["inter"], w["ne"], w["topk"], w["K"]
        d.Ks = w.get("Ks", 0) or 0
        keep = {}

        def arr(key, dt):
            a = w.get(key)
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            if dt == np.float16:
                a = np.ascontiguousarray(a, np.float16).view(np.uint16)
            keep[key] = a
            return a.ctypes.data

        d.router, d.sgate = arr("router", np.uint16), arr("sgate", np.uint16)
        for f, key, dt in (("gt", "gate.trellis", np.uint16), ("ut", "up.trellis", np.uint16),
                           ("dt", "down.trellis", np.uint16), ("gsu", "gate.suh", np.float16),
                           ("gsv", "gate.svh", np.float16), ("usu", "up.suh", np.float16),
                           ("usv", "up.svh", np.float16), ("dsu", "down.suh", np.float16),
                           ("dsv", "down.svh", np.float16), ("sgt", "sgate_proj.trellis", np.uint16),
                           ("sut", "sup_proj.trellis", np.uint16), ("sdt", "sdown_proj.trellis", np.uint16),
                           ("sgsu", "sgate_proj.suh", np.float16), ("sgsv", "sgate_proj.svh", np.float16),
                           ("susu", "sup_proj.suh", np.float16), ("susv", "sup_proj.svh", np.float16),
                           ("sdsu", "sdown_proj.suh", np.float16), ("sdsv", "sdown_proj.svh", np.float16)):
            setattr(d, f, arr(key, dt))
        p = self.lib.ne_moe_create(C.byref(d))
        if not p:
            raise EngineError(f"ne_moe_create: {self.last_error()}")
        return MoeLayer(self, p)

    def moe_load(self, pack, prefix, topk):
        p = self.lib.ne_moe_load(pack.ptr, prefix.encode(), topk)
        if not p:
            raise EngineError(f"ne_moe_load({prefix}): {self.last_error()}")
        return MoeLayer(self, p, keep=(pack,))

    def moe_synth(self, hid, inter, ne, topk, K, has_shared=True, Ks=None, seed=0):
        p = self.lib.ne_moe_synth(hid, inter, ne, topk, K, int(bool(has_shared)), Ks or K, seed)
        if not p:
            raise EngineError(f"ne_moe_synth: {self.last_error()}")
        return MoeLayer(self, p)

    def moe_time(self, layers, R, x, warmup=3, reps=20):
        arr = (C.c_void_p * len(layers))(*[m.ptr for m in layers])
        us = C.c_double(0)
        self._ok(self.lib.ne_moe_time(arr, len(layers), R, x.ptr, warmup, reps, C.byref(us)), "ne_moe_time")
        return us.value

    def lin_time(self, lins, R, x, warmup=3, reps=20):
        """GPU microseconds per linear over a graph of the given linears at R rows (ne_exl3_lin_time)."""
        arr = (C.c_void_p * len(lins))(*[m.ptr for m in lins])
        us = C.c_double(0)
        self._ok(self.lib.ne_exl3_lin_time(arr, len(lins), R, x.ptr, warmup, reps, C.byref(us)), "ne_exl3_lin_time")
        return us.value

    def lin_time_multi(self, lins, R, x, group, warmup=3, reps=20):
        """GPU microseconds per replay of the linears recorded together, `group` per launch (ne_exl3_lin_time_multi)."""
        arr = (C.c_void_p * len(lins))(*[m.ptr for m in lins])
        us = C.c_double(0)
        self._ok(self.lib.ne_exl3_lin_time_multi(arr, len(lins), group, R, x.ptr, warmup, reps, C.byref(us)),
                 "ne_exl3_lin_time_multi")
        return us.value

    def lin_run_multi(self, lins, xs):
        """ne_exl3_lin_run_multi: linear i on rows xs[i] (f32 [R][in_i], one R for all); returns the outputs"""
        R = np.atleast_2d(xs[0]).shape[0]
        xb = [self.from_numpy(np.ascontiguousarray(np.atleast_2d(x), np.float32)) for x in xs]
        yb = [self.alloc(R * m.out * 4) for m in lins]
        n = len(lins)
        self._ok(self.lib.ne_exl3_lin_run_multi((C.c_void_p * n)(*[m.ptr for m in lins]), n, R,
                                                (C.c_void_p * n)(*[b.ptr for b in xb]), (C.c_uint64 * n)(),
                                                (C.c_void_p * n)(*[b.ptr for b in yb]), (C.c_uint64 * n)(), None),
                 "ne_exl3_lin_run_multi")
        return [b.download(np.float32, (R, m.out)) for b, m in zip(yb, lins)]

    def moe_time_kernels(self, layers, R, x, reps=5):
        arr = (C.c_void_p * len(layers))(*[m.ptr for m in layers])
        names = (C.c_char * 16 * 8)()
        us = (C.c_double * 8)()
        n = C.c_int(8)
        self._ok(self.lib.ne_moe_time_kernels(arr, len(layers), R, x.ptr, reps, names, us, C.byref(n)),
                 "ne_moe_time_kernels")
        return {names[i].value.decode(): us[i] for i in range(n.value)}
