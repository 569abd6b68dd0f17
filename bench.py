"""Benchmark: the fused 5-bit EXL3 MoE decode layer at M=1 on one MI355X.

A step is one pass of the MoE hot path over a chain of `--layers` distinct synthetic layers (HID 2048, INTER 512,
512 routed experts + 1 shared expert, top-10, K5 everywhere), captured once as a HIP graph and replayed. Distinct
layers (32 x 1.01 GB resident in HBM, 24 MB touched each) keep every weight read coming from HBM rather than the
256 MB Infinity Cache. Inputs are resident in HBM before the timed region.

value = effective packed-weight GB/s (algorithmic bytes of the touched experts' trellis + suh + svh, the shared
expert and the router, per layer, / time per layer). The roofline entry is the dominant kernel's algorithmic bytes /
its mean duration (HIP events on the library stream). The CPU baseline is the oracle's OpenMP restatement of the
same layer timed on the host's cores on a bounded sample.

    python bench.py [--steps K] [--warmup W] [--layers L]
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
HID, INTER, NE, TOPK, K = 2048, 512, 512, 10, 5


def kernel_bytes(hid=HID, inter=INTER, ne=NE, topk=TOPK, k=K, shared=1):
    """Algorithmic HBM bytes per launch of each kernel of the layer step at M=1 (weights only)."""
    ns = topk + shared
    tr = hid * inter * k // 8
    return {"router": ne * hid * 2,
            "gateup": ns * 2 * (tr + hid * 2),
            "down": ns * (tr + 3 * inter * 2),
            "combine": ns * hid * 2}


def profiled_traffic(kernel):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 PMC summary (FETCH_SIZE and
    WRITE_SIZE, each scaled by the copy-probe factor), or None when no summary covers it."""
    f = ROOT / "profiles" / "moe_step_k5_config2.md"
    if kernel != "fused" or not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def cpu_baseline(seconds=10.0):
    """The oracle's OpenMP layer (router over 512 experts + top-10 + 10 routed and 1 shared K5 expert) on the
    host's cores; per-layer time from a bounded sample. All 512 experts are resident in host memory (1 GB) and each
    layer routes a different input row, so the experts a layer touches change from layer to layer, as on the GPU.
    Returns a dict for the JSON line."""
    from ijah_amd import synth
    from oracle import oracle as O
    O.build()
    rng = np.random.default_rng(99)
    w = synth.moe_layer(99, hid=HID, inter=INTER, ne=NE, topk=TOPK, K=K, shared=True, Ks=K)
    W = O.MoeWeights(w)
    xs = synth.bf16_values(rng, 64, HID)
    # the host's cores, as many as this process may use: the GPU box grants each job a CPU share through
    # OMP_NUM_THREADS (16 per GPU), whatever nproc reports
    host = os.cpu_count() or 1
    threads = min(host, int(os.environ.get("OMP_NUM_THREADS") or host))
    n, t0 = 0, time.perf_counter()
    while True:
        x = xs[n % len(xs)][None]
        lg = O.router_logits(x[0], w["router"])
        ids, wt = O.route(lg, TOPK)
        rt = np.concatenate([ids, wt.view(np.uint32)])[None].astype(np.uint32)
        _, used = O.moe_experts(W, x, rt, fast_threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el > seconds or n >= 5000:
            break
    us = el / n * 1e6
    total = sum(kernel_bytes().values())
    return {"value": round(total / (us * 1e-6) / 1e9, 3), "unit": "GB/s", "cores": int(used), "host_cores": host,
            "cpu_share": f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}", "kind": "port",
            "us_per_layer": round(us, 1),
            "sample": f"{n} M=1 layers over 64 input rows (router 512x2048 + top-10 + 11 K5 experts of 2048x512x3, "
                      f"all 512 experts resident in host memory) in {el:.1f}s"}


def measure_m1(eng, hid, inter, shared, n_layers, steps, seed, k=K):
    """The one-row step (fused launch) of another layer form: the reference's own shape (hidden 2560, inter 640) and/or
    its 8-bit affine shared expert ("q8", the form of its real packs) instead of an EXL3 one; a chain of n_layers
    distinct synthetic layers in one graph, as the headline line. Returns a dict for the JSON line."""
    from ijah_amd import synth
    layers = [eng.moe_synth(hid, inter, NE, TOPK, k, shared, k, seed=seed + 7919 * i) for i in range(n_layers)]
    xb = eng.from_numpy(synth.bf16_values(np.random.default_rng(seed), 1, hid))
    yb = eng.alloc(hid * 4)
    for m in layers:
        m.run_bufs(1, xb, yb)
    eng.sync()
    byts = float(np.mean([m.bytes(1) for m in layers]))
    us = eng.moe_time(layers, 1, xb, warmup=2, reps=steps)
    kus = eng.moe_time_kernels(layers[:4], 1, xb, reps=2)
    for m in layers:
        m.free()
    gbs = byts / (us * 1e-6) / 1e9
    out = {"hidden": hid, "intermediate": inter, "shared": "8-bit affine g128" if shared == "q8" else f"EXL3 K{k}",
           "fused": "fused" in kus, "us_per_layer": round(us, 2), "bytes_per_layer": int(byts),
           "GBps": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}
    if (hid, inter, shared) == (2560, 640, "q8"):
        # the reference's own layer form at M=1 on its hardware (Apple M5 Max): router + shared gate/up + top-10
        # 14.1 us, gate/up 45.4 us, down + combine 31.8 us (27.5-29.4 after its load hoist) in context
        # (docs/kernels.md:136-142, 167); another machine, quoted beside this one, not a vs_baseline
        out["reference_m5max_us"] = [87.0, 91.3]
    print(f"m1 {hid}x{inter} shared={shared}: {out}", file=sys.stderr, flush=True)
    return out


def moe_flops(R, hid=HID, inter=INTER, topk=TOPK, shared=1):
    """Algorithmic flops of the layer's expert GEMMs at R rows (gate, up, down per slot; router excluded)."""
    return 2.0 * 3 * hid * inter * R * (topk + shared)


def measure_batch(eng, R, n_layers, steps, seed, k=K, shared=True):
    """The layer at R rows (BASELINE.json config 4 at R = 16, config 5 at R = 4096) on the grouped matrix-core path:
    a chain of n_layers distinct synthetic layers in one HIP graph, experts and shared expert at k bits. Returns a
    dict for the JSON line."""
    from ijah_amd import synth
    layers = [eng.moe_synth(HID, INTER, NE, TOPK, k, shared, k, seed=seed + 7919 * i) for i in range(n_layers)]
    x = synth.bf16_values(np.random.default_rng(seed), R, HID)
    xb = eng.from_numpy(x)
    yb = eng.alloc(R * HID * 4)
    for m in layers:
        m.run_bufs(R, xb, yb)
    eng.sync()
    byts = float(np.mean([m.bytes(R) for m in layers]))
    us = eng.moe_time(layers, R, xb, warmup=2, reps=steps)
    fl = moe_flops(R)
    out = {"rows": R, "K": k, "shared": "8-bit affine g128" if shared == "q8" else f"EXL3 K{k}",
           "layers_per_step": n_layers, "us_per_layer": round(us, 2),
           "tokens_per_s_per_layer": round(R * 1e6 / us, 1),
           "weight_bytes_per_layer": int(byts), "weight_GBps": round(byts / (us * 1e-6) / 1e9, 1),
           "expert_gemm_TFLOPs": round(fl / (us * 1e-6) / 1e12, 2),
           "pct_f16_mfma_peak": round(100 * fl / (us * 1e-6) / 2.5e15, 2)}
    for m in layers:
        m.free()
    return out


TRUNK = [("q", 2048, 4096, 6), ("k", 2048, 512, 6), ("v", 2048, 512, 6), ("o", 4096, 2048, 6),
         ("lm_head", 2048, 151936, 8)]


def measure_trunk(eng, R, steps, seed, min_bytes=300e6):
    """the trunk linears at R rows, each shape timed over a graph of distinct copies whose
    weights total >= min_bytes (beyond the 256 MB last-level cache, so every replay streams from HBM). Returns
    {name: {us, bytes, GBps, pct_hbm_peak}} plus the q+k+v+o sum."""
    from ijah_amd import synth
    out = {}
    x = synth.bf16_values(np.random.default_rng(seed), R, 4096)
    xb = eng.from_numpy(x)
    for name, inp, o, K in TRUNK:
        rng = np.random.default_rng(seed + inp + o + K)
        t, su, sv = synth.linear(rng, inp, o, K)
        nbytes = t.nbytes + su.nbytes + sv.nbytes
        copies = int(min(64, max(2, np.ceil(min_bytes / nbytes))))
        lins = [eng.exl3_linear(t, su, sv) for _ in range(copies)]
        del t
        us = eng.lin_time(lins, R, xb, warmup=2, reps=max(3, steps))
        for m in lins:
            m.free()
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"in": inp, "out": o, "K": K, "us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1),
                     "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}
        print(f"trunk {name} R={R}: {out[name]}", file=sys.stderr, flush=True)
    # q, k and v in one launch (one input, three linears: record_multi), over copies of the triple
    trip = []
    for name, inp, o, K in TRUNK[:3]:
        rng = np.random.default_rng(seed + inp + o + K)
        trip.append(synth.linear(rng, inp, o, K))
    nb = sum(t.nbytes + su.nbytes + sv.nbytes for t, su, sv in trip)
    copies = int(min(32, max(2, np.ceil(min_bytes / nb))))
    lins = [eng.exl3_linear(*w) for _ in range(copies) for w in trip]
    del trip
    us = eng.lin_time_multi(lins, R, xb, group=3, warmup=2, reps=max(3, steps)) / copies
    for m in lins:
        m.free()
    gbs = nb / (us * 1e-6) / 1e9
    out["qkv_one_launch"] = {"us": round(us, 3), "bytes": int(nb), "GBps": round(gbs, 1),
                             "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}
    print(f"trunk qkv one launch R={R}: {out['qkv_one_launch']}", file=sys.stderr, flush=True)
    # at R rows the weights are read once for all rows: "GBps" is weight bytes over time
    qkvo = sum(out[n]["us"] for n in ("q", "k", "v", "o"))
    qkvo_b = sum(out[n]["bytes"] for n in ("q", "k", "v", "o"))
    out["qkvo_sum"] = {"us": round(qkvo, 3), "GBps": round(qkvo_b / (qkvo * 1e-6) / 1e9, 1)}
    q1 = out["qkv_one_launch"]["us"] + out["o"]["us"]
    out["qkv_one_launch_plus_o"] = {"us": round(q1, 3), "GBps": round(qkvo_b / (q1 * 1e-6) / 1e9, 1)}
    return out


# the reference's own trunk shapes with published M=1 timings on its hardware (docs/trunk6.md:93-100)
TRUNK_REF = [("2560x10240_k6", 2560, 10240, 6, 39.4), ("2560x12288_k6", 2560, 12288, 6, 46.9),
             ("2560x640_k6", 2560, 640, 6, 11.0), ("320x10240_k8", 320, 10240, 8, 9.0)]


def measure_trunk_ref(eng, steps, seed, min_bytes=300e6):
    """The reference's trunk shapes at M=1, timed as measure_trunk (graphs over distinct copies beyond the last-level
    cache); the reference's published us on its M5 Max beside each (a different machine: context, not a target)."""
    from ijah_amd import synth
    out = {}
    xb = eng.from_numpy(synth.bf16_values(np.random.default_rng(seed), 1, 2560))
    for name, inp, o, K, ref_us in TRUNK_REF:
        t, su, sv = synth.linear(np.random.default_rng(seed + inp + o), inp, o, K)
        nbytes = t.nbytes + su.nbytes + sv.nbytes
        copies = int(min(64, max(2, np.ceil(min_bytes / nbytes))))
        lins = [eng.exl3_linear(t, su, sv) for _ in range(copies)]
        us = eng.lin_time(lins, 1, xb, warmup=2, reps=max(3, steps))
        for m in lins:
            m.free()
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1),
                     "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2), "reference_m5max_us": ref_us}
        print(f"trunk ref {name}: {out[name]}", file=sys.stderr, flush=True)
    return out


def run_trunk_eager(eng, steps, seed):
    """Config 3's trunk linears launched one by one (ne_exl3_lin_run, and q/k/v through ne_exl3_lin_run_multi), no
    graphs: a kernel trace of this run gives each shape's kernel time at 1 and 16 rows."""
    from ijah_amd import synth
    lins = {}
    for name, inp, o, K in TRUNK:
        rng = np.random.default_rng(seed + inp + o + K)
        lins[name] = eng.exl3_linear(*synth.linear(rng, inp, o, K))
    out = {}
    for R in (1, 16):
        x = synth.bf16_values(np.random.default_rng(seed + R), R, 4096)
        for name, inp, o, K in TRUNK:
            xb, yb = eng.from_numpy(np.ascontiguousarray(x[:, :inp])), eng.alloc(R * o * 4)
            for _ in range(steps):
                lins[name].run_bufs(R, xb, yb)
        q = [lins[n] for n in ("q", "k", "v")]
        for _ in range(steps):
            eng.lin_run_multi(q, [x[:, :2048]] * 3)
        eng.sync()
        out[f"R{R}"] = steps
    for m in lins.values():
        m.free()
    return {"trunk_eager_runs": out}


class Probes:
    """The measurement probes' own library (ijah_amd/_lib/libijah_probes.so, kept out of the product library):
    ijah_probe_run launches a probe kernel by name on device addresses of the engine's buffers."""

    def __init__(self):
        import ctypes as C
        self.C = C
        self.lib = C.CDLL(str(ROOT / "ijah_amd" / "_lib" / "libijah_probes.so"))
        f = self.lib.ijah_probe_run
        f.restype = C.c_int
        f.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_uint, C.c_int,
                      C.POINTER(C.c_double), C.c_char_p, C.c_int]

    def run(self, name, args, grid, tg, K=-1, variant=-1, tg_mem=0, reps=1):
        """args: Buf, (Buf, byte offset) or a numpy scalar; returns the GPU ms of `reps` launches"""
        C = self.C
        slots = []
        for a in args:
            if isinstance(a, tuple):
                slots.append(a[0].gpu_address() + int(a[1]))
            elif hasattr(a, "gpu_address"):
                slots.append(a.gpu_address())
            else:
                slots.append(int(np.asarray(a).astype(np.int64)) & 0xFFFFFFFFFFFFFFFF)
        arr = (C.c_uint64 * len(slots))(*slots)
        ms, err = C.c_double(0), C.create_string_buffer(256)
        rc = self.lib.ijah_probe_run(name.encode(), K, variant, arr, len(slots), (C.c_uint * 3)(*grid),
                                     (C.c_uint * 3)(*tg), tg_mem, reps, C.byref(ms), err, 256)
        if rc:
            raise RuntimeError(f"probe {name}: {err.value.decode()}")
        return ms.value


def run_stream_probe(eng, total_mb=24, region_mb=2048):
    """probe_stream: 256 workgroups x 16 waves (the fused step's shape) stream total_mb of cold data (a different
    slice of a region_mb buffer each launch, beyond the 256 MB last-level cache), per wave total_mb / 4096, into LDS
    (mode 0) or registers (mode 1); and the same bytes over 1024 x 4 waves. us per launch (median of 8)."""
    pl = Probes()
    region = eng.alloc(region_mb << 20)
    res = eng.alloc(4096 * 64 * 4)
    out = {}
    nb = total_mb << 20
    # one pass over the whole region first: the first touch of its pages (address translation) would otherwise be
    # charged to whichever shape runs first
    for off in range(0, (region_mb << 20) - nb + 1, nb):
        pl.run("probe_stream", [(region, off), np.uint32(nb // 4096 // 1024 * 1024), np.int32(1), res], (256, 1, 1),
               (1024, 1, 1), tg_mem=16 * 4096)
    for shape in ((256, 1024), (512, 512), (1024, 256)):
        waves = shape[0] * shape[1] // 64
        per = nb // waves // 1024 * 1024
        for mode in (0, 1):
            ts, off = [], 0
            for i in range(10):
                if off + nb > (region_mb << 20):
                    off = 0
                t = pl.run("probe_stream", [(region, off), np.uint32(per), np.int32(mode), res],
                           (shape[0], 1, 1), (shape[1], 1, 1), tg_mem=(shape[1] // 64) * 4096)
                off += nb
                if i >= 2:
                    ts.append(t)
            us = 1e3 * float(np.median(ts))
            out[f"wg{shape[0]}x{shape[1] // 64}_{'lds' if mode == 0 else 'vgpr'}"] = {
                "us": round(us, 2), "TBps": round(waves * per / (us * 1e-6) / 1e12, 2), "KB_per_wave": per // 1024}
    region.free()
    res.free()
    return out


def run_probes(eng, iters=4000):
    """probe_mix (ijah_amd/csrc/probes.hip) on every CU at 1, 2, 4 and 8 waves per SIMD: mode 0 decode only, 1 MFMA
    only, 2 decode feeding each wave's MFMA chain, 3 even waves decode / odd waves MFMA (ms per launch). Decode: weights
    per second and SIMD cycles per weight at the measured shader clock; MFMA: dense f16 TFLOP/s."""
    cus = 256
    pl = Probes()
    out = {}
    for K in (5, 8):
        rng = np.random.default_rng(K)
        tiles = eng.from_numpy(rng.integers(0, 1 << 32, 8 * 64 * K // 4, dtype=np.uint32))
        for wps in (1, 2, 4, 8):
            grid = cus * wps  # 4 waves per workgroup: wps waves per SIMD
            res = eng.alloc(grid * 4 * 64 * 4)
            t, cyc = {}, {}
            for mode in range(4):
                pl.run("probe_mix", [tiles, np.int32(iters), np.int32(mode), res], (grid, 1, 1), (256, 1, 1),
                       K=K, tg_mem=4 * 8 * 64 * K)  # warm
                t[mode] = pl.run("probe_mix", [tiles, np.int32(iters), np.int32(mode), res], (grid, 1, 1),
                                 (256, 1, 1), K=K, tg_mem=4 * 8 * 64 * K, reps=3) / 3
                w = res.download(np.uint32, (grid * 4, 64))
                cyc[mode] = float(np.median(w[:, 1]))
                if mode == 0:  # where the waves ran: distinct (XCC, SE, SH, CU) and waves per SIMD; the s_memtime rate
                    hw, xcc = w[:, 2].astype(np.int64), w[:, 3].astype(np.int64) & 0xF
                    cu = (xcc << 8) | ((hw >> 8) & 0xFF)
                    simd = (cu << 2) | ((hw >> 4) & 3)
                    places = {"cus_used": int(len(np.unique(cu))),
                              "max_waves_per_simd": int(np.bincount(np.unique(simd, return_inverse=True)[1]).max()),
                              "memtime_MHz": round(float(np.median(w[:, 1] / np.maximum(w[:, 4], 1))) * 100, 1)}
            waves = grid * 4
            clk = places["memtime_MHz"] * 1e6  # the shader clock the waves saw (s_memtime vs the 100 MHz counter)
            wts = waves * iters * 8 * 512  # weights decoded in modes 0 and 2
            flops = waves * iters * 8 * 2 * 32 * 32 * 16  # modes 1 and 2
            simds = cus * 4
            key = f"K{K}_w{wps}"
            out[key] = {
                "ms": {str(m): round(v, 4) for m, v in t.items()},
                "decode_Gweights_s": round(wts / (t[0] * 1e-3) / 1e9, 1),
                "decode_simd_cycles_per_weight": round(t[0] * 1e-3 * clk * simds / wts, 4),
                "mfma_TFLOPs": round(flops / (t[1] * 1e-3) / 1e12, 1),
                "fused_vs_sum": round(t[2] / (t[0] + t[1]), 3),  # 1.0: no overlap, max/sum: full overlap
                "fused_vs_max": round(t[2] / max(t[0], t[1]), 3),
                "split_vs_half_sum": round(t[3] / ((t[0] + t[1]) / 2), 3),
                "wave_cycles_median": {str(m): cyc[m] for m in cyc},
                # s_memtime cycles per weight of one wave (its own view, no sharing assumptions)
                "wave_cycles_per_weight_decode": round(cyc[0] / (iters * 8 * 512), 4),
                **places,
            }
            if K == 5:  # four chains per decoded tile pair (a 128-row grouped GEMM), accumulators in VGPRs / AGPRs
                for ag in (0, 1):
                    tx = {}
                    for mode in (0, 1):
                        kw = dict(K=K, variant=ag, tg_mem=4 * 8 * 64 * K)
                        args = [tiles, np.int32(iters), np.int32(mode), res]
                        pl.run("probe_x4", args, (grid, 1, 1), (256, 1, 1), **kw)
                        tx[mode] = pl.run("probe_x4", args, (grid, 1, 1), (256, 1, 1), reps=3, **kw) / 3
                    out[key][f"x4_{'agpr' if ag else 'vgpr'}"] = {
                        "ms_chains": round(tx[0], 4), "ms_decode_chains": round(tx[1], 4),
                        "vs_max": round(tx[1] / max(t[0], tx[0]), 3), "vs_sum": round(tx[1] / (t[0] + tx[0]), 3)}
            res.free()
            print(f"probe {key}: {out[key]}", file=sys.stderr, flush=True)
        # the same decode through a 64 KB LDS codebook table (probe_lut): one workgroup per CU of 4, 8 or 16 waves
        for nw in (4, 8, 16):
            res = eng.alloc(cus * nw * 64 * 4)
            t = {}
            for mode in (0, 1, 2, 3):
                args = [tiles, np.int32(iters), np.int32(mode), res]
                kw = dict(K=K, tg_mem=65536 + nw * 8 * 64 * K)
                pl.run("probe_lut", args, (cus, 1, 1), (nw * 64, 1, 1), **kw)
                t[mode] = pl.run("probe_lut", args, (cus, 1, 1), (nw * 64, 1, 1), reps=3, **kw) / 3
            w = res.download(np.uint32, (cus * nw, 64))
            wts = cus * nw * iters * 8 * 512
            clk = float(np.median(w[:, 1] / np.maximum(w[:, 4], 1))) * 100e6
            key = f"K{K}_lut_w{nw // 4}"
            out[key] = {"ms": {str(m): round(v, 4) for m, v in t.items()},
                        "decode_Gweights_s": round(wts / (t[0] * 1e-3) / 1e9, 1),
                        "decode_simd_cycles_per_weight": round(t[0] * 1e-3 * clk * cus * 4 / wts, 4),
                        "with_mfma_vs_decode": round(t[2] / t[0], 3),
                        "half_table_Gweights_s": round(wts / (t[1] * 1e-3) / 1e9, 1),
                        "quarter_table_Gweights_s": round(wts / (t[3] * 1e-3) / 1e9, 1),
                        "mismatched_words": int(w[:, 5].sum())}
            res.free()
            print(f"probe {key}: {out[key]}", file=sys.stderr, flush=True)
        tiles.free()
    return out


def measure_hc_read(eng, R, steps, seed, hid=2560, lr=320, K=6, copies=96):
    """The hyper-connection read (ne_hc_read: prep, down linear + silu epilogue, up linear + output epilogue) at R rows on
    synthetic EXL3 mixes of the reference shape. GPU time per call from HIP events around its launches (median over
    calls). The mixes are 4.9 MB: each call reads its own device copy of them, out of `copies` (96 copies = 470
    MB, beyond the 256 MB last-level cache), so the weights come from HBM as in a model's layer chain."""
    from ijah_amd import synth
    from ijah_amd.engine import hc_read
    rng = np.random.default_rng(seed)
    dn, up = synth.linear(rng, 4 * hid, lr, K), synth.linear(rng, lr, 4 * hid, K)
    mixes = [(eng.exl3_linear(*dn), eng.exl3_linear(*up)) for _ in range(copies)]
    h = eng.from_numpy(rng.standard_normal((R, 4, hid)).astype(np.float32))
    nw = eng.from_numpy(synth.bf16((1 + 0.1 * rng.standard_normal(4 * hid)).astype(np.float32)))
    iw = eng.from_numpy(synth.bf16((rng.standard_normal((4, 4 * hid)) / 100).astype(np.float32)))
    mix, inj, out = eng.alloc(R * lr * 4), eng.alloc(R * 32), eng.alloc(R * hid * 4)
    for m in mixes:  # every copy once, untimed: its scratch sized for R rows (470 MB still cycle through the cache)
        hc_read(*m, R, h, nw, iw, mix, inj, out)
    ms = [hc_read(*mixes[i % copies], R, h, nw, iw, mix, inj, out, timed=True) for i in range(max(10, min(steps, copies)))]
    res = {"rows": R, "hid": hid, "mix_rows": lr, "K": K, "us": round(1e3 * float(np.median(ms)), 3),
           # the down linear and the up linear; hc_prep as a launch of its own above one row (at one row the down
           # linear's workgroups run it); and the up linear's input prepared by a launch of its own when its tile
           # pairs would repeat too much preparation (the library's rule: pairs R > 256 and pairs R in > 256 * 2048)
           "launches": 2 + int(R > 1 or hid % 512 != 0 or hid > 4096)
                       + int(4 * hid // 32 * R > 256 and 4 * hid // 32 * R * lr > 256 * 2048),
           "weights": f"{copies} distinct copies"}
    for ld, lu in mixes:
        ld.free()
        lu.free()
    print(f"hc read R={R}: {res}", file=sys.stderr, flush=True)
    return res


TRACE_FIELDS = {0: "start", 1: "pre-route work done", 2: "route known", 3: "requests issued", 4: "gate/up chunks done",
                5: "h blocks loaded", 6: "down partials stored", 7: "end", 8: "first routed tile in",
                9: "last gate/up chunk done", 10: "down tiles decoded", 11: "prep suh requested", 12: "barrier 1",
                13: "gate/up tiles requested", 15: "shared prep done", 16: "routed prep start",
                18: "routed suh in", 24: "route: keys", 25: "route: sorted", 26: "route: top-k rounds",
                27: "route: softmax"}


def run_moe_trace(eng, layers, seed):
    """The fused M=1 step's per-wave timeline (trace mode: ne_moe_configure "trace"; stamps kept in
    LDS, written at the end of each launch): a `layers`-layer graph timed as bench does, then for the middle layer
    the stamp of each step in us from the launch's first wave start, p0 / p50 / p100 over the waves that reach it."""
    from ijah_amd import synth
    lyr = [eng.moe_synth(2048, 512, 512, 10, 5, True, 5, seed=seed + 7919 * i).configure("trace", 1)
           for i in range(layers)]
    x = eng.from_numpy(synth.bf16_values(np.random.default_rng(seed), 1, 2048))
    us = eng.moe_time(lyr, 1, x, warmup=2, reps=5)
    out = np.zeros(8 * 65536, np.uint64)
    eng.lib.ne_moe_read(lyr[layers // 2].ptr, b"trace", out.ctypes.data, out.nbytes)
    t = out[: 256 * 16 * 32].astype(np.int64).reshape(256, 16, 32)
    base = t[:, :, 0][t[:, :, 0] > 0].min()
    rows = []
    for f, name in TRACE_FIELDS.items():
        m = t[:, :, f] > 0
        if m.any():
            v = (t[:, :, f][m] - base) / 100.0  # 100 MHz wall clock
            rows.append((float(np.median(v)), name, round(float(v.min()), 2), round(float(np.median(v)), 2),
                         round(float(v.max()), 2), int(m.sum())))
    rows.sort()
    for _, name, p0, p50, p100, n in rows:
        print(f"{name:26s} {p0:7.2f} {p50:7.2f} {p100:7.2f}  waves={n}", flush=True)
    xcc = t[:, 0, 31].astype(np.int64)  # the XCD each workgroup ran on
    same = int(np.sum(xcc == np.arange(len(xcc)) % 8))
    print(f"workgroups on XCD (workgroup % 8): {same} of {len(xcc)}; XCD of workgroups 0-15: {xcc[:16].tolist()}; "
          f"XCDs of each class workgroup % 8: {[sorted(set(xcc[r::8].tolist())) for r in range(8)]}", flush=True)
    # where the skew sits: per workgroup the latest wave's stamp, by XCD (workgroup % 8) and the slowest workgroups
    for f in (1, 24, 2, 13, 8, 9, 5, 6):
        v = np.where(t[:, :, f] > 0, (t[:, :, f] - base) / 100.0, np.nan)
        wg = np.nanmax(v, axis=1)
        by_xcd = [round(float(np.nanmedian(wg[x::8])), 2) for x in range(8)]
        slow = np.argsort(-np.nan_to_num(wg, nan=-1))[:6]
        print(f"{TRACE_FIELDS[f]:26s} per-XCD median {by_xcd}  slowest wg {slow.tolist()} "
              f"{[round(float(wg[i]), 2) for i in slow]}", flush=True)
    return {"us_per_layer_traced": round(us, 3), "layers": layers}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batch", action="store_true", help="skip the verify (R=16) and prefill (R=4096) lines")
    ap.add_argument("--eager-only", action="store_true",
                    help="run the layer chain eagerly --steps times and exit (for rocprofv3 --pmc passes)")
    ap.add_argument("--no-trunk", action="store_true", help="skip the trunk (config 3) lines")
    ap.add_argument("--no-m1-forms", action="store_true",
                    help="skip the one-row lines of the other layer forms (8-bit shared expert, hidden 2560)")
    ap.add_argument("--trunk-only", action="store_true", help="only measure the trunk linears (config 3) and exit")
    ap.add_argument("--trunk-eager", action="store_true",
                    help="only run the trunk linears (config 3, 1 and 16 rows, q/k/v also as one launch) eagerly "
                         "--steps times, no graphs (for rocprofv3 kernel traces), and exit")
    ap.add_argument("--hc-only", action="store_true", help="only measure the hyper-connection read and exit")
    ap.add_argument("--batch-rows", type=int, default=0, metavar="R",
                    help="only measure the grouped matrix-core layer at R rows (a 4-layer graph) and exit")
    ap.add_argument("--q8", action="store_true", help="with --batch-rows: the 8-bit affine shared expert")
    ap.add_argument("--moe-trace", action="store_true",
                    help="the fused M=1 step's per-wave timeline (trace mode), then exit")
    ap.add_argument("--probe", action="store_true",
                    help="only run the decode / matrix-core probes (decode cost per weight, MFMA and decode overlap)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="only run the plain copy kernel over MB MiB 5 times (scales --pmc byte counters) and exit")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); the MoE layer shards by "
              "expert across GPUs by design, but no multi-GPU figure is produced here", file=sys.stderr)
        sys.exit(2)

    import ijah_amd
    eng = ijah_amd.load_engine()
    if a.copy_probe:
        n = a.copy_probe << 20
        src, dst = eng.alloc(n), eng.alloc(n)
        for _ in range(5):
            Probes().run("copy_u128", [src, dst, np.uint64(n // 16)], (2048, 1, 1), (256, 1, 1))
        print(json.dumps({"copy_probe_bytes": n, "launches": 5}), flush=True)
        return
    if a.moe_trace:
        print(json.dumps(run_moe_trace(eng, 16, a.seed + 11)), flush=True)
        return
    if a.probe:
        print(json.dumps({"stream": run_stream_probe(eng), "stream96": run_stream_probe(eng, 96), **run_probes(eng)}),
              flush=True)
        return
    if a.hc_only:
        print(json.dumps({"hc_read_m1": measure_hc_read(eng, 1, a.steps, a.seed + 5),
                          "hc_read_m16": measure_hc_read(eng, 16, a.steps, a.seed + 6)}), flush=True)
        return
    if a.trunk_eager:
        print(json.dumps(run_trunk_eager(eng, a.steps, a.seed)), flush=True)
        return
    if a.trunk_only:
        print(json.dumps({"m1": measure_trunk(eng, 1, a.steps, a.seed), "m16": measure_trunk(eng, 16, a.steps, a.seed),
                          "hc_read_m1": measure_hc_read(eng, 1, a.steps, a.seed + 5),
                          "hc_read_m16": measure_hc_read(eng, 16, a.steps, a.seed + 6)}),
              flush=True)
        return
    if a.batch_rows:
        print(json.dumps(measure_batch(eng, a.batch_rows, 4, a.steps, a.seed + a.batch_rows,
                                       shared="q8" if a.q8 else True)), flush=True)
        return
    t_setup = time.perf_counter()
    layers = [eng.moe_synth(HID, INTER, NE, TOPK, K, True, K, seed=a.seed * 1000 + i) for i in range(a.layers)]
    from ijah_amd import synth
    x = synth.bf16_values(np.random.default_rng(a.seed), 1, HID)
    xb = eng.from_numpy(x)
    ybufs = [eng.alloc(HID * 4) for _ in layers]
    for m, yb in zip(layers, ybufs):  # eager pass: routes resident, byte counts
        m.run_bufs(1, xb, yb)
    eng.sync()
    layer_bytes = [m.bytes(1) for m in layers]
    bytes_per_layer = float(np.mean(layer_bytes))
    print(f"setup {time.perf_counter() - t_setup:.1f}s, {a.layers} layers, {bytes_per_layer / 1e6:.2f} MB/layer",
          file=sys.stderr, flush=True)

    if a.eager_only:
        for _ in range(a.steps):
            for m, yb in zip(layers, ybufs):
                m.run_bufs(1, xb, yb)
        eng.sync()
        print(json.dumps({"eager_layers": a.steps * a.layers, "bytes_per_layer": int(bytes_per_layer)}), flush=True)
        return

    eng.sync()
    wall0 = time.perf_counter()
    us_layer = eng.moe_time(layers, 1, xb, warmup=a.warmup, reps=a.steps)
    eng.sync()
    wall = time.perf_counter() - wall0
    ms_per_step = us_layer * a.layers / 1000.0
    gbs = bytes_per_layer / (us_layer * 1e-6) / 1e9

    kus = eng.moe_time_kernels(layers, 1, xb, reps=max(2, a.steps // 10))
    kb = kernel_bytes()
    kb["fused"] = sum(kb.values())
    staged = [k for k in kus if k != "fused"]
    dom = "fused" if "fused" in kus else max(staged, key=lambda k: kus[k])
    achieved = kb[dom] / (kus[dom] * 1e-6) / 1e9
    print("kernels (us per launch): " + ", ".join(f"{k} {v:.2f} ({kb[k] / (v * 1e-6) / 1e9:.0f} GB/s)"
                                                 for k, v in kus.items()), file=sys.stderr, flush=True)

    extra = {}
    for m in layers:  # the M=1 layers' memory is no longer needed
        m.free()
    layers = []
    if not a.no_m1_forms:
        extra["m1_q8_shared"] = measure_m1(eng, HID, INTER, "q8", 16, a.steps, a.seed + 31)
        extra["m1_2560x640"] = measure_m1(eng, 2560, 640, True, 16, a.steps, a.seed + 32)
        extra["m1_2560x640_q8_shared"] = measure_m1(eng, 2560, 640, "q8", 16, a.steps, a.seed + 33)
    if not a.no_batch:
        for R in (2, 4, 8):  # the reference's draft sizes (docs/mtp.md:987-993)
            extra[f"verify_r{R}"] = measure_batch(eng, R, 32, max(5, a.steps // 5), a.seed + R)
            print(f"verify R={R}: {extra[f'verify_r{R}']}", file=sys.stderr, flush=True)
        extra["verify_r16"] = measure_batch(eng, 16, 32, max(5, a.steps // 5), a.seed + 16)
        print(f"verify R=16: {extra['verify_r16']}", file=sys.stderr, flush=True)
        extra["verify_r16_k4"] = measure_batch(eng, 16, 32, max(5, a.steps // 5), a.seed + 17, k=4)
        print(f"verify R=16 K4: {extra['verify_r16_k4']}", file=sys.stderr, flush=True)
        extra["prefill_r4096"] = measure_batch(eng, 4096, 4, 3, a.seed + 4096)
        print(f"prefill R=4096: {extra['prefill_r4096']}", file=sys.stderr, flush=True)
        extra["prefill_r4096_q8_shared"] = measure_batch(eng, 4096, 4, 3, a.seed + 4097, shared="q8")
        print(f"prefill R=4096 q8 shared: {extra['prefill_r4096_q8_shared']}", file=sys.stderr, flush=True)
    if not a.no_trunk:
        extra["trunk_m1"] = measure_trunk(eng, 1, max(5, a.steps // 5), a.seed + 3)
        extra["trunk_m16"] = measure_trunk(eng, 16, max(5, a.steps // 5), a.seed + 4)
        extra["trunk_reference_shapes_m1"] = measure_trunk_ref(eng, max(5, a.steps // 5), a.seed + 7)
        extra["hc_read_m1"] = measure_hc_read(eng, 1, a.steps, a.seed + 5)
        extra["hc_read_m16"] = measure_hc_read(eng, 16, a.steps, a.seed + 6)
    cpu = None if a.no_cpu else cpu_baseline()
    line = {
        "metric": "MoE layer us + effective packed-weight GB/s (% HBM peak), 5-bit EXL3, M=1",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u16 trellis -> fp16 weights, f32 accumulate", "data": "synthetic (seeded, device-generated)",
        "config": {"workload": "fused MoE decode layer, M=1 (BASELINE config 2)", "hidden": HID, "intermediate": INTER,
                   "experts": NE, "shared_experts": 1, "topk": TOPK, "K": K, "rows": 1,
                   "layers_per_step": a.layers, "parallelism": "none (1 GPU)"},
        "us_per_layer": round(us_layer, 3), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "tokens_per_s_per_layer": round(1e6 / us_layer, 1), "bytes_per_layer": int(bytes_per_layer),
        "wall_s_timed": round(wall, 3),
        "kernels_us": {k: round(v, 3) for k, v in kus.items()},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(dom),
                     "bytes_per_launch": kb[dom]},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
