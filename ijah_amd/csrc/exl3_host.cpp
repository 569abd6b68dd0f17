// Hot-path entry points (include/ijah_exl3.h): EXL3 linears and the fused MoE layer, resident in HBM.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <set>

#include "kernels.h"
#include "pack.h"

using namespace ijah;

namespace {

int had_size(int d) {  // reference tools/convert_trunk_enc.py:59-63
  for (int n : {128, 64, 32, 16})
    if (d % n == 0) return n;
  throw Error(strfmt("no Hadamard size for %d", d));
}
float had_scale(int n) { return (float)(1.0 / std::sqrt((double)n)); }

template <typename T>
T *dev_alloc(size_t count) {
  void *p = nullptr;
  if (count) IJ_HIP(hipMalloc(&p, count * sizeof(T)));
  return (T *)p;
}
void dev_free(void *p) {
  if (p) (void)hipFree(p);
}

// Copies the tiles of a trellis [IT][OT][16K] (pack layout) into the re-laid order [OT/2][IT][2] at dst (host).
void relay_tiles(const uint16_t *src, int IT, int OT, int K, uint8_t *dst) {
  const size_t tb = 32u * (size_t)K;
  const int OTp = OT + (OT & 1);
  for (int tk = 0; tk < IT; tk++)
    for (int tn = 0; tn < OTp; tn++) {
      uint8_t *d = dst + relaid_tile(IT, tk, tn) * tb;
      if (tn < OT) memcpy(d, (const uint8_t *)src + ((size_t)tk * OT + tn) * tb, tb);
      else memset(d, 0, tb);
    }
}

void check_dims(int in, int out, int K) {
  IJ_CHECK(in > 0 && out > 0 && in % 16 == 0 && out % 16 == 0, "EXL3 dims %d x %d must be multiples of 16", in, out);
  IJ_CHECK(K >= 2 && K <= 8, "EXL3 K=%d not instantiated (2..8)", K);
  had_size(in);
  had_size(out);
}

}  // namespace

// ---------------------------------------------------------------------------------------------------- linear
struct ne_exl3_lin {
  int in = 0, out = 0, K = 0, IT = 0, OT = 0, OTp = 0, had_in = 0, had_out = 0;
  uint32_t *tiles = nullptr;
  uint16_t *suh = nullptr, *svh = nullptr;
  uint16_t *xh = nullptr;  // [kLinMaxRows][in]
  float *part = nullptr;   // [S][part_rows][OTp*16]: k group partials
  uint32_t *cnt = nullptr; // per 128-column output block (the one-launch path's completion counters)
  bool one_launch = true;  // IJAH_LIN_PATH=staged at creation: prep, GEMM and finish as three launches
  int part_rows = 0;
  float *hc_scr = nullptr;  // the HC read's scratch when this is its up linear (xn, u, ip), hc_rows rows
  int hc_rows = 0;
  ~ne_exl3_lin() {
    dev_free(hc_scr);
    dev_free(tiles);
    dev_free(suh);
    dev_free(svh);
    dev_free(xh);
    dev_free(part);
    dev_free(cnt);
  }
  // k groups (the partials each output column sums in the finisher): fixed by the shape
  int groups() const { return (IT + kLinGroupKt - 1) / kLinGroupKt; }
  // the input preparation runs inside the GEMM (each tile pair's workgroups prepare their own k chunks) unless that
  // repeats too much work: many tile pairs times many rows take one prep launch instead (same results)
  // the rows prepared once by a launch of their own when many tile pairs would each prepare them again (measured:
  // 16 rows of q / o 2048->4096 / 4096->2048, 128 pairs, take 15 us so against 16.6 us preparing in each workgroup),
  // unless the input is short enough that preparing it again in each workgroup costs less than a launch (the HC
  // read's up linear, 320 -> 10240)
  bool prep_launch(int R) const { return (long)(OTp / 2) * R > 256 && (long)(OTp / 2) * R * in > 256L * 2048; }
  // many tile pairs (a vocabulary head): one workgroup per pair loops over the k groups (same results)
  bool k_loop(int R) const { return OTp / 2 >= 2048 && groups() <= 16 && R <= 4 && prep_launch(R); }
  // the same linears at 5..32 rows: 8 tile pairs per workgroup share each k chunk's staged rows (same results)
  bool k_wide(int R) const { return OTp / 2 >= 2048 && R > 4 && R <= kLinMaxRows && prep_launch(R); }
};

static ne_exl3_lin *lin_create(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh, int in, int out,
                               int K) {
  check_dims(in, out, K);
  IJ_CHECK(trellis && suh && svh, "null array");
  ensure_device();
  stream();  // the library's stream exists before any run (the allocation-free run then sets nothing up)
  auto l = std::make_unique<ne_exl3_lin>();
  l->in = in;
  l->out = out;
  l->K = K;
  l->IT = in / 16;
  l->OT = out / 16;
  l->OTp = l->OT + (l->OT & 1);
  l->had_in = had_size(in);
  l->had_out = had_size(out);
  const size_t tbytes = (size_t)l->IT * l->OTp * 32 * K;
  std::vector<uint8_t> host(tbytes);
  relay_tiles(trellis, l->IT, l->OT, K, host.data());
  l->tiles = (uint32_t *)dev_alloc<uint8_t>(tbytes);
  IJ_HIP(hipMemcpy(l->tiles, host.data(), tbytes, hipMemcpyHostToDevice));
  l->suh = dev_alloc<uint16_t>(in);
  l->svh = dev_alloc<uint16_t>(out);
  IJ_HIP(hipMemcpy(l->suh, suh, 2u * in, hipMemcpyHostToDevice));
  IJ_HIP(hipMemcpy(l->svh, svh, 2u * out, hipMemcpyHostToDevice));
  l->xh = dev_alloc<uint16_t>((size_t)kLinMaxRows * in);
  const size_t nc = (size_t)((out + 127) / 128) * kSyncStride;
  l->cnt = dev_alloc<uint32_t>(nc);
  IJ_HIP(hipMemset(l->cnt, 0, nc * 4));
  l->one_launch = true;
  return l.release();
}

extern "C" {

NE_API ne_exl3_lin *ne_exl3_lin_create(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh, int in,
                                       int out, int K) {
  ne_exl3_lin *r = nullptr;
  c_call([&] { r = lin_create(trellis, suh, svh, in, out, K); });
  return r;
}

NE_API ne_exl3_lin *ne_exl3_lin_load(const ne_pack *p, const char *prefix) {
  ne_exl3_lin *r = nullptr;
  c_call([&] {
    IJ_CHECK(p && prefix, "null argument");
    const std::string pre = prefix;
    const TensorInfo &t = p->pack->need(pre + ".trellis", NE_U16, {-1, -1, -1});
    const int in = (int)t.shape[0] * 16, out = (int)t.shape[1] * 16;
    IJ_CHECK(t.shape[2] % 16 == 0, "%s.trellis: last dim %lld not 16 K", prefix, (long long)t.shape[2]);
    const int K = (int)t.shape[2] / 16;
    const TensorInfo &su = p->pack->need(pre + ".suh", NE_F16, {in});
    const TensorInfo &sv = p->pack->need(pre + ".svh", NE_F16, {out});
    r = lin_create((const uint16_t *)t.host, (const uint16_t *)su.host, (const uint16_t *)sv.host, in, out, K);
  });
  return r;
}

NE_API void ne_exl3_lin_free(ne_exl3_lin *l) {
  if (l) {
    (void)hipStreamSynchronize(stream());
    delete l;
  }
}

NE_API int ne_exl3_lin_info(const ne_exl3_lin *l, int *in, int *out, int *K) {
  return c_call([&] {
    IJ_CHECK(l, "null linear");
    if (in) *in = l->in;
    if (out) *out = l->out;
    if (K) *K = l->K;
  });
}

// Captures `work` on s into an executable graph. The capture is always ended, also when `work` throws: a stream left
// capturing would record every later launch into an abandoned graph.
static hipGraphExec_t capture_graph(hipStream_t s, hipGraph_t &g, const std::function<void()> &work) {
  IJ_HIP(hipStreamSynchronize(s));
  IJ_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  try {
    work();
  } catch (...) {
    hipGraph_t dead = nullptr;
    (void)hipStreamEndCapture(s, &dead);
    if (dead) (void)hipGraphDestroy(dead);
    throw;
  }
  IJ_HIP(hipStreamEndCapture(s, &g));
  hipGraphExec_t ge = nullptr;
  IJ_HIP(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  return ge;
}

static void timed(hipStream_t s, double *gpu_ms, const std::function<void()> &work) {
  if (!gpu_ms) {
    work();
    return;
  }
  hipEvent_t e0, e1;
  IJ_HIP(hipEventCreate(&e0));
  IJ_HIP(hipEventCreate(&e1));
  IJ_HIP(hipEventRecord(e0, s));
  work();
  IJ_HIP(hipEventRecord(e1, s));
  IJ_HIP(hipEventSynchronize(e1));
  float ms = 0.f;
  IJ_HIP(hipEventElapsedTime(&ms, e0, e1));
  *gpu_ms = ms;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
}

}  // extern "C"

// The buffers of one run taken from caller-provided scratch instead of the linear's own (the allocation-free entry
// point): completion counters, prepared input, k-split partials.
struct LinScratch {
  uint32_t *cnt;
  uint16_t *xh;
  float *part;
};

// LinArgs of one run at R rows (the k group partials grown to R rows as needed, or taken from sc)
static LinArgs lin_args(ne_exl3_lin *l, int R, const float *x, float *y, const LinEpi &epi = LinEpi(),
                        const LinScratch *sc = nullptr) {
  const bool kloop = l->one_launch && l->k_loop(R);
  const bool wide = l->one_launch && epi.kind != 8 && l->k_wide(R);
  const int S = kloop ? 1 : l->groups();
  if (!sc && R > l->part_rows) {  // never while the stream is captured: a captured launch would keep the freed buffer
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    IJ_HIP(hipStreamIsCapturing(stream(), &cs));
    IJ_CHECK(cs == hipStreamCaptureStatusNone, "linear: partial scratch must grow before a stream capture");
    dev_free(l->part);
    l->part = dev_alloc<float>((size_t)S * R * l->OTp * 16);
    l->part_rows = R;
  }
  LinArgs a;
  a.tiles = l->tiles;
  a.suh = l->suh;
  a.svh = l->svh;
  a.in = l->in;
  a.out = l->out;
  a.K = l->K;
  a.IT = l->IT;
  a.OT = l->OT;
  a.had_in = l->had_in;
  a.had_out = l->had_out;
  a.sc_in = had_scale(l->had_in);
  a.sc_out = had_scale(l->had_out);
  a.R = R;
  a.S = S;
  a.x = x;
  a.y = y;
  a.xh = sc ? sc->xh : l->xh;
  a.part = sc ? sc->part : l->part;
  a.epi = epi;
  a.cnt = l->one_launch ? (sc ? sc->cnt : l->cnt) : nullptr;
  a.xh_in = (!l->one_launch || l->prep_launch(R)) ? 1 : 0;
  a.kloop = kloop ? 1 : wide ? 2 : 0;
  return a;
}

static void lin_launch(ne_exl3_lin *l, int R, const float *x, float *y, hipStream_t s,
                       const LinEpi &epi = LinEpi(), const LinScratch *sc = nullptr) {
  launch_lin(lin_args(l, R, x, y, epi, sc), s);
}
// several linears at R rows: one launch per run of consecutive linears of one K and path (at most `group` each)
static void lin_launch_multi(ne_exl3_lin *const *l, int n, int R, const float *const *x, float *const *y,
                             const LinEpi *epi, hipStream_t s, int group = kLinMulti) {
  LinArgs a[kLinMulti];
  int k = 0;
  for (int i = 0; i < n; i++) {
    const LinArgs ai = lin_args(l[i], R, x[i], y[i], epi ? epi[i] : LinEpi());
    if (k > 0 && (k == group || ai.K != a[0].K || (bool)ai.cnt != (bool)a[0].cnt || ai.kloop != a[0].kloop ||
                  ai.kloop == 2)) {
      launch_lin_multi(a, k, s);
      k = 0;
    }
    a[k++] = ai;
  }
  if (k) launch_lin_multi(a, k, s);
}

static size_t lin_part_bytes(const ne_exl3_lin *l, int R) { return (size_t)l->groups() * R * l->OTp * 16 * 4; }
// Scratch bytes of one run at R rows from the caller-provided scratch: counters, prepared input, partials, each part
// on a 256-byte boundary
static size_t lin_scratch_layout(const ne_exl3_lin *l, int R, LinScratch *sc, uint8_t *base) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t ncnt = (size_t)((l->out + 127) / 128) * kSyncStride;
  const size_t o_xh = up(ncnt * 4), o_part = o_xh + up((size_t)R * l->in * 2);
  const size_t total = o_part + up(lin_part_bytes(l, R));
  if (sc) {
    sc->cnt = (uint32_t *)base;
    sc->xh = (uint16_t *)(base + o_xh);
    sc->part = (float *)(base + o_part);
  }
  return total;
}

extern "C" {

NE_API int ne_exl3_lin_run(ne_exl3_lin *l, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                           double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(l && x && y, "null argument");
    IJ_CHECK(R >= 1 && R <= kLinMaxRows, "rows %d (1..%d)", R, kLinMaxRows);
    IJ_CHECK(x_off % 4 == 0 && y_off % 4 == 0, "offsets must be 4-byte aligned");
    IJ_CHECK(x_off + (uint64_t)R * l->in * 4 <= x->size, "x buffer too small for [%d][%d] f32", R, l->in);
    IJ_CHECK(y_off + (uint64_t)R * l->out * 4 <= y->size, "y buffer too small for [%d][%d] f32", R, l->out);
    const float *xp = (const float *)((const char *)ne_dev(x) + x_off);
    float *yp = (float *)((char *)ne_dev(y) + y_off);
    timed(stream(), gpu_ms, [&] { lin_launch(l, R, xp, yp, stream()); });
  });
}

NE_API int ne_exl3_lin_run_noalloc(ne_exl3_lin *l, int R, const ne_buf *x, uint64_t x_off, ne_buf *y,
                                   uint64_t y_off) {
  return c_call([&] {
    IJ_CHECK(l && x && y, "null argument");
    IJ_CHECK(R >= 1 && R <= kLinMaxRows, "rows %d (1..%d)", R, kLinMaxRows);
    IJ_CHECK(x_off % 4 == 0 && y_off % 4 == 0, "offsets must be 4-byte aligned");
    IJ_CHECK(x_off + (uint64_t)R * l->in * 4 <= x->size, "x buffer too small for [%d][%d] f32", R, l->in);
    IJ_CHECK(y_off + (uint64_t)R * l->out * 4 <= y->size, "y buffer too small for [%d][%d] f32", R, l->out);
    const size_t need = lin_scratch_layout(l, R, nullptr, nullptr);
    IJ_CHECK(need <= kNoAllocScratchBytes,
             "no-alloc linear %d -> %d at %d rows needs %zu bytes of scratch; the maximum is %zu (use fewer rows "
             "or ne_exl3_lin_run)", l->in, l->out, R, need, kNoAllocScratchBytes);
    ensure_device();
    LinScratch sc;
    lin_scratch_layout(l, R, &sc, noalloc_scratch());
    const hipStream_t s = stream();
    // the block counters start at zero (the previous call on this GPU left them so unless it failed)
    launch_zero_u32(sc.cnt, (size_t)((l->out + 127) / 128) * kSyncStride, s);
    lin_launch(l, R, (const float *)((const char *)ne_dev(x) + x_off), (float *)((char *)ne_dev(y) + y_off), s, LinEpi(),
               &sc);
    IJ_HIP(hipGetLastError());
  });
}

NE_API int ne_exl3_lin_run_epi(ne_exl3_lin *l, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                               const ne_exl3_epi *epi, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(l && x && y && epi, "null argument");
    IJ_CHECK(R >= 1 && R <= kLinMaxRows, "rows %d (1..%d)", R, kLinMaxRows);
    IJ_CHECK(x_off % 4 == 0 && y_off % 4 == 0, "offsets must be 4-byte aligned");
    const int k = epi->kind;
    IJ_CHECK(k == 0 || k == 1 || k == 2 || k == 3 || k == 5 || k == 6 || k == 7,
             "epilogue %d (0, 1, 2, 3, 5, 6 or 7; 4 and 8 are not supported)", k);
    const int ldy = epi->ldy ? epi->ldy : l->out;
    IJ_CHECK(ldy >= l->out, "ldy %d below out %d", ldy, l->out);
    IJ_CHECK(x_off + (uint64_t)R * l->in * 4 <= x->size, "x buffer too small for [%d][%d] f32", R, l->in);
    IJ_CHECK(y_off + ((uint64_t)(R - 1) * ldy + l->out) * 4 <= y->size, "y buffer too small for %d rows of stride %d",
             R, ldy);
    LinEpi e;
    e.kind = k;
    e.refr = epi->refr ? 1 : 0;
    e.ldy = ldy;
    auto need = [&](const ne_buf *b, uint64_t bytes, const char *name) -> float * {
      IJ_CHECK(b && b->size >= bytes, "epilogue %d: %s missing or under %llu bytes", k, name,
               (unsigned long long)bytes);
      return (float *)ne_dev(b);
    };
    if (k == 1) {
      IJ_CHECK(epi->hc >= 1 && epi->hc <= 8, "epilogue 1: hc %d (1..8)", epi->hc);
      e.hc = epi->hc;
      const uint64_t hb = (uint64_t)R * e.hc * l->out * 4;
      e.e0 = need(epi->e0, hb, "e0 (h)");
      e.e1 = need(epi->e1, (uint64_t)R * 8 * 4, "e1 (inj)");
      e.e2 = need(epi->e2, hb, "e2 (hout)");
    } else if (k == 6) {
      e.e0 = need(epi->e0, (uint64_t)l->out * 2, "e0 (A_log)");
      e.e1 = need(epi->e1, (uint64_t)l->out * 2, "e1 (dt_bias)");
    } else if (k == 7) {
      IJ_CHECK(l->out <= 640, "epilogue 7: out %d above 640 (512 + one 128-wide key)", l->out);
      e.e0 = need(epi->e0, 512, "e0 (key cache)");
      e.e1 = need(epi->e1, 4, "e1 (position)");
      e.cap = (int)std::min<uint64_t>(epi->e0->size / 512, 1u << 30);
    }
    const float *xp = (const float *)((const char *)ne_dev(x) + x_off);
    float *yp = (float *)((char *)ne_dev(y) + y_off);
    timed(stream(), gpu_ms, [&] { lin_launch(l, R, xp, yp, stream(), e); });
  });
}

NE_API int ne_hc_read(ne_exl3_lin *down, ne_exl3_lin *up, int R, const ne_buf *h, const ne_buf *hc_norm,
                      const ne_buf *inject, ne_buf *mix, ne_buf *inj, ne_buf *out, int refr, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(down && up && h && hc_norm && inject && mix && inj && out, "null argument");
    IJ_CHECK(R >= 1 && R <= kLinMaxRows, "rows %d (1..%d)", R, kLinMaxRows);
    const int hcd = up->out, hid = hcd / 4, lr = down->out;
    IJ_CHECK(hcd % 4 == 0 && down->in == hcd && up->in == lr,
             "down [%d -> %d] and up [%d -> %d] must be 4 hid -> lr -> 4 hid", down->in, down->out, up->in, up->out);
    IJ_CHECK(hid % 64 == 0, "hid %d must be a multiple of 64", hid);
    IJ_CHECK(h->size >= (uint64_t)R * hcd * 4, "h buffer too small for [%d][4][%d] f32", R, hid);
    IJ_CHECK(hc_norm->size >= (uint64_t)hcd * 2, "hc_norm must hold %d bf16", hcd);
    IJ_CHECK(inject->size >= (uint64_t)4 * hcd * 2, "inject must hold [4][%d] bf16", hcd);
    IJ_CHECK(mix->size >= (uint64_t)R * lr * 4, "mix buffer too small for [%d][%d] f32", R, lr);
    IJ_CHECK(inj->size >= (uint64_t)R * 8 * 4, "inj buffer too small for [%d][8] f32", R);
    IJ_CHECK(out->size >= (uint64_t)R * hid * 4, "out buffer too small for [%d][%d] f32", R, hid);
    IJ_CHECK(hid % 128 == 0, "hid %d must be a multiple of 128", hid);
    const int nbs = hid / 128;
    if (R > up->hc_rows) {
      dev_free(up->hc_scr);
      const size_t nctr = (size_t)(1 + kLinMaxRows) * nbs * kSyncStride;
      up->hc_scr = dev_alloc<float>((size_t)kLinMaxRows * (2 * (size_t)hcd + 16 * (size_t)((hid + 255) / 256)) + nctr);
      up->hc_rows = kLinMaxRows;
      float *c0 = up->hc_scr + (size_t)kLinMaxRows * (2 * (size_t)hcd + 16 * (size_t)((hid + 255) / 256));
      IJ_HIP(hipMemset(c0, 0, nctr * 4));  // the output counters (each reset by its last arrival)
    }
    float *xn = up->hc_scr, *u = xn + (size_t)kLinMaxRows * hcd, *ip = u + (size_t)kLinMaxRows * hcd;
    uint32_t *ctr = (uint32_t *)(up->hc_scr + (size_t)kLinMaxRows * (2 * (size_t)hcd + 16 * (size_t)((hid + 255) / 256)));
    const float *hp = (const float *)ne_dev(h);
    const uint16_t *nw = (const uint16_t *)ne_dev(hc_norm);
    float *injp = (float *)ne_dev(inj);
    LinEpi act;  // the down linear's epilogue: mix = rr(silu(rr(v) / 4))
    act.kind = 2;
    act.refr = refr ? 1 : 0;
    LinEpi fin;  // the up linear's: u to scratch, then the output columns and gates (kind 8)
    fin.kind = 8;
    fin.refr = act.refr;
    fin.hid = hid;
    fin.e0 = u;
    fin.e1 = const_cast<float *>(hp);
    fin.e2 = (float *)ne_dev(out);
    fin.e3 = ip;
    fin.e4 = injp;
    fin.w16 = nw;
    fin.ctr = ctr;
    timed(stream(), gpu_ms, [&] {
      hipStream_t s = stream();
      // one row: hc_prep's step runs inside the down linear's workgroups (one launch fewer, the same bits)
      LinArgs da = lin_args(down, R, hp, (float *)ne_dev(mix), act);
      if (R == 1 && !da.xh_in && !da.kloop && da.cnt && hid % 512 == 0 && hid <= 4096) {
        da.hc.nw = nw;
        da.hc.iw = (const uint16_t *)ne_dev(inject);
        da.hc.ip = ip;
        da.hc.inj = injp;
        da.hc.hid = hid;
        launch_lin(da, s);
      } else {
        launch_hc_prep(hp, nw, (const uint16_t *)ne_dev(inject), xn, ip, injp, R, hid, s);
        lin_launch(down, R, xn, (float *)ne_dev(mix), s, act);
      }
      lin_launch(up, R, (const float *)ne_dev(mix), u, s, fin);
    });
  });
}

}  // extern "C"

// n linears at R rows reading x, captured once (one launch per linear, or multi-linear launches) and replayed:
// GPU time per replay in us
static double lin_time(ne_exl3_lin *const *lins, int n, int R, const ne_buf *x, int warmup, int reps, int group) {
  IJ_CHECK(lins && n >= 1 && x && reps >= 1 && R >= 1 && R <= kLinMaxRows, "bad arguments");
  size_t ytot = 0;
  for (int i = 0; i < n; i++) {
    IJ_CHECK(lins[i], "null linear %d", i);
    IJ_CHECK((uint64_t)R * lins[i]->in * 4 <= x->size, "x buffer too small for linear %d", i);
    ytot += (size_t)R * lins[i]->out;
  }
  hipStream_t s = stream();
  float *ys = dev_alloc<float>(ytot);
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  auto cleanup = [&] {
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    dev_free(ys);
  };
  double ms = 0;
  try {
    for (int i = 0; i < n; i++) lin_args(lins[i], R, nullptr, nullptr);  // grow the partials before capture
    std::vector<const float *> xp(n, (const float *)ne_dev(x));
    std::vector<float *> yp(n);
    for (int i = 0, yo = 0; i < n; yo += R * lins[i]->out, i++) yp[i] = ys + yo;
    ge = capture_graph(s, g, [&] {
      if (group > 1) {
        lin_launch_multi(lins, n, R, xp.data(), yp.data(), nullptr, s, group);
      } else {
        for (int i = 0; i < n; i++) lin_launch(lins[i], R, xp[i], yp[i], s);
      }
    });
    for (int i = 0; i < warmup; i++) IJ_HIP(hipGraphLaunch(ge, s));
    timed(s, &ms, [&] {
      for (int i = 0; i < reps; i++) IJ_HIP(hipGraphLaunch(ge, s));
    });
  } catch (...) {
    cleanup();
    throw;
  }
  cleanup();
  return ms * 1000.0 / reps;
}

extern "C" {

NE_API int ne_exl3_lin_time(ne_exl3_lin *const *lins, int n, int R, const ne_buf *x, int warmup, int reps,
                            double *us_per_lin) {
  return c_call([&] {
    IJ_CHECK(us_per_lin, "null argument");
    *us_per_lin = lin_time(lins, n, R, x, warmup, reps, 1) / n;
  });
}

NE_API int ne_exl3_lin_time_multi(ne_exl3_lin *const *lins, int n, int group, int R, const ne_buf *x, int warmup,
                                  int reps, double *us) {
  return c_call([&] {
    IJ_CHECK(us && group >= 1 && group <= kLinMulti, "bad arguments");
    *us = lin_time(lins, n, R, x, warmup, reps, group);
  });
}

NE_API int ne_exl3_lin_run_multi(ne_exl3_lin *const *lins, int n, int R, const ne_buf *const *x,
                                 const uint64_t *x_off, ne_buf *const *y, const uint64_t *y_off, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(lins && x && y && x_off && y_off && n >= 1 && n <= 64, "bad arguments");
    IJ_CHECK(R >= 1 && R <= kLinMaxRows, "rows %d (1..%d)", R, kLinMaxRows);
    std::vector<const float *> xp(n);
    std::vector<float *> yp(n);
    for (int i = 0; i < n; i++) {
      IJ_CHECK(lins[i] && x[i] && y[i], "null linear / buffer %d", i);
      IJ_CHECK(x_off[i] % 4 == 0 && y_off[i] % 4 == 0, "offsets must be 4-byte aligned");
      IJ_CHECK(x_off[i] + (uint64_t)R * lins[i]->in * 4 <= x[i]->size, "x %d too small for [%d][%d] f32", i, R,
               lins[i]->in);
      IJ_CHECK(y_off[i] + (uint64_t)R * lins[i]->out * 4 <= y[i]->size, "y %d too small for [%d][%d] f32", i, R,
               lins[i]->out);
      xp[i] = (const float *)((const char *)ne_dev(x[i]) + x_off[i]);
      yp[i] = (float *)((char *)ne_dev(y[i]) + y_off[i]);
    }
    timed(stream(), gpu_ms, [&] { lin_launch_multi(lins, n, R, xp.data(), yp.data(), nullptr, stream()); });
  });
}

NE_API int ne_exl3_lin_decode(ne_exl3_lin *l, ne_buf *w, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(l && w, "null argument");
    IJ_CHECK(w->size >= (uint64_t)l->in * l->out * 2, "w buffer too small for [%d][%d] fp16", l->in, l->out);
    timed(stream(), gpu_ms, [&] { launch_decode(l->tiles, l->IT, l->OT, l->K, (uint16_t *)ne_dev(w), stream()); });
  });
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------------- MoE layer
// The few-row MoE kernels' partials and block counters, one pool per layer shape shared by every layer of that shape
// (the layers run one after another on the library's stream; the counters are back at zero after each launch). A
// pool only grows (counters zeroed), never while a stream is captured. A grown pool's old arrays are kept until the
// process ends: a graph captured earlier, or another layer, may still hold their addresses; every launch takes the
// pool's current arrays (few_pool_now), which are at least as large as any layer's need.
struct FewPool {
  uint64_t *part = nullptr;
  uint32_t *ep = nullptr;
  int chunks = 0;
};
static std::mutex g_few_mu;
static std::map<std::pair<int, int>, FewPool> g_few_pools;
static std::vector<FewPool> g_few_retired;
static void few_pool(int hid, int inter, int chunks, uint64_t **part, uint32_t **ep) {
  std::lock_guard<std::mutex> g(g_few_mu);
  FewPool &p = g_few_pools[{hid, inter}];
  if (chunks > p.chunks) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    IJ_HIP(hipStreamIsCapturing(stream(), &cs));
    IJ_CHECK(cs == hipStreamCaptureStatusNone, "MoE: few-row scratch must grow before a stream capture");
    if (p.part) g_few_retired.push_back(p);
    const size_t np = moe_batch_few_part(chunks, hid, inter), ne = moe_batch_few_epochs(chunks, inter);
    p.part = dev_alloc<uint64_t>(np);
    p.ep = dev_alloc<uint32_t>(ne);
    IJ_HIP(hipMemset(p.part, 0, np * 8));
    IJ_HIP(hipMemset(p.ep, 0, ne * 4));
    p.chunks = chunks;
  }
  *part = p.part;
  *ep = p.ep;
}
// the pool's current arrays (no growth): what a launch uses
static void few_pool_now(int hid, int inter, uint64_t **part, uint32_t **ep, int *chunks) {
  std::lock_guard<std::mutex> g(g_few_mu);
  const FewPool &p = g_few_pools[{hid, inter}];
  *part = p.part;
  *ep = p.ep;
  *chunks = p.chunks;
}

struct ne_moe {
  int hid = 0, inter = 0, ne = 0, topk = 0, K = 0, Ks = 0, has_shared = 0, has_sgate = 0, ksplit = 4;
  ExpertLayout lay, slay;
  uint8_t *experts = nullptr, *shared = nullptr;
  uint8_t *q8 = nullptr;       // the 8-bit affine shared expert (q8_offsets), in place of an EXL3 shared slot
  float *q8gu = nullptr, *q8o = nullptr;  // its per-row outputs (staged and batched paths)
  uint16_t *q8bf = nullptr;               // its weight bytes as bf16 (the many-row matrix-core form)
  uint16_t *router = nullptr;  // [ne + has_sgate][hid]
  int Rcap = 0;
  float *logits = nullptr, *sgv = nullptr, *guo = nullptr, *dn = nullptr;
  uint16_t *hprep = nullptr;
  uint32_t *route = nullptr, *sync = nullptr, *plan = nullptr;
  float *part = nullptr;      // the fused step's tagged partials
  size_t part_floats = 0;
  uint32_t *fsync = nullptr;  // the fused step's launch epoch
  int plan_grid = 0;  // fused step: its grid (0: no plan, the staged path runs)
  int plan_slots = 0; // fused step: the LDS slots its plan uses
  MoeBatchBufs bat;   // batched path (R >= 2)
  int bat_R = 0;      // rows the batched buffers hold
  bool batch = true;  // R >= 2 on the grouped matrix-core path (ne_moe_configure "staged": the staged kernels)
  uint64_t *trace = nullptr;  // ne_moe_configure "trace": per-wave wall-clock stamps of the fused step
  bool fused = true;  // one persistent launch per step (ne_moe_configure "staged": four launches)
  int last_R = 0;
  float *last_y = nullptr;
  ~ne_moe() {
    for (void *p : std::initializer_list<void *>{experts, shared, q8, q8bf, q8gu, q8o, router, logits, sgv, guo, dn, route,
                                                 sync, trace, hprep, plan, part, fsync})
      dev_free(p);
    free_batch();
  }
  int nslot() const { return topk + has_shared; }
  void free_batch() {
    for (void *p : std::initializer_list<void *>{bat.bk, bat.chunks, bat.rows, bat.xh, bat.hh, bat.dnw}) dev_free(p);
    bat = MoeBatchBufs();
    bat_R = 0;
  }
  bool batch_ok(int R) const {
    return batch && R >= 2 && moe_batch_supported(K, has_shared ? Ks : K, hid, inter, ne, topk);
  }
  void ensure_batch(int R) {
    if (R <= bat_R || !batch_ok(R)) return;
    free_batch();
    if (moe_batch_few(R, hid, inter, K, has_shared ? Ks : K)) {
      bat.vmax_chunks = moe_batch_few_chunks(R, ne, topk, has_shared);
      few_pool(hid, inter, bat.vmax_chunks, &bat.vpart, &bat.vep);
    }
    const size_t S = (size_t)R * nslot();
    bat.max_chunks = std::max(moe_batch_max_chunks(R, ne, topk, has_shared), bat.vmax_chunks);
    bat.bk = dev_alloc<uint32_t>(3 * (size_t)(ne + 1) + 2);
    IJ_HIP(hipMemset(bat.bk, 0, sizeof(uint32_t) * (3 * (size_t)(ne + 1) + 2)));  // bat_hist adds into the counts
    bat.chunks = dev_alloc<uint32_t>(3 * (size_t)bat.max_chunks);
    bat.rows = dev_alloc<uint32_t>(S);
    bat.xh = dev_alloc<uint16_t>(S * 2 * hid);
    bat.hh = dev_alloc<uint16_t>(S * inter);
    bat.dnw = dev_alloc<float>(S * hid);
    bat_R = R;
  }
  size_t logit_floats(int R) const {
    return std::max<size_t>((size_t)R * (ne + 1), (size_t)kLogitReplicas * moe_logit_stride(ne));
  }
  void ensure_scratch(int R) {
    if (R <= Rcap) return;
    for (void *p : std::initializer_list<void *>{logits, sgv, guo, dn, route, sync, hprep, q8gu, q8o}) dev_free(p);
    q8gu = q8o = nullptr;
    const size_t S = (size_t)R * nslot();
    if (q8) {
      q8gu = dev_alloc<float>((size_t)R * 2 * inter);
      q8o = dev_alloc<float>((size_t)R * hid);
    }
    logits = dev_alloc<float>(logit_floats(R));
    IJ_HIP(hipMemset(logits, 0, sizeof(float) * logit_floats(R)));  // the fused kernel's launch tags start at 1
    sgv = dev_alloc<float>(R);
    guo = dev_alloc<float>(S * 2 * ksplit * inter);
    dn = dev_alloc<float>(S * hid);
    hprep = dev_alloc<uint16_t>(S * inter);
    if (!plan && fused && moe_fused_supported(K, has_shared ? Ks : K, 1, hid, inter, ne, topk, q8 != nullptr)) {
      const MoePlan pl = moe_fused_plan(hid, inter, topk, nslot(), moe_fused_grid(), q8 != nullptr,
                                        moe_fused_slots(K, has_shared ? Ks : K, hid, inter));
      if (pl.ok) {
        plan = dev_alloc<uint32_t>(pl.words.size());
        IJ_HIP(hipMemcpy(plan, pl.words.data(), pl.words.size() * 4, hipMemcpyHostToDevice));
        part = dev_alloc<float>(pl.part_floats);
        part_floats = pl.part_floats;
        IJ_HIP(hipMemset(part, 0, sizeof(float) * pl.part_floats));  // tagged partials: tag 0 is never a launch's
        fsync = dev_alloc<uint32_t>(moe_fused_sync_words(nslot(), hid, inter));
        IJ_HIP(hipMemset(fsync, 0, 4 * moe_fused_sync_words(nslot(), hid, inter)));
        plan_grid = pl.grid;
        plan_slots = pl.slots;
      }
    }
    route = dev_alloc<uint32_t>((size_t)R * 2 * topk);
    IJ_HIP(hipMemset(route, 0, sizeof(uint32_t) * R * 2 * topk));
    sync = dev_alloc<uint32_t>(sync_words(R, nslot(), hid, inter));
    IJ_HIP(hipMemset(sync, 0, 4 * sync_words(R, nslot(), hid, inter)));
    Rcap = R;
    ensure_batch(R);
  }
  MoeArgs args(int R, const float *x, float *y) const {
    MoeArgs a;
    a.x = x;
    a.y = y;
    a.R = R;
    a.hid = hid;
    a.inter = inter;
    a.ne = ne;
    a.topk = topk;
    a.nslot = nslot();
    a.router = router;
    a.has_sgate = has_sgate;
    a.experts = experts;
    a.shared = shared;
    a.lay = lay;
    a.slay = slay;
    a.had_hid = had_size(hid);
    a.had_inter = had_size(inter);
    a.sc_hid = had_scale(a.had_hid);
    a.sc_inter = had_scale(a.had_inter);
    a.ksplit = ksplit;
    a.logits = logits;
    a.route = route;
    a.sgv = sgv;
    a.guo = guo;
    a.dn = dn;
    a.sync = sync;
    a.trace = trace;
    a.hprep = hprep;
    a.units = plan;
    a.part = part;
    a.fsync = fsync;
    a.fused_slots = plan_slots;
    a.q8 = q8;
    a.q8bf = q8bf;
    a.q8gu = q8gu;
    a.q8o = q8o;
    return a;
  }
  // a failed cross-workgroup wait leaves the error word set: report it and clear the counters
  void check_sync(hipStream_t s) {
    uint32_t err = 0;
    IJ_HIP(hipMemcpyAsync(&err, sync + kSyncErrWord, 4, hipMemcpyDeviceToHost, s));
    IJ_HIP(hipStreamSynchronize(s));
    if (err) {
      IJ_HIP(hipMemsetAsync(sync, 0, 4 * sync_words(Rcap, nslot(), hid, inter), s));
      IJ_HIP(hipMemsetAsync(logits, 0, sizeof(float) * logit_floats(Rcap), s));  // launch tags restart with the epoch
      if (fsync) IJ_HIP(hipMemsetAsync(fsync, 0, 4 * moe_fused_sync_words(nslot(), hid, inter), s));
      if (part) IJ_HIP(hipMemsetAsync(part, 0, sizeof(float) * part_floats, s));  // the epoch restarts: no stale tags
      IJ_HIP(hipStreamSynchronize(s));
      throw Error("moe: a cross-workgroup wait timed out (layer output invalid)");
    }
  }
  bool fused_ok(int R) const { return fused && plan_grid > 0 && R == 1; }
  // hc: the hyper-connection write's fields (MoeArgs::hc ...), or null for the plain layer
  void launch(int R, const float *x, float *y, hipStream_t s, const MoeArgs *hc = nullptr) const {
    MoeArgs a = args(R, x, y);
    if (hc) {
      a.hc = hc->hc;
      a.refr = hc->refr;
      a.hc_h = hc->hc_h;
      a.hc_inj = hc->hc_inj;
      a.hc_out = hc->hc_out;
    }
    if (batch_ok(R) && R <= bat_R) {
      MoeBatchBufs b = bat;
      if (b.vpart) {  // the shape's pool may have grown (for another layer) since this layer took its arrays
        int pc = 0;
        few_pool_now(hid, inter, &b.vpart, &b.vep, &pc);
        IJ_CHECK(pc >= b.vmax_chunks, "MoE: few-row pool smaller than the layer's need");
        b.vmax_chunks = pc;
      }
      if (q8) launch_moe_q8(a, s);  // independent of the route; the batch's combine reads its output
      launch_moe_batch(a, b, s);
      return;
    }
    if (fused_ok(R)) {
      launch_moe_fused(a, plan_grid, s);
      return;
    }
    launch_moe_router(a, s);
    if (q8) launch_moe_q8(a, s);
    launch_moe_gateup(a, s);
    launch_moe_down(a, s);
    launch_moe_combine(a, s);
  }
};

namespace {

void moe_check_dims(int hid, int inter, int ne, int topk) {
  IJ_CHECK(hid % 128 == 0 && inter % 32 == 0, "MoE hid %d must be a multiple of 128, inter %d of 32", hid, inter);
  IJ_CHECK(hid % 8 == 0 && hid / 2 <= 4096 && inter <= 4096, "MoE dims too large for one workgroup's LDS");
  IJ_CHECK(ne >= 1 && ne <= 1024 && topk >= 1 && topk <= 32 && topk <= ne, "MoE ne %d / topk %d out of range", ne,
           topk);
  had_size(hid);
  had_size(inter);
}

// one expert's (or the shared expert's) block in the re-laid layout, built on the host
void build_block(const ExpertLayout &L, int hid, int inter, const uint16_t *tr[3], const uint16_t *su[3],
                 const uint16_t *sv[3], uint8_t *dst) {
  memset(dst, 0, L.bytes);
  const int dims[3][2] = {{hid, inter}, {hid, inter}, {inter, hid}};
  for (int p = 0; p < 3; p++) {
    relay_tiles(tr[p], dims[p][0] / 16, dims[p][1] / 16, L.K, dst + L.tr[p]);
    memcpy(dst + L.su[p], su[p], 2u * dims[p][0]);
    memcpy(dst + L.sv[p], sv[p], 2u * dims[p][1]);
  }
}

ne_moe *moe_create(const ne_moe_desc &d) {
  moe_check_dims(d.hid, d.inter, d.ne, d.topk);
  IJ_CHECK(d.K >= 2 && d.K <= 8, "routed K %d (2..8)", d.K);
  IJ_CHECK(d.router && d.gt && d.ut && d.dt && d.gsu && d.gsv && d.usu && d.usv && d.dsu && d.dsv,
           "missing routed expert or router arrays");
  const bool sh = d.sgt != nullptr, q8 = d.qgw != nullptr;
  IJ_CHECK(!sh || (d.sut && d.sdt && d.sgsu && d.sgsv && d.susu && d.susv && d.sdsu && d.sdsv),
           "shared expert arrays incomplete");
  IJ_CHECK(!(sh && q8), "two shared experts (EXL3 and 8-bit): give one");
  IJ_CHECK(!q8 || (d.quw && d.qdw && d.qgs && d.qgb && d.qus && d.qub && d.qds && d.qdb),
           "8-bit shared expert arrays incomplete");
  IJ_CHECK(!q8 || d.qgroup == kQ8Group, "8-bit shared expert: group %d (the MoE layer takes %d, as the reference's "
           "fn_moe kernels)", d.qgroup, kQ8Group);
  IJ_CHECK(!q8 || moe_q8_supported(d.hid, d.inter), "8-bit shared expert: %d x %d not supported", d.hid, d.inter);
  IJ_CHECK(!sh || (d.Ks >= 2 && d.Ks <= 8), "shared K %d (2..8)", d.Ks);
  ensure_device();
  auto m = std::make_unique<ne_moe>();
  m->hid = d.hid;
  m->inter = d.inter;
  m->ne = d.ne;
  m->topk = d.topk;
  m->K = d.K;
  m->Ks = sh ? d.Ks : 0;
  m->has_shared = sh;
  m->has_sgate = d.sgate != nullptr;
  m->lay = expert_layout(d.hid, d.inter, d.K);
  const size_t tsz[3] = {(size_t)d.hid * d.inter * d.K / 16, (size_t)d.hid * d.inter * d.K / 16,
                         (size_t)d.inter * d.hid * d.K / 16};
  m->experts = dev_alloc<uint8_t>((size_t)d.ne * m->lay.bytes);
  const int chunk = 16;
  std::vector<uint8_t> host((size_t)chunk * m->lay.bytes);
  for (int e0 = 0; e0 < d.ne; e0 += chunk) {
    const int n = std::min(chunk, d.ne - e0);
    for (int i = 0; i < n; i++) {
      const size_t e = (size_t)(e0 + i);
      const uint16_t *tr[3] = {d.gt + e * tsz[0], d.ut + e * tsz[1], d.dt + e * tsz[2]};
      const uint16_t *su[3] = {d.gsu + e * d.hid, d.usu + e * d.hid, d.dsu + e * d.inter};
      const uint16_t *sv[3] = {d.gsv + e * d.inter, d.usv + e * d.inter, d.dsv + e * d.hid};
      build_block(m->lay, d.hid, d.inter, tr, su, sv, host.data() + (size_t)i * m->lay.bytes);
    }
    IJ_HIP(hipMemcpy(m->experts + (size_t)e0 * m->lay.bytes, host.data(), (size_t)n * m->lay.bytes,
                     hipMemcpyHostToDevice));
  }
  if (sh) {
    m->slay = expert_layout(d.hid, d.inter, d.Ks);
    std::vector<uint8_t> sb(m->slay.bytes);
    const uint16_t *tr[3] = {d.sgt, d.sut, d.sdt};
    const uint16_t *su[3] = {d.sgsu, d.susu, d.sdsu};
    const uint16_t *sv[3] = {d.sgsv, d.susv, d.sdsv};
    build_block(m->slay, d.hid, d.inter, tr, su, sv, sb.data());
    m->shared = dev_alloc<uint8_t>(m->slay.bytes);
    IJ_HIP(hipMemcpy(m->shared, sb.data(), sb.size(), hipMemcpyHostToDevice));
  }
  if (q8) {  // weight bytes as stored; each group's bf16 scale and bias joined into one word
    const Q8Off o = q8_offsets(d.hid, d.inter);
    std::vector<uint8_t> qb(q8_block_bytes(d.hid, d.inter));
    const uint32_t *w[3] = {d.qgw, d.quw, d.qdw};
    const uint16_t *sc[3] = {d.qgs, d.qus, d.qds}, *bi[3] = {d.qgb, d.qub, d.qdb};
    const int rows[3] = {d.inter, d.inter, d.hid}, in[3] = {d.hid, d.hid, d.inter};
    for (int p = 0; p < 3; p++) {
      memcpy(qb.data() + o.w[p], w[p], (size_t)rows[p] * in[p]);
      uint32_t *sb = (uint32_t *)(qb.data() + o.sb[p]);
      for (size_t i = 0; i < (size_t)rows[p] * (in[p] / kQ8Group); i++) sb[i] = sc[p][i] | (uint32_t)bi[p][i] << 16;
    }
    m->q8 = dev_alloc<uint8_t>(qb.size());
    IJ_HIP(hipMemcpy(m->q8, qb.data(), qb.size(), hipMemcpyHostToDevice));
    m->q8bf = dev_alloc<uint16_t>(3ull * d.hid * d.inter);
    launch_q8_bf16(m->q8, m->q8bf, d.hid, d.inter, stream());
    IJ_HIP(hipStreamSynchronize(stream()));
  }
  const size_t rrows = (size_t)d.ne + m->has_sgate;
  m->router = dev_alloc<uint16_t>(rrows * d.hid);
  IJ_HIP(hipMemcpy(m->router, d.router, 2u * d.ne * d.hid, hipMemcpyHostToDevice));
  if (m->has_sgate) IJ_HIP(hipMemcpy(m->router + (size_t)d.ne * d.hid, d.sgate, 2u * d.hid, hipMemcpyHostToDevice));
  IJ_CHECK((d.hid / 16) % m->ksplit == 0 && ((d.hid / 16) / m->ksplit) % 8 == 0, "ksplit %d does not divide hid %d",
           m->ksplit, d.hid);
  m->ensure_scratch(1);
  return m.release();
}

}  // namespace

extern "C" {

NE_API ne_moe *ne_moe_create(const ne_moe_desc *d) {
  ne_moe *r = nullptr;
  c_call([&] {
    IJ_CHECK(d, "null descriptor");
    r = moe_create(*d);
  });
  return r;
}

NE_API ne_moe *ne_moe_load(const ne_pack *p, const char *prefix, int topk) {
  ne_moe *r = nullptr;
  c_call([&] {
    IJ_CHECK(p && prefix, "null argument");
    const Pack &P = *p->pack;
    const std::string mp = prefix;
    const TensorInfo &rw = P.need(mp + "gate.weight", NE_BF16, {-1, -1});
    ne_moe_desc d;
    memset(&d, 0, sizeof d);
    d.ne = (int)rw.shape[0];
    d.hid = (int)rw.shape[1];
    d.topk = topk;
    d.router = (const uint16_t *)rw.host;
    if (P.has(mp + "shared_expert_gate.weight"))
      d.sgate = (const uint16_t *)P.need(mp + "shared_expert_gate.weight", NE_BF16, {}).host;
    const TensorInfo &gt = P.need(mp + "switch_mlp.gate_proj.trellis", NE_U16, {d.ne, d.hid / 16, -1, -1});
    d.inter = (int)gt.shape[2] * 16;
    IJ_CHECK(gt.shape[3] % 16 == 0, "switch_mlp.gate_proj.trellis: last dim not 16 K");
    d.K = (int)gt.shape[3] / 16;
    const int64_t tl = 16 * d.K;
    auto T = [&](const char *n, std::initializer_list<int64_t> s) {
      return (const uint16_t *)P.need(mp + n, -1, s).host;
    };
    d.gt = (const uint16_t *)gt.host;
    d.ut = T("switch_mlp.up_proj.trellis", {d.ne, d.hid / 16, d.inter / 16, tl});
    d.dt = T("switch_mlp.down_proj.trellis", {d.ne, d.inter / 16, d.hid / 16, tl});
    d.gsu = T("switch_mlp.gate_proj.suh", {d.ne, d.hid});
    d.gsv = T("switch_mlp.gate_proj.svh", {d.ne, d.inter});
    d.usu = T("switch_mlp.up_proj.suh", {d.ne, d.hid});
    d.usv = T("switch_mlp.up_proj.svh", {d.ne, d.inter});
    d.dsu = T("switch_mlp.down_proj.suh", {d.ne, d.inter});
    d.dsv = T("switch_mlp.down_proj.svh", {d.ne, d.hid});
    for (const char *n : {"gate_proj", "up_proj", "down_proj"})
      for (const char *s : {"suh", "svh"})
        IJ_CHECK(P.need(mp + "switch_mlp." + n + "." + s, -1, {}).dtype == NE_F16, "%s: suh/svh must be F16", n);
    const bool sh_exl3 = P.has(mp + "shared_expert.gate_proj.trellis"),
               sh_q8 = P.has(mp + "shared_expert.gate_proj.weight");
    if (!sh_exl3 && !sh_q8) {  // nothing else may be there: a shared expert in another form is refused, not dropped
      for (const std::string &n : P.names())
        IJ_CHECK(n.compare(0, mp.size() + 14, mp + "shared_expert.") != 0,
                 "%s: shared expert in a form this layer does not take (EXL3 .trellis or 8-bit .weight/.scales/"
                 ".biases)", n.c_str());
      IJ_CHECK(!d.sgate, "%sshared_expert_gate.weight without a shared expert", mp.c_str());
    }
    if (sh_q8) {  // the reference's 8-bit affine shared expert (layer.mm:39-61 q8, :186-193)
      const int rows[3] = {d.inter, d.inter, d.hid}, in[3] = {d.hid, d.hid, d.inter};
      const char *nm[3] = {"shared_expert.gate_proj", "shared_expert.up_proj", "shared_expert.down_proj"};
      const uint32_t **w[3] = {&d.qgw, &d.quw, &d.qdw};
      const uint16_t **sc[3] = {&d.qgs, &d.qus, &d.qds}, **bi[3] = {&d.qgb, &d.qub, &d.qdb};
      for (int p = 0; p < 3; p++) {
        const std::string b = mp + nm[p];
        *w[p] = (const uint32_t *)P.need(b + ".weight", NE_U32, {rows[p], in[p] / 4}).host;
        const TensorInfo &s = P.need(b + ".scales", NE_BF16, {rows[p], -1});
        IJ_CHECK(s.shape[1] > 0 && in[p] % s.shape[1] == 0, "%s.scales: shape [%lld, %lld]", b.c_str(),
                 (long long)s.shape[0], (long long)s.shape[1]);
        const int g = in[p] / (int)s.shape[1];
        IJ_CHECK(g == kQ8Group, "%s: group %d; the MoE layer's 8-bit shared expert takes g%d (reference "
                 "layer.mm:191-192)", b.c_str(), g, kQ8Group);
        *sc[p] = (const uint16_t *)s.host;
        *bi[p] = (const uint16_t *)P.need(b + ".biases", NE_BF16, {rows[p], s.shape[1]}).host;
      }
      d.qgroup = kQ8Group;
    } else if (sh_exl3) {
      const TensorInfo &sg = P.need(mp + "shared_expert.gate_proj.trellis", NE_U16, {d.hid / 16, d.inter / 16, -1});
      d.Ks = (int)sg.shape[2] / 16;
      const int64_t ts = 16 * d.Ks;
      d.sgt = (const uint16_t *)sg.host;
      d.sut = T("shared_expert.up_proj.trellis", {d.hid / 16, d.inter / 16, ts});
      d.sdt = T("shared_expert.down_proj.trellis", {d.inter / 16, d.hid / 16, ts});
      d.sgsu = T("shared_expert.gate_proj.suh", {d.hid});
      d.sgsv = T("shared_expert.gate_proj.svh", {d.inter});
      d.susu = T("shared_expert.up_proj.suh", {d.hid});
      d.susv = T("shared_expert.up_proj.svh", {d.inter});
      d.sdsu = T("shared_expert.down_proj.suh", {d.inter});
      d.sdsv = T("shared_expert.down_proj.svh", {d.hid});
    }
    r = moe_create(d);
  });
  return r;
}

NE_API ne_moe *ne_moe_synth(int hid, int inter, int ne, int topk, int K, int has_shared, int Ks, uint64_t seed) {
  ne_moe *r = nullptr;
  c_call([&] {
    moe_check_dims(hid, inter, ne, topk);
    IJ_CHECK(K >= 2 && K <= 8 && (!has_shared || (Ks >= 2 && Ks <= 8)), "K out of range");
    ensure_device();
    auto m = std::make_unique<ne_moe>();
    m->hid = hid;
    m->inter = inter;
    m->ne = ne;
    m->topk = topk;
    m->K = K;
    IJ_CHECK(has_shared >= 0 && has_shared <= 2, "has_shared %d (0 none, 1 EXL3, 2 8-bit)", has_shared);
    IJ_CHECK(has_shared != 2 || moe_q8_supported(hid, inter), "8-bit shared expert: %d x %d not supported", hid,
             inter);
    m->Ks = has_shared == 1 ? Ks : 0;
    m->has_shared = has_shared == 1;
    m->lay = expert_layout(hid, inter, K);
    hipStream_t s = stream();
    m->experts = dev_alloc<uint8_t>((size_t)ne * m->lay.bytes);
    launch_fill_u32((uint32_t *)m->experts, (size_t)ne * m->lay.bytes / 4, seed * 7 + 1, s);
    auto scales = [&](uint8_t *blk, const ExpertLayout &L, uint64_t sd) {
      const int dims[3][2] = {{hid, inter}, {hid, inter}, {inter, hid}};
      for (int p = 0; p < 3; p++) {
        launch_fill_scale_f16((uint16_t *)(blk + L.su[p]), dims[p][0], sd * 131 + 2 * p, s);
        launch_fill_scale_f16((uint16_t *)(blk + L.sv[p]), dims[p][1], sd * 131 + 2 * p + 1, s);
      }
    };
    for (int e = 0; e < ne; e++) scales(m->experts + (size_t)e * m->lay.bytes, m->lay, seed * 100003 + e);
    if (has_shared == 2) {
      const Q8Off o = q8_offsets(hid, inter);
      m->q8 = dev_alloc<uint8_t>(q8_block_bytes(hid, inter));
      launch_fill_u32((uint32_t *)m->q8, o.sb[0] / 4, seed * 7 + 3, s);
      const int in[3] = {hid, hid, inter};
      for (int p = 0; p < 3; p++)
        launch_fill_q8_sb((uint32_t *)(m->q8 + o.sb[p]), (uint64_t)inter * hid / kQ8Group, in[p], seed * 13 + p, s);
      m->q8bf = dev_alloc<uint16_t>(3ull * hid * inter);
      launch_q8_bf16(m->q8, m->q8bf, hid, inter, s);
    }
    if (has_shared == 1) {
      m->slay = expert_layout(hid, inter, Ks);
      m->shared = dev_alloc<uint8_t>(m->slay.bytes);
      launch_fill_u32((uint32_t *)m->shared, m->slay.bytes / 4, seed * 7 + 3, s);
      scales(m->shared, m->slay, seed * 100003 + 999983);
    }
    m->router = dev_alloc<uint16_t>((size_t)ne * hid);
    launch_fill_normal_bf16(m->router, (size_t)ne * hid, seed * 7 + 5, (float)(1.0 / std::sqrt((double)hid)), s);
    IJ_CHECK((hid / 16) % m->ksplit == 0 && ((hid / 16) / m->ksplit) % 8 == 0, "ksplit %d does not divide hid %d",
             m->ksplit, hid);
    m->ensure_scratch(1);
    IJ_HIP(hipStreamSynchronize(s));
    r = m.release();
  });
  return r;
}

NE_API void ne_moe_free(ne_moe *m) {
  if (m) {
    (void)hipStreamSynchronize(stream());
    delete m;
  }
}

NE_API int ne_moe_info(const ne_moe *m, int *hid, int *inter, int *ne, int *topk, int *K, int *slots) {
  return c_call([&] {
    IJ_CHECK(m, "null layer");
    if (hid) *hid = m->hid;
    if (inter) *inter = m->inter;
    if (ne) *ne = m->ne;
    if (topk) *topk = m->topk;
    if (K) *K = m->K;
    if (slots) *slots = m->nslot();
  });
}

NE_API int ne_moe_run(ne_moe *m, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(m && x && y, "null argument");
    IJ_CHECK(R >= 1 && R <= 4096, "rows %d (1..4096)", R);
    IJ_CHECK(x_off % 16 == 0 && y_off % 4 == 0, "x offset must be 16-byte aligned, y offset 4-byte aligned");
    IJ_CHECK(x_off + (uint64_t)R * m->hid * 4 <= x->size, "x buffer too small for [%d][%d] f32", R, m->hid);
    IJ_CHECK(y_off + (uint64_t)R * m->hid * 4 <= y->size, "y buffer too small for [%d][%d] f32", R, m->hid);
    m->ensure_scratch(R);
    const float *xp = (const float *)((const char *)ne_dev(x) + x_off);
    float *yp = (float *)((char *)ne_dev(y) + y_off);
    timed(stream(), gpu_ms, [&] { m->launch(R, xp, yp, stream()); });
    m->last_R = R;
    m->last_y = yp;
    if (gpu_ms) m->check_sync(stream());
  });
}

NE_API int ne_moe_run_hc(ne_moe *m, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                         const ne_moe_hc *hc, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(m && x && y && hc, "null argument");
    IJ_CHECK(R >= 1 && R <= 4096, "rows %d (1..4096)", R);
    IJ_CHECK(x_off % 16 == 0 && y_off % 4 == 0, "x offset must be 16-byte aligned, y offset 4-byte aligned");
    IJ_CHECK(x_off + (uint64_t)R * m->hid * 4 <= x->size, "x buffer too small for [%d][%d] f32", R, m->hid);
    IJ_CHECK(y_off + (uint64_t)R * m->hid * 4 <= y->size, "y buffer too small for [%d][%d] f32", R, m->hid);
    IJ_CHECK(hc->hc >= 1 && hc->hc <= 8, "hc %d (1..8 streams)", hc->hc);
    const uint64_t hb = (uint64_t)R * hc->hc * m->hid * 4;
    IJ_CHECK(hc->h && hc->h->size >= hb, "h missing or under %llu bytes ([R][hc][hid] f32)", (unsigned long long)hb);
    IJ_CHECK(hc->hout && hc->hout->size >= hb, "hout missing or under %llu bytes", (unsigned long long)hb);
    IJ_CHECK(hc->inj && hc->inj->size >= (uint64_t)R * 32, "inj missing or under %d bytes ([R][8] f32)", R * 32);
    m->ensure_scratch(R);
    MoeArgs f;
    f.hc = hc->hc;
    f.refr = hc->refr ? 1 : 0;
    f.hc_h = (const float *)ne_dev(hc->h);
    f.hc_inj = (const float *)ne_dev(hc->inj);
    f.hc_out = (float *)ne_dev(hc->hout);
    const float *xp = (const float *)((const char *)ne_dev(x) + x_off);
    float *yp = (float *)((char *)ne_dev(y) + y_off);
    timed(stream(), gpu_ms, [&] { m->launch(R, xp, yp, stream(), &f); });
    m->last_R = R;
    m->last_y = yp;
    if (gpu_ms) m->check_sync(stream());
  });
}

NE_API int ne_moe_read(ne_moe *m, const char *name, void *dst, uint64_t nbytes) {
  return c_call([&] {
    IJ_CHECK(m && name && (dst || nbytes == 0), "null argument");
    IJ_CHECK(m->last_R > 0, "no run yet");
    m->check_sync(stream());
    const int R = m->last_R, S = R * m->nslot();
    const std::string n = name;
    std::vector<uint8_t> out;
    auto fetch = [&](const void *src, size_t bytes) {
      out.resize(bytes);
      IJ_HIP(hipMemcpy(out.data(), src, bytes, hipMemcpyDeviceToHost));
    };
    if (n == "logits") {
      std::vector<float> all((size_t)R * (m->ne + 1));
      IJ_HIP(hipMemcpy(all.data(), m->logits, all.size() * 4, hipMemcpyDeviceToHost));
      out.resize((size_t)R * m->ne * 4);
      // the fused kernel keeps its launch tag in the low 16 bits of each (bf16-valued) logit
      for (float &v : all) v = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & 0xFFFF0000u);
      for (int r = 0; r < R; r++) memcpy(out.data() + (size_t)r * m->ne * 4, &all[(size_t)r * (m->ne + 1)], 4u * m->ne);
    } else if (n == "route") {
      fetch(m->route, (size_t)R * 2 * m->topk * 4);
    } else if (n == "shared_gate") {
      fetch(m->sgv, (size_t)R * 4);
    } else if (n == "shared_q8") {  // the 8-bit shared expert's rounded output o [R][hid]
      IJ_CHECK(m->q8, "the layer has no 8-bit shared expert");
      if (m->fused_ok(R)) {  // tagged u64 values: the f32 in the low word
        std::vector<uint64_t> t((size_t)m->hid);
        const uint64_t *src = (const uint64_t *)m->part + moe_fused_q8_index(m->hid, m->inter, m->nslot()) +
                              2 * (size_t)m->inter;
        IJ_HIP(hipMemcpy(t.data(), src, t.size() * 8, hipMemcpyDeviceToHost));
        out.resize(t.size() * 4);
        for (size_t i = 0; i < t.size(); i++) memcpy(out.data() + 4 * i, &t[i], 4);
      } else {
        fetch(m->q8o, (size_t)R * m->hid * 4);
      }
    } else if ((n == "experts_gu" || n == "experts_dn") && m->batch_ok(R)) {
      IJ_CHECK(false, "\"%s\" is not kept by the batched path (R >= 2); IJAH_MOE_PATH=staged keeps it", name);
    } else if (n == "experts_gu" && m->fused_ok(R)) {  // the fused step stores the summed inner outputs
      fetch(m->guo, (size_t)S * 2 * m->inter * 4);
    } else if (n == "experts_gu") {
      std::vector<float> g((size_t)S * 2 * m->ksplit * m->inter);
      IJ_HIP(hipMemcpy(g.data(), m->guo, g.size() * 4, hipMemcpyDeviceToHost));
      std::vector<float> o((size_t)S * 2 * m->inter, 0.f);
      for (int sp = 0; sp < S * 2; sp++)
        for (int k = 0; k < m->ksplit; k++)
          for (int j = 0; j < m->inter; j++)
            o[(size_t)sp * m->inter + j] += g[((size_t)sp * m->ksplit + k) * m->inter + j];
      out.resize(o.size() * 4);
      memcpy(out.data(), o.data(), out.size());
    } else if (n == "experts_dn") {
      fetch(m->dn, (size_t)S * m->hid * 4);
    } else if (n == "trace") {
      IJ_CHECK(m->trace, "no trace (ne_moe_configure(m, \"trace\", 1) before the run)");
      fetch(m->trace, (size_t)8 * 8 * 65536);
    } else if (n == "mlp_out") {
      fetch(m->last_y, (size_t)R * m->hid * 4);
    } else {
      throw Error(strfmt("unknown intermediate %s", name));
    }
    memcpy(dst, out.data(), std::min<uint64_t>(nbytes, out.size()));
  });
}

NE_API int ne_moe_configure(ne_moe *m, const char *key, int value) {
  return c_call([&] {
    IJ_CHECK(m && key, "null argument");
    const std::string k = key;
    IJ_HIP(hipStreamSynchronize(stream()));
    if (k == "staged") {
      m->fused = m->batch = value == 0;
    } else if (k == "trace") {
      dev_free(m->trace);
      m->trace = nullptr;
      if (value) {
        m->trace = dev_alloc<uint64_t>((size_t)8 * 65536);
        IJ_HIP(hipMemset(m->trace, 0, 8 * 8 * 65536));
      }
    } else {
      throw Error(strfmt("unknown option %s (staged, trace)", key));
    }
  });
}

NE_API int ne_exl3_lin_configure(ne_exl3_lin *l, const char *key, int value) {
  return c_call([&] {
    IJ_CHECK(l && key, "null argument");
    IJ_CHECK(std::string(key) == "staged", "unknown option %s (staged)", key);
    IJ_HIP(hipStreamSynchronize(stream()));
    l->one_launch = value == 0;
  });
}

NE_API int ne_moe_decode(ne_moe *m, int e, int proj, ne_buf *w, double *gpu_ms) {
  return c_call([&] {
    IJ_CHECK(m && w, "null argument");
    IJ_CHECK(proj >= 0 && proj <= 2, "proj %d (0 gate, 1 up, 2 down)", proj);
    IJ_CHECK(e >= 0 && (e < m->ne || (e == m->ne && m->has_shared)), "expert %d out of range", e);
    const bool sh = e == m->ne;
    const ExpertLayout &L = sh ? m->slay : m->lay;
    const uint8_t *blk = sh ? m->shared : m->experts + (size_t)e * m->lay.bytes;
    const int in = proj == 2 ? m->inter : m->hid, out = proj == 2 ? m->hid : m->inter;
    IJ_CHECK(w->size >= (uint64_t)in * out * 2, "w buffer too small");
    timed(stream(), gpu_ms, [&] {
      launch_decode((const uint32_t *)(blk + L.tr[proj]), in / 16, out / 16, L.K, (uint16_t *)ne_dev(w), stream());
    });
  });
}

NE_API int ne_moe_bytes(const ne_moe *m, int R, uint64_t *bytes) {
  return c_call([&] {
    IJ_CHECK(m && bytes, "null argument");
    IJ_CHECK(m->last_R >= R && R >= 1, "run the layer at R rows first");
    IJ_HIP(hipStreamSynchronize(stream()));
    std::vector<uint32_t> rt((size_t)R * 2 * m->topk);
    IJ_HIP(hipMemcpy(rt.data(), m->route, rt.size() * 4, hipMemcpyDeviceToHost));
    std::set<uint32_t> uniq;
    for (int r = 0; r < R; r++)
      for (int k = 0; k < m->topk; k++) uniq.insert(rt[(size_t)r * 2 * m->topk + k]);
    auto per_expert = [&](int K) {
      const uint64_t w = (uint64_t)m->hid * m->inter;
      return 3 * w * K / 8 + 2u * (uint64_t)(3 * (m->hid + m->inter));
    };
    uint64_t b = uniq.size() * per_expert(m->K);
    if (m->has_shared) b += per_expert(m->Ks);
    if (m->q8) b += q8_block_bytes(m->hid, m->inter);  // weight bytes + bf16 scales and biases
    b += 2u * (uint64_t)(m->ne + m->has_sgate) * m->hid;
    *bytes = b;
  });
}

NE_API int ne_moe_time(ne_moe *const *layers, int n, int R, const ne_buf *x, int warmup, int reps,
                       double *us_per_layer) {
  return c_call([&] {
    IJ_CHECK(layers && n >= 1 && x && us_per_layer && reps >= 1, "bad arguments");
    for (int i = 0; i < n; i++) {
      IJ_CHECK(layers[i], "null layer %d", i);
      IJ_CHECK(layers[i]->hid == layers[0]->hid, "layers differ in hid");
      layers[i]->ensure_scratch(R);
    }
    const int hid = layers[0]->hid;
    IJ_CHECK((uint64_t)R * hid * 4 <= x->size, "x buffer too small");
    hipStream_t s = stream();
    float *ys = dev_alloc<float>((size_t)n * R * hid);
    const float *xp = (const float *)ne_dev(x);
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    auto cleanup = [&] {
      if (ge) (void)hipGraphExecDestroy(ge);
      if (g) (void)hipGraphDestroy(g);
      dev_free(ys);
    };
    try {
      ge = capture_graph(s, g, [&] {
        for (int i = 0; i < n; i++) layers[i]->launch(R, xp, ys + (size_t)i * R * hid, s);
      });
      for (int i = 0; i < warmup; i++) IJ_HIP(hipGraphLaunch(ge, s));
      double ms = 0;
      timed(s, &ms, [&] {
        for (int i = 0; i < reps; i++) IJ_HIP(hipGraphLaunch(ge, s));
      });
      *us_per_layer = ms * 1000.0 / ((double)reps * n);
      for (int i = 0; i < n; i++) layers[i]->check_sync(s);
      for (int i = 0; i < n; i++) {
        layers[i]->last_R = R;
        layers[i]->last_y = nullptr;
      }
    } catch (...) {
      cleanup();
      throw;
    }
    cleanup();
  });
}

NE_API int ne_moe_time_kernels(ne_moe *const *layers, int n, int R, const ne_buf *x, int reps, char names[][16],
                               double *us, int *n_kinds) {
  return c_call([&] {
    IJ_CHECK(layers && n >= 1 && x && us && n_kinds && names && reps >= 1, "bad arguments");
    IJ_CHECK(*n_kinds >= 5, "need room for 5 kernel kinds");
    const int hid = layers[0]->hid;
    IJ_CHECK((uint64_t)R * hid * 4 <= x->size, "x buffer too small");
    hipStream_t s = stream();
    float *ys = dev_alloc<float>((size_t)n * R * hid);
    const float *xp = (const float *)ne_dev(x);
    std::vector<MoeArgs> a;
    for (int i = 0; i < n; i++) {
      layers[i]->ensure_scratch(R);
      a.push_back(layers[i]->args(R, xp, ys + (size_t)i * R * hid));
      layers[i]->launch(R, xp, ys + (size_t)i * R * hid, s);
    }
    auto fused = [](const MoeArgs &x, hipStream_t st) { launch_moe_fused(x, 0, st); };
    void (*fns[5])(const MoeArgs &, hipStream_t) = {launch_moe_router, launch_moe_gateup, launch_moe_down,
                                                    launch_moe_combine, fused};
    const char *nm[5] = {"router", "gateup", "down", "combine", "fused"};
    bool all_fused = true;
    for (int i = 0; i < n; i++) all_fused = all_fused && layers[i]->fused_ok(R);
    const int kinds = all_fused ? 5 : 4;
    try {
      for (int k = 0; k < kinds; k++) {
        double ms = 0;
        timed(s, &ms, [&] {
          for (int r = 0; r < reps; r++)
            for (int i = 0; i < n; i++) fns[k](a[i], s);
        });
        snprintf(names[k], 16, "%s", nm[k]);
        us[k] = ms * 1000.0 / ((double)reps * n);
      }
    } catch (...) {
      dev_free(ys);
      throw;
    }
    IJ_HIP(hipStreamSynchronize(s));
    dev_free(ys);
    for (int i = 0; i < n; i++) layers[i]->check_sync(s);
    *n_kinds = kinds;
  });
}

}  // extern "C"
