/* CPU oracle for the EXL3 trellis decode + MoE / trunk linear path (test infrastructure only; see the header).
 *
 * Citations are file:line in the reference tree (publicExcess/ijah). The reference's own CPU decoder
 * (tools/opref.py:142-160 -> exl3_codec.decode_inner) lives in an external module that is not in the reference tree
 * (tools/refenv.py:5-7, tools/convert_trunk_enc.py:27-41), so the bit layout here is restated from the reference's
 * Metal readers, which the reference reports agree with that codec to rel 2.3e-7 on 342 real matrices
 * (docs/trunk6.md:74-84).
 */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ formats */
uint16_t orc_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t ax = u & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to infinity */
  if (ax < 0x38800000u) {                                  /* below 2^-14: binary16 subnormal, unit 2^-24 */
    float a;
    memcpy(&a, &ax, 4);
    return (uint16_t)(sign | (uint32_t)lrintf(a * 16777216.0f)); /* exact scaling, RNE (default mode) */
  }
  uint32_t m = ax + 0xFFFu + ((ax >> 13) & 1u); /* RNE on the 13 dropped bits */
  m -= (uint32_t)(127 - 15) << 23;
  return (uint16_t)(sign | (m >> 13));
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t u;
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f);
    memcpy(&u, &v, 4);
    u |= sign;
  } else if (e == 31) {
    u = sign | 0x7F800000u | (m << 13);
  } else {
    u = sign | ((e + 112u) << 23) | (m << 13);
  }
  float r;
  memcpy(&r, &u, 4);
  return r;
}

float orc_bf16r(float x) { /* kernels/ne_common.h:23-26 */
  uint32_t u;
  memcpy(&u, &x, 4);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

float orc_bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* ------------------------------------------------------------------------------------------------ codebook */
/* kernels/ne_common.h:139-144 (twin kernels/prefill/pf_moe.metal:164-169): cw &= 0x7FFF;
 * r = (cw * 0xCBAC1FED) & 0x8FFF8FFF ^ 0x3B603B60; value = fp16(fp16(r_lo) + fp16(r_hi)).
 * Both halves lie in +-[2^-3, 2^1), so their f32 sum is exact and one RNE to fp16 equals the half + half. */
uint16_t orc_mcg(uint32_t cw) {
  const uint32_t r = (((cw & 0x7FFFu) * 0xCBAC1FEDu) & 0x8FFF8FFFu) ^ 0x3B603B60u;
  const float a = orc_f16_to_f32((uint16_t)(r & 0xFFFFu));
  const float b = orc_f16_to_f32((uint16_t)(r >> 16));
  return orc_f32_to_f16(a + b);
}

/* slot s = 8 l + j, l = lane 0..31, q = l & 3, c = l >> 2: j 0..3 -> rows (2q, 2q+1, 2q+8, 2q+9)[j] at col c,
 * j 4..7 -> the same rows at col c + 8 (kernels/ne_common.h:105-108; kernels/trunk6/trunk6.metal:611-629). */
void orc_slot_rc(int s, int *row, int *col) {
  const int l = s >> 3, j = s & 7, q = l & 3, c = l >> 2;
  static const int rsel[4] = {0, 1, 8, 9};
  *row = 2 * q + rsel[j & 3];
  *col = c + 8 * (j >> 2);
}

/* the pack's u16 halfwords read as little-endian u32 words (kernels/ne_common.h:106-107) */
static uint32_t tile_word(const uint16_t *tile, int w) {
  return (uint32_t)tile[2 * w] | ((uint32_t)tile[2 * w + 1] << 16);
}
/* ring bit p: bit 31 - (p & 31) of word p >> 5 (MSB first; kernels/trunk6/trunk6.metal:116) */
static int ring_bit(const uint16_t *tile, int K, long p) {
  const long tot = 256L * K;
  p %= tot;
  if (p < 0) p += tot;
  return (int)((tile_word(tile, (int)(p >> 5)) >> (31 - (p & 31))) & 1u);
}

/* The definition: the codeword of slot i is the 16 ring bits that END at bit (i+1) K (mod 256 K), first bit most
 * significant (kernels/ne_common.h:110-138: window start 8K lane + 256K + K - 16, codeword j at OFF + 16 + jK). */
void orc_tile_cw_ring(const uint16_t *tile, int K, uint16_t cw[256]) {
  for (int i = 0; i < 256; i++) {
    const long end = (long)(i + 1) * K;
    uint32_t v = 0;
    for (long p = end - 16; p < end; p++) v = (v << 1) | (uint32_t)ring_bit(tile, K, p);
    cw[i] = (uint16_t)v;
  }
}

static uint32_t cw_at(uint32_t vx, uint32_t vy, uint32_t E) { /* kernels/ne_common.h:133-138 */
  const uint32_t c = 64u - E;
  if (c >= 32u) return (vx >> (c - 32u)) & 0xFFFFu;
  if (c <= 16u) return (vy >> c) & 0xFFFFu;
  return ((vx << (32u - c)) | (vy >> c)) & 0xFFFFu;
}

/* kernels/ne_common.h:109-157: lane_load<K>, lane_funnel<K>, win_off<K>, dec8<K> codeword positions */
int orc_tile_cw_lane(const uint16_t *tile, int K, uint16_t cw[256]) {
  if (K < 4 || K > 6) return -1;
  const uint32_t NW = 8u * (uint32_t)K, TOT = 256u * (uint32_t)K, S0 = TOT + (uint32_t)K - 16u;
  const int aligned = (8 * K) % 32 == 0;
  const uint32_t OFF = aligned ? ((256u * (uint32_t)K + (uint32_t)K - 16u) & 31u) : 0u;
  for (uint32_t lane = 0; lane < 32u; lane++) {
    uint32_t s = 8u * (uint32_t)K * lane + S0;
    s = (s >= TOT) ? s - TOT : s;
    const uint32_t i0 = s >> 5u;
    const uint32_t i1 = (i0 + 1u >= NW) ? i0 + 1u - NW : i0 + 1u;
    const uint32_t i2 = (i1 + 1u >= NW) ? i1 + 1u - NW : i1 + 1u;
    const uint32_t wx = tile_word(tile, (int)i0), wy = tile_word(tile, (int)i1);
    const uint32_t wz = aligned ? 0u : tile_word(tile, (int)i2);
    uint32_t vx = wx, vy = wy;
    if (!aligned) {
      const uint32_t a = (8u * (uint32_t)K * lane + TOT + (uint32_t)K - 16u) & 31u;
      vx = (wx << a) | ((wy >> 1u) >> (31u - a));
      vy = (wy << a) | ((wz >> 1u) >> (31u - a));
    }
    for (uint32_t j = 0; j < 8u; j++) cw[8u * lane + j] = (uint16_t)cw_at(vx, vy, OFF + 16u + j * (uint32_t)K);
  }
  return 0;
}

/* kernels/trunk6/trunk6.metal:91-127: t6_lane, t6_load, t6_dec (window 15 + 7K bits; K8 lane-independent) */
int orc_tile_cw_t6(const uint16_t *tile, int K, uint16_t cw[256]) {
  if (K < 1 || K > 8) return -1;
  const uint32_t NW = 8u * (uint32_t)K, TOT = 256u * (uint32_t)K;
  for (uint32_t ln = 0; ln < 32u; ln++) {
    uint32_t s = (8u * ln + 1u) * (uint32_t)K + TOT - 15u;
    s = s >= TOT ? s - TOT : s;
    const uint32_t i0 = s >> 5u;
    const uint32_t i1 = i0 + 1u >= NW ? i0 + 1u - NW : i0 + 1u;
    const uint32_t i2 = i1 + 1u >= NW ? i1 + 1u - NW : i1 + 1u;
    const uint32_t a = s & 31u;
    const uint32_t wx = tile_word(tile, (int)i0), wy = tile_word(tile, (int)i1), wz = tile_word(tile, (int)i2);
    for (uint32_t j = 0; j < 8u; j++) {
      uint32_t c;
      if (K == 8) {
        const uint32_t E = 40u + 8u * j;
        c = E <= 64u ? cw_at(wx, wy, E) : cw_at(wy, wz, E - 32u);
      } else {
        const uint32_t vx = (wx << a) | ((wy >> 1u) >> (31u - a));
        const uint32_t vy = (wy << a) | ((wz >> 1u) >> (31u - a));
        c = cw_at(vx, vy, j * (uint32_t)K + 15u);
      }
      cw[8u * ln + j] = (uint16_t)c;
    }
  }
  return 0;
}

/* W'[16 tk + r][16 tn + c] = mcg(codeword of the slot at (r, c)); tile (tk, tn) at halfword offset
 * (tk * out/16 + tn) * 16K (kernels/trunk6/trunk6.h:30, tools/convert_trunk_enc.py:12) */
void orc_decode(const uint16_t *trellis, int in, int out, int K, uint16_t *w) {
  const int IT = in / 16, OT = out / 16;
  for (int tk = 0; tk < IT; tk++)
    for (int tn = 0; tn < OT; tn++) {
      const uint16_t *tile = trellis + ((size_t)tk * OT + tn) * 16 * K;
      uint16_t cw[256];
      orc_tile_cw_ring(tile, K, cw);
      for (int s = 0; s < 256; s++) {
        int r, c;
        orc_slot_rc(s, &r, &c);
        w[(size_t)(16 * tk + r) * out + 16 * tn + c] = orc_mcg(cw[s]);
      }
    }
}

/* ------------------------------------------------------------------------------------------------ Hadamard */
int orc_had_size(int d) { /* tools/convert_trunk_enc.py:59-63 */
  const int ns[4] = {128, 64, 32, 16};
  for (int i = 0; i < 4; i++)
    if (d % ns[i] == 0) return ns[i];
  return -1;
}
float orc_had_scale(int n) { return (float)(1.0 / sqrt((double)n)); }

/* Sylvester butterflies over index bits 0, 1, ..., lo + hi and lo - hi, in f32, then one multiply by f32(1/sqrt n):
 * the element order of kernels/ne_common.h:93-103 (lane bits 0..4, then registers: bit 5, bit 6) and
 * tests/trunk6/check_kernels.py:47-60. */
void orc_fwht_f32(float *v, int n, int had) {
  const float sc = orc_had_scale(had);
  for (int b0 = 0; b0 < n; b0 += had) {
    float *x = v + b0;
    for (int bit = 1; bit < had; bit <<= 1)
      for (int i = 0; i < had; i++)
        if (!(i & bit)) {
          const float lo = x[i], hi = x[i + bit];
          x[i] = lo + hi;
          x[i + bit] = lo - hi;
        }
    for (int i = 0; i < had; i++) x[i] *= sc;
  }
}
void orc_fwht_f64(double *v, int n, int had) {
  const double sc = 1.0 / sqrt((double)had);
  for (int b0 = 0; b0 < n; b0 += had) {
    double *x = v + b0;
    for (int bit = 1; bit < had; bit <<= 1)
      for (int i = 0; i < had; i++)
        if (!(i & bit)) {
          const double lo = x[i], hi = x[i + bit];
          x[i] = lo + hi;
          x[i + bit] = lo - hi;
        }
    for (int i = 0; i < had; i++) x[i] *= sc;
  }
}

/* ------------------------------------------------------------------------------------------------ linear */
/* prepared input: f32 x * suh, f32 FWHT, rounded to fp16 (kernels/trunk6/trunk6.metal:68-85) */
static void prep_in(const float *x, const uint16_t *suh, int in, float *xh) {
  const int had = orc_had_size(in);
  for (int i = 0; i < in; i++) xh[i] = x[i] * orc_f16_to_f32(suh[i]);
  orc_fwht_f32(xh, in, had);
  for (int i = 0; i < in; i++) xh[i] = orc_f16_to_f32(orc_f32_to_f16(xh[i]));
}

/* o[out] = xh[in] @ W' (W' fp16 bits [in][out]) accumulated in f64 */
static void inner_gemv(const float *xh, const uint16_t *w, int in, int out, double *o) {
  for (int j = 0; j < out; j++) o[j] = 0.0;
  for (int i = 0; i < in; i++) {
    const double xv = xh[i];
    if (xv == 0.0) continue;
    const uint16_t *row = w + (size_t)i * out;
    for (int j = 0; j < out; j++) o[j] += xv * (double)orc_f16_to_f32(row[j]);
  }
}

/* output side: f32 H_ho then * svh (kernels/trunk6/trunk6.metal:199-214) */
static void finish_out(const double *o, const uint16_t *svh, int out, float *y) {
  float *t = (float *)malloc(sizeof(float) * (size_t)out);
  for (int j = 0; j < out; j++) t[j] = (float)o[j];
  orc_fwht_f32(t, out, orc_had_size(out));
  for (int j = 0; j < out; j++) y[j] = t[j] * orc_f16_to_f32(svh[j]);
  free(t);
}

void orc_exl3_linear(const float *x, int R, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                     int in, int out, int K, float *y) {
  uint16_t *w = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)in * out);
  float *xh = (float *)malloc(sizeof(float) * (size_t)in);
  double *o = (double *)malloc(sizeof(double) * (size_t)out);
  orc_decode(trellis, in, out, K, w);
  for (int r = 0; r < R; r++) {
    prep_in(x + (size_t)r * in, suh, in, xh);
    inner_gemv(xh, w, in, out, o);
    finish_out(o, svh, out, y + (size_t)r * out);
  }
  free(w);
  free(xh);
  free(o);
}

/* y = x @ W, W = diag(suh) H_hi W' H_ho diag(svh), all f64 (tools/convert_trunk_enc.py:125-128): H is symmetric so
 * x @ W = ((H_hi (x * suh)) @ W') H_ho * svh */
void orc_exl3_linear_exact(const float *x, int R, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                           int in, int out, int K, double *y) {
  uint16_t *w = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)in * out);
  double *xs = (double *)malloc(sizeof(double) * (size_t)in);
  orc_decode(trellis, in, out, K, w);
  for (int r = 0; r < R; r++) {
    double *yr = y + (size_t)r * out;
    for (int i = 0; i < in; i++) xs[i] = (double)x[(size_t)r * in + i] * orc_f16_to_f32(suh[i]);
    orc_fwht_f64(xs, in, orc_had_size(in));
    for (int j = 0; j < out; j++) yr[j] = 0.0;
    for (int i = 0; i < in; i++)
      for (int j = 0; j < out; j++) yr[j] += xs[i] * (double)orc_f16_to_f32(w[(size_t)i * out + j]);
    orc_fwht_f64(yr, out, orc_had_size(out));
    for (int j = 0; j < out; j++) yr[j] *= orc_f16_to_f32(svh[j]);
  }
  free(w);
  free(xs);
}

/* The fused epilogues of a finished linear output v [R][out] (kernels/trunk6/trunk6.metal:129-197, t6_epi_col;
 * rr = bf16 rounding when refr, kernels/ne_common.h:27-29 for rr, silu and sigm). y rows are ldy floats apart.
 * kind 1: e0, e2 f32 [R][hc][out], e1 f32 [R][8]; 6: e0 = A_log, e1 = dt_bias (bf16 [out]); 7: e0 f32 key cache
 * of rows of 128 (cap rows), e1 u32 [1] = first row T. Returns -1 for kinds it does not cover (4, 8). */
static float rr_(float x, int refr) { return refr ? orc_bf16r(x) : x; }
int orc_lin_epi(const float *v, int R, int out, int kind, int refr, int hc, int ldy, float *y, void *e0, void *e1,
                float *e2, long cap) {
  for (int r = 0; r < R; r++)
    for (int c = 0; c < out; c++) {
      const float x = v[(size_t)r * out + c];
      float *yo = y + (size_t)r * ldy + c;
      switch (kind) {
        case 0: *yo = x; break;
        case 1: { /* trunk6.metal:152-158 */
          const float br = rr_(x, refr);
          *yo = br;
          for (int s = 0; s < hc; s++) {
            const size_t o = ((size_t)r * hc + s) * out + c;
            e2[o] = rr_(((float *)e0)[o] + rr_(br * ((float *)e1)[r * 8 + s], refr), refr);
          }
          break;
        }
        case 2: { /* trunk6.metal:159-160 */
          const float t = rr_(x, refr) * 0.25f;
          *yo = rr_(t / (1.0f + expf(-t)), refr);
          break;
        }
        case 3: *yo = rr_(x, refr); break; /* trunk6.metal:161-162 */
        case 5: *yo = rr_(1.0f / (1.0f + expf(-rr_(x, refr))), refr); break; /* trunk6.metal:180-181 */
        case 6: { /* trunk6.metal:182-188 */
          const float ex = expf(orc_bf16_to_f32(((uint16_t *)e0)[c])), dt = orc_bf16_to_f32(((uint16_t *)e1)[c]);
          const float u = rr_(rr_(x, refr) + dt, refr);
          const float sp = rr_(u > 20.0f ? u : logf(1.0f + expf(u)), refr);
          *yo = expf(-ex * sp);
          break;
        }
        case 7: { /* trunk6.metal:189-196 */
          *yo = x;
          const long t = (long)((uint32_t *)e1)[0] + r;
          if (c >= 512 && t < cap) ((float *)e0)[(size_t)t * 128 + (c - 512)] = x;
          break;
        }
        default: return -1;
      }
    }
  return 0;
}

/* ------------------------------------------------------------------------------------------------ router */
/* kernels/fn_moe.metal:50-66: logits = x . router row (bf16 weights), rr() to bf16 (reference rounding on) */
void orc_router_logits(const float *x, const uint16_t *rw, int ne, int hid, int round_bf16, float *logits) {
  for (int e = 0; e < ne; e++) {
    double a = 0.0;
    for (int i = 0; i < hid; i++) a += (double)x[i] * (double)orc_bf16_to_f32(rw[(size_t)e * hid + i]);
    logits[e] = round_bf16 ? orc_bf16r((float)a) : (float)a;
  }
}

/* kernels/fn_moe.metal:76-112,131: top-k by logit, the lower index wins ties (simd_min over tied winners);
 * p_k = exp(l_k - l_max) / sum_top exp(l_j - l_max) in f32 = softmax over all experts renormalised over the top k */
void orc_route(const float *logits, int ne, int topk, uint32_t *ids, float *w) {
  char *used = (char *)calloc((size_t)ne, 1);
  float vals[64];
  for (int k = 0; k < topk; k++) {
    int best = -1;
    for (int e = 0; e < ne; e++)
      if (!used[e] && (best < 0 || logits[e] > logits[best])) best = e;
    used[best] = 1;
    ids[k] = (uint32_t)best;
    vals[k] = logits[best];
  }
  float s = 0.0f;
  for (int k = 0; k < topk; k++) {
    w[k] = expf(vals[k] - vals[0]);
    s += w[k];
  }
  for (int k = 0; k < topk; k++) w[k] = w[k] / s;
  free(used);
}

/* ------------------------------------------------------------------------------------------------ MoE layer */
typedef struct {
  int in, out, K;
  const uint16_t *t, *su, *sv;
} lin_view;

static lin_view routed(const orc_moe *m, int proj, int e) {
  lin_view v;
  const int hid = m->hid, inter = m->inter;
  v.K = m->K;
  v.in = proj == 2 ? inter : hid;
  v.out = proj == 2 ? hid : inter;
  const size_t tsz = (size_t)v.in * v.out * m->K / 16; /* halfwords per expert projection */
  const uint16_t *t = proj == 0 ? m->gt : proj == 1 ? m->ut : m->dt;
  const uint16_t *su = proj == 0 ? m->gsu : proj == 1 ? m->usu : m->dsu;
  const uint16_t *sv = proj == 0 ? m->gsv : proj == 1 ? m->usv : m->dsv;
  v.t = t + (size_t)e * tsz;
  v.su = su + (size_t)e * v.in;
  v.sv = sv + (size_t)e * v.out;
  return v;
}
static lin_view shared(const orc_moe *m, int proj) {
  lin_view v;
  v.K = m->Ks;
  v.in = proj == 2 ? m->inter : m->hid;
  v.out = proj == 2 ? m->hid : m->inter;
  v.t = proj == 0 ? m->sgt : proj == 1 ? m->sut : m->sdt;
  v.su = proj == 0 ? m->sgsu : proj == 1 ? m->susu : m->sdsu;
  v.sv = proj == 0 ? m->sgsv : proj == 1 ? m->susv : m->sdsv;
  return v;
}

/* One expert at kernel arithmetic, scaled by wk, added into y (f32):
 *  D2 (kernels/fn_moe.metal:290-342): inner_g / inner_u = fp16(H128(x * suh)) @ W'   (raw, before H_ho)
 *  D3 (kernels/fn_moe.metal:370-415): g = H(inner_g) * svh_g, u = H(inner_u) * svh_u, h = H(silu(g) u * suh_d) -> fp16,
 *     o = h @ W'_d, v = H(o) * svh_d * wk */
static void expert_emul(const lin_view L[3], const float *x, float wk, float *v_out) {
  const int hid = L[0].in, inter = L[0].out;
  float *xh = (float *)malloc(sizeof(float) * (size_t)hid);
  double *o = (double *)malloc(sizeof(double) * (size_t)(hid > inter ? hid : inter));
  float *gu[2];
  uint16_t *w = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)hid * inter);
  for (int p = 0; p < 2; p++) {
    gu[p] = (float *)malloc(sizeof(float) * (size_t)inter);
    prep_in(x, L[p].su, hid, xh);
    orc_decode(L[p].t, hid, inter, L[p].K, w);
    inner_gemv(xh, w, hid, inter, o);
    for (int j = 0; j < inter; j++) gu[p][j] = (float)o[j];
    orc_fwht_f32(gu[p], inter, orc_had_size(inter));
    for (int j = 0; j < inter; j++) gu[p][j] *= orc_f16_to_f32(L[p].sv[j]);
  }
  float *hh = (float *)malloc(sizeof(float) * (size_t)inter);
  for (int j = 0; j < inter; j++) {
    const float g = gu[0][j], u = gu[1][j];
    hh[j] = g / (1.0f + expf(-g)) * u * orc_f16_to_f32(L[2].su[j]);
  }
  orc_fwht_f32(hh, inter, orc_had_size(inter));
  for (int j = 0; j < inter; j++) hh[j] = orc_f16_to_f32(orc_f32_to_f16(hh[j]));
  orc_decode(L[2].t, inter, hid, L[2].K, w);
  inner_gemv(hh, w, inter, hid, o);
  float *t = (float *)malloc(sizeof(float) * (size_t)hid);
  for (int j = 0; j < hid; j++) t[j] = (float)o[j];
  orc_fwht_f32(t, hid, orc_had_size(hid));
  for (int j = 0; j < hid; j++) v_out[j] = t[j] * orc_f16_to_f32(L[2].sv[j]) * wk;
  free(t);
  free(hh);
  free(gu[0]);
  free(gu[1]);
  free(w);
  free(o);
  free(xh);
}

void orc_q8_linear(const float *x, int R, const uint8_t *w, const uint16_t *s, const uint16_t *b, int in, int out,
                   int group, float *y) {
  const int ng = in / group;
  for (int r = 0; r < R; r++)
    for (int o = 0; o < out; o++) {
      double acc = 0.0;
      for (int g = 0; g < ng; g++) {
        double qx = 0.0, sx = 0.0; /* dot16q: (sum q x, sum x) per chunk, here per group */
        for (int i = g * group; i < (g + 1) * group; i++) {
          const double xv = x[(size_t)r * in + i];
          qx += (double)w[(size_t)o * in + i] * xv;
          sx += xv;
        }
        acc += (double)orc_bf16_to_f32(s[(size_t)o * ng + g]) * qx + (double)orc_bf16_to_f32(b[(size_t)o * ng + g]) * sx;
      }
      y[(size_t)r * out + o] = (float)acc;
    }
}

void orc_q8_shared(const orc_moe *m, const float *x, int refr, float *o) {
  const int hid = m->hid, inter = m->inter;
  float *g = (float *)malloc(sizeof(float) * (size_t)inter), *u = (float *)malloc(sizeof(float) * (size_t)inter);
  orc_q8_linear(x, 1, m->qgw, m->qgs, m->qgb, hid, inter, m->qgroup, g);
  orc_q8_linear(x, 1, m->quw, m->qus, m->qub, hid, inter, m->qgroup, u);
  for (int j = 0; j < inter; j++) {
    const float gv = rr_(g[j], refr), uv = rr_(u[j], refr);
    g[j] = rr_(gv / (1.0f + expf(-gv)) * uv, refr); /* kernels/fn_moe.metal:267-268 */
  }
  orc_q8_linear(g, 1, m->qdw, m->qds, m->qdb, inter, hid, m->qgroup, o);
  for (int c = 0; c < hid; c++) o[c] = rr_(o[c], refr); /* :288 rr(simd_sum) */
  free(g);
  free(u);
}

/* y[r] = sum over slots k in order (v_k) + sg * v_shared: the finisher's fixed slot order (kernels/fn_moe.metal:440-447,
 * kernels/prefill/pf_moe.metal:149-155); the shared expert's gate is sigmoid(logit) when the pack has
 * shared_expert_gate, else 1. */
int orc_moe_experts(const orc_moe *m, const float *x, int R, const uint32_t *route, const float *sg, float *y) {
  const int hid = m->hid;
  float *v = (float *)malloc(sizeof(float) * (size_t)hid);
  for (int r = 0; r < R; r++) {
    const float *xr = x + (size_t)r * hid;
    float *yr = y + (size_t)r * hid;
    for (int j = 0; j < hid; j++) yr[j] = 0.0f;
    for (int k = 0; k < m->topk; k++) {
      const uint32_t e = route[(size_t)r * 2 * m->topk + k];
      float wk;
      memcpy(&wk, &route[(size_t)r * 2 * m->topk + m->topk + k], 4);
      lin_view L[3] = {routed(m, 0, (int)e), routed(m, 1, (int)e), routed(m, 2, (int)e)};
      expert_emul(L, xr, wk, v);
      for (int j = 0; j < hid; j++) yr[j] += v[j];
    }
    if (m->sgt) {
      lin_view L[3] = {shared(m, 0), shared(m, 1), shared(m, 2)};
      expert_emul(L, xr, sg ? sg[r] : 1.0f, v);
      for (int j = 0; j < hid; j++) yr[j] += v[j];
    }
    if (m->qgw) { /* the 8-bit shared expert, reference rounding on */
      orc_q8_shared(m, xr, 1, v);
      const float gk = sg ? sg[r] : 1.0f;
      for (int j = 0; j < hid; j++) yr[j] += gk * v[j];
    }
  }
  free(v);
  return 0;
}

static void expert_exact(const lin_view L[3], const float *x, double wk, double *v_out) {
  const int hid = L[0].in, inter = L[0].out;
  double *gu[2];
  double *xs = (double *)malloc(sizeof(double) * (size_t)hid);
  uint16_t *w = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)hid * inter);
  for (int p = 0; p < 2; p++) {
    gu[p] = (double *)calloc((size_t)inter, sizeof(double));
    for (int i = 0; i < hid; i++) xs[i] = (double)x[i] * orc_f16_to_f32(L[p].su[i]);
    orc_fwht_f64(xs, hid, orc_had_size(hid));
    orc_decode(L[p].t, hid, inter, L[p].K, w);
    for (int i = 0; i < hid; i++)
      for (int j = 0; j < inter; j++) gu[p][j] += xs[i] * (double)orc_f16_to_f32(w[(size_t)i * inter + j]);
    orc_fwht_f64(gu[p], inter, orc_had_size(inter));
    for (int j = 0; j < inter; j++) gu[p][j] *= orc_f16_to_f32(L[p].sv[j]);
  }
  double *hh = (double *)malloc(sizeof(double) * (size_t)inter);
  for (int j = 0; j < inter; j++) {
    const double g = gu[0][j], u = gu[1][j];
    hh[j] = g / (1.0 + exp(-g)) * u * orc_f16_to_f32(L[2].su[j]);
  }
  orc_fwht_f64(hh, inter, orc_had_size(inter));
  orc_decode(L[2].t, inter, hid, L[2].K, w);
  for (int j = 0; j < hid; j++) v_out[j] = 0.0;
  for (int i = 0; i < inter; i++)
    for (int j = 0; j < hid; j++) v_out[j] += hh[i] * (double)orc_f16_to_f32(w[(size_t)i * hid + j]);
  orc_fwht_f64(v_out, hid, orc_had_size(hid));
  for (int j = 0; j < hid; j++) v_out[j] *= orc_f16_to_f32(L[2].sv[j]) * wk;
  free(hh);
  free(gu[0]);
  free(gu[1]);
  free(w);
  free(xs);
}

int orc_moe_experts_exact(const orc_moe *m, const float *x, int R, const uint32_t *route, const float *sg,
                          double *y) {
  const int hid = m->hid;
  double *v = (double *)malloc(sizeof(double) * (size_t)hid);
  for (int r = 0; r < R; r++) {
    double *yr = y + (size_t)r * hid;
    for (int j = 0; j < hid; j++) yr[j] = 0.0;
    for (int k = 0; k < m->topk; k++) {
      const uint32_t e = route[(size_t)r * 2 * m->topk + k];
      float wk;
      memcpy(&wk, &route[(size_t)r * 2 * m->topk + m->topk + k], 4);
      lin_view L[3] = {routed(m, 0, (int)e), routed(m, 1, (int)e), routed(m, 2, (int)e)};
      expert_exact(L, x + (size_t)r * hid, wk, v);
      for (int j = 0; j < hid; j++) yr[j] += v[j];
    }
    if (m->sgt) {
      lin_view L[3] = {shared(m, 0), shared(m, 1), shared(m, 2)};
      expert_exact(L, x + (size_t)r * hid, sg ? sg[r] : 1.0, v);
      for (int j = 0; j < hid; j++) yr[j] += v[j];
    }
    if (m->qgw) { /* no bf16 rounding points: the plain f64 shared expert */
      float *o = (float *)malloc(sizeof(float) * (size_t)hid);
      orc_q8_shared(m, x + (size_t)r * hid, 0, o);
      for (int j = 0; j < hid; j++) yr[j] += (sg ? sg[r] : 1.0) * (double)o[j];
      free(o);
    }
  }
  free(v);
  return 0;
}

static float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

int orc_moe_layer(const orc_moe *m, const float *x, int R, float *y, float *logits, uint32_t *route) {
  const int ne = m->ne, topk = m->topk, hid = m->hid;
  float *lg = (float *)malloc(sizeof(float) * (size_t)(ne + 1));
  uint32_t *rt = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)R * 2 * topk);
  float *sg = (float *)malloc(sizeof(float) * (size_t)R);
  for (int r = 0; r < R; r++) {
    const float *xr = x + (size_t)r * hid;
    orc_router_logits(xr, m->router, ne, hid, 1, lg);
    if (logits) memcpy(logits + (size_t)r * ne, lg, sizeof(float) * (size_t)ne);
    float w[64];
    orc_route(lg, ne, topk, rt + (size_t)r * 2 * topk, w);
    memcpy(rt + (size_t)r * 2 * topk + topk, w, sizeof(float) * (size_t)topk);
    sg[r] = 1.0f;
    if (m->sgate) {
      float l;
      orc_router_logits(xr, m->sgate, 1, hid, 1, &l);
      sg[r] = sigmoidf_(l);
    }
  }
  if (route) memcpy(route, rt, sizeof(uint32_t) * (size_t)R * 2 * topk);
  orc_moe_experts(m, x, R, rt, sg, y);
  free(lg);
  free(rt);
  free(sg);
  return 0;
}

/* The hyper-connection read's steps around its down / up linears (kernels/trunk6/t6_epi.metal:16-97), 4 streams of
 * hid per row. prep (:16-50): inv_s = 1/sqrt(sum(h_s^2) / hid + 1e-6), xn = (h w) inv_s, ip[r][s][j] = (sum_i
 * inject_j[s hid + i] (h w)[i]) inv_s, inj[r][4 + s] = inv_s. out (:80-97): v_s = rr(rr(sigmoid(rr(u_s))) rr((h_s
 * inv_s) w_s)), out = rr(((v_0 + v_1) + (v_2 + v_3)) / 4); gates (:53-78) inj[r][j] = rr(2 sigmoid(rr(sum_s ip) / 4)).
 * Sums over i in f64 (the GPU's f32 order is its own). */
void orc_hc_prep(const float *h, const uint16_t *nw, const uint16_t *iw, int R, int hid, float *xn, float *ip,
                 float *inj) {
  const size_t hcd = 4 * (size_t)hid;
  for (int r = 0; r < R; r++)
    for (int s = 0; s < 4; s++) {
      const float *hr = h + r * hcd + (size_t)s * hid;
      double ss = 0.0, a[4] = {0, 0, 0, 0};
      for (int i = 0; i < hid; i++) {
        const float xv = hr[i] * orc_bf16_to_f32(nw[s * hid + i]);
        ss += (double)hr[i] * hr[i];
        for (int k = 0; k < 4; k++) a[k] += (double)orc_bf16_to_f32(iw[k * hcd + s * hid + i]) * xv;
      }
      const float inv = 1.0f / sqrtf((float)ss / (float)hid + 1e-6f);
      for (int i = 0; i < hid; i++) xn[r * hcd + s * hid + i] = hr[i] * orc_bf16_to_f32(nw[s * hid + i]) * inv;
      for (int k = 0; k < 4; k++) ip[(r * 4 + s) * 4 + k] = (float)a[k] * inv;
      inj[r * 8 + 4 + s] = inv;
    }
}

void orc_hc_out(const float *u, const float *h, const uint16_t *nw, const float *ip, int R, int hid, int refr,
                float *inj, float *out) {
  const size_t hcd = 4 * (size_t)hid;
  for (int r = 0; r < R; r++) {
    for (int c = 0; c < hid; c++) {
      float v[4];
      for (int s = 0; s < 4; s++) {
        const size_t row = (size_t)s * hid + c;
        const float inv = inj[r * 8 + 4 + s];
        const float sg = rr_(sigmoidf_(rr_(u[r * hcd + row], refr)), refr);
        v[s] = rr_(sg * rr_(h[r * hcd + row] * inv * orc_bf16_to_f32(nw[row]), refr), refr);
      }
      out[(size_t)r * hid + c] = rr_(((v[0] + v[1]) + (v[2] + v[3])) * 0.25f, refr);
    }
    for (int j = 0; j < 4; j++) {
      float t = 0.0f;
      for (int s = 0; s < 4; s++) t += ip[(r * 4 + s) * 4 + j];
      inj[r * 8 + j] = rr_(2.0f * sigmoidf_(rr_(t, refr) * 0.25f), refr);
    }
  }
}

/* The layer with the hyper-connection write (kernels/fn_moe.metal:7-10 finisher, :420-448): the routed sum s (slot
 * order) and the gated shared term t kept apart; sg = rr(sigmoid(shared logit)) (:421, :444 rr(sgt)); y = branch =
 * rr(rr(s) + rr(t)); hout[r][st][c] = rr(h[r][st][c] + rr(branch * inj[r][st])), inj [R][8]. rr = bf16 when refr. */
void orc_hc_write(const float *s, const float *t, int R, int hid, int hc, int refr, const float *h, const float *inj,
                  float *y, float *hout) {
  for (int r = 0; r < R; r++)
    for (int c = 0; c < hid; c++) {
      const size_t i = (size_t)r * hid + c;
      const float br = rr_(rr_(s[i], refr) + rr_(t ? t[i] : 0.0f, refr), refr);
      y[i] = br;
      for (int st = 0; st < hc; st++) {
        const size_t o = ((size_t)r * hc + st) * hid + c;
        hout[o] = rr_(h[o] + rr_(br * inj[r * 8 + st], refr), refr);
      }
    }
}

int orc_moe_layer_hc(const orc_moe *m, const float *x, int R, int hc, int refr, const float *h, const float *inj,
                     float *y, float *hout) {
  const int ne = m->ne, topk = m->topk, hid = m->hid;
  float *lg = (float *)malloc(sizeof(float) * (size_t)(ne + 1));
  uint32_t *rt = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)2 * topk);
  float *s = (float *)calloc((size_t)hid, sizeof(float)), *t = (float *)calloc((size_t)hid, sizeof(float));
  float *v = (float *)malloc(sizeof(float) * (size_t)hid);
  for (int r = 0; r < R; r++) {
    const float *xr = x + (size_t)r * hid;
    orc_router_logits(xr, m->router, ne, hid, 1, lg);
    float w[64];
    orc_route(lg, ne, topk, rt, w);
    float sg = 1.0f;
    if (m->sgate) {
      float l;
      orc_router_logits(xr, m->sgate, 1, hid, 1, &l);
      sg = sigmoidf_(l);
    }
    sg = rr_(sg, refr);
    for (int j = 0; j < hid; j++) s[j] = t[j] = 0.0f;
    for (int k = 0; k < topk; k++) {
      lin_view L[3] = {routed(m, 0, (int)rt[k]), routed(m, 1, (int)rt[k]), routed(m, 2, (int)rt[k])};
      expert_emul(L, xr, w[k], v);
      for (int j = 0; j < hid; j++) s[j] += v[j];
    }
    if (m->sgt) {
      lin_view L[3] = {shared(m, 0), shared(m, 1), shared(m, 2)};
      expert_emul(L, xr, sg, t);
    }
    if (m->qgw) {
      orc_q8_shared(m, xr, refr, t);
      for (int j = 0; j < hid; j++) t[j] *= sg;
    }
    orc_hc_write(s, t, 1, hid, hc, refr, h + (size_t)r * hc * hid, inj + (size_t)r * 8, y + (size_t)r * hid,
                 hout + (size_t)r * hc * hid);
  }
  free(lg);
  free(rt);
  free(s);
  free(t);
  free(v);
  return 0;
}

/* ------------------------------------------------------------------------------------------------ CPU baseline */
static float g_mcg_tab[1 << 15];
static int g_mcg_ready = 0;
static void mcg_table_init(void) {
  if (g_mcg_ready) return;
  for (uint32_t c = 0; c < (1u << 15); c++) g_mcg_tab[c] = orc_f16_to_f32(orc_mcg(c));
  g_mcg_ready = 1;
}

/* one 16-column tile stripe of an EXL3 matrix: o[16] += xh[16 tk..] . W'[.., 16 tn..] over tiles k0..k1 */
static void stripe_dot(const uint16_t *trellis, int OT, int K, int tn, int k0, int k1, const float *xh, float *o) {
  const int NW = 8 * K;
  static const int rsel[4] = {0, 1, 8, 9};
  for (int tk = k0; tk < k1; tk++) {
    const uint16_t *tile = trellis + ((size_t)tk * OT + tn) * 16 * K;
    uint32_t wd[64];
    for (int w = 0; w < NW; w++) wd[w] = tile_word(tile, w);
    const float *xt = xh + 16 * tk;
    for (int s = 0; s < 256; s++) {
      const int start = ((s + 1) * K - 15 + 256 * K) % (256 * K);
      const int w0 = start >> 5, w1 = (w0 + 1) % NW;
      const uint64_t win = ((uint64_t)wd[w0] << 32) | wd[w1];
      const uint32_t cw = (uint32_t)(win >> (64 - 15 - (start & 31))) & 0x7FFFu;
      const int l = s >> 3, j = s & 7;
      const int row = 2 * (l & 3) + rsel[j & 3], col = (l >> 2) + 8 * (j >> 2);
      o[col] += xt[row] * g_mcg_tab[cw];
    }
  }
}

int orc_moe_experts_fast(const orc_moe *m, const float *x, int R, const uint32_t *route, const float *sg, float *y,
                         int nthreads) {
  mcg_table_init();
  const int hid = m->hid, inter = m->inter, topk = m->topk;
  const int nslot = topk + (m->sgt ? 1 : 0);
  const int S = R * nslot;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
  const int used = omp_get_max_threads();
#else
  const int used = 1;
#endif
  float *xh = (float *)malloc(sizeof(float) * (size_t)S * 2 * hid);
  float *gu = (float *)malloc(sizeof(float) * (size_t)S * 2 * inter);
  float *hh = (float *)malloc(sizeof(float) * (size_t)S * inter);
  float *dn = (float *)malloc(sizeof(float) * (size_t)S * hid);
  lin_view *L = (lin_view *)malloc(sizeof(lin_view) * (size_t)S * 3);
  float *wk = (float *)malloc(sizeof(float) * (size_t)S);
  for (int r = 0; r < R; r++)
    for (int k = 0; k < nslot; k++) {
      const int sl = r * nslot + k;
      for (int p = 0; p < 3; p++) {
        if (k < topk) L[sl * 3 + p] = routed(m, p, (int)route[(size_t)r * 2 * topk + k]);
        else L[sl * 3 + p] = shared(m, p);
      }
      if (k < topk) memcpy(&wk[sl], &route[(size_t)r * 2 * topk + topk + k], 4);
      else wk[sl] = sg ? sg[r] : 1.0f;
    }
#pragma omp parallel for schedule(static)
  for (int t = 0; t < S * 2; t++) {
    const int sl = t >> 1, p = t & 1;
    prep_in(x + (size_t)(sl / nslot) * hid, L[sl * 3 + p].su, hid, xh + (size_t)t * hid);
  }
  const int OTg = inter / 16;
#pragma omp parallel for schedule(dynamic, 4)
  for (int t = 0; t < S * 2 * OTg; t++) {
    const int sp = t / OTg, tn = t % OTg, sl = sp >> 1, p = sp & 1;
    float o[16] = {0};
    stripe_dot(L[sl * 3 + p].t, OTg, L[sl * 3 + p].K, tn, 0, hid / 16, xh + (size_t)sp * hid, o);
    for (int c = 0; c < 16; c++) gu[(size_t)sp * inter + 16 * tn + c] = o[c];
  }
#pragma omp parallel for schedule(static)
  for (int sl = 0; sl < S; sl++) {
    float *g = gu + (size_t)sl * 2 * inter, *u = g + inter, *h = hh + (size_t)sl * inter;
    orc_fwht_f32(g, inter, orc_had_size(inter));
    orc_fwht_f32(u, inter, orc_had_size(inter));
    for (int j = 0; j < inter; j++) {
      const float gv = g[j] * orc_f16_to_f32(L[sl * 3].sv[j]), uv = u[j] * orc_f16_to_f32(L[sl * 3 + 1].sv[j]);
      h[j] = gv / (1.0f + expf(-gv)) * uv * orc_f16_to_f32(L[sl * 3 + 2].su[j]);
    }
    orc_fwht_f32(h, inter, orc_had_size(inter));
    for (int j = 0; j < inter; j++) h[j] = orc_f16_to_f32(orc_f32_to_f16(h[j]));
  }
  const int OTd = hid / 16;
#pragma omp parallel for schedule(dynamic, 4)
  for (int t = 0; t < S * OTd; t++) {
    const int sl = t / OTd, tn = t % OTd;
    float o[16] = {0};
    stripe_dot(L[sl * 3 + 2].t, OTd, L[sl * 3 + 2].K, tn, 0, inter / 16, hh + (size_t)sl * inter, o);
    for (int c = 0; c < 16; c++) dn[(size_t)sl * hid + 16 * tn + c] = o[c];
  }
#pragma omp parallel for schedule(static)
  for (int sl = 0; sl < S; sl++) {
    float *d = dn + (size_t)sl * hid;
    orc_fwht_f32(d, hid, orc_had_size(hid));
    for (int j = 0; j < hid; j++) d[j] *= orc_f16_to_f32(L[sl * 3 + 2].sv[j]) * wk[sl];
  }
  for (int r = 0; r < R; r++)
    for (int j = 0; j < hid; j++) {
      float s = 0.0f;
      for (int k = 0; k < nslot; k++) s += dn[(size_t)(r * nslot + k) * hid + j];
      y[(size_t)r * hid + j] = s;
    }
  free(xh);
  free(gu);
  free(hh);
  free(dn);
  free(L);
  free(wk);
  return used;
}
