/* CPU oracle for the EXL3 trellis decode + MoE / trunk linear path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (ijah_amd/) links, loads or calls this code; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg do, and there only as the checker / the timed CPU baseline.
 *
 * Every function restates the reference algorithm (publicExcess/ijah) in plain C. Citations are file:line in the
 * reference tree. The reference ships no golden vectors for this path and its CPU decoder (the external exl3_codec
 * module, no pinned version) cannot run here, so each function is pinned by tests/test_oracle.py against something
 * it shares no code with:
 *   orc_f32_to_f16 / orc_f16_to_f32 / orc_bf16r: numpy IEEE fp16 on 4,000 values + edge cases; bf16 tie known answers.
 *   orc_mcg:              known answers (cw 0 -> 0x3F60, cw 1) and all 2^15 codewords against numpy uint32 arithmetic.
 *   orc_tile_cw_ring/lane/t6: the three readers agree on random tiles (K 1..8), a pure-Python ring walk, constant
 *                         tiles, and single-bit placement (each bit lands in exactly the windows that cover it).
 *   orc_slot_rc / orc_decode: bijection + the reference row/column formula; decode vs per-tile codeword lookups.
 *   orc_fwht_*:           the textbook Sylvester matrix (parity of popcount(i & j)), blocks of 16..128.
 *   orc_exl3_linear*:     explicit-matrix numpy restatement diag(suh) H W' H diag(svh).
 *   orc_lin_epi:          numpy closed forms per kind (silu, sigmoid, softplus, exp decay) with bf16 rounding points
 *                         placed independently, and the rounding switch off vs plain float math.
 *   orc_router_logits / orc_route: numpy dot + bf16 rounding; ties to the lower index vs numpy stable argsort.
 *   orc_moe_*:            explicit numpy restatement of SwiGLU experts and the slot-order combine.
 *   orc_hc_prep / orc_hc_out: numpy closed forms (rms, inject dots, sigmoid-weighted stream mean) and, composed with
 *                         the oracle linears, an f64 numpy restatement of the whole HC read.
 *   orc_hc_write / orc_moe_layer_hc: numpy closed form of the finisher; with rounding off the branch equals the plain
 *                         layer's slot-order sum bit for bit; the shared term is the plain layer minus its routed part.
 * Parity versus upstream exllamav3's codec itself stays unpinned (the module is absent); the restatement follows
 * the reference's Metal kernels, which the reference checks against that codec (docs/trunk6.md:74-84).
 */
#ifndef IJAH_EXL3_ORACLE_H
#define IJAH_EXL3_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---- */
uint16_t orc_f32_to_f16(float f); /* IEEE binary16, round to nearest even */
float orc_f16_to_f32(uint16_t h);
float orc_bf16r(float x);          /* round to bf16 (RNE) and back to f32: kernels/ne_common.h:23-26 */
float orc_bf16_to_f32(uint16_t b);

/* ---- EXL3 codebook and trellis readers ---- */
uint16_t orc_mcg(uint32_t cw);     /* window-15 MCG codeword -> fp16 bits: kernels/ne_common.h:139-144 */
/* slot s (0..255) -> row, col inside a 16x16 tile: kernels/ne_common.h:105-108, kernels/trunk6/trunk6.metal:611-629 */
void orc_slot_rc(int s, int *row, int *col);
/* codeword (16 bits; the decoder uses the low 15) of every slot of one tile (16K u16 halfwords).
 * ring: brute force over the tail-biting ring of 256K bits (the definition).
 * lane: kernels/ne_common.h:109-157 lane_load/lane_funnel/cw_at, K 4..6.
 * t6:   kernels/trunk6/trunk6.metal:91-127 t6_lane/t6_load/t6_dec, K 1..8. */
void orc_tile_cw_ring(const uint16_t *tile, int K, uint16_t cw[256]);
int orc_tile_cw_lane(const uint16_t *tile, int K, uint16_t cw[256]);
int orc_tile_cw_t6(const uint16_t *tile, int K, uint16_t cw[256]);
/* W' [in][out] as fp16 bits from trellis U16 [in/16][out/16][16K] */
void orc_decode(const uint16_t *trellis, int in, int out, int K, uint16_t *w);

/* ---- Hadamard ---- */
int orc_had_size(int d);                       /* tools/convert_trunk_enc.py:59-63 */
float orc_had_scale(int n);                    /* f32(1/sqrt(n)) */
void orc_fwht_f32(float *v, int n, int had);   /* blocks of `had`, butterfly bits 0,1,..; then * 1/sqrt(had) */
void orc_fwht_f64(double *v, int n, int had);

/* ---- EXL3 linear: y[R][out] = x[R][in] @ W, W = diag(suh) H_hi W' H_ho diag(svh) ---- */
/* kernel arithmetic: f32 x*suh, f32 FWHT, fp16 prep, f64 dot with exact fp16 W', f32 H_ho, * svh
 * (tests/trunk6/check_kernels.py:96-98, kernels/trunk6/trunk6.metal:68-85,199-214) */
void orc_exl3_linear(const float *x, int R, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                     int in, int out, int K, float *y);
/* fused epilogues of a finished linear output (kernels/trunk6/trunk6.metal:129-197): kinds 0, 1, 2, 3, 5, 6, 7 */
int orc_lin_epi(const float *v, int R, int out, int kind, int refr, int hc, int ldy, float *y, void *e0, void *e1,
                float *e2, long cap);
/* exact: everything in f64, no fp16 rounding of the input (tools/convert_trunk_enc.py:125-128) */
void orc_exl3_linear_exact(const float *x, int R, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                           int in, int out, int K, double *y);

/* ---- router (kernels/fn_moe.metal:50-131) ---- */
/* logits[ne] = bf16r(f32(x . rw[e])) when round_bf16 (the reference's default rounding, FC 0 on) */
void orc_router_logits(const float *x, const uint16_t *rw, int ne, int hid, int round_bf16, float *logits);
/* top-k by logit (ties -> lower index), weights exp(l - l_max) / sum over the top k, f32 */
void orc_route(const float *logits, int ne, int topk, uint32_t *ids, float *w);

/* ---- fused MoE layer at R rows (kernels/fn_moe.metal D1-D3, tools/opref.py:417-435) ---- */
typedef struct {
  int hid, inter, ne, topk, K;   /* K = routed expert bits */
  const uint16_t *router;        /* BF16 [ne][hid] */
  const uint16_t *sgate;         /* BF16 [hid] shared-expert gate row, or NULL (shared weight 1) */
  /* routed: trellis [ne][in/16][out/16][16K], suh [ne][in], svh [ne][out] */
  const uint16_t *gt, *ut, *dt, *gsu, *gsv, *usu, *usv, *dsu, *dsv;
  /* shared expert (NULL = none): same per-projection layout without the expert dim; bits Ks */
  int Ks;
  const uint16_t *sgt, *sut, *sdt, *sgsu, *sgsv, *susu, *susv, *sdsu, *sdsv;
  /* the shared expert in 8-bit affine form instead (NULL qgw = none; exclusive with sgt): weight bytes [rows][in]
   * (gate/up [inter][hid], down [hid][inter]), scales / biases BF16 [rows][in / qgroup] */
  int qgroup;
  const uint8_t *qgw, *quw, *qdw;
  const uint16_t *qgs, *qgb, *qus, *qub, *qds, *qdb;
} orc_moe;
/* 8-bit affine linear (kernels/ne_common.h:33-88 q8row_dev / dot16q, MLX layout): y[r][o] = sum over groups g of
 * s[o][g] sum_{i in g} q[o][i] x[r][i] + b[o][g] sum_{i in g} x[r][i], summed in f64, returned in f32 */
void orc_q8_linear(const float *x, int R, const uint8_t *w, const uint16_t *s, const uint16_t *b, int in, int out,
                   int group, float *y);
/* the layer's 8-bit shared expert on one row (kernels/fn_moe.metal:40-47, :264-290): g = rr(gate x), u = rr(up x),
 * h = rr(silu(g) u), o = rr(down h); rr = bf16 when refr. o [hid]. */
void orc_q8_shared(const orc_moe *m, const float *x, int refr, float *o);
/* kernel arithmetic; y [R][hid] f32; logits [R][ne] (may be NULL); route [R][2 topk] u32 (ids, f32 weight bits,
 * may be NULL). Returns 0. */
int orc_moe_layer(const orc_moe *m, const float *x, int R, float *y, float *logits, uint32_t *route);
/* the hyper-connection read's prep and output steps (kernels/trunk6/t6_epi.metal:16-97) */
void orc_hc_prep(const float *h, const uint16_t *nw, const uint16_t *iw, int R, int hid, float *xn, float *ip,
                 float *inj);
void orc_hc_out(const float *u, const float *h, const uint16_t *nw, const float *ip, int R, int hid, int refr,
                float *inj, float *out);
/* the hyper-connection write (kernels/fn_moe.metal:437-448) from the routed sum s and gated shared term t (t may be
 * null), and the layer with it (shared gate rounded to bf16 when refr) */
void orc_hc_write(const float *s, const float *t, int R, int hid, int hc, int refr, const float *h, const float *inj,
                  float *y, float *hout);
int orc_moe_layer_hc(const orc_moe *m, const float *x, int R, int hc, int refr, const float *h, const float *inj,
                     float *y, float *hout);
/* Same layer given a route (ids + f32 weights [R][2 topk]) and shared gate value per row (sg may be NULL -> 1):
 * separates the routing decision from the expert math in tests. */
int orc_moe_experts(const orc_moe *m, const float *x, int R, const uint32_t *route, const float *sg, float *y);
/* f64 "exact" layer from the same route: no fp16 rounding anywhere, f64 math throughout */
int orc_moe_experts_exact(const orc_moe *m, const float *x, int R, const uint32_t *route, const float *sg, double *y);

/* ---- CPU baseline (timed in bench.py): the same layer math, OpenMP over slots and column tiles,
 * a 2^15-entry MCG table instead of the multiply. Returns the number of threads used. ---- */
int orc_moe_experts_fast(const orc_moe *m, const float *x, int R, const uint32_t *route, const float *sg, float *y,
                         int nthreads);

#ifdef __cplusplus
}
#endif
#endif
