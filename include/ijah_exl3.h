/* EXL3 hot path on MI355X: trellis-decode fused into the MoE expert linears and the trunk linears.
 *
 * These entry points are the hot path's own C ABI. The reference adds such entry points in their own headers
 * (reference include/engine.h:11-12); each function cites the reference interface whose job it takes over. All
 * tensors are device buffers (ne_buf from engine.h); activations are f32 row-major, as in the reference kernels.
 * Errors: 0 / -1 (NULL) + ne_last_error(), as engine.h. Every function that takes gpu_ms (may be NULL) waits for
 * its GPU work and reports the GPU time of it; the others enqueue on the library stream and return.
 */
#ifndef IJAH_EXL3_H
#define IJAH_EXL3_H
#include "engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- buffers on a discrete GPU ---- */
/* Writes the whole host mirror returned by ne_buf_contents back to the device now (changed bytes also go on their
 * own before the next library call that uses the buffer, unless that call is made while the library stream is
 * being captured into a graph: flush before a capture). No reference counterpart: the reference's buffers are
 * unified memory (reference include/engine.h:6-7), where this is a no-op. */
NE_API int ne_buf_flush(ne_buf *b);
/* Waits for all queued GPU work of the library (the reference's Recorder::wait, core/recorder.h:76). */
NE_API int ne_sync(void);
/* The library's HIP stream (a hipStream_t; NULL with ne_last_error set if no device), so that a caller can capture
 * library calls into its own HIP graph (hipStreamBeginCapture on it, the calls, hipStreamEndCapture) or order its own
 * work against them. Calls that allocate refuse to grow scratch during a capture; ne_exl3_lin_run_noalloc allocates
 * nothing. No reference counterpart: the reference records into its own command buffers (core/recorder.h). */
NE_API void *ne_stream(void);

/* ---- pack alignment ----
 * reference core/pack_align.h:1-25 (ne::align_pack, the engine-cli `align-pack` command): writes into dst_dir a copy of
 * the pack in src_dir whose every tensor's data starts at a multiple of align bytes of its shard. Aligned shards,
 * config.json and other files become symbolic links to the source; a misaligned shard is rewritten (tensor order kept,
 * offsets rounded up, header padded with spaces), read back and compared byte for byte before it is renamed into
 * place; a rerun keeps shards already copied. dry_run: only count (dst_dir untouched). Returns 0, or -1 with
 * ne_last_error(). */
typedef struct {
  uint64_t tensors, misaligned_tensors, misaligned_bytes, files_rewritten, files_linked, files_kept, bytes_written;
} ne_pack_align_stats;
NE_API int ne_pack_align(const char *src_dir, const char *dst_dir, uint64_t align, int dry_run,
                         ne_pack_align_stats *stats);

/* ---- one EXL3 linear: y[R][out] = x[R][in] @ W, W = diag(suh) H_in W' H_out diag(svh) ----
 * trellis U16 [in/16][out/16][16K] (tile (tk, tn) = W'[16tk.., 16tn..] in the reference's slot order), suh F16 [in],
 * svh F16 [out]; K 1..8; in, out multiples of 16 and of their Hadamard sizes (128, 64, 32 or 16). */
typedef struct ne_exl3_lin ne_exl3_lin;
/* reference kernels/trunk6/trunk6.mm:39-66 (t6::load of "<prefix>.trellis/.suh/.svh"); the tiles are re-laid in HBM
 * for the GEMV's streaming order (pairs of output tiles, k-major inside a pair). */
NE_API ne_exl3_lin *ne_exl3_lin_load(const ne_pack *p, const char *prefix);
/* same from host arrays in the pack's layout */
NE_API ne_exl3_lin *ne_exl3_lin_create(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh, int in,
                                       int out, int K);
NE_API void ne_exl3_lin_free(ne_exl3_lin *l);
NE_API int ne_exl3_lin_info(const ne_exl3_lin *l, int *in, int *out, int *K);
/* reference kernels/trunk6/trunk6.mm:232-249 (t6::record: SIMD path R 1..8, matrix-op path t6_nax above that):
 * x f32 [R][in] at x_off, y f32 [R][out] at y_off; R 1..32 (1..8 on the VALU GEMV, 9..32 on the matrix cores). */
NE_API int ne_exl3_lin_run(ne_exl3_lin *l, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                           double *gpu_ms);
/* ne_exl3_lin_run that allocates nothing: no counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). Its block counters, prepared input and k group partials live
 * in one fixed 32 MiB scratch array per GPU, held until the process ends; a run needing more (e.g. a 151936-wide
 * vocabulary head at 32 rows) is rejected with an error. Same results as ne_exl3_lin_run. Every call on one GPU
 * shares that array: calls that overlap on one GPU (other streams or threads) race. Not timed (no gpu_ms). */
NE_API int ne_exl3_lin_run_noalloc(ne_exl3_lin *l, int R, const ne_buf *x, uint64_t x_off, ne_buf *y,
                                   uint64_t y_off);
/* A fused epilogue on a linear's finished outputs v (reference kernels/trunk6/trunk6.metal:129-197, t6_epi_col, the
 * layer graph's q8 epilogues; rr = round to bf16 when refr, the reference rounding switch FC 0):
 *   0 none     y = v
 *   1 out_hc   y = b = rr(v); e2[r][s][c] = rr(e0[r][s][c] + rr(b e1[r][s])), s < hc (e0, e2 f32 [R][hc][out];
 *              e1 f32 [R][8])
 *   2 hc act   y = rr(silu(rr(v) / 4))
 *   3 round    y = rr(v)
 *   5 beta     y = rr(sigmoid(rr(v)))  (the reference's y[r][48 + c] of gb [R][96]: y_off = 192 bytes, ldy = 96)
 *   6 decay    y = exp(-exp(A_log[c]) sp), sp = rr(softplus(rr(rr(v) + dt_bias[c]))) (e0 = A_log, e1 = dt_bias,
 *              bf16 [out]; the reference's gb [R][96]: ldy = 96)
 *   7 iqk      y = v; for c >= 512, e0[(T + r) 128 + c - 512] = v (e0 f32 key cache of rows of 128, e1 u32 [1] = T;
 *              rows T + r beyond e0's size are not written)
 * Kind 4 (GDN conv1d with state) is not provided; kind 8 (the HC read's output step, through counters) runs inside
 * ne_hc_read only. ldy = y's row stride
 * in floats (0: out). */
typedef struct ne_exl3_epi {
  int kind, refr, hc, ldy;
  const ne_buf *e0, *e1, *e2;
} ne_exl3_epi;
/* ne_exl3_lin_run with a fused epilogue (reference kernels/trunk6/trunk6.mm:232-249 with T6_EPI / T6_LDY set,
 * trunk6.metal:199-222 t6_finish) */
NE_API int ne_exl3_lin_run_epi(ne_exl3_lin *l, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                               const ne_exl3_epi *epi, double *gpu_ms);
/* The hyper-connection read on EXL3 mixes (reference models/flash_next/layer_t6.mm:89-133, t6_hc_read, with
 * kernels/trunk6/t6_epi.metal:16-97; rr = bf16 rounding when refr): for each row and stream s of h f32 [R][4][hid],
 * inv_s = 1/sqrt(mean(h_s^2) + 1e-6), xn = h w inv_s (w = hc_norm bf16 [4 hid]); mix f32 [R][lr] = rr(silu(rr(down(xn))
 * / 4)) (down: 4 hid -> lr); u = up(mix) (lr -> 4 hid); out f32 [R][hid] = rr(((v_0 + v_1) + (v_2 + v_3)) / 4),
 * v_s = rr(rr(sigmoid(rr(u_s))) rr(h_s inv_s w_s)); inj f32 [R][8] = the 4 block-inject gates rr(2 sigmoid(rr(sum_s
 * inject_j . (h_s w_s) inv_s) / 4)) (inject bf16 [4][4 hid]), then inv_0..3. out is the MoE (or attention) input and
 * inj the gates of the HC write that follows (ne_moe_run_hc). R 1..32. */
NE_API int ne_hc_read(ne_exl3_lin *down, ne_exl3_lin *up, int R, const ne_buf *h, const ne_buf *hc_norm,
                      const ne_buf *inject, ne_buf *mix, ne_buf *inj, ne_buf *out, int refr, double *gpu_ms);
/* n linears at R rows, all reading x (f32 [R][in_i]) and writing scratch outputs, captured once in a HIP graph and
 * replayed reps times after warmup replays: us_per_lin = GPU time per linear (HIP events). Replaces the reference's
 * differential timing of the trunk stages (kernels/trunk6/trunk6.mm:232-249 replays, core/bench.h:21-24). */
NE_API int ne_exl3_lin_time(ne_exl3_lin *const *lins, int n, int R, const ne_buf *x, int warmup, int reps,
                            double *us_per_lin);
/* ne_exl3_lin_time with the linears recorded together, consecutive runs of up to `group` (1..4) linears of one K per
 * launch: us = GPU time of all n per replay (reference kernels/trunk6/trunk6.mm:251-280, record_multi, timed as one
 * stage). */
NE_API int ne_exl3_lin_time_multi(ne_exl3_lin *const *lins, int n, int group, int R, const ne_buf *x, int warmup,
                                  int reps, double *us);
/* reference kernels/trunk6/trunk6.h:78 (t6::record_multi): n linears at R rows recorded to run concurrently, linear i
 * from x[i] at x_off[i] into y[i] at y_off[i] (each its own scratch); consecutive linears of one K share a launch.
 * R 1..32. */
NE_API int ne_exl3_lin_run_multi(ne_exl3_lin *const *lins, int n, int R, const ne_buf *const *x,
                                 const uint64_t *x_off, ne_buf *const *y, const uint64_t *y_off, double *gpu_ms);
/* W' decoded on the GPU from the re-laid tiles: fp16 bits [in][out] into w (at least in*out*2 bytes). Replaces the
 * reference's decoded-weight check through exl3_codec.decode_inner (tests/trunk6/check_kernels.py:86). */
NE_API int ne_exl3_lin_decode(ne_exl3_lin *l, ne_buf *w, double *gpu_ms);

/* ---- fused MoE layer (router + softmax/top-k + routed and shared EXL3 experts + weighted combine) ---- */
typedef struct ne_moe ne_moe;
/* Host arrays in the pack's layout (reference models/flash_next/layer.mm:180-196, MoeW of layer.h:37):
 *   router BF16 [ne][hid]; sgate BF16 [hid] or NULL (no shared_expert_gate: the shared expert is added with weight 1);
 *   routed gate/up/down: trellis U16 [ne][in/16][out/16][16K], suh F16 [ne][in], svh F16 [ne][out];
 *   shared expert, at most one of two forms (all NULL = none):
 *     EXL3: gate/up/down trellis U16 [in/16][out/16][16 Ks], suh, svh;
 *     8-bit affine (the reference's Q8, layer.h:21; the form of its real packs): weight U32 [rows][in/4] (bytes
 *     row-major), scales and biases BF16 [rows][in/qgroup], w = scale q + bias; qgroup 128; gate and up [inter][hid],
 *     down [hid][inter]. Its outputs are rounded to bf16 as the reference's (kernels/fn_moe.metal:47,268,288). */
typedef struct {
  int hid, inter, ne, topk, K, Ks;
  const uint16_t *router, *sgate;
  const uint16_t *gt, *ut, *dt, *gsu, *gsv, *usu, *usv, *dsu, *dsv;
  const uint16_t *sgt, *sut, *sdt, *sgsu, *sgsv, *susu, *susv, *sdsu, *sdsv;
  int qgroup;
  const uint32_t *qgw, *quw, *qdw;
  const uint16_t *qgs, *qgb, *qus, *qub, *qds, *qdb;
} ne_moe_desc;
NE_API ne_moe *ne_moe_create(const ne_moe_desc *d);
/* reference models/flash_next/layer.mm:180-196 (MoeW from "<prefix>gate.weight", "switch_mlp.*", "shared_expert.*",
 * "shared_expert_gate.weight"); prefix like "language_model.model.layers.0.mlp." The pack's expert tensors are
 * re-laid so each expert's trellis tiles, suh and svh are one contiguous 256-byte-aligned block in HBM. */
NE_API ne_moe *ne_moe_load(const ne_pack *p, const char *prefix, int topk);
/* Seeded synthetic layer generated on the device (no host copy): trellis uniform u16, suh / svh = +-|N(1, 0.1)|,
 * router BF16 N(0, 1/hid) (logits ~ N(0,1) for N(0,1) inputs). has_shared: 1 = an EXL3 shared expert of Ks bits,
 * 2 = an 8-bit affine one (g128: weight bytes uniform, scale = |N(1, 0.1)| / (74 sqrt(in)), bias = -127.5 scale).
 * No reference counterpart (the reference benchmarks real packs); it feeds the benchmark at full size. */
NE_API ne_moe *ne_moe_synth(int hid, int inter, int ne, int topk, int K, int has_shared, int Ks, uint64_t seed);
NE_API void ne_moe_free(ne_moe *m);
/* reference models/flash_next/layer.h:244-263 (ne_fn_layer_run_stage(l, 5): moe_router, moe_gateup, moe_down):
 * x f32 [R][hid] -> y f32 [R][hid] = sum over the top-k slots in slot order of w_k expert_k(x) + g * shared(x). */
NE_API int ne_moe_run(ne_moe *m, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                      double *gpu_ms);
/* The hyper-connection write fused into the layer's combine (reference kernels/fn_moe.metal:7-10 and :420-448, the
 * finisher of fn_moe_down; rr = bf16 rounding when refr, the reference rounding switch FC 0): the shared gate is
 * rr(sigmoid(logit)), y = branch = rr(rr(sum of the routed slots in slot order) + rr(gate * shared expert)), and
 * hout[r][s][c] = rr(h[r][s][c] + rr(branch * inj[r][s])) for s < hc. h, hout f32 [R][hc][hid] (hout may be h: each
 * element is read and written by one thread); inj f32 [R][8]. */
typedef struct ne_moe_hc {
  int hc, refr;
  const ne_buf *h, *inj;
  ne_buf *hout;
} ne_moe_hc;
NE_API int ne_moe_run_hc(ne_moe *m, int R, const ne_buf *x, uint64_t x_off, ne_buf *y, uint64_t y_off,
                         const ne_moe_hc *hc, double *gpu_ms);
/* reference models/flash_next/layer.h:258-262 (ne_fn_layer_read) for the MoE intermediates of the last run:
 * "logits" f32 [R][ne], "route" u32 [R][2 topk] (ids, f32 weight bits), "shared_gate" f32 [R],
 * "experts_gu" f32 [R][slots][2][inter] (gate / up inner outputs before H_out), "experts_dn" f32 [R][slots][hid]
 * (down inner outputs before H_out), "mlp_out" f32 [R][hid], "shared_q8" f32 [R][hid] (the 8-bit shared expert's
 * rounded output before its gate). Copies at most nbytes; returns 0. */
NE_API int ne_moe_read(ne_moe *m, const char *name, void *dst, uint64_t nbytes);
/* Layer options (no reference counterpart: the reference picks its dispatch forms by function constants at build):
 *   "staged" 1: every row count on the four staged launches (router, gate/up, down, combine) instead of the fused
 *               one-row step (R = 1) and the grouped matrix-core kernels (R >= 2); 0: the default choice;
 *   "trace"  1: the fused step keeps per-wave wall-clock stamps of its phases (ne_moe_read "trace"); 0: off.
 * Waits for queued work first. Returns 0, or -1 for an unknown key. */
NE_API int ne_moe_configure(ne_moe *m, const char *key, int value);
/* Linear options: "staged" 1 = three launches (prep, GEMM, finish) instead of one; 0: one launch (default). */
NE_API int ne_exl3_lin_configure(ne_exl3_lin *l, const char *key, int value);
/* Expert e's projection proj (0 gate, 1 up, 2 down; e == ne: the shared expert) decoded from the re-laid HBM block:
 * fp16 bits [in][out] into w. */
NE_API int ne_moe_decode(ne_moe *m, int e, int proj, ne_buf *w, double *gpu_ms);
NE_API int ne_moe_info(const ne_moe *m, int *hid, int *inter, int *ne, int *topk, int *K, int *slots);
/* Bytes one layer step at R rows reads from HBM by algorithm: the touched experts' trellis + suh + svh (distinct
 * experts of the last run's route), the shared expert and the router. */
NE_API int ne_moe_bytes(const ne_moe *m, int R, uint64_t *bytes);
/* Chain of n layers (layer i's output feeds layer i+1; layers may repeat), captured once in a HIP graph and replayed
 * reps times after warmup replays: us_per_layer = GPU time per layer (HIP events on the library stream). Replaces the
 * reference's differential timing (ne_fn_layer_time, models/flash_next/layer.h:266-267; core/bench.h:21-24). */
NE_API int ne_moe_time(ne_moe *const *layers, int n, int R, const ne_buf *x, int warmup, int reps,
                       double *us_per_layer);
/* Per-kernel timing of the same chain: launches each kernel kind alone, reps times per layer, and returns the mean
 * duration in microseconds of each: the staged path's "router", "gateup", "down", "combine", and "fused" (the whole
 * step in one persistent launch) when instantiated for the layer's bit widths. n_kinds: capacity in (>= 5), count out. */
NE_API int ne_moe_time_kernels(ne_moe *const *layers, int n, int R, const ne_buf *x, int reps, char names[][16],
                               double *us, int *n_kinds);

#ifdef __cplusplus
}
#endif
#endif /* IJAH_EXL3_H */
