// Host-side view of the HIP kernels: registry for ne_run_kernel and the launch wrappers the entry points use.
#pragma once
#include <string>
#include <vector>

#include "common.h"

namespace ijah {

struct KernelEntry {
  std::string name;
  const void *fn;
  std::vector<uint32_t> arg_sizes;
  int K;  // function constant 10 (-1: not specialised on it)
  int R;  // function constant 16
};
// name + optional function constants (index 10 = K, 16 = R) -> entry, or nullptr
const KernelEntry *find_kernel(const char *name, const ne_fconst *fc, int nfc);

// Byte offsets of one expert's (or one linear's) regions inside its HBM block. Tiles of a projection are re-laid as
// [n-pair p][k-tile tk][2], so a workgroup working on output tiles (2p, 2p+1) streams one contiguous span.
struct ExpertLayout {
  int K = 0;
  uint64_t tr[3] = {0, 0, 0};  // gate, up, down trellis
  uint64_t su[3] = {0, 0, 0};  // F16 input scales
  uint64_t sv[3] = {0, 0, 0};  // F16 output scales
  uint64_t bytes = 0;          // block stride (256-byte multiple)
};
ExpertLayout expert_layout(int hid, int inter, int K);
// halfword index of tile (tk, tn) of a [IT][OT] matrix in the re-laid order (OT padded to even)
inline uint64_t relaid_tile(int IT, int tk, int tn) { return ((uint64_t)(tn >> 1) * IT + tk) * 2 + (tn & 1); }

struct MoeArgs {
  const float *x;
  float *y;
  int R, hid, inter, ne, topk, nslot;  // nslot = topk + (shared expert ? 1 : 0)
  const uint16_t *router;              // BF16 [ne + has_sgate][hid]
  int has_sgate;
  const uint8_t *experts;              // ne blocks of stride lay.bytes
  const uint8_t *shared;               // shared block (layout slay) or null
  ExpertLayout lay, slay;
  int had_hid, had_inter;
  float sc_hid, sc_inter;              // f32(1/sqrt(had))
  int ksplit;                          // gate/up k splits
  float *logits;                       // [R][ne + 1]
  uint32_t *route;                     // [R][2 topk]
  float *sgv;                          // [R]
  float *guo;                          // [R nslot][2][ksplit][inter]
  float *dn;                           // [R nslot][hid]
  uint32_t *sync;                      // counters: see sync_words(); zero between launches (kernels reset them)
  uint64_t *trace;                     // fused kernel: per-wave wall-clock stamps of its phases, or null
  uint16_t *hprep;                     // fused kernel: [R nslot][inter] fp16 down inputs (kp order)
  const uint32_t *units;               // fused kernel: the plan words (MoePlan::words) in device memory
  float *part;                         // fused kernel: column partial sums (MoePlan::part_floats)
  uint32_t *fsync;                     // fused kernel: its counters (moe_fused_sync_words), zero when created
  int fused_slots = 0;                 // fused kernel: LDS slots of its plan (MoePlan::slots)
  // The hyper-connection write fused into the combine (reference kernels/fn_moe.metal:7-10, 420-448), on when hc > 0
  // (rr = bf16 rounding when refr): the shared gate is rr(sigmoid), y = branch = rr(rr(routed sum) + rr(gated shared)),
  // hc_out[r][s][c] = rr(hc_h[r][s][c] + rr(branch hc_inj[r][s])) for s < hc; hc_h, hc_out f32 [R][hc][hid], hc_inj
  // f32 [R][8].
  int hc = 0, refr = 1;
  const float *hc_h = nullptr, *hc_inj = nullptr;
  float *hc_out = nullptr;
  // The shared expert in the reference's 8-bit affine form (q8_offsets), in place of an EXL3 shared
  // slot (nslot == topk then): g = rr(gate . x), u = rr(up . x), h = rr(silu(g) u), o = rr(down . h) (rr: bf16 when
  // refr); the combine adds the shared gate times o after the routed slots. Null: none.
  const uint8_t *q8 = nullptr;
  const uint16_t *q8bf = nullptr;  // its weight bytes as bf16 values [3 matrices], for the many-row form
  float *q8gu = nullptr;  // [R][2 inter] g, u (staged and batched paths)
  float *q8o = nullptr;   // [R][hid] o
};
// Byte offsets inside the 8-bit shared expert's block: gate, up, down weight bytes, then their group words.
constexpr int kQ8Group = 128;
struct Q8Off {  // byte offsets inside the 8-bit block
  uint64_t w[3], sb[3];
};
__host__ __device__ inline Q8Off q8_offsets(int hid, int inter) {
  Q8Off o;
  const uint64_t gu = (uint64_t)inter * hid;
  o.w[0] = 0;
  o.w[1] = gu;
  o.w[2] = 2 * gu;
  o.sb[0] = 3 * gu;
  o.sb[1] = o.sb[0] + gu / kQ8Group * 4;
  o.sb[2] = o.sb[1] + gu / kQ8Group * 4;
  return o;
}
__host__ __device__ inline uint64_t q8_block_bytes(int hid, int inter) {
  return 3 * (uint64_t)inter * hid + 3 * (uint64_t)inter * hid / kQ8Group * 4;
}
// the 8-bit shared expert's two launches for the staged and batched paths (moe_q8.hip): q8gu, then q8o
void launch_moe_q8(const MoeArgs &a, hipStream_t s);
void launch_q8_bf16(const uint8_t *q8, uint16_t *bf, int hid, int inter, hipStream_t s);  // weight bytes -> bf16
bool moe_q8_supported(int hid, int inter);
void launch_moe_router(const MoeArgs &a, hipStream_t s);
void launch_moe_gateup(const MoeArgs &a, hipStream_t s);
void launch_moe_down(const MoeArgs &a, hipStream_t s);
void launch_moe_combine(const MoeArgs &a, hipStream_t s);
// The whole layer step of one row in one persistent launch (moe_fused.hip): grid = moe_fused_grid() workgroups, all
// resident together. The plan splits the gate/up and down work evenly over every wave of that grid.
struct MoePlan {
  bool ok = false;
  int grid = 0;
  std::vector<uint32_t> words;  // kPW words per workgroup: task ranges, prep keys, h blocks, per-wave unit words
  size_t part_floats = 0;
  int slots = 0;                // LDS slots (8 k tile pairs each) the busiest workgroup uses
};
int moe_fused_grid();
// q8: the 8-bit shared expert runs beside the routed work (its tagged hand-offs are added to the partials)
// slots: the LDS slots the instance has room for (moe_fused_slots)
MoePlan moe_fused_plan(int hid, int inter, int topk, int nslot, int grid, bool q8, int slots);
int moe_fused_slots(int K, int KS, int hid, int inter);  // 0: not instantiated
bool moe_fused_supported(int K, int KS, int R, int hid, int inter, int ne, int topk, bool q8 = false);
inline size_t moe_fused_sync_words(int nslot, int hid, int inter) {
  return 64 * (1 + (size_t)nslot * (inter / 128) + hid / 128);
}
void launch_moe_fused(const MoeArgs &a, int grid, hipStream_t s);
// u64 index in the fused step's partials of the 8-bit shared expert's tagged values: [2 inter] gate / up, [hid] down
size_t moe_fused_q8_index(int hid, int inter, int nslot);
const void *moe_fused_kernel(int K, int KS, int hid, int inter);  // nullptr if not instantiated
// The batched layer (moe_batch.hip) for R >= 2 rows: device buffers sized by the host for R rows.
struct MoeBatchBufs {
  uint32_t *bk = nullptr;      // [ne + 1] counts, [ne + 1] offsets, [ne + 1] cursors, 1 chunk count, 1 arrival count
  uint32_t *chunks = nullptr;  // [max_chunks][3] (expert, first sorted row, rows)
  uint32_t *rows = nullptr;    // [R nslot] sorted row -> slot r * nslot + k
  uint16_t *xh = nullptr;      // [R nslot][2][hid] prepared gate / up inputs, fp16, kp order
  uint16_t *hh = nullptr;      // [R nslot][inter] prepared down inputs
  float *dnw = nullptr;        // [R][nslot][hid] weighted slot outputs
  int max_chunks = 0;
  // few rows (moe_batch_few): the k group partials and the (chunk, block) epochs, shared by the layers of one shape
  uint64_t *vpart = nullptr;   // [chunk][2][inter / 32][4 rows][32] f32 pair sums (u64 words of storage)
  uint32_t *vep = nullptr;     // [chunk][inter / 128] counters, kSyncStride apart, zero between launches
  int vmax_chunks = 0;
};
bool moe_batch_supported(int K, int KS, int hid, int inter, int ne, int topk);
bool moe_batch_exact(const MoeArgs &a);  // the batch keeps the one-row step's arithmetic (few rows)
int moe_batch_max_chunks(int R, int ne, int topk, bool shared);
// few rows: the grouped-k kernels (R <= 32, exact arithmetic, intermediate size within their LDS); their chunk bound
// (one chunk per touched expert) and scratch
bool moe_batch_few(int R, int hid, int inter, int K, int KS);
int moe_batch_few_chunks(int R, int ne, int topk, bool shared);
size_t moe_batch_few_part(int chunks, int hid, int inter);  // u64 words of vpart
size_t moe_batch_few_epochs(int chunks, int inter);         // u32 words of vep
void launch_moe_batch(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t s);
// Fused step logits: kLogitReplicas copies of [ne + 1] floats, moe_logit_stride(ne) floats apart (replica 0 is the
// [R = 1][ne + 1] logits buffer the staged path uses); the copies spread the workgroups' polling over memory channels.
constexpr int kLogitReplicas = 32;
__host__ __device__ inline int moe_logit_stride(int ne) { return (ne + 1 + 63) / 64 * 64 + 1024; }
// The sync block for R rows: header counters, per-slot gate/up counters, per-(row, 128-column block) counters; every
// counter sits alone in a 256-byte line so that polling workgroups do not contend on one line.
constexpr int kSyncStride = 64;  // u32 words between counters
// the allocation-free linear's scratch (per GPU, for the process's lifetime): counters, prepared input, partials
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;
uint8_t *noalloc_scratch();  // this device's scratch address (taken at device set-up or the first call on it)
void launch_zero_u32(uint32_t *p, size_t n, hipStream_t s);  // p[0 .. n) = 0 by a kernel (capture-safe)
inline size_t sync_words(int R, int nslot, int hid, int inter) {
  return kSyncStride * (8 + (size_t)R * nslot + (size_t)R * ((hid + 127) / 128) +
                        (size_t)R * nslot * ((inter + 127) / 128));
}
enum { kSyncErrWord = 3 * kSyncStride };

// Fused epilogue of a linear's finished outputs v (after H_out and svh) (reference kernels/trunk6/trunk6.metal:129-197,
// t6_epi_col; rr = round to bf16 when refr): 0 y = v; 1 out_hc y = br = rr(v), e2[r][s][c] = rr(e0[r][s][c] +
// rr(br e1[r][s])) for s < hc (e0, e2 f32 [R][hc][out], e1 f32 [R][8]); 2 y = rr(silu(rr(v) / 4)); 3 y = rr(v);
// 5 y = rr(sigmoid(rr(v))); 6 y = exp(-exp(A_log[c]) softplus_rr(rr(rr(v) + dt_bias[c]))) (e0 = A_log, e1 = dt_bias,
// bf16 [out]); 7 y = v, and for c >= 512 e0[(T + r) 128 + c - 512] = v (e0 f32 cache rows of 128, e1 u32 [1] = T).
// y rows are ldy floats apart; row0 = the launch's first row among the caller's (row-grouped launches); cap = e0's
// rows of 128 for kind 7 (cache rows at or beyond it are not written).
// Kind 8 (internal to the HC read, reference trunk6.metal:223-258 t6_hc_out fused into the up linear's finisher):
// u is stored to e0 [R][4 hid] and counted per 128-column block of a stream (ctr); the last of the four streams'
// blocks writes out e2 [R][hid] from u, h (e1), the norm (w16) and inv (e4 [R][8] + 4), and, for the first block,
// the gates e4[r][0..3] from the inject partials e3 [R][4][hid / 256][4].
struct LinEpi {
  int kind = 0, refr = 1, hc = 4, ldy = 0, row0 = 0, cap = 0, hid = 0;
  float *e0 = nullptr, *e1 = nullptr, *e2 = nullptr, *e3 = nullptr, *e4 = nullptr;
  const uint16_t *w16 = nullptr;
  uint32_t *ctr = nullptr;  // kind 8: [hid / 128] (one-launch finisher), then [R][hid / 128], kSyncStride apart
};
// The HC read's input step folded into its down linear at one row (nw null: off). The linear's x is then the streams h
// [4 hid] and its input x_i (nw_i) inv_s, inv_s = 1 / rms of stream s, summed in hc_prep's order so the bits are
// hc_prep's; the workgroups of the first tile pair also store hc_prep's inject partials ip and inv_s (inj[4 + s]).
constexpr int kHcStreams = 4;
struct LinHcIn {
  const uint16_t *nw = nullptr, *iw = nullptr;
  float *ip = nullptr, *inj = nullptr;
  int hid = 0;
};
struct LinArgs {
  const uint32_t *tiles;  // re-laid trellis
  const uint16_t *suh, *svh;
  int in, out, K, IT, OT, had_in, had_out;
  float sc_in, sc_out;
  int R, S;               // rows, k groups (S = ceil(IT / kLinGroupKt): fixed by the shape, not by R)
  const float *x;
  float *y;
  uint16_t *xh;           // [R][in] prepared fp16 input (scratch)
  float *part;            // [S][R][OTp * 16] (scratch): k group partials
  uint32_t *cnt;          // per 128-column output block, kSyncStride apart, zero between launches (the block's last
                          // arriver resets it); null: the staged three-kernel path (prep, GEMM, finish)
  int xh_in;              // 1: xh holds this run's prepared rows (a prep launch ran); 0: the GEMM prepares its chunks
  int kloop;              // 1: one workgroup per tile pair loops over the k groups (S = 1: one total per pair)
  LinEpi epi;
  LinHcIn hc;
};
constexpr int kLinMaxRows = 32;
// The k order of every linear: k chunks of 8 k tiles (one MFMA chain from zero each), folded left in k groups of
// 4 chunks, the groups folded left by the finisher; a row's outputs do not depend on the other rows or on R.
constexpr int kLinChunkKt = 8, kLinGroupKt = 32;
constexpr int kLinMulti = 4;  // linears of one multi-linear launch
void launch_lin(const LinArgs &a, hipStream_t s);
// several linears at the same row count in one launch (reference kernels/trunk6/trunk6.h:78, record_multi); each its
// own input, output, scratch and epilogue. Linears of different K go to separate launches.
void launch_lin_multi(const LinArgs *a, int n, hipStream_t s);
// The hyper-connection read around its two EXL3 linears (reference models/flash_next/layer_t6.mm:89-133, t6_hc_read,
// with kernels/trunk6/t6_epi.metal:16-97): h f32 [R][4][hid], hc_norm bf16 [4 hid], inject bf16 [4][4 hid].
// hc_prep: xn [R][4 hid] = h w inv_s (inv_s = 1/rms of stream s), ip [R][4 streams][ceil(hid / 256) chunks][4
// gates] = the inject dots of h w over each chunk (times inv_s), inj[r][4 + s] = inv_s. The up linear's finisher
// (LinEpi kind 8) then writes out [R][hid] and the gates inj[r][j < 4] = rr(2 sigmoid(rr(sum_s ip[r][s][j]) / 4)).
void launch_hc_prep(const float *h, const uint16_t *nw, const uint16_t *iw, float *xn, float *ip, float *inj, int R,
                    int hid, hipStream_t s);
// raise the dynamic LDS limits of the kernels that need it: once, at device set-up (capi.cpp ensure_device)
void init_batch_attrs();
void init_fused_attrs();
void init_lin_attrs();
// W' fp16 bits [IT*16][OT*16] from re-laid tiles
void launch_decode(const uint32_t *tiles, int IT, int OT, int K, uint16_t *w, hipStream_t s);

// device-side seeded fills (synthetic packs)
void launch_fill_u32(uint32_t *p, uint64_t n, uint64_t seed, hipStream_t s);
void launch_fill_scale_f16(uint16_t *p, uint64_t n, uint64_t seed, hipStream_t s);        // +-|N(1, 0.1)|
void launch_fill_normal_bf16(uint16_t *p, uint64_t n, uint64_t seed, float stddev, hipStream_t s);
void launch_fill_q8_sb(uint32_t *p, uint64_t n, int in, uint64_t seed, hipStream_t s);  // 8-bit group words

}  // namespace ijah
