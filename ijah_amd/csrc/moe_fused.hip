// The fused MoE decode step (one input row) in one persistent launch on CDNA4: router, top-k, the routed and shared
// experts' gate/up and down EXL3 GEMVs with SwiGLU, and the weighted combine (reference kernels/fn_moe.metal:26-452,
// driven by models/flash_next/layer.mm:532-568).
//
// One 16-wave workgroup per CU, all resident. Data moves between workgroups only as tagged values: a u64 holding
// the f32 value and the launch's 32-bit tag (router logits carry a 16-bit tag in their zero low bits), stored and
// polled with device-coherent (sc1) accesses. A consumer sees the data itself arrive, so a hand-off costs one store's
// visibility (~0.45 us between XCDs), with no counters, atomics or store-completion waits in between.
//
// Work (a host-built plan; slots in plan order: the shared expert first, then the routed slots):
//   gate/up  tasks (matrix m = 2 slot + proj, group g of 4 tile-pair columns, k group of 512, tile pair): four
//            128-wide k chunks, each on a wave of its own (the SIMDs share the decode), each chunk's sum a chain of 8
//            MFMAs from zero; the chunk sums folded left, stored as the column's partial of that k group; a column's
//            value is the left fold of its k group partials. The sums do not depend on how the tasks are spread over
//            workgroups, and the batched kernels fold their k chunks the same way, so a row of a batch is
//            bit-identical to the one-row step. Workgroup b takes an equal run of the routed tasks and of the shared
//            expert's; the shared expert's tiles are requested at launch, before the route is known.
//   down     units (slot, 128-wide block cb of the intermediate, 128-column output block c, pair) of 8 k tiles, one
//            per wave: a workgroup takes an equal run. It computes the h blocks its units read (H(g) svh_g, H(u)
//            svh_u, SwiGLU, suh_d, H, fp16) from the gate/up partials itself, then stores one tagged partial per unit.
//   combine  16 workgroups, one per 128-column output block: per slot the cb partials in order, H, svh_d, the route
//            weight; the slots in slot order (the shared one last); the hyper-connection write when asked.
// The launch tag comes from a u64 epoch that workgroup 0 advances at its end with one store.
// Inside a workgroup, waves meet at barriers only where every wave's data is needed (the epoch, the route, the order
// of the requests, the combine); elsewhere an LDS flag bit per producer (prepared input chunks, h sums, h blocks) or
// a per-task LDS counter (the wave completing a task's fourth k chunk folds it) lets a wave wait only for what it
// reads. The gate/up k chunks, which every workgroup's h blocks wait for, run at raised wave priority; the down
// units' decode yields to them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

#include "exl3_device.h"
#include "kernels.h"
#include "moe_device.h"

namespace ijah {

namespace {

constexpr int kWaves = 16;
// Control wave: polls the logits and ranks them. Vector memory waits are in order, so a wave with tile streams in
// flight would wait for them before its poll results: the control wave requests no tiles before the route.
constexpr int kCtl = kWaves - 1;
constexpr int kDnKt = 8;           // k tiles of a down unit (one 128-wide h block) and of a k chunk (LDS slot size)
constexpr int kGrp = 4;            // k chunks per k group (a gate/up task: 32 k tiles of one tile pair)
constexpr int kMaxSlots = 64;      // LDS slots (8 k tile pairs each) per workgroup: at most (6-bit slot field); the
                                   // instance's LDS sets the real count (fused_slots)
constexpr int kUnitsPerWave = 4;
constexpr int kMaxGT = 10;         // gate/up tasks per workgroup (shared and routed)
constexpr int kMaxPrep = 12;       // routed prepared k chunks per workgroup (3 k groups)
constexpr int kMaxDn = 2;          // down units per wave
constexpr uint32_t kDnReuse = 1u << 22;  // down unit word: its tiles go into a gate/up chunk's slot, after that chunk
constexpr int kSpw = 8;            // the waves preparing the shared k group's chunks: kSpw .. kSpw + 3
constexpr int kMaxH = 4;           // h blocks per workgroup (2 loader waves each)
constexpr uint32_t kURouted = 1, kUShared = 2, kUDown = 3;  // unit word types (bits 31:30)
constexpr int kMaxExpertsV = 1024;
constexpr int kMaxTopkV = 16;      // the combine stages svh_d of every slot in LDS
constexpr int kPW = 128;           // plan words per workgroup (two per lane)
constexpr uint32_t kNone = ~0u;
constexpr uint32_t kSpin = 1u << 22;  // bounded waits: far beyond any real wait
enum { kWordErr = kSyncErrWord };

// plan word offsets (per workgroup)
enum {
  P_RT0 = 0, P_NRT,                    // routed gate/up tasks [rt0, rt0 + nrt) (global task index)
  P_ST0, P_NST,                        // shared gate/up tasks
  P_NRP, P_RP,                         // routed prep groups: count, then 3 keys (matrix * NKG + k group)
  P_SPK = P_RP + 3,                    // the shared tasks' prep key (proj * NKG + k group), or kNone
  P_COMB,                              // combine output block, or kNone
  P_NH, P_HB,                          // h blocks: count, then kMaxH ids (slot * NBI + cb); bit 31: store its g / u sums
  P_U = 16                             // per wave kUnitsPerWave unit words: type << 30 | LDS slot << 24 | payload
};                                     // (a k chunk of a gate/up task: prep group << 8 | task - rt0 (or - st0) << 2 |
                                       // chunk; down unit: kDnReuse | h slot << 20 | unit), or kNone

__device__ __forceinline__ uint32_t ld_relaxed(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ int dma_ops(uint32_t bytes) { return (int)((bytes + 1023u) >> 10); }
constexpr int had_of(int d) { return d % 128 == 0 ? 128 : d % 64 == 0 ? 64 : d % 32 == 0 ? 32 : 16; }
__device__ __forceinline__ uint32_t rfl(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }


// Trace mode (a.trace set; a measurement aid): per-wave wall-clock stamps kept in LDS, so that they add nothing to the
// wave's vector-memory counter (which the hand-counted waits rely on), and written out at the end of the launch:
// trace[(workgroup * 16 + wave) * 32 + field]; fields 0-7 the phases, 8-15 and 16-23 finer steps, 24-27 the route's,
// 31 the XCD the workgroup ran on.
constexpr int kTraceFields = 32;
__device__ __forceinline__ uint64_t *trace_lds() {
  __shared__ uint64_t t[kWaves * kTraceFields];
  return t;
}
__device__ __forceinline__ void stamp_at(const MoeArgs &a, int field) {
  if (a.trace && (threadIdx.x & 63) == 0) trace_lds()[(threadIdx.x >> 6) * kTraceFields + field] = wall_clock64();
}
__device__ __forceinline__ void stamp(const MoeArgs &a, int field) { stamp_at(a, field); }
__device__ __forceinline__ void stamp_w(const MoeArgs &a, int field) { stamp_at(a, 8 + field); }
__device__ __forceinline__ void stamp_x(const MoeArgs &a, int field) { stamp_at(a, 16 + field); }
__device__ __forceinline__ void stamp_r(const MoeArgs &a, int field) { stamp_at(a, 24 + field); }
__device__ __forceinline__ void trace_out(const MoeArgs &a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (a.trace && lane < kTraceFields)
    a.trace[((uint64_t)blockIdx.x * kWaves + wave) * kTraceFields + lane] = trace_lds()[wave * kTraceFields + lane];
}

struct DnUnit {  // a down unit of a wave: global unit index (-1: none) and where its data sits
  int unit = -1, slot = 0, hs = 0, end = 0, ls = 0, cb = 0, c = 0, p = 0;
  bool reuse = false, shared = false;
};

struct Route {  // the workgroup's copy of the route of the row
  uint32_t id[kMaxTopkV];
  float w[kMaxTopkV];
  float sg;
};

// plan slot ls (the shared expert first): the reference's slot index j (routed k -> k, shared -> topk)
__device__ __forceinline__ bool slot_shared(const MoeArgs &a, int ls) { return a.nslot > a.topk && ls == 0; }
__device__ __forceinline__ int slot_j(const MoeArgs &a, int ls) {
  return a.nslot > a.topk ? (ls == 0 ? a.topk : ls - 1) : ls;
}
__device__ __forceinline__ const uint8_t *slot_block(const MoeArgs &a, const Route &rt, int ls) {
  if (slot_shared(a, ls)) return a.shared;
  uint32_t e = rt.id[slot_j(a, ls)];
  e = e < (uint32_t)a.ne ? e : 0u;  // out-of-range ids clamp to expert 0, as the reference masks with NE - 1
  return a.experts + (uint64_t)e * a.lay.bytes;
}
// region offsets of a slot's block, picked with constant member indices (a dynamic index into the kernel-argument
// struct would become a vector load, and its wait would also wait for the wave's outstanding tile streams)
__device__ __forceinline__ uint64_t tr_off(const MoeArgs &a, int ls, int proj) {
  const ExpertLayout &L = slot_shared(a, ls) ? a.slay : a.lay;
  return proj == 0 ? L.tr[0] : proj == 1 ? L.tr[1] : L.tr[2];
}
__device__ __forceinline__ uint64_t su_off(const MoeArgs &a, int ls, int proj) {
  const ExpertLayout &L = slot_shared(a, ls) ? a.slay : a.lay;
  return proj == 0 ? L.su[0] : proj == 1 ? L.su[1] : L.su[2];
}
__device__ __forceinline__ uint64_t sv_off(const MoeArgs &a, int ls, int proj) {
  const ExpertLayout &L = slot_shared(a, ls) ? a.slay : a.lay;
  return proj == 0 ? L.sv[0] : proj == 1 ? L.sv[1] : L.sv[2];
}

// ---------------------------------------------------------------------------------------------------- router
// Router row b + G w on wave w (reference kernels/fn_moe.metal:50-67): the bf16 row and x straight into registers;
// the logit is rounded to bf16 (the reference rounding), so its low 16 bits are zero and carry the tag. It goes to
// kLogitReplicas copies so that the polling workgroups spread over memory channels.
template <int HID>
struct RouterRow {
  uint4 wv[HID / 512];
  float4 x0[HID / 512], x1[HID / 512];
};
template <int HID>
__device__ __forceinline__ bool router_active(const MoeArgs &a) {
  return (int)blockIdx.x + (int)gridDim.x * (int)(threadIdx.x >> 6) < a.ne + a.has_sgate;
}
template <int HID>
__device__ __forceinline__ void router_load(const MoeArgs &a, RouterRow<HID> &r) {
  constexpr int NC = HID / 512;
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x + (int)gridDim.x * (int)(threadIdx.x >> 6);
  const uint16_t *w = a.router + (uint64_t)row * HID;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    r.wv[j] = *(const uint4 *)(w + j * 512 + lane * 8);
    r.x0[j] = *(const float4 *)(a.x + j * 512 + lane * 8);
    r.x1[j] = *(const float4 *)(a.x + j * 512 + lane * 8 + 4);
  }
}
template <int HID>
__device__ __forceinline__ void router_finish(const MoeArgs &a, const RouterRow<HID> &r, uint32_t tag16) {
  constexpr int NC = HID / 512;
  const int lane = threadIdx.x & 63;
  const int row = (int)blockIdx.x + (int)gridDim.x * (int)(threadIdx.x >> 6);
  const uint4 *wv = r.wv;
  const float4 *x0 = r.x0, *x1 = r.x1;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    acc = fmaf(x0[j].x, bf16_f32(wv[j].x & 0xFFFFu), acc);
    acc = fmaf(x0[j].y, bf16_f32(wv[j].x >> 16), acc);
    acc = fmaf(x0[j].z, bf16_f32(wv[j].y & 0xFFFFu), acc);
    acc = fmaf(x0[j].w, bf16_f32(wv[j].y >> 16), acc);
    acc = fmaf(x1[j].x, bf16_f32(wv[j].z & 0xFFFFu), acc);
    acc = fmaf(x1[j].y, bf16_f32(wv[j].z >> 16), acc);
    acc = fmaf(x1[j].z, bf16_f32(wv[j].w & 0xFFFFu), acc);
    acc = fmaf(x1[j].w, bf16_f32(wv[j].w >> 16), acc);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  const uint32_t v = (__float_as_uint(bf16_round(acc)) & 0xFFFF0000u) | tag16;
  const int stride = moe_logit_stride(a.ne);
  if (lane < kLogitReplicas) st_cg((uint32_t *)a.logits + lane * stride + row, v);
}

// descending bitonic sort of J keys held in registers (J a power of two; compile-time indices)
template <int J>
__device__ __forceinline__ void sort_desc(uint32_t (&k)[J]) {
#pragma unroll
  for (int s = 2; s <= J; s <<= 1)
#pragma unroll
    for (int d = s >> 1; d > 0; d >>= 1)
#pragma unroll
      for (int i = 0; i < J; i++) {
        const int l = i ^ d;
        if (l > i) {
          const uint32_t hi = max(k[i], k[l]), lo = min(k[i], k[l]);
          if ((i & s) == 0) {
            k[i] = hi;
            k[l] = lo;
          } else {
            k[i] = lo;
            k[l] = hi;
          }
        }
      }
}
// The route, by the control wave of every workgroup (reference kernels/fn_moe.metal:76-131): waits until every logit
// carries this launch's tag (bounded), then top-k by logit with ties to the lower index, weights exp(l - l_max) / sum
// over the top k in f32 summed in slot order, and the shared gate. Each lane sorts its J keys once; a round takes the
// wave max of the lanes' heads and the winning lane shifts its list. A NaN logit ranks as -inf (weight 0).
// Only the ids are published here (every wave's requests need them); the weights and the shared gate, which only the
// combine reads, follow in route_weights from mykey (lane t < topk: the t-th largest key) and sgl (the shared gate's
// logit), after the control wave has issued its own requests.
template <int J>
__device__ bool route_wave(const MoeArgs &a, Route *rt, uint32_t tag16, uint32_t &mykey_out, float &sgl_out) {
  const int lane = threadIdx.x & 63, n = a.ne + a.has_sgate;
  const uint32_t *lg = (const uint32_t *)a.logits + (blockIdx.x % kLogitReplicas) * moe_logit_stride(a.ne);
  uint32_t v[J + 1];
  bool ok = false;
  for (uint32_t it = 0; it < kSpin; it++) {
    bool mine = true;
#pragma unroll
    for (int j = 0; j <= J; j++) {
      const int i = j * 64 + lane;
      v[j] = i < n ? ld_cg(lg + i) : tag16;
      mine = mine && ((v[j] & 0xFFFFu) == tag16);
    }
    if (__all(mine)) {
      ok = true;
      break;
    }
    if ((it & 63u) == 63u && ld_relaxed(a.sync + kWordErr)) break;
    __builtin_amdgcn_s_sleep(1);
  }
  stamp(a, 1);
  if (!ok) {
    if (lane == 0) atomicOr(a.sync + kWordErr, 1u);
    return false;
  }
  uint32_t key[J];
  float sgl = 0.f;
#pragma unroll
  for (int j = 0; j <= J; j++) {
    const int i = j * 64 + lane;
    const float val = __uint_as_float(v[j] & 0xFFFF0000u);
    if (j < J) {  // topk_key, branch-free: NaN -> -inf (max), -0 -> +0 (+ 0), then the order transform
      const uint32_t u = __float_as_uint(fmaxf(val, -INFINITY) + 0.f);
      const uint32_t k = ((u ^ ((uint32_t)((int)u >> 31) | 0x80000000u)) & 0xFFFF0000u) | (0xFFFFu - (uint32_t)i);
      key[j] = i < a.ne ? k : 0u;
    }
    if (i == a.ne) sgl = val;
  }
  sgl = __shfl(sgl, a.ne & 63, 64);
  stamp_r(a, 0);
  sort_desc<J>(key);
  stamp_r(a, 1);
  uint32_t mykey = 0u;  // lane t < topk: the t-th largest key
  for (int t = 0; t < a.topk; t++) {
    const uint32_t m = wave_max_u32(key[0]);
    mykey = lane == t ? m : mykey;
    const bool win = key[0] == m;
#pragma unroll
    for (int j = 0; j < J - 1; j++) key[j] = win ? key[j + 1] : key[j];
    key[J - 1] = win ? 0u : key[J - 1];
  }
  const uint32_t id = 0xFFFFu - (mykey & 0xFFFFu);
  if (lane < a.topk) rt->id[lane] = id;
  mykey_out = mykey;
  sgl_out = sgl;
  stamp_r(a, 2);
  return true;
}
// the route's weights and shared gate (see route_wave); workgroup 0 also writes the route to the route / shared-gate
// buffers for the host
__device__ void route_weights(const MoeArgs &a, Route *rt, uint32_t mykey, float sgl) {
  const int lane = threadIdx.x & 63;
  const uint32_t id = 0xFFFFu - (mykey & 0xFFFFu);
  const float top = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(key_value(mykey)), 0));
  const float pk = lane < a.topk ? expf(key_value(mykey) - top) : 0.f;
  float sum = 0.f;
  for (int k = 0; k < a.topk; k++) sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pk), k));
  const float wk = pk / sum;
  const float sg = moe_shared_gate(a, sgl);
  if (lane < a.topk) {
    rt->w[lane] = wk;
    if (blockIdx.x == 0) {
      st_cg(a.route + lane, id);
      st_cg(a.route + a.topk + lane, __float_as_uint(wk));
    }
  }
  if (lane == 0) {
    rt->sg = sg;
    if (blockIdx.x == 0) st_cg(a.sgv, sg);
  }
  stamp_r(a, 3);
}

// ---------------------------------------------------------------------------------------------------- tiles
// n k tiles of pair p starting at k0 of a re-laid matrix with IT k tiles (tile bytes tb) into LDS at dst; returns the
// number of 1 KB requests issued
__device__ __forceinline__ int stream_tiles(const uint8_t *tr, int IT, int p, int k0, int n, uint32_t tb, uint8_t *dst) {
  const int lane = threadIdx.x & 63;
  const uint8_t *src = tr + ((uint64_t)p * IT + k0) * 2 * tb;
  const uint32_t bytes = (uint32_t)n * 2 * tb;
  for (uint32_t o = 0; o < bytes; o += 1024)
    if (o + (uint32_t)lane * 16 < bytes)
      __builtin_amdgcn_global_load_lds((const void *)(src + o + lane * 16),
                                       (__attribute__((address_space(3))) void *)(dst + o), 16, 0, 0);
  return dma_ops(bytes);
}
// k tiles [kt0, kt1) of a staged pair times the prepared input xs (kp order, xs[16 kt] = k tile kt), on the matrix
// cores: A repeats the input row in all 32 rows, so row 0 of the product (lanes 0-31, acc[0]) holds the pair's 32
// column sums
// (at most MAXN tiles: unrolled, so that the tile and input offsets fold into the LDS reads' immediates)
template <int K, int MAXN>
__device__ __forceinline__ void pair_mfma(const uint8_t *tl, const _Float16 *xs, int kt0, int kt1, f32x16 &acc) {
  const uint8_t *t = tl + kt0 * 64 * K;
  const _Float16 *xa = xs + kt0 * 16 + 8 * ((threadIdx.x & 63) >> 5);
  const int n = kt1 - kt0;
#pragma unroll
  for (int i = 0; i < MAXN; i++) {
    if (i < n) {
      const f16x8 bv = decode_pair<K>(t, i);
      const f16x8 av = *(const f16x8 *)(xa + i * 16);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
    }
  }
}
__device__ __forceinline__ void zero16(f32x16 &v) {
#pragma unroll
  for (int i = 0; i < 16; i++) v[i] = 0.f;
}
// one 128-chunk of prepared input: fp16(H(x suh)) in kp order, from the suh chunk staged at dst (in place)
template <int HH>
__device__ __forceinline__ void prep_chunk(const float *x, int chunk, _Float16 *dst, float sc) {
  const int lane = threadIdx.x & 63;
  const float s0 = (float)dst[lane], s1 = (float)dst[lane + 64];
  float v0 = x[chunk * 128 + lane] * s0, v1 = x[chunk * 128 + lane + 64] * s1;
  fwht2(v0, v1, lane, HH, sc);
  dst[kp(lane)] = to_f16(v0);
  dst[kp(lane + 64)] = to_f16(v1);
}

// The 8-bit shared expert (reference kernels/fn_moe.metal:40-46 and :264-290). Before the route is known, wave
// kSpw + i takes gate / up row b + G i (all waves of the grid together: the 2 inter rows) and stores it tagged
// (part_q8[row]), and waves kSpw .. kSpw + 3 request their down rows b + G (i + 4 j). Those rows wait in the registers
// of the shared EXL3 down unit's operands (this form has no such unit) until the wave's gate/up chunks are done: then
// wave kSpw polls every gate and up value, computes h = rr(silu(g) u) into LDS and sets s_q8, and the four waves store
// their down rows tagged (part_q8[2 inter + row]), which the combine reads. So no wave holds the workgroup's route
// barrier, and with it every wave's routed requests, while the grid's gate and up values are on their way. The row
// arithmetic is q8_dot (moe_device.h), as in the staged and batched paths.
constexpr int kQ8GuWaves = 6, kQ8DnWaves = 4, kQ8DnPerWave = 4;
template <int HID, int INTER>
__device__ __forceinline__ void q8_gu(const MoeArgs &a, uint64_t *part_q8, uint32_t tag) {
  constexpr int NQG = (HID + 1023) / 1024;
  const int lane = threadIdx.x & 63, qi = (int)rfl(threadIdx.x >> 6) - kSpw, G = (int)gridDim.x, b = (int)blockIdx.x;
  if (qi < 0 || qi >= kQ8GuWaves) return;
  const Q8Off o = q8_offsets(HID, INTER);
  const int grow = b + G * qi;
  if (grow < 2 * INTER) {
    const int proj = grow >= INTER ? 1 : 0, r = grow - proj * INTER;
    Q8Row<NQG> w;
    q8_load<NQG>(a.q8 + o.w[proj] + (uint64_t)r * HID, (const uint32_t *)(a.q8 + o.sb[proj]) + (uint64_t)r * (HID / kQ8Group),
                 HID, w);
    const float v = q8_dot<NQG>(w, a.x, HID);
    if (lane == 0) st_tag(part_q8 + grow, moe_rr(v, a.refr), tag);
  }
}
// the down rows of wave kSpw + qi (qi < kQ8DnWaves) into st: row j's 16-byte chunk in st[j], the group words in st[4]
template <int HID, int INTER>
__device__ __forceinline__ void q8_dn_load(const MoeArgs &a, int qi, f16x8 (&st)[kDnKt]) {
  static_assert(INTER <= 1024 && kQ8DnPerWave <= 4 && kQ8DnPerWave + 1 <= kDnKt, "one chunk per row, in st");
  const int G = (int)gridDim.x, b = (int)blockIdx.x;
  const Q8Off o = q8_offsets(HID, INTER);
  uint32_t sbw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < kQ8DnPerWave; j++) {
    const int row = b + G * (qi + kQ8DnWaves * j);
    Q8Row<1> r;
    r.w[0] = make_uint4(0, 0, 0, 0);
    r.sb[0] = 0u;
    if (row < HID)
      q8_load<1>(a.q8 + o.w[2] + (uint64_t)row * INTER, (const uint32_t *)(a.q8 + o.sb[2]) + (uint64_t)row * (INTER / kQ8Group),
                 INTER, r);
    st[j] = __builtin_bit_cast(f16x8, r.w[0]);
    sbw[j] = r.sb[0];
  }
  st[kQ8DnPerWave] = __builtin_bit_cast(f16x8, make_uint4(sbw[0], sbw[1], sbw[2], sbw[3]));
}
template <int HID, int INTER>
__device__ __forceinline__ void q8_dn_finish(const MoeArgs &a, int qi, uint64_t *part_q8, uint32_t tag, float *hq,
                                             uint32_t *s_q8, const f16x8 (&st)[kDnKt]) {
  constexpr int NI = INTER / 64;
  const int lane = threadIdx.x & 63, G = (int)gridDim.x, b = (int)blockIdx.x;
  if (qi == 0) {  // every gate / up row of the grid, then h into LDS
    float gv[NI], uv[NI];
    bool got = false;
    for (uint32_t it = 0; it < kSpin; it++) {
      bool all = true;
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const uint64_t tg = ld_cg(part_q8 + lane + 64 * i), tu = ld_cg(part_q8 + INTER + lane + 64 * i);
        all = all && tag_ok(tg, tag) && tag_ok(tu, tag);
        gv[i] = tag_val(tg);
        uv[i] = tag_val(tu);
      }
      if (__all(all)) {
        got = true;
        break;
      }
      if ((it & 15u) == 15u && ld_relaxed(a.sync + kWordErr)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (!got && lane == 0) atomicOr(a.sync + kWordErr, 1u);
#pragma unroll
    for (int i = 0; i < NI; i++) hq[lane + 64 * i] = q8_act(gv[i], uv[i], a.refr);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) atomicOr(s_q8, 1u);
  }
  bool got = false;
  for (uint32_t it = 0; it < kSpin; it++) {
    if (__hip_atomic_load(s_q8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & 1u) {
      got = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!got && lane == 0) atomicOr(a.sync + kWordErr, 1u);
  asm volatile("" ::: "memory");
  const uint4 sbw = __builtin_bit_cast(uint4, st[kQ8DnPerWave]);
  const uint32_t sbs[4] = {sbw.x, sbw.y, sbw.z, sbw.w};
#pragma unroll
  for (int j = 0; j < kQ8DnPerWave; j++) {
    const int row = b + G * (qi + kQ8DnWaves * j);
    if (row < HID) {
      Q8Row<1> r;
      r.w[0] = __builtin_bit_cast(uint4, st[j]);
      r.sb[0] = sbs[j];
      const float v = q8_dot<1>(r, hq, INTER);
      if (lane == 0) st_tag(part_q8 + 2 * INTER + row, moe_rr(v, a.refr), tag);
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------------------------------- the kernel
template <int K, int KS, int HID, int INTER>
__global__ __launch_bounds__(1024, 1) void moe_step(MoeArgs a) {
  constexpr int IT = HID / 16, NP = INTER / 32, NG = NP / 4, NBI = INTER / 128, NBLK = HID / 128;
  constexpr int NKG = HID / (128 * kGrp);  // k groups
  constexpr int ITd = INTER / 16, UPS = NBI * NBLK * 4;  // down units per slot
  constexpr int HH = had_of(HID), HI = had_of(INTER);
  constexpr uint32_t SLOT = kDnKt * 64 * (K > KS ? K : KS);  // LDS bytes of one slot (8 k tile pairs)
  extern __shared__ __attribute__((aligned(16))) uint8_t tiles[];  // kMaxSlots x SLOT; the combine reuses it
  __shared__ __attribute__((aligned(16))) _Float16 prep[kMaxPrep][128];   // routed prep group i's chunk c at 4 i + c
  __shared__ __attribute__((aligned(16))) _Float16 sprep[kGrp][128];      // the shared prep group's chunks
  __shared__ __attribute__((aligned(16))) _Float16 hl[kMaxH][128];
  __shared__ float hsum[kMaxH][2][128];
  __shared__ float csum[kMaxGT][kGrp][32];                                 // k chunk sums of the gate/up tasks
  __shared__ uint32_t tcnt[kMaxGT];                                        // chunk sums of each task in LDS
  __shared__ uint32_t s_prep;                                              // prep chunks ready: routed bits 0-11, shared 16-19
  __shared__ uint32_t s_hrdy;  // h sums loaded: bit 2 h slot + proj; h block ready: bit 8 + h slot
  __shared__ __attribute__((aligned(16))) uint16_t hvec[kMaxH][3][128];   // svh_g, svh_u, suh_d of each h block
  __shared__ __attribute__((aligned(16))) uint16_t csv[kMaxTopkV + 1][128]; // the combine's svh_d per slot
  __shared__ __attribute__((aligned(16))) float xl[HID];                    // the input row (staged at launch)
  __shared__ Route rt;
  __shared__ uint32_t s_tag, s_ok, s_q8;
  __shared__ __attribute__((aligned(16))) float hq[INTER];                 // the 8-bit shared expert's h
  const int lane = threadIdx.x & 63, wave = (int)rfl(threadIdx.x >> 6);
  const int hs = a.nslot > a.topk ? 1 : 0;
  // ---- 0. every launch-time load at once, so that their latencies overlap rather than add: the router rows, the
  // epoch and x into LDS (control wave; its polls' waits cover these requests), then the workgroup's plan words (one
  // per lane, read before any tile request and picked with readlane: a vector load later would wait for the wave's
  // tile streams)
  const bool rrow = router_active<HID>(a);
  RouterRow<HID> rr;
  if (rrow) router_load<HID>(a, rr);
  uint64_t ep = 0;
  if (wave == kCtl) {
    __builtin_amdgcn_s_setprio(3);  // the route is the critical path: this wave first on its SIMD
    ep = ld_cg((const uint64_t *)a.fsync);  // every lane (one request; no branch whose end would wait for it)
    stream_tiles((const uint8_t *)a.x, 0, 0, 0, HID / 4, 8, (uint8_t *)xl);  // 4 HID bytes
  }
  const uint32_t plw0 = a.units[(size_t)blockIdx.x * kPW + lane], plw1 = a.units[(size_t)blockIdx.x * kPW + 64 + lane];
  auto PL = [&](int i) {
    return (uint32_t)(i < 64 ? __builtin_amdgcn_readlane((int)plw0, i) : __builtin_amdgcn_readlane((int)plw1, i - 64));
  };
  uint64_t *part_gu = (uint64_t *)a.part;                                   // [column][NKG groups][32]
  uint64_t *part_dn = part_gu + (size_t)a.nslot * 2 * NP * NKG * 32;        // [slot][cb][HID]
  const float sch = a.sc_hid, sci = a.sc_inter;
  // this wave's units (plan words; tiles in LDS slot `slot`): k chunks of gate/up tasks (a task: 32 k tiles of one
  // tile pair, four k chunks of 8; each chunk's sum a chain of 8 MFMAs from zero, into LDS; the task's chunk sums are
  // folded left in k order and stored as the column's partial of that k group), and at most one down unit (8 k
  // tiles: one h block)
  uint32_t uw[kUnitsPerWave];
#pragma unroll
  for (int k = 0; k < kUnitsPerWave; k++) uw[k] = PL(P_U + kUnitsPerWave * wave + k);
  const uint32_t rt0 = PL(P_RT0), st0 = PL(P_ST0), spk = PL(P_SPK), nst = PL(P_NST), nrt = PL(P_NRT);
  const int nrp = (int)PL(P_NRP), nh = (int)PL(P_NH);
  const uint32_t comb = PL(P_COMB);
  // task t (global, tile pair fastest) -> matrix (2 slot + proj for a routed one, proj for a shared one), group,
  // k group, pair
  auto task = [&](uint32_t t, int &m, int &g, int &kg, int &p) {
    p = (int)(t & 3u);
    kg = (int)((t >> 2) % NKG);
    g = (int)((t / (4 * NKG)) % NG);
    m = (int)(t / (4 * NKG * NG));
  };
  int nops = 0;  // tile / vector requests (loads) this wave has issued: waits count the ones issued after
  if (a.trace && lane < kTraceFields) trace_lds()[wave * kTraceFields + lane] = 0;
  stamp(a, 0);
  if (a.trace && (threadIdx.x & 63) == 0) {  // field 31: the XCD this workgroup runs on
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    trace_lds()[(threadIdx.x >> 6) * kTraceFields + 31] = xcc & 0xFu;
  }

  // the router logits, then the shared expert's units and its suh chunks once this workgroup's logits are out
  if (threadIdx.x == 0) s_ok = 1;
  if (threadIdx.x < kMaxGT) tcnt[threadIdx.x] = 0;
  if (threadIdx.x == 0) s_prep = 0;
  if (threadIdx.x == 0) s_hrdy = 0;
  if (threadIdx.x == 0) s_q8 = 0;
  uint32_t ep_lo = (uint32_t)ep;
  asm volatile("" : "+v"(ep_lo));  // its first use here, after the plan words' request (not at the branch's end)
  if (wave == kCtl && lane == 0) s_tag = ep_lo + 1u;
  lds_barrier();  // the epoch is known
  const uint32_t tag = s_tag, tag16 = (tag - 1u) % 65535u + 1u;
  // a k chunk's sum into LDS; the wave completing a task's fourth chunk folds the four in k order and stores the
  // column's k-group partial at once (task index: the shared tasks, then the routed ones)
  auto task_done = [&](int ti, bool sh, int c, float v) {
    if (lane < 32) csum[ti][c][lane] = v;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the sums are in LDS before the count says so
    uint32_t prev = 0;
    if (lane == 0) prev = atomicAdd(&tcnt[ti], 1u);
    prev = (uint32_t)__shfl((int)prev, 0, 64);
    asm volatile("" ::: "memory");
    if (prev != kGrp - 1) return;
    if (lane < 32) {
      int m, g, kg, p;
      task(sh ? st0 + (uint32_t)ti : rt0 + (uint32_t)ti - nst, m, g, kg, p);
      float sv = csum[ti][0][lane];
#pragma unroll
      for (int cc = 1; cc < kGrp; cc++) sv = sv + csum[ti][cc][lane];
      const uint32_t col =
          sh ? (uint32_t)(m * NP + g * 4 + p) : (uint32_t)(((hs + m / 2) * 2 + (m & 1)) * NP + g * 4 + p);
      st_tag(part_gu + ((size_t)col * NKG + kg) * 32 + lane, sv, tag);
    }
  };
  if (rrow) router_finish<HID>(a, rr, tag16);
  lds_barrier();  // this workgroup's logits are out: the router rows had HBM to themselves
  uint64_t *const part_q8 = part_dn + (size_t)a.nslot * NBI * HID;
  const int q8w = wave - kSpw;  // the 8-bit shared expert's down waves: 0 .. kQ8DnWaves - 1
  const bool q8dn = a.q8 && q8w >= 0 && q8w < kQ8DnWaves;
  f16x8 dw[kDnKt];  // the shared EXL3 down unit's B operands, or (8-bit shared expert) this wave's down rows
  if (a.q8) q8_gu<HID, INTER>(a, part_q8, tag);
  if (q8dn) q8_dn_load<HID, INTER>(a, q8w, dw);
  const bool sprep_w = spk != kNone && wave >= kSpw && wave < kSpw + kGrp;
  if (sprep_w && lane < 16) {  // chunk c of the shared prep group's suh
    const int proj = (int)(spk / NKG), kc = (int)(spk % NKG) * kGrp + (wave - kSpw);
    const uint8_t *src = a.shared + (proj ? a.slay.su[1] : a.slay.su[0]) + kc * 256;
    __builtin_amdgcn_global_load_lds((const void *)(src + lane * 16),
                                     (__attribute__((address_space(3))) void *)(sprep[wave - kSpw]), 16, 0, 0);
  }
#pragma unroll
  for (int k = 0; k < kUnitsPerWave; k++) {
    const uint32_t u = uw[k];
    if (u == kNone) continue;
    const uint32_t type = u >> 30, slot = (u >> 24) & 0x3Fu;
    if (type == kUShared) {
      int m, g, kg, p;
      task(st0 + ((u >> 2) & 0xFu), m, g, kg, p);
      stream_tiles(a.shared + (m ? a.slay.tr[1] : a.slay.tr[0]), IT, g * 4 + p, (kg * kGrp + (int)(u & 3u)) * 8, 8,
                   32u * KS, tiles + slot * SLOT);
    } else if (type == kUDown && hs && (int)(u & 0xFFFFFu) / UPS == 0) {  // the shared slot's down unit
      const int du = (int)(u & 0xFFFFFu), cb = (du / (NBLK * 4)) % NBI, c = (du / 4) % NBLK, p = du % 4;
      stream_tiles(a.shared + a.slay.tr[2], ITd, c * 4 + p, cb * kDnKt, kDnKt, 32u * KS, tiles + slot * SLOT);
    }
  }

  // ---- 1. route (control wave), shared to every wave through LDS
  uint32_t rkey = 0u;  // the control wave: its lane's route key and the shared gate's logit, for route_weights
  float rsgl = 0.f;
  if (wave == kCtl) {
    const bool ok = a.ne <= 512 ? route_wave<8>(a, &rt, tag16, rkey, rsgl) : route_wave<16>(a, &rt, tag16, rkey, rsgl);
    if (!ok && lane == 0) s_ok = 0;
    __builtin_amdgcn_s_setprio(0);  // from here on a wave like the others (it takes routed units)
    stamp(a, 2);
  } else {
    stamp(a, 1);
  }
  lds_barrier();
  if (wave != kCtl) stamp(a, 2);
  const bool ok = s_ok != 0;

  // ---- 2. requests, in the order they are consumed. A CU returns its waves' requests roughly in issue order, and a
  // wave issues all its requests before the next wave of its SIMD does: so every wave first requests the routed prep
  // chunks' suh (a workgroup barrier: every wave's, ahead of any tile stream), then its routed gate/up tasks' tiles.
  // Its routed down units' tiles and the small vectors of the later phases go out once its gate/up chunks are done,
  // so the gate/up tiles every h block waits for do not share the HBM queues with them.
  int end_u[kUnitsPerWave];  // per unit: requests issued up to and including its own
#pragma unroll
  for (int k = 0; k < kUnitsPerWave; k++) end_u[k] = 0;
  const int n_su = ok && wave < kGrp * nrp ? 1 : 0;
  if (n_su && lane < 16) {  // suh of chunk wave & 3 of routed prep group wave >> 2
    const uint32_t key = PL(P_RP + (wave >> 2));
    const int m = (int)(key / NKG), ls = hs + m / 2, kc = (int)(key % NKG) * kGrp + (wave & 3);
    const uint8_t *src = slot_block(a, rt, ls) + su_off(a, ls, m & 1) + kc * 256;
    __builtin_amdgcn_global_load_lds((const void *)(src + lane * 16),
                                     (__attribute__((address_space(3))) void *)(prep[wave]), 16, 0, 0);
  }
  nops += n_su;
  const int end_su = nops;
  stamp_w(a, 3);
  lds_barrier();  // every prep chunk's suh is requested ahead of the tile streams
  stamp_w(a, 4);
  if (ok) {
#pragma unroll
    for (int k = 0; k < kUnitsPerWave; k++) {
      const uint32_t u = uw[k];
      if (u == kNone || (u >> 30) != kURouted) continue;
      int m, g, kg, p;
      task(rt0 + ((u >> 2) & 0xFu), m, g, kg, p);
      const int ls = hs + m / 2;
      nops += stream_tiles(slot_block(a, rt, ls) + tr_off(a, ls, m & 1), IT, g * 4 + p, (kg * kGrp + (int)(u & 3u)) * 8,
                           8, 32u * K, tiles + ((u >> 24) & 0x3Fu) * SLOT);
      end_u[k] = nops;
    }
  }
  stamp_w(a, 5);
  // this wave's down units (at most kMaxDn, in plan order: a shared one comes first, its tiles requested at launch):
  // the routed ones' tiles are requested once the wave's gate/up chunks are done (into their own LDS slots, or, for
  // shapes whose units outnumber the slots, those of finished chunks); the first one is decoded before its h block
  // is ready, a second one after the first one's product is stored
  DnUnit D0, D1;
#pragma unroll
  for (int k = 0; k < kUnitsPerWave; k++)
    if (uw[k] != kNone && (uw[k] >> 30) == kUDown) {
      DnUnit &D = D0.unit < 0 ? D0 : D1;
      D.unit = (int)(uw[k] & 0xFFFFFu);
      D.hs = (int)((uw[k] >> 20) & 3u);
      D.slot = (int)((uw[k] >> 24) & 0x3Fu);
      D.reuse = (uw[k] & kDnReuse) != 0;
      D.ls = D.unit / UPS;
      D.cb = (D.unit / (NBLK * 4)) % NBI;
      D.c = (D.unit / 4) % NBLK;
      D.p = D.unit % 4;
      D.shared = hs && D.ls == 0;
    }
  auto issue_dn = [&](DnUnit &D) {
    nops += stream_tiles(slot_block(a, rt, D.ls) + tr_off(a, D.ls, 2), ITd, D.c * 4 + D.p, D.cb * kDnKt, kDnKt,
                         32u * K, tiles + D.slot * SLOT);
    D.end = nops;
  };
  // the route's weights, which only the combine reads (past later barriers), once this wave's requests are out
  if (ok && wave == kCtl) route_weights(a, &rt, rkey, rsgl);
  stamp(a, 3);
  // the shared expert while the routed tiles are on their way (its requests went out before the route): its prep
  // chunks, its k chunks and its down unit's B operands; then the routed prep (suh chunk -> fp16(H(x suh)) in kp
  // order, x from LDS: a global load now would wait for the tile streams)
  wait_vm(nops);  // the requests issued before the route
  // LDS flags (bits of s_prep, s_hrdy): a producer sets its bit after its LDS writes; a consumer waits only for the
  // bits it reads (bounded: a wait that never ends marks the launch invalid)
  auto flag_set = [&](uint32_t *w, uint32_t bit) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) atomicOr(w, bit);
  };
  auto flag_wait = [&](uint32_t *w, uint32_t bits) {
    bool got = false;
    for (uint32_t it = 0; it < kSpin; it++) {
      if ((__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & bits) == bits) {
        got = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!got && lane == 0) atomicOr(a.sync + kWordErr, 1u);
    asm volatile("" ::: "memory");
  };
  auto prep_ready = [&](uint32_t bit) { flag_set(&s_prep, bit); };
  auto prep_wait = [&](uint32_t bit) { flag_wait(&s_prep, bit); };
  if (sprep_w) {
    prep_chunk<HH>(xl, (int)(spk % NKG) * kGrp + (wave - kSpw), sprep[wave - kSpw], sch);
    prep_ready(1u << (16 + wave - kSpw));
  }
  stamp_w(a, 7);
  // ---- 3. gate/up k chunks: the shared ones (tiles in since before the route) and the shared down unit's B
  // operands while the routed tiles are on their way, then the routed ones as their tiles arrive; each chunk's sum
  // into LDS, and the fold of a task's chunk sums in k order by the wave completing it
  stamp_x(a, 0);
  // the gate/up k chunks feed every workgroup's h blocks (the step's critical path): their waves go first on their
  // SIMDs; the down units' decode, which waits for the h blocks anyway, yields to them
  __builtin_amdgcn_s_setprio(2);
  if (n_su) {
    wait_vm(nops - end_su);
    stamp_x(a, 2);
    const uint32_t key = PL(P_RP + (wave >> 2));
    prep_chunk<HH>(xl, (int)(key % NKG) * kGrp + (wave & 3), prep[wave], sch);
    prep_ready(1u << wave);
  }
  if (ok) {
#pragma unroll
    for (int k = 0; k < kUnitsPerWave; k++) {
      const uint32_t u = uw[k];
      if (u == kNone || (u >> 30) != kUShared) continue;
      const int c = (int)(u & 3u);
      prep_wait(1u << (16 + c));
      f32x16 acc;
      zero16(acc);
      pair_mfma<KS, 8>(tiles + ((u >> 24) & 0x3Fu) * SLOT, &sprep[c][0], 0, 8, acc);
      task_done((int)((u >> 2) & 0xFu), true, c, acc[0]);
    }
    if (D0.shared) {
#pragma unroll
      for (int kt = 0; kt < kDnKt; kt++) dw[kt] = decode_pair<KS>(tiles + D0.slot * SLOT, kt);
    }
  }
  if (ok) {
    constexpr uint32_t pb = 64u * K;  // bytes of one k tile pair
    bool fst = true;
#pragma unroll
    for (int k = 0; k < kUnitsPerWave; k++) {
      const uint32_t u = uw[k];
      if (u == kNone || (u >> 30) != kURouted) continue;
      const uint8_t *tl = tiles + ((u >> 24) & 0x3Fu) * SLOT;
      const int c = (int)(u & 3u);
      const _Float16 *xs = &prep[kGrp * ((u >> 8) & 3u) + c][0] + 8 * (lane >> 5);
      prep_wait(1u << (kGrp * ((u >> 8) & 3u) + c));
      const int first = end_u[k] - dma_ops(8 * pb);  // requests issued before this chunk's
      f32x16 acc;
      zero16(acc);
#pragma unroll
      for (int kt = 0; kt < 8; kt++) {
        const int req = (int)(((uint32_t)(kt + 1) * pb - 1u) >> 10);  // the request completing k tile kt
        if (kt == 0 || req != (int)(((uint32_t)kt * pb - 1u) >> 10)) wait_vm(nops - (first + req + 1));
        if (kt == 0 && fst) stamp_w(a, 0);
        const f16x8 bv = decode_pair<K>(tl, kt);
        const f16x8 av = *(const f16x8 *)(xs + kt * 16);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
      }
      task_done((int)(nst + ((u >> 2) & 0xFu)), false, c, acc[0]);
      fst = false;
    }
  }
  __builtin_amdgcn_s_setprio(0);
  stamp_w(a, 1);
  stamp(a, 4);
  if (ok) {  // the routed down units' tiles (into their own slots, or those of gate/up chunks this wave has finished)
    if (D0.unit >= 0 && !D0.shared) issue_dn(D0);
    if (D1.unit >= 0) issue_dn(D1);
  }
  if (ok) {
    // (after the gate/up chunks, as the down tiles) small vectors the later phases read, into LDS: the h prologue's svh_g, svh_u, suh_d of block `wave`; the
    // combine's svh_d of slot ls = wave (mod 16)
    if (wave < nh) {
      const uint32_t hb = PL(P_HB + wave) & 0x7FFFFFFFu;
      const int ls = (int)(hb / NBI), cb = (int)(hb % NBI);
      const uint8_t *blk = slot_block(a, rt, ls);
      const uint64_t offs[3] = {sv_off(a, ls, 0), sv_off(a, ls, 1), su_off(a, ls, 2)};
#pragma unroll
      for (int v = 0; v < 3; v++)
        if (lane < 16)
          __builtin_amdgcn_global_load_lds((const void *)(blk + offs[v] + cb * 256 + lane * 16),
                                           (__attribute__((address_space(3))) void *)(hvec[wave][v]), 16, 0, 0);
      nops += 3;
    }
    if (comb != kNone) {
      for (int ls = wave; ls < a.nslot; ls += kWaves) {
        if (lane < 16)
          __builtin_amdgcn_global_load_lds(
              (const void *)(slot_block(a, rt, ls) + sv_off(a, ls, 2) + comb * 256 + lane * 16),
              (__attribute__((address_space(3))) void *)(csv[ls]), 16, 0, 0);
        nops++;
      }
    }
  }

  // the 8-bit shared expert's down rows (their loads went out before the route), before dw takes this wave's first
  // routed down unit
  if (ok && q8dn) q8_dn_finish<HID, INTER>(a, q8w, part_q8, tag, hq, &s_q8, dw);

  // ---- 4. the first routed down unit's tiles into B operands; the h blocks from the gate/up partials (the NKG k
  // group sums of each column folded left in k order)
  if (ok && D0.unit >= 0 && !D0.shared) {
    wait_vm(nops - D0.end);
#pragma unroll
    for (int kt = 0; kt < kDnKt; kt++) dw[kt] = decode_pair<K>(tiles + D0.slot * SLOT, kt);
  }
  stamp_w(a, 2);
  // h loaders: the first 2 nh waves, which the SIMDs serve first (oldest first); wave (h slot, proj), lane: columns
  // o = lane, lane + 64 of the block
  if (ok && wave < 2 * nh) {
    __builtin_amdgcn_s_setprio(1);  // the h path comes before the down decode of other waves on this SIMD
    const int hslot = wave >> 1, proj = wave & 1;
    const uint32_t hb = PL(P_HB + hslot) & 0x7FFFFFFFu;
    const int ls = (int)(hb / NBI), cb = (int)(hb % NBI);
    const uint32_t col0 = (uint32_t)((ls * 2 + proj) * NP + cb * 4 + (lane >> 5)), col1 = col0 + 2;
    const uint64_t *src0 = part_gu + (size_t)col0 * NKG * 32 + (lane & 31);
    const uint64_t *src1 = part_gu + (size_t)col1 * NKG * 32 + (lane & 31);
    float s0 = 0.f, s1 = 0.f;
    bool got = false;
    for (uint32_t it = 0; it < kSpin; it++) {
      bool all = true;
#pragma unroll
      for (int jj = 0; jj < NKG; jj++) {
        const uint64_t t0 = ld_cg(src0 + jj * 32), t1 = ld_cg(src1 + jj * 32);
        all = all && tag_ok(t0, tag) && tag_ok(t1, tag);
        s0 = jj == 0 ? tag_val(t0) : s0 + tag_val(t0);
        s1 = jj == 0 ? tag_val(t1) : s1 + tag_val(t1);
      }
      if (__all(all)) {
        got = true;
        break;
      }
      if ((it & 15u) == 15u && ld_relaxed(a.sync + kWordErr)) break;
    }
    if (!got) atomicOr(a.sync + kWordErr, 1u);
    hsum[hslot][proj][lane] = s0;
    hsum[hslot][proj][lane + 64] = s1;
    if (PL(P_HB + hslot) >> 31) {  // the inner gate / up output, for reads
      float *gu = a.guo + ((size_t)slot_j(a, ls) * 2 + proj) * INTER + cb * 128;
      st_cg(gu + lane, s0);
      st_cg(gu + lane + 64, s1);
    }
    flag_set(&s_hrdy, 1u << wave);
  }
  stamp(a, 5);
  if (ok && wave < nh) {  // the down prologue of h block `wave` (reference kernels/fn_moe.metal:370-384)
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's svh_g / svh_u / suh_d prefetches have landed
    flag_wait(&s_hrdy, 3u << (2 * wave));  // its gate and up sums
    const uint16_t *svg = hvec[wave][0], *svu = hvec[wave][1], *sud = hvec[wave][2];
    float g0v = hsum[wave][0][lane], g1v = hsum[wave][0][lane + 64];
    float u0v = hsum[wave][1][lane], u1v = hsum[wave][1][lane + 64];
    fwht2(g0v, g1v, lane, HI, sci);
    fwht2(u0v, u1v, lane, HI, sci);
    g0v = g0v * h2f(svg[lane]);
    u0v = u0v * h2f(svu[lane]);
    g1v = g1v * h2f(svg[lane + 64]);
    u1v = u1v * h2f(svu[lane + 64]);
    float h0 = g0v / (1.f + expf(-g0v)) * u0v * h2f(sud[lane]);
    float h1 = g1v / (1.f + expf(-g1v)) * u1v * h2f(sud[lane + 64]);
    fwht2(h0, h1, lane, HI, sci);
    hl[wave][kp(lane)] = to_f16(h0);
    hl[wave][kp(lane + 64)] = to_f16(h1);
    flag_set(&s_hrdy, 1u << (8 + wave));
  }
  __builtin_amdgcn_s_setprio(0);
  // ---- 5. down: 8 k tiles of h against the unit's decoded tiles; one tagged partial per unit
  auto down_unit = [&](const DnUnit &D) {
    flag_wait(&s_hrdy, 1u << (8 + D.hs));  // its h block
    f32x16 d;
    zero16(d);
    const _Float16 *ha = &hl[D.hs][0] + 8 * (lane >> 5);
#pragma unroll
    for (int kt = 0; kt < kDnKt; kt++)
      d = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const f16x8 *)(ha + kt * 16), dw[kt], d, 0, 0, 0);
    if (lane < 32) st_tag(part_dn + ((size_t)D.ls * NBI + D.cb) * HID + D.c * 128 + D.p * 32 + lane, d[0], tag);
  };
  if (ok && D0.unit >= 0) down_unit(D0);
  if (ok && D1.unit >= 0) {  // a routed unit (the plan gives a wave at most one shared down unit, first)
    wait_vm(nops - D1.end);
#pragma unroll
    for (int kt = 0; kt < kDnKt; kt++) dw[kt] = decode_pair<K>(tiles + D1.slot * SLOT, kt);
    down_unit(D1);
  }
  stamp(a, 6);

  // ---- 7. combine of output block c (16 workgroups): per slot the cb partials in order -> H, svh_d, weight; the
  // slots in slot order (routed, then the shared one) -> y (reference kernels/fn_moe.metal:420-450)
  if (ok && comb != kNone) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the svh_d prefetches of every wave have landed
    const int c = (int)comb, o = threadIdx.x & 127;
    float *cv = (float *)tiles;  // [nslot][128]
    // thread: column o, slots g, g + 8, g + 16 (g = t / 128), all polled together
    const int g = threadIdx.x >> 7;
    const uint64_t *src = part_dn + c * 128 + o;
    const uint64_t *qsrc = part_dn + (size_t)a.nslot * NBI * HID + 2 * INTER + c * 128 + o;  // 8-bit shared o
    const bool qpoll = a.q8 && g == 0;
    float sv[3] = {0.f, 0.f, 0.f}, qv = 0.f;
    bool got = false;
    for (uint32_t it = 0; it < kSpin; it++) {
      bool all = true;
      if (qpoll) {
        const uint64_t t = ld_cg(qsrc);
        all = tag_ok(t, tag);
        qv = tag_val(t);
      }
#pragma unroll
      for (int q = 0; q < 3; q++) {
        const int ls = g + 8 * q;
        if (ls < a.nslot) {
#pragma unroll
          for (int cb = 0; cb < NBI; cb++) {
            const uint64_t t = ld_cg(src + ((size_t)ls * NBI + cb) * HID);
            all = all && tag_ok(t, tag);
            sv[q] = cb == 0 ? tag_val(t) : sv[q] + tag_val(t);
          }
        }
      }
      if (__all(all)) {
        got = true;
        break;
      }
      if ((it & 15u) == 15u && ld_relaxed(a.sync + kWordErr)) break;
    }
    if (!got) atomicOr(a.sync + kWordErr, 1u);
    lds_barrier();  // every wave is past its decodes: the tiles' LDS is free for the combine
#pragma unroll
    for (int q = 0; q < 3; q++)
      if (g + 8 * q < a.nslot) cv[(g + 8 * q) * 128 + o] = sv[q];
    lds_barrier();
    for (int ls = wave; ls < a.nslot; ls += kWaves) {
      const int j = slot_j(a, ls), i0 = c * 128 + lane, i1 = i0 + 64;
      float v0 = cv[ls * 128 + lane], v1 = cv[ls * 128 + lane + 64];
      st_cg(a.dn + (size_t)j * HID + i0, v0);  // inner down outputs, for reads
      st_cg(a.dn + (size_t)j * HID + i1, v1);
      fwht2(v0, v1, lane, HH, sch);
      const float w = slot_shared(a, ls) ? rt.sg : rt.w[j];
      cv[ls * 128 + lane] = v0 * h2f(csv[ls][lane]) * w;
      cv[ls * 128 + lane + 64] = v1 * h2f(csv[ls][lane + 64]) * w;
    }
    lds_barrier();
    if (wave < 2) {
      const int i = c * 128 + wave * 64 + lane, oo = wave * 64 + lane;
      float yv = 0.f;
      for (int k = 0; k < a.topk; k++) yv += cv[(hs + k) * 128 + oo];
      const float sh = hs ? cv[oo] : a.q8 ? rt.sg * qv : 0.f;
      a.y[i] = moe_finish(a, 0, i, yv, sh);
    }
  }
  stamp(a, 7);
  trace_out(a);
  // ---- done: workgroup 0 advances the epoch (one store). It finishes only after every workgroup published its
  // router logit, i.e. after every workgroup read this launch's epoch.
  if (blockIdx.x == 0 && threadIdx.x == 0) st_cg((uint64_t *)a.fsync, (uint64_t)tag);
}

// ---------------------------------------------------------------------------------------------------- host side
namespace {
using StepFn = const void *;
template <int HID, int INTER>
StepFn step_for_k(int K, int KS) {
#define IJ_STEP(k, ks) \
  if (K == k && KS == ks) return (StepFn)&moe_step<k, ks, HID, INTER>;
  IJ_STEP(4, 4) IJ_STEP(5, 5) IJ_STEP(6, 6) IJ_STEP(4, 6) IJ_STEP(5, 6) IJ_STEP(4, 5)
#undef IJ_STEP
  return nullptr;
}
StepFn step_fn(int K, int KS, int hid, int inter) {
  if (hid == 2560 && inter == 640) return step_for_k<2560, 640>(K, KS);  // the reference's own shape
  if (hid == 2048 && inter == 512) return step_for_k<2048, 512>(K, KS);
  if (hid == 1024 && inter == 256) return step_for_k<1024, 256>(K, KS);
  return nullptr;
}
uint32_t slot_bytes(int K, int KS) { return kDnKt * 64 * std::max(K, KS); }
}  // namespace

int moe_fused_grid() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    IJ_HIP(hipGetDevice(&dev));
    IJ_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  return cus;
}

// The work plan (see the kernel's header). Returns ok = false when the shape does not fit the kernel's per-wave
// limits; the layer then runs the staged path.
MoePlan moe_fused_plan(int hid, int inter, int topk, int nslot, int G, bool q8, int slots) {
  MoePlan pl;
  slots = std::min(slots, kMaxSlots);
  const int NP = inter / 32, NG = NP / 4, NBI = inter / 128, NBLK = hid / 128, UPS = NBI * NBLK * 4;
  const int NKG = hid / (128 * kGrp), hs = nslot > topk ? 1 : 0, NCOL = nslot * 2 * NP;
  if (inter % 128 || hid % (128 * kGrp) || G < 1 || NBLK > G) return pl;
  std::vector<uint32_t> w((size_t)G * kPW, kNone);
  // gate/up tasks (matrix, group, k group, pair; pair fastest): routed and shared; down units: shared, routed
  const long TR = (long)topk * 2 * NG * NKG * 4, TS = hs ? 2L * NG * NKG * 4 : 0;
  const long US = hs ? UPS : 0, UR = (long)topk * UPS;
  auto key_of = [&](long t) { return (uint32_t)((t / (4L * NKG * NG)) * NKG + (t / 4) % NKG); };  // matrix, k group
  std::vector<int> hb_first((size_t)nslot * NBI, -1);
  int used = 0;  // LDS slots the busiest workgroup needs
  // output block c combines on workgroup c G / NBLK + c % 8: spread over the grid and, as workgroups go to the 8
  // XCDs in turn, over the XCDs (c G / NBLK alone is a multiple of 8 at G = 256, NBLK = 16: all on one XCD, whose
  // link then carries every combine's polls)
  auto comb_b = [&](int c) { return c * G / NBLK + (G >= 8 * NBLK ? c % 8 : 0); };
  // the combining workgroups take no routed down unit: the combine waits for the last down partial, so they poll
  // from early on instead of storing some of the last
  // (only while that leaves every other wave at most one down unit: a second one is decoded after the first one's
  // product is stored, on the step's tail)
  std::vector<char> comb_wg(G, 0);
  if (G >= 2 * NBLK && UR + US <= (long)(G - NBLK) * kWaves)
    for (int c = 0; c < NBLK; c++) comb_wg[comb_b(c)] = 1;
  std::vector<long> ur0(G + 1, 0);  // routed down units [ur0[b], ur0[b + 1]) of workgroup b
  {
    long nw = 0;
    for (int b = 0; b < G; b++) nw += comb_wg[b] ? 0 : 1;
    long k = 0;
    for (int b = 0; b < G; b++) {
      ur0[b] = UR * k / nw;
      k += comb_wg[b] ? 0 : 1;
    }
    ur0[G] = UR;
  }
  for (int b = 0; b < G; b++) {
    uint32_t *pw = &w[(size_t)b * kPW];
    const long t0 = TR * b / G, t1 = TR * (b + 1) / G, s0 = TS * b / G, s1 = TS * (b + 1) / G;
    if (t1 - t0 > 16 || s1 - s0 > 16) return pl;
    pw[P_RT0] = (uint32_t)t0;
    pw[P_NRT] = (uint32_t)(t1 - t0);
    pw[P_ST0] = (uint32_t)s0;
    pw[P_NST] = (uint32_t)(s1 - s0);
    // prep groups: the distinct (matrix, k group) of the routed run (at most 3); one of the shared run
    std::vector<uint32_t> keys;
    for (long t = t0; t < t1; t++)
      if (std::find(keys.begin(), keys.end(), key_of(t)) == keys.end()) keys.push_back(key_of(t));
    if ((int)keys.size() * kGrp > kMaxPrep) return pl;
    pw[P_NRP] = (uint32_t)keys.size();
    for (size_t i = 0; i < keys.size(); i++) pw[P_RP + i] = keys[i];
    for (long t = s0; t < s1; t++)
      if (key_of(t) != key_of(s0)) return pl;
    if (s1 > s0) pw[P_SPK] = key_of(s0);
    int slot = 0;
    std::vector<int> nu(kWaves, 0), simd(4, 0), ndn(kWaves, 0);
    std::vector<std::vector<uint32_t>> rs(kWaves);  // per wave: LDS slots of its routed chunks, free for a down unit
    // every unit (a k chunk or a down unit: 8 k tile pairs to decode) goes to the wave whose SIMD has the least routed
    // work so far (then the wave with the fewest units): after the route the decode is the step's VALU bound, and a
    // SIMD's waves share it. The shared expert's units (requested before the route) go to waves kSpw .. kCtl - 1: not the control
    // wave (it polls the logits meanwhile) and not the routed prep waves (their prep gates the routed chunks). A down
    // unit goes to a wave without one if any can take it (a wave holds at most kMaxDn, a shared one only as its
    // first); once the LDS slots run out, a routed down unit takes a slot of one of its wave's routed chunks (its
    // tiles are requested after that chunk is done).
    auto put = [&](bool pre_route, uint32_t word) {
      const uint32_t type = word >> 30;
      const bool dn = type == kUDown, reuse = dn && !pre_route && slot >= slots;
      int best = -1;
      for (int w = pre_route ? kSpw : 0; w < (pre_route ? kCtl : kWaves); w++) {
        if (nu[w] >= kUnitsPerWave || (dn && ndn[w] >= (pre_route ? 1 : kMaxDn)) || (reuse && rs[w].empty())) continue;
        const bool fewer_dn = dn && best >= 0 && ndn[w] < ndn[best];
        const bool same_dn = !dn || best < 0 || ndn[w] == ndn[best];
        if (best < 0 || fewer_dn ||
            (same_dn && (simd[w % 4] < simd[best % 4] || (simd[w % 4] == simd[best % 4] && nu[w] < nu[best]))))
          best = w;
      }
      if (best < 0) return -1;
      uint32_t sl;
      if (reuse) {
        sl = rs[best].front();
        rs[best].erase(rs[best].begin());
        word |= kDnReuse;
      } else {
        if (slot >= slots) return -1;
        sl = (uint32_t)slot++;
      }
      pw[P_U + kUnitsPerWave * best + nu[best]++] = word | sl << 24;
      if (type == kURouted) rs[best].push_back(sl);
      simd[best % 4] += pre_route ? 0 : 1;  // the shared units run while the routed tiles are on their way
      ndn[best] += dn ? 1 : 0;
      used = std::max(used, slot);
      return best;
    };
    // gate/up tasks: the shared ones first (requested before the route), then the routed ones
    if ((s1 - s0) + (t1 - t0) > kMaxGT) return pl;
    for (long t = s0; t < s1; t++)
      for (int c = 0; c < kGrp; c++)
        if (put(true, kUShared << 30 | (uint32_t)(t - s0) << 2 | (uint32_t)c) < 0) return pl;
    for (long t = t0; t < t1; t++) {
      const uint32_t pg = (uint32_t)(std::find(keys.begin(), keys.end(), key_of(t)) - keys.begin());
      for (int c = 0; c < kGrp; c++)
        if (put(false, kURouted << 30 | pg << 8 | (uint32_t)(t - t0) << 2 | (uint32_t)c) < 0) return pl;
    }
    // down units (global unit index: the shared slot's first)
    std::vector<long> units;
    for (long u = US * b / G; u < US * (b + 1) / G; u++) units.push_back(u);
    for (long u = ur0[b]; u < ur0[b + 1]; u++) units.push_back(US + u);
    std::vector<uint32_t> hbs;
    for (size_t i = 0; i < units.size(); i++) {
      const long u = units[i];
      const uint32_t id = (uint32_t)((u / UPS) * NBI + (u / (NBLK * 4)) % NBI);
      size_t h = 0;
      while (h < hbs.size() && hbs[h] != id) h++;
      if (h == hbs.size()) hbs.push_back(id);
      if (h >= (size_t)kMaxH) return pl;
      if (put(u < US, kUDown << 30 | (uint32_t)h << 20 | (uint32_t)u) < 0) return pl;
    }
    pw[P_NH] = (uint32_t)hbs.size();
    for (size_t i = 0; i < hbs.size(); i++) {
      uint32_t v = hbs[i];
      if (hb_first[hbs[i]] < 0) {  // the first workgroup computing an h block also stores its g / u sums
        hb_first[hbs[i]] = b;
        v |= 1u << 31;
      }
      pw[P_HB + i] = v;
    }
  }
  for (int c = 0; c < NBLK; c++) w[(size_t)comb_b(c) * kPW + P_COMB] = (uint32_t)c;
  pl.words = w;
  // tagged partials (u64 = 2 floats): gate/up [column][NKG k groups][32], down [slot][cb][hid]
  // and, with the 8-bit shared expert, its gate / up [2 inter] and down [hid] rows
  pl.part_floats = 2 * ((size_t)NCOL * NKG * 32 + (size_t)nslot * NBI * hid + (q8 ? 2 * (size_t)inter + hid : 0));
  pl.grid = G;
  pl.slots = used;
  pl.ok = true;
  return pl;
}

size_t moe_fused_q8_index(int hid, int inter, int nslot) {
  const size_t NCOL = (size_t)nslot * 2 * (inter / 32), NKG = hid / (128 * kGrp), NBI = inter / 128;
  return NCOL * NKG * 32 + (size_t)nslot * NBI * hid;
}

bool moe_fused_supported(int K, int KS, int R, int hid, int inter, int ne, int topk, bool q8) {
  const int G = moe_fused_grid();
  const bool q8ok = !q8 || (moe_q8_supported(hid, inter) && 2 * inter <= kQ8GuWaves * G &&
                            hid <= kQ8DnWaves * kQ8DnPerWave * G);
  return R == 1 && step_fn(K, KS, hid, inter) != nullptr && ne <= kMaxExpertsV && topk <= kMaxTopkV && q8ok;
}

void launch_moe_fused(const MoeArgs &a, int grid, hipStream_t s) {
  const int KS = a.nslot > a.topk ? a.slay.K : a.lay.K;
  const StepFn f = step_fn(a.lay.K, KS, a.hid, a.inter);
  IJ_CHECK(f && a.R == 1, "fused MoE step not instantiated for K%d / shared K%d at %d x %d, R %d", a.lay.K, KS, a.hid,
           a.inter, a.R);
  if (grid <= 0) grid = moe_fused_grid();
  IJ_CHECK(grid * kWaves >= a.ne + a.has_sgate, "fused MoE: %d router rows on %d workgroups", a.ne + a.has_sgate, grid);
  IJ_CHECK(a.units && a.part && a.fsync, "fused MoE: no plan");
  IJ_CHECK(a.fused_slots > 0 && a.fused_slots <= moe_fused_slots(a.lay.K, KS, a.hid, a.inter),
           "fused MoE: %d LDS slots planned", a.fused_slots);
  const size_t lds = (size_t)a.fused_slots * slot_bytes(a.lay.K, KS);  // (limit raised by init_fused_attrs)
  void *args[] = {const_cast<MoeArgs *>(&a)};
  IJ_HIP(hipLaunchKernel(f, dim3(grid), dim3(64 * kWaves), args, lds, s));
}

const void *moe_fused_kernel(int K, int KS, int hid, int inter) { return step_fn(K, KS, hid, inter); }

// The LDS slots an instance has room for: the CU's 160 KB less its static LDS, in slots of 8 k tile pairs (at most
// kMaxSlots, the slot field's range).
constexpr size_t kCuLds = 160 * 1024;
int moe_fused_slots(int K, int KS, int hid, int inter) {
  const StepFn f = step_fn(K, KS, hid, inter);
  if (!f) return 0;
  static std::mutex mu;
  static std::map<const void *, int> cache;
  std::lock_guard<std::mutex> g(mu);
  auto it = cache.find(f);
  if (it != cache.end()) return it->second;
  hipFuncAttributes at;
  IJ_HIP(hipFuncGetAttributes(&at, f));
  const int n = (int)std::min<size_t>(kMaxSlots, (kCuLds - at.sharedSizeBytes) / slot_bytes(K, KS));
  cache[f] = n;
  return n;
}

// every instance's dynamic LDS limit, once at device set-up (never inside a stream capture)
void init_fused_attrs() {
  for (int hid : {1024, 2048, 2560})
    for (int K = 4; K <= 6; K++)
      for (int KS = 4; KS <= 6; KS++)
        if (const StepFn f = step_fn(K, KS, hid, hid / 4))
          IJ_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)(moe_fused_slots(K, KS, hid, hid / 4) * slot_bytes(K, KS))));
}

}  // namespace ijah
