// The fused MoE decode step (one input row) in one persistent launch on CDNA4: router, top-k, the routed and shared
// experts' gate/up and down EXL3 GEMVs with SwiGLU, and the weighted combine (reference kernels/fn_moe.metal:26-452,
// driven by models/flash_next/layer.mm:532-568).
//
// One 16-wave workgroup per CU. Every wave of the grid gets, from a host-built plan, an equal slice of the layer's
// gate/up work and of its down work: consecutive k tiles of output tile pairs ("columns"), at most two segments each.
// The step:
//   1. router: wave w of workgroup b computes router row b + G w and stores its bf16 logit with this launch's tag in
//      the (always zero) low 16 bits; waves whose gate/up slice belongs to the shared expert request its tiles.
//   2. route: one wave of every workgroup waits until all logits carry the tag and ranks them itself (no exchange).
//   3. gate/up: each wave streams its slice's tiles into its own LDS area (global_load_lds), prepares the input
//      chunks it needs (x * suh, Hadamard, fp16), decodes and multiplies, and stores one partial per column segment.
//      Per (slot, 128-column block) a counter collects the partials; the workgroup that completes it sums them in
//      segment order and applies the down prologue (H, svh, SwiGLU, suh_d, H) into fp16 `hprep`.
//   4. down: each wave streams and decodes its down slice into registers while the gate/up blocks finish, waits for
//      its slot's blocks, multiplies, and stores its partials; the workgroup completing a 128-column block of the
//      output combines it: per slot the partials in segment order, H, svh and the route weight, slots in slot order.
// Cross-workgroup data moves through coherent (sc1) stores and loads; counters are single atomics per workgroup and
// target; every wait is bounded and raises the error word. The last workgroup out resets the counters and advances
// the launch epoch. All workgroups must be resident together (grid = CU count, one workgroup per CU).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "exl3_device.h"
#include "kernels.h"
#include "moe_device.h"

namespace ijah {

namespace {

constexpr int kWaves = 16;
// Control wave: the route and the counting run on the last wave, which requests no tiles before the route. Vector
// memory waits are in order, so a wave with tile streams in flight would wait for them before any load or atomic
// result of its control duty.
constexpr int kCtl = kWaves - 1;
constexpr int kMaxGu = 12;                 // gate/up k tiles per wave (its LDS area)
constexpr int kMaxDn = 8;                  // down k tiles per wave (held decoded in registers)
constexpr int kMaxSeg = 16;                // partial sums per column
constexpr int kMaxPrep = 8;                 // prepared 128-chunks of input per workgroup (shared by its waves)
constexpr int kMaxExpertsV = 1024;
constexpr int kMaxTopkV = 32;
constexpr uint32_t kSpin = 1u << 22;       // bounded waits: polls of ~0.1-1 us each, far beyond any real wait
enum { kWordErr = kSyncErrWord };  // the error word of the layer's sync block (shared with the staged kernels)
// The fused step's own counters (MoeArgs::fsync), one per 256-byte line, never reset: line 0 holds a u64 count of
// finished workgroups over all launches, so a launch's epoch e = count / grid; then fin[nslot * NBI] (gate/up
// partials per (slot, 128-column block)) and blk[NBLK] (slots stored per output block), which grow by the same
// amount T every launch and are compared as (value - e T) mod 2^32. No workgroup has to reset anything at the end.

__device__ __forceinline__ uint32_t ld_relaxed(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void mark(const MoeArgs &a, int field) {
  if (a.trace && threadIdx.x == 0) a.trace[(uint64_t)blockIdx.x * 8 + field] = wall_clock64();
}
// second trace row of the workgroup, written by lane 0 of the calling wave
__device__ __forceinline__ void mark2(const MoeArgs &a, int field) {
  if (a.trace && (threadIdx.x & 63) == 0) a.trace[(uint64_t)(256 + blockIdx.x) * 8 + field] = wall_clock64();
}
// Workgroup barrier ordering LDS (ds_*) and scalar traffic only. Outstanding vector memory operations, including the
// wave's LDS-DMA tile streams, stay in flight: __syncthreads() would wait for them (its release fence covers the LDS
// the DMA writes). Every use here exchanges only ds_write data; each wave waits for its own DMA itself.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// s_waitcnt vmcnt(n) for a run-time n: at most n vector memory operations of this wave still outstanding (n above 15
// waits as for 15, which only waits longer). Operation completion is counted in issue order.
__device__ __forceinline__ void wait_vm(int n) {
  switch (n < 15 ? n : 15) {
#define IJ_VM(k) \
  case k: __builtin_amdgcn_s_waitcnt(0x0F70 | k); break;
    IJ_VM(0) IJ_VM(1) IJ_VM(2) IJ_VM(3) IJ_VM(4) IJ_VM(5) IJ_VM(6) IJ_VM(7)
    IJ_VM(8) IJ_VM(9) IJ_VM(10) IJ_VM(11) IJ_VM(12) IJ_VM(13) IJ_VM(14) IJ_VM(15)
#undef IJ_VM
  }
}
// global_load_lds instructions a stream of `bytes` issues (one per 1 KB)
__device__ __forceinline__ int dma_ops(uint32_t bytes) { return (int)((bytes + 1023u) >> 10); }
constexpr int had_of(int d) { return d % 128 == 0 ? 128 : d % 64 == 0 ? 64 : d % 32 == 0 ? 32 : 16; }

struct Seg {  // a segment of a wave's slice: k tiles [k0, k0 + n) of column col; partial jj of that column
  int col, k0, n, jj;
};
__device__ __forceinline__ Seg seg_of(uint32_t d) {
  return {(int)(d & 0xFFFu), (int)((d >> 12) & 0xFFu), (int)((d >> 20) & 0x7Fu), (int)(d >> 27)};
}

struct Route {  // the workgroup's copy of the route of the row
  uint32_t id[kMaxTopkV];
  float w[kMaxTopkV];
  float sg;
};

// slot order in the plan (ls): the shared expert first (its work needs no route), then the routed slots k = 0..topk-1.
// Slot index j as the reference numbers it: routed k -> k, shared -> topk.
__device__ __forceinline__ int slot_j(const MoeArgs &a, int ls) {
  return a.nslot > a.topk ? (ls == 0 ? a.topk : ls - 1) : ls;
}
__device__ __forceinline__ bool slot_shared(const MoeArgs &a, int ls) { return a.nslot > a.topk && ls == 0; }
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
// Router row b + G w on wave w (reference kernels/fn_moe.metal:50-67): the bf16 row and x are loaded straight into
// registers; the logit is rounded to bf16 (the reference rounding), so its low 16 bits are zero and carry the tag.
// It goes to kLogitReplicas copies (a few KB apart), so that the workgroups polling for the logits spread over as many
// memory channels instead of all reading the same lines.
template <int HID>
__device__ __forceinline__ void router_row(const MoeArgs &a, const uint32_t *tag_lds) {
  constexpr int NC = HID / 512;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = (int)blockIdx.x + (int)gridDim.x * wave;
  const bool active = row < a.ne + a.has_sgate;
  uint4 wv[NC];
  float4 x0[NC], x1[NC];
  if (active) {
    const uint16_t *w = a.router + (uint64_t)row * HID;
#pragma unroll
    for (int j = 0; j < NC; j++) {
      wv[j] = *(const uint4 *)(w + j * 512 + lane * 8);
      x0[j] = *(const float4 *)(a.x + j * 512 + lane * 8);
      x1[j] = *(const float4 *)(a.x + j * 512 + lane * 8 + 4);
    }
  }
  lds_barrier();  // the tag (thread 0) is visible after this
  if (!active) return;
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
  const uint32_t v = (__float_as_uint(bf16_round(acc)) & 0xFFFF0000u) | *tag_lds;
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
// The route, by one wave of every workgroup (reference kernels/fn_moe.metal:76-131): waits until every logit carries
// this launch's tag (bounded), then top-k by logit with ties to the lower index, weights exp(l - l_max) / sum over the
// top k in f32 summed in slot order, and the shared gate sigmoid(logit). Each lane sorts its J keys once; a round
// takes the wave max of the lanes' heads and the winning lane shifts its list. A NaN logit ranks as -inf (weight 0).
// Workgroup 0 also writes the route to the route / shared-gate buffers for the host.
template <int J>
__device__ bool route_wave(const MoeArgs &a, Route *rt, uint32_t tag) {
  const int lane = threadIdx.x & 63, n = a.ne + a.has_sgate;
  const uint32_t *lg = (const uint32_t *)a.logits + (blockIdx.x % kLogitReplicas) * moe_logit_stride(a.ne);
  uint32_t v[J + 1];
  bool ok = false;
  for (uint32_t it = 0; it < kSpin; it++) {
    bool mine = true;
#pragma unroll
    for (int j = 0; j <= J; j++) {
      const int i = j * 64 + lane;
      v[j] = i < n ? ld_cg(lg + i) : tag;
      mine = mine && ((v[j] & 0xFFFFu) == tag);
    }
    if (__all(mine)) {
      ok = true;
      if (a.trace && lane == 0) {
        a.trace[(uint64_t)(5000 + blockIdx.x) * 8] = wall_clock64();
        a.trace[(uint64_t)(5000 + blockIdx.x) * 8 + 2] = it;
      }
      break;
    }
    if ((it & 63u) == 63u && ld_relaxed(a.sync + kWordErr)) break;
    __builtin_amdgcn_s_sleep(1);
  }
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
    if (j < J) key[j] = i < a.ne ? topk_key(val, i) : 0u;
    if (i == a.ne) sgl = val;
  }
  sgl = __shfl(sgl, a.ne & 63, 64);
  sort_desc<J>(key);
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
  if (a.trace && lane == 0) a.trace[(uint64_t)(5000 + blockIdx.x) * 8 + 1] = wall_clock64();
  const float top = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(key_value(mykey)), 0));
  const float pk = lane < a.topk ? expf(key_value(mykey) - top) : 0.f;
  float sum = 0.f;
  for (int k = 0; k < a.topk; k++) sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pk), k));
  const float wk = pk / sum;
  const float sg = moe_shared_gate(a, sgl);
  if (lane < a.topk) {
    rt->id[lane] = id;
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
  return true;
}

// ---------------------------------------------------------------------------------------------------- streaming
// n k tiles of pair p starting at k0 of a re-laid matrix with IT k tiles (tile bytes tb) into LDS at dst
__device__ __forceinline__ void stream_tiles(const uint8_t *tr, int IT, int p, int k0, int n, uint32_t tb, uint8_t *dst) {
  const int lane = threadIdx.x & 63;
  const uint8_t *src = tr + ((uint64_t)p * IT + k0) * 2 * tb;
  const uint32_t bytes = (uint32_t)n * 2 * tb;
  for (uint32_t o = 0; o < bytes; o += 1024)
    if (o + (uint32_t)lane * 16 < bytes)
      __builtin_amdgcn_global_load_lds((const void *)(src + o + lane * 16),
                                       (__attribute__((address_space(3))) void *)(dst + o), 16, 0, 0);
}
// one wave: output tile pair over k tiles [kt0, kt1) staged in LDS, on the matrix cores: the weights are decoded
// straight into the B operand of v_mfma_f32_32x32x16_f16 and A repeats the prepared input row (xs, kp order) in all
// 32 rows, so every row of the product holds the pair's 32 column sums: lanes 0-31 read them from acc[0].
template <int K>
__device__ __forceinline__ void pair_mfma_range(const uint8_t *tl, const _Float16 *xs, int kt0, int kt1, f32x16 &acc) {
  constexpr int TW = 8 * K;
  const int lane = threadIdx.x & 63;
  const BLane<K> B = b_lane<K>((uint32_t)lane);
  const uint32_t *T = (const uint32_t *)tl + B.tile * TW;
  const _Float16 *xa = xs + 8 * (lane >> 5);
#pragma unroll 4
  for (int kt = kt0; kt < kt1; kt++) {
    const uint32_t *T0 = T + kt * 2 * TW;
    TileWords w0, w1;
    w0.w0 = T0[B.g0.i0];
    w0.w1 = T0[B.g0.i1];
    w0.w2 = kThreeWords<K> ? T0[B.g0.i2] : 0u;
    w1.w0 = T0[B.g1.i0];
    w1.w1 = T0[B.g1.i1];
    w1.w2 = kThreeWords<K> ? T0[B.g1.i2] : 0u;
    const f16x8 av = *(const f16x8 *)(xa + kt * 16);
    f16x2 l0, h0, l1, h1;
    decode4<K>(w0, B.g0.sh, l0, h0);
    decode4<K>(w1, B.g1.sh, l1, h1);
    const f16x8 bv = {l0.x, l0.y, h0.x, h0.y, l1.x, l1.y, h1.x, h1.y};
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
  }
}
// decode k tiles [0, n) of the staged pair tiles into the lane's B operands w[kt] (the wave's down slice)
template <int K>
__device__ __forceinline__ void decode_b(const uint8_t *tl, int n, f16x8 (&w)[kMaxDn]) {
  constexpr int TW = 8 * K;
  const int lane = threadIdx.x & 63;
  const BLane<K> B = b_lane<K>((uint32_t)lane);
  const uint32_t *T = (const uint32_t *)tl + B.tile * TW;
#pragma unroll
  for (int kt = 0; kt < kMaxDn; kt++) {
    if (kt < n) {
      const uint32_t *T0 = T + kt * 2 * TW;
      TileWords w0, w1;
      w0.w0 = T0[B.g0.i0];
      w0.w1 = T0[B.g0.i1];
      w0.w2 = kThreeWords<K> ? T0[B.g0.i2] : 0u;
      w1.w0 = T0[B.g1.i0];
      w1.w1 = T0[B.g1.i1];
      w1.w2 = kThreeWords<K> ? T0[B.g1.i2] : 0u;
      f16x2 l0, h0, l1, h1;
      decode4<K>(w0, B.g0.sh, l0, h0);
      decode4<K>(w1, B.g1.sh, l1, h1);
      w[kt] = f16x8{l0.x, l0.y, h0.x, h0.y, l1.x, l1.y, h1.x, h1.y};
    }
  }
}
// ---------------------------------------------------------------------------------------------------- counting
// Each wave posts up to two counter indices (or ~0u) in ids[2 wave + s]; wave kCtl merges runs of equal neighbours
// and adds each run to its counter with one atomic. All threads call it (barriers inside).
__device__ void add_runs(uint32_t *ctr, const uint32_t *ids) {
  const int lane = threadIdx.x & 63;
  lds_barrier();
  if ((int)(threadIdx.x >> 6) == kCtl) {
    const bool in = lane < 2 * kWaves;
    const uint32_t id = in ? ids[lane] : ~0u;
    const uint32_t nxt = __shfl_down(id, 1, 64);
    const uint32_t prv = __shfl_up(id, 1, 64);
    const bool valid = id != ~0u;
    const bool head = valid && (lane == 0 || prv != id);
    const bool tail = valid && (lane == 2 * kWaves - 1 || nxt != id);
    const uint64_t tails = __ballot(tail);
    if (head) atomicAdd(ctr + (uint64_t)id * kSyncStride, (uint32_t)__builtin_ctzll(tails >> lane) + 1u);
  }
  lds_barrier();
}

// The partials of one output column c32 of a gate/up column, [column][kMaxSeg][32] floats: every segment slot is loaded
// (lanes of a wave read 32 consecutive floats per load; the slots past ns hold stale data and are not added), then the
// ns valid ones are summed in segment order.
struct Partials {
  float v[kMaxSeg];
};
__device__ __forceinline__ Partials load_partials(const float *p) {
  Partials r;
#pragma unroll
  for (int jj = 0; jj < kMaxSeg; jj++) r.v[jj] = ld_cg(p + jj * 32);
  return r;
}
__device__ __forceinline__ float sum_partials(const Partials &r, int ns) {
  float s = r.v[0];
#pragma unroll
  for (int jj = 1; jj < kMaxSeg; jj++) s = jj < ns ? s + r.v[jj] : s;
  return s;
}

}  // namespace

// ---------------------------------------------------------------------------------------------------- the kernel
template <int K, int KS, int HID, int INTER>
__global__ __launch_bounds__(1024, 1) void moe_step(MoeArgs a) {
  constexpr int KM = K > KS ? K : KS;
  constexpr int IT = HID / 16, ITd = INTER / 16, NPg = INTER / 32, NBI = INTER / 128,
                NBLK = HID / 128, HH = had_of(HID), HI = had_of(INTER);
  constexpr uint32_t GUB = kMaxGu * 64 * KM, AREA = GUB + kMaxDn * 64 * KM;  // a wave's gate/up + down tile bytes
  extern __shared__ __attribute__((aligned(16))) uint8_t tiles[];  // kWaves x AREA
  // the workgroup's prepared input chunks (suh by DMA, then fp16(H(x suh)) in place); later the slot's down input
  constexpr int PW = kMaxPrep * 128 > INTER ? kMaxPrep * 128 : INTER;
  __shared__ __attribute__((aligned(16))) _Float16 prepw[PW];
  __shared__ __attribute__((aligned(16))) float xl[HID];  // the input row
  __shared__ Route rt;
  __shared__ uint32_t s_tag, s_ok, s_ep, ids[2 * kWaves];
  const float sch = a.sc_hid, sci = a.sc_inter;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, G = (int)gridDim.x;
  const int NW = G * kWaves, CG = a.nslot * 2 * NPg;
  const uint32_t *plan = a.units;
  // per wave: gate/up segments s0, s1 and the index of each one's first chunk in the workgroup's prepared input;
  // per workgroup: the count of its prepared chunks and each one's (matrix << 8 | chunk)
  const uint32_t *pwp = plan + 3 * (blockIdx.x * kWaves + wave);
  const uint32_t *wpl = plan + 3 * NW + blockIdx.x * (1 + kMaxPrep);
  uint2 pw = *(const uint2 *)pwp;
  uint32_t pidx = pwp[2], np = wpl[0], pe = wpl[1 + (wave < kMaxPrep ? wave : 0)];
  pw.x = __builtin_amdgcn_readfirstlane(pw.x);  // wave-uniform: scalar registers and branches
  pw.y = __builtin_amdgcn_readfirstlane(pw.y);
  pidx = __builtin_amdgcn_readfirstlane(pidx);
  np = __builtin_amdgcn_readfirstlane(np);
  pe = __builtin_amdgcn_readfirstlane(pe);
  const bool preps = wave < (int)np;  // this wave prepares chunk `wave` of the workgroup's list
  const uint32_t *gu_nseg = plan + 3 * NW + G * (1 + kMaxPrep), *fin_tgt = gu_nseg + CG;
  uint32_t *sync = a.sync;
  uint32_t *fin_cnt = a.fsync + kSyncStride;                  // [ls * NBI + cb]: gate/up partials of a block
  uint32_t *blk_cnt = fin_cnt + a.nslot * NBI * kSyncStride;  // [c]: slots stored of output block c
  float *part_gu = a.part, *part_dn = a.part + (size_t)CG * kMaxSeg * 32;  // gate/up partials; weighted slot outputs
  uint8_t *area = tiles + wave * AREA;
  mark(a, 0);
  if (threadIdx.x == 0) {
    const uint64_t e = ld_cg((const uint64_t *)a.fsync) / (uint64_t)G;
    s_tag = (uint32_t)(e % 65535u) + 1u;  // 1..65535, never the initial 0
    s_ep = (uint32_t)e;
  }

  const Seg g0 = seg_of(pw.x), g1 = seg_of(pw.y);
  // gate/up column c = (ls * 2 + proj) * NPg + p; down column c = ls * NPd + p
  auto gu_ls = [&](const Seg &s) { return s.col / (2 * NPg); };
  auto gu_proj = [&](const Seg &s) { return (s.col / NPg) & 1; };
  auto gu_p = [&](const Seg &s) { return s.col % NPg; };
  auto tbytes = [&](int ls) { return 32u * (uint32_t)(slot_shared(a, ls) ? KS : K); };
  const uint32_t off1 = (uint32_t)g0.n * 2 * (g0.n ? tbytes(gu_ls(g0)) : 0u);  // second segment's LDS offset
  auto issue_gu = [&](const Seg &s, uint32_t off) {
    const int ls = gu_ls(s);
    stream_tiles(slot_block(a, rt, ls) + tr_off(a, ls, gu_proj(s)), IT, gu_p(s), s.k0, s.n, tbytes(ls), area + off);
  };

  // ---- 1. router; the control wave stages x in LDS; the shared expert's gate/up tiles need no route
  if (wave == kCtl) {
#pragma unroll
    for (int o = 0; o < HID * 4; o += 1024)
      __builtin_amdgcn_global_load_lds((const void *)((const uint8_t *)a.x + o + lane * 16),
                                       (__attribute__((address_space(3))) void *)((uint8_t *)xl + o), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x is in LDS before the next barrier
  }
  router_row<HID>(a, &s_tag);
  mark(a, 1);
  const bool pre0 = wave != kCtl && g0.n && slot_shared(a, gu_ls(g0));
  const bool pre1 = wave != kCtl && g1.n && slot_shared(a, gu_ls(g1));
  if (pre0) issue_gu(g0, 0);
  if (pre1) issue_gu(g1, off1);

  // ---- 2. route
  if (threadIdx.x == 0) s_ok = 1;
  lds_barrier();
  if (wave == kCtl) {
    const bool ok = a.ne <= 512 ? route_wave<8>(a, &rt, s_tag) : route_wave<16>(a, &rt, s_tag);
    if (!ok && lane == 0) s_ok = 0;
  }
  lds_barrier();
  mark(a, 2);
  const bool ok = s_ok != 0;

  // ---- 3. gate/up. Requests, in order: the suh of the chunk the wave prepares (waves below the workgroup's chunk
  // count), its gate/up tiles (unless already requested), the down tiles. Then: suh -> the prepared chunk -> a
  // barrier; each 1 KB of gate/up tiles -> the k tiles it completes.
  // down: workgroup b < nslot * NBLK owns slot ls_d's 128-column output block bd; wave w takes pair 4 bd + w / 4,
  // k quarter w % 4 (QK k tiles)
  constexpr int QK = ITd / 4;
  const bool has_dn = ok && (int)blockIdx.x < a.nslot * NBLK;
  const int ls_d = (int)blockIdx.x / NBLK, bd = (int)blockIdx.x % NBLK, dpair = bd * 4 + (wave >> 2), dq = wave & 3;
  const uint32_t gb0 = g0.n ? (uint32_t)g0.n * 2 * tbytes(gu_ls(g0)) : 0u, gb1 = g1.n ? (uint32_t)g1.n * 2 * tbytes(gu_ls(g1)) : 0u;
  const int n_g0 = (ok && !pre0) ? dma_ops(gb0) : 0, n_g1 = (ok && !pre1) ? dma_ops(gb1) : 0;
  const int n_dn = has_dn ? dma_ops((uint32_t)QK * 2 * tbytes(ls_d)) : 0;
  const int pm = (int)(pe >> 8), pc = (int)(pe & 0xFFu);  // the chunk this wave prepares: matrix, 128-chunk
  if (ok && preps && lane < 16) {  // its suh chunk (256 bytes)
    const uint8_t *src = slot_block(a, rt, pm >> 1) + su_off(a, pm >> 1, pm & 1) + pc * 256;
    __builtin_amdgcn_global_load_lds((const void *)(src + lane * 16),
                                     (__attribute__((address_space(3))) void *)(prepw + wave * 128), 16, 0, 0);
  }
  if (ok && g0.n && !pre0) issue_gu(g0, 0);
  if (ok && g1.n && !pre1) issue_gu(g1, off1);
  if (has_dn) stream_tiles(slot_block(a, rt, ls_d) + tr_off(a, ls_d, 2), ITd, dpair, dq * QK, QK, tbytes(ls_d), area + GUB);
  if (a.trace && lane == 0) a.trace[(uint64_t)(512 + blockIdx.x * kWaves + wave) * 8 + 3] = wall_clock64();
  if (ok && preps) {  // fp16(H(x * suh)) of the chunk, in kp order, in place of its suh
    wait_vm(n_g0 + n_g1 + n_dn);  // the suh chunk is in
    _Float16 *dst = prepw + wave * 128;
    const float s0 = (float)dst[lane], s1 = (float)dst[lane + 64];
    float v0 = xl[pc * 128 + lane] * s0, v1 = xl[pc * 128 + lane + 64] * s1;
    fwht2(v0, v1, lane, HH, sch);
    dst[kp(lane)] = to_f16(v0);
    dst[kp(lane + 64)] = to_f16(v1);
  }
  lds_barrier();  // every chunk of the workgroup is prepared
  if (a.trace && lane == 0) a.trace[(uint64_t)(512 + blockIdx.x * kWaves + wave) * 8 + 4] = wall_clock64();
  mark(a, 3);
  // a segment's dot, k tiles taken as each 1 KB request lands (n_after: requests issued after the segment's; stores
  // come only after both segments, so they are never counted as "after": a wait may be stricter, never looser)
  auto gu_dot = [&](const Seg &s, uint32_t off, const _Float16 *pr, int n_seg, int n_after, f32x16 &acc) {
    const _Float16 *xs = pr + (s.k0 - 8 * (s.k0 / 8)) * 16;
    const bool sh = slot_shared(a, gu_ls(s));
    const uint32_t pb = 2 * tbytes(gu_ls(s));  // bytes of one k tile pair
    int kt0 = 0;
    const int steps = n_seg > 0 ? n_seg : 1;
    for (int j = 0; j < steps; j++) {
      if (n_seg > 0) wait_vm(n_after + n_seg - 1 - j);
      if (a.trace && lane == 0 && j == steps - 1) a.trace[(uint64_t)(512 + blockIdx.x * kWaves + wave) * 8 + 1] = wall_clock64();
      if (a.trace && lane == 0 && j == 0 && n_seg > 0) a.trace[(uint64_t)(512 + blockIdx.x * kWaves + wave) * 8 + 5] = wall_clock64();
      const int kt1 = j == steps - 1 ? s.n : (int)((uint32_t)(j + 1) * 1024u / pb);
      if (kt1 > kt0) {
        if (sh)
          pair_mfma_range<KS>(area + off, xs, kt0, kt1, acc);
        else
          pair_mfma_range<K>(area + off, xs, kt0, kt1, acc);
        kt0 = kt1;
      }
    }
  };
  auto gu_store = [&](const Seg &s, const f32x16 &acc) {
    if (lane < 32) st_cg(part_gu + ((size_t)s.col * kMaxSeg + s.jj) * 32 + lane, acc[0]);  // [column][kMaxSeg][32]
  };
  f32x16 ga, gb;
#pragma unroll
  for (int i = 0; i < 16; i++) ga[i] = gb[i] = 0.f;
  if (ok && g0.n) gu_dot(g0, 0, prepw + (pidx & 0xFu) * 128, n_g0, n_g1 + n_dn, ga);
  if (ok && g1.n) gu_dot(g1, off1, prepw + ((pidx >> 4) & 0xFu) * 128, n_g1, n_dn, gb);
  if (a.trace && lane == 0) a.trace[(uint64_t)(512 + blockIdx.x * kWaves + wave) * 8 + 2] = wall_clock64();
  if (ok && g0.n) gu_store(g0, ga);
  if (ok && g1.n) gu_store(g1, gb);
  if (wave == 0) mark2(a, 0);
  __builtin_amdgcn_s_waitcnt(0);  // partials stored before they are counted
  if (wave == 0) mark2(a, 1);
  if (a.trace && lane == 0) a.trace[(uint64_t)(512 + blockIdx.x * kWaves + wave) * 8] = wall_clock64();
  if (lane == 0) {
    ids[2 * wave] = (ok && g0.n) ? (uint32_t)(gu_ls(g0) * NBI + gu_p(g0) / 4) : ~0u;
    ids[2 * wave + 1] = (ok && g1.n) ? (uint32_t)(gu_ls(g1) * NBI + gu_p(g1) / 4) : ~0u;
  }
  if (a.trace && threadIdx.x == 0) a.trace[(uint64_t)(256 + blockIdx.x) * 8 + 6] = wall_clock64();
  add_runs(fin_cnt, ids);
  mark(a, 4);
  // ---- 4. down. The workgroup of (slot ls_d, output block bd) first finishes the slot's gate/up blocks itself:
  // wave cb < NBI waits until every partial of block cb is stored, sums them in segment order and applies the down
  // prologue (reference kernels/fn_moe.metal:370-384): g = H(inner_g) svh_g, u = H(inner_u) svh_u,
  // h = H(silu(g) u suh_d) -> fp16 in kp order, into LDS. Its down slice is decoded into registers meanwhile.
  f16x8 dw[kMaxDn];
  if (has_dn) {
    if (slot_shared(a, ls_d)) decode_b<KS>(area + GUB, QK, dw);
    else decode_b<K>(area + GUB, QK, dw);
  }
  mark(a, 5);
  _Float16 *hl = prepw;  // the slot's down input, INTER halves (the prepared chunks are no longer read)
  if (has_dn && wave < NBI) {
    const int cb = wave, ls = ls_d, id = ls * NBI + cb;
    bool got = false;
    if (lane == 0) {
      for (uint32_t it = 0; it < kSpin; it++) {
        if (ld_relaxed(fin_cnt + id * kSyncStride) - s_ep * fin_tgt[id] >= fin_tgt[id]) {
          got = true;
          break;
        }
        if ((it & 63u) == 63u && ld_relaxed(sync + kWordErr)) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (!got) atomicOr(sync + kWordErr, 1u);
    }
    if (__shfl(got ? 1 : 0, 0, 64)) {
      mark2(a, 2);
      const uint8_t *blk = slot_block(a, rt, ls);
      const int i0 = cb * 128 + lane, i1 = i0 + 64;
      Partials pp[2][2];
      int ns[2][2];
#pragma unroll
      for (int proj = 0; proj < 2; proj++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int i = cb * 128 + h * 64 + lane, c = (ls * 2 + proj) * NPg + i / 32;
          pp[proj][h] = load_partials(part_gu + (size_t)c * kMaxSeg * 32 + (i & 31));
          ns[proj][h] = (int)gu_nseg[c];
        }
      const uint16_t *svg = (const uint16_t *)(blk + sv_off(a, ls, 0)), *svu = (const uint16_t *)(blk + sv_off(a, ls, 1));
      const uint16_t *sud = (const uint16_t *)(blk + su_off(a, ls, 2));
      const float sg0 = h2f(svg[i0]), sg1 = h2f(svg[i1]), su0 = h2f(svu[i0]), su1 = h2f(svu[i1]);
      const float sd0 = h2f(sud[i0]), sd1 = h2f(sud[i1]);
      float gu[2][2];
#pragma unroll
      for (int proj = 0; proj < 2; proj++)
#pragma unroll
        for (int h = 0; h < 2; h++) gu[proj][h] = sum_partials(pp[proj][h], ns[proj][h]);
      mark2(a, 3);
      float g0v = gu[0][0], g1v = gu[0][1], u0v = gu[1][0], u1v = gu[1][1];
      fwht2(g0v, g1v, lane, HI, sci);
      fwht2(u0v, u1v, lane, HI, sci);
      g0v = g0v * sg0;
      u0v = u0v * su0;
      g1v = g1v * sg1;
      u1v = u1v * su1;
      float h0 = g0v / (1.f + expf(-g0v)) * u0v * sd0;
      float h1 = g1v / (1.f + expf(-g1v)) * u1v * sd1;
      fwht2(h0, h1, lane, HI, sci);
      hl[cb * 128 + kp(lane)] = to_f16(h0);
      hl[cb * 128 + kp(lane + 64)] = to_f16(h1);
      if (bd == 0) {  // inner gate / up outputs, for reads (one workgroup per slot; nothing waits for them)
        float *gsum = a.guo + (size_t)slot_j(a, ls) * 2 * INTER;
        st_cg(gsum + i0, gu[0][0]);
        st_cg(gsum + i1, gu[0][1]);
        st_cg(gsum + INTER + i0, gu[1][0]);
        st_cg(gsum + INTER + i1, gu[1][1]);
      }
      mark2(a, 4);
    }
  }
  bool dok = has_dn;
  lds_barrier();
  mark(a, 6);
  float(*red)[32] = (float(*)[32])tiles;  // [wave][32] column sums: the tile areas are no longer read
  if (dok) {  // on the matrix cores, A = the down input repeated in all rows (as the gate/up dot)
    const _Float16 *hp = hl + dq * QK * 16 + 8 * (lane >> 5);
    f16x8 hv[kMaxDn];
#pragma unroll
    for (int kt = 0; kt < QK; kt++) hv[kt] = *(const f16x8 *)(hp + kt * 16);
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
#pragma unroll
    for (int kt = 0; kt < QK; kt++) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(hv[kt], dw[kt], acc, 0, 0, 0);
    if (lane < 32) red[wave][lane] = acc[0];
  }
  lds_barrier();
  mark(a, 7);
  if (dok && wave == 0) {
    const int j = slot_j(a, ls_d), i0 = bd * 128 + lane, i1 = i0 + 64;
    const uint16_t *sv = (const uint16_t *)(slot_block(a, rt, ls_d) + sv_off(a, ls_d, 2));
    const float s0 = h2f(sv[i0]), s1 = h2f(sv[i1]);
    float v[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {  // column 64 h + lane of the block: pair (64 h + lane) / 32, quarters in order
      const int w4 = ((h * 64 + lane) >> 5) * 4, c = lane & 31;
      v[h] = ((red[w4][c] + red[w4 + 1][c]) + red[w4 + 2][c]) + red[w4 + 3][c];
    }
    st_cg(a.dn + (size_t)j * HID + i0, v[0]);  // inner down outputs, for reads
    st_cg(a.dn + (size_t)j * HID + i1, v[1]);
    fwht2(v[0], v[1], lane, HH, sch);
    const float w = slot_shared(a, ls_d) ? rt.sg : rt.w[j];
    float *ys = part_dn + (size_t)j * HID;  // per-slot weighted outputs
    st_cg(ys + i0, v[0] * s0 * w);
    st_cg(ys + i1, v[1] * s1 * w);
    __builtin_amdgcn_s_waitcnt(0);
    uint32_t old = 0;
    if (lane == 0) old = atomicAdd(blk_cnt + bd * kSyncStride, 1u);
    old = __shfl(old, 0, 64);
    if (a.trace && lane == 0) a.trace[(uint64_t)(6001 + blockIdx.x) * 8 + 3] = wall_clock64();
    if (old - s_ep * (uint32_t)a.nslot == (uint32_t)a.nslot - 1u) {  // every slot of the block is stored: y = the sum
                                                                     // over the slots in slot order
      constexpr int U = 12;  // slots loaded in one batch
      float yv[2] = {0.f, 0.f}, sh[2] = {0.f, 0.f};  // routed sum in slot order; the shared slot
      for (int j0 = 0; j0 < a.nslot; j0 += U) {
        float t[U][2];
#pragma unroll
        for (int u = 0; u < U; u++)
          if (j0 + u < a.nslot) {
            t[u][0] = ld_cg(part_dn + (size_t)(j0 + u) * HID + i0);
            t[u][1] = ld_cg(part_dn + (size_t)(j0 + u) * HID + i1);
          }
#pragma unroll
        for (int u = 0; u < U; u++)
          if (j0 + u < a.topk) {
            yv[0] += t[u][0];
            yv[1] += t[u][1];
          } else if (j0 + u < a.nslot) {
            sh[0] = t[u][0];
            sh[1] = t[u][1];
          }
      }
      a.y[i0] = moe_finish(a, 0, i0, yv[0], sh[0]);
      a.y[i1] = moe_finish(a, 0, i1, yv[1], sh[1]);
      if (a.trace && lane == 0) a.trace[(uint64_t)(6001 + blockIdx.x) * 8 + 4] = wall_clock64();
    }
  }

  // ---- done: count this workgroup (the next launch derives its epoch from the count)
  if (threadIdx.x == 0) atomicAdd((unsigned long long *)a.fsync, 1ull);
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
  if (hid == 2048 && inter == 512) return step_for_k<2048, 512>(K, KS);
  if (hid == 1024 && inter == 256) return step_for_k<1024, 256>(K, KS);
  if (hid == 2560 && inter == 640) return step_for_k<2560, 640>(K, KS);
  return nullptr;
}
size_t step_lds(int K, int KS) { return (size_t)kWaves * (kMaxGu + kMaxDn) * 64 * std::max(K, KS); }  // = kWaves AREA
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

// Gate/up work plan. The 2 nslot gate/up matrices (m = 2 ls + proj, NPg tile-pair columns x IT k tiles each) are
// cut by k rows: workgroup b takes an equal run of the nslot * 2 * IT (matrix, k tile) rows, all NPg columns of
// them. Its kWaves / NPg waves per column split the run's k range; a run that crosses into the next matrix gives each
// wave a second segment. So a workgroup needs the prepared input of only the 128-chunks its k rows cover (one or two
// per matrix), which it computes once and shares in LDS.
MoePlan moe_fused_plan(int hid, int inter, int topk, int nslot, int G) {
  MoePlan pl;
  const int IT = hid / 16, ITd = inter / 16, NPg = inter / 32, NBI = inter / 128, NBLK = hid / 128;
  const int NW = G * kWaves, CG = nslot * 2 * NPg, NM = nslot * 2;
  const long TR = (long)NM * IT;  // k rows
  const int W = NPg > 0 && kWaves % NPg == 0 ? kWaves / NPg : 0;  // waves per column
  const long rows = (TR + G - 1) / G;
  pl.ok = W > 0 && rows <= IT && (rows + W - 1) / W <= kMaxGu && CG < 4096 && IT < 256 && ITd % 4 == 0 &&
          ITd / 4 <= kMaxDn && nslot * NBLK <= G;
  if (!pl.ok) return pl;
  std::vector<uint32_t> wv((size_t)NW * 3, 0u), prep((size_t)G * (1 + kMaxPrep), 0u), gnseg(CG, 0u);
  for (int b = 0; b < G; b++) {
    const long r0 = std::min<long>((long)b * rows, TR), r1 = std::min<long>(r0 + rows, TR);
    std::vector<uint32_t> chunks;  // (m << 8 | c), sorted
    int nseg = 0;
    for (long r = r0; r < r1;) {  // parts of the run inside one matrix
      const int m = (int)(r / IT), k0 = (int)(r % IT), kn = (int)std::min<long>(r1 - r, IT - k0);
      for (int c = k0 / 8; c <= (k0 + kn - 1) / 8; c++) chunks.push_back((uint32_t)m << 8 | (uint32_t)c);
      for (int w = 0; w < kWaves; w++) {
        const int col = m * NPg + w % NPg, sub = w / NPg;
        const int a0 = k0 + (int)((long)kn * sub / W), a1 = k0 + (int)((long)kn * (sub + 1) / W);
        if (a1 <= a0) continue;
        uint32_t *seg = &wv[((size_t)b * kWaves + w) * 3];
        const int si = seg[0] ? 1 : 0;
        if (si == 1 && seg[1]) { pl.ok = false; return pl; }
        seg[si] = (uint32_t)col | (uint32_t)a0 << 12 | (uint32_t)(a1 - a0) << 20 | gnseg[col] << 27;
        gnseg[col]++;
      }
      nseg++;
      r += kn;
    }
    if ((int)chunks.size() > kMaxPrep) { pl.ok = false; return pl; }
    prep[(size_t)b * (1 + kMaxPrep)] = (uint32_t)chunks.size();
    for (size_t i = 0; i < chunks.size(); i++) prep[(size_t)b * (1 + kMaxPrep) + 1 + i] = chunks[i];
    for (int w = 0; w < kWaves; w++) {  // each segment's first chunk in the workgroup's list
      uint32_t *seg = &wv[((size_t)b * kWaves + w) * 3];
      for (int si = 0; si < 2; si++) {
        if (!seg[si]) continue;
        const int col = (int)(seg[si] & 0xFFFu), k0 = (int)((seg[si] >> 12) & 0xFFu);
        const uint32_t key = (uint32_t)(col / NPg) << 8 | (uint32_t)(k0 / 8);
        const size_t idx = (size_t)(std::find(chunks.begin(), chunks.end(), key) - chunks.begin());
        seg[2] |= (uint32_t)idx << (4 * si);
      }
    }
    (void)nseg;
  }
  for (int c = 0; c < CG; c++)
    if (gnseg[c] > (uint32_t)kMaxSeg) { pl.ok = false; return pl; }
  std::vector<uint32_t> fin_t((size_t)nslot * NBI, 0u);
  for (int c = 0; c < CG; c++) fin_t[(c / (2 * NPg)) * NBI + (c % NPg) / 4] += gnseg[c];
  pl.words = wv;
  pl.words.insert(pl.words.end(), prep.begin(), prep.end());
  pl.words.insert(pl.words.end(), gnseg.begin(), gnseg.end());
  pl.words.insert(pl.words.end(), fin_t.begin(), fin_t.end());
  pl.part_floats = (size_t)CG * kMaxSeg * 32 + (size_t)nslot * hid;
  pl.grid = G;
  return pl;
}

bool moe_fused_supported(int K, int KS, int R, int hid, int inter, int ne, int topk) {
  return R == 1 && step_fn(K, KS, hid, inter) != nullptr && ne <= kMaxExpertsV && topk <= kMaxTopkV &&
         topk <= 64;
}

void launch_moe_fused(const MoeArgs &a, int grid, hipStream_t s) {
  const int KS = a.nslot > a.topk ? a.slay.K : a.lay.K;
  const StepFn f = step_fn(a.lay.K, KS, a.hid, a.inter);
  IJ_CHECK(f && a.R == 1, "fused MoE step not instantiated for K%d / shared K%d at %d x %d, R %d", a.lay.K, KS, a.hid,
           a.inter, a.R);
  if (grid <= 0) grid = moe_fused_grid();
  IJ_CHECK(grid * kWaves >= a.ne + a.has_sgate, "fused MoE: %d router rows on %d workgroups", a.ne + a.has_sgate, grid);
  const size_t lds = step_lds(a.lay.K, KS);
  static std::vector<StepFn> attr_set;  // functions whose dynamic LDS limit is raised already
  if (std::find(attr_set.begin(), attr_set.end(), f) == attr_set.end()) {
    IJ_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set.push_back(f);
  }
  void *args[] = {const_cast<MoeArgs *>(&a)};
  IJ_HIP(hipLaunchKernel(f, dim3(grid), dim3(64 * kWaves), args, lds, s));
}

const void *moe_fused_kernel(int K, int KS, int hid, int inter) { return step_fn(K, KS, hid, inter); }

}  // namespace ijah
