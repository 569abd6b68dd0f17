// EXL3 kernels: trellis decode, trunk GEMV, the staged MoE layer and the device-side fills (CDNA4, wave64).
// The format, the wave64 lane mapping and the Hadamard order are described in exl3_device.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "exl3_device.h"
#include "kernels.h"
#include "moe_device.h"

namespace ijah {

// ------------------------------------------------------------------------------------------------ layouts
static uint64_t align256(uint64_t n) { return (n + 255u) & ~(uint64_t)255u; }

ExpertLayout expert_layout(int hid, int inter, int K) {
  ExpertLayout L;
  L.K = K;
  const uint64_t tile = 32u * (uint64_t)K;
  const int dims[3][2] = {{hid, inter}, {hid, inter}, {inter, hid}};
  uint64_t o = 0;
  for (int p = 0; p < 3; p++) {
    const int IT = dims[p][0] / 16, OT = dims[p][1] / 16, OTp = OT + (OT & 1);
    L.tr[p] = o;
    o = align256(o + (uint64_t)IT * OTp * tile);
  }
  for (int p = 0; p < 3; p++) {
    L.su[p] = o;
    o = align256(o + 2u * (uint64_t)dims[p][0]);
    L.sv[p] = o;
    o = align256(o + 2u * (uint64_t)dims[p][1]);
  }
  L.bytes = o;
  return L;
}

// ------------------------------------------------------------------------------------------------ shared GEMV core
// A workgroup (4 waves) multiplies the LDS-staged prepared input (fp16, kp order; xs[0] = input row 16*k0) with
// output tiles (2p, 2p+1) over k tiles [k0, k1) of a re-laid matrix; wave w takes k tiles k0 + w + 4j. The tile words
// of up to kPrefetch iterations are loaded into registers in one batch (pair_load) so that their HBM latency overlaps
// the caller's input preparation; pair_dot then decodes and accumulates. Per lane: partial sums of its column for the
// two tiles, reduced over the four lanes sharing the column.
constexpr int kPrefetch = 8;
template <int K>
struct PairBuf {
  TileWords w[kPrefetch][2];
};
template <int K>
__device__ __forceinline__ void pair_load(PairBuf<K> &b, const uint32_t *__restrict__ pair_base, const TileLane<K> &L,
                                          int tk0, int k1) {
  constexpr int TW = 8 * K;
#pragma unroll
  for (int j = 0; j < kPrefetch; j++) {
    const int tk = tk0 + 4 * j;
    if (tk < k1) {
      const uint32_t *T0 = pair_base + (uint64_t)tk * 2 * TW;
      b.w[j][0] = load_tile<K>(T0, L);
      b.w[j][1] = load_tile<K>(T0 + TW, L);
    }
  }
}
template <int K>
__device__ __forceinline__ void pair_dot(const PairBuf<K> &b, const TileLane<K> &L, int tk0, int k0, int k1,
                                         const _Float16 *xs, float &acc0, float &acc1) {
  const int q = ((threadIdx.x & 63) >> 1) & 3;
#pragma unroll
  for (int j = 0; j < kPrefetch; j++) {
    const int tk = tk0 + 4 * j;
    if (tk < k1) {
      const f16x4 xv = *(const f16x4 *)(xs + (tk - k0) * 16 + 4 * q);
      f16x2 a0, b0, a1, b1;
      decode4<K>(b.w[j][0], L.sh, a0, b0);
      decode4<K>(b.w[j][1], L.sh, a1, b1);
      acc0 = dot4(a0, b0, xv, acc0);
      acc1 = dot4(a1, b1, xv, acc1);
    }
  }
}
// The whole pair GEMV for spans beyond one prefetch batch; `b` already holds the first batch (loaded by the caller
// before its prologue).
template <int K>
__device__ __forceinline__ void pair_gemv(PairBuf<K> &b, const uint32_t *__restrict__ pair_base, const TileLane<K> &L,
                                          int k0, int k1, const _Float16 *xs, float &acc0, float &acc1) {
  const int tkw = k0 + (int)(threadIdx.x >> 6);
  acc0 = 0.f;
  acc1 = 0.f;
  for (int tk0 = tkw; tk0 < k1; tk0 += 4 * kPrefetch) {
    if (tk0 != tkw) pair_load<K>(b, pair_base, L, tk0, k1);
    pair_dot<K>(b, L, tk0, k0, k1, xs, acc0, acc1);
  }
  lane_col_reduce(acc0, acc1);
}

// sums the 4 waves' column partials in a fixed order; result on threads 0..31 (column 32p + tid)
__device__ __forceinline__ float pair_reduce(float acc0, float acc1, float *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = (lane >> 3) + 8 * (lane & 1);
  if ((lane & 6) == 0) {
    red[wave * 32 + col] = acc0;
    red[wave * 32 + 16 + col] = acc1;
  }
  __syncthreads();
  float s = 0.f;
  if (threadIdx.x < 32) s = (red[threadIdx.x] + red[32 + threadIdx.x]) + (red[64 + threadIdx.x] + red[96 + threadIdx.x]);
  return s;
}

#define IJ_DISPATCH_K(K_, CALL)                     \
  switch (K_) {                                    \
    case 2: { constexpr int KK = 2; CALL; } break; \
    case 3: { constexpr int KK = 3; CALL; } break; \
    case 4: { constexpr int KK = 4; CALL; } break; \
    case 5: { constexpr int KK = 5; CALL; } break; \
    case 6: { constexpr int KK = 6; CALL; } break; \
    case 7: { constexpr int KK = 7; CALL; } break; \
    case 8: { constexpr int KK = 8; CALL; } break; \
    default: break;                                \
  }

// ------------------------------------------------------------------------------------------------ MoE: D1 router
// Router GEMV (reference kernels/fn_moe.metal:50-67): one wave per router row (ne experts + the shared-expert gate row
// when present), logits rounded to bf16 (the reference rounding). The last workgroup to arrive (atomic counter, reset
// by it for the next launch / graph replay) ranks the logits and writes the route (kernels/fn_moe.metal:76-131):
// top-k by logit, the lower index first on ties, weights exp(l - l_max) / sum over the top k in f32 (summed in slot
// order), and the shared gate sigmoid(logit).
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopk = 32;

// ------------------------------------------------------------------------------------------------ top-k
// Top-k of lv[0..ne) (bf16-valued, ne <= 1024, k <= 32): wave 0 holds 16 keys per lane and runs k rounds of
// wave max + clear; ids land in sid[0..k) in order. All threads of the block call it (barrier at the end).
__device__ void block_topk(const float *lv, int ne, int k, uint32_t *cand, uint32_t *sid) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  (void)cand;
  if (wave == 0) {
    uint32_t key[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int i = j * 64 + lane;
      key[j] = i < ne ? topk_key(lv[i], i) : 0u;
    }
    for (int t = 0; t < k; t++) {
      uint32_t m = 0u;
#pragma unroll
      for (int j = 0; j < 16; j += 2) m = max(m, max(key[j], key[j + 1]));
      m = wave_max_u32(m);
      if (lane == 0) sid[t] = 0xFFFFu - (m & 0xFFFFu);
#pragma unroll
      for (int j = 0; j < 16; j++) key[j] = key[j] == m ? 0u : key[j];
    }
  }
  __syncthreads();
}

// slot (row r, k): routed expert route[r][k] (ids past ne clamp to 0, as the reference masks with NE - 1) or the
// shared expert (k == topk). Offsets are picked as scalars so no layout struct is copied to scratch.
struct SlotRef {
  const uint8_t *blk;
  int K, sh;
};
__device__ __forceinline__ SlotRef slot_ref(const MoeArgs &a, int r, int k) {
  SlotRef s;
  if (k < a.topk) {
    uint32_t e = ld_cg(a.route + (uint64_t)r * 2 * a.topk + k);
    e = e < (uint32_t)a.ne ? e : 0u;
    s.blk = a.experts + (uint64_t)e * a.lay.bytes;
    s.K = a.lay.K;
    s.sh = 0;
  } else {
    s.blk = a.shared;
    s.K = a.slay.K;
    s.sh = 1;
  }
  return s;
}
__device__ __forceinline__ uint64_t off_tr(const MoeArgs &a, int sh, int p) { return sh ? a.slay.tr[p] : a.lay.tr[p]; }
__device__ __forceinline__ uint64_t off_su(const MoeArgs &a, int sh, int p) { return sh ? a.slay.su[p] : a.lay.su[p]; }
__device__ __forceinline__ uint64_t off_sv(const MoeArgs &a, int sh, int p) { return sh ? a.slay.sv[p] : a.lay.sv[p]; }

// ------------------------------------------------------------------------------------------------ cross-workgroup sync
// Counters live in a per-layer u32 block (MoeArgs::sync). Producers write their data, fence (agent-scope release)
// and add to a counter; consumers spin on a relaxed agent-scope load (thread 0, s_sleep between polls), then fence
// (acquire) before reading. Every spin is bounded: past the limit, or once any workgroup has flagged an error, it
// gives up and the unit is skipped, so every wave reaches the kernel's end whatever happens.
constexpr uint32_t kSpinLimit = 1u << 22;  // polls of ~0.1-1 us each: seconds, far beyond any real wait
enum {
  kSyncHead = 0,
  kSyncRouterDone = kSyncStride,
  kSyncRouteReady = 2 * kSyncStride,
  kSyncErr = kSyncErrWord,
  kSyncSlots = 8 * kSyncStride
};

__device__ __forceinline__ uint32_t ld_acq(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// thread 0 waits for *p >= v; all threads return whether it was reached (uniform). The data the counter guards is
// read with ld_cg afterwards.
__device__ bool block_wait_geq(uint32_t *sync, const uint32_t *p, uint32_t v, int *flag) {
  if (threadIdx.x == 0) {
    int ok = 0;
    for (uint32_t it = 0; it < kSpinLimit; it++) {
      if (ld_acq(p) >= v) {
        ok = 1;
        break;
      }
      if ((it & 63u) == 63u && ld_acq(sync + kSyncErr)) break;
      __builtin_amdgcn_s_sleep(2);
    }
    if (!ok) atomicOr(sync + kSyncErr, 1u);
    *flag = ok;
  }
  __syncthreads();
  return *flag != 0;
}
// every wave's st_cg stores completed (s_waitcnt 0, then the barrier), then thread 0 adds 1 to *p; returns the old
// value on every thread
__device__ uint32_t block_signal(uint32_t *p, int *flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) *flag = (int)atomicAdd(p, 1u);
  __syncthreads();
  const uint32_t old = (uint32_t)*flag;
  __syncthreads();
  return old;
}

// ------------------------------------------------------------------------------------------------ MoE: D1 router
// Router GEMV (reference kernels/fn_moe.metal:50-67): one wave per router row (ne experts, then the shared-expert gate
// row when present), every weight chunk of the row loaded before the dot; logits rounded to bf16 (the reference
// rounding).
constexpr int kRouterChunks = 8;  // hid <= 8 * 512
// xs: LDS staging for one input row (hid floats); every thread of the workgroup calls this (barriers inside)
__device__ void router_rows(const MoeArgs &a, int unit, float *xs) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = unit * (int)(blockDim.x >> 6) + wave;
  const bool active = row < a.ne + a.has_sgate;
  const uint16_t *w = a.router + (uint64_t)(active ? row : 0) * a.hid;
  uint4 wv[kRouterChunks];
#pragma unroll
  for (int j = 0; j < kRouterChunks; j++) {
    const int e = j * 512 + lane * 8;
    wv[j] = (active && e < a.hid) ? *(const uint4 *)(w + e) : make_uint4(0, 0, 0, 0);
  }
  for (int r = 0; r < a.R; r++) {
    __syncthreads();
    for (int i = threadIdx.x; i < a.hid / 4; i += blockDim.x)
      ((float4 *)xs)[i] = ((const float4 *)(a.x + (uint64_t)r * a.hid))[i];
    __syncthreads();
    if (!active) continue;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < kRouterChunks; j++) {
      const int e = j * 512 + lane * 8;
      if (e < a.hid) {
        const float4 x0 = *(const float4 *)(xs + e), x1 = *(const float4 *)(xs + e + 4);
        acc = fmaf(x0.x, bf16_f32(wv[j].x & 0xFFFFu), acc);
        acc = fmaf(x0.y, bf16_f32(wv[j].x >> 16), acc);
        acc = fmaf(x0.z, bf16_f32(wv[j].y & 0xFFFFu), acc);
        acc = fmaf(x0.w, bf16_f32(wv[j].y >> 16), acc);
        acc = fmaf(x1.x, bf16_f32(wv[j].z & 0xFFFFu), acc);
        acc = fmaf(x1.y, bf16_f32(wv[j].z >> 16), acc);
        acc = fmaf(x1.z, bf16_f32(wv[j].w & 0xFFFFu), acc);
        acc = fmaf(x1.w, bf16_f32(wv[j].w >> 16), acc);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) st_cg(a.logits + (uint64_t)r * (a.ne + 1) + row, bf16_round(acc));
  }
}

// Route of every row from the logits (reference kernels/fn_moe.metal:76-131): top-k by logit, the lower index first
// on ties, weights exp(l - l_max) / sum over the top k in f32 (summed in slot order), shared gate sigmoid(logit).
// Called by one workgroup after every router row is written.
__device__ void route_rows(const MoeArgs &a, float *lv, uint32_t *cand, uint32_t *sid) {
  const int ld = a.ne + 1;
  for (int r = 0; r < a.R; r++) {
    for (int i = threadIdx.x; i < a.ne; i += blockDim.x) lv[i] = ld_cg(a.logits + (uint64_t)r * ld + i);
    __syncthreads();
    block_topk(lv, a.ne, a.topk, cand, sid);
    if (threadIdx.x == 0) {
      float pr[kMaxTopk];
      const float top = lv[sid[0]];
      float s = 0.f;
      for (int k = 0; k < a.topk; k++) {
        pr[k] = expf(lv[sid[k]] - top);
        s += pr[k];
      }
      uint32_t *rt = a.route + (uint64_t)r * 2 * a.topk;
      for (int k = 0; k < a.topk; k++) {
        st_cg(rt + k, sid[k]);
        st_cg(rt + a.topk + k, __float_as_uint(pr[k] / s));
      }
      st_cg(a.sgv + r, moe_shared_gate(a, a.has_sgate ? ld_cg(a.logits + (uint64_t)r * ld + a.ne) : 0.f));
    }
    __syncthreads();
  }
}

// optional unit trace (MoeArgs::trace): [u][0] = wall clock at the take, [1] = after the unit's waits, [2] = done,
// [3] = workgroup id
__device__ __forceinline__ void trace_mark(const MoeArgs &a, int u, int total, int field) {
  if (a.trace && threadIdx.x == 0 && u < total) {
    a.trace[(uint64_t)u * 8 + field] = wall_clock64();
  }
}

// ------------------------------------------------------------------------------------------------ MoE: D2 gate/up
// One unit = (slot, gate|up, output tile pair p, k split ks): prefetch the unit's tiles, prep x * suh -> H -> fp16
// into LDS for the k span (reference kernels/fn_moe.metal:304-312), pair GEMV; guo holds the raw inner outputs per
// k split (summed in order by the down unit).
template <int K>
__device__ void gateup_unit(const MoeArgs &a, const SlotRef &sr, int slot, int proj, int p, int ks, _Float16 *prep,
                            float *red, int tu = 1 << 30, int ttot = 0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = slot / a.nslot;
  const int IT = a.hid >> 4, ktn = IT / a.ksplit, k0 = ks * ktn, n = ktn * 16;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const uint32_t *pb = (const uint32_t *)(sr.blk + off_tr(a, sr.sh, proj)) + (uint64_t)p * IT * 2 * 8 * K;
  PairBuf<K> buf;
  pair_load<K>(buf, pb, L, k0 + wave, k0 + ktn);
  const float *x = a.x + (uint64_t)r * a.hid + k0 * 16;
  const uint16_t *su = (const uint16_t *)(sr.blk + off_su(a, sr.sh, proj)) + k0 * 16;
  for (int c = wave; c * 128 < n; c += 4) {
    const int i0 = c * 128 + lane, i1 = i0 + 64;
    float v0 = i0 < n ? x[i0] * h2f(su[i0]) : 0.f;
    float v1 = i1 < n ? x[i1] * h2f(su[i1]) : 0.f;
    fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
    if (i0 < n) prep[kp(i0)] = to_f16(v0);
    if (i1 < n) prep[kp(i1)] = to_f16(v1);
  }
  __syncthreads();
  trace_mark(a, tu, ttot, 3);
  float acc0, acc1;
  pair_gemv<K>(buf, pb, L, k0, k0 + ktn, prep, acc0, acc1);
  const float s = pair_reduce(acc0, acc1, red);
  trace_mark(a, tu, ttot, 4);
  const int o = p * 32 + (int)threadIdx.x;
  if (threadIdx.x < 32 && o < a.inter) st_cg(a.guo + (((uint64_t)slot * 2 + proj) * a.ksplit + ks) * a.inter + o, s);
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------ MoE: D3 down
// One unit = (slot, output tile pair p). The down tiles are prefetched first; then (fused kernel) the unit waits for
// its slot's gate/up outputs; prologue (reference kernels/fn_moe.metal:370-384): g = H(guo_g) * svh_g,
// u = H(guo_u) * svh_u, h = H(silu(g) u * suh_d) -> fp16 LDS; then the pair GEMV over all inter k tiles. dn holds the
// raw down outputs (H_out, svh and the route weight are applied by the combine). Returns false if the wait failed.
template <int K>
__device__ bool down_unit(const MoeArgs &a, const SlotRef &sr, int slot, int p, _Float16 *prep, float *red,
                          const uint32_t *wait_ctr, uint32_t wait_val, int *flag) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int inter = a.inter;
  const int IT = inter >> 4;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const uint32_t *pb = (const uint32_t *)(sr.blk + off_tr(a, sr.sh, 2)) + (uint64_t)p * IT * 2 * 8 * K;
  PairBuf<K> buf;
  pair_load<K>(buf, pb, L, wave, IT);
  if (wait_ctr && !block_wait_geq(a.sync, wait_ctr, wait_val, flag)) return false;
  const float *gp = a.guo + (uint64_t)slot * 2 * a.ksplit * inter;
  const float *up = gp + (uint64_t)a.ksplit * inter;
  const uint16_t *gsv = (const uint16_t *)(sr.blk + off_sv(a, sr.sh, 0));
  const uint16_t *usv = (const uint16_t *)(sr.blk + off_sv(a, sr.sh, 1));
  const uint16_t *dsu = (const uint16_t *)(sr.blk + off_su(a, sr.sh, 2));
  for (int c = wave; c * 128 < inter; c += 4) {
    const int i0 = c * 128 + lane, i1 = i0 + 64;
    const bool m0 = i0 < inter, m1 = i1 < inter;
    float g0 = m0 ? ld_cg(gp + i0) : 0.f, g1 = m1 ? ld_cg(gp + i1) : 0.f;
    float u0 = m0 ? ld_cg(up + i0) : 0.f, u1 = m1 ? ld_cg(up + i1) : 0.f;
    for (int s = 1; s < a.ksplit; s++) {
      if (m0) {
        g0 += ld_cg(gp + s * inter + i0);
        u0 += ld_cg(up + s * inter + i0);
      }
      if (m1) {
        g1 += ld_cg(gp + s * inter + i1);
        u1 += ld_cg(up + s * inter + i1);
      }
    }
    fwht2(g0, g1, lane, a.had_inter, a.sc_inter);
    fwht2(u0, u1, lane, a.had_inter, a.sc_inter);
    float h0 = 0.f, h1 = 0.f;
    if (m0) {
      g0 = g0 * h2f(gsv[i0]);
      u0 = u0 * h2f(usv[i0]);
      h0 = g0 / (1.f + expf(-g0)) * u0 * h2f(dsu[i0]);
    }
    if (m1) {
      g1 = g1 * h2f(gsv[i1]);
      u1 = u1 * h2f(usv[i1]);
      h1 = g1 / (1.f + expf(-g1)) * u1 * h2f(dsu[i1]);
    }
    fwht2(h0, h1, lane, a.had_inter, a.sc_inter);
    if (m0) prep[kp(i0)] = to_f16(h0);
    if (m1) prep[kp(i1)] = to_f16(h1);
  }
  __syncthreads();
  float acc0, acc1;
  pair_gemv<K>(buf, pb, L, 0, IT, prep, acc0, acc1);
  const float s = pair_reduce(acc0, acc1, red);
  const int o = p * 32 + (int)threadIdx.x;
  if (threadIdx.x < 32 && o < a.hid) st_cg(a.dn + (uint64_t)slot * a.hid + o, s);
  __syncthreads();
  return true;
}

// ------------------------------------------------------------------------------------------------ MoE: combine
// y[r][128 c ..] = sum over slots in slot order of H(dn) * svh_d * w_k, the shared slot last with its gate
// (reference kernels/fn_moe.metal:412-447); 4 waves take the slots round-robin, the sum runs in slot order from LDS.
constexpr int kMaxSlots = kMaxTopk + 1;
__device__ void combine_block(const MoeArgs &a, int r, int c, float (*vs)[128]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i0 = c * 128 + lane, i1 = i0 + 64;
  const bool m0 = i0 < a.hid, m1 = i1 < a.hid;
  const int nw = (int)(blockDim.x >> 6);
  for (int k = wave; k < a.nslot; k += nw) {
    const int slot = r * a.nslot + k;
    const SlotRef sr = slot_ref(a, r, k);
    const float w = k < a.topk ? __uint_as_float(ld_cg(a.route + (uint64_t)r * 2 * a.topk + a.topk + k))
                               : ld_cg(a.sgv + r);
    const float *d = a.dn + (uint64_t)slot * a.hid;
    const uint16_t *sv = (const uint16_t *)(sr.blk + off_sv(a, sr.sh, 2));
    float v0 = m0 ? ld_cg(d + i0) : 0.f, v1 = m1 ? ld_cg(d + i1) : 0.f;
    const float s0 = m0 ? h2f(sv[i0]) : 0.f, s1 = m1 ? h2f(sv[i1]) : 0.f;
    fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
    vs[k][lane] = v0 * s0 * w;
    vs[k][lane + 64] = v1 * s1 * w;
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    const int i = c * 128 + threadIdx.x;
    float s = 0.f;
    for (int k = 0; k < a.topk; k++) s += vs[k][threadIdx.x];
    const float t = a.nslot > a.topk ? vs[a.topk][threadIdx.x]
                    : a.q8 && i < a.hid ? ld_cg(a.sgv + r) * a.q8o[(uint64_t)r * a.hid + i]
                                        : 0.f;
    if (i < a.hid) a.y[(uint64_t)r * a.hid + i] = moe_finish(a, r, i, s, t);
  }
  __syncthreads();
}

// ------------------------------------------------------------------------------------------------ staged kernels
// D1..D3 + combine as four launches (the reference's dispatch structure, kernels/fn_moe.metal). The router's last
// workgroup to arrive (atomic counter, reset by it) computes the route.
__global__ __launch_bounds__(256) void moe_router(MoeArgs a) {
  __shared__ float lv[kMaxExperts];
  __shared__ uint32_t sid[kMaxTopk];
  __shared__ uint32_t cand[4 * kMaxTopk];
  __shared__ int flag;
  __shared__ float xs[kRouterChunks * 512];
  router_rows(a, blockIdx.x, xs);
  if (block_signal(a.sync + kSyncRouterDone, &flag) != gridDim.x - 1u) return;
  route_rows(a, lv, cand, sid);
  if (threadIdx.x == 0) atomicExch(a.sync + kSyncRouterDone, 0u);
}

constexpr int kMaxPrep = 4096;  // halves of prepared input per workgroup

__global__ __launch_bounds__(256) void moe_gateup(MoeArgs a) {
  __shared__ _Float16 prep[kMaxPrep];
  __shared__ float red[128];
  int b = blockIdx.x;
  const int NP = (a.inter / 16 + 1) / 2;
  const int ks = b % a.ksplit;
  b /= a.ksplit;
  const int p = b % NP;
  b /= NP;
  const int proj = b & 1, slot = b >> 1;
  const SlotRef sr = slot_ref(a, slot / a.nslot, slot % a.nslot);
  IJ_DISPATCH_K(sr.K, gateup_unit<KK>(a, sr, slot, proj, p, ks, prep, red));
}

__global__ __launch_bounds__(256) void moe_down(MoeArgs a) {
  __shared__ _Float16 prep[kMaxPrep];
  __shared__ float red[128];
  __shared__ int flag;
  const int NP = (a.hid / 16 + 1) / 2;
  const int p = blockIdx.x % NP, slot = blockIdx.x / NP;
  const SlotRef sr = slot_ref(a, slot / a.nslot, slot % a.nslot);
  IJ_DISPATCH_K(sr.K, down_unit<KK>(a, sr, slot, p, prep, red, nullptr, 0u, &flag));
}

__global__ __launch_bounds__(256) void moe_combine(MoeArgs a) {
  __shared__ float vs[kMaxSlots][128];
  const int nch = (a.hid + 127) / 128;
  combine_block(a, blockIdx.x / nch, blockIdx.x % nch, vs);
}


// ------------------------------------------------------------------------------------------------ trunk linear
// a finished output v of row r, column c through the linear's epilogue into y (and the epilogue's side buffers)
__device__ __forceinline__ float epi_rr(float x, int refr) { return refr ? bf16_round(x) : x; }
__device__ __forceinline__ float epi_bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ void lin_store(const LinArgs &a, int r, int c, float v) {
  const LinEpi &e = a.epi;
  float *y = a.y + (uint64_t)r * (e.ldy ? e.ldy : a.out) + c;
  const int q = e.refr, R = e.row0 + r;
  switch (e.kind) {
    case 1: {
      const float br = epi_rr(v, q);
      *y = br;
      for (int s = 0; s < e.hc; s++) {
        const uint64_t o = ((uint64_t)R * e.hc + s) * a.out + c;
        e.e2[o] = epi_rr(e.e0[o] + epi_rr(br * e.e1[R * 8 + s], q), q);
      }
      break;
    }
    case 2: {
      const float t = epi_rr(v, q) * 0.25f;
      *y = epi_rr(t / (1.f + expf(-t)), q);
      break;
    }
    case 3: *y = epi_rr(v, q); break;
    case 5: *y = epi_rr(1.f / (1.f + expf(-epi_rr(v, q))), q); break;
    case 6: {
      const float ex = expf(epi_bf(((const uint16_t *)e.e0)[c])), dt = epi_bf(((const uint16_t *)e.e1)[c]);
      const float u = epi_rr(epi_rr(v, q) + dt, q);
      const float sp = epi_rr(u > 20.f ? u : logf(1.f + expf(u)), q);
      *y = expf(-ex * sp);
      break;
    }
    case 8: st_cg(e.e0 + (uint64_t)R * a.out + c, v); break;
    case 7:
      *y = v;
      if (c >= 512) {
        const uint64_t t = (uint64_t)((const uint32_t *)e.e1)[0] + R;
        if (t < (uint64_t)e.cap) e.e0[t * 128 + (c - 512)] = v;
      }
      break;
    default: *y = v;
  }
}

// The HC read's output step fused into the up linear's finisher (LinEpi kind 8; reference
// kernels/trunk6/t6_epi.metal:80-97 for the arithmetic): for each of up to B output columns i0, i0 + stride, ..
// below n (row r0 + i / 128, column cs * 128 + i % 128 of the hid outputs) the four streams' u (coherent loads: other
// workgroups stored them) and the other operands are all requested first, then each column is finished: one round
// trip for B columns instead of one per column.
template <int B>
__device__ __forceinline__ void hc_fin_cols(const LinArgs &a, int r0, int cs, int i0, int stride, int n) {
  const LinEpi &e = a.epi;
  const int hid = e.hid, q = e.refr;
  float u[B][4], y[B][4], inv[B][4], w[B][4];
#pragma unroll
  for (int b = 0; b < B; b++) {
    const int i = min(i0 + b * stride, n - 1), r = r0 + i / 128, cc = cs * 128 + i % 128;
#pragma unroll
    for (int st = 0; st < 4; st++) {
      const uint64_t row = (uint64_t)st * hid + cc;
      u[b][st] = ld_cg(e.e0 + (uint64_t)r * a.out + row);
      y[b][st] = e.e1[(uint64_t)r * a.out + row];
      inv[b][st] = e.e4[r * 8 + 4 + st];
      w[b][st] = epi_bf(e.w16[row]);
    }
  }
#pragma unroll
  for (int b = 0; b < B; b++) {
    const int i = i0 + b * stride;
    if (i < n) {
      const int r = r0 + i / 128, cc = cs * 128 + i % 128;
      float v[4];
#pragma unroll
      for (int st = 0; st < 4; st++) {
        const float sg = epi_rr(1.f / (1.f + expf(-epi_rr(u[b][st], q))), q);
        v[st] = epi_rr(sg * epi_rr(y[b][st] * inv[b][st] * w[b][st], q), q);
      }
      e.e2[(uint64_t)r * hid + cc] = epi_rr(((v[0] + v[1]) + (v[2] + v[3])) * 0.25f, q);
    }
  }
}
// the row's four inject gates from the prep's partials, on one whole wave (lane = (chunk phase, stream, gate))
__device__ __forceinline__ void hc_fin_gates(const LinArgs &a, int r, int lane) {
  const LinEpi &e = a.epi;
  const int nch = (e.hid + 255) / 256, j = lane & 3, st = (lane >> 2) & 3, ph = lane >> 4;
  float t = 0.f;
  for (int ch = ph; ch < nch; ch += 4) t += e.e3[((r * 4 + st) * nch + ch) * 4 + j];
  t += __shfl_xor(t, 16, 64);  // the chunk phases
  t += __shfl_xor(t, 32, 64);
  t += __shfl_xor(t, 4, 64);   // the streams
  t += __shfl_xor(t, 8, 64);
  if (lane < 4) e.e4[r * 8 + lane] = epi_rr(2.f / (1.f + expf(-epi_rr(t, e.refr) * 0.25f)), e.refr);
}
// after a finisher stored u for rows [r0, r1) of 128-column block cb: the last of the four streams' blocks of those
// columns (counter ctr, reset by it) writes their outputs; the first column block's last arrival also the gates
__device__ void hc_fin_block(const LinArgs &a, uint32_t *ctr, int r0, int r1, int cb, int *flag) {
  const int nbs = a.epi.hid / 128, cs = cb % nbs, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = (int)(blockDim.x >> 6);
  if (block_signal(ctr, flag) != 3u) return;
  if (threadIdx.x == 0) st_cg(ctr, 0u);
  const int n = (r1 - r0) * 128;
  for (int i0 = threadIdx.x; i0 < n; i0 += 4 * (int)blockDim.x) hc_fin_cols<4>(a, r0, cs, i0, (int)blockDim.x, n);
  if (cs == 0)
    for (int r = r0 + wave; r < r1; r += nw) hc_fin_gates(a, r, lane);
}

// lin_prep: xh[r][kp(i)] = fp16(H_in(x * suh)) (reference kernels/trunk6/trunk6.metal:68-85), grid R x ceil(in/128).
__global__ __launch_bounds__(64) void lin_prep(LinArgs a) {
  const int nch = (a.in + 127) / 128;
  const int r = blockIdx.x / nch, c = blockIdx.x % nch, lane = threadIdx.x;
  const int i0 = c * 128 + lane, i1 = i0 + 64;
  const float *x = a.x + (uint64_t)r * a.in;
  float v0 = i0 < a.in ? x[i0] * h2f(a.suh[i0]) : 0.f;
  float v1 = i1 < a.in ? x[i1] * h2f(a.suh[i1]) : 0.f;
  fwht2(v0, v1, lane, a.had_in, a.sc_in);
  if (i0 < a.in) a.xh[(uint64_t)r * a.in + kp(i0)] = f2h(v0);
  if (i1 < a.in) a.xh[(uint64_t)r * a.in + kp(i1)] = f2h(v1);
}

// The finished outputs of 128-column block cb for row r: the k group partials folded left in k order, H_out, svh, the
// epilogue (reference kernels/trunk6/trunk6.metal:199-214, t6_finish). coherent: the partials were stored by other
// workgroups of this launch (device-coherent loads); else by an earlier launch.
// Rows r0, r0 + rs, .. (NR of them, those below R) of output block cb: each row's k-group partials folded left in
// group order, H_out, svh and the epilogue. The partials of all NR rows are requested together (rounds of 8 groups
// for one row, 4 for several), so a wave finishing several rows pays one round trip per round, not one per row.
template <int NR>
__device__ void lin_finish_rows(const LinArgs &a, int r0, int rs, int cb, bool coherent) {
  const int lane = threadIdx.x & 63, OTp = a.OT + (a.OT & 1);
  const int i0 = cb * 128 + lane, i1 = i0 + 64;
  const bool m0 = i0 < a.out, m1 = i1 < a.out;
  const int j0 = m0 ? i0 : 0, j1 = m1 ? i1 : 0;
  float v0[NR], v1[NR];
#pragma unroll
  for (int q = 0; q < NR; q++) v0[q] = v1[q] = 0.f;
  constexpr int B = NR == 1 ? 8 : 4;  // groups requested together (2 NR B values in flight per lane)
  for (int g0 = 0; g0 < a.S; g0 += B) {
    float t0[NR][B], t1[NR][B];
#pragma unroll
    for (int q = 0; q < NR; q++) {
      const int r = min(r0 + q * rs, a.R - 1);
#pragma unroll
      for (int j = 0; j < B; j++) {
        const float *pp = a.part + ((uint64_t)min(g0 + j, a.S - 1) * a.R + r) * OTp * 16;
        t0[q][j] = coherent ? ld_cg(pp + j0) : pp[j0];
        t1[q][j] = coherent ? ld_cg(pp + j1) : pp[j1];
      }
    }
#pragma unroll
    for (int q = 0; q < NR; q++)
#pragma unroll
      for (int j = 0; j < B; j++)
        if (g0 + j < a.S) {
          v0[q] = g0 + j == 0 ? t0[q][j] : v0[q] + t0[q][j];
          v1[q] = g0 + j == 0 ? t1[q][j] : v1[q] + t1[q][j];
        }
  }
#pragma unroll
  for (int q = 0; q < NR; q++) {
    const int r = r0 + q * rs;
    if (r >= a.R) break;
    float w0 = m0 ? v0[q] : 0.f, w1 = m1 ? v1[q] : 0.f;
    fwht2(w0, w1, lane, a.had_out, a.sc_out);
    if (m0) lin_store(a, r, i0, w0 * h2f(a.svh[i0]));
    if (m1) lin_store(a, r, i1, w1 * h2f(a.svh[i1]));
  }
}
__device__ void lin_finish_row(const LinArgs &a, int r, int cb, bool coherent) {
  lin_finish_rows<1>(a, r, 1, cb, coherent);
}
// the block's rows over the workgroup's 4 waves (wave c: rows c, c + 4, ..), four rows per request round
__device__ void lin_finish_block(const LinArgs &a, int c, int cb) {
  if (a.R <= 4) {
    if (c < a.R) lin_finish_rows<1>(a, c, 4, cb, true);
  } else {
    for (int r = c; r < a.R; r += 16) lin_finish_rows<4>(a, r, 4, cb, true);
  }
}

// lin_mx: up to kLinMulti linears at R <= 32 rows in one launch, on the matrix cores (reference
// kernels/trunk6/trunk6.metal: t6_prep :68-85, t6_simd / t6_nax, t6_finish :199-214; trunk6.mm record_multi).
// Workgroup (linear, tile pair p, k group g), 4 waves; wave c takes k chunk c of the group (8 k tiles):
//   1. requests the chunk's tiles into its LDS slot; prepares the chunk's input rows (fp16(H_in(x suh)), kp order)
//      in LDS meanwhile (x and suh requested before the tiles, so that waiting for them does not wait for the
//      tiles), or (xh_in) requests the rows a prep launch wrote;
//   2. decodes the tiles straight into the B operand of v_mfma_f32_32x32x16_f16 (A: the input rows; a row beyond R
//      repeats row R - 1, its products unused) in one chain from zero;
// then the chunk sums of the 4 waves are folded left in LDS and stored as the group's partials (device-coherent
// stores); the last workgroup to store into a 128-column output block (a counter per block, which it resets to 0)
// finishes the block's rows. (Staged path: no counter; lin_finish finishes.)
// Every row's arithmetic is the same at any R: a row of a batch is bit-identical to that row run alone.
struct LinMulti {
  int n;
  int wg0[kLinMulti + 1];  // first workgroup of each linear
  LinArgs l[kLinMulti];
};
__device__ __forceinline__ LinArgs lin_pick(const LinMulti &m, int i) {  // uniform i; no dynamic struct indexing
  return i == 0 ? m.l[0] : i == 1 ? m.l[1] : i == 2 ? m.l[2] : m.l[3];
}
// LDS of one wave: its tiles (8 k tile pairs), then RT prepared rows of its chunk (128 halves each)
template <int K, int RT>
constexpr uint32_t lin_wave_lds() { return kLinChunkKt * 64 * K + RT * 256; }
template <int K, int RT>
constexpr uint32_t lin_mx_lds() { return 4 * lin_wave_lds<K, RT>() + 4 * RT * 32 * 4; }

template <int K, int RT>
__global__ __launch_bounds__(256) void lin_mx(LinMulti m) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int flag;
  int li = 0;
#pragma unroll
  for (int i = 1; i < kLinMulti; i++)
    if (i < m.n && (int)blockIdx.x >= m.wg0[i]) li = i;
  const LinArgs a = lin_pick(m, li);
  const int NP = (a.OT + 1) / 2, OTp = 2 * NP, R = a.R;
  const int b = (int)blockIdx.x - m.wg0[li], p = b % NP, g = b / NP;
  const int lane = threadIdx.x & 63, c = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kt0 = g * kLinGroupKt + c * kLinChunkKt, nkt = max(0, min(kLinChunkKt, a.IT - kt0));
  uint8_t *tl = lds + c * lin_wave_lds<K, RT>();
  _Float16 *xs = (_Float16 *)(tl + kLinChunkKt * 64 * K);
  float *csum = (float *)(lds + 4 * lin_wave_lds<K, RT>());  // [4 chunks][RT rows][32 columns]
  const int e0 = kt0 * 16, i0 = e0 + lane, i1 = i0 + 64;    // the chunk's elements of this lane
  const int cb = p / 4;
  // 1. input rows and tiles
  float xv0[RT], xv1[RT], s0 = 0.f, s1 = 0.f;
  if (!a.xh_in && nkt > 0) {
    s0 = i0 < a.in ? h2f(a.suh[i0]) : 0.f;
    s1 = i1 < a.in ? h2f(a.suh[i1]) : 0.f;
#pragma unroll
    for (int r = 0; r < RT; r++)
      if (r < R) {
        xv0[r] = i0 < a.in ? a.x[(uint64_t)r * a.in + i0] : 0.f;
        xv1[r] = i1 < a.in ? a.x[(uint64_t)r * a.in + i1] : 0.f;
      }
  }
  // (HC read, one row) hc_prep's loads, requested with x and suh: the stream's values for its sum of squares (thread
  // t: columns t + 256 u of stream hs, hc_prep's batch of 16) and the norm weights of the wave's columns; the first
  // tile pair's workgroups also the norm and inject weights of the group's two 256-column chunks (thread t: column
  // t of each)
  constexpr int kHcB = 16;
  const bool hcin = RT == 1 && a.hc.nw != nullptr;
  const int hhid = a.hc.hid, hs = hcin ? g * kLinGroupKt * 16 / hhid : 0;
  float hq[kHcB], nw0 = 0.f, nw1 = 0.f, cx[2] = {0.f, 0.f}, cw[2][4] = {};
  if constexpr (RT == 1) {
    if (hcin) {
      const float *hr = a.x + (uint64_t)hs * hhid;
#pragma unroll
      for (int u = 0; u < kHcB; u++) {
        const int j = 256 * u + (int)threadIdx.x;
        hq[u] = hr[j < hhid ? j : 0];
      }
      nw0 = epi_bf(a.hc.nw[i0]);
      nw1 = epi_bf(a.hc.nw[i1]);
      if (p == 0) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const int j = g * kLinGroupKt * 16 + q * 256 + (int)threadIdx.x;
          cx[q] = a.x[j] * epi_bf(a.hc.nw[j]);
#pragma unroll
          for (int k = 0; k < 4; k++) cw[q][k] = epi_bf(a.hc.iw[(uint64_t)k * 4 * hhid + j]);
        }
      }
    }
  }
  int ndma = 0;
  if (nkt > 0) {
    const uint8_t *src = (const uint8_t *)a.tiles + ((uint64_t)p * a.IT + kt0) * 64 * K;
    const uint32_t bytes = (uint32_t)nkt * 64 * K;
    for (uint32_t o = 0; o < bytes; o += 1024, ndma++)
      if (o + (uint32_t)lane * 16 < bytes)
        __builtin_amdgcn_global_load_lds((const void *)(src + o + lane * 16),
                                         (__attribute__((address_space(3))) void *)(tl + o), 16, 0, 0);
    if (a.xh_in) {  // rows r .. r + 3 per request: 16 lanes of 16 bytes each (the chunk's nkt * 32 bytes)
      for (int r = 0; r < R; r += 4) {
        const int rr = r + (lane >> 4), q = lane & 15;
        if (rr < R && q * 16 < nkt * 32)
          __builtin_amdgcn_global_load_lds((const void *)(a.xh + (uint64_t)rr * a.in + e0 + q * 8),
                                           (__attribute__((address_space(3))) void *)(xs + r * 128), 16, 0, 0);
      }
    }
  }
  if (!a.xh_in && nkt > 0) wait_vm(ndma);  // x and suh are in (the tiles, requested after them, may not be)
  if constexpr (RT == 1) {
    if (hcin) {  // hc_prep's sums (same order: per thread, the wave's xor butterfly, the four waves left to right)
      __shared__ float hred[4][9];
      float t[9];
      t[0] = 0.f;
#pragma unroll
      for (int u = 0; u < kHcB; u++)
        if (256 * u + (int)threadIdx.x < hhid) t[0] += hq[u] * hq[u];
#pragma unroll
      for (int q = 0; q < 2; q++)
#pragma unroll
        for (int k = 0; k < 4; k++) t[1 + 4 * q + k] = cw[q][k] * cx[q];
#pragma unroll
      for (int k = 0; k < 9; k++)
        for (int o = 32; o >= 1; o >>= 1) t[k] += __shfl_xor(t[k], o, 64);
      if (lane == 0)
#pragma unroll
        for (int k = 0; k < 9; k++) hred[c][k] = t[k];
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 9; k++) t[k] = ((hred[0][k] + hred[1][k]) + hred[2][k]) + hred[3][k];
      const float inv = 1.f / sqrtf(t[0] / (float)hhid + 1e-6f);
      xv0[0] = (xv0[0] * nw0) * inv;
      xv1[0] = (xv1[0] * nw1) * inv;
      if (p == 0) {  // hc_prep's other outputs for this group's two chunks of stream hs
        const int nch = (hhid + 255) / 256, ch0 = (g * kLinGroupKt * 16 - hs * hhid) / 256;
        if (threadIdx.x < 8)
          a.hc.ip[(hs * nch + ch0 + (int)threadIdx.x / 4) * 4 + threadIdx.x % 4] = t[1 + threadIdx.x] * inv;
        if (threadIdx.x == 0 && ch0 == 0) a.hc.inj[kHcStreams + hs] = inv;
      }
    }
  }
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  if (nkt > 0) {
    if (!a.xh_in) {
#pragma unroll
      for (int r = 0; r < RT; r++)
        if (r < R) {
          float v0 = xv0[r] * s0, v1 = xv1[r] * s1;
          fwht2(v0, v1, lane, a.had_in, a.sc_in);
          xs[r * 128 + kp((uint32_t)lane)] = to_f16(v0);
          xs[r * 128 + kp((uint32_t)lane + 64)] = to_f16(v1);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the tiles (and rows) are in LDS
    // 2. the chunk's chain on the matrix cores
    const _Float16 *xa = xs + min(lane & 31, R - 1) * 128 + 8 * (lane >> 5);
    acc = mfma_chunk<K, kLinChunkKt>(tl, xa, nkt, acc);
  }
  // 3. chunk sums (lane (n, h), value i: row 8 (i / 4) + 4 h + i % 4, column n) -> LDS; the group's fold -> partials
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    if (r < RT && r < R) csum[(c * RT + r) * 32 + (lane & 31)] = acc[i];
  }
  __syncthreads();
  const int nc = (min(kLinGroupKt, a.IT - g * kLinGroupKt) + kLinChunkKt - 1) / kLinChunkKt;
  for (int e = threadIdx.x; e < R * 32; e += 256) {
    const int r = e >> 5, n = e & 31;
    float v = csum[r * 32 + n];
    for (int cc = 1; cc < nc; cc++) v = v + csum[(cc * RT + r) * 32 + n];
    st_cg(a.part + ((uint64_t)g * R + r) * OTp * 16 + p * 32 + n, v);
  }
  if (!a.cnt) return;
  // 4. the last workgroup of the 128-column output block finishes its rows
  const int npb = min(4, NP - 4 * cb);
  uint32_t *ctr = a.cnt + (uint64_t)cb * kSyncStride;
  if (block_signal(ctr, &flag) != (uint32_t)(npb * a.S - 1)) return;
  if (threadIdx.x == 0) st_cg(ctr, 0u);
  lin_finish_block(a, c, cb);
  if (a.epi.kind == 8)
    hc_fin_block(a, a.epi.ctr + (uint64_t)(cb % (a.epi.hid / 128)) * kSyncStride, a.epi.row0, a.epi.row0 + R, cb,
                 &flag);
}

// lin_mxl: lin_mx for linears with many tile pairs (a vocabulary head), one workgroup per tile pair looping over the
// k groups: wave c takes chunk c of every group, the next group's requests in flight while one decodes; the chunk sums
// go to LDS, and at the end each (row, column) folds the chunks of each group left and the groups left - the order of
// lin_mx, so the results are bit-identical - and stores one total per pair (S = 1). The block's last arriving pair
// finishes it, as in lin_mx.
template <int K, int RT>
constexpr uint32_t lin_mxl_wave() { return kLinChunkKt * 64 * K + RT * 256; }
template <int K, int RT>
constexpr uint32_t lin_mxl_lds(int G) { return 8 * lin_mxl_wave<K, RT>() + (uint32_t)G * 4 * RT * 32 * 4; }
constexpr int kLinLoopMaxGroups = 16;  // in <= 8192
template <int K, int RT>
__global__ __launch_bounds__(256) void lin_mxl(LinMulti m) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  int li = 0;
#pragma unroll
  for (int i = 1; i < kLinMulti; i++)
    if (i < m.n && (int)blockIdx.x >= m.wg0[i]) li = i;
  const LinArgs a = lin_pick(m, li);
  const int NP = (a.OT + 1) / 2, OTp = 2 * NP, R = a.R, IT = a.IT, G = (IT + kLinGroupKt - 1) / kLinGroupKt;
  const int p = (int)blockIdx.x - m.wg0[li];
  const int lane = threadIdx.x & 63, c = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float *csum = (float *)(lds + 8 * lin_mxl_wave<K, RT>());  // [group][4 chunks][RT][32]
  const int cb = p / 4;
  __shared__ int flag;
  const uint8_t *tiles = (const uint8_t *)a.tiles + (uint64_t)p * IT * 64 * K;
  auto stage = [&](int g) {  // group g's requests into buffer g & 1 (the rows come from the prep launch)
    const int kt0 = g * kLinGroupKt + c * kLinChunkKt, nkt = max(0, min(kLinChunkKt, IT - kt0));
    uint8_t *tl = lds + (2 * c + (g & 1)) * lin_mxl_wave<K, RT>();
    _Float16 *xs = (_Float16 *)(tl + kLinChunkKt * 64 * K);
    int n = 0;
    if (nkt > 0) {
      const uint32_t bytes = (uint32_t)nkt * 64 * K;
      for (uint32_t o = 0; o < bytes; o += 1024, n++)
        if (o + (uint32_t)lane * 16 < bytes)
          __builtin_amdgcn_global_load_lds((const void *)(tiles + (uint64_t)kt0 * 64 * K + o + lane * 16),
                                           (__attribute__((address_space(3))) void *)(tl + o), 16, 0, 0);
      for (int r = 0; r < R; r += 4, n++) {
        const int rr = r + (lane >> 4), q = lane & 15;
        if (rr < R && q * 16 < nkt * 32)
          __builtin_amdgcn_global_load_lds((const void *)(a.xh + (uint64_t)rr * a.in + kt0 * 16 + q * 8),
                                           (__attribute__((address_space(3))) void *)(xs + r * 128), 16, 0, 0);
      }
    }
    return n;
  };
  stage(0);
  for (int g = 0; g < G; g++) {
    const int nnext = g + 1 < G ? stage(g + 1) : 0;
    wait_vm(nnext);  // group g's requests are in (the next group's may not be)
    const int kt0 = g * kLinGroupKt + c * kLinChunkKt, nkt = max(0, min(kLinChunkKt, IT - kt0));
    const uint8_t *tl = lds + (2 * c + (g & 1)) * lin_mxl_wave<K, RT>();
    const _Float16 *xa = (const _Float16 *)(tl + kLinChunkKt * 64 * K) + min(lane & 31, R - 1) * 128 + 8 * (lane >> 5);
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
    acc = mfma_chunk<K, kLinChunkKt>(tl, xa, nkt, acc);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      if (r < RT && r < R) csum[((g * 4 + c) * RT + r) * 32 + (lane & 31)] = acc[i];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this buffer's reads are done before it is refilled
  }
  __syncthreads();
  for (int e = threadIdx.x; e < R * 32; e += 256) {
    float tot = 0.f;
    for (int g = 0; g < G; g++) {
      const int nc = (min(kLinGroupKt, IT - g * kLinGroupKt) + kLinChunkKt - 1) / kLinChunkKt;
      float v = csum[(g * 4) * RT * 32 + e];
      for (int cc = 1; cc < nc; cc++) v = v + csum[(g * 4 + cc) * RT * 32 + e];
      tot = g == 0 ? v : tot + v;
    }
    st_cg(a.part + (uint64_t)(e >> 5) * OTp * 16 + p * 32 + (e & 31), tot);
  }
  if (!a.cnt) return;
  const int npb = min(4, NP - 4 * cb);
  uint32_t *ctr = a.cnt + (uint64_t)cb * kSyncStride;
  if (block_signal(ctr, &flag) != (uint32_t)(npb - 1)) return;
  if (threadIdx.x == 0) st_cg(ctr, 0u);
  lin_finish_block(a, c, cb);
  if (a.epi.kind == 8)
    hc_fin_block(a, a.epi.ctr + (uint64_t)(cb % (a.epi.hid / 128)) * kSyncStride, a.epi.row0, a.epi.row0 + R, cb,
                 &flag);
}

// lin_mxw: lin_mx for wide linears (a vocabulary head) at 5..32 rows. Workgroup (8 tile pairs = two 128-column
// output blocks, k group g), 8 waves; wave w takes pair 8 bp + w through the group's k chunks, each one MFMA chain
// from zero folded left in registers (lin_mx's order: the same bits), the next chunk's requests in flight while one
// decodes. A chunk's input rows are staged in LDS once for the 8 waves (lin_mx stages them per wave). The group
// partials, the block counters and the finish are lin_mx's (two blocks per workgroup).
template <int K, int RT, int NW>
constexpr uint32_t lin_mxw_stage() { return RT * 256 + NW * kLinChunkKt * 64 * K; }
template <int K, int RT, int NW>
constexpr uint32_t lin_mxw_lds() { return 2 * lin_mxw_stage<K, RT, NW>(); }
template <int K, int RT, int NW>
__global__ __launch_bounds__(64 * NW) void lin_mxw(LinMulti m) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // the only LDS (4 pairs, 16 rows, K8: 40 KB, 4
                                                                  // workgroups per CU)
  const LinArgs a = m.l[0];  // one linear per launch
  const int NP = (a.OT + 1) / 2, OTp = 2 * NP, R = a.R, IT = a.IT, NBP = (NP + NW - 1) / NW;
  const int bp = (int)blockIdx.x % NBP, g = (int)blockIdx.x / NBP;
  const int lane = threadIdx.x & 63, w = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), p = bp * NW + w;
  const bool live = p < NP;
  const int nck = min(kLinGroupKt / kLinChunkKt, (IT - g * kLinGroupKt + kLinChunkKt - 1) / kLinChunkKt);
  const uint8_t *tiles = (const uint8_t *)a.tiles + (uint64_t)min(p, NP - 1) * IT * 64 * K;
  // chunk c's requests into stage buffer c & 1: this wave's tiles, then the row quads 4 j .. 4 j + 3 with j = w mod 8
  auto stage = [&](int c) {
    const int kt0 = g * kLinGroupKt + c * kLinChunkKt, nkt = min(kLinChunkKt, IT - kt0);
    uint8_t *sb = lds + (c & 1) * lin_mxw_stage<K, RT, NW>();
    uint8_t *tl = sb + RT * 256 + w * kLinChunkKt * 64 * K;
    int n = 0;
    if (live) {
      const uint32_t bytes = (uint32_t)nkt * 64 * K;
      for (uint32_t o = 0; o < bytes; o += 1024, n++)
        if (o + (uint32_t)lane * 16 < bytes)
          __builtin_amdgcn_global_load_lds((const void *)(tiles + (uint64_t)kt0 * 64 * K + o + lane * 16),
                                           (__attribute__((address_space(3))) void *)(tl + o), 16, 0, 0);
    }
    for (int j = w; 4 * j < R; j += NW, n++) {
      const int rr = 4 * j + (lane >> 4), q = lane & 15;
      if (rr < R && q * 16 < nkt * 32)
        __builtin_amdgcn_global_load_lds((const void *)(a.xh + (uint64_t)rr * a.in + kt0 * 16 + q * 8),
                                         (__attribute__((address_space(3))) void *)(sb + 4 * j * 256), 16, 0, 0);
    }
    return n;
  };
  stage(0);
  f32x16 v;
#pragma unroll
  for (int i = 0; i < 16; i++) v[i] = 0.f;
  for (int c = 0; c < nck; c++) {
    int nn = 0;
    if (c + 1 < nck) {
      __syncthreads();  // every wave is done with chunk c - 1's buffer before it is refilled
      nn = stage(c + 1);
    }
    wait_vm(nn);      // this wave's requests of chunk c are in (chunk c + 1's may not be)
    __syncthreads();  // and every wave's (the rows)
    if (live) {
      const int kt0 = g * kLinGroupKt + c * kLinChunkKt, nkt = min(kLinChunkKt, IT - kt0);
      const uint8_t *sb = lds + (c & 1) * lin_mxw_stage<K, RT, NW>();
      const _Float16 *xa = (const _Float16 *)sb + min(lane & 31, R - 1) * 128 + 8 * (lane >> 5);
      f32x16 acc;
#pragma unroll
      for (int i = 0; i < 16; i++) acc[i] = 0.f;
      acc = mfma_chunk<K, kLinChunkKt>(sb + RT * 256 + w * kLinChunkKt * 64 * K, xa, nkt, acc);
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = c == 0 ? acc[i] : v[i] + acc[i];
    }
  }
  if (live)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      if (r < RT && r < R) st_cg(a.part + ((uint64_t)g * R + r) * OTp * 16 + p * 32 + (lane & 31), v[i]);
    }
  if (!a.cnt) return;
  // each of the (one or two) blocks: its last arriving k group finishes it (waves 0-3 the first, 4-7 the second)
  const int nb = min(NW / 4, (NP - NW * bp + 3) / 4);
  uint32_t last = 0;
  for (int b = 0; b < nb; b++) {
    uint32_t *ctr = a.cnt + (uint64_t)((NW / 4) * bp + b) * kSyncStride;
    // the flag word in the stage buffers: block_signal's barrier comes after every wave's last chunk
    if (block_signal(ctr, (int *)lds) == (uint32_t)(a.S - 1)) {
      last |= 1u << b;
      if (threadIdx.x == 0) st_cg(ctr, 0u);
    }
  }
  const int b = w >> 2;
  if (last & (1u << b)) lin_finish_block(a, w & 3, (NW / 4) * bp + b);
}

// lin_finish: the finisher of the staged path, grid R x ceil(out/128) (one workgroup per row and output block)
__global__ __launch_bounds__(64) void lin_finish(LinArgs a) {
  __shared__ int flag;
  const int nch = (a.out + 127) / 128;
  const int r = blockIdx.x / nch, c = blockIdx.x % nch;
  lin_finish_row(a, r, c, false);
  if (a.epi.kind == 8) {
    const int nbs = a.epi.hid / 128, rg = a.epi.row0 + r;
    hc_fin_block(a, a.epi.ctr + (uint64_t)(nbs + rg * nbs + c % nbs) * kSyncStride, rg, rg + 1, c, &flag);
  }
}

// ------------------------------------------------------------------------------------------------ HC read
// The hyper-connection read's elementwise steps around the down and up linears (reference
// kernels/trunk6/t6_epi.metal:16-97). Four streams of hid columns per row; rr = bf16 rounding when refr.

// workgroup (row r, stream s, 256-column chunk ch), 256 threads (reference t6e_hc_prep, :16-50): every workgroup
// sums the whole stream's squares (independent loads, hid floats from L2), then prepares its own chunk:
// xn = (h w) inv, ip[r][s][ch][j] = (inject_j . (h w) over the chunk) inv, inj[r][4 + s] = inv (chunk 0).
__global__ __launch_bounds__(256) void hc_prep(const float *__restrict__ h, const uint16_t *__restrict__ nw,
                                               const uint16_t *__restrict__ iw, float *__restrict__ xn,
                                               float *__restrict__ ip, float *__restrict__ inj, int hid) {
  __shared__ float red[4][5];
  const int nch = (hid + 255) / 256;
  const int ch = blockIdx.x % nch, rs = blockIdx.x / nch, r = rs / kHcStreams, s = rs % kHcStreams;
  const int hcd = kHcStreams * hid, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float *hr = h + (uint64_t)r * hcd + (uint64_t)s * hid;
  // every load first (one round trip): the chunk's h, norm and inject weights, then the stream in batches of 16
  const int i = ch * 256 + threadIdx.x;
  const bool in = i < hid;
  const int ic = in ? i : 0;
  const float hv = hr[ic], wv = epi_bf(nw[s * hid + ic]);
  uint16_t iwv[4];
#pragma unroll
  for (int k = 0; k < 4; k++) iwv[k] = iw[(uint64_t)k * hcd + s * hid + ic];
  float ss = 0.f;
  constexpr int B = 16;
  for (int i0 = 0; i0 < hid; i0 += 256 * B) {
    float v[B];
#pragma unroll
    for (int u = 0; u < B; u++) {
      const int j = i0 + 256 * u + threadIdx.x;
      v[u] = hr[j < hid ? j : 0];
    }
#pragma unroll
    for (int u = 0; u < B; u++)
      if (i0 + 256 * u + (int)threadIdx.x < hid) ss += v[u] * v[u];
  }
  const float xv = in ? hv * wv : 0.f;
  float t[5] = {ss, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 4; k++) t[1 + k] = in ? epi_bf(iwv[k]) * xv : 0.f;
#pragma unroll
  for (int k = 0; k < 5; k++)
    for (int o = 32; o >= 1; o >>= 1) t[k] += __shfl_xor(t[k], o, 64);
  if (lane == 0)
    for (int k = 0; k < 5; k++) red[wave][k] = t[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 5; k++) t[k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
  const float inv = 1.f / sqrtf(t[0] / (float)hid + 1e-6f);
  if (in) xn[(uint64_t)r * hcd + s * hid + i] = xv * inv;
  if (threadIdx.x < 4) ip[((r * kHcStreams + s) * nch + ch) * 4 + threadIdx.x] = t[1 + threadIdx.x] * inv;
  if (threadIdx.x == 0 && ch == 0) inj[r * 8 + kHcStreams + s] = inv;
}

void launch_hc_prep(const float *h, const uint16_t *nw, const uint16_t *iw, float *xn, float *ip, float *inj, int R,
                    int hid, hipStream_t s) {
  hipLaunchKernelGGL(hc_prep, dim3(R * kHcStreams * ((hid + 255) / 256)), dim3(256), 0, s, h, nw, iw, xn, ip, inj,
                     hid);
}

// ------------------------------------------------------------------------------------------------ decode
// W' fp16 bits [IT*16][OT*16] from re-laid tiles: one wave per tile, grid ceil(IT * OTp / 4) x 256.
template <int K>
__global__ __launch_bounds__(256) void exl3_decode(const uint32_t *tiles, int IT, int OT, uint16_t *w) {
  const int lane = threadIdx.x & 63;
  const int OTp = OT + (OT & 1);
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= IT * OTp) return;
  const int j = t & 1, tk = (t >> 1) % IT, tn = 2 * ((t >> 1) / IT) + j;
  if (tn >= OT) return;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const TileWords tw = load_tile<K>(tiles + (uint64_t)t * 8 * K, L);
  f16x2 a, b;
  decode4<K>(tw, L.sh, a, b);
  const int q = (lane >> 1) & 3, col = (lane >> 3) + 8 * (lane & 1);
  const int rows[4] = {2 * q, 2 * q + 1, 2 * q + 8, 2 * q + 9};
  const _Float16 v[4] = {a.x, a.y, b.x, b.y};
  const uint64_t ld = (uint64_t)OT * 16;
#pragma unroll
  for (int i = 0; i < 4; i++)
    w[(uint64_t)(16 * tk + rows[i]) * ld + 16 * tn + col] = __builtin_bit_cast(uint16_t, v[i]);
}

// ------------------------------------------------------------------------------------------------ synthetic fills
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float gauss(uint64_t seed, uint64_t i) {  // Box-Muller on two 24-bit uniforms
  const uint64_t h = splitmix64(seed ^ (i * 0xD1B54A32D192ED03ull));
  const float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
  const float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
  return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
}
__global__ void fill_u32(uint32_t *p, uint64_t n, uint64_t seed) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = (uint32_t)splitmix64(seed * 0x100000001B3ull + i);
}
__global__ void fill_scale_f16(uint16_t *p, uint64_t n, uint64_t seed) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float m = fabsf(1.0f + 0.1f * gauss(seed, i));
    const bool neg = splitmix64(seed + 0x51ED27u + i) & 1u;
    p[i] = f2h(neg ? -m : m);
  }
}
// 8-bit affine group words (scale bf16 low, bias bf16 high): scale = |N(1, 0.1)| / (74 sqrt(in)) (a uniform byte has
// a standard deviation of ~74), bias = -127.5 scale, so that a row's weights have mean ~0 and variance ~1 / in
__global__ void fill_q8_sb(uint32_t *p, uint64_t n, int in, uint64_t seed) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float sc = bf16_round(fabsf(1.0f + 0.1f * gauss(seed, i)) / (74.f * sqrtf((float)in)));
    const float bi = bf16_round(-127.5f * sc);
    p[i] = (__float_as_uint(sc) >> 16) | (__float_as_uint(bi) & 0xFFFF0000u);
  }
}
__global__ void fill_normal_bf16(uint16_t *p, uint64_t n, uint64_t seed, float sd) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float v = sd * gauss(seed, i);
    p[i] = (uint16_t)(__float_as_uint(bf16_round(v)) >> 16);
  }
}

// ------------------------------------------------------------------------------------------------ launchers
static unsigned fill_grid(uint64_t n) {
  const uint64_t g = (n + 255) / 256;
  return (unsigned)(g < 65536 ? (g ? g : 1) : 65536);
}
void launch_fill_u32(uint32_t *p, uint64_t n, uint64_t seed, hipStream_t s) {
  hipLaunchKernelGGL(fill_u32, dim3(fill_grid(n)), dim3(256), 0, s, p, n, seed);
}
void launch_fill_scale_f16(uint16_t *p, uint64_t n, uint64_t seed, hipStream_t s) {
  hipLaunchKernelGGL(fill_scale_f16, dim3(fill_grid(n)), dim3(256), 0, s, p, n, seed);
}
void launch_fill_q8_sb(uint32_t *p, uint64_t n, int in, uint64_t seed, hipStream_t s) {
  hipLaunchKernelGGL(fill_q8_sb, dim3(fill_grid(n)), dim3(256), 0, s, p, n, in, seed);
}
void launch_fill_normal_bf16(uint16_t *p, uint64_t n, uint64_t seed, float sd, hipStream_t s) {
  hipLaunchKernelGGL(fill_normal_bf16, dim3(fill_grid(n)), dim3(256), 0, s, p, n, seed, sd);
}

void launch_moe_router(const MoeArgs &a, hipStream_t s) {
  const int rows = a.ne + a.has_sgate;
  hipLaunchKernelGGL(moe_router, dim3((rows + 3) / 4), dim3(256), 0, s, a);
}
void launch_moe_gateup(const MoeArgs &a, hipStream_t s) {
  const int NP = (a.inter / 16 + 1) / 2;
  hipLaunchKernelGGL(moe_gateup, dim3(a.R * a.nslot * 2 * NP * a.ksplit), dim3(256), 0, s, a);
}
void launch_moe_down(const MoeArgs &a, hipStream_t s) {
  const int NP = (a.hid / 16 + 1) / 2;
  hipLaunchKernelGGL(moe_down, dim3(a.R * a.nslot * NP), dim3(256), 0, s, a);
}
void launch_moe_combine(const MoeArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(moe_combine, dim3(a.R * ((a.hid + 127) / 128)), dim3(256), 0, s, a);
}
static int rows_tier(int R) { return R <= 1 ? 1 : R <= 2 ? 2 : R <= 4 ? 4 : R <= 8 ? 8 : R <= 16 ? 16 : 32; }
template <int K>
static const void *lin_mx_fn(int RT) {
  switch (RT) {
    case 1: return (const void *)&lin_mx<K, 1>;
    case 2: return (const void *)&lin_mx<K, 2>;
    case 4: return (const void *)&lin_mx<K, 4>;
    case 8: return (const void *)&lin_mx<K, 8>;
    case 16: return (const void *)&lin_mx<K, 16>;
    default: return (const void *)&lin_mx<K, 32>;
  }
}
static const void *lin_mx_any(int K, int RT) {
  const void *f = nullptr;
  IJ_DISPATCH_K(K, f = lin_mx_fn<KK>(RT));
  return f;
}
template <int K>
static const void *lin_mxl_fn(int RT) {
  switch (RT) {
    case 1: return (const void *)&lin_mxl<K, 1>;
    case 2: return (const void *)&lin_mxl<K, 2>;
    case 4: return (const void *)&lin_mxl<K, 4>;
    case 8: return (const void *)&lin_mxl<K, 8>;
    case 16: return (const void *)&lin_mxl<K, 16>;
    default: return (const void *)&lin_mxl<K, 32>;
  }
}
static const void *lin_mxl_any(int K, int RT) {
  const void *f = nullptr;
  IJ_DISPATCH_K(K, f = lin_mxl_fn<KK>(RT));
  return f;
}
template <int K>
static size_t lin_mxl_lds_fn(int RT, int G) {
  switch (RT) {
    case 1: return lin_mxl_lds<K, 1>(G);
    case 2: return lin_mxl_lds<K, 2>(G);
    case 4: return lin_mxl_lds<K, 4>(G);
    case 8: return lin_mxl_lds<K, 8>(G);
    case 16: return lin_mxl_lds<K, 16>(G);
    default: return lin_mxl_lds<K, 32>(G);
  }
}
static size_t lin_mxl_lds_any(int K, int RT, int G) {
  size_t n = 0;
  IJ_DISPATCH_K(K, n = lin_mxl_lds_fn<KK>(RT, G));
  return n;
}
constexpr int kLinWideWaves = 4;  // tile pairs (waves) per wide workgroup: one output block (8 measured slower)
template <int K>
static const void *lin_mxw_fn(int RT) {
  return RT <= 8 ? (const void *)&lin_mxw<K, 8, kLinWideWaves>
                 : RT <= 16 ? (const void *)&lin_mxw<K, 16, kLinWideWaves> : (const void *)&lin_mxw<K, 32, kLinWideWaves>;
}
static const void *lin_mxw_any(int K, int RT) {
  const void *f = nullptr;
  IJ_DISPATCH_K(K, f = lin_mxw_fn<KK>(RT));
  return f;
}
template <int K>
static size_t lin_mxw_lds_fn(int RT) {
  return RT <= 8    ? lin_mxw_lds<K, 8, kLinWideWaves>()
         : RT <= 16 ? lin_mxw_lds<K, 16, kLinWideWaves>()
                    : lin_mxw_lds<K, 32, kLinWideWaves>();
}
static size_t lin_mxw_lds_any(int K, int RT) {
  size_t n = 0;
  IJ_DISPATCH_K(K, n = lin_mxw_lds_fn<KK>(RT));
  return n;
}
template <int K>
static size_t lin_mx_lds_fn(int RT) {
  switch (RT) {
    case 1: return lin_mx_lds<K, 1>();
    case 2: return lin_mx_lds<K, 2>();
    case 4: return lin_mx_lds<K, 4>();
    case 8: return lin_mx_lds<K, 8>();
    case 16: return lin_mx_lds<K, 16>();
    default: return lin_mx_lds<K, 32>();
  }
}
static size_t lin_mx_lds_any(int K, int RT) {
  size_t n = 0;
  IJ_DISPATCH_K(K, n = lin_mx_lds_fn<KK>(RT));
  return n;
}

void launch_lin_multi(const LinArgs *l, int n, hipStream_t s) {
  IJ_CHECK(n >= 1 && n <= kLinMulti, "multi-linear launch of %d linears (1..%d)", n, kLinMulti);
  LinMulti m{};
  m.n = n;
  int wg = 0;
  for (int i = 0; i < n; i++) {
    const LinArgs &a = l[i];
    // every buffer a (possibly captured) launch uses is present, and the k groups fixed by the shape
    const int G = (a.IT + kLinGroupKt - 1) / kLinGroupKt;
    IJ_CHECK(a.tiles && a.suh && a.svh && a.x && a.y && a.xh && a.part && a.S == (a.kloop == 1 ? 1 : G),
             "linear launch: missing buffer or bad k groups (S %d of %d k tiles)", a.S, a.IT);
    IJ_CHECK(!a.kloop || (a.xh_in && G <= kLinLoopMaxGroups), "linear launch: the k-group loop needs the prep launch");
    IJ_CHECK(a.kloop != 2 || (n == 1 && a.R > 4 && a.R <= kLinMaxRows && a.cnt && a.epi.kind != 8),
             "linear launch: the wide form takes one linear of 5..32 rows with its counters and no HC epilogue");
    IJ_CHECK(!a.hc.nw || (n == 1 && a.R == 1 && !a.kloop && !a.xh_in && a.cnt && a.hc.iw && a.hc.ip && a.hc.inj &&
                          a.in == kHcStreams * a.hc.hid && a.hc.hid % 512 == 0 && a.hc.hid <= 4096),
             "linear launch: the HC read's input step folds into a one-row, one-launch down linear only");
    IJ_CHECK(a.K == l[0].K && a.R == l[0].R && a.R >= 1 && a.R <= kLinMaxRows && (bool)a.cnt == (bool)l[0].cnt &&
                 a.kloop == l[0].kloop,
             "multi-linear launch: K, R and path must agree");
    if (a.xh_in) hipLaunchKernelGGL(lin_prep, dim3(a.R * ((a.in + 127) / 128)), dim3(64), 0, s, a);
    m.l[i] = a;
    m.wg0[i] = wg;
    wg += a.kloop == 2 ? ((a.OT + 1) / 2 + kLinWideWaves - 1) / kLinWideWaves * a.S
                       : ((a.OT + 1) / 2) * (a.kloop ? 1 : a.S);
  }
  m.wg0[n] = wg;
  const int RT = rows_tier(l[0].R);
  void *args[] = {&m};
  if (l[0].kloop == 2) {
    IJ_HIP(hipLaunchKernel(lin_mxw_any(l[0].K, RT), dim3(wg), dim3(64 * kLinWideWaves), args,
                           lin_mxw_lds_any(l[0].K, RT), s));
  } else if (l[0].kloop) {
    int G = 0;
    for (int i = 0; i < n; i++) G = std::max(G, (l[i].IT + kLinGroupKt - 1) / kLinGroupKt);
    IJ_HIP(hipLaunchKernel(lin_mxl_any(l[0].K, RT), dim3(wg), dim3(256), args, lin_mxl_lds_any(l[0].K, RT, G), s));
  } else {
    IJ_HIP(hipLaunchKernel(lin_mx_any(l[0].K, RT), dim3(wg), dim3(256), args, lin_mx_lds_any(l[0].K, RT), s));
  }
  if (!l[0].cnt)  // staged path: the finisher as its own launch
    for (int i = 0; i < n; i++)
      hipLaunchKernelGGL(lin_finish, dim3(l[i].R * ((l[i].out + 127) / 128)), dim3(64), 0, s, l[i]);
}
void launch_lin(const LinArgs &a, hipStream_t s) { launch_lin_multi(&a, 1, s); }

// the dynamic LDS limits of lin_mx, once at device set-up
void init_lin_attrs() {
  for (int K = 2; K <= 8; K++)
    for (int RT : {1, 2, 4, 8, 16, 32})
      IJ_HIP(hipFuncSetAttribute(lin_mx_any(K, RT), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)lin_mx_lds_any(K, RT)));
  for (int K = 2; K <= 8; K++)
    for (int RT : {1, 2, 4, 8, 16, 32})
      IJ_HIP(hipFuncSetAttribute(lin_mxl_any(K, RT), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)std::min<size_t>(160 * 1024 - 256, lin_mxl_lds_any(K, RT, kLinLoopMaxGroups))));
  for (int K = 2; K <= 8; K++)
    for (int RT : {8, 16, 32})
      IJ_HIP(hipFuncSetAttribute(lin_mxw_any(K, RT), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)lin_mxw_lds_any(K, RT)));
}

static const void *decode_fn(int K) {
  const void *f = nullptr;
  IJ_DISPATCH_K(K, f = (const void *)&exl3_decode<KK>);
  return f;
}
void launch_decode(const uint32_t *tiles, int IT, int OT, int K, uint16_t *w, hipStream_t s) {
  const int OTp = OT + (OT & 1);
  const void *f = decode_fn(K);
  IJ_CHECK(f, "decode: K %d not instantiated", K);
  void *args[] = {&tiles, &IT, &OT, &w};
  IJ_HIP(hipLaunchKernel(f, dim3((IT * OTp + 3) / 4), dim3(256), args, 0, s));
}

// ------------------------------------------------------------------------------------------------ registry
static std::vector<KernelEntry> build_registry() {
  std::vector<KernelEntry> v;
  const uint32_t P = sizeof(void *), I = sizeof(int);
  for (int K = 2; K <= 8; K++) {
    v.push_back({"exl3_decode", decode_fn(K), {P, I, I, P}, K, -1});
    for (int RT : {1, 2, 4, 8, 16, 32}) v.push_back({"lin_mx", lin_mx_any(K, RT), {(uint32_t)sizeof(LinMulti)}, K, RT});
  }
  v.push_back({"lin_prep", (const void *)&lin_prep, {(uint32_t)sizeof(LinArgs)}, -1, -1});
  v.push_back({"lin_finish", (const void *)&lin_finish, {(uint32_t)sizeof(LinArgs)}, -1, -1});
  v.push_back({"moe_router", (const void *)&moe_router, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  v.push_back({"moe_gateup", (const void *)&moe_gateup, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  v.push_back({"moe_down", (const void *)&moe_down, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  v.push_back({"moe_combine", (const void *)&moe_combine, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  for (int K = 4; K <= 6; K++)
    for (int KS = 4; KS <= 6; KS++)
      if (const void *f = moe_fused_kernel(K, KS, 2048, 512))
        v.push_back({"moe_step_2048x512_ks" + std::to_string(KS), f, {(uint32_t)sizeof(MoeArgs)}, K, -1});
  v.push_back({"fill_u32", (const void *)&fill_u32, {P, 8, 8}, -1, -1});
  return v;
}

const KernelEntry *find_kernel(const char *name, const ne_fconst *fc, int nfc) {
  static const std::vector<KernelEntry> reg = build_registry();
  int K = -1, R = -1;
  for (int i = 0; i < nfc; i++) {
    if (fc[i].index == 10) K = (int)fc[i].bits;
    else if (fc[i].index == 16) R = (int)fc[i].bits;
  }
  for (const KernelEntry &e : reg) {
    if (e.name != name) continue;
    if (e.K >= 0 && K >= 0 && e.K != K) continue;
    if (e.R >= 0 && R >= 0 && e.R != R) continue;
    return &e;
  }
  return nullptr;
}

}  // namespace ijah
