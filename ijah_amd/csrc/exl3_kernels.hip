// EXL3 trellis decode fused into GEMV / MoE expert kernels for CDNA4 (gfx950), wave64.
//
// Format (reference kernels/ne_common.h:105-161, kernels/trunk6/trunk6.metal:87-127): a 16x16 tile of W' is a
// tail-biting ring of 256 K bits held as 16 K u16 halfwords read as little-endian u32 words, bits consumed MSB
// first. The codeword of slot i is the 15 ring bits ending at bit (i+1) K; its value is the MCG codebook entry
// fp16(fp16(r_lo) + fp16(r_hi)), r = (cw * 0xCBAC1FED) & 0x8FFF8FFF ^ 0x3B603B60. Slot s = 8l + j of the reference's
// 32-lane order holds row (2q, 2q+1, 2q+8, 2q+9)[j & 3] (q = l & 3) at column (l >> 2) + 8 (j >> 2).
//
// Wave64 mapping (this build's own): lane m of a wave owns slots 4m .. 4m+3 of a tile, i.e. rows 2q, 2q+1, 2q+8,
// 2q+9 (q = (m >> 1) & 3) of column (m >> 3) + 8 (m & 1). Its four codewords span 15 + 3K ring bits starting at
// (4m + 1) K - 15: one funnel shift (v_alignbit) of two words for K <= 5, two funnels of three words above. The input
// is staged in LDS as fp16 in the reference's k-permuted order (kp), so a lane's four rows are one 8-byte read, and the
// four weights meet it in two v_dot2_f32_f16. Lanes sharing a column differ in lane bits 1-2: two xor-shuffles reduce.
//
// Hadamard transforms hold 128 elements as (lane, lane + 64) and run the butterflies over index bits 0..6 in order
// (lane shuffles for bits 0-5, the register pair for bit 6) with lo + hi / lo - hi in f32, then one multiply by
// f32(1/sqrt n): the same operations, in the same order, as the reference's fwht128 / t6_fwht
// (kernels/ne_common.h:93-103, kernels/trunk6/trunk6.metal:42-51), so the fp16-rounded prepared input is
// bit-identical to the reference arithmetic. The library is compiled with -ffp-contract=off for that reason.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "kernels.h"

namespace ijah {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------------ scalar helpers
__device__ __forceinline__ float bf16_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float bf16_round(float x) {  // reference kernels/ne_common.h:23-26
  uint32_t u = __float_as_uint(x);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  return __uint_as_float(u);
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// f32 -> fp16 (RNE) of a value already rounded to f32: the empty asm keeps the compiler from folding a preceding
// multiply into the conversion (v_fma_mix*), which would round once from the exact product instead of twice.
__device__ __forceinline__ _Float16 to_f16(float f) {
  asm("" : "+v"(f));
  return (_Float16)f;
}
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, to_f16(f)); }
// position of input p inside its 16-block in the lane order (2q, 2q+1, 2q+8, 2q+9): reference kernels/ne_common.h:158-161
__device__ __forceinline__ uint32_t kp(uint32_t p) {
  return (p & ~15u) | (((p & 7u) >> 1) << 2) | (p & 1u) | (((p >> 3) & 1u) << 1);
}

// Data handed between workgroups (logits, route, gate/up and down partials) moves with device-coherent accesses
// (agent-scope relaxed atomics: sc1 loads / stores, which bypass the per-XCD L2's non-coherent lines), so ordering
// needs only s_waitcnt + barriers: no agent-scope fence, which on CDNA writes back or invalidates the whole L2.
template <typename T>
__device__ __forceinline__ T ld_cg(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_cg(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------ Hadamard
// normalised Sylvester H_N (N = 16..128) on a 128-chunk held as (lane, lane + 64); blocks of N are contiguous.
__device__ __forceinline__ void fwht2(float &v0, float &v1, int lane, int N, float sc) {
#pragma unroll
  for (int bit = 1; bit < 64; bit <<= 1) {
    if (bit < N) {
      const float p0 = __shfl_xor(v0, bit, 64), p1 = __shfl_xor(v1, bit, 64);
      const bool up = (lane & bit) != 0;
      v0 = up ? p0 - v0 : v0 + p0;
      v1 = up ? p1 - v1 : v1 + p1;
    }
  }
  if (N >= 128) {
    const float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
  }
  v0 *= sc;
  v1 *= sc;
}

// ------------------------------------------------------------------------------------------------ trellis reader
template <int K>
struct TileLane {
  uint32_t i0, i1, i2, sh;  // word indices inside the tile; funnel shift
};
// Lane m's window starts at ring bit S = (4m + 1) K - 15 (mod 256 K). Taking i0 = floor((S - 1) / 32) puts the
// window's first bit at a' = S - 32 i0 in [1, 32] of words (i0, i0+1), so v_alignbit(w0, w1, 32 - a') yields the
// window's first 32 bits with no special case for a' = 32.
template <int K>
__device__ __forceinline__ TileLane<K> tile_lane(uint32_t m) {
  constexpr uint32_t NW = 8u * K, TOT = 256u * K;
  const uint32_t S = ((4u * m + 1u) * K + TOT - 15u) % TOT;
  const uint32_t Sm1 = (S + TOT - 1u) % TOT;
  TileLane<K> t;
  t.i0 = Sm1 >> 5;
  t.i1 = (t.i0 + 1u) % NW;
  t.i2 = (t.i0 + 2u) % NW;
  t.sh = 31u - (Sm1 & 31u);
  return t;
}
template <int K>
constexpr bool kThreeWords = (15 + 3 * K > 32);

struct TileWords {
  uint32_t w0, w1, w2;
};
template <int K>
__device__ __forceinline__ TileWords load_tile(const uint32_t *__restrict__ T, const TileLane<K> &L) {
  TileWords w;
  w.w0 = __builtin_nontemporal_load(T + L.i0);
  w.w1 = __builtin_nontemporal_load(T + L.i1);
  w.w2 = kThreeWords<K> ? __builtin_nontemporal_load(T + L.i2) : 0u;
  return w;
}

// MCG window-15 codebook (reference kernels/ne_common.h:139-144): r = cw * 0xCBAC1FED mod 2^32, masked, xored;
// value = fp16(r_lo) + fp16(r_hi) rounded once (RNE), as the reference's half + half.
// The 32-bit multiply is quarter rate on CDNA; cw < 2^15 lets two full-rate 24-bit multiplies form it:
// v_mul_u32_u24 (SDWA, dst WORD_1) writes lo16(cw * 0xCBAC) << 16, v_mad_u32_u24 adds cw * 0x1FED.
__device__ __forceinline__ uint32_t mcg_bits(uint32_t cw) {
  uint32_t t, r;
  asm("v_mul_u32_u24_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
      : "=v"(t)
      : "v"(cw), "s"(0xCBACu));
  asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(r) : "v"(cw), "s"(0x1FEDu), "v"(t));
  return (r & 0x8FFF8FFFu) ^ 0x3B603B60u;
}
// two codewords -> their fp16 values packed (c0 low, c1 high): each v_add_f16 (SDWA) adds the two halves of one r
// and writes one half of the result, so no pack instruction is needed.
__device__ __forceinline__ f16x2 mcg_pair(uint32_t c0, uint32_t c1) {
  const uint32_t r0 = mcg_bits(c0), r1 = mcg_bits(c1);
  uint32_t d;
  asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
      : "=v"(d)
      : "v"(r0));
  asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
      : "+v"(d)
      : "v"(r1));
  return __builtin_bit_cast(f16x2, d);
}

// The lane's four weights: a = rows (2q, 2q+1), b = rows (2q+8, 2q+9) of its column.
template <int K>
__device__ __forceinline__ void decode4(const TileWords &w, uint32_t sh, f16x2 &a, f16x2 &b) {
  uint32_t c[4];
  const uint32_t hi = __builtin_amdgcn_alignbit(w.w0, w.w1, sh);
  if constexpr (!kThreeWords<K>) {
#pragma unroll
    for (int i = 0; i < 4; i++) c[i] = (hi >> (17 - i * K)) & 0x7FFFu;
  } else {
    const uint32_t lo = __builtin_amdgcn_alignbit(w.w1, w.w2, sh);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int s = 49 - i * K;
      c[i] = (s >= 32 ? (hi >> (s - 32)) : __builtin_amdgcn_alignbit(hi, lo, (uint32_t)s)) & 0x7FFFu;
    }
  }
  a = mcg_pair(c[0], c[1]);
  b = mcg_pair(c[2], c[3]);
}

__device__ __forceinline__ float dot4(f16x2 a, f16x2 b, f16x4 x, float acc) {
  acc = __builtin_amdgcn_fdot2(a, f16x2{x.x, x.y}, acc, false);
  return __builtin_amdgcn_fdot2(b, f16x2{x.z, x.w}, acc, false);
}

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
__device__ __forceinline__ void lane_col_reduce(float &acc0, float &acc1) {
  acc0 += __shfl_xor(acc0, 2, 64);
  acc0 += __shfl_xor(acc0, 4, 64);
  acc1 += __shfl_xor(acc1, 2, 64);
  acc1 += __shfl_xor(acc1, 4, 64);
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
// Wave-wide max of a u32 (DPP within rows of 16, then the 4 rows' maxima through readlane): uniform result.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  // every lane of a row holds the row max; row_bcast:15 / :31 carry it to the next row(s); lane 63 ends with all
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));  // row_bcast:15
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}
// Order key of a bf16-valued logit and its index: a larger key is a larger logit, equal logits order the lower index
// first (the reference's tie rule, kernels/fn_moe.metal:84,105). NaN ranks as -inf, -0 as +0. Zero is below every key.
__device__ __forceinline__ uint32_t topk_key(float v, int i) {
  if (v != v) v = -INFINITY;
  if (v == 0.f) v = 0.f;
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (u & 0xFFFF0000u) | (0xFFFFu - (uint32_t)i);
}
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
      st_cg(a.sgv + r, a.has_sgate ? 1.f / (1.f + expf(-ld_cg(a.logits + (uint64_t)r * ld + a.ne))) : 1.f);
    }
    __syncthreads();
  }
}

// optional unit trace (MoeArgs::trace): [u][0] = wall clock at the take, [1] = after the unit's waits, [2] = done,
// [3] = workgroup id
__device__ __forceinline__ void trace_mark(const MoeArgs &a, int u, int total, int field) {
  if (a.trace && threadIdx.x == 0 && u < total) {
    a.trace[(uint64_t)u * 8 + field] = wall_clock64();
    if (field == 0) a.trace[(uint64_t)u * 8 + 7] = blockIdx.x;
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
    float y = 0.f;
    for (int k = 0; k < a.nslot; k++) y += vs[k][threadIdx.x];
    if (i < a.hid) a.y[(uint64_t)r * a.hid + i] = y;
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

// ------------------------------------------------------------------------------------------------ fused layer kernel
// The whole layer step in one launch, one 8-wave workgroup per CU. Work comes from three ordered queues (atomic heads):
//   A: router units (one router row per wave); the last to finish computes the route and publishes it;
//   G: gate/up wave units (slot, gate|up, k split, output tile pair): [shared slots][routed slots, slot-major];
//   D: down wave units (slot, output tile pair), per row the shared slot first.
// A wave unit is one output tile pair over 32 k tiles (64 tiles: 10 KB at K5), the work of one wave. Each round a
// workgroup takes NG gate/up and ND down units and streams all their tiles straight into LDS (global_load_lds_dwordx4)
// before computing, so the chip has nearly the whole layer's expert weights in flight once the route is known, and
// every CU takes part in both the gate/up and the down phase. A round's gate/up units are computed and signalled
// before its down units wait, so a round never waits on itself; units only wait on units earlier in the queues,
// which running workgroups hold, so progress does not depend on how many workgroups are resident. The last down unit
// of each (row, 128-column block) combines it (fixed slot order). The last workgroup to leave resets every counter
// for the next launch.
constexpr int kF2Waves = 16;
constexpr int kF2KT = 32;    // k tiles per wave unit
constexpr int kMaxRows = 4;  // rows (tokens) of one fused step
constexpr uint32_t kF2UnitBytesK = 2 * kF2KT * 32;  // LDS bytes of one wave unit's tiles per unit of K (x K)
enum {
  kSyncHeadG = 4 * kSyncStride,
  kSyncHeadD = 5 * kSyncStride,
  kSyncRouteReady2 = 6 * kSyncStride,
  kSyncExit = 7 * kSyncStride
};
// units per round (gate/up, down) by the widest bit width: the LDS holds NG + ND wave units
template <int KM>
struct F2Take {
  static constexpr int NG = KM <= 6 ? 6 : 5;
  static constexpr int ND = KM <= 6 ? 3 : 2;
};

struct F2Shape {
  int nA, NPg, NPd, gu_slot, nsh, nG, nD, nblk, IT, ITd;
};
__device__ __forceinline__ F2Shape f2_shape(const MoeArgs &a) {
  F2Shape f;
  f.nA = (a.ne + a.has_sgate + kF2Waves - 1) / kF2Waves;  // one router row per wave
  f.NPg = a.inter / 32;
  f.NPd = a.hid / 32;
  f.gu_slot = 2 * a.ksplit * f.NPg;
  f.nsh = (a.nslot > a.topk) ? a.R * f.gu_slot : 0;
  f.nG = f.nsh + a.R * a.topk * f.gu_slot;
  f.nD = a.R * a.nslot * f.NPd;
  f.nblk = a.hid / 128;
  f.IT = a.hid / 16;
  f.ITd = a.inter / 16;
  return f;
}

struct F2Route {  // the workgroup's copy of the route
  uint32_t id[kMaxRows][kMaxTopk];
  float w[kMaxRows][kMaxTopk];
  float sg[kMaxRows];
  int ready;
};

struct F2Unit {
  int valid, r, k, slot, proj, ks, p, sh;
};
__device__ __forceinline__ F2Unit f2_gu_unit(const MoeArgs &a, const F2Shape &f, int v) {
  F2Unit u;
  u.valid = v < f.nG;
  int w;
  if (v < f.nsh) {
    u.r = v / f.gu_slot;
    u.k = a.topk;
    w = v % f.gu_slot;
  } else {
    const int v2 = v - f.nsh, sidx = v2 / f.gu_slot;
    u.r = sidx / a.topk;
    u.k = sidx % a.topk;
    w = v2 % f.gu_slot;
  }
  u.proj = w / (a.ksplit * f.NPg);
  u.ks = (w / f.NPg) % a.ksplit;
  u.p = w % f.NPg;
  u.slot = u.r * a.nslot + u.k;
  u.sh = u.k >= a.topk;
  return u;
}
__device__ __forceinline__ F2Unit f2_dn_unit(const MoeArgs &a, const F2Shape &f, int v) {
  F2Unit u;
  u.valid = v < f.nD;
  const int q = v / f.NPd, j = q % a.nslot;
  u.p = v % f.NPd;
  u.r = q / a.nslot;
  u.k = (a.nslot > a.topk) ? (j == 0 ? a.topk : j - 1) : j;
  u.slot = u.r * a.nslot + u.k;
  u.sh = u.k >= a.topk;
  u.proj = 2;
  u.ks = 0;
  return u;
}

// Route of every row from the logits, by the last router workgroup, published to the route / shared-gate buffers.
__device__ void f2_route_publish(const MoeArgs &a, float *lv, uint32_t *cand, uint32_t *sid, int tu) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ld = a.ne + 1;
  for (int r = 0; r < a.R; r++) {
    for (int i = threadIdx.x; i < a.ne; i += blockDim.x) lv[i] = ld_cg(a.logits + (uint64_t)r * ld + i);
    __syncthreads();
    trace_mark(a, tu, 1 << 30, 3);
    block_topk(lv, a.ne, a.topk, cand, sid);
    trace_mark(a, tu, 1 << 30, 4);
    if (wave == 0) {
      const uint32_t id = lane < a.topk ? sid[lane] : 0u;
      const float top = lv[sid[0]];
      const float pk = lane < a.topk ? expf(lv[id] - top) : 0.f;
      float s = 0.f;
      for (int k = 0; k < a.topk; k++) s += __shfl(pk, k, 64);  // slot order, as the reference's finisher
      if (lane < a.topk) {
        st_cg(a.route + (uint64_t)r * 2 * a.topk + lane, id);
        st_cg(a.route + (uint64_t)r * 2 * a.topk + a.topk + lane, __float_as_uint(pk / s));
      }
      if (lane == 0)
        st_cg(a.sgv + r, a.has_sgate ? 1.f / (1.f + expf(-ld_cg(a.logits + (uint64_t)r * ld + a.ne))) : 1.f);
    }
    __syncthreads();
  }
}
// the workgroup's copy of the published route (waits for it)
__device__ bool f2_route_fetch(const MoeArgs &a, F2Route *rt, int *flag) {
  if (!block_wait_geq(a.sync, a.sync + kSyncRouteReady2, 1u, flag)) return false;
  for (int i = threadIdx.x; i < a.R * a.topk; i += blockDim.x) {
    const int r = i / a.topk, k = i % a.topk;
    rt->id[r][k] = ld_cg(a.route + (uint64_t)r * 2 * a.topk + k);
    rt->w[r][k] = __uint_as_float(ld_cg(a.route + (uint64_t)r * 2 * a.topk + a.topk + k));
  }
  if (threadIdx.x < a.R) rt->sg[threadIdx.x] = ld_cg(a.sgv + threadIdx.x);
  if (threadIdx.x == 0) rt->ready = 1;
  __syncthreads();
  return true;
}

__device__ __forceinline__ const uint8_t *f2_block(const MoeArgs &a, const F2Route *rt, int r, int k) {
  if (k >= a.topk) return a.shared;
  uint32_t e = rt->id[r][k];
  e = e < (uint32_t)a.ne ? e : 0u;
  return a.experts + (uint64_t)e * a.lay.bytes;
}

// stream a wave unit's tiles (pair p, k tiles [k0, k0 + nkt) of a re-laid matrix) into this wave's LDS buffer
__device__ __forceinline__ void f2_stream(const uint8_t *tr, int IT, int p, int k0, int nkt, uint32_t tb,
                                          uint8_t *dst) {
  const int lane = threadIdx.x & 63;
  const uint8_t *src = tr + ((uint64_t)p * IT + k0) * 2 * tb;
  const uint32_t bytes = (uint32_t)nkt * 2 * tb;
  for (uint32_t o = 0; o < bytes; o += 1024)
    if (o + (uint32_t)lane * 16 < bytes)
      __builtin_amdgcn_global_load_lds((const void *)(src + o + lane * 16),
                                       (__attribute__((address_space(3))) void *)(dst + o), 16, 0, 0);
}

// one wave: its unit's output tile pair over nkt k tiles from the LDS-staged tiles; returns the two column sums on
// the lanes with (lane & 6) == 0 (column (lane >> 3) + 8 (lane & 1) of each tile)
template <int K>
__device__ __forceinline__ void f2_pair_dot(const uint8_t *tl, const _Float16 *xs, int nkt, float &acc0, float &acc1) {
  constexpr int TW = 8 * K;
  const int lane = threadIdx.x & 63;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const int q = (lane >> 1) & 3;
  acc0 = 0.f;
  acc1 = 0.f;
  const uint32_t *T = (const uint32_t *)tl;
#pragma unroll 4
  for (int kt = 0; kt < nkt; kt++) {
    const uint32_t *T0 = T + kt * 2 * TW;
    TileWords wa, wb;
    wa.w0 = T0[L.i0];
    wa.w1 = T0[L.i1];
    wa.w2 = kThreeWords<K> ? T0[L.i2] : 0u;
    wb.w0 = T0[TW + L.i0];
    wb.w1 = T0[TW + L.i1];
    wb.w2 = kThreeWords<K> ? T0[TW + L.i2] : 0u;
    const f16x4 xv = *(const f16x4 *)(xs + kt * 16 + 4 * q);
    f16x2 a0, b0, a1, b1;
    decode4<K>(wa, L.sh, a0, b0);
    decode4<K>(wb, L.sh, a1, b1);
    acc0 = dot4(a0, b0, xv, acc0);
    acc1 = dot4(a1, b1, xv, acc1);
  }
  lane_col_reduce(acc0, acc1);
}

// combine for (row r, 128-column block c) from the workgroup's route copy (the arithmetic of combine_block)
__device__ void f2_combine(const MoeArgs &a, const F2Route *rt, int r, int c, float (*vs)[128]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (int)(blockDim.x >> 6);
  const int i0 = c * 128 + lane, i1 = i0 + 64;
  for (int k = wave; k < a.nslot; k += nw) {
    const int slot = r * a.nslot + k;
    const uint8_t *blk = f2_block(a, rt, r, k);
    const int sh = k >= a.topk;
    const float w = sh ? rt->sg[r] : rt->w[r][k];
    const float *d = a.dn + (uint64_t)slot * a.hid;
    const uint16_t *sv = (const uint16_t *)(blk + off_sv(a, sh, 2));
    float v0 = ld_cg(d + i0), v1 = ld_cg(d + i1);
    const float s0 = h2f(sv[i0]), s1 = h2f(sv[i1]);
    fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
    vs[k][lane] = v0 * s0 * w;
    vs[k][lane + 64] = v1 * s1 * w;
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    float y = 0.f;
    for (int k = 0; k < a.nslot; k++) y += vs[k][threadIdx.x];
    a.y[(uint64_t)r * a.hid + c * 128 + threadIdx.x] = y;
  }
  __syncthreads();
}

// Gate/up block finisher: the last gate/up unit of (slot, 128-column block cb of inter) sums the k splits in order and
// applies the down unit's prologue (reference kernels/fn_moe.metal:370-384): g = H(inner_g) * svh_g,
// u = H(inner_u) * svh_u, h = H(silu(g) u * suh_d), rounded to fp16 and stored in the k-permuted order the down units
// stage (hprep). One wave; `stage` = 128 halves of this wave's LDS.
constexpr int kMaxKsplit = 8;
__device__ void f2_gu_finish(const MoeArgs &a, const uint8_t *blk, int sh, int slot, int cb, _Float16 *stage) {
  const int lane = threadIdx.x & 63, inter = a.inter;
  const float *gp = a.guo + (uint64_t)slot * 2 * a.ksplit * inter;
  const float *up = gp + (uint64_t)a.ksplit * inter;
  const int i0 = cb * 128 + lane, i1 = i0 + 64;
  float gv[kMaxKsplit][2], uv[kMaxKsplit][2];
#pragma unroll
  for (int s2 = 0; s2 < kMaxKsplit; s2++) {  // every partial requested before the first is used
    if (s2 < a.ksplit) {
      gv[s2][0] = ld_cg(gp + s2 * inter + i0);
      gv[s2][1] = ld_cg(gp + s2 * inter + i1);
      uv[s2][0] = ld_cg(up + s2 * inter + i0);
      uv[s2][1] = ld_cg(up + s2 * inter + i1);
    }
  }
  const float sg0 = h2f(((const uint16_t *)(blk + off_sv(a, sh, 0)))[i0]);
  const float sg1 = h2f(((const uint16_t *)(blk + off_sv(a, sh, 0)))[i1]);
  const float su0 = h2f(((const uint16_t *)(blk + off_sv(a, sh, 1)))[i0]);
  const float su1 = h2f(((const uint16_t *)(blk + off_sv(a, sh, 1)))[i1]);
  const float sd0 = h2f(((const uint16_t *)(blk + off_su(a, sh, 2)))[i0]);
  const float sd1 = h2f(((const uint16_t *)(blk + off_su(a, sh, 2)))[i1]);
  float g0 = gv[0][0], g1 = gv[0][1], u0 = uv[0][0], u1 = uv[0][1];
#pragma unroll
  for (int s2 = 1; s2 < kMaxKsplit; s2++) {
    if (s2 < a.ksplit) {
      g0 += gv[s2][0];
      g1 += gv[s2][1];
      u0 += uv[s2][0];
      u1 += uv[s2][1];
    }
  }
  fwht2(g0, g1, lane, a.had_inter, a.sc_inter);
  fwht2(u0, u1, lane, a.had_inter, a.sc_inter);
  g0 = g0 * sg0;
  u0 = u0 * su0;
  g1 = g1 * sg1;
  u1 = u1 * su1;
  float h0 = g0 / (1.f + expf(-g0)) * u0 * sd0;
  float h1 = g1 / (1.f + expf(-g1)) * u1 * sd1;
  fwht2(h0, h1, lane, a.had_inter, a.sc_inter);
  stage[kp(lane)] = to_f16(h0);
  stage[kp(lane + 64)] = to_f16(h1);
  __builtin_amdgcn_wave_barrier();
  const uint32_t word = ((const uint32_t *)stage)[lane];  // 128 halves = 64 words, one per lane
  st_cg((uint32_t *)(a.hprep + (uint64_t)slot * inter + cb * 128) + lane, word);
}

#define IJ_F2_K(SH, CALL)   \
  if (SH) {                 \
    constexpr int KK = KS;  \
    CALL;                   \
  } else {                  \
    constexpr int KK = K;   \
    CALL;                   \
  }

template <int K, int KS>
__global__ __launch_bounds__(1024, 1) void moe_fused(MoeArgs a) {
  constexpr int KM = K > KS ? K : KS;
  constexpr int NG = F2Take<KM>::NG, ND = F2Take<KM>::ND;
  constexpr uint32_t UB = kF2UnitBytesK * KM;  // LDS bytes per wave unit buffer
  extern __shared__ __attribute__((aligned(16))) uint8_t f2_tiles[];  // (NG + ND) x UB
  __shared__ _Float16 prep_g[NG][512];
  __shared__ _Float16 prep_d[ND][512];
  __shared__ float red[kF2Waves][32];
  __shared__ float lv[kMaxExperts];
  __shared__ uint32_t sid[kMaxTopk];
  __shared__ float vs[kMaxSlots][128];
  __shared__ F2Route rt;
  __shared__ int flag, s_g, s_d, s_last[ND], s_fin[NG];
  const F2Shape f = f2_shape(a);
  uint32_t *sync = a.sync;
  uint32_t *gu_done = sync + kSyncSlots;                        // [slot * kSyncStride]: finished 128-blocks
  uint32_t *blk_cnt = gu_done + a.R * a.nslot * kSyncStride;    // [(r * nblk + c) * kSyncStride]
  uint32_t *fin_cnt = blk_cnt + a.R * f.nblk * kSyncStride;     // [(slot * nbi + cb) * kSyncStride]
  const int nbi = a.inter / 128;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = (int)gridDim.x;
  if (threadIdx.x == 0) rt.ready = 0;

  // ---- queue A: router rows (the first G statically, one per workgroup); the last to finish publishes the route
  for (int u = blockIdx.x;;) {
    if (u >= f.nA) break;
    trace_mark(a, u, 1 << 30, 0);
    router_rows(a, u, &vs[0][0]);
    trace_mark(a, u, 1 << 30, 1);
    if (block_signal(sync + kSyncRouterDone, &flag) == (uint32_t)f.nA - 1u) {
      f2_route_publish(a, lv, nullptr, sid, u);
      trace_mark(a, u, 1 << 30, 5);
      block_signal(sync + kSyncRouteReady2, &flag);
    }
    trace_mark(a, u, 1 << 30, 2);
    if (threadIdx.x == 0) s_g = G + (int)atomicAdd(sync + kSyncHead, 1u);
    __syncthreads();
    u = s_g;
    __syncthreads();
  }

  // ---- rounds of NG gate/up + ND down wave units; the first round is static, later ones come from the heads.
  // Waves: gate/up task w < 2 NG = unit w / 2, k half w % 2; down task w < 4 ND = unit w / 4, k quarter w % 4;
  // stream: wave w < NG + ND loads unit buffer w (gate/up units first).
  for (int round = 0;; round++) {
    if (round > 0) {
      if (threadIdx.x == 0) {
        s_g = G * NG + (int)atomicAdd(sync + kSyncHeadG, (uint32_t)NG);
        s_d = G * ND + (int)atomicAdd(sync + kSyncHeadD, (uint32_t)ND);
      }
      __syncthreads();
    }
    const int g0 = round > 0 ? s_g : (int)blockIdx.x * NG, d0 = round > 0 ? s_d : (int)blockIdx.x * ND;
    __syncthreads();
    if (g0 >= f.nG && d0 >= f.nD) break;
    const int tu = f.nA + g0 / NG;
    trace_mark(a, tu, 1 << 30, 0);
    bool routed = false;
#pragma unroll
    for (int i = 0; i < NG; i++) routed |= (g0 + i < f.nG) && (g0 + i >= f.nsh);
    routed |= d0 < f.nD;
    if (routed && !rt.ready && !f2_route_fetch(a, &rt, &flag)) continue;
    trace_mark(a, tu, 1 << 30, 1);

    const int gi = wave >> 1, gh = wave & 1, dj = wave >> 2, dq = wave & 3;
    const F2Unit Gt = f2_gu_unit(a, f, g0 + gi);                 // this wave's gate/up task unit
    const bool hasG = wave < 2 * NG && Gt.valid;
    const uint8_t *gblk = hasG ? f2_block(a, &rt, Gt.r, Gt.k) : nullptr;
    // gate/up prep inputs (this wave's two 128-chunks of its unit's 512) first, then the tile stream
    float xv[4], sv[4];
    if (hasG) {
      const float *x = a.x + (uint64_t)Gt.r * a.hid + Gt.ks * kF2KT * 16 + gh * 256;
      const uint16_t *su = (const uint16_t *)(gblk + off_su(a, Gt.sh, Gt.proj)) + Gt.ks * kF2KT * 16 + gh * 256;
#pragma unroll
      for (int h = 0; h < 4; h++) {
        xv[h] = x[h * 64 + lane];
        sv[h] = h2f(su[h * 64 + lane]);
      }
    }
    if (wave < NG + ND) {  // stream one unit's tiles
      const bool isg = wave < NG;
      const F2Unit S = isg ? f2_gu_unit(a, f, g0 + wave) : f2_dn_unit(a, f, d0 + wave - NG);
      if (S.valid) {
        const uint8_t *sblk = f2_block(a, &rt, S.r, S.k);
        const uint32_t tb = 32u * (uint32_t)(S.sh ? KS : K);
        if (isg)
          f2_stream(sblk + off_tr(a, S.sh, S.proj), f.IT, S.p, S.ks * kF2KT, kF2KT, tb, f2_tiles + (uint32_t)wave * UB);
        else
          f2_stream(sblk + off_tr(a, S.sh, 2), f.ITd, S.p, 0, f.ITd, tb, f2_tiles + (uint32_t)wave * UB);
      }
    }
    if (hasG) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float v0 = xv[2 * h] * sv[2 * h], v1 = xv[2 * h + 1] * sv[2 * h + 1];
        fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
        const int e = gh * 256 + h * 128 + lane;
        prep_g[gi][kp(e)] = to_f16(v0);
        prep_g[gi][kp(e + 64)] = to_f16(v1);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    trace_mark(a, tu, 1 << 30, 2);

    // gate/up: each wave half the unit's k tiles; the second half's sums meet the first's in LDS (fixed order)
    float g_acc0 = 0.f, g_acc1 = 0.f;
    if (hasG) {
      const uint8_t *tl = f2_tiles + (uint32_t)gi * UB + (uint32_t)gh * (kF2KT / 2) * 2 * 32u * (Gt.sh ? KS : K);
      IJ_F2_K(Gt.sh, f2_pair_dot<KK>(tl, prep_g[gi] + gh * (kF2KT / 2) * 16, kF2KT / 2, g_acc0, g_acc1));
      if (gh == 1 && (lane & 6) == 0) {
        const int col = (lane >> 3) + 8 * (lane & 1);
        red[wave][col] = g_acc0;
        red[wave][16 + col] = g_acc1;
      }
    }
    __syncthreads();
    if (hasG && gh == 0 && (lane & 6) == 0) {
      const int col = (lane >> 3) + 8 * (lane & 1);
      float *g = a.guo + (((uint64_t)Gt.slot * 2 + Gt.proj) * a.ksplit + Gt.ks) * a.inter + Gt.p * 32;
      st_cg(g + col, g_acc0 + red[wave + 1][col]);
      st_cg(g + 16 + col, g_acc1 + red[wave + 1][16 + col]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // count the units per (slot, 128-column block); the last one of a block finishes it (one wave per block)
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < NG; i++) {
        s_fin[i] = -1;
        const F2Unit Gi = f2_gu_unit(a, f, g0 + i);
        if (!Gi.valid) continue;
        const int cb = Gi.p / 4;
        const uint32_t old = atomicAdd(fin_cnt + (Gi.slot * nbi + cb) * kSyncStride, 1u);
        if (old == 8u * (uint32_t)a.ksplit - 1u) s_fin[i] = Gi.slot * nbi + cb;  // 2 proj x ksplit x 4 pairs
      }
    }
    __syncthreads();
    if (wave < NG && s_fin[wave] >= 0) {
      const int fs = s_fin[wave] / nbi, cb = s_fin[wave] % nbi;
      f2_gu_finish(a, f2_block(a, &rt, fs / a.nslot, fs % a.nslot), (fs % a.nslot) >= a.topk, fs, cb,
                   prep_g[wave]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < NG; i++)
        if (s_fin[i] >= 0) atomicAdd(gu_done + (s_fin[i] / nbi) * kSyncStride, 1u);
    }
    trace_mark(a, tu, 1 << 30, 3);
    if (d0 >= f.nD) continue;

    // down: wait for each unit's slot, stage its finished input, each wave a quarter of the k tiles, sums in LDS
    bool ok = true;
#pragma unroll
    for (int i = 0; i < ND; i++) {
      const F2Unit Di = f2_dn_unit(a, f, d0 + i);
      if (Di.valid && ok) ok = block_wait_geq(sync, gu_done + Di.slot * kSyncStride, (uint32_t)nbi, &flag);
    }
    if (!ok) continue;
    trace_mark(a, tu, 1 << 30, 4);
    const F2Unit Dt = f2_dn_unit(a, f, d0 + dj);
    const bool hasD = wave < 4 * ND && Dt.valid;
    if (hasD) {  // wave q of the unit stages words [64 q, 64 q + 64) of the slot's inter / 2 words
      const uint32_t *hp = (const uint32_t *)(a.hprep + (uint64_t)Dt.slot * a.inter);
      const int wi = dq * 64 + lane;
      if (wi * 2 < a.inter) ((uint32_t *)prep_d[dj])[wi] = ld_cg(hp + wi);
    }
    __syncthreads();
    float d_acc0 = 0.f, d_acc1 = 0.f;
    const int qkt = f.ITd / 4;  // k tiles per quarter
    if (hasD) {
      const uint8_t *tl = f2_tiles + (uint32_t)(NG + dj) * UB + (uint32_t)dq * qkt * 2 * 32u * (Dt.sh ? KS : K);
      IJ_F2_K(Dt.sh, f2_pair_dot<KK>(tl, prep_d[dj] + dq * qkt * 16, qkt, d_acc0, d_acc1));
      if (dq > 0 && (lane & 6) == 0) {
        const int col = (lane >> 3) + 8 * (lane & 1);
        red[wave][col] = d_acc0;
        red[wave][16 + col] = d_acc1;
      }
    }
    __syncthreads();
    if (hasD && dq == 0 && (lane & 6) == 0) {
      const int col = (lane >> 3) + 8 * (lane & 1);
      float *d = a.dn + (uint64_t)Dt.slot * a.hid + Dt.p * 32;
      st_cg(d + col, ((d_acc0 + red[wave + 1][col]) + red[wave + 2][col]) + red[wave + 3][col]);
      st_cg(d + 16 + col, ((d_acc1 + red[wave + 1][16 + col]) + red[wave + 2][16 + col]) + red[wave + 3][16 + col]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    trace_mark(a, tu, 1 << 30, 5);
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < ND; i++) {
        s_last[i] = -1;
        const F2Unit Di = f2_dn_unit(a, f, d0 + i);
        if (!Di.valid) continue;
        const int c = Di.p / 4;  // 128-column block of the pair's 32 columns
        const uint32_t old = atomicAdd(blk_cnt + (Di.r * f.nblk + c) * kSyncStride, 1u);
        if (old == 4u * (uint32_t)a.nslot - 1u) s_last[i] = Di.r * f.nblk + c;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < ND; i++) {
      const int rb = s_last[i];
      if (rb >= 0) f2_combine(a, &rt, rb / f.nblk, rb % f.nblk, vs);
    }
    trace_mark(a, tu, 1 << 30, 6);
  }
  // the last workgroup to leave resets the counters for the next launch
  if (threadIdx.x == 0 && atomicAdd(sync + kSyncExit, 1u) == gridDim.x - 1u) {
    for (int i = 0; i < a.R * a.nslot; i++) st_cg(gu_done + i * kSyncStride, 0u);
    for (int i = 0; i < a.R * f.nblk; i++) st_cg(blk_cnt + i * kSyncStride, 0u);
    for (int i = 0; i < a.R * a.nslot * nbi; i++) st_cg(fin_cnt + i * kSyncStride, 0u);
    st_cg(sync + kSyncRouterDone, 0u);
    st_cg(sync + kSyncRouteReady2, 0u);
    st_cg(sync + kSyncHead, 0u);
    st_cg(sync + kSyncHeadG, 0u);
    st_cg(sync + kSyncHeadD, 0u);
    __builtin_amdgcn_s_waitcnt(0);
    atomicExch(sync + kSyncExit, 0u);
  }
}
#undef IJ_F2_K

// ------------------------------------------------------------------------------------------------ trunk linear
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

// lin_gemv: grid = OT/2 pairs x S k-splits; 256 threads; xs = the split's span of xh for RT rows (zeros past R).
// part[s][r][OTp*16] = raw inner outputs.
template <int K, int RT>
__global__ __launch_bounds__(256) void lin_gemv(LinArgs a) {
  extern __shared__ _Float16 xs[];
  const int NP = (a.OT + 1) / 2, OTp = 2 * NP;
  const int p = blockIdx.x % NP, s = blockIdx.x / NP;
  const int span = a.IT / a.S, k0 = s * span, k1 = k0 + span, n = span * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const uint32_t *pb = a.tiles + (uint64_t)p * a.IT * 2 * 8 * K;
  PairBuf<K> buf;
  pair_load<K>(buf, pb, L, k0 + wave, k1);
  for (int i = threadIdx.x; i < RT * n / 8; i += blockDim.x) {
    const int r = (i * 8) / n, o = (i * 8) % n;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < a.R) v = *(const uint4 *)(a.xh + (uint64_t)r * a.in + k0 * 16 + o);
    *(uint4 *)(xs + r * n + o) = v;
  }
  __syncthreads();
  const int q = (lane >> 1) & 3;
  float acc0[RT], acc1[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) acc0[r] = acc1[r] = 0.f;
  for (int tk0 = k0 + wave; tk0 < k1; tk0 += 4 * kPrefetch) {
    if (tk0 != k0 + wave) pair_load<K>(buf, pb, L, tk0, k1);
#pragma unroll
    for (int j = 0; j < kPrefetch; j++) {
      const int tk = tk0 + 4 * j;
      if (tk < k1) {
        f16x2 a0, b0, a1, b1;
        decode4<K>(buf.w[j][0], L.sh, a0, b0);
        decode4<K>(buf.w[j][1], L.sh, a1, b1);
#pragma unroll
        for (int r = 0; r < RT; r++) {
          const f16x4 xv = *(const f16x4 *)(xs + r * n + (tk - k0) * 16 + 4 * q);
          acc0[r] = dot4(a0, b0, xv, acc0[r]);
          acc1[r] = dot4(a1, b1, xv, acc1[r]);
        }
      }
    }
  }
  __shared__ float red[4 * 32 * RT];
  const int col = (lane >> 3) + 8 * (lane & 1);
#pragma unroll
  for (int r = 0; r < RT; r++) {
    float v0 = acc0[r], v1 = acc1[r];
    v0 += __shfl_xor(v0, 2, 64);
    v0 += __shfl_xor(v0, 4, 64);
    v1 += __shfl_xor(v1, 2, 64);
    v1 += __shfl_xor(v1, 4, 64);
    if ((lane & 6) == 0) {
      red[(r * 4 + wave) * 32 + col] = v0;
      red[(r * 4 + wave) * 32 + 16 + col] = v1;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < a.R * 32; i += blockDim.x) {
    const int r = i / 32, t = i % 32;
    const float v = (red[(r * 4 + 0) * 32 + t] + red[(r * 4 + 1) * 32 + t]) +
                    (red[(r * 4 + 2) * 32 + t] + red[(r * 4 + 3) * 32 + t]);
    a.part[((uint64_t)s * a.R + r) * OTp * 16 + p * 32 + t] = v;
  }
}

// lin_finish: y = H_out(sum over splits in order) * svh (reference kernels/trunk6/trunk6.metal:199-214),
// grid R x ceil(out/128).
__global__ __launch_bounds__(64) void lin_finish(LinArgs a) {
  const int nch = (a.out + 127) / 128;
  const int r = blockIdx.x / nch, c = blockIdx.x % nch, lane = threadIdx.x;
  const int OTp = a.OT + (a.OT & 1);
  const int i0 = c * 128 + lane, i1 = i0 + 64;
  const bool m0 = i0 < a.out, m1 = i1 < a.out;
  float v0 = 0.f, v1 = 0.f;
  for (int s = 0; s < a.S; s++) {
    const float *pp = a.part + ((uint64_t)s * a.R + r) * OTp * 16;
    if (m0) v0 += pp[i0];
    if (m1) v1 += pp[i1];
  }
  fwht2(v0, v1, lane, a.had_out, a.sc_out);
  if (m0) a.y[(uint64_t)r * a.out + i0] = v0 * h2f(a.svh[i0]);
  if (m1) a.y[(uint64_t)r * a.out + i1] = v1 * h2f(a.svh[i1]);
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
// Plain device copy of n16 16-byte words; the byte-count probe that scales HBM traffic counters (FETCH_SIZE,
// WRITE_SIZE) to bytes.
__global__ __launch_bounds__(256) void copy_u128(const uint4 *src, uint4 *dst, uint64_t n16) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
__global__ void fill_scale_f16(uint16_t *p, uint64_t n, uint64_t seed) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) {
    const float m = fabsf(1.0f + 0.1f * gauss(seed, i));
    const bool neg = splitmix64(seed + 0x51ED27u + i) & 1u;
    p[i] = f2h(neg ? -m : m);
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
static const void *fused_fn(int K, int KS) {
#define IJ_FUSED_CASE(k, ks) \
  if (K == k && KS == ks) return (const void *)&moe_fused<k, ks>;
  IJ_FUSED_CASE(4, 4) IJ_FUSED_CASE(5, 5) IJ_FUSED_CASE(6, 6) IJ_FUSED_CASE(4, 6) IJ_FUSED_CASE(5, 6)
  IJ_FUSED_CASE(4, 8) IJ_FUSED_CASE(5, 8) IJ_FUSED_CASE(6, 8)
#undef IJ_FUSED_CASE
  return nullptr;
}
static size_t fused_lds(int K, int KS) {
  const int KM = std::max(K, KS);
  return (size_t)(KM <= 6 ? F2Take<6>::NG + F2Take<6>::ND : F2Take<8>::NG + F2Take<8>::ND) * kF2UnitBytesK * KM;
}
// shapes the fused kernel serves: units of 2 output tile pairs x 32 k tiles, at most kMaxRows rows
bool moe_fused_supported(int K, int KS, int R, int hid, int inter, int ksplit) {
  return fused_fn(K, KS) != nullptr && R <= kMaxRows && hid % 512 == 0 && hid / 16 == ksplit * kF2KT &&
         inter % 128 == 0 && inter / 16 <= kF2KT && inter <= 512;
}
int moe_fused_grid(int K, int KS) {
  const void *f = fused_fn(K, KS);
  IJ_CHECK(f, "fused MoE kernel not instantiated for K%d / shared K%d", K, KS);
  int dev = 0, cus = 0;
  IJ_HIP(hipGetDevice(&dev));
  IJ_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  return cus;
}
void launch_moe_fused(const MoeArgs &a, int grid, hipStream_t s) {
  const int KS = a.nslot > a.topk ? a.slay.K : a.lay.K;
  const void *f = fused_fn(a.lay.K, KS);
  IJ_CHECK(f, "fused MoE kernel not instantiated for K%d / shared K%d", a.lay.K, KS);
  const size_t lds = fused_lds(a.lay.K, KS);
  static bool attr_set[9][9] = {};
  if (!attr_set[a.lay.K][KS]) {
    IJ_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set[a.lay.K][KS] = true;
  }
  void *args[] = {const_cast<MoeArgs *>(&a)};
  IJ_HIP(hipLaunchKernel(f, dim3(grid > 0 ? grid : moe_fused_grid(a.lay.K, KS)), dim3(64 * kF2Waves), args, lds, s));
}

template <int K>
static const void *lin_gemv_fn(int RT) {
  switch (RT) {
    case 1: return (const void *)&lin_gemv<K, 1>;
    case 2: return (const void *)&lin_gemv<K, 2>;
    case 4: return (const void *)&lin_gemv<K, 4>;
    default: return (const void *)&lin_gemv<K, 8>;
  }
}
static const void *lin_gemv_any(int K, int RT) {
  const void *f = nullptr;
  IJ_DISPATCH_K(K, f = lin_gemv_fn<KK>(RT));
  return f;
}
static int rows_tier(int R) { return R <= 1 ? 1 : R <= 2 ? 2 : R <= 4 ? 4 : 8; }

void launch_lin(const LinArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(lin_prep, dim3(a.R * ((a.in + 127) / 128)), dim3(64), 0, s, a);
  const int RT = rows_tier(a.R);
  const size_t lds = (size_t)RT * (a.IT / a.S) * 16 * sizeof(uint16_t);
  void *args[] = {const_cast<LinArgs *>(&a)};
  const int NP = (a.OT + 1) / 2;
  IJ_HIP(hipLaunchKernel(lin_gemv_any(a.K, RT), dim3(NP * a.S), dim3(256), args, lds, s));
  hipLaunchKernelGGL(lin_finish, dim3(a.R * ((a.out + 127) / 128)), dim3(64), 0, s, a);
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
    for (int RT : {1, 2, 4, 8}) v.push_back({"lin_gemv", lin_gemv_any(K, RT), {(uint32_t)sizeof(LinArgs)}, K, RT});
  }
  v.push_back({"lin_prep", (const void *)&lin_prep, {(uint32_t)sizeof(LinArgs)}, -1, -1});
  v.push_back({"lin_finish", (const void *)&lin_finish, {(uint32_t)sizeof(LinArgs)}, -1, -1});
  v.push_back({"moe_router", (const void *)&moe_router, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  v.push_back({"moe_gateup", (const void *)&moe_gateup, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  v.push_back({"moe_down", (const void *)&moe_down, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  v.push_back({"moe_combine", (const void *)&moe_combine, {(uint32_t)sizeof(MoeArgs)}, -1, -1});
  for (int K = 4; K <= 6; K++)
    for (int KS : {4, 5, 6, 8})
      if (fused_fn(K, KS)) v.push_back({"moe_fused_ks" + std::to_string(KS), fused_fn(K, KS), {(uint32_t)sizeof(MoeArgs)}, K, -1});
  v.push_back({"fill_u32", (const void *)&fill_u32, {P, 8, 8}, -1, -1});
  v.push_back({"copy_u128", (const void *)&copy_u128, {P, P, 8}, -1, -1});
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
