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

// MCG window-15 codebook (reference kernels/ne_common.h:139-144); half + half rounds once (RNE) like the reference.
__device__ __forceinline__ _Float16 mcg(uint32_t cw) {
  const uint32_t r = ((cw * 0xCBAC1FEDu) & 0x8FFF8FFFu) ^ 0x3B603B60u;
  const f16x2 h = __builtin_bit_cast(f16x2, r);
  return h.x + h.y;
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
  a = f16x2{mcg(c[0]), mcg(c[1])};
  b = f16x2{mcg(c[2]), mcg(c[3])};
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
// One workgroup (4 waves) multiplies the LDS-staged prepared input span (fp16, kp order, `xs` = rows [16*tk0, ...))
// with output tiles (2p, 2p+1) over k tiles [k0, k1) of a re-laid matrix; waves stride k by 4. Returns per lane the
// partial sums of its column for the two tiles, reduced over the four lanes sharing the column.
template <int K>
__device__ __forceinline__ void pair_gemv(const uint32_t *__restrict__ tiles, int IT, int p, int k0, int k1,
                                          const _Float16 *xs, float &acc0, float &acc1) {
  constexpr int TW = 8 * K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const int q = (lane >> 1) & 3;
  acc0 = 0.f;
  acc1 = 0.f;
  const uint32_t *base = tiles + (uint64_t)p * IT * 2 * TW;
#pragma unroll 4
  for (int tk = k0 + wave; tk < k1; tk += 4) {
    const uint32_t *T0 = base + (uint64_t)tk * 2 * TW;
    const TileWords wa = load_tile<K>(T0, L), wb = load_tile<K>(T0 + TW, L);
    const f16x4 xv = *(const f16x4 *)(xs + (tk - k0) * 16 + 4 * q);
    f16x2 a0, b0, a1, b1;
    decode4<K>(wa, L.sh, a0, b0);
    decode4<K>(wb, L.sh, a1, b1);
    acc0 = dot4(a0, b0, xv, acc0);
    acc1 = dot4(a1, b1, xv, acc1);
  }
  acc0 += __shfl_xor(acc0, 2, 64);
  acc0 += __shfl_xor(acc0, 4, 64);
  acc1 += __shfl_xor(acc1, 2, 64);
  acc1 += __shfl_xor(acc1, 4, 64);
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

__global__ __launch_bounds__(256) void moe_router(MoeArgs a) {
  __shared__ float lv[kMaxExperts];
  __shared__ uint32_t sid[kMaxTopk];
  __shared__ float sval[kMaxTopk];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nrows = a.ne + a.has_sgate;
  const int row = blockIdx.x * 4 + wave;
  const int ld = a.ne + 1;
  if (row < nrows) {
    const uint16_t *w = a.router + (uint64_t)row * a.hid;
    for (int r = 0; r < a.R; r++) {
      const float *x = a.x + (uint64_t)r * a.hid;
      float acc = 0.f;
      for (int c = lane; c * 8 < a.hid; c += 64) {
        const uint4 wv = *(const uint4 *)(w + c * 8);
        const float4 x0 = *(const float4 *)(x + c * 8), x1 = *(const float4 *)(x + c * 8 + 4);
        acc = fmaf(x0.x, bf16_f32(wv.x & 0xFFFFu), acc);
        acc = fmaf(x0.y, bf16_f32(wv.x >> 16), acc);
        acc = fmaf(x0.z, bf16_f32(wv.y & 0xFFFFu), acc);
        acc = fmaf(x0.w, bf16_f32(wv.y >> 16), acc);
        acc = fmaf(x1.x, bf16_f32(wv.z & 0xFFFFu), acc);
        acc = fmaf(x1.y, bf16_f32(wv.z >> 16), acc);
        acc = fmaf(x1.z, bf16_f32(wv.w & 0xFFFFu), acc);
        acc = fmaf(x1.w, bf16_f32(wv.w >> 16), acc);
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
      if (lane == 0) a.logits[(uint64_t)r * ld + row] = bf16_round(acc);
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = (atomicAdd(a.ctr, 1u) == gridDim.x - 1u) ? 1 : 0;
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int r = 0; r < a.R; r++) {
    for (int i = threadIdx.x; i < a.ne; i += blockDim.x) {
      const float v = __hip_atomic_load(a.logits + (uint64_t)r * ld + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      lv[i] = (v != v) ? -INFINITY : v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.ne; i += blockDim.x) {
      const float v = lv[i];
      int rank = 0;
      for (int j = 0; j < a.ne; j++) {
        const float u = lv[j];
        rank += (u > v) || (u == v && j < i);
      }
      if (rank < a.topk) {
        sid[rank] = (uint32_t)i;
        sval[rank] = v;
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float pr[kMaxTopk];
      const float top = sval[0];
      float s = 0.f;
      for (int k = 0; k < a.topk; k++) {
        pr[k] = expf(sval[k] - top);
        s += pr[k];
      }
      uint32_t *rt = a.route + (uint64_t)r * 2 * a.topk;
      for (int k = 0; k < a.topk; k++) {
        rt[k] = sid[k];
        rt[a.topk + k] = __float_as_uint(pr[k] / s);
      }
      float g = 1.f;
      if (a.has_sgate) {
        const float l = __hip_atomic_load(a.logits + (uint64_t)r * ld + a.ne, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        g = 1.f / (1.f + expf(-l));
      }
      a.sgv[r] = g;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) atomicExch(a.ctr, 0u);
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
    uint32_t e = a.route[(uint64_t)r * 2 * a.topk + k];
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

// ------------------------------------------------------------------------------------------------ MoE: D2 gate/up
// grid = R nslot x 2 (gate, up) x inter/32 (output tile pairs) x ksplit; 256 threads. Prep x * suh -> H -> fp16 into
// LDS for the workgroup's k span (reference kernels/fn_moe.metal:304-312), then the pair GEMV; guo holds the raw
// inner outputs per k split (summed in order by D3).
template <int K>
__device__ void gateup_body(const MoeArgs &a, const SlotRef &sr, int slot, int proj, int p, int ks, _Float16 *prep,
                            float *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = slot / a.nslot;
  const int IT = a.hid >> 4, ktn = IT / a.ksplit, k0 = ks * ktn, n = ktn * 16;
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
  float acc0, acc1;
  pair_gemv<K>((const uint32_t *)(sr.blk + off_tr(a, sr.sh, proj)), IT, p, k0, k0 + ktn, prep, acc0, acc1);
  const float s = pair_reduce(acc0, acc1, red);
  const int o = p * 32 + (int)threadIdx.x;
  if (threadIdx.x < 32 && o < a.inter) a.guo[(((uint64_t)slot * 2 + proj) * a.ksplit + ks) * a.inter + o] = s;
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
  IJ_DISPATCH_K(sr.K, gateup_body<KK>(a, sr, slot, proj, p, ks, prep, red));
}

// ------------------------------------------------------------------------------------------------ MoE: D3 down
// grid = R nslot x hid/32 (output tile pairs); 256 threads. Prologue (reference kernels/fn_moe.metal:370-384):
// g = H(guo_g) * svh_g, u = H(guo_u) * svh_u, h = H(silu(g) u * suh_d) -> fp16 LDS; then the down pair GEMV over all
// inter k tiles; dn holds the raw down outputs (H_out, svh and the route weight are applied by the combine).
template <int K>
__device__ void down_body(const MoeArgs &a, const SlotRef &sr, int slot, int p, _Float16 *prep, float *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int inter = a.inter;
  const float *gp = a.guo + (uint64_t)slot * 2 * a.ksplit * inter;
  const float *up = gp + (uint64_t)a.ksplit * inter;
  const uint16_t *gsv = (const uint16_t *)(sr.blk + off_sv(a, sr.sh, 0));
  const uint16_t *usv = (const uint16_t *)(sr.blk + off_sv(a, sr.sh, 1));
  const uint16_t *dsu = (const uint16_t *)(sr.blk + off_su(a, sr.sh, 2));
  for (int c = wave; c * 128 < inter; c += 4) {
    const int i0 = c * 128 + lane, i1 = i0 + 64;
    const bool m0 = i0 < inter, m1 = i1 < inter;
    float g0 = m0 ? gp[i0] : 0.f, g1 = m1 ? gp[i1] : 0.f, u0 = m0 ? up[i0] : 0.f, u1 = m1 ? up[i1] : 0.f;
    for (int s = 1; s < a.ksplit; s++) {
      if (m0) {
        g0 += gp[s * inter + i0];
        u0 += up[s * inter + i0];
      }
      if (m1) {
        g1 += gp[s * inter + i1];
        u1 += up[s * inter + i1];
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
  pair_gemv<K>((const uint32_t *)(sr.blk + off_tr(a, sr.sh, 2)), inter >> 4, p, 0, inter >> 4, prep, acc0, acc1);
  const float s = pair_reduce(acc0, acc1, red);
  const int o = p * 32 + (int)threadIdx.x;
  if (threadIdx.x < 32 && o < a.hid) a.dn[(uint64_t)slot * a.hid + o] = s;
}

__global__ __launch_bounds__(256) void moe_down(MoeArgs a) {
  __shared__ _Float16 prep[kMaxPrep];
  __shared__ float red[128];
  const int NP = (a.hid / 16 + 1) / 2;
  const int p = blockIdx.x % NP, slot = blockIdx.x / NP;
  const SlotRef sr = slot_ref(a, slot / a.nslot, slot % a.nslot);
  IJ_DISPATCH_K(sr.K, down_body<KK>(a, sr, slot, p, prep, red));
}

// ------------------------------------------------------------------------------------------------ MoE: combine
// y[r] = sum over slots in slot order of H(dn) * svh_d * w_k, the shared slot last with its gate
// (reference kernels/fn_moe.metal:412-447). grid = R x ceil(hid/128), one wave.
__global__ __launch_bounds__(64) void moe_combine(MoeArgs a) {
  const int nch = (a.hid + 127) / 128;
  const int r = blockIdx.x / nch, c = blockIdx.x % nch, lane = threadIdx.x;
  const int i0 = c * 128 + lane, i1 = i0 + 64;
  const bool m0 = i0 < a.hid, m1 = i1 < a.hid;
  float y0 = 0.f, y1 = 0.f;
  for (int k = 0; k < a.nslot; k++) {
    const int slot = r * a.nslot + k;
    const SlotRef sr = slot_ref(a, r, k);
    const float w = k < a.topk ? __uint_as_float(a.route[(uint64_t)r * 2 * a.topk + a.topk + k]) : a.sgv[r];
    const float *d = a.dn + (uint64_t)slot * a.hid;
    float v0 = m0 ? d[i0] : 0.f, v1 = m1 ? d[i1] : 0.f;
    fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
    const uint16_t *sv = (const uint16_t *)(sr.blk + off_sv(a, sr.sh, 2));
    if (m0) y0 += v0 * h2f(sv[i0]) * w;
    if (m1) y1 += v1 * h2f(sv[i1]) * w;
  }
  if (m0) a.y[(uint64_t)r * a.hid + i0] = y0;
  if (m1) a.y[(uint64_t)r * a.hid + i1] = y1;
}

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
  constexpr int TW = 8 * K;
  const int NP = (a.OT + 1) / 2, OTp = 2 * NP;
  const int p = blockIdx.x % NP, s = blockIdx.x / NP;
  const int span = a.IT / a.S, k0 = s * span, n = span * 16;
  for (int i = threadIdx.x; i < RT * n / 8; i += blockDim.x) {
    const int r = (i * 8) / n, o = (i * 8) % n;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (r < a.R) v = *(const uint4 *)(a.xh + (uint64_t)r * a.in + k0 * 16 + o);
    *(uint4 *)(xs + r * n + o) = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const TileLane<K> L = tile_lane<K>((uint32_t)lane);
  const int q = (lane >> 1) & 3;
  float acc0[RT], acc1[RT];
#pragma unroll
  for (int r = 0; r < RT; r++) acc0[r] = acc1[r] = 0.f;
  const uint32_t *base = a.tiles + (uint64_t)p * a.IT * 2 * TW;
#pragma unroll 2
  for (int tk = k0 + wave; tk < k0 + span; tk += 4) {
    const uint32_t *T0 = base + (uint64_t)tk * 2 * TW;
    const TileWords wa = load_tile<K>(T0, L), wb = load_tile<K>(T0 + TW, L);
    f16x2 a0, b0, a1, b1;
    decode4<K>(wa, L.sh, a0, b0);
    decode4<K>(wb, L.sh, a1, b1);
#pragma unroll
    for (int r = 0; r < RT; r++) {
      const f16x4 xv = *(const f16x4 *)(xs + r * n + (tk - k0) * 16 + 4 * q);
      acc0[r] = dot4(a0, b0, xv, acc0[r]);
      acc1[r] = dot4(a1, b1, xv, acc1[r]);
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
  hipLaunchKernelGGL(moe_combine, dim3(a.R * ((a.hid + 127) / 128)), dim3(64), 0, s, a);
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
