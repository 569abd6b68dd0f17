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
// (4m + 1) K - 15: funnel shifts (v_alignbit) of two words, except at K 7 (three words). The input
// is staged in LDS as fp16 in the reference's k-permuted order (kp), so a lane's four rows are one 8-byte read, and the
// four weights meet it in two v_dot2_f32_f16. Lanes sharing a column differ in lane bits 1-2: two xor-shuffles reduce.
//
// Hadamard transforms hold 128 elements as (lane, lane + 64) and run the butterflies over index bits 0..6 in order
// (lane shuffles for bits 0-5, the register pair for bit 6) with lo + hi / lo - hi in f32, then one multiply by
// f32(1/sqrt n): the same operations, in the same order, as the reference's fwht128 / t6_fwht
// (kernels/ne_common.h:93-103, kernels/trunk6/trunk6.metal:42-51), so the fp16-rounded prepared input is
// bit-identical to the reference arithmetic. The library is compiled with -ffp-contract=off for that reason.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

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
// The value of lane (lane ^ bit) for bit = 1 .. 32, all in VALU: DPP inside rows of 16 (xor 4 = half-mirror then
// quad reverse, xor 8 = mirror then half-mirror), the gfx950 row / half swaps (v_permlane16/32_swap) across rows.
template <int BIT>
__device__ __forceinline__ float xor_lane(float v, int lane) {
  const int x = __float_as_int(v);
  if constexpr (BIT == 1) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  } else if constexpr (BIT == 2) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  } else if constexpr (BIT == 4) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);            // row_half_mirror: i ^ 7
    return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x1B, 0xF, 0xF, false));    // quad_perm 3,2,1,0: ^ 3
  } else if constexpr (BIT == 8) {
    const int t = __builtin_amdgcn_mov_dpp(x, 0x140, 0xF, 0xF, false);            // row_mirror: i ^ 15
    return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x141, 0xF, 0xF, false));   // row_half_mirror: ^ 7
  } else if constexpr (BIT == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
  }
}
template <int BIT>
__device__ __forceinline__ void fwht_stage(float &v0, float &v1, int lane) {
  const float p0 = xor_lane<BIT>(v0, lane), p1 = xor_lane<BIT>(v1, lane);
  // partner + (-1 or +1) v: one fused op, rounded once, so exactly p - v on the upper lanes and v + p on the others
  const float sg = (lane & BIT) ? -1.f : 1.f;
  v0 = __builtin_fmaf(sg, v0, p0);
  v1 = __builtin_fmaf(sg, v1, p1);
}
// normalised Sylvester H_N (N = 16..128) on a 128-chunk held as (lane, lane + 64); blocks of N are contiguous.
__device__ __forceinline__ void fwht2(float &v0, float &v1, int lane, int N, float sc) {
  fwht_stage<1>(v0, v1, lane);
  fwht_stage<2>(v0, v1, lane);
  fwht_stage<4>(v0, v1, lane);
  fwht_stage<8>(v0, v1, lane);
  if (N > 16) fwht_stage<16>(v0, v1, lane);
  if (N > 32) fwht_stage<32>(v0, v1, lane);
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
__host__ __device__ constexpr uint32_t group_sm1(int K, uint32_t m) {
  return ((4u * m + 1u) * K + 256u * K - 16u) % (256u * K);  // S - 1
}
template <int K>
__device__ __forceinline__ TileLane<K> tile_lane(uint32_t m) {
  constexpr uint32_t NW = 8u * K;
  const uint32_t Sm1 = group_sm1(K, m);
  TileLane<K> t;
  t.i0 = Sm1 >> 5;
  t.i1 = (t.i0 + 1u) % NW;
  t.i2 = (t.i0 + 2u) % NW;
  t.sh = 31u - (Sm1 & 31u);
  return t;
}
// A group's codewords span 15 + 3K bits from bit a' = 32 - sh of words (i0, i1, ...). For K 6 and 8 every group
// start puts a' <= 49 - 3K (sh >= 3K - 17), so the window ends inside word i1 and no third word is read; only K 7
// needs one.
template <int K>
constexpr bool two_word_windows() {
  for (uint32_t m = 0; m < 64; m++)
    if ((int)(31u - (group_sm1(K, m) & 31u)) < 3 * K - 17) return false;
  return true;
}
template <int K>
constexpr bool kThreeWords = (15 + 3 * K > 32) && !two_word_windows<K>();
// sh when it is the same for every group (K 8: 7), else -1
template <int K>
constexpr int const_sh() {
  const uint32_t s = 31u - (group_sm1(K, 0) & 31u);
  for (uint32_t m = 1; m < 64; m++)
    if (31u - (group_sm1(K, m) & 31u) != s) return -1;
  return (int)s;
}
template <int K>
constexpr int kConstSh = const_sh<K>();

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

// ------------------------------------------------------------------------------------------------ matrix cores
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// The matrix-core B operand of lane l is column n = l % 32 of the pair (tile n / 16, column c = n % 16), k values
// 8 (l / 32) .. + 8: the trellis groups (c, q) with q = 2 (l / 32) and q + 1, four consecutive k each. Group m of a
// tile (weights 4m .. 4m + 3 of the bitstream) holds column c = (m >> 3) + 8 (m & 1), k quarter q = (m >> 1) & 3.
__device__ __forceinline__ uint32_t group_of(uint32_t c, uint32_t q) { return ((c & 7u) << 3) | (q << 1) | (c >> 3); }
template <int K>
struct BLane {
  TileLane<K> g0, g1;  // the lane's two groups
  uint32_t tile;       // 0 or 1: which tile of the pair
};
template <int K>
__device__ __forceinline__ BLane<K> b_lane(uint32_t lane) {
  const uint32_t n = lane & 31u, q = 2u * (lane >> 5);
  BLane<K> b;
  b.g0 = tile_lane<K>(group_of(n & 15u, q));
  b.g1 = tile_lane<K>(group_of(n & 15u, q + 1u));
  b.tile = n >> 4;
  return b;
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

// The group's four codewords (15 bits each, at window bits K i .. K i + 14) from its words and shift.
template <int K>
__device__ __forceinline__ void codewords4(const TileWords &w, uint32_t sh, uint32_t (&c)[4]) {
  const uint32_t hi = __builtin_amdgcn_alignbit(w.w0, w.w1, sh);  // window bits 0 .. 31
  if constexpr (!kThreeWords<K>) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = 17 - i * K;  // codeword i's lowest bit in hi; below 0: it ends -r bits past hi, still in w1
      if (r >= 0)
        c[i] = (hi >> r) & 0x7FFFu;
      else
        c[i] = (kConstSh<K> == -r ? w.w1 : __builtin_amdgcn_alignbit(w.w0, w.w1, sh - (uint32_t)(-r))) & 0x7FFFu;
    }
  } else {
    const uint32_t lo = __builtin_amdgcn_alignbit(w.w1, w.w2, sh);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int s = 49 - i * K;
      c[i] = (s >= 32 ? (hi >> (s - 32)) : __builtin_amdgcn_alignbit(hi, lo, (uint32_t)s)) & 0x7FFFu;
    }
  }
}
// The lane's four weights: a = rows (2q, 2q+1), b = rows (2q+8, 2q+9) of its column.
template <int K>
__device__ __forceinline__ void decode4(const TileWords &w, uint32_t sh, f16x2 &a, f16x2 &b) {
  uint32_t c[4];
  codewords4<K>(w, sh, c);
  a = mcg_pair(c[0], c[1]);
  b = mcg_pair(c[2], c[3]);
}

// s_waitcnt vmcnt(n) for a run-time n (6-bit count: low 4 bits at [3:0], high 2 at [15:14]; n above 63 waits as for
// 63, which only waits longer); completion is counted in issue order, stores included
__device__ __forceinline__ void wait_vm(int n) {
  switch (n < 63 ? n : 63) {
#define IJ_VM(k) \
  case k: __builtin_amdgcn_s_waitcnt(0x0F70 | ((k) & 15) | (((k) >> 4) << 14)); break;
#define IJ_VM4(k) IJ_VM(k) IJ_VM(k + 1) IJ_VM(k + 2) IJ_VM(k + 3)
    IJ_VM4(0) IJ_VM4(4) IJ_VM4(8) IJ_VM4(12) IJ_VM4(16) IJ_VM4(20) IJ_VM4(24) IJ_VM4(28)
    IJ_VM4(32) IJ_VM4(36) IJ_VM4(40) IJ_VM4(44) IJ_VM4(48) IJ_VM4(52) IJ_VM4(56) IJ_VM4(60)
#undef IJ_VM4
#undef IJ_VM
  }
}
// Tagged values between workgroups of one launch: the f32 value in the low word and the launch's tag in the high
// word, stored and polled with device-coherent accesses, so that a consumer sees the data itself arrive.
__device__ __forceinline__ void st_tag(uint64_t *p, float v, uint32_t tag) {
  st_cg(p, (uint64_t)__float_as_uint(v) | ((uint64_t)tag << 32));
}
__device__ __forceinline__ float tag_val(uint64_t t) { return __uint_as_float((uint32_t)t); }
__device__ __forceinline__ bool tag_ok(uint64_t t, uint32_t tag) { return (uint32_t)(t >> 32) == tag; }
// the same with the count capped at 15 (waits at least as long): a 16-case switch, for k loops where the 64-case one
// costs registers
__device__ __forceinline__ void wait_vm15(int n) {
  switch (n < 15 ? n : 15) {
#define IJ_VM(k) \
  case k: __builtin_amdgcn_s_waitcnt(0x0F70 | (k)); break;
    IJ_VM(0) IJ_VM(1) IJ_VM(2) IJ_VM(3) IJ_VM(4) IJ_VM(5) IJ_VM(6) IJ_VM(7)
    IJ_VM(8) IJ_VM(9) IJ_VM(10) IJ_VM(11) IJ_VM(12) IJ_VM(13) IJ_VM(14) IJ_VM(15)
#undef IJ_VM
  }
}
// the B operand of k tile kt of a pair staged in LDS (tile pairs of 64 K bytes in k order; the trellis words decoded
// straight into v_mfma_f32_32x32x16_f16's B)
template <int K>
__device__ __forceinline__ f16x8 decode_pair(const uint8_t *tl, int kt) {
  constexpr int TW = 8 * K;
  const int lane = threadIdx.x & 63;
  const BLane<K> B = b_lane<K>((uint32_t)lane);
  const uint32_t *T0 = (const uint32_t *)tl + B.tile * TW + kt * 2 * TW;
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
  return f16x8{l0.x, l0.y, h0.x, h0.y, l1.x, l1.y, h1.x, h1.y};
}
// One MFMA chain over the first nkt (<= NT) tile pairs staged at tl, onto acc; xa: the lane's A operand of tile 0
// (tile kt at xa + 16 kt). A full chunk takes a branch-free path, so the tiles' LDS reads can be issued ahead of the
// decode; the products and their order are the same on both paths.
template <int K, int NT>
__device__ __forceinline__ f32x16 mfma_chunk(const uint8_t *tl, const _Float16 *xa, int nkt, f32x16 acc) {
  if (nkt == NT) {
#pragma unroll
    for (int kt = 0; kt < NT; kt++)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const f16x8 *)(xa + kt * 16), decode_pair<K>(tl, kt), acc, 0, 0,
                                                   0);
    return acc;
  }
#pragma unroll
  for (int kt = 0; kt < NT; kt++)
    if (kt < nkt)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const f16x8 *)(xa + kt * 16), decode_pair<K>(tl, kt), acc, 0, 0,
                                                   0);
  return acc;
}
__device__ __forceinline__ float dot4(f16x2 a, f16x2 b, f16x4 x, float acc) {
  acc = __builtin_amdgcn_fdot2(a, f16x2{x.x, x.y}, acc, false);
  return __builtin_amdgcn_fdot2(b, f16x2{x.z, x.w}, acc, false);
}

// ------------------------------------------------------------------------------------------------ reductions
// column sums of a lane pair-tile product: lanes sharing a column differ in lane bits 1-2
__device__ __forceinline__ void lane_col_reduce(float &acc0, float &acc1) {
  acc0 += __shfl_xor(acc0, 2, 64);
  acc0 += __shfl_xor(acc0, 4, 64);
  acc1 += __shfl_xor(acc1, 2, 64);
  acc1 += __shfl_xor(acc1, 4, 64);
}
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
// bf16-valued logit back from its order key (the inverse of topk_key on the top 16 bits)
__device__ __forceinline__ float key_value(uint32_t key) {
  const uint32_t h = key >> 16;
  return __uint_as_float((h & 0x8000u) ? (h & 0x7FFFu) << 16 : (~h & 0xFFFFu) << 16);
}

}  // namespace ijah
