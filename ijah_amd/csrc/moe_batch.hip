// The MoE layer for a batch of rows (speculative verify, prefill): router GEMM, per-row top-k, slots sorted by
// expert, and grouped expert GEMMs on the matrix cores that decode each expert's EXL3 tiles once per 128-row chunk
// and feed them to v_mfma_f32_32x32x16_f16 (reference kernels/prefill/pf_moe.metal:26-338 and
// kernels/fn_moe.metal:677-884, driven by prefill.mm:235-276).
//
// Launches, in order:
//   bat_router   logits[R][ne (+ shared gate)] = bf16(x . router) in f32 (reference kernels/fn_moe.metal:50-67)
//   bat_route    per row: top-k, ties to the lower index, weights exp(l - l_max) / sum (kernels/fn_moe.metal:76-131)
//   bat_hist     slots per expert: LDS histograms of slices of the route, merged with global atomics
//   bat_scan     one workgroup: per-expert offsets of the
//                expert-sorted slot list (the shared expert's rows last) and the list of 128-row chunks (expert,
//                first row, rows) the GEMMs run over (kernels/prefill/pf_moe.metal:26-83)
//   bat_place_prep  one wave per slot: its place in its expert's rows (row order inside an expert does not change
//                any result: every row is computed independently) and that row of the A operand,
//                xh[row][proj] = fp16(H(x[token] * suh_e,proj)) in kp order for the gate and the up projection (each
//                linear has its own suh) (kernels/prefill/pf_moe.metal:85-110)
//   bat_gateup   per (chunk, 128-column block ib of inter): gate and up GEMMs on the matrix cores, then the down
//                prologue on the block: hh[row][ib] = fp16(H(silu(H(g) svh_g) H(u) svh_u suh_d)) (:111-140)
//   bat_down     per (chunk, 256 columns of hid): the down GEMM, then H, svh_d and the slot's route weight, stored
//                per (token, slot) (:141-161)
//   bat_combine  y[token] = sum over the token's slots in slot order
//
// Matrix-core operands (this build's layout): a 16-row k tile of A is held in the reference's kp order, so lane
// (m, h) of v_mfma_f32_32x32x16_f16 reads row m, k positions [8h, 8h + 8) as one 16-byte LDS read. Matrix-core lane
// (n, h) decodes its B operand itself: the trellis groups (column n % 16, quads 2h and 2h + 1) of tile n / 16 of the
// pair, i.e. kp positions 8h .. 8h + 7: the same k permutation on both operands.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "exl3_device.h"
#include "ring_schedule.h"
#include "kernels.h"
#include "moe_device.h"

namespace ijah {

namespace {


constexpr int kChunkRows = 128;   // rows of one GEMM chunk (4 matrix-core row blocks of 32)
constexpr int kRowBlocks = kChunkRows / 32;

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void dma16(const void *src, void *lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_dst, 16, 0, 0);
}
// The same through a buffer resource: wave-uniform base in the descriptor, per-lane byte offset voff, uniform byte
// offset soff (a scalar register): the streams of the k loop then cost no vector address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(const void *base) {
  const uint64_t b = (uint64_t)base;  // wave-uniform by construction; readfirstlane tells the compiler so
  // (readfirstlane returns int: widen through uint32_t, or a low word with bit 31 set would sign-extend)
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                     (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32;
  return __builtin_amdgcn_make_buffer_rsrc((void *)u, (short)0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, void *lds_dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_dst, 16, voff,
                                          __builtin_amdgcn_readfirstlane(soff), 0, 0);
}

// the expert block and layout of expert e (e == ne: the shared expert)
__device__ __forceinline__ const uint8_t *expert_block(const MoeArgs &a, int e) {
  return e >= a.ne ? a.shared : a.experts + (uint64_t)e * a.lay.bytes;
}
__device__ __forceinline__ uint64_t tr_of(const MoeArgs &a, int e, int proj) {
  const ExpertLayout &L = e >= a.ne ? a.slay : a.lay;
  return proj == 0 ? L.tr[0] : proj == 1 ? L.tr[1] : L.tr[2];
}
__device__ __forceinline__ uint64_t su_of(const MoeArgs &a, int e, int proj) {
  const ExpertLayout &L = e >= a.ne ? a.slay : a.lay;
  return proj == 0 ? L.su[0] : proj == 1 ? L.su[1] : L.su[2];
}
__device__ __forceinline__ uint64_t sv_of(const MoeArgs &a, int e, int proj) {
  const ExpertLayout &L = e >= a.ne ? a.slay : a.lay;
  return proj == 0 ? L.sv[0] : proj == 1 ? L.sv[1] : L.sv[2];
}

// Work item of this workgroup for a 1-D grid over nitems items (grid a multiple of 8): consecutive workgroups go to
// the 8 XCDs in turn, so each XCD takes a contiguous eighth of the items; items that share an operand (the column
// blocks of one chunk) then run together on one XCD and share its L2. False for workgroups past the work.
__device__ __forceinline__ bool xcd_item(int nitems, int &item) {
  const int b = blockIdx.x, xcd = b & 7, idx = b >> 3, q = nitems >> 3, r = nitems & 7;
  if (idx >= q + (xcd < r ? 1 : 0)) return false;
  item = xcd * q + min(xcd, r) + idx;
  return true;
}
}  // namespace

// ---------------------------------------------------------------------------------------------------- router
// logits[r][c] = bf16(x[r] . router[c]) for c < ne + has_sgate on the matrix cores. A workgroup covers 32 rows and
// CT 32-column tiles; its 8 waves are CT column tiles x KSP k splits, summed in LDS in split order. Few rows take
// CT = 1, KSP = 8 (the k split keeps the chip busy); many rows take CT = 4, KSP = 2, so that each row of x is read
// by a quarter as many workgroups. k steps of 16: x is split into bf16 hi + lo (x - hi rounded again), two MFMAs per
// step, so the product carries about 16 mantissa bits of x: within f32 rounding of the reference's f32 dot for
// these logits.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kRouterWaves = 8;
template <int CT>
__global__ __launch_bounds__(512) void bat_router(MoeArgs a) {
  constexpr int KSP = kRouterWaves / CT;
  __shared__ float red[kRouterWaves][16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ncol = a.ne + a.has_sgate;
  const int rt = blockIdx.x, ct = blockIdx.y * CT + wave % CT, ks = wave / CT;  // 32-row tile, 32-column tile
  const bool live = ct * 32 < ncol;
  const int m = lane & 31, h = lane >> 5;
  const int row = min(rt * 32 + m, a.R - 1), col = min(ct * 32 + m, ncol - 1);
  const int kn = a.hid / KSP, kb = ks * kn;  // this wave's k range (a multiple of 32 long)
  static_assert(kRouterWaves % CT == 0, "waves per tile");
  const float *xp = a.x + (uint64_t)row * a.hid + kb + 8 * h;
  const uint16_t *wp = a.router + (uint64_t)col * a.hid + kb + 8 * h;
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  // k steps in batches of U, the next batch's loads in flight while this one multiplies (kn is a multiple of 32,
  // so batches are whole: kn / 16 steps, U = 2)
  constexpr int U = 2;
  float4 xv[2][U][2];
  uint4 wv[2][U];
  auto load = [&](int b, int k0) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      xv[b][u][0] = *(const float4 *)(xp + k0 + 16 * u);
      xv[b][u][1] = *(const float4 *)(xp + k0 + 16 * u + 4);
      wv[b][u] = *(const uint4 *)(wp + k0 + 16 * u);
    }
  };
  auto mul = [&](int b) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const float xs[8] = {xv[b][u][0].x, xv[b][u][0].y, xv[b][u][0].z, xv[b][u][0].w,
                           xv[b][u][1].x, xv[b][u][1].y, xv[b][u][1].z, xv[b][u][1].w};
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        hi[e] = (__bf16)xs[e];
        lo[e] = (__bf16)(xs[e] - (float)hi[e]);
      }
      const bf16x8 wb = __builtin_bit_cast(bf16x8, wv[b & 1][u]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, wb, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, wb, acc, 0, 0, 0);
    }
  };
  if (live) {
    load(0, 0);
    for (int k0 = 0; k0 < kn; k0 += 32 * U) {  // two batches per trip, so the buffer index stays compile-time
      if (k0 + 16 * U < kn) load(1, k0 + 16 * U);
      mul(0);
      if (k0 + 32 * U < kn) load(0, k0 + 32 * U);
      if (k0 + 16 * U < kn) mul(1);
    }
  }
#pragma unroll
  for (int i = 0; i < 16; i++) red[wave][i][lane] = acc[i];
  __syncthreads();
  for (int o = threadIdx.x; o < CT * 16 * 64; o += kRouterWaves * 64) {
    const int c = o / (16 * 64), i = (o >> 6) & 15, l = o & 63;
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < KSP; k++) v += red[k * CT + c][i][l];
    const int r = rt * 32 + 4 * (l >> 5) + (i & 3) + 8 * (i >> 2), cc = (blockIdx.y * CT + c) * 32 + (l & 31);
    if (r < a.R && cc < ncol) a.logits[(uint64_t)r * (a.ne + 1) + cc] = bf16_round(v);
  }
}

// Many rows: a workgroup covers 64 rows x 128 columns over the whole k range, wave (rb, ct) = wave (rb = wave / 4,
// ct = wave % 4) one 32 x 32 tile. The x rows are shared by the four column waves, so the workgroup stages each
// 64-wide k chunk of them once through LDS, already split into bf16 hi and lo (the conversion runs once per element
// per workgroup, and the rows cross from L2 once); each wave streams its own router columns from memory one chunk
// ahead. Same arithmetic as bat_router (hi and lo products summed in f32), one k order.
constexpr int kRtKc = 64, kRtRows = 64, kRtPitch = kRtKc + 8;  // k chunk, rows, LDS row pitch in bf16 (conflict-free)
__global__ __launch_bounds__(512, 2) void bat_router_rows(MoeArgs a, int ngroups) {
  __shared__ __attribute__((aligned(16))) __bf16 xs[2][2][kRtRows * kRtPitch];  // [buffer][hi, lo]
  int item;
  if (!xcd_item(ngroups * ((a.ne + a.has_sgate + 127) / 128), item)) return;
  const int ncol = a.ne + a.has_sgate, ncg = (ncol + 127) / 128, rg = item / ncg, cg = item % ncg;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, rb = wave >> 2, ct = cg * 4 + (wave & 3);
  const int m = lane & 31, h = lane >> 5;
  const bool live = ct * 32 < ncol;
  // staging: thread t converts row t / 8, k [8 (t % 8), +8) of the chunk
  const int srow = threadIdx.x >> 3, sk = (threadIdx.x & 7) * 8;
  const float *xp = a.x + (uint64_t)min(rg * kRtRows + srow, a.R - 1) * a.hid + sk;
  const uint16_t *wp = a.router + (uint64_t)min(ct * 32 + m, ncol - 1) * a.hid + 8 * h;
  const int nch = a.hid / kRtKc;
  float4 xr[2];
  uint4 wv[2][kRtKc / 16];
  auto load_x = [&](int c) {
    xr[0] = *(const float4 *)(xp + c * kRtKc);
    xr[1] = *(const float4 *)(xp + c * kRtKc + 4);
  };
  auto load_w = [&](int b, int c) {
#pragma unroll
    for (int u = 0; u < kRtKc / 16; u++) wv[b][u] = *(const uint4 *)(wp + c * kRtKc + 16 * u);
  };
  auto stage = [&](int b) {
    const float v[8] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w, xr[1].x, xr[1].y, xr[1].z, xr[1].w};
    bf16x8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      hi[e] = (__bf16)v[e];
      lo[e] = (__bf16)(v[e] - (float)hi[e]);
    }
    *(bf16x8 *)&xs[b][0][srow * kRtPitch + sk] = hi;
    *(bf16x8 *)&xs[b][1][srow * kRtPitch + sk] = lo;
  };
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  auto mul = [&](int b) {
    const __bf16 *ph = &xs[b][0][(rb * 32 + m) * kRtPitch + 8 * h], *pl = &xs[b][1][(rb * 32 + m) * kRtPitch + 8 * h];
#pragma unroll
    for (int u = 0; u < kRtKc / 16; u++) {
      const bf16x8 hi = *(const bf16x8 *)(ph + 16 * u), lo = *(const bf16x8 *)(pl + 16 * u);
      const bf16x8 wb = __builtin_bit_cast(bf16x8, wv[b][u]);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, wb, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, wb, acc, 0, 0, 0);
    }
  };
  // chunk c: stage it (its x already in registers), request chunk c + 1, one barrier, multiply. The buffer written
  // at chunk c + 1 was last read at chunk c - 1, before every wave passed chunk c's barrier.
  load_x(0);
  if (live) load_w(0, 0);
  for (int c = 0; c < nch; c += 2) {
    stage(0);
    if (c + 1 < nch) {
      load_x(c + 1);
      if (live) load_w(1, c + 1);
    }
    __syncthreads();
    if (live) mul(0);
    if (c + 1 < nch) {
      stage(1);
      if (c + 2 < nch) {
        load_x(c + 2);
        if (live) load_w(0, c + 2);
      }
      __syncthreads();
      if (live) mul(1);
    }
  }
  if (!live) return;
  const int cc = ct * 32 + m;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int r = rg * kRtRows + rb * 32 + 4 * h + (i & 3) + 8 * (i >> 2);
    if (r < a.R && cc < ncol) a.logits[(uint64_t)r * (a.ne + 1) + cc] = bf16_round(acc[i]);
  }
}

// Few rows (speculative verify): logits with the one-row step's arithmetic, so that a row of a batch routes exactly
// as it would alone. Wave w of workgroup (b, r): router column 4 b + w for row r; lane l holds elements
// [512 j + 8 l, +8) of the column, j < hid / 512 (all requested at once), and chains one fmaf per element in that
// order, then the lanes' sums meet in an xor butterfly over lane distances 32, 16, .., 1 (reference
// kernels/fn_moe.metal:50-67).
constexpr int kRouterExactChunks = 16;  // hid <= 8192
// NC: the chunk bound the registers are sized for (hid / 512 <= NC): 4 at hid 2048 keeps the wave at ~50 registers
// (eight waves per SIMD to cover the loads' latency) instead of ~200 for the largest hidden size
template <int NC>
__global__ __launch_bounds__(256) void bat_router_exact(MoeArgs a) {
  const int lane = threadIdx.x & 63, col = blockIdx.x * 4 + (threadIdx.x >> 6), r = blockIdx.y, nc = a.hid / 512;
  if (col >= a.ne + a.has_sgate) return;
  const uint16_t *w = a.router + (uint64_t)col * a.hid + lane * 8;
  const float *x = a.x + (uint64_t)r * a.hid + lane * 8;
  uint4 wv[NC];
  float4 x0[NC], x1[NC];
#pragma unroll
  for (int j = 0; j < NC; j++)
    if (j < nc) {
      wv[j] = *(const uint4 *)(w + j * 512);
      x0[j] = *(const float4 *)(x + j * 512);
      x1[j] = *(const float4 *)(x + j * 512 + 4);
    }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NC; j++)
    if (j < nc) {
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
  if (lane == 0) a.logits[(uint64_t)r * (a.ne + 1) + col] = bf16_round(acc);
}

// ---------------------------------------------------------------------------------------------------- route
// one wave per row
template <int J>
__device__ void route_one(const MoeArgs &a, int r, uint32_t *lid = nullptr) {
  const int lane = threadIdx.x & 63;
  const float *lg = a.logits + (uint64_t)r * (a.ne + 1);
  const float sgl = a.has_sgate ? lg[a.ne] : 0.f;  // the shared-expert gate logit, requested with the others
  uint32_t key[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int i = j * 64 + lane;
    key[j] = i < a.ne ? topk_key(lg[i], i) : 0u;
  }
#pragma unroll
  for (int s = 2; s <= J; s <<= 1)
#pragma unroll
    for (int d = s >> 1; d > 0; d >>= 1)
#pragma unroll
      for (int i = 0; i < J; i++) {
        const int l = i ^ d;
        if (l > i) {
          const uint32_t hi = max(key[i], key[l]), lo = min(key[i], key[l]);
          key[i] = (i & s) == 0 ? hi : lo;
          key[l] = (i & s) == 0 ? lo : hi;
        }
      }
  uint32_t mykey = 0u;
  for (int t = 0; t < a.topk; t++) {
    const uint32_t m = wave_max_u32(key[0]);
    mykey = lane == t ? m : mykey;
    const bool win = key[0] == m;
#pragma unroll
    for (int j = 0; j < J - 1; j++) key[j] = win ? key[j + 1] : key[j];
    key[J - 1] = win ? 0u : key[J - 1];
  }
  const uint32_t id = lane < a.topk ? 0xFFFFu - (mykey & 0xFFFFu) : 0u;  // lanes past topk: expert 0, unused
  // the selected logits come back out of their keys (no second load), as in the fused step
  const float top = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(key_value(mykey)), 0));
  const float pk = lane < a.topk ? expf(key_value(mykey) - top) : 0.f;
  float sum = 0.f;
  for (int k = 0; k < a.topk; k++) sum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pk), k));
  if (lane < a.topk) {  // device-coherent stores: bat_route_place's last workgroup reads other workgroups' routes
    st_cg(a.route + (uint64_t)r * 2 * a.topk + lane, id);
    st_cg(a.route + (uint64_t)r * 2 * a.topk + a.topk + lane, __float_as_uint(pk / sum));
    if (lid) lid[r * a.topk + lane] = id;  // the caller's LDS copy of the ids
  }
  if (lane == 0) a.sgv[r] = moe_shared_gate(a, sgl);
}
__global__ __launch_bounds__(256) void bat_route(MoeArgs a) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.R) return;
  if (a.ne <= 512)
    route_one<8>(a, r);
  else
    route_one<16>(a, r);
}

// ---------------------------------------------------------------------------------------------------- sort
// Routed slots per expert: each workgroup takes a contiguous run of the route's [R][2 topk] words (ids, then
// weights) in 16-byte groups, counts the ids among them in LDS and adds its nonzero counts to bk[0 .. ne) (zero on
// entry: set at allocation and again by bat_scan once it has read them).
constexpr int kHistGroups = 64;
__global__ __launch_bounds__(256) void bat_hist(MoeArgs a, uint32_t *bk) {
  __shared__ uint32_t sc[1024];
  const int tid = threadIdx.x;
  for (int e = tid; e < a.ne; e += 256) sc[e] = 0u;
  __syncthreads();
  const int stride = 2 * a.topk, total = a.R * stride, groups = (total + 3) / 4;
  const int per = (groups + kHistGroups - 1) / kHistGroups, gb = blockIdx.x * per, ge = min(gb + per, groups);
  for (int g = gb + tid; g < ge; g += 256) {
    const int w0 = 4 * g;
    uint4 v;
    if (w0 + 4 <= total) {
      v = *(const uint4 *)(a.route + w0);
    } else {  // the last, partial group
      const uint32_t *w = a.route + w0;
      const int left = total - w0;
      v = make_uint4(w[0], left > 1 ? w[1] : 0u, left > 2 ? w[2] : 0u, 0u);
    }
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (w0 + q < total && (w0 + q) % stride < a.topk) atomicAdd(&sc[w4[q] < (uint32_t)a.ne ? w4[q] : 0u], 1u);
  }
  __syncthreads();
  for (int e = tid; e < a.ne; e += 256)
    if (sc[e]) atomicAdd(bk + e, sc[e]);
}
// One workgroup: offsets (exclusive scan over experts; the shared expert's R rows last), the chunk list and the
// placement cursors. bk: [ne + 1] counts (in; routed experts from bat_hist), [ne + 1] offsets, [ne + 1] cursors, then
// 1 chunk count; chunks: u32x3.
// With self_count (few rows) the workgroup counts the route itself instead (one launch fewer).
__global__ __launch_bounds__(1024) void bat_scan(MoeArgs a, uint32_t *bk, uint32_t *chunks, int max_chunks,
                                                 int self_count, uint32_t crows) {
  __shared__ uint32_t sc[1024 + 1], cc[1024 + 1];
  const int tid = threadIdx.x, n = a.ne + (a.nslot > a.topk ? 1 : 0);
  uint32_t *counts = bk, *offs = bk + (a.ne + 1), *cursor = offs + (a.ne + 1), *nchunks = cursor + (a.ne + 1);
  if (!self_count) {
    sc[tid] = tid < a.ne ? counts[tid] : 0u;
  } else {
    // routed slots per expert: a histogram of the route ids in LDS (one workgroup: no global atomics to contend)
    // The route is [R][2 topk] words (ids, then weights): each thread takes a contiguous run of whole 16-byte groups,
    // loaded together, and adds the ids among them.
    sc[tid] = 0u;
    __syncthreads();
    {
      const int stride = 2 * a.topk, total = a.R * stride, groups = (total + 3) / 4;
      const int per = (groups + 1023) / 1024, g0 = tid * per, g1 = min(g0 + per, groups);
      constexpr int B = 8;  // groups requested at once
      int col = (g0 * 4) % stride;  // column of the next word inside its row (ids below topk)
      for (int g = g0; g < g1; g += B) {
        uint4 v[B];
#pragma unroll
        for (int j = 0; j < B; j++)
          if (g + j < g1) {
            if ((g + j) * 4 + 4 <= total) {
              v[j] = *(const uint4 *)(a.route + (size_t)(g + j) * 4);
            } else {  // the last, partial group
              const uint32_t *w = a.route + (size_t)(g + j) * 4;
              const int left = total - (g + j) * 4;
              v[j] = make_uint4(w[0], left > 1 ? w[1] : 0u, left > 2 ? w[2] : 0u, 0u);
            }
          }
#pragma unroll
        for (int j = 0; j < B; j++)
          if (g + j < g1) {
            const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
              if ((g + j) * 4 + q < total && col < a.topk) {
                const uint32_t e = w4[q];
                atomicAdd(&sc[e < (uint32_t)a.ne ? e : 0u], 1u);
              }
              col = col + 1 == stride ? 0 : col + 1;
            }
          }
      }
    }
  }
  __syncthreads();
  const uint32_t c = tid < a.ne ? sc[tid] : (tid < n ? (uint32_t)a.R : 0u);  // the shared expert takes every row
  __syncthreads();
  if (tid < a.ne) counts[tid] = 0u;  // ready for the next layer's bat_hist
  sc[tid] = c;
  cc[tid] = (c + crows - 1) / crows;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // inclusive Hillis-Steele scans of rows and chunks
    const uint32_t v = tid >= d ? sc[tid - d] : 0u, w = tid >= d ? cc[tid - d] : 0u;
    __syncthreads();
    sc[tid] += v;
    cc[tid] += w;
    __syncthreads();
  }
  if (tid < n) {
    const uint32_t off = sc[tid] - c, ch0 = cc[tid] - (c + crows - 1) / crows;
    offs[tid] = off;
    cursor[tid] = 0u;
    for (uint32_t r = 0, q = ch0; r < c; r += crows, q++)
      if ((int)q < max_chunks) {
        chunks[3 * q] = (uint32_t)tid;
        chunks[3 * q + 1] = off + r;
        chunks[3 * q + 2] = min(c - r, crows);
      }
  }
  if (tid == 0) *nchunks = min(cc[n > 0 ? n - 1 : 0], (uint32_t)max_chunks);
}
// Few rows (R <= 32): the route, the chunk list and the placement in one workgroup (three launches fewer). Waves take
// rows for the top-k (route_one: the one-row step's keys and weights); then the routed slots per expert are counted in
// LDS, scanned into offsets and chunks of at most crows rows (the shared expert takes every row, last), and each slot
// takes its row in its expert's list (rows[row] = r * nslot + k; the order inside an expert changes no result).
// The route of 4 rows per workgroup (waves 0-3, one per SIMD: the top-k rounds are a serial chain on one wave), then
// the workgroup that arrives last (a count in bk, reset by it) places every slot: per-expert counts, offsets and the
// chunk list (as bat_scan, chunks of at most crows rows), and each slot's row in its expert's list.
constexpr int kRouteRows = 4;
__global__ __launch_bounds__(1024) void bat_route_place(MoeArgs a, uint32_t *bk, uint32_t *chunks, int max_chunks,
                                                        uint32_t crows, uint32_t *rows) {
  __shared__ uint32_t sc[1024], cc[1024], offl[1024], cur[1024], lid[1024];
  __shared__ uint32_t s_last;
  const int tid = threadIdx.x, wave = tid >> 6, n = a.ne + (a.nslot > a.topk ? 1 : 0);
  const int r = (int)blockIdx.x * kRouteRows + wave;
  if (wave < kRouteRows && r < a.R) {
    if (a.ne <= 512)
      route_one<8>(a, r);
    else
      route_one<16>(a, r);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's route stores have completed
  __syncthreads();
  uint32_t *arrived = bk + 3 * (a.ne + 1) + 1;
  if (tid == 0) s_last = atomicAdd(arrived, 1u) == gridDim.x - 1 ? 1u : 0u;
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) st_cg(arrived, 0u);  // for the next launch
  for (int q = tid; q < a.R * a.topk; q += 1024)  // every row's ids, as stored
    lid[q] = ld_cg(a.route + (uint64_t)(q / a.topk) * 2 * a.topk + q % a.topk);
  sc[tid] = 0u;
  cur[tid] = 0u;
  __syncthreads();
  for (int s = tid; s < a.R * a.topk; s += 1024) {
    const uint32_t e = lid[s];
    atomicAdd(&sc[e < (uint32_t)a.ne ? e : 0u], 1u);
  }
  __syncthreads();
  const uint32_t c = tid < a.ne ? sc[tid] : (tid < n ? (uint32_t)a.R : 0u);  // the shared expert takes every row
  // inclusive scans of rows and chunks: within each wave by lane shifts, then the 16 wave totals by wave 0
  const int lane = tid & 63;
  uint32_t sv = c, cv = (c + crows - 1) / crows;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t v = (uint32_t)__shfl_up((int)sv, d, 64), w = (uint32_t)__shfl_up((int)cv, d, 64);
    if (lane >= d) {
      sv += v;
      cv += w;
    }
  }
  __shared__ uint32_t wsum[2][16];
  if (lane == 63) {
    wsum[0][wave] = sv;
    wsum[1][wave] = cv;
  }
  __syncthreads();
  if (wave == 0 && lane < 32) {  // lanes 0-15: the rows' wave totals; 16-31: the chunks'
    const int t = lane & 15, arr = lane >> 4;
    uint32_t x = wsum[arr][t];
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) {
      const uint32_t v = (uint32_t)__shfl_up((int)x, d, 16);
      if (t >= d) x += v;
    }
    wsum[arr][t] = x;  // inclusive over waves
  }
  __syncthreads();
  sc[tid] = sv + (wave > 0 ? wsum[0][wave - 1] : 0u);
  cc[tid] = cv + (wave > 0 ? wsum[1][wave - 1] : 0u);
  __syncthreads();
  if (tid < n) {
    const uint32_t off = sc[tid] - c, ch0 = cc[tid] - (c + crows - 1) / crows;
    offl[tid] = off;
    for (uint32_t r = 0, q = ch0; r < c; r += crows, q++)
      if ((int)q < max_chunks) {
        chunks[3 * q] = (uint32_t)tid;
        chunks[3 * q + 1] = off + r;
        chunks[3 * q + 2] = min(c - r, crows);
      }
  }
  if (tid == 0) bk[3 * (a.ne + 1)] = min(cc[n > 0 ? n - 1 : 0], (uint32_t)max_chunks);
  __syncthreads();
  for (int s = tid; s < a.R * a.nslot; s += 1024) {
    const int r = s / a.nslot, k = s % a.nslot;
    uint32_t e = (uint32_t)a.ne, pos = (uint32_t)r;  // the shared expert's list is every token in order
    if (k < a.topk) {
      e = lid[r * a.topk + k];
      e = e < (uint32_t)a.ne ? e : 0u;
      pos = atomicAdd(&cur[e], 1u);
    }
    rows[offl[e] + pos] = (uint32_t)s;
  }
}
// One wave per slot (r, k): takes the slot's row in its expert's list (rows[row] = r * nslot + k; k == topk: the
// shared expert, whose list is every token in order) and writes that row of the A operand:
// xh[row] = [gate | up] fp16(H(x[r] * suh_e)) in kp order (the two projections have their own suh).
// The 128-wide Hadamard runs on the matrix cores. H_128 = H_4 (x) H_32 in the split i = 32 q + j, so for the 32
// vectors of a tile (gate and up of 16 blocks) the wave multiplies each 32-chunk q' by H_32
// (v_mfma_f32_32x32x16_f16, H as the A operand, the vectors as B), then combines the four chunk products with H_4 in
// registers. The rows of H_32 are permuted so that output row m lands where the matrix-core layout lets one lane
// hold 16 consecutive kp positions (16 h + i, i = 0..15, of each 32-chunk): every lane then stores 32 contiguous
// bytes per chunk. Each vector is scaled by a power of two (its largest element to [2^14, 2^15)) and split into f16
// hi + lo, both rounded to nearest (about 23 bits reach the products, summed in f32): a result differs from a
// butterfly transform's by f32 rounding only.
__device__ __forceinline__ uint32_t kp_inv32(uint32_t u) {  // kp restricted to 0..31, inverted
  return (u & 16u) | (((u >> 1) & 1u) << 3) | (((u >> 2) & 3u) << 1) | (u & 1u);
}
// LDS per wave (16-byte units; a pad unit after every 64, so a direct-to-LDS load of 64 lanes fills one run):
//   x part:  block b of the tile (128 f32 = 32 units) in run b / 2; an odd block is rotated by 8 units:
//            unit u of block b at 65 (b / 2) + 32 (b % 2) + ((u + 8 (b % 2)) % 32)
//   su part: projection p, block b (128 f16 = 16 units) at 260 p + 65 (b / 4) + 16 (b % 4) + ((u + 4 (b % 4)) % 16)
//   output (reuses the x part): vector v (32 = gate blocks, then up blocks; 16 units) at
//            65 (v / 4) + 16 (v % 4) + ((c + 4 (v % 4)) % 16)
// With these, every matrix-core fragment read and every output write of 8 consecutive lanes hits 8 distinct 4-bank
// groups, each lane's unit offsets differ from one per-lane base by compile-time amounts, and each load lane's
// source offset is the same for all runs (the loads are 1 KB contiguous each: loading the fragments straight into
// registers, 16 scattered bytes per lane, is slower).
constexpr int kPrepUnits = 1040;  // x / output part 520 units, su part 520
constexpr int kPrepWaves = 4;
constexpr size_t kPrepLds = (size_t)kPrepWaves * kPrepUnits * 16;
__global__ __launch_bounds__(64 * kPrepWaves, 2) void bat_place_prep(MoeArgs a, uint32_t *bk, uint32_t *rows,
                                                                      uint16_t *xh) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int s = blockIdx.x * kPrepWaves + wave;  // wave-uniform, so the row's buffer descriptors are too
  if (s >= a.R * a.nslot) return;
  uint8_t *lx = lds + (size_t)wave * kPrepUnits * 16, *lsu = lx + 520 * 16;
  // routed slots first (row-major), then the shared expert's rows in order
  const int nrs = a.R * a.topk;
  const int r = s < nrs ? s / a.topk : s - nrs, k = s < nrs ? s % a.topk : a.topk;
  const int n = lane & 31, h = lane >> 5, proj = n >> 4, bl = n & 15, nb = a.hid / 128;
  const float *x = a.x + (uint64_t)r * a.hid;
  // load lanes: source byte offsets inside a run (x: two blocks of 512 B; su: four blocks of 256 B)
  const uint32_t vx = lane < 32 ? 16u * lane : 512u + 16u * ((lane - 40) & 31);
  const uint32_t vs = 256u * (lane >> 4) + 16u * (((lane & 15) - 4 * (lane >> 4)) & 15);
  // the tile's x (blocks past the row's end read zeros); the first tile's is requested before the route is read
  auto load_x = [&](int t0) {
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)(x + t0 * 128), (short)0,
                                                                        (a.hid - t0 * 128) * 4, 0x00020000);
#pragma unroll
    for (int j = 0; j < 8; j++) dma16_buf(rx, vx, 1024u * j, lx + 65 * 16 * j);
  };
  load_x(0);
  const uint32_t *offs = bk + (a.ne + 1);
  uint32_t *cursor = bk + 2 * (a.ne + 1);
  int e = a.ne;
  if (k < a.topk) {
    e = (int)a.route[(uint64_t)r * 2 * a.topk + k];
    e = e < a.ne ? e : 0;
  }
  e = __builtin_amdgcn_readfirstlane(e);  // one slot per wave: the expert's layout then stays in scalar registers
  // the slot's row, first needed by the stores: the cursor atomic is requested here and its result waited for there.
  // (The cursor's address goes through an empty asm so that the compiler sees a per-lane address: its rewrite of a
  // uniform-address atomic would consume the result, and so wait for it, right away.)
  uint32_t pos = (uint32_t)r;  // the shared expert's list is every token in order
  if (lane == 0 && k < a.topk) {
    uint32_t *pc = cursor + e;
    asm volatile("" : "+v"(pc));
    pos = __hip_atomic_fetch_add((__attribute__((address_space(1))) uint32_t *)pc, 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);  // a global (not flat) atomic: no wait for the LDS loads
  }
  const uint32_t base = offs[e];
  // A operand: lane (m = n, h) holds H_32[j(m)][16 st + 8 h + t] for k steps st = 0, 1, where output row m is kp
  // position d = 16 ((m >> 2) & 1) + 4 (m >> 3) + (m & 3) of the chunk, i.e. element j(m) = kp^-1(d)
  f16x8 hA[2];
  {
    const uint32_t j = kp_inv32(16u * ((n >> 2) & 1) + 4u * (n >> 3) + (n & 3));
#pragma unroll
    for (int st = 0; st < 2; st++)
#pragma unroll
      for (int t = 0; t < 8; t++)
        hA[st][t] = (__builtin_popcount(j & (uint32_t)(16 * st + 8 * h + t)) & 1) ? (_Float16)-1.f : (_Float16)1.f;
  }
  // fragment bases (bytes) per chunk q: x units 8 q + 4 st + 2 h + w, su units 4 q + 2 st + h, output units 4 q + 2 h + w
  uint32_t xb[4], sb[4], ob[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int odd = bl & 1, m4 = bl & 3, v4 = n & 3;
    xb[q] = 16u * (65 * (bl >> 1) + 32 * odd + 8 * ((q + odd) & 3) + 2 * h);
    sb[q] = 16u * (260 * proj + 65 * (bl >> 2) + 16 * m4 + 4 * ((q + m4) & 3) + h);
    ob[q] = 16u * (65 * (n >> 2) + 16 * v4 + 4 * ((q + v4) & 3) + 2 * h);
  }
  // store lanes: unit c = lane % 16 of vector 4 j + lane / 16 (store j); its global offset is 16 lane bytes
  const uint32_t rb = 16u * (16 * (lane >> 4) + (((lane & 15) + 4 * (lane >> 4)) & 15));
  const uint8_t *eb = expert_block(a, e);
  const uint16_t *sug = (const uint16_t *)(eb + su_of(a, e, 0)), *suu = (const uint16_t *)(eb + su_of(a, e, 1));
  uint16_t *orow_p = nullptr;
  for (int t0 = 0; t0 < nb; t0 += 16) {
    const int nbl = min(nb - t0, 16);  // blocks of this tile; loads past the row's end read zeros
    {
      if (t0 > 0) load_x(t0);
      const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc((void *)(sug + t0 * 128), (short)0,
                                                                          (a.hid - t0 * 128) * 2, 0x00020000);
      const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc((void *)(suu + t0 * 128), (short)0,
                                                                          (a.hid - t0 * 128) * 2, 0x00020000);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        dma16_buf(rg, vs, 1024u * j, lsu + 65 * 16 * j);
        dma16_buf(ru, vs, 1024u * j, lsu + (260 + 65 * j) * 16);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the tile is in LDS
    // v = x * suh for this lane's 64 elements of vector n, and the vector's largest |v| (lanes n and n + 32)
    float v[4][2][8];
    float mx = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int st = 0; st < 2; st++) {
        const float4 x0 = *(const float4 *)(lx + xb[q] + 16 * (4 * st));
        const float4 x1 = *(const float4 *)(lx + xb[q] + 16 * (4 * st + 1));
        const f16x8 sh = *(const f16x8 *)(lsu + sb[q] + 16 * (2 * st));
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int t = 0; t < 8; t++) {
          v[q][st][t] = __builtin_fmaf(xv[t], (float)sh[t], 0.f);
          mx = fmaxf(mx, fabsf(v[q][st][t]));
        }
      }
    mx = fmaxf(mx, xor_lane<32>(mx, lane));
    // exact power-of-two scale putting the largest |v| in [2^14, 2^15): the split then stays clear of both the f16
    // overflow and its subnormals; the output takes the inverse scale with 1/sqrt(128)
    const int ex = min(max(141 - (int)((__float_as_uint(mx) >> 23) & 0xFFu), -126), 127);
    const float osc = __builtin_ldexpf(a.sc_hid, -ex);
    f32x16 acc[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int i = 0; i < 16; i++) acc[q][i] = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int st = 0; st < 2; st++) {
        f16x8 hi, lo;
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const float w = __builtin_ldexpf(v[q][st][t], ex);  // hi, lo rounded to nearest: v - hi exact in f32
          hi[t] = (_Float16)w;
          lo[t] = (_Float16)(w - (float)hi[t]);
        }
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(hA[st], hi, acc[q], 0, 0, 0);
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_f16(hA[st], lo, acc[q], 0, 0, 0);
      }
    // H_4 over the chunk products: out_q = sum_q' (-1)^popcount(q & q') T_q', scaled, to f16 in the output part
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float a0 = acc[0][i] + acc[1][i], a1 = acc[0][i] - acc[1][i];
      const float a2 = acc[2][i] + acc[3][i], a3 = acc[2][i] - acc[3][i];
      acc[0][i] = (a0 + a2) * osc;
      acc[1][i] = (a1 + a3) * osc;
      acc[2][i] = (a0 - a2) * osc;
      acc[3][i] = (a1 - a3) * osc;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; i++)
        w[i] = __builtin_bit_cast(uint32_t, f16x2{(_Float16)acc[q][2 * i], (_Float16)acc[q][2 * i + 1]});
      *(uint4 *)(lx + ob[q]) = make_uint4(w[0], w[1], w[2], w[3]);
      *(uint4 *)(lx + ob[q] + 16) = make_uint4(w[4], w[5], w[6], w[7]);
    }
    __builtin_amdgcn_wave_barrier();  // one wave's LDS accesses run in order: its writes are seen by its reads
    // the row: gate at [0, hid), up at [hid, 2 hid); store j covers vectors 4 j .. 4 j + 3, 1 KB contiguous
    orow_p = xh + (uint64_t)((uint32_t)__builtin_amdgcn_readfirstlane(base) +
                             (uint32_t)__builtin_amdgcn_readfirstlane(pos)) * 2 * a.hid;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint4 w = *(const uint4 *)(lx + rb + 65 * 16 * j);
      const int vb = 4 * (j & 3) + (lane >> 4);
      if (vb < nbl) *(uint4 *)((uint8_t *)(orow_p + (j >> 2) * a.hid + (t0 + 4 * (j & 3)) * 128) + 16 * lane) = w;
    }
    __builtin_amdgcn_wave_barrier();  // the next tile's loads into LDS come after these reads
  }
  if (lane == 0) rows[(orow_p - xh) / (2 * a.hid)] = (uint32_t)(r * a.nslot + k);
}

// Few rows (speculative verify): the placement, then the one-row step's prepared input.
// bat_place_rows: one thread per slot (r, k): its row in its expert's list (rows[row] = r * nslot + k; the shared
// expert's list is every token in order; the order inside an expert changes no result).
__global__ __launch_bounds__(256) void bat_place_rows(MoeArgs a, uint32_t *bk, uint32_t *rows) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s >= a.R * a.nslot) return;
  const int r = s / a.nslot, k = s % a.nslot;
  const uint32_t *offs = bk + (a.ne + 1);
  uint32_t *cursor = bk + 2 * (a.ne + 1);
  int e = a.ne;
  uint32_t pos = (uint32_t)r;
  if (k < a.topk) {
    e = (int)a.route[(uint64_t)r * 2 * a.topk + k];
    e = e < a.ne ? e : 0;
    pos = atomicAdd(cursor + e, 1u);
  }
  rows[offs[e] + pos] = (uint32_t)s;
}
// bat_prep_rows: wave (row, 128-wide chunk c, projection) of the placed rows: a lane butterfly per chunk,
// v = x * suh (f32), H_128 with 1/sqrt(128), fp16, kp order (reference kernels/fn_moe.metal:140-160)
__global__ __launch_bounds__(256) void bat_prep_rows(MoeArgs a, const uint32_t *rows, uint16_t *xh) {
  const int lane = threadIdx.x & 63, nq = 2 * (a.hid / 128);
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6), row = w / nq, q = w % nq, proj = q & 1, c = q >> 1;
  if (row >= a.R * a.nslot) return;
  const uint32_t s = rows[row];
  const int r = (int)s / a.nslot, k = (int)s % a.nslot;
  int e = a.ne;
  if (k < a.topk) {
    e = (int)a.route[(uint64_t)r * 2 * a.topk + k];
    e = e < a.ne ? e : 0;
  }
  const uint16_t *su = (const uint16_t *)(expert_block(a, e) + su_of(a, e, proj)) + c * 128;
  const float *x = a.x + (uint64_t)r * a.hid + c * 128;
  float v0 = x[lane] * h2f(su[lane]), v1 = x[lane + 64] * h2f(su[lane + 64]);
  fwht2(v0, v1, lane, 128, a.sc_hid);
  uint16_t *o = xh + ((uint64_t)row * 2 + proj) * a.hid + c * 128;
  o[kp((uint32_t)lane)] = f2h(v0);
  o[kp((uint32_t)lane + 64)] = f2h(v1);
}

// ---------------------------------------------------------------------------------------------------- grouped GEMM
// One workgroup (8 waves, two per SIMD) multiplies a chunk of up to 128 expert-sorted rows of A by one tile pair (32
// columns) per wave of the expert's re-laid matrix (IT k tiles, IT even), two k tiles per step. There are NA A
// operands (fp16, kp order, row stride lda halves, the second at A + ahalf): wave w multiplies operand aidx. Both
// stream through LDS rings: A (shared; each wave requests 16 of its rows) kDA steps ahead, and each wave's own B
// tiles kDB steps ahead, so that enough weight bytes are in flight per CU to cover the memory latency.
// acc[rb] = rows 32 rb.., the wave's 32 columns, in the matrix-core layout.
constexpr int kWavesG = 8;
// Two workgroups share a CU (so four waves per SIMD hide each other's latency): each keeps under 80 KB of LDS.
// Steps (of 2 k tiles) requested ahead: A kDA, B kDB; the B ring's slot count is a multiple of the A ring's, so that
// the k loop, unrolled by the B ring's length, addresses every ring slot with compile-time offsets.
template <int K>
constexpr int kDA = K >= 6 ? 1 : 2;
template <int K>
constexpr int kDB = K >= 6 ? 3 : 5;
// NR: rows of a chunk, 128 (4 row blocks) or 32 (1 row block, for at most 32 rows: a quarter of the A ring, so that
// three workgroups share a CU)
template <int K, int NA, int NR = kChunkRows>
struct GemmIo {
  static constexpr uint32_t TB = 32u * K;                  // bytes of one 16x16 tile
  static constexpr uint32_t PB = 2 * 2 * TB;               // a wave's B bytes per step (a pair x 2 k tiles)
  static constexpr uint32_t AB = NA * NR * 64;             // A bytes per step (NA x NR rows x 32 halves)
  static constexpr int DA = kDA<K>, DB = kDB<K>;
  static constexpr int RA = DA + 1, RB = DB + 1;           // ring slots
  static constexpr uint32_t LDS_RING = RA * AB + kWavesG * RB * PB;
  // the epilogues: row-major, 32 x 256 floats; transposed (NR = 128 only), 32 x 32 float tiles with a 36-float row
  // pitch: 8 (down), 8 + 4 (gate/up)
  static constexpr uint32_t EPI = NR == kChunkRows ? (NA == 2 ? 12u : 8u) * 32u * 36u * 4u : 32u * 256u * 4u;
  static constexpr uint32_t LDS = LDS_RING > EPI ? LDS_RING : EPI;
  // requests per A step: NR = 128, each wave loads 16 rows of each operand; NR = 32, each wave one slice of
  // NA NR / 8 rows (its lanes past 4 rows each idle)
  static constexpr int OA = NR == kChunkRows ? NA : 1, OB = (PB + 1023) / 1024;
  static constexpr int NRB = NR / 32;
  static_assert(LDS <= 81920, "two workgroups per CU");
  static_assert(NR == kChunkRows || (NR == 32 && LDS <= 53248), "three workgroups per CU at 32 rows");
  static_assert(RB % RA == 0 && DB > DA, "ring shapes");
};
template <int OA, int OB, int DA, int DB>
__device__ __forceinline__ void wait_step(int t, int NS) {
  static_assert(kAfterSteady<OA, OB, DA> <= 15, "vmcnt immediate");
  if (steady_step<DB>(t, NS))
    __builtin_amdgcn_s_waitcnt(0x0F70 | kAfterSteady<OA, OB, DA>);
  else
    wait_vm15(after_step<OA, OB, DA, DB>(t, NS));
}

// decodes the lane's B operand for both k tiles of one step straight from the ring bytes src
template <int K>
__device__ __forceinline__ void decode_step(const uint8_t *src, const BLane<K> &B, f16x8 (&bf)[2]) {
  constexpr int TW = 8 * K;
  const uint32_t *T = (const uint32_t *)src + B.tile * TW;
  TileWords w[4];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const uint32_t *Tu = T + u * 2 * TW;
    w[2 * u].w0 = Tu[B.g0.i0];
    w[2 * u].w1 = Tu[B.g0.i1];
    w[2 * u].w2 = kThreeWords<K> ? Tu[B.g0.i2] : 0u;
    w[2 * u + 1].w0 = Tu[B.g1.i0];
    w[2 * u + 1].w1 = Tu[B.g1.i1];
    w[2 * u + 1].w2 = kThreeWords<K> ? Tu[B.g1.i2] : 0u;
  }
#pragma unroll
  for (int u = 0; u < 2; u++) {
    f16x2 l0, h0, l1, h1;
    decode4<K>(w[2 * u], B.g0.sh, l0, h0);
    decode4<K>(w[2 * u + 1], B.g1.sh, l1, h1);
    bf[u] = f16x8{l0.x, l0.y, h0.x, h0.y, l1.x, l1.y, h1.x, h1.y};
  }
}

// quarter swizzle of A row r: distinct 16-byte bank groups for rows r .. r + 7 (eight lanes of a 128-byte read phase)
// and for rows r .. r + 15 (sixteen lanes of a 256-byte phase), rows aligned to 8
__device__ __forceinline__ int a_swz(int r) { return ((r >> 1) ^ ((r >> 3) & 1)) & 3; }
// TR: the weights are the matrix cores' A operand and the rows their B operand, so acc[rb] holds the transposed
// product: lane (n, h) value i = output column 8 (i / 4) + 4 h + i % 4 of the wave's 32, row 32 rb + n.
// FG > 0 (k range a whole number of 128-wide k chunks from a chunk boundary): the one-row step's summation order
// instead of one chain: each k chunk's sum a chain of 8 MFMAs from zero, the chunk sums folded left in groups of FG,
// the group sums folded left (FG at least the chunk count: one left fold over the chunks).
template <int K, int NA, bool TR = false, int NR = kChunkRows, int FG = 0>
__device__ void chunk_gemm(const uint16_t *A, int lda, int ahalf, int aidx, int nrows, const uint8_t *tr, int IT,
                           int pair, uint8_t *lds, f32x16 (&acc)[NR / 32], uint64_t *dbg, int kt0, int nkt) {
  using Io = GemmIo<K, NA, NR>;
  constexpr int NRB = Io::NRB;
  constexpr int DA = Io::DA, U = Io::RB;  // the k loop is unrolled by the B ring's length
  const int lane = threadIdx.x & 63, NS = nkt / 2;  // k tiles [kt0, kt0 + nkt) of IT (nkt even)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t *ring_a = lds;
  uint8_t *ring_b = lds + Io::RA * Io::AB + wave * Io::RB * Io::PB;
  const BLane<K> BL = b_lane<K>((uint32_t)lane);
  const int nrb = (nrows + 31) / 32;
#pragma unroll
  for (int rb = 0; rb < NRB; rb++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[rb][i] = 0.f;
  static_assert(FG == 0 || !TR, "the one-row order on row-major products");
  f32x16 grp[FG ? NRB : 1], tot[FG ? NRB : 1];  // FG: the open group's fold, the closed groups' fold
  // A(t): NR = 128: 16 rows of this wave per operand; NR = 32: the wave's slice of RW = 4 NA rows of operand
  // (RW w) / 32. Row r's 64 bytes (four 16-byte quarters q: k 8q .. 8q + 7) sit at r * 64 with quarter q in position
  // q ^ a_swz(r), so that a read of one quarter of consecutive rows is free of bank conflicts. DMA lane l fills
  // position l % 4 of row r0 + l / 4 (r0 the wave's first row). Stream addresses are a wave-uniform base plus a fixed
  // per-lane offset.
  constexpr int RW = NR == kChunkRows ? 16 : 4 * NA;
  const int ao = NR == kChunkRows ? 0 : (wave * RW) / NR, r0 = NR == kChunkRows ? wave * 16 : (wave * RW) % NR;
  const int rr = min(r0 + (lane >> 2), nrows - 1);
  const uint32_t a_off = (uint32_t)(rr * lda + ((lane & 3) ^ a_swz(r0 + (lane >> 2))) * 8) * 2;
  const __amdgpu_buffer_rsrc_t ra = stream_rsrc(A + kt0 * 16);
  auto issue_a = [&](int t, int slot) {
    if constexpr (NR == kChunkRows) {
#pragma unroll
      for (int o = 0; o < NA; o++)
        dma16_buf(ra, a_off, (uint32_t)(o * ahalf * 2 + t * 64), ring_a + slot * Io::AB + o * NR * 64 + wave * 1024);
    } else {
      if (lane < 4 * RW)  // one request per wave and step (the idle lanes load nothing)
        dma16_buf(ra, a_off, (uint32_t)(ao * ahalf * 2 + t * 64), ring_a + slot * Io::AB + ao * NR * 64 + r0 * 64);
    }
  };
  // B(t): the wave's pair at k tiles 2t, 2t + 1 (contiguous)
  const __amdgpu_buffer_rsrc_t rb =
      stream_rsrc(tr + ((uint64_t)__builtin_amdgcn_readfirstlane(pair) * IT + kt0) * 2 * Io::TB);
  auto issue_b = [&](int t, int slot) {
#pragma unroll
    for (uint32_t o = 0; o < Io::PB; o += 1024)
      if (o + (uint32_t)lane * 16 < Io::PB)
        dma16_buf(rb, o + (uint32_t)lane * 16, (uint32_t)t * Io::PB, ring_b + slot * Io::PB + o);
  };
  // step s begins when A(s) and B(s) are in: every wave's rows of A(s) landed (barrier), and every wave has read
  // its fragments of A(s - 1), whose ring slot the step's A request then reuses. sb = s mod RB (compile-time).
  f16x8 bf[2];
  auto begin_step = [&](int s, int sb) {
    wait_step<Io::OA, Io::OB, DA, Io::DB>(s, NS);
    lds_barrier();
    if (s + DA < NS) issue_a(s + DA, (sb + DA) % Io::RA);
    if (s + Io::DB < NS) issue_b(s + Io::DB, (sb + Io::DB) % Io::RB);
    decode_step<K>(ring_b + sb * Io::PB, BL, bf);
  };
  for (int j = 0; j < Io::DB && j < NS; j++) {
    if (j < DA) issue_a(j, j % Io::RA);
    issue_b(j, j);
  }
  begin_step(0, 0);
  const uint8_t *a_lane = ring_a + aidx * NR * 64 + (lane & 31) * 64;
  const int q0 = ((lane >> 5) ^ a_swz(lane & 31)) * 16, q1 = ((2 + (lane >> 5)) ^ a_swz(lane & 31)) * 16;
  for (int t0 = 0; t0 < NS; t0 += U) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = t0 + u;
      if (t >= NS) break;
      const uint8_t *at = a_lane + (u % Io::RA) * Io::AB;
      const f16x8 b0 = bf[0], b1 = bf[1];
#pragma unroll
      for (int h = 0; h < 2; h++) {  // k tile h of the step for every row block: no two dependent MFMAs adjacent
        f16x8 af[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; rb++) af[rb] = *(const f16x8 *)(at + rb * 2048 + (h ? q1 : q0));
#pragma unroll
        for (int rb = 0; rb < NRB; rb++)
          if (rb < nrb)
            acc[rb] = TR ? __builtin_amdgcn_mfma_f32_32x32x16_f16(h ? b1 : b0, af[rb], acc[rb], 0, 0, 0)
                         : __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rb], h ? b1 : b0, acc[rb], 0, 0, 0);
      }
      if constexpr (FG > 0) {
        if (((t + 1) & 3) == 0) {  // k chunk (t + 1) / 4 - 1 complete (4 steps of 2 k tiles)
          const int c = (t + 1) / 4 - 1, ci = c % FG;
#pragma unroll
          for (int rb = 0; rb < NRB; rb++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
              grp[rb][i] = ci == 0 ? acc[rb][i] : grp[rb][i] + acc[rb][i];
              acc[rb][i] = 0.f;
            }
          if (ci == FG - 1) {
#pragma unroll
            for (int rb = 0; rb < NRB; rb++)
#pragma unroll
              for (int i = 0; i < 16; i++) tot[rb][i] = c + 1 == FG ? grp[rb][i] : tot[rb][i] + grp[rb][i];
          }
        }
      }
      // the matrix cores run while the next step's tiles decode
      if (t + 1 < NS) begin_step(t + 1, (u + 1) % U);
    }
  }
  if constexpr (FG > 0) {
    const int nc = NS / 4;  // k chunks; closed groups, and an open one past them
    const bool closed = nc >= FG, open = nc % FG != 0;
#pragma unroll
    for (int rb = 0; rb < NRB; rb++)
#pragma unroll
      for (int i = 0; i < 16; i++) acc[rb][i] = !closed ? grp[rb][i] : open ? tot[rb][i] + grp[rb][i] : tot[rb][i];
  }
}

// ---------------------------------------------------------------------------------------------------- Hadamard on
// the matrix cores, for a transposed product tile (lane (n, h) value i = column c = 8 (i / 4) + 4 h + i % 4 of 32,
// row n). H_128 over 128 columns = H_4 (x) H_32 in the split 32 q + j: each wave multiplies its own 32 columns by H_32
// here; the four waves of a 128-block combine with H_4 through LDS. With the columns of H permuted by c(k) (bits 2 and
// 3 of k swapped), k step st's B operand is values 8 st .. 8 st + 7 of the tile itself; output row m of the product
// is element J(m) of the chunk, J chosen by the caller for the layout it wants.
__device__ __forceinline__ uint32_t swap23(uint32_t k) { return (k & ~12u) | (((k >> 2) & 1u) << 3) | (((k >> 3) & 1u) << 2); }
template <typename J>
__device__ __forceinline__ void h32_operand(int lane, J jmap, f16x8 (&hA)[2]) {
  const uint32_t j = jmap((uint32_t)(lane & 31));
#pragma unroll
  for (int st = 0; st < 2; st++)
#pragma unroll
    for (int t = 0; t < 8; t++)
      hA[st][t] = (__builtin_popcount(j & swap23((uint32_t)(16 * st + 8 * (lane >> 5) + t))) & 1) ? (_Float16)-1.f
                                                                                                : (_Float16)1.f;
}
// T = H_32 . tile per row n: each row scaled by a power of two (its largest element to [2^14, 2^15), taken over the
// lane pair n, n + 32), split into f16 hi + lo rounded to nearest (about 23 bits, summed in f32), scaled back.
__device__ __forceinline__ f32x16 h32_tile(const f32x16 &v, const f16x8 (&hA)[2], int lane) {
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
  mx = fmaxf(mx, xor_lane<32>(mx, lane));
  const int ex = min(max(141 - (int)((__float_as_uint(mx) >> 23) & 0xFFu), -126), 127);
  f32x16 T;
#pragma unroll
  for (int i = 0; i < 16; i++) T[i] = 0.f;
#pragma unroll
  for (int st = 0; st < 2; st++) {
    f16x8 hi, lo;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const float w = __builtin_ldexpf(v[8 * st + t], ex);
      hi[t] = (_Float16)w;
      lo[t] = (_Float16)(w - (float)hi[t]);
    }
    T = __builtin_amdgcn_mfma_f32_32x32x16_f16(hA[st], hi, T, 0, 0, 0);
    T = __builtin_amdgcn_mfma_f32_32x32x16_f16(hA[st], lo, T, 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 16; i++) T[i] = __builtin_ldexpf(T[i], -ex);
  return T;
}

// EX (few rows, speculative verify): the one-row step's arithmetic throughout, so that every row is bit-identical
// to that row run alone: k chunk sums folded in its order, and the SiLU with the precise exp and divide.
constexpr int kFoldGroup = 4;        // gate/up: k chunks per group (the one-row step's tasks span 512 of k)
constexpr int kFoldAll = 1 << 20;    // down: one left fold over the k chunks (the one-row step's per-block partials)
// gate/up: chunk ch, 128-column block ib of inter; wave w: projection w / 4 (gate, up), pair 4 ib + w % 4
template <int K, int KS, bool TR, int NR, bool EX = false>
__global__ __launch_bounds__(512, NR == kChunkRows || EX ? 4 : 6) void bat_gateup(MoeArgs a, const uint32_t *bk, const uint32_t *chunks,
                                                     const uint32_t *rows, const uint16_t *xh, uint16_t *hh) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nib = a.inter / 128;
  int item;
  if (!xcd_item((int)bk[3 * (a.ne + 1)] * nib, item)) return;
  const int ch = item / nib, ib = item % nib;
  const int e = (int)chunks[3 * ch], row0 = (int)chunks[3 * ch + 1], nrows = (int)chunks[3 * ch + 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, proj = wave >> 2;
  const uint8_t *blk = expert_block(a, e);
  static_assert(!TR || NR == kChunkRows, "transposed products at 128-row chunks");
  constexpr int NRB = NR / 32;
  f32x16 acc[NRB];
  const uint16_t *A = xh + (uint64_t)row0 * 2 * a.hid;  // [row][gate | up][hid]
  const int pair = ib * 4 + (wave & 3);
  if (e >= a.ne)
    chunk_gemm<KS, 2, TR, NR, EX ? kFoldGroup : 0>(A, 2 * a.hid, a.hid, proj, nrows, blk + tr_of(a, e, proj), a.hid / 16,
                                                   pair, lds, acc, a.trace, 0, a.hid / 16);
  else
    chunk_gemm<K, 2, TR, NR, EX ? kFoldGroup : 0>(A, 2 * a.hid, a.hid, proj, nrows, blk + tr_of(a, e, proj), a.hid / 16,
                                                  pair, lds, acc, a.trace, 0, a.hid / 16);
  if constexpr (!TR) {
  // epilogue per 32-row block: columns to LDS as [32][256] f32 (gate 0..127, up 128..255), then one wave per row
  float *ot = (float *)lds;
  const uint16_t *svg = (const uint16_t *)(blk + sv_of(a, e, 0)) + ib * 128;
  const uint16_t *svu = (const uint16_t *)(blk + sv_of(a, e, 1)) + ib * 128;
  const uint16_t *sud = (const uint16_t *)(blk + su_of(a, e, 2)) + ib * 128;
  const float sg0 = h2f(svg[lane]), sg1 = h2f(svg[lane + 64]), su0 = h2f(svu[lane]), su1 = h2f(svu[lane + 64]);
  const float sd0 = h2f(sud[lane]), sd1 = h2f(sud[lane + 64]);
  const int nrb = (nrows + 31) / 32;
#pragma unroll
  for (int rb = 0; rb < NRB; rb++) {  // compile-time rb: acc stays in registers
    if (rb >= nrb) break;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = 4 * (lane >> 5) + (i & 3) + 8 * (i >> 2), col = proj * 128 + (wave & 3) * 32 + (lane & 31);
      ot[r * 256 + col] = acc[rb][i];
    }
    __syncthreads();
    for (int r = wave; r < 32 && rb * 32 + r < nrows; r += kWavesG) {
      float g0 = ot[r * 256 + lane], g1 = ot[r * 256 + 64 + lane];
      float u0 = ot[r * 256 + 128 + lane], u1 = ot[r * 256 + 192 + lane];
      fwht2(g0, g1, lane, a.had_inter, a.sc_inter);
      fwht2(u0, u1, lane, a.had_inter, a.sc_inter);
      g0 = g0 * sg0;
      u0 = u0 * su0;
      g1 = g1 * sg1;
      u1 = u1 * su1;
      // SiLU with the hardware exp2 and reciprocal (~1 ulp each; the layer's tolerance is 1e-2), or (EX) as the
      // one-row step computes it
      float h0, h1;
      if constexpr (EX) {
        h0 = g0 / (1.f + expf(-g0)) * u0 * sd0;
        h1 = g1 / (1.f + expf(-g1)) * u1 * sd1;
      } else {
        h0 = g0 * __builtin_amdgcn_rcpf(1.f + __expf(-g0)) * u0 * sd0;
        h1 = g1 * __builtin_amdgcn_rcpf(1.f + __expf(-g1)) * u1 * sd1;
      }
      fwht2(h0, h1, lane, a.had_inter, a.sc_inter);
      uint16_t *out = hh + (uint64_t)(row0 + rb * 32 + r) * a.inter + ib * 128;
      out[kp(lane)] = f2h(h0);
      out[kp(lane + 64)] = f2h(h1);
    }
  }
    return;
  } else {
  // epilogue per 32-row block, with the tiles transposed (wave w: projection w / 4, chunk q = w % 4 of block ib):
  //  1. every wave: H_32 on its tile (element j = 8 (i / 4) + 4 h + i % 4 at lane (n, h) value i), tile to LDS;
  //  2. waves 0..3 (chunk q): H_4 over the gate tiles and over the up tiles gives g and u of columns 32 q + j; then
  //     h = silu(g svh_g / sqrt(128)) u svh_u / sqrt(128) suh_d, already in the layout of a tile, and H_32 on it
  //     with the rows in kp order (lane (n, h) value i = kp position 16 h + i of the chunk), to LDS;
  //  3. wave w takes rows 4 w .. 4 w + 3 whole: lane l combines kp positions 2 l, 2 l + 1 with H_4, / sqrt(128), and
  //     each row leaves as one 256-byte store.
  const int q = wave & 3, n = lane & 31, h = lane >> 5;
  f16x8 hA1[2], hA2[2];
  h32_operand(lane, [](uint32_t m) { return m; }, hA1);
  h32_operand(lane, [](uint32_t m) { return kp_inv32(16u * ((m >> 2) & 1u) + 4u * (m >> 3) + (m & 3u)); }, hA2);
  // scales of this lane's columns in step 2: 32 q + 8 g + 4 h + r (natural order inside block ib), read per block
  const int c0 = ib * 128 + 32 * q + 4 * h;
  const uint16_t *pg = (const uint16_t *)(blk + sv_of(a, e, 0)) + c0, *pu = (const uint16_t *)(blk + sv_of(a, e, 1)) + c0;
  const uint16_t *pd = (const uint16_t *)(blk + su_of(a, e, 2)) + c0;
  const float sc = a.sc_inter;
  // LDS: 8 step-1 tiles then 4 step-2 tiles of 32 rows x 32 elements, row pitch 36 floats
  float *x1 = (float *)lds, *x2 = x1 + 8 * 32 * 36;
  const int nrb = (nrows + 31) / 32;
#pragma unroll
  for (int rb = 0; rb < NRB; rb++) {
    if (rb >= nrb) break;
    const f32x16 T = h32_tile(acc[rb], hA1, lane);
    __syncthreads();  // the ring (first block) or the previous block's tiles are no longer read
#pragma unroll
    for (int g = 0; g < 4; g++)
      *(float4 *)(x1 + (wave * 32 + n) * 36 + 8 * g + 4 * h) = make_float4(T[4 * g], T[4 * g + 1], T[4 * g + 2], T[4 * g + 3]);
    __syncthreads();
    if (wave < 4) {
      f32x16 hv;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const f16x4 sgv = *(const f16x4 *)(pg + 8 * g), suv = *(const f16x4 *)(pu + 8 * g), sdv = *(const f16x4 *)(pd + 8 * g);
        float4 gs = {0.f, 0.f, 0.f, 0.f}, us = gs;
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
          const float sgn = (__builtin_popcount(q & qq) & 1) ? -1.f : 1.f;
          const float4 tg = *(const float4 *)(x1 + (qq * 32 + n) * 36 + 8 * g + 4 * h);
          const float4 tu = *(const float4 *)(x1 + ((4 + qq) * 32 + n) * 36 + 8 * g + 4 * h);
          gs.x = __builtin_fmaf(sgn, tg.x, gs.x);
          gs.y = __builtin_fmaf(sgn, tg.y, gs.y);
          gs.z = __builtin_fmaf(sgn, tg.z, gs.z);
          gs.w = __builtin_fmaf(sgn, tg.w, gs.w);
          us.x = __builtin_fmaf(sgn, tu.x, us.x);
          us.y = __builtin_fmaf(sgn, tu.y, us.y);
          us.z = __builtin_fmaf(sgn, tu.z, us.z);
          us.w = __builtin_fmaf(sgn, tu.w, us.w);
        }
        const float gv[4] = {gs.x, gs.y, gs.z, gs.w}, uv[4] = {us.x, us.y, us.z, us.w};
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float gg = gv[r] * sc * (float)sgv[r], uu = uv[r] * sc * (float)suv[r];
          // SiLU with the hardware exp2 and reciprocal (~1 ulp each; the layer's tolerance is 1e-2)
          hv[4 * g + r] = gg * __builtin_amdgcn_rcpf(1.f + __expf(-gg)) * uu * (float)sdv[r];
        }
      }
      const f32x16 T2 = h32_tile(hv, hA2, lane);
#pragma unroll
      for (int g = 0; g < 4; g++)
        *(float4 *)(x2 + (q * 32 + n) * 36 + 16 * h + 4 * g) = make_float4(T2[4 * g], T2[4 * g + 1], T2[4 * g + 2], T2[4 * g + 3]);
    }
    __syncthreads();
    const int oq = lane >> 4, op = 2 * (lane & 15);  // this lane's kp positions 32 oq + op, + 1
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const int nr = wave * 4 + rr, r = rb * 32 + nr;
      if (r >= nrows) break;
      float o0 = 0.f, o1 = 0.f;
#pragma unroll
      for (int qq = 0; qq < 4; qq++) {
        const float sgn = (__builtin_popcount(oq & qq) & 1) ? -1.f : 1.f;
        const float2 t = *(const float2 *)(x2 + (qq * 32 + nr) * 36 + op);
        o0 = __builtin_fmaf(sgn, t.x, o0);
        o1 = __builtin_fmaf(sgn, t.y, o1);
      }
      *(uint32_t *)(hh + (uint64_t)(row0 + r) * a.inter + ib * 128 + 2 * lane) =
          __builtin_bit_cast(uint32_t, f16x2{(_Float16)(o0 * sc), (_Float16)(o1 * sc)});
    }
  }
  }
}

// down: chunk ch, 256 columns of hid (output blocks 2 ob2, 2 ob2 + 1); wave w: pair 8 ob2 + w. Output per
// (token, slot): H over each 128-column block, svh_d, the slot's route weight.
template <int K, int KS, bool TR, int NR, bool EX = false>
__global__ __launch_bounds__(512, NR == kChunkRows || EX ? 4 : 6) void bat_down(MoeArgs a, const uint32_t *bk, const uint32_t *chunks,
                                                   const uint32_t *rows, const uint16_t *hh, float *dnw) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nob = a.hid / 256;
  int item;
  if (!xcd_item((int)bk[3 * (a.ne + 1)] * nob, item)) return;
  const int ch = item / nob, ob2 = item % nob;
  const int e = (int)chunks[3 * ch], row0 = (int)chunks[3 * ch + 1], nrows = (int)chunks[3 * ch + 2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint8_t *blk = expert_block(a, e);
  // each row's slot (token, k) and route weight, gathered once into LDS (the slot ids requested before the GEMM)
  __shared__ uint32_t m_dst[kChunkRows];
  __shared__ float m_w[kChunkRows];
  const int mt = threadIdx.x;
  const uint32_t sl = mt < nrows ? rows[row0 + mt] : 0u;
  static_assert(!TR || NR == kChunkRows, "transposed products at 128-row chunks");
  constexpr int NRB = NR / 32;
  f32x16 acc[NRB];
  const uint16_t *A = hh + (uint64_t)row0 * a.inter;
  if (e >= a.ne)
    chunk_gemm<KS, 1, TR, NR, EX ? kFoldAll : 0>(A, a.inter, 0, 0, nrows, blk + tr_of(a, e, 2), a.inter / 16,
                                                 ob2 * 8 + wave, lds, acc, nullptr, 0, a.inter / 16);
  else
    chunk_gemm<K, 1, TR, NR, EX ? kFoldAll : 0>(A, a.inter, 0, 0, nrows, blk + tr_of(a, e, 2), a.inter / 16,
                                                ob2 * 8 + wave, lds, acc, nullptr, 0, a.inter / 16);
  if (mt < nrows) {
    const int tok = sl / a.nslot, k = sl % a.nslot;
    m_dst[mt] = sl;
    m_w[mt] = k >= a.topk ? a.sgv[tok] : __uint_as_float(a.route[(uint64_t)tok * 2 * a.topk + a.topk + k]);
  }
  if constexpr (!TR) {
  float *ot = (float *)lds;  // [32][256]
  const uint16_t *sv = (const uint16_t *)(blk + sv_of(a, e, 2)) + ob2 * 256;
  float s[2][2];
#pragma unroll
  for (int bb = 0; bb < 2; bb++) {
    s[bb][0] = h2f(sv[bb * 128 + lane]);
    s[bb][1] = h2f(sv[bb * 128 + lane + 64]);
  }
  const int nrb = (nrows + 31) / 32;
#pragma unroll
  for (int rb = 0; rb < NRB; rb++) {
    if (rb >= nrb) break;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int r = 4 * (lane >> 5) + (i & 3) + 8 * (i >> 2), col = wave * 32 + (lane & 31);
      ot[r * 256 + col] = acc[rb][i];
    }
    __syncthreads();
    for (int r = wave; r < 32 && rb * 32 + r < nrows; r += kWavesG) {
      const float w = m_w[rb * 32 + r];
      float *out = dnw + (uint64_t)m_dst[rb * 32 + r] * a.hid + ob2 * 256;  // slot sl = token * nslot + k
#pragma unroll
      for (int bb = 0; bb < 2; bb++) {
        float v0 = ot[r * 256 + bb * 128 + lane], v1 = ot[r * 256 + bb * 128 + 64 + lane];
        fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
        out[bb * 128 + lane] = v0 * s[bb][0] * w;
        out[bb * 128 + lane + 64] = v1 * s[bb][1] * w;
      }
    }
  }
  } else {
  // epilogue: wave w holds columns 32 w .. of this 256 (block bb = w / 4, chunk q = w % 4) for every row, transposed.
  // Per 32-row block: H_32 on the wave's tile (output element j = 16 h + i of the chunk at lane (n, h)), the tiles to
  // LDS; then wave w takes rows 4 w .. 4 w + 3 whole: lane l combines columns 4 l .. 4 l + 3 with H_4 across the four
  // chunks of its block, applies 1/sqrt(128), svh_d and the slot's route weight, and the row leaves as one 1 KB store.
  f16x8 hA[2];
  h32_operand(lane, [](uint32_t m) { return 16u * ((m >> 2) & 1u) + 4u * (m >> 3) + (m & 3u); }, hA);
  const int cb = lane >> 5, cq = (lane >> 3) & 3, cj = 4 * (lane & 7);  // this lane's columns: block, chunk, element
  float sv[4];
  {
    const uint16_t *svp = (const uint16_t *)(blk + sv_of(a, e, 2)) + ob2 * 256 + 4 * lane;
#pragma unroll
    for (int t = 0; t < 4; t++) sv[t] = h2f(svp[t]) * a.sc_hid;
  }
  // 8 tiles of 32 rows x 32 columns: tile w, row n, element j at (w 32 + n) 36 + j floats (the pad spreads the
  // rows of one write over the banks)
  float *xt = (float *)lds;
  const int nrb = (nrows + 31) / 32;
#pragma unroll
  for (int rb = 0; rb < NRB; rb++) {
    if (rb >= nrb) break;
    const f32x16 T = h32_tile(acc[rb], hA, lane);
    __syncthreads();  // the ring (first block) or the previous block's rows are no longer read
    {
      float *tp = xt + (wave * 32 + (lane & 31)) * 36 + 16 * (lane >> 5);
#pragma unroll
      for (int g = 0; g < 4; g++) *(float4 *)(tp + 4 * g) = make_float4(T[4 * g], T[4 * g + 1], T[4 * g + 2], T[4 * g + 3]);
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const int n = wave * 4 + rr, r = rb * 32 + n;
      if (r >= nrows) break;
      float4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int qq = 0; qq < 4; qq++) {
        const float4 t = *(const float4 *)(xt + ((cb * 4 + qq) * 32 + n) * 36 + cj);
        const float sg = (__builtin_popcount(cq & qq) & 1) ? -1.f : 1.f;
        o.x = __builtin_fmaf(sg, t.x, o.x);
        o.y = __builtin_fmaf(sg, t.y, o.y);
        o.z = __builtin_fmaf(sg, t.z, o.z);
        o.w = __builtin_fmaf(sg, t.w, o.w);
      }
      const float w = m_w[r];
      *(float4 *)(dnw + (uint64_t)m_dst[r] * a.hid + ob2 * 256 + 4 * lane) =  // slot = token nslot + k
          make_float4(o.x * sv[0] * w, o.y * sv[1] * w, o.z * sv[2] * w, o.w * sv[3] * w);
    }
  }
  }
}

// y[r] = sum over the row's slots in slot order (routed k = 0..topk-1, then the shared expert)
__global__ __launch_bounds__(256) void bat_combine(MoeArgs a, const float *__restrict__ dnw) {
  const int r = blockIdx.x, i = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (i >= a.hid) return;
  float4 y = {0.f, 0.f, 0.f, 0.f}, sh = {0.f, 0.f, 0.f, 0.f};  // routed sum in slot order; the shared slot
  const float *p = dnw + (uint64_t)r * a.nslot * a.hid + i;
  constexpr int B = 6;  // slots requested together; summed in slot order
  for (int k0 = 0; k0 < a.nslot; k0 += B) {
    f32x4 v[B];
#pragma unroll
    for (int j = 0; j < B; j++)
      if (k0 + j < a.nslot) v[j] = __builtin_nontemporal_load((const f32x4 *)(p + (uint64_t)(k0 + j) * a.hid));
#pragma unroll
    for (int j = 0; j < B; j++)
      if (k0 + j < a.topk) {
        y.x += v[j][0];
        y.y += v[j][1];
        y.z += v[j][2];
        y.w += v[j][3];
      } else if (k0 + j < a.nslot) {
        sh = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
      }
  }
  if (a.q8) {  // the 8-bit shared expert: its gate times its output
    const float g = a.sgv[r];
    const float4 o = *(const float4 *)(a.q8o + (uint64_t)r * a.hid + i);
    sh = make_float4(g * o.x, g * o.y, g * o.z, g * o.w);
  }
  *(float4 *)(a.y + (uint64_t)r * a.hid + i) =
      make_float4(moe_finish(a, r, i, y.x, sh.x), moe_finish(a, r, i + 1, y.y, sh.y), moe_finish(a, r, i + 2, y.z, sh.z),
                  moe_finish(a, r, i + 3, y.w, sh.w));
}


// ---------------------------------------------------------------------------------------------------- few rows
// Speculative verify (at most 32 rows, so an expert's rows are one chunk) with the k order of the one-row step and of
// the trunk linear, spread so that every SIMD decodes:
//   bat_gu_grp  workgroup (chunk, 128-column block cb of inter, projection, pair q of the block), looping over the k
//               groups of 512 (the next group's requests in flight while one decodes); wave c takes k chunk c of each
//               group (8 k tiles, one MFMA chain from zero); the chunk sums are folded left in LDS, the groups left in
//               registers, and the pair's sums stored (device-coherent). The last of the block's 8 workgroups to
//               arrive (a counter per block, reset by it) writes the block's rows of hh (H(g) svh_g, SiLU, H(u)
//               svh_u, suh_d, H, fp16, kp order);
//   bat_dn_blk  workgroup (chunk, 128-column output block c), wave q one pair: every k chunk of inter (chains from zero,
//               folded left), then H, svh_d and the slot's route weight per row (no hand-off between workgroups).
// The partials and counters live in one pool per layer shape, shared by the layers (one stream; every counter is back
// at zero when a launch ends).
// the workgroup's arrival at a counter after its stores completed; returns the count before it
__device__ uint32_t block_signal8(uint32_t *p, int *flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) *flag = (int)atomicAdd(p, 1u);
  __syncthreads();
  const uint32_t old = (uint32_t)*flag;
  __syncthreads();
  return old;
}
constexpr int kVChunk = 8;  // k tiles of a k chunk
constexpr int kFewChunkRows = 4;  // rows of a chunk on the few-row path (its LDS tier)
constexpr int kFewMaxGroups = 8;  // k groups of 512 (hidden size up to 4096)
template <int KD, int RT>
__device__ __forceinline__ f32x16 v_chain(const uint8_t *tl, const _Float16 *xs, int pitch, int nkt, int nrows) {
  const int lane = threadIdx.x & 63;
  const _Float16 *xa = xs + min(lane & 31, nrows - 1) * pitch + 8 * (lane >> 5);
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  acc = mfma_chunk<KD, kVChunk>(tl, xa, nkt, acc);
  return acc;
}
// bytes staged per wave and buffer: 8 k tile pairs at the larger K, then RT rows of the chunk (128 halves each); two
// buffers per wave (the next k group's requests in flight while this one decodes)
template <int KM, int RT>
constexpr uint32_t v_gu_wave() { return kVChunk * 64 * KM + RT * 256; }
// (the chunk sums of every group stay in registers through the k loop, then go to the wave's own buffers)
template <int KM, int RT>
constexpr uint32_t v_gu_lds(int G) {
  static_assert(2 * v_gu_wave<KM, RT>() >= kFewMaxGroups * RT * 32 * 4, "a wave's chunk sums fit its buffers");
  return 8 * v_gu_wave<KM, RT>() + 0 * G;
}

template <int K, int KS, int RT>
__global__ __launch_bounds__(256) void bat_gu_grp(MoeArgs a, const uint32_t *bk, const uint32_t *chunks,
                                                  const uint16_t *xh, uint16_t *hh, uint64_t *part, uint32_t *epochs) {
  constexpr int KM = K > KS ? K : KS;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int NP = a.inter / 32, NBI = a.inter / 128, IT = a.hid / 16, G = (IT + 31) / 32;
  const int upc = NBI * 8, ch = (int)blockIdx.x / upc, rem = (int)blockIdx.x % upc;
  if (ch >= (int)bk[3 * (a.ne + 1)]) return;
  const int q = rem & 3, proj = (rem >> 2) & 1, cb = rem >> 3, p = cb * 4 + q;
  const int e = (int)chunks[3 * ch], row0 = (int)chunks[3 * ch + 1], nrows = (int)chunks[3 * ch + 2];
  const int lane = threadIdx.x & 63, c = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool sh = e >= a.ne;
  const int KE = sh ? KS : K;
  // after the k loop: wave c's chunk sums [k group][RT][32] at the start of its own two buffers
  auto csum_at = [&](int cw) { return (float *)(lds + 2 * cw * v_gu_wave<KM, RT>()); };
  float cs[kFewMaxGroups][4];  // this wave's chunk sum of each group: rows 0..3 of its 32 columns (lanes 0-31)
  __shared__ int flag;
  uint32_t *ctr = epochs + ((uint64_t)ch * NBI + cb) * kSyncStride;
  float *pf = (float *)part;
  const uint8_t *blk = expert_block(a, e);
  const uint8_t *tr = blk + tr_of(a, e, proj) + (uint64_t)p * IT * 64 * KE;
  // requests of k group g into buffer g & 1: this wave's chunk of tiles, then its rows; returns their count
  auto stage = [&](int g) {
    const int kt0 = g * 32 + c * kVChunk, nkt = max(0, min(kVChunk, IT - kt0));
    uint8_t *tl = lds + (2 * c + (g & 1)) * v_gu_wave<KM, RT>();
    _Float16 *xs = (_Float16 *)(tl + kVChunk * 64 * KM);
    int n = 0;
    if (nkt > 0) {
      const uint32_t bytes = (uint32_t)nkt * 64 * KE;
      for (uint32_t o = 0; o < bytes; o += 1024, n++)
        if (o + (uint32_t)lane * 16 < bytes) dma16(tr + (uint64_t)kt0 * 64 * KE + o + lane * 16, tl + o);
      for (int r = 0; r < nrows; r += 4, n++) {  // rows r .. r + 3: 16 lanes of 16 bytes each
        const int rr = r + (lane >> 4), qq = lane & 15;
        if (rr < nrows && qq * 16 < nkt * 32)
          dma16(xh + ((uint64_t)(row0 + rr) * 2 + proj) * a.hid + kt0 * 16 + qq * 8, xs + r * 128);
      }
    }
    return n;
  };
  stage(0);
  // each wave on its own through the k groups (no barrier until every chunk sum is in LDS)
  for (int g = 0; g < G; g++) {
    const int nnext = g + 1 < G ? stage(g + 1) : 0;
    wait_vm15(nnext);  // group g's requests are in (the next group's may not be)
    const int kt0 = g * 32 + c * kVChunk, nkt = max(0, min(kVChunk, IT - kt0));
    const uint8_t *tl = lds + (2 * c + (g & 1)) * v_gu_wave<KM, RT>();
    const _Float16 *xs = (const _Float16 *)(tl + kVChunk * 64 * KM);
    f32x16 acc;
    if (sh && KS != K)
      acc = v_chain<KS, RT>(tl, xs, 128, nkt, nrows);
    else
      acc = v_chain<K, RT>(tl, xs, 128, nkt, nrows);
    static_assert(RT <= 4, "rows 0..3 of the product: values 0..3 of lanes 0-31");
#pragma unroll
    for (int gg = 0; gg < kFewMaxGroups; gg++)  // a compile-time register index
      if (gg == g)
#pragma unroll
        for (int i = 0; i < 4; i++) cs[gg][i] = acc[i];
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this group's buffer reads are done before it is refilled
  }
  __builtin_amdgcn_s_waitcnt(0);  // every request of this wave has landed: its buffers are free
  {
    float *mine = csum_at(c);
#pragma unroll
    for (int gg = 0; gg < kFewMaxGroups; gg++)
      if (gg < G && lane < 32)
#pragma unroll
        for (int r = 0; r < RT; r++)
          if (r < nrows) mine[(gg * RT + r) * 32 + lane] = cs[gg][r];
  }
  __syncthreads();
  // per (row, column): the chunks of each group folded left, the groups folded left
  const int ent = threadIdx.x;
  float tot = 0.f;
  if (ent < nrows * 32)
    for (int g = 0; g < G; g++) {
      const int nc = (min(32, IT - g * 32) + kVChunk - 1) / kVChunk;
      float v = csum_at(0)[g * RT * 32 + ent];
      for (int cc = 1; cc < nc; cc++) v = v + csum_at(cc)[g * RT * 32 + ent];
      tot = g == 0 ? v : tot + v;
    }
  if (ent < nrows * 32)
    st_cg(pf + ((((uint64_t)ch * 2 + proj) * NP + p) * kFewChunkRows + (ent >> 5)) * 32 + (ent & 31), tot);
  // the last of the block's 8 workgroups (2 projections x 4 pairs) finishes it and resets its counter
  if (block_signal8(ctr, &flag) != 7u) return;
  if (threadIdx.x == 0) st_cg(ctr, 0u);
  // the block's finisher: rows r = wave, wave + 4, ..; lane: columns o = lane, lane + 64 of block cb
  const uint16_t *svg = (const uint16_t *)(blk + sv_of(a, e, 0)) + cb * 128;
  const uint16_t *svu = (const uint16_t *)(blk + sv_of(a, e, 1)) + cb * 128;
  const uint16_t *sud = (const uint16_t *)(blk + su_of(a, e, 2)) + cb * 128;
  const int pr0 = cb * 4 + (lane >> 5), n0 = lane & 31;  // column lane: pair pr0; column lane + 64: pair pr0 + 2
  for (int r = c; r < nrows; r += 4) {
    float gs[2], us[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      gs[h] = ld_cg(pf + ((((uint64_t)ch * 2 + 0) * NP + pr0 + 2 * h) * kFewChunkRows + r) * 32 + n0);
      us[h] = ld_cg(pf + ((((uint64_t)ch * 2 + 1) * NP + pr0 + 2 * h) * kFewChunkRows + r) * 32 + n0);
    }
    float g0 = gs[0], g1 = gs[1], u0 = us[0], u1 = us[1];
    fwht2(g0, g1, lane, a.had_inter, a.sc_inter);
    fwht2(u0, u1, lane, a.had_inter, a.sc_inter);
    g0 = g0 * h2f(svg[lane]);
    u0 = u0 * h2f(svu[lane]);
    g1 = g1 * h2f(svg[lane + 64]);
    u1 = u1 * h2f(svu[lane + 64]);
    float h0 = g0 / (1.f + expf(-g0)) * u0 * h2f(sud[lane]);
    float h1 = g1 / (1.f + expf(-g1)) * u1 * h2f(sud[lane + 64]);
    fwht2(h0, h1, lane, a.had_inter, a.sc_inter);
    uint16_t *out = hh + (uint64_t)(row0 + r) * a.inter + cb * 128;
    out[kp((uint32_t)lane)] = f2h(h0);
    out[kp((uint32_t)lane + 64)] = f2h(h1);
  }
}

// LDS: per wave two buffers of one k chunk (8 k tile pairs at the larger K), then the chunk's RT rows of hh (inter
// halves each), then the [RT][128] outputs (about 26 KB at K5, inter 512: six workgroups per CU)
template <int KM, int RT>
__host__ __device__ constexpr uint32_t v_dn_lds(int inter) {
  return 4u * 2u * kVChunk * 64 * KM + (uint32_t)RT * inter * 2 + RT * 128 * 4;
}
template <int K, int KS, int RT>
__global__ __launch_bounds__(256) void bat_dn_blk(MoeArgs a, const uint32_t *bk, const uint32_t *chunks,
                                                  const uint32_t *rows, const uint16_t *hh, float *dnw) {
  constexpr int KM = K > KS ? K : KS;
  constexpr uint32_t kBuf = kVChunk * 64 * KM;  // one k chunk's LDS buffer
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int NBLK = a.hid / 128, ITd = a.inter / 16, ch = (int)blockIdx.x / NBLK, cblk = (int)blockIdx.x % NBLK;
  if (ch >= (int)bk[3 * (a.ne + 1)]) return;
  const int e = (int)chunks[3 * ch], row0 = (int)chunks[3 * ch + 1], nrows = (int)chunks[3 * ch + 2];
  const int lane = threadIdx.x & 63, q = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6), p = cblk * 4 + q;
  const bool sh = e >= a.ne;
  const int KE = sh ? KS : K;
  uint8_t *tl = lds + q * 2 * kBuf;  // this wave's two chunk buffers
  _Float16 *xs = (_Float16 *)(lds + 4 * 2 * kBuf);
  float *ot = (float *)(lds + 4 * 2 * kBuf + RT * a.inter * 2);
  const uint8_t *blk = expert_block(a, e);
  // each row's slot (token, k) and route weight; then the rows of hh (nrows x inter halves, contiguous; 1 KB per
  // request, spread over the 4 waves), then the wave's first two k chunks; each later chunk is requested into the
  // buffer its chunk two before has left, so the next chunk is in flight while one decodes
  const uint32_t sl = lane < nrows ? rows[row0 + lane] : 0u;
  {
    const uint32_t rb = (uint32_t)nrows * a.inter * 2;
    const uint8_t *hs = (const uint8_t *)(hh + (uint64_t)row0 * a.inter);
    for (uint32_t o = (uint32_t)q * 1024; o < rb; o += 4096)
      if (o + (uint32_t)lane * 16 < rb) dma16(hs + o + lane * 16, (uint8_t *)xs + o);
  }
  const uint32_t cbytes = kVChunk * 64 * KE;
  const int cops = (int)((cbytes + 1023) / 1024), NC = ITd / kVChunk;
  const uint8_t *src = blk + tr_of(a, e, 2) + (uint64_t)p * ITd * 64 * KE;
  auto stage = [&](int cc) {
    for (uint32_t o = 0; o < cbytes; o += 1024)
      if (o + (uint32_t)lane * 16 < cbytes) dma16(src + (uint64_t)cc * cbytes + o + lane * 16, tl + (cc & 1) * kBuf + o);
  };
  stage(0);
  if (NC > 1) stage(1);
  wait_vm15(NC > 1 ? 2 * cops : cops);  // this wave's rows of hh are in
  __syncthreads();                      // every wave's
  f32x16 s;
  for (int cc = 0; cc < NC; cc++) {  // the k chunks of inter, folded left
    wait_vm15(cc + 1 < NC ? cops : 0);  // chunk cc's tiles are in (chunk cc + 1's may not be)
    const uint8_t *tb = tl + (cc & 1) * kBuf;
    f32x16 acc = (sh && KS != K) ? v_chain<KS, RT>(tb, xs + cc * kVChunk * 16, a.inter, kVChunk, nrows)
                                 : v_chain<K, RT>(tb, xs + cc * kVChunk * 16, a.inter, kVChunk, nrows);
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] = cc == 0 ? acc[i] : s[i] + acc[i];
    if (cc + 2 < NC) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this buffer's reads are done before it is refilled
      stage(cc + 2);
    }
  }
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int r = 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    if (r < RT && r < nrows) ot[r * 128 + q * 32 + (lane & 31)] = s[i];
  }
  __syncthreads();
  const uint16_t *svd = (const uint16_t *)(blk + sv_of(a, e, 2)) + cblk * 128;
  const float s0 = h2f(svd[lane]), s1 = h2f(svd[lane + 64]);
  for (int r = q; r < nrows; r += 4) {
    const uint32_t slr = (uint32_t)__shfl((int)sl, r, 64);
    const int tok = (int)(slr / a.nslot), k = (int)(slr % a.nslot);
    const float w = k >= a.topk ? a.sgv[tok] : __uint_as_float(a.route[(uint64_t)tok * 2 * a.topk + a.topk + k]);
    float v0 = ot[r * 128 + lane], v1 = ot[r * 128 + 64 + lane];
    fwht2(v0, v1, lane, a.had_hid, a.sc_hid);
    float *out = dnw + (uint64_t)slr * a.hid + cblk * 128;
    out[lane] = v0 * s0 * w;
    out[lane + 64] = v1 * s1 * w;
  }
}

// ---------------------------------------------------------------------------------------------------- host side
namespace {
template <int K, int KS, bool TR, int NR, bool EX = false>
void launch_gemms_as(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t s) {
  // chunk_gemm runs k in steps of 2 tiles: an odd tile count would drop the last tile
  IJ_CHECK(a.hid % 32 == 0 && a.inter % 32 == 0, "grouped GEMM: k tiles must be even (hid %d, inter %d)", a.hid,
           a.inter);
  // the routed (K) and shared (KS) chunks use ring layouts of their own widths: room for the larger of each
  const size_t lg = std::max(GemmIo<K, 2, NR>::LDS, GemmIo<KS, 2, NR>::LDS);
  const size_t ld = std::max(GemmIo<K, 1, NR>::LDS, GemmIo<KS, 1, NR>::LDS);
  hipLaunchKernelGGL((bat_gateup<K, KS, TR, NR, EX>), dim3((b.max_chunks * (a.inter / 128) + 7) & ~7),
                     dim3(64 * kWavesG), lg, s, a, b.bk, b.chunks, b.rows, b.xh, b.hh);
  hipLaunchKernelGGL((bat_down<K, KS, TR, NR, EX>), dim3((b.max_chunks * (a.hid / 256) + 7) & ~7), dim3(64 * kWavesG),
                     ld, s, a, b.bk, b.chunks, b.rows, b.hh, b.dnw);
}
// Chunks of many rows (8 or more per routed expert on average) take the transposed products and the matrix-core
// Hadamard epilogues; chunks of a row or two (speculative verify) the row-major products and lane butterflies, which
// cost less there.
// At most 32 rows (speculative verify) no chunk exceeds 32 rows: the one-row-block form, three workgroups per CU,
// with the one-row step's arithmetic (every row bit-identical to the row run alone).
template <int K, int KS>
void launch_gemms(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t s) {
  if (moe_batch_exact(a))
    launch_gemms_as<K, KS, false, 32, true>(a, b, s);
  else if (a.R <= 32)
    launch_gemms_as<K, KS, false, 32>(a, b, s);
  else if ((int64_t)a.R * a.topk >= 8LL * a.ne)
    launch_gemms_as<K, KS, true, kChunkRows>(a, b, s);
  else
    launch_gemms_as<K, KS, false, kChunkRows>(a, b, s);
}
}  // namespace

template <int K, int KS, int RT>
void launch_few_rt(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t s) {
  constexpr int KM = K > KS ? K : KS;
  const int NBI = a.inter / 128, NBLK = a.hid / 128;
  const size_t lg = v_gu_lds<KM, RT>(a.hid / 512), ld = v_dn_lds<KM, RT>(a.inter);
  hipLaunchKernelGGL((bat_gu_grp<K, KS, RT>), dim3(b.vmax_chunks * NBI * 8), dim3(256), lg, s, a, b.bk, b.chunks,
                     b.xh, b.hh, b.vpart, b.vep);
  hipLaunchKernelGGL((bat_dn_blk<K, KS, RT>), dim3(b.vmax_chunks * NBLK), dim3(256), ld, s, a, b.bk, b.chunks, b.rows,
                     b.hh, b.dnw);
}
template <int K, int KS>
void launch_few(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t s) {
  launch_few_rt<K, KS, kFewChunkRows>(a, b, s);
}
template <int K, int KS, int RT>
static void few_attrs_rt() {
  constexpr int KM = K > KS ? K : KS;
  IJ_HIP(hipFuncSetAttribute((const void *)&bat_gu_grp<K, KS, RT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)v_gu_lds<KM, RT>(kFewMaxGroups)));
  IJ_HIP(hipFuncSetAttribute((const void *)&bat_dn_blk<K, KS, RT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024));
}
template <int K, int KS>
static void few_attrs() {
  few_attrs_rt<K, KS, kFewChunkRows>();
}

// Raises the dynamic LDS limit of every kernel that needs more than the default, once at device set-up: never
// lazily at a first launch, which may happen inside a stream capture.
template <int K, int KS, bool TR, int NR, bool EX = false>
static void gemm_attrs() {
  const size_t lg = std::max(GemmIo<K, 2, NR>::LDS, GemmIo<KS, 2, NR>::LDS);
  const size_t ld = std::max(GemmIo<K, 1, NR>::LDS, GemmIo<KS, 1, NR>::LDS);
  IJ_HIP(hipFuncSetAttribute((const void *)&bat_gateup<K, KS, TR, NR, EX>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lg));
  IJ_HIP(hipFuncSetAttribute((const void *)&bat_down<K, KS, TR, NR, EX>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)ld));
}
template <int K, int KS>
static void gemm_attrs_all() {
  gemm_attrs<K, KS, true, kChunkRows>();
  gemm_attrs<K, KS, false, 32, true>();
  gemm_attrs<K, KS, false, 32>();
  gemm_attrs<K, KS, false, kChunkRows>();
}
void init_batch_attrs() {
  IJ_HIP(hipFuncSetAttribute((const void *)&bat_place_prep, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPrepLds));
  gemm_attrs_all<4, 4>(); gemm_attrs_all<5, 5>(); gemm_attrs_all<6, 6>(); gemm_attrs_all<4, 5>();
  gemm_attrs_all<4, 6>(); gemm_attrs_all<5, 6>(); gemm_attrs_all<5, 4>(); gemm_attrs_all<6, 4>();
  gemm_attrs_all<6, 5>();
  few_attrs<4, 4>(); few_attrs<5, 5>(); few_attrs<6, 6>(); few_attrs<4, 5>(); few_attrs<4, 6>(); few_attrs<5, 6>();
  few_attrs<5, 4>(); few_attrs<6, 4>(); few_attrs<6, 5>();
}

// Few rows: every kernel keeps the one-row step's arithmetic (hidden size a multiple of 512 for its router rows)
bool moe_batch_exact(const MoeArgs &a) { return a.R <= 32 && a.hid % 512 == 0; }
static size_t v_dn_bytes(int inter, int KM) {  // bat_dn_blk's LDS (v_dn_lds at run-time K)
  return 4ull * 2 * kVChunk * 64 * KM + (size_t)kFewChunkRows * inter * 2 + (size_t)kFewChunkRows * 128 * 4;
}
bool moe_batch_few(int R, int hid, int inter, int K, int KS) {
  return R <= 32 && hid % 512 == 0 && hid / 512 <= kFewMaxGroups && v_dn_bytes(inter, std::max(K, KS)) <= 160 * 1024;
}
int moe_batch_few_chunks(int R, int ne, int topk, bool shared) {
  // chunks of at most kFewChunkRows rows: one per touched expert, plus one per further kFewChunkRows rows
  return std::min(ne, R * topk) + (R * topk + kFewChunkRows - 1) / kFewChunkRows +
         (shared ? (R + kFewChunkRows - 1) / kFewChunkRows : 0);
}
size_t moe_batch_few_part(int chunks, int hid, int inter) {
  (void)hid;
  return (size_t)chunks * 2 * (inter / 32) * kFewChunkRows * 32;
}
size_t moe_batch_few_epochs(int chunks, int inter) { return (size_t)chunks * (inter / 128) * kSyncStride; }

bool moe_batch_supported(int K, int KS, int hid, int inter, int ne, int topk) {
  const bool ks = (K >= 4 && K <= 6) && (KS >= 4 && KS <= 6);
  return ks && hid % 256 == 0 && inter % 128 == 0 && hid <= 8192 && inter <= 4096 && ne < 1024 && topk <= 32;
}
int moe_batch_max_chunks(int R, int ne, int topk, bool shared) {
  return (R * topk + kChunkRows - 1) / kChunkRows + ne + (shared ? (R + kChunkRows - 1) / kChunkRows : 0) + 1;
}

void launch_moe_batch(const MoeArgs &a, const MoeBatchBufs &b, hipStream_t s) {
  const int ncol = a.ne + a.has_sgate, S = a.R * a.nslot;
  if (a.R >= 512) {
    const int ng = (a.R + kRtRows - 1) / kRtRows;
    hipLaunchKernelGGL(bat_router_rows, dim3((ng * ((ncol + 127) / 128) + 7) & ~7), dim3(512), 0, s, a, ng);
  } else if (moe_batch_exact(a)) {
    IJ_CHECK(a.hid / 512 <= kRouterExactChunks, "few-row router: hidden %d above %d", a.hid, 512 * kRouterExactChunks);
    const int nc = a.hid / 512;
    if (nc <= 4)
      hipLaunchKernelGGL(bat_router_exact<4>, dim3((ncol + 3) / 4, a.R), dim3(256), 0, s, a);
    else if (nc <= 8)
      hipLaunchKernelGGL(bat_router_exact<8>, dim3((ncol + 3) / 4, a.R), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(bat_router_exact<kRouterExactChunks>, dim3((ncol + 3) / 4, a.R), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(bat_router<1>, dim3((a.R + 31) / 32, (ncol + 31) / 32), dim3(64 * kRouterWaves), 0, s, a);
  }
  const int KS = a.nslot > a.topk ? a.slay.K : a.lay.K;
  const bool few = moe_batch_exact(a) && b.vpart && moe_batch_few(a.R, a.hid, a.inter, a.lay.K, KS);
  if (few) {  // route, chunks and placement in one workgroup
    IJ_CHECK(a.ne < 1024 && a.R * a.nslot <= 1024 * 32 && a.R * a.topk <= 1024, "few-row MoE: %d experts, %d slots",
             a.ne, a.R * a.topk);
    hipLaunchKernelGGL(bat_route_place, dim3((a.R + kRouteRows - 1) / kRouteRows), dim3(1024), 0, s, a, b.bk, b.chunks,
                       b.max_chunks,
                       (uint32_t)kFewChunkRows, b.rows);
  } else {
    hipLaunchKernelGGL(bat_route, dim3((a.R + 3) / 4), dim3(256), 0, s, a);
    const int self_count = a.R * a.topk < 4096;  // few slots: counted inside bat_scan
    if (!self_count) hipLaunchKernelGGL(bat_hist, dim3(kHistGroups), dim3(256), 0, s, a, b.bk);
    hipLaunchKernelGGL(bat_scan, dim3(1), dim3(1024), 0, s, a, b.bk, b.chunks, b.max_chunks, self_count,
                       (uint32_t)kChunkRows);
  }
  IJ_CHECK(a.had_hid == 128, "batched MoE: hidden size %d needs a 128-wide Hadamard", a.hid);
  if (few) {
    hipLaunchKernelGGL(bat_prep_rows, dim3((S * 2 * (a.hid / 128) + 3) / 4), dim3(256), 0, s, a, b.rows, b.xh);
  } else if (moe_batch_exact(a)) {
    hipLaunchKernelGGL(bat_place_rows, dim3((S + 255) / 256), dim3(256), 0, s, a, b.bk, b.rows);
    hipLaunchKernelGGL(bat_prep_rows, dim3((S * 2 * (a.hid / 128) + 3) / 4), dim3(256), 0, s, a, b.rows, b.xh);
  } else
    hipLaunchKernelGGL(bat_place_prep, dim3((S + kPrepWaves - 1) / kPrepWaves), dim3(64 * kPrepWaves), kPrepLds, s,
                       a, b.bk, b.rows, b.xh);
  if (few) {
    IJ_CHECK(b.vmax_chunks >= moe_batch_few_chunks(a.R, a.ne, a.topk, a.nslot > a.topk), "few-row MoE: scratch");
    bool ok = false;
#define IJ_FEW(k, ks)                                  \
  if (!ok && a.lay.K == k && KS == ks) {               \
    launch_few<k, ks>(a, b, s);                        \
    ok = true;                                         \
  }
    IJ_FEW(4, 4) IJ_FEW(5, 5) IJ_FEW(6, 6) IJ_FEW(4, 5) IJ_FEW(4, 6) IJ_FEW(5, 6) IJ_FEW(5, 4) IJ_FEW(6, 4) IJ_FEW(6, 5)
#undef IJ_FEW
    IJ_CHECK(ok, "few-row MoE: K%d / shared K%d not instantiated", a.lay.K, KS);
    hipLaunchKernelGGL(bat_combine, dim3(a.R, (a.hid + 1023) / 1024), dim3(256), 0, s, a, b.dnw);
    return;
  }
  bool done = false;
#define IJ_BAT(k, ks)                        \
  if (!done && a.lay.K == k && KS == ks) {   \
    launch_gemms<k, ks>(a, b, s);            \
    done = true;                             \
  }
  IJ_BAT(4, 4) IJ_BAT(5, 5) IJ_BAT(6, 6) IJ_BAT(4, 5) IJ_BAT(4, 6) IJ_BAT(5, 6) IJ_BAT(5, 4) IJ_BAT(6, 4) IJ_BAT(6, 5)
#undef IJ_BAT
  IJ_CHECK(done, "batched MoE: K%d / shared K%d not instantiated", a.lay.K, KS);
  hipLaunchKernelGGL(bat_combine, dim3(a.R, (a.hid + 1023) / 1024), dim3(256), 0, s, a, b.dnw);
}

}  // namespace ijah
