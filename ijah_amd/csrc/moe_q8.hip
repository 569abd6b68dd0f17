// The MoE layer's shared expert in the reference's 8-bit affine form, for the staged and batched paths (the one-row
// fused step computes the same rows inside its launch, moe_fused.hip): reference kernels/fn_moe.metal:40-46 (shared
// gate / up rows in the router dispatch) and :264-290 (shared down rows on rr(silu(g) u)), with the row dot of
// kernels/ne_common.h:58-88. Each row's arithmetic is q8_chunk / q8_wave_sum (moe_device.h), the same in every path.
//
//   moe_q8_gu  wave per gate / up row (its weights held in registers), looping over a block of kQ8Rows input rows:
//              q8gu[t][row] = rr(row . x_t) (gate rows 0 .. inter-1, up rows inter .. 2 inter-1)
//   moe_q8_dn  workgroup of 4 waves: h[t] = rr(silu(g_t) u_t) for its block of input rows into LDS, then 4 down rows
//              per wave: q8o[t][row] = rr(row . h_t)
#include <hip/hip_runtime.h>

#include <algorithm>

#include "exl3_device.h"
#include "kernels.h"
#include "moe_device.h"

namespace ijah {

namespace {

constexpr int kQ8Rows = 8;          // input rows per workgroup (x / h reads per loaded weight row)
constexpr int kQ8MaxInter = 1024;   // h of kQ8Rows rows in LDS
constexpr int kQ8DnRows = 4;        // down rows per wave
constexpr int kQ8FewRows = 32;      // above: the matrix-core form

template <int NCH>
__global__ __launch_bounds__(256) void moe_q8_gu(MoeArgs a) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= 2 * a.inter) return;
  const Q8Off o = q8_offsets(a.hid, a.inter);
  const int proj = row >= a.inter ? 1 : 0, rr = row - proj * a.inter;
  Q8Row<NCH> w;
  q8_load<NCH>(a.q8 + o.w[proj] + (uint64_t)rr * a.hid,
               (const uint32_t *)(a.q8 + o.sb[proj]) + (uint64_t)rr * (a.hid / kQ8Group), a.hid, w);
  const int t1 = min(a.R, (int)(blockIdx.y + 1) * kQ8Rows);
  for (int t = blockIdx.y * kQ8Rows; t < t1; t++) {
    const float v = q8_dot<NCH>(w, a.x + (uint64_t)t * a.hid, a.hid);
    if (lane == 0) a.q8gu[(uint64_t)t * 2 * a.inter + row] = moe_rr(v, a.refr);
  }
}

template <int NCH>
__global__ __launch_bounds__(256) void moe_q8_dn(MoeArgs a) {
  __shared__ __attribute__((aligned(16))) float h[kQ8Rows * kQ8MaxInter];
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  const int t0 = blockIdx.y * kQ8Rows, nt = min(a.R - t0, kQ8Rows);
  for (int i = threadIdx.x; i < nt * a.inter; i += blockDim.x) {
    const int t = i / a.inter, j = i - t * a.inter;
    const float *gu = a.q8gu + (uint64_t)(t0 + t) * 2 * a.inter;
    h[t * a.inter + j] = q8_act(gu[j], gu[a.inter + j], a.refr);
  }
  __syncthreads();
  const Q8Off o = q8_offsets(a.hid, a.inter);
  for (int k = 0; k < kQ8DnRows; k++) {
    const int row = (blockIdx.x * 4 + wave) * kQ8DnRows + k;
    if (row >= a.hid) break;
    Q8Row<NCH> w;
    q8_load<NCH>(a.q8 + o.w[2] + (uint64_t)row * a.inter,
                 (const uint32_t *)(a.q8 + o.sb[2]) + (uint64_t)row * (a.inter / kQ8Group), a.inter, w);
    for (int t = 0; t < nt; t++) {
      const float v = q8_dot<NCH>(w, h + t * a.inter, a.inter);
      if (lane == 0) a.q8o[(uint64_t)(t0 + t) * a.hid + row] = moe_rr(v, a.refr);
    }
  }
}

// ---------------------------------------------------------------------------------------------------- many rows
// R > 32 (prefill): the same rows on the matrix cores. The weight bytes are held a second time as bf16 (exact: a
// byte has at most 8 significant bits), x is split into bf16 hi + lo (16 significant bits reach the products), and
// v_mfma_f32_32x32x16_bf16 sums each group of 128 inputs from zero; per group acc = fmaf(s, P, acc) and
// acc = fmaf(b, sum of x over the group, acc). Rows agree with the one-row arithmetic within f32 rounding (the
// many-row path's bar).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
constexpr int kMmRows = 128, kMmCols = 64;  // workgroup tile: 4 waves x 32 rows, 2 blocks of 32 outputs each

// y[t][o] = rr(row o . x[t]) for t < R, o < nout (a multiple of 64): x f32 rows ldx apart, weights bf16 [nout][in],
// group words [nout][in / 128]
__global__ __launch_bounds__(256) void moe_q8_mm(const float *x, int ldx, int R, const uint16_t *wbf,
                                                 const uint32_t *sb, int in, float *y, int ldy, int refr) {
  __shared__ float sxl[4][32];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, m = lane & 31, h = lane >> 5;
  const int t0 = blockIdx.x * kMmRows + 32 * w, o0 = blockIdx.y * kMmCols;
  const float *xp = x + (uint64_t)min(t0 + m, R - 1) * ldx + 8 * h;
  const uint16_t *wp0 = wbf + (uint64_t)(o0 + m) * in + 8 * h, *wp1 = wp0 + (uint64_t)32 * in;
  const int ng = in / kQ8Group;
  f32x16 tot[2], P[2];
#pragma unroll
  for (int i = 0; i < 16; i++) tot[0][i] = tot[1][i] = 0.f;
  for (int g = 0; g < ng; g++) {
#pragma unroll
    for (int i = 0; i < 16; i++) P[0][i] = P[1][i] = 0.f;
    float sx = 0.f;
#pragma unroll
    for (int st = 0; st < 8; st++) {
      const int k = g * kQ8Group + 16 * st;
      const float4 x0 = *(const float4 *)(xp + k), x1 = *(const float4 *)(xp + k + 4);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        hi[e] = (__bf16)xs[e];
        lo[e] = (__bf16)(xs[e] - (float)hi[e]);
        sx = sx + xs[e];
      }
      const bf16x8 w0 = *(const bf16x8 *)(wp0 + k), w1 = *(const bf16x8 *)(wp1 + k);
      P[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, w0, P[0], 0, 0, 0);
      P[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, w0, P[0], 0, 0, 0);
      P[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, w1, P[1], 0, 0, 0);
      P[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, w1, P[1], 0, 0, 0);
    }
    sx += __shfl_xor(sx, 32, 64);  // the row's sum over the group (lanes m and m + 32 hold its two halves)
    if (h == 0) sxl[w][m] = sx;
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int ob = 0; ob < 2; ob++) {
      const uint32_t word = sb[(uint64_t)(o0 + 32 * ob + m) * ng + g];
      const float sc = bf16_f32(word & 0xFFFFu), bi = bf16_f32(word >> 16);
#pragma unroll
      for (int i = 0; i < 16; i++) {  // lane holds column o0 + 32 ob + m, rows 8 (i / 4) + 4 h + i % 4
        tot[ob][i] = __builtin_fmaf(sc, P[ob][i], tot[ob][i]);
        tot[ob][i] = __builtin_fmaf(bi, sxl[w][8 * (i / 4) + 4 * h + i % 4], tot[ob][i]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
#pragma unroll
  for (int ob = 0; ob < 2; ob++)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int t = t0 + 8 * (i / 4) + 4 * h + i % 4;
      if (t < R) y[(uint64_t)t * ldy + o0 + 32 * ob + m] = moe_rr(tot[ob][i], refr);
    }
}
// h = rr(silu(g) u) in place of g: q8gu[t][j] for j < inter (the down GEMM's input rows, 2 inter apart)
__global__ __launch_bounds__(256) void moe_q8_act(float *gu, int R, int inter, int refr) {
  const uint64_t i = blockIdx.x * 256ull + threadIdx.x;
  if (i >= (uint64_t)R * inter) return;
  const uint64_t t = i / inter, j = i % inter;
  float *row = gu + t * 2 * inter;
  row[j] = q8_act(row[j], row[inter + j], refr);
}
// the weight bytes as bf16 values (exact), once at set-up
__global__ void q8_to_bf16(const uint8_t *w, uint16_t *o, uint64_t n) {
  for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256)
    o[i] = (uint16_t)(__float_as_uint((float)w[i]) >> 16);
}

template <int NCH>
void launch_gu(const MoeArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(moe_q8_gu<NCH>, dim3((2 * a.inter + 3) / 4, (a.R + kQ8Rows - 1) / kQ8Rows), dim3(256), 0, s, a);
}
template <int NCH>
void launch_dn(const MoeArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(moe_q8_dn<NCH>, dim3((a.hid + 4 * kQ8DnRows - 1) / (4 * kQ8DnRows), (a.R + kQ8Rows - 1) / kQ8Rows),
                     dim3(256), 0, s, a);
}

}  // namespace

bool moe_q8_supported(int hid, int inter) {
  return hid % kQ8Group == 0 && inter % kQ8Group == 0 && hid <= 8192 && inter <= kQ8MaxInter && inter % 64 == 0;
}

void launch_q8_bf16(const uint8_t *q8, uint16_t *bf, int hid, int inter, hipStream_t s) {
  const uint64_t n = 3ull * hid * inter;
  hipLaunchKernelGGL(q8_to_bf16, dim3((unsigned)std::min<uint64_t>(4096, (n + 255) / 256)), dim3(256), 0, s, q8, bf, n);
}

void launch_moe_q8(const MoeArgs &a, hipStream_t s) {
  IJ_CHECK(a.q8 && a.q8gu && a.q8o, "8-bit shared expert: no block or scratch");
  IJ_CHECK(moe_q8_supported(a.hid, a.inter), "8-bit shared expert: %d x %d not supported", a.hid, a.inter);
  if (a.R > kQ8FewRows && a.q8bf) {  // many rows: the matrix cores
    const Q8Off o = q8_offsets(a.hid, a.inter);
    const uint32_t *sb = (const uint32_t *)(a.q8 + o.sb[0]);
    const int rb = (a.R + kMmRows - 1) / kMmRows;
    hipLaunchKernelGGL(moe_q8_mm, dim3(rb, 2 * a.inter / kMmCols), dim3(256), 0, s, a.x, a.hid, a.R, a.q8bf, sb, a.hid,
                       a.q8gu, 2 * a.inter, a.refr);
    hipLaunchKernelGGL(moe_q8_act, dim3((unsigned)(((uint64_t)a.R * a.inter + 255) / 256)), dim3(256), 0, s, a.q8gu,
                       a.R, a.inter, a.refr);
    hipLaunchKernelGGL(moe_q8_mm, dim3(rb, a.hid / kMmCols), dim3(256), 0, s, (const float *)a.q8gu, 2 * a.inter, a.R,
                       a.q8bf + 2ull * a.inter * a.hid, (const uint32_t *)(a.q8 + o.sb[2]), a.inter, a.q8o, a.hid,
                       a.refr);
    return;
  }
  const int ng = (a.hid + 1023) / 1024;
  if (ng <= 2)
    launch_gu<2>(a, s);
  else if (ng <= 4)
    launch_gu<4>(a, s);
  else
    launch_gu<8>(a, s);
  launch_dn<1>(a, s);  // inter <= 1024: one chunk per lane
}

}  // namespace ijah
