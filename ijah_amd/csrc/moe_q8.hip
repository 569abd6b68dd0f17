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

#include "exl3_device.h"
#include "kernels.h"
#include "moe_device.h"

namespace ijah {

namespace {

constexpr int kQ8Rows = 8;          // input rows per workgroup (x / h reads per loaded weight row)
constexpr int kQ8MaxInter = 1024;   // h of kQ8Rows rows in LDS
constexpr int kQ8DnRows = 4;        // down rows per wave

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

void launch_moe_q8(const MoeArgs &a, hipStream_t s) {
  IJ_CHECK(a.q8 && a.q8gu && a.q8o, "8-bit shared expert: no block or scratch");
  IJ_CHECK(moe_q8_supported(a.hid, a.inter), "8-bit shared expert: %d x %d not supported", a.hid, a.inter);
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
