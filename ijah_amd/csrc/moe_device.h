// Device helpers shared by the three MoE layer paths (fused single-row, staged, batched).
#pragma once
#include "exl3_device.h"
#include "kernels.h"

namespace ijah {

__device__ __forceinline__ float moe_rr(float x, int refr) { return refr ? bf16_round(x) : x; }

// the shared-expert gate of a row from its (bf16-valued) logit: sigmoid, rounded to bf16 under the hyper-connection
// write with rounding on (reference kernels/fn_moe.metal:421 and :444, rr(sgt))
__device__ __forceinline__ float moe_shared_gate(const MoeArgs &a, float logit) {
  const float sg = a.has_sgate ? 1.f / (1.f + expf(-logit)) : 1.f;
  return a.hc > 0 ? moe_rr(sg, a.refr) : sg;
}

// Row r's output at column c from its routed sum s (slots 0..topk-1 summed in slot order) and the gated shared term
// t (0 without a shared expert). Plain: y = s + t, the slot-order sum. With the hyper-connection write (reference
// kernels/fn_moe.metal:437-448): y = branch = rr(rr(s) + rr(t)), and the hc streams of hc_out are written.
__device__ __forceinline__ float moe_finish(const MoeArgs &a, int r, int c, float s, float t) {
  if (a.hc <= 0) return s + t;
  const int q = a.refr;
  const float br = moe_rr(moe_rr(s, q) + moe_rr(t, q), q);
  for (int st = 0; st < a.hc; st++) {
    const uint64_t o = ((uint64_t)r * a.hc + st) * a.hid + c;
    a.hc_out[o] = moe_rr(a.hc_h[o] + moe_rr(br * a.hc_inj[r * 8 + st], q), q);
  }
  return br;
}

}  // namespace ijah

namespace ijah {

// ---------------------------------------------------------------------------------------------------- 8-bit shared
// The shared expert in the reference's 8-bit affine form (MLX layout: weight bytes [rows][in], bf16 scale and bias
// per group of kQ8Group inputs; w = scale q + bias; reference kernels/ne_common.h:33-88, q8row_dev / q8rows_dev, used
// for the shared gate / up at kernels/fn_moe.metal:40-46 and the shared down at :264-290). In HBM the group's scale and
// bias are one u32 word (scale low, bias high), [rows][in / kQ8Group], after the three weight arrays.
// Every path computes one row's dot the same way, so a row's value depends on nothing but its inputs (the one-row
// step and the batched kernels agree bit for bit): lane l takes the 16-byte chunks c = l, l + 64, ... of the row; per
// chunk qx = sum q_i x_i (an fmaf chain in byte order) and sx = sum x_i (in order), then acc = fmaf(s, qx, acc),
// acc = fmaf(b, sx, acc); the lanes meet in an xor butterfly over 32, 16, ..., 1, so every lane ends with the sum.
// (Rows of at most 512 inputs use lanes 0..31 only: the first butterfly step adds exact zeros.)
// one 16-byte chunk of a row (bytes w, group word sb) against 16 inputs x0..x3, onto acc
__device__ __forceinline__ float q8_chunk(uint4 w, uint32_t sb, float4 x0, float4 x1, float4 x2, float4 x3, float acc) {
  const float xs[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w, x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float qx = (float)(ws[0] & 0xFFu) * xs[0];
  float sx = xs[0];
#pragma unroll
  for (int i = 1; i < 16; i++) {
    qx = __builtin_fmaf((float)((ws[i >> 2] >> (8 * (i & 3))) & 0xFFu), xs[i], qx);
    sx = sx + xs[i];
  }
  acc = __builtin_fmaf(bf16_f32(sb & 0xFFFFu), qx, acc);
  return __builtin_fmaf(bf16_f32(sb >> 16), sx, acc);
}
__device__ __forceinline__ float q8_wave_sum(float acc) {
  acc += __shfl_xor(acc, 32, 64);
  acc += __shfl_xor(acc, 16, 64);
  acc += __shfl_xor(acc, 8, 64);
  acc += __shfl_xor(acc, 4, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 1, 64);
  return acc;
}
// the shared SwiGLU input of the down rows: h = rr(silu(g) u) from the rounded gate / up outputs (reference
// kernels/fn_moe.metal:265-268)
__device__ __forceinline__ float q8_act(float g, float u, int refr) { return moe_rr(g / (1.f + expf(-g)) * u, refr); }

// the 16-byte chunks of a row that lane l owns: c = l + 64 j, j < NCH
template <int NCH>
struct Q8Row {
  uint4 w[NCH];
  uint32_t sb[NCH];
};
template <int NCH>
__device__ __forceinline__ void q8_load(const uint8_t *w, const uint32_t *sb, int in, Q8Row<NCH> &r) {
  const int lane = threadIdx.x & 63, nc = in / 16;
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    const int c = lane + 64 * j;
    r.w[j] = c < nc ? *(const uint4 *)(w + 16 * c) : make_uint4(0, 0, 0, 0);
    r.sb[j] = c < nc ? sb[16 * c / kQ8Group] : 0u;
  }
}
// the row's dot with x (f32 [in], global or LDS): every lane returns it
template <int NCH>
__device__ __forceinline__ float q8_dot(const Q8Row<NCH> &r, const float *x, int in) {
  const int lane = threadIdx.x & 63, nc = in / 16;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    const int c = lane + 64 * j;
    if (c < nc) {
      const float4 *xp = (const float4 *)(x + 16 * c);
      acc = q8_chunk(r.w[j], r.sb[j], xp[0], xp[1], xp[2], xp[3], acc);
    }
  }
  return q8_wave_sum(acc);
}

}  // namespace ijah
