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
