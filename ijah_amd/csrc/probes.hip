// Measurement probes behind the kernels' design (registered by name for ne_run_kernel; bench.py --probe drives them):
//   probe_decode<K>  the trellis decode alone: every wave decodes the same 8 LDS-resident tile pairs into matrix-core
//                    B operands over and over (the LDS reads included), so the time is the decode's VALU cost per
//                    weight with no memory traffic;
//   probe_mix<K>     decode and matrix cores on one SIMD: mode 0 decode only, 1 MFMA only (the chain length of the
//                    real kernels: one dependent 32x32x16 f16 MFMA per decoded tile pair), 2 each wave decodes a tile
//                    and feeds it to its MFMA chain (the fused loop of the GEMMs), 3 even waves decode and odd waves
//                    run MFMA chains (specialised waves). Comparing the times says whether the two overlap.
//   probe_stream     cold streams into LDS (global_load_lds) against plain 16-byte loads into registers.
// Per wave (64 words of out): lane 0 the results folded (so that nothing is optimised away), lane 1 the s_memtime
// ticks of its loop, lanes 2-3 its HW_ID and XCC_ID (where it ran), lane 4 the loop in 100 MHz real-time ticks.
#include <hip/hip_runtime.h>

#include "exl3_device.h"
#include "kernels.h"

namespace ijah {

namespace {

constexpr int kProbeTiles = 8;  // tile pairs per wave's LDS slot

// a wave's slot: 8 tile pairs copied from tiles (the same for every wave)
template <int K>
__device__ __forceinline__ uint8_t *probe_stage(const uint8_t *tiles, uint8_t *lds) {
  constexpr uint32_t B = kProbeTiles * 64 * K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint8_t *slot = lds + wave * B;
  for (uint32_t o = lane * 16; o < B; o += 1024) *(uint4 *)(slot + o) = *(const uint4 *)(tiles + o);
  __syncthreads();
  return slot;
}

template <int K>
__global__ __launch_bounds__(256) void probe_mix(const uint8_t *tiles, int iters, int mode, uint32_t *out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint8_t *slot = probe_stage<K>(tiles, lds);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool dec = mode == 0 || mode == 2 || (mode == 3 && (wave & 1) == 0);
  const bool mma = mode == 1 || mode == 2 || (mode == 3 && (wave & 1) == 1);
  uint32_t h = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  f16x8 a, bfix;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (lane + i));
    bfix[i] = (_Float16)(0.002f * (lane - i));
  }
  for (int it = 0; it < iters; it++) {
    asm volatile("" ::: "memory");  // the slot is read again every pass
#pragma unroll
    for (int kt = 0; kt < kProbeTiles; kt++) {
      f16x8 b = bfix;
      if (dec) {
        b = decode_pair<K>(slot, kt);
        const uint4 u = __builtin_bit_cast(uint4, b);
        h ^= u.x ^ u.y ^ u.z ^ u.w;
      }
      if (mma) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) s += acc[i];
  const uint32_t cyc = (uint32_t)(__builtin_amdgcn_s_memtime() - t0);
  const uint32_t rt = (uint32_t)(__builtin_amdgcn_s_memrealtime() - r0);  // 100 MHz ticks
  uint32_t hw, xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  // lane 0: the sink; lane 1: s_memtime ticks of the wave's work; lane 2: HW_ID; lane 3: XCC_ID; lane 4: the
  // same interval in 100 MHz real-time ticks
  const uint32_t v = lane == 1 ? cyc : lane == 2 ? hw : lane == 3 ? xcc : lane == 4 ? rt : (h ^ __float_as_uint(s));
  out[(blockIdx.x * 4 + wave) * 64 + lane] = v;
}

// probe_stream: every wave streams `bytes` (a multiple of 1 KB) from its own span of src: mode 0 into LDS with
// global_load_lds (1 KB per request, the fused kernels' tile streams), mode 1 into registers with 16-byte loads
// (folded into a checksum). One wait at the end; lane 1 of out records the wave's s_memtime ticks.
__global__ __launch_bounds__(1024) void probe_stream(const uint8_t *src, uint32_t bytes, int mode, uint32_t *out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const uint8_t *p = src + ((uint64_t)blockIdx.x * nw + wave) * bytes;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  uint32_t h = 0;
  if (mode == 0) {
    uint8_t *dst = lds + wave * 4096;  // 4 KB per wave, reused round robin (the data is not read)
    for (uint32_t o = 0; o < bytes; o += 1024)
      __builtin_amdgcn_global_load_lds((const void *)(p + o + lane * 16),
                                       (__attribute__((address_space(3))) void *)(dst + (o & 4095)), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    h = ((const uint32_t *)dst)[lane];
  } else {
    uint4 acc = make_uint4(0, 0, 0, 0);
    for (uint32_t o = 0; o < bytes; o += 8192) {
      uint4 v[8];
#pragma unroll
      for (int j = 0; j < 8; j++)
        v[j] = o + j * 1024 < bytes ? *(const uint4 *)(p + o + j * 1024 + lane * 16) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        acc.x ^= v[j].x;
        acc.y ^= v[j].y;
        acc.z ^= v[j].z;
        acc.w ^= v[j].w;
      }
    }
    h = acc.x ^ acc.y ^ acc.z ^ acc.w;
  }
  const uint32_t cyc = (uint32_t)(__builtin_amdgcn_s_memtime() - t0);
  out[(blockIdx.x * nw + wave) * 64 + lane] = lane == 1 ? cyc : h;
}

}  // namespace

size_t probe_lds(int K) { return (size_t)4 * kProbeTiles * 64 * K; }

void probe_kernels(std::vector<KernelEntry> &v) {
  const uint32_t P = sizeof(void *), I = sizeof(int);
  v.push_back({"probe_mix", (const void *)&probe_mix<2>, {P, I, I, P}, 2, -1});
  v.push_back({"probe_mix", (const void *)&probe_mix<3>, {P, I, I, P}, 3, -1});
  v.push_back({"probe_mix", (const void *)&probe_mix<4>, {P, I, I, P}, 4, -1});
  v.push_back({"probe_mix", (const void *)&probe_mix<5>, {P, I, I, P}, 5, -1});
  v.push_back({"probe_mix", (const void *)&probe_mix<6>, {P, I, I, P}, 6, -1});
  v.push_back({"probe_mix", (const void *)&probe_mix<7>, {P, I, I, P}, 7, -1});
  v.push_back({"probe_mix", (const void *)&probe_mix<8>, {P, I, I, P}, 8, -1});
  v.push_back({"probe_stream", (const void *)&probe_stream, {P, I, I, P}, -1, -1});
}

}  // namespace ijah
