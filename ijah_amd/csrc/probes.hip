// Measurement probes behind the kernels' design, built into their own library (ijah_amd/_lib/libijah_probes.so,
// never into the product library) and launched by name through ijah_probe_run (bench.py --probe, --copy-probe):
//   probe_decode<K>  the trellis decode alone: every wave decodes the same 8 LDS-resident tile pairs into matrix-core
//                    B operands over and over (the LDS reads included), so the time is the decode's VALU cost per
//                    weight with no memory traffic;
//   probe_mix<K>     decode and matrix cores on one SIMD: mode 0 decode only, 1 MFMA only (the chain length of the
//                    real kernels: one dependent 32x32x16 f16 MFMA per decoded tile pair), 2 each wave decodes a tile
//                    and feeds it to its MFMA chain (the fused loop of the GEMMs), 3 even waves decode and odd waves
//                    run MFMA chains (specialised waves). Comparing the times says whether the two overlap.
//   probe_stream     cold streams into LDS (global_load_lds) against plain 16-byte loads into registers;
//   copy_u128        a plain device copy: the byte count that scales HBM traffic counters (FETCH_SIZE, WRITE_SIZE).
// Per wave (64 words of out): lane 0 the results folded (so that nothing is optimised away), lane 1 the s_memtime
// ticks of its loop, lanes 2-3 its HW_ID and XCC_ID (where it ran), lane 4 the loop in 100 MHz real-time ticks.
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "exl3_device.h"

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


// probe_lut<K>: the trellis decode through a 32768-entry fp16 codebook table in LDS (64 KB, built by the workgroup
// from the same arithmetic at launch) instead of evaluating the codebook per weight: a field extract, an address and
// one 2-byte LDS read per weight. One workgroup per CU, blockDim / 256 waves per SIMD. Mode 0 decode only, mode 2
// decode feeding each wave's MFMA chain, modes 1 and 3 a mix of table and evaluated tile pairs; lane 5 of out: the lanes' weights that differ from decode_pair (checked once
// before the timed loop).
template <int K>
__device__ __forceinline__ f16x8 decode_pair_lut(const uint8_t *tl, int kt, const _Float16 *lut) {
  constexpr int TW = 8 * K;
  const int lane = threadIdx.x & 63;
  const BLane<K> B = b_lane<K>((uint32_t)lane);
  const uint32_t *T0 = (const uint32_t *)tl + B.tile * TW + kt * 2 * TW;
  TileWords w[2];
  w[0].w0 = T0[B.g0.i0];
  w[0].w1 = T0[B.g0.i1];
  w[0].w2 = kThreeWords<K> ? T0[B.g0.i2] : 0u;
  w[1].w0 = T0[B.g1.i0];
  w[1].w1 = T0[B.g1.i1];
  w[1].w2 = kThreeWords<K> ? T0[B.g1.i2] : 0u;
  const uint32_t sh[2] = {B.g0.sh, B.g1.sh};
  f16x8 r;
#pragma unroll
  for (int g = 0; g < 2; g++) {
    uint32_t c[4];
    codewords4<K>(w[g], sh[g], c);
#pragma unroll
    for (int i = 0; i < 4; i++) r[4 * g + i] = lut[c[i]];
  }
  return r;
}
template <int K>
__global__ __launch_bounds__(1024) void probe_lut(const uint8_t *tiles, int iters, int mode, uint32_t *out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  _Float16 *lut = (_Float16 *)lds;
  constexpr uint32_t B = kProbeTiles * 64 * K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (uint32_t c = threadIdx.x; c < 32768u; c += blockDim.x) {
    const f16x2 v = mcg_pair(c, c);
    lut[c] = v.x;
  }
  uint8_t *slot = lds + 65536 + wave * B;
  for (uint32_t o = lane * 16; o < B; o += 1024) *(uint4 *)(slot + o) = *(const uint4 *)(tiles + o);
  __syncthreads();
  uint32_t bad = 0;
#pragma unroll
  for (int kt = 0; kt < kProbeTiles; kt++) {
    const uint4 u = __builtin_bit_cast(uint4, decode_pair_lut<K>(slot, kt, lut));
    const uint4 v = __builtin_bit_cast(uint4, decode_pair<K>(slot, kt));
    bad += (u.x != v.x) + (u.y != v.y) + (u.z != v.z) + (u.w != v.w);
  }
  uint32_t h = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; i++) acc[i] = 0.f;
  f16x8 a;
#pragma unroll
  for (int i = 0; i < 8; i++) a[i] = (_Float16)(0.001f * (lane + i));
  for (int it = 0; it < iters; it++) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int kt = 0; kt < kProbeTiles; kt++) {
      // mode 1/3: a mix, tile pairs kt % 4 < 2 (mode 1) or kt % 4 < 1 (mode 3) through the table, the others evaluated
      const bool use_lut = mode == 1 ? (kt & 3) < 2 : mode == 3 ? (kt & 3) < 1 : true;
      const f16x8 b = use_lut ? decode_pair_lut<K>(slot, kt, lut) : decode_pair<K>(slot, kt);
      const uint4 u = __builtin_bit_cast(uint4, b);
      h ^= u.x ^ u.y ^ u.z ^ u.w;
      if (mode == 2) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) s += acc[i];
  const uint32_t cyc = (uint32_t)(__builtin_amdgcn_s_memtime() - t0);
  const uint32_t rt = (uint32_t)(__builtin_amdgcn_s_memrealtime() - r0);
  const uint32_t v = lane == 1 ? cyc : lane == 4 ? rt : lane == 5 ? bad : (h ^ __float_as_uint(s));
  out[(blockIdx.x * (blockDim.x >> 6) + wave) * 64 + lane] = v;
}


// probe_x4<K, AG>: each decoded tile pair feeds four independent MFMA chains (the ratio of a 128-row grouped GEMM);
// mode 0 the four chains alone (a fixed operand), mode 1 decode + chains. AG: the accumulators in AGPRs (the MFMA
// written as inline asm with an "a" operand), else in VGPRs. Output as probe_mix.
template <int K, bool AG>
__global__ __launch_bounds__(256) void probe_x4(const uint8_t *tiles, int iters, int mode, uint32_t *out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint8_t *slot = probe_stage<K>(tiles, lds);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t h = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  f32x16 acc[4];
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[r][i] = 0.f;
  f16x8 a, bfix;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (lane + i));
    bfix[i] = (_Float16)(0.002f * (lane - i));
  }
  for (int it = 0; it < iters; it++) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int kt = 0; kt < kProbeTiles; kt++) {
      f16x8 b = bfix;
      if (mode == 1) {
        b = decode_pair<K>(slot, kt);
        const uint4 u = __builtin_bit_cast(uint4, b);
        h ^= u.x ^ u.y ^ u.z ^ u.w;
      }
#pragma unroll
      for (int r = 0; r < 4; r++) {
        if constexpr (AG)
          asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc[r]) : "v"(a), "v"(b));
        else
          acc[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[r], 0, 0, 0);
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int i = 0; i < 16; i++) s += acc[r][i];
  const uint32_t cyc = (uint32_t)(__builtin_amdgcn_s_memtime() - t0);
  const uint32_t rt = (uint32_t)(__builtin_amdgcn_s_memrealtime() - r0);
  const uint32_t v = lane == 1 ? cyc : lane == 4 ? rt : (h ^ __float_as_uint(s));
  out[(blockIdx.x * 4 + wave) * 64 + lane] = v;
}

}  // namespace

struct ProbeEntry {
  const char *name;
  const void *fn;
  std::vector<uint32_t> arg_sizes;
  int K;  // -1: any
  int v;  // variant (-1: any)
};
__global__ __launch_bounds__(256) void copy_u128(const uint4 *src, uint4 *dst, uint64_t n16) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
const std::vector<ProbeEntry> &probes() {
  const uint32_t P = sizeof(void *), I = sizeof(int);
  static const std::vector<ProbeEntry> v = {
      {"probe_mix", (const void *)&probe_mix<2>, {P, I, I, P}, 2, -1},
      {"probe_mix", (const void *)&probe_mix<3>, {P, I, I, P}, 3, -1},
      {"probe_mix", (const void *)&probe_mix<4>, {P, I, I, P}, 4, -1},
      {"probe_mix", (const void *)&probe_mix<5>, {P, I, I, P}, 5, -1},
      {"probe_mix", (const void *)&probe_mix<6>, {P, I, I, P}, 6, -1},
      {"probe_mix", (const void *)&probe_mix<7>, {P, I, I, P}, 7, -1},
      {"probe_mix", (const void *)&probe_mix<8>, {P, I, I, P}, 8, -1},
      {"probe_lut", (const void *)&probe_lut<5>, {P, I, I, P}, 5, -1},
      {"probe_lut", (const void *)&probe_lut<8>, {P, I, I, P}, 8, -1},
      {"probe_x4", (const void *)&probe_x4<5, false>, {P, I, I, P}, 5, 0},
      {"probe_x4", (const void *)&probe_x4<5, true>, {P, I, I, P}, 5, 1},
      {"probe_stream", (const void *)&probe_stream, {P, I, I, P}, -1, -1},
      {"copy_u128", (const void *)&copy_u128, {P, P, 8}, -1, -1},
  };
  return v;
}

}  // namespace ijah

// args: nargs slots of 8 bytes each (a device address or a value in the low bytes, as the kernel's argument sizes say);
// runs reps launches and waits; *ms = their GPU time. Returns 0, or -1 with a message in err (errlen bytes).
extern "C" __attribute__((visibility("default"))) int ijah_probe_run(const char *name, int K, int variant,
                                                                   const uint64_t *args, int nargs,
                                                                   const unsigned *grid, const unsigned *block,
                                                                   unsigned lds, int reps, double *ms, char *err,
                                                                   int errlen) {
  using namespace ijah;
  auto fail = [&](const char *m) {
    snprintf(err, (size_t)errlen, "%s", m);
    return -1;
  };
  static bool attrs = false;
  if (!attrs) {
    for (const void *f : {(const void *)&probe_lut<5>, (const void *)&probe_lut<8>})
      if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 65536 + 16 * kProbeTiles * 64 * 8))
        return fail("hipFuncSetAttribute failed");
    attrs = true;
  }
  for (const ProbeEntry &e : probes()) {
    if (strcmp(e.name, name) || (e.K >= 0 && e.K != K) || (e.v >= 0 && e.v != variant)) continue;
    if ((int)e.arg_sizes.size() != nargs) return fail("argument count");
    std::vector<void *> addr(nargs);
    for (int i = 0; i < nargs; i++) addr[i] = const_cast<uint64_t *>(args + i);  // little-endian: low bytes first
    hipEvent_t a, b;
    if (hipEventCreate(&a) || hipEventCreate(&b)) return fail("hipEventCreate failed");
    hipEventRecord(a, nullptr);
    for (int r = 0; r < reps; r++)
      if (hipLaunchKernel(e.fn, dim3(grid[0], grid[1], grid[2]), dim3(block[0], block[1], block[2]), addr.data(), lds,
                          nullptr) != hipSuccess)
        return fail("launch failed");
    hipEventRecord(b, nullptr);
    if (hipEventSynchronize(b) != hipSuccess) return fail("probe failed on the GPU");
    float t = 0.f;
    hipEventElapsedTime(&t, a, b);
    *ms = t;
    hipEventDestroy(a);
    hipEventDestroy(b);
    return 0;
  }
  return fail("no such probe");
}
