// Measured ceilings of the device (gfx950), for the benchmark's roofline:
//   mfma_peak_kernel  chains of independent v_mfma_f32_32x32x16_bf16 on
//                     register operands, no memory traffic, on every SIMD
//                     (the bf16 MFMA rate the chip sustains under full load,
//                     at the clock it holds there), with the shader clock
//                     counted against the 100 MHz constant clock;
//   copy_peak_kernel  a 16-byte-per-lane streaming copy (the HBM rate a
//                     read + write stream reaches).
// No counterpart in the reference (measurement aids of this build).
#include "common.h"
#include "mfma.h"

namespace {

constexpr int kPeakChains = 4;  // independent accumulators per wave (each MFMA depends on the one four back)

__global__ __launch_bounds__(256) void mfma_peak_kernel(int64_t iters, float* __restrict__ sink,
                                                        uint64_t* __restrict__ clocks) {
  const int lane = threadIdx.x & 63;
  uint64_t c0 = 0, r0 = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    c0 = clock64();
    r0 = wall_clock64();
  }
  // operands that depend on the lane (not foldable), accumulators chained
  // through every iteration (not removable)
  uint4 ua, ub;
  ua.x = 0x3f803f80u ^ (uint32_t)lane; ua.y = ua.x + 1; ua.z = ua.x + 2; ua.w = ua.x + 3;
  ub.x = 0x3c003c00u ^ (uint32_t)(lane << 3); ub.y = ub.x + 5; ub.z = ub.x + 6; ub.w = ub.x + 7;
  const bf16x8 a = as_bf16x8(ua), b = as_bf16x8(ub);
  f32x16 acc[kPeakChains];
#pragma unroll
  for (int c = 0; c < kPeakChains; ++c) acc[c] = f32x16_zero();
  for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < kPeakChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kPeakChains; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[c][r];
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clocks[0] = clock64() - c0;
    clocks[1] = wall_clock64() - r0;
  }
}

__global__ __launch_bounds__(256) void copy_peak_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                        int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const uint4 x0 = src[i], x1 = src[i + stride], x2 = src[i + 2 * stride], x3 = src[i + 3 * stride];
    dst[i] = x0;
    dst[i + stride] = x1;
    dst[i + 2 * stride] = x2;
    dst[i + 3 * stride] = x3;
  }
  for (; i < n; i += stride) dst[i] = src[i];
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  return cus;
}

}  // namespace

extern "C" {

int prism_mfma_peak(int64_t iters, float* sink, int64_t sink_len, uint64_t* clocks, int64_t* flops,
                    hipStream_t stream) {
  PRISM_REQUIRE(sink && clocks && flops, "prism_mfma_peak: null pointer");
  PRISM_REQUIRE(iters >= 1, "prism_mfma_peak: iters must be positive");
  const int cus = device_cus();
  PRISM_REQUIRE(cus > 0, "prism_mfma_peak: no device");
  const int64_t blocks = 2LL * cus;  // two 4-wave workgroups per CU: two waves per SIMD
  PRISM_REQUIRE(sink_len >= blocks * 256, "prism_mfma_peak: sink needs %lld floats", (long long)(blocks * 256));
  *flops = blocks * 4 * iters * kPeakChains * (2LL * 32 * 32 * 16);
  mfma_peak_kernel<<<(unsigned)blocks, 256, 0, stream>>>(iters, sink, clocks);
  PRISM_LAUNCH_CHECK("prism_mfma_peak");
  return PRISM_OK;
}

int prism_copy_peak(const void* src, void* dst, int64_t bytes, hipStream_t stream) {
  PRISM_REQUIRE(src && dst, "prism_copy_peak: null pointer");
  PRISM_REQUIRE(bytes > 0 && bytes % 16 == 0, "prism_copy_peak: bytes must be a positive multiple of 16");
  const int cus = device_cus();
  PRISM_REQUIRE(cus > 0, "prism_copy_peak: no device");
  copy_peak_kernel<<<(unsigned)(8 * cus), 256, 0, stream>>>((const uint4*)src, (uint4*)dst, bytes / 16);
  PRISM_LAUNCH_CHECK("prism_copy_peak");
  return PRISM_OK;
}

}  // extern "C"
