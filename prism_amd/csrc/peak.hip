// Measured ceilings of the device (gfx950), for the benchmark's roofline:
//   mfma_peak_kernel  chains of independent v_mfma_f32_32x32x16_bf16 on
//                     register operands, no memory traffic, on every SIMD
//                     (the bf16 MFMA rate the chip sustains under full load,
//                     at the clock it holds there), with the shader clock
//                     counted against the 100 MHz constant clock;
//   copy_peak_kernel  a 16-byte-per-lane streaming copy (the HBM rate a
//                     read + write stream reaches);
//   tile_stream_peak_kernel  the attention kernels' tile stream without their
//                     math: 32 KB stages of two 16 KB tiles copied into LDS by
//                     global_load_lds_dwordx4 (the forward's plan: waves 0 and
//                     1 issue sixteen 1 KB instructions each), completed and
//                     published with a barrier, one stage in flight per
//                     workgroup, two workgroups per CU; tiles drawn
//                     pseudo-randomly from the source buffer (over a buffer the
//                     Infinity Cache holds but the L2s do not, the rate the
//                     forward's K/V stream can reach).
// No counterpart in the reference (measurement aids of this build).
#include "common.h"
#include "mfma.h"
#include "tile_dma.h"

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

constexpr int kStreamTile = 16384;  // bytes of one 64 x 128 bf16 tile
using StreamRT = RowTile<128>;
static_assert(StreamRT::BYTES == kStreamTile, "stream tiles are 64 x 128 bf16");

// the two tiles of stage j of a workgroup: a 64-bit LCG per workgroup,
// wave-uniform (the same arithmetic is restated by the GPU test)
__device__ __forceinline__ uint64_t stream_lcg(uint64_t h) {
  return h * 6364136223846793005ull + 1442695040888963407ull;
}

__global__ __launch_bounds__(256, 2) void tile_stream_peak_kernel(const uint8_t* __restrict__ src, int64_t ntiles,
                                                                  int64_t steps, uint32_t* __restrict__ sink) {
  __shared__ __align__(16) uint8_t smem[2 * 2 * kStreamTile];  // two stages of two tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const uint32_t soff0 = StreamRT::src_offset(w & 1, lane), soff1 = StreamRT::src_offset((w & 1) + 2, lane);
  const uint32_t lds0 = lds_addr(smem);
  uint64_t h = (uint64_t)blockIdx.x + 1;
  for (int64_t j = 0; j < steps; ++j) {
    h = stream_lcg(h);
    const int64_t ta = (int64_t)((h >> 17) % (uint64_t)ntiles);
    h = stream_lcg(h);
    const int64_t tb = (int64_t)((h >> 17) % (uint64_t)ntiles);
    if (w < 2) {
      const char* a = (const char*)uniform_ptr(src + ta * kStreamTile);
      const char* b = (const char*)uniform_ptr(src + tb * kStreamTile);
      const uint32_t base = lds0 + (uint32_t)((j & 1) * 2 * kStreamTile);
#pragma unroll
      for (int s = 0; s < StreamRT::KB; ++s) {
        const int i = w + 2 * s;                            // instruction of the stage
        const int t = i < StreamRT::KB ? i : i - StreamRT::KB;  // instruction of its tile
        dma_b128((s & 1) ? soff1 : soff0, (i < StreamRT::KB ? a : b) + 4096 * (t >> 2), base + (uint32_t)i * 1024u);
      }
    }
    dma_wait_all();
    __syncthreads();
  }
  // the first word of the last stage: lane 0 of instruction 0, tile ta
  if (tid == 0) sink[blockIdx.x] = *reinterpret_cast<const uint32_t*>(smem + ((steps - 1) & 1) * 2 * kStreamTile);
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

int prism_tile_stream_peak(const void* src, int64_t bytes, int64_t steps, uint32_t* sink, int64_t sink_len,
                           int64_t* moved, hipStream_t stream) {
  PRISM_REQUIRE(src && sink && moved, "prism_tile_stream_peak: null pointer");
  PRISM_REQUIRE(((uintptr_t)src & 15) == 0, "prism_tile_stream_peak: src must be 16-byte aligned");
  PRISM_REQUIRE(bytes >= kStreamTile && bytes % kStreamTile == 0,
                "prism_tile_stream_peak: bytes must be a positive multiple of %d", kStreamTile);
  PRISM_REQUIRE(steps >= 1, "prism_tile_stream_peak: steps must be positive");
  const int cus = device_cus();
  PRISM_REQUIRE(cus > 0, "prism_tile_stream_peak: no device");
  const int64_t blocks = 2LL * cus;  // two workgroups per CU, as the forward kernel
  PRISM_REQUIRE(sink_len >= blocks, "prism_tile_stream_peak: sink needs %lld words", (long long)blocks);
  *moved = blocks * steps * 2 * kStreamTile;
  tile_stream_peak_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const uint8_t*)src, bytes / kStreamTile, steps,
                                                                sink);
  PRISM_LAUNCH_CHECK("prism_tile_stream_peak");
  return PRISM_OK;
}

}  // extern "C"
