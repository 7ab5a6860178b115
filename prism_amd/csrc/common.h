// Shared device/host helpers for the prism_bsa HIP library (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#define PRISM_F32 0
#define PRISM_BF16 1

#define PRISM_OK 0
#define PRISM_EINVAL 1
#define PRISM_EHIP 2

// ------------------------------------------------------------ host error state
void prism_set_error(const char* fmt, ...);

#define PRISM_REQUIRE(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      prism_set_error(__VA_ARGS__);              \
      return PRISM_EINVAL;                       \
    }                                            \
  } while (0)

#define PRISM_LAUNCH_CHECK(what)                                               \
  do {                                                                         \
    hipError_t _e = hipGetLastError();                                         \
    if (_e != hipSuccess) {                                                    \
      prism_set_error("%s: launch failed: %s", what, hipGetErrorString(_e));   \
      return PRISM_EHIP;                                                       \
    }                                                                          \
  } while (0)

// ------------------------------------------------------------ scalar helpers
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ float ldf(const void* p, int dtype, int64_t i) {
  return dtype == PRISM_BF16 ? bf2f(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

// Candidate block shapes (bt, bh, bw), table order of the reference's
// dynamic_block_shape.py:6-27: seven 64-token shapes, then six 128-token shapes.
__constant__ static const int8_t kCand[13][3] = {
    {4, 4, 4}, {8, 2, 4}, {8, 4, 2}, {2, 4, 8}, {2, 8, 4}, {4, 2, 8}, {4, 8, 2},
    {2, 8, 8}, {8, 2, 8}, {8, 8, 2}, {4, 4, 8}, {4, 8, 4}, {8, 4, 4},
};
#define PRISM_NCAND 13

// Rearranged position r (0..511) inside a zone of shape c -> local flat
// coordinate lt*64 + lh*8 + lw (blocks t-major, then h, then w; tokens inside a
// block t-major, then h, then w).
__device__ __forceinline__ int local_of_rearr(int c, int r) {
  const int bt = kCand[c][0], bh = kCand[c][1], bw = kCand[c][2];
  const int bsz = bt * bh * bw, Nh = 8 / bh, Nw = 8 / bw;
  const int blk = r / bsz, off = r - blk * bsz;
  const int nt = blk / (Nh * Nw), nh = (blk / Nw) % Nh, nw = blk % Nw;
  const int it = off / (bh * bw), ih = (off / bw) % bh, iw = off % bw;
  return ((nt * bt + it) * 8 + (nh * bh + ih)) * 8 + (nw * bw + iw);
}

// THW token index of local coordinate lf in zone z of a ZT x ZH x ZW zone grid.
__device__ __forceinline__ int64_t token_of(int z, int lf, int ZH, int ZW, int Hg, int Wg) {
  const int zt = z / (ZH * ZW), zh = (z / ZW) % ZH, zw = z % ZW;
  const int lt = lf >> 6, lh = (lf >> 3) & 7, lw = lf & 7;
  return ((int64_t)(zt * 8 + lt) * Hg + zh * 8 + lh) * Wg + zw * 8 + lw;
}

// The input grid T x H x W inside the zone grid (the zone grid is the input
// grid rounded up to multiples of 8; positions outside the input are the
// padding of wan_video_dit.py:342-400, read as zero and invalid).
struct GridBox {
  int T, H, W;
};
// token of local coordinate lf of zone z in the input grid, or -1 (padding)
__device__ __forceinline__ int64_t token_in(int z, int lf, int ZH, int ZW, GridBox b) {
  const int zt = z / (ZH * ZW), zh = (z / ZW) % ZH, zw = z % ZW;
  const int t = zt * 8 + (lf >> 6), h = zh * 8 + ((lf >> 3) & 7), w = zw * 8 + (lf & 7);
  if (t >= b.T || h >= b.H || w >= b.W) return -1;
  return ((int64_t)t * b.H + h) * b.W + w;
}
// host check: the input grid is non-empty and fits inside the zone grid
inline bool box_ok(int T, int Hg, int Wg, int Tin, int Hin, int Win) {
  return Tin > 0 && Hin > 0 && Win > 0 && Tin <= T && Hin <= Hg && Win <= Wg;
}

// ------------------------------------------------------------ canonical math
// canon_exp: Cody-Waite reduction with the Cephes split of ln 2, degree-7
// Taylor polynomial (Horner, fused), exact power-of-two scale.  x < -87 -> 0.
__device__ __forceinline__ float canon_exp(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  if (x > 88.0f) return __uint_as_float(0x7f800000u);
  if (x < -87.0f) return 0.0f;
  float t = x * 1.44269504f;
  float n = floorf(t + 0.5f);
  float r = __builtin_fmaf(-n, 0.693359375f, x);
  r = __builtin_fmaf(-n, -2.12194440e-4f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// canon_log2 of a positive normal x: m in [sqrt(1/2), sqrt(2)), 2*atanh series
// of s = (m-1)/(m+1) to s^11, log2 x = e + ln(m) * log2(e).
__device__ __forceinline__ float canon_log2(float x) {
#pragma clang fp contract(off)
  const uint32_t u = __float_as_uint(x);
  int e = (int)((u >> 23) & 0xffu) - 127;
  float m = __uint_as_float((u & 0x7fffffu) | 0x3f800000u);
  if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float z = s * s;
  float p = 0.0909090909f;
  p = __builtin_fmaf(p, z, 0.111111111f);
  p = __builtin_fmaf(p, z, 0.142857143f);
  p = __builtin_fmaf(p, z, 0.2f);
  p = __builtin_fmaf(p, z, 0.333333333f);
  const float s2 = s + s;
  const float lnm = __builtin_fmaf(s2 * z, p, s2);
  return __builtin_fmaf(lnm, 1.44269504f, (float)e);
}

// exact floor(w * 2^F) for finite w >= 0
__device__ __forceinline__ uint64_t fixp(float w, int F) {
  const uint32_t u = __float_as_uint(w);
  int e = (int)((u >> 23) & 0xffu);
  uint64_t m = u & 0x7fffffu;
  if (e == 0) e = 1; else m |= 0x800000u;
  int sh = e - 150 + F;
  if (sh >= 0) return m << sh;
  sh = -sh;
  return sh >= 64 ? 0ull : (m >> sh);
}

// ------------------------------------------------------------ wave reductions
// 64-lane xor butterfly; every lane ends with the same value.  The fp32
// version fixes the canonical channel-sum order used for bit-exact parity.
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma clang fp contract(off)
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max_xor(float v) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// inclusive prefix sum across the 64 lanes
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v, int lane) {
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}
