// MFMA operand helpers shared by the attention kernels (gfx950).
//
// v_mfma_f32_32x32x16_bf16 operand layout (64 lanes, g = lane / 32, l32 = lane % 32):
//   A (32 x 16): lane holds A[l32][8g .. 8g+7]
//   B (16 x 32): lane holds B[8g .. 8g+7][l32]
//   C (32 x 32): lane holds C[8(r/4) + 4g + r%4][l32] in register r (16 registers)
// A C block of 64 rows (two 32-row accumulators acc[0], acc[1]) becomes the B
// operand of a following MFMA over k = those 64 rows in four 16-row steps
// tt: step tt uses rows 16tt + {4g..4g+3, 8+4g..8+4g+3} as k-slots 8g..8g+7
// (a permutation of k inside each 16-row group, applied identically to A).
// The matching A operand is read from a row-major tile in LDS by transposing
// reads (TrOperand in tile_dma.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t* p) {
  return as_bf16x8(*reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ f32x16 f32x16_zero() {
  f32x16 z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.0f;
  return z;
}
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
// round-to-nearest-even bf16 pair (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
// B operand of k-step tt from a 64-row accumulator pair (see the header comment)
__device__ __forceinline__ bf16x8 b_from_acc(const f32x16* acc, int tt) {
  const int h = tt >> 1, j0 = 2 * (tt & 1);
  uint4 pb;
  pb.x = pack_bf16(acc[h][4 * j0 + 0], acc[h][4 * j0 + 1]);
  pb.y = pack_bf16(acc[h][4 * j0 + 2], acc[h][4 * j0 + 3]);
  pb.z = pack_bf16(acc[h][4 * j0 + 4], acc[h][4 * j0 + 5]);
  pb.w = pack_bf16(acc[h][4 * j0 + 6], acc[h][4 * j0 + 7]);
  return as_bf16x8(pb);
}
// max(a, b) for non-NaN inputs without NaN canonicalisation (v_med3 with
// +inf folds into v_max3_f32 chains)
__device__ __forceinline__ float fmax_nn(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, __builtin_inff()); }

// x combined with the value of lane (l xor 32) by a symmetric op: one
// v_permlane32_swap puts both halves' values in every lane
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_nn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_add(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x if bit b of bits is set, else -inf: the signed one-bit field extract
// (v_bfe_i32) is the all-ones / zero select mask and one three-input bit
// operation (v_bitop3_b32) merges, two independent VALU ops per element
// instead of a compare, a VCC hazard and a select
__device__ __forceinline__ float keep_or_ninf(float x, uint32_t bits, int b) {
  const uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)bits, (uint32_t)b, 1u);
  return __uint_as_float((__float_as_uint(x) & m) | (~m & 0xff800000u));
}

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) = 0
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// 4 MB L2) in increasing id order, so the resident workgroups at any moment
// are a window of consecutive ids.  Map hardware ids in chunks of 8*G: inside
// a chunk, XCD x takes the G consecutive logical ids [x*G, (x+1)*G) (tiles
// that select overlapping lists share one L2), and the chunks advance through
// the logical order together, so the whole GPU works on one neighbourhood of
// one head at a time (its K/V stay resident in the 256 MB Infinity Cache).
// Ids past the last full chunk map to themselves; a bijection on [0, n).
template <int G>
__device__ __forceinline__ int xcd_group_remap(int bid, int n) {
  const int full = n / (8 * G) * (8 * G);
  if (bid >= full) return bid;
  const int chunk = bid / (8 * G), xcd = bid & 7, slot = (bid >> 3) % G;
  return chunk * 8 * G + xcd * G + slot;
}
