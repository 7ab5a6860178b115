// Work lists for the paired-tile attention kernels (gfx950).
//
// The attention kernels run one workgroup per PAIR of tiles (2p, 2p+1) and
// walk the sorted union of the two tiles' lists, staging each listed tile once
// for both.  prism_pair_union builds those unions from any per-row list
// (per-query-tile key lists for the forward and dQ passes, per-key-tile query
// lists for dK/dV): entry = tile << 3 | partial << 2 | in_second << 1 | in_first.
// It replaces the per-iteration merge of two list cursors, whose dependent
// index loads sat on the critical path of every key tile.
//
// prism_tile_masks packs the per-token key validity of each 64-token tile into
// one 64-bit word (bit j = token j valid), read with one scalar load by the
// kernels for tiles marked partial.  prism_lse_to_m2 converts the forward's
// natural-log LSE into the base-2 row maximum the backward exponentiates
// against, with -inf (a row that saw no valid key) mapped to +inf so that
// exp2(s - m2) is exactly 0 for it without a per-element test.
#include "common.h"

namespace {

constexpr int kUnionWin = 8192;  // tiles per LDS bitmap window (256 words)

// one 256-thread workgroup per row pair
__global__ __launch_bounds__(256) void pair_union_kernel(const int64_t* __restrict__ start,
                                                         const int32_t* __restrict__ len,
                                                         const int32_t* __restrict__ cols, int64_t Nc,
                                                         const uint64_t* __restrict__ tile_masks, int64_t ucap,
                                                         int64_t* __restrict__ ustart, int32_t* __restrict__ ulen,
                                                         int32_t* __restrict__ ucols) {
  __shared__ uint32_t bmA[kUnionWin / 32], bmB[kUnionWin / 32];
  __shared__ uint32_t wtot[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t p = blockIdx.x;
  const int64_t rA = 2 * p, rB = rA + 1;
  const int32_t* A = cols + start[rA];
  const int32_t* B = cols + start[rB];
  const int nA = len[rA], nB = len[rB];
  // list entries index column tiles inside one head (0 .. Nc-1), as does tile_masks
  int32_t* out = ucols + p * ucap;
  int count = 0;
  for (int64_t w0 = 0; w0 < Nc; w0 += kUnionWin) {
    bmA[tid] = 0u;
    bmB[tid] = 0u;
    __syncthreads();
    for (int i = tid; i < nA; i += 256) {
      const int64_t t = (int64_t)A[i] - w0;
      if (t >= 0 && t < kUnionWin && A[i] < Nc) atomicOr(&bmA[t >> 5], 1u << (t & 31));
    }
    for (int i = tid; i < nB; i += 256) {
      const int64_t t = (int64_t)B[i] - w0;
      if (t >= 0 && t < kUnionWin && B[i] < Nc) atomicOr(&bmB[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    const uint32_t a = bmA[tid], b = bmB[tid];
    uint32_t u = a | b;
    const uint32_t c = __popc(u);
    const uint32_t incl = wave_incl_scan_u32(c, lane);
    if (lane == 63) wtot[w] = incl;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t t = wtot[k];
      before += k < w ? t : 0u;
      total += t;
    }
    int pos = count + (int)(before + incl - c);
    while (u) {
      const int bit = __ffs(u) - 1;
      u &= u - 1;
      const int64_t tile = w0 + 32 * tid + bit;
      int e = (int)(tile << 3) | (int)((a >> bit) & 1u) | (int)(((b >> bit) & 1u) << 1);
      if (tile_masks && tile_masks[tile] != ~0ull) e |= 4;
      out[pos++] = e;
    }
    count += (int)total;
    __syncthreads();
  }
  if (tid == 0) {
    ustart[p] = p * ucap;
    ulen[p] = count;
  }
}

// one wave per tile: bit j of masks[t] = valid[64 t + j] != 0
__global__ __launch_bounds__(256) void tile_masks_kernel(const uint8_t* __restrict__ valid, int64_t Nt,
                                                         uint64_t* __restrict__ masks) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= Nt) return;
  const uint64_t m = __ballot(valid[t * 64 + lane] != 0);
  if (lane == 0) masks[t] = m;
}

__global__ __launch_bounds__(256) void lse_to_m2_kernel(const float* __restrict__ lse, int64_t n, float* __restrict__ m2) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float x = lse[i];
  m2[i] = x == -__builtin_inff() ? __builtin_inff() : x * 1.4426950408889634f;
}

}  // namespace

extern "C" {

int prism_pair_union(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, const uint64_t* tile_masks, int64_t ucap, int64_t* ustart, int32_t* ulen,
                     int32_t* ucols, hipStream_t stream) {
  PRISM_REQUIRE(start && len && cols && ustart && ulen && ucols, "prism_pair_union: null pointer");
  PRISM_REQUIRE(rows >= 0 && rows % 2 == 0, "prism_pair_union: rows must be even (pairs of tiles)");
  PRISM_REQUIRE(row_tiles > 0 && row_tiles % 2 == 0 && rows % row_tiles == 0,
                "prism_pair_union: rows must be a multiple of an even row_tiles (tiles per head)");
  PRISM_REQUIRE(col_tiles > 0 && col_tiles < (1ll << 28), "prism_pair_union: col_tiles out of range");
  PRISM_REQUIRE(ucap >= col_tiles, "prism_pair_union: ucap must be >= col_tiles");
  const int64_t pairs = rows / 2;
  if (pairs == 0) return PRISM_OK;
  PRISM_REQUIRE(pairs < (1ll << 31), "prism_pair_union: too many pairs");
  pair_union_kernel<<<(unsigned)pairs, 256, 0, stream>>>(start, len, cols, col_tiles, tile_masks, ucap, ustart, ulen, ucols);
  PRISM_LAUNCH_CHECK("prism_pair_union");
  return PRISM_OK;
}

int prism_tile_masks(const uint8_t* valid, int64_t Nt, uint64_t* masks, hipStream_t stream) {
  PRISM_REQUIRE(valid && masks, "prism_tile_masks: null pointer");
  PRISM_REQUIRE(Nt >= 0, "prism_tile_masks: negative N_tiles");
  if (Nt == 0) return PRISM_OK;
  tile_masks_kernel<<<(unsigned)((Nt + 3) / 4), 256, 0, stream>>>(valid, Nt, masks);
  PRISM_LAUNCH_CHECK("prism_tile_masks");
  return PRISM_OK;
}

int prism_lse_to_m2(const float* lse, int64_t n, float* m2, hipStream_t stream) {
  PRISM_REQUIRE(lse && m2, "prism_lse_to_m2: null pointer");
  PRISM_REQUIRE(n >= 0, "prism_lse_to_m2: negative length");
  if (n == 0) return PRISM_OK;
  lse_to_m2_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(lse, n, m2);
  PRISM_LAUNCH_CHECK("prism_lse_to_m2");
  return PRISM_OK;
}

}  // extern "C"
