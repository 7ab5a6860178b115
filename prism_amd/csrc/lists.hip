// Work lists for the paired-tile attention kernels (gfx950).
//
// The attention kernels run one workgroup per PAIR of tiles (2p, 2p+1) and
// walk the sorted union of the two tiles' lists, staging each listed tile once
// for both.  prism_pair_union builds those unions from any per-row list
// (per-query-tile key lists for the forward and dQ passes, per-key-tile query
// lists for dK/dV): entry = tile << 3 | partial << 2 | in_second << 1 | in_first.
// It replaces the per-iteration merge of two list cursors, whose dependent
// index loads sat on the critical path of every key tile.  prism_quad_union
// does the same for QUADS of tiles (two pairs of a zone, for the forward and
// dQ kernels that take four query tiles per workgroup): entry = tile << 5 |
// partial << 4 | one member bit per row.
//
// prism_tile_masks packs the per-token key validity of each 64-token tile into
// one 64-bit word (bit j = token j valid), read with one scalar load by the
// kernels for tiles marked partial.  prism_lse_to_m2 converts the forward's
// natural-log LSE into the base-2 row maximum the backward exponentiates
// against, with -inf (a row that saw no valid key) mapped to +inf so that
// exp2(s - m2) is exactly 0 for it without a per-element test.
// prism_lists_csr_offsets / prism_lists_csr_fill turn any (start, len, cols)
// lists into compact CSR (int32 offsets, entries stored once, O(nnz) memory).
#include "common.h"
#include "validate.h"

namespace {

constexpr int kUnionWin = 8192;  // tiles per LDS bitmap window (256 words)

// one 256-thread workgroup per group of R rows (R = 2: a pair, R = 4: a quad);
// the group's rows are R p .. R p + R - 1 of the head, or pairmap[R p + k]
// (row indices inside the head).  Entries: tile << (R + 1) | partial << R |
// member bits (bit k: row k lists the tile).
template <int R>
__global__ __launch_bounds__(256) void pair_union_kernel(const int64_t* __restrict__ start,
                                                    const int32_t* __restrict__ len,
                                                    const int32_t* __restrict__ cols, int64_t Nr, int64_t Nc,
                                                    const int32_t* __restrict__ pairmap,
                                                    const uint64_t* __restrict__ tile_masks, int64_t ucap,
                                                    int64_t* __restrict__ ustart, int32_t* __restrict__ ulen,
                                                    int32_t* __restrict__ ucols) {
  __shared__ uint32_t bm[R][kUnionWin / 32];
  __shared__ uint32_t wtot[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t p = blockIdx.x;
  const int64_t head0 = (R * p) / Nr * Nr;
  const int32_t* L[R];
  int nl[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t r = pairmap ? head0 + pairmap[R * p + k] : R * p + k;
    L[k] = cols + start[r];
    nl[k] = len[r];
  }
  // list entries index column tiles inside one head (0 .. Nc-1), as does tile_masks
  int32_t* out = ucols + p * ucap;
  int count = 0;
  for (int64_t w0 = 0; w0 < Nc; w0 += kUnionWin) {
#pragma unroll
    for (int k = 0; k < R; ++k) bm[k][tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < R; ++k)
      for (int i = tid; i < nl[k]; i += 256) {
        const int64_t t = (int64_t)L[k][i] - w0;
        if (t >= 0 && t < kUnionWin && L[k][i] < Nc) atomicOr(&bm[k][t >> 5], 1u << (t & 31));
      }
    __syncthreads();
    uint32_t mb[R], u = 0u;
#pragma unroll
    for (int k = 0; k < R; ++k) {
      mb[k] = bm[k][tid];
      u |= mb[k];
    }
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
      int e = (int)(tile << (R + 1));
#pragma unroll
      for (int k = 0; k < R; ++k) e |= (int)(((mb[k] >> bit) & 1u) << k);
      if (tile_masks && tile_masks[tile] != ~0ull) e |= 1 << R;
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

// ------------------------------------------------------------ tile pairing
// Tiles are paired inside groups of 8 consecutive tiles of a head (a zone of
// the dynamic layout; 8 neighbouring chunks of the uniform one; the last
// group of a head may be smaller, always even).  Every perfect matching of the
// group is scored by the summed list overlap |A n B| of its pairs, and the
// best one (lowest matching index on ties) is taken: the paired kernels walk
// |A u B| = |A| + |B| - |A n B| list entries per pair, so the best matching
// has the fewest idle wave slots.  Matching m of g rows: the first free row
// pairs with the (m mod (g-1))-th other free row, then m /= (g-1), and so on.
constexpr int kGroup = 8;
constexpr int kPairWin = 8192;  // column tiles per bitmap window

__device__ __forceinline__ int num_matchings(int g) { return g == 8 ? 105 : g == 6 ? 15 : g == 4 ? 3 : 1; }

// rows of matching m of a group of g rows as pairs (pa[k], pb[k]), k < g/2,
// ordered by their first row
__device__ __forceinline__ void decode_matching(int m, int g, int* pa, int* pb) {
  int freel[kGroup];
  int nf = g;
  for (int i = 0; i < g; ++i) freel[i] = i;
  for (int k = 0; k < g / 2; ++k) {
    const int a = freel[0];
    const int c = m % (nf - 1);
    m /= (nf - 1);
    const int b = freel[1 + c];
    pa[k] = a;
    pb[k] = b;
    // remove positions 0 and 1 + c
    int w = 0;
    for (int i = 1; i < nf; ++i)
      if (i != 1 + c) freel[w++] = freel[i];
    nf -= 2;
  }
}

// one 256-thread workgroup per group of one head
__global__ __launch_bounds__(256) void pair_tiles_kernel(const int64_t* __restrict__ start,
                                                         const int32_t* __restrict__ len,
                                                         const int32_t* __restrict__ cols, int64_t Nr, int64_t Nc,
                                                         int64_t groups_per_head, int32_t* __restrict__ pairmap) {
  __shared__ uint32_t bm[kGroup][kPairWin / 32];
  __shared__ uint32_t inter[kGroup][kGroup];
  __shared__ uint64_t best_key;
  const int tid = threadIdx.x;
  const int64_t hd = blockIdx.x / groups_per_head, grp = blockIdx.x - hd * groups_per_head;
  const int64_t r0 = grp * kGroup;
  const int g = (int)(Nr - r0 < kGroup ? Nr - r0 : kGroup);
  if (tid < kGroup * kGroup) inter[tid / kGroup][tid % kGroup] = 0u;
  if (tid == 0) best_key = 0ull;
  for (int64_t w0 = 0; w0 < Nc; w0 += kPairWin) {
    for (int i = tid; i < kGroup * (kPairWin / 32); i += 256) (&bm[0][0])[i] = 0u;
    __syncthreads();
    for (int r = 0; r < g; ++r) {
      const int64_t row = hd * Nr + r0 + r;
      const int32_t* A = cols + start[row];
      const int n = len[row];
      for (int i = tid; i < n; i += 256) {
        const int64_t t = (int64_t)A[i] - w0;
        if (t >= 0 && t < kPairWin && A[i] < Nc) atomicOr(&bm[r][t >> 5], 1u << (t & 31));
      }
    }
    __syncthreads();
    // |A_a n A_b| for a < b: thread tid takes words tid, tid + 256
    for (int a = 0; a < g; ++a)
      for (int b = a + 1; b < g; ++b) {
        uint32_t c = 0;
        for (int i = tid; i < kPairWin / 32; i += 256) c += __popc(bm[a][i] & bm[b][i]);
        c = wave_sum_u32(c);
        if ((tid & 63) == 0 && c) atomicAdd(&inter[a][b], c);
      }
    __syncthreads();
  }
  const int nm = num_matchings(g);
  int pa[kGroup / 2], pb[kGroup / 2];
  if (tid < nm) {
    decode_matching(tid, g, pa, pb);
    uint32_t total = 0;
    for (int k = 0; k < g / 2; ++k) total += inter[pa[k]][pb[k]];
    // larger overlap first, then the lower matching index
    atomicMax((unsigned long long*)&best_key, ((uint64_t)total << 8) | (uint64_t)(255 - tid));
  }
  __syncthreads();
  if (tid == 0) {
    const int m = 255 - (int)(best_key & 255ull);
    decode_matching(m, g, pa, pb);
    int32_t* out = pairmap + hd * Nr + r0;
    for (int k = 0; k < g / 2; ++k) {
      out[2 * k] = (int32_t)(r0 + pa[k]);
      out[2 * k + 1] = (int32_t)(r0 + pb[k]);
    }
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

// ------------------------------------------------------------------ launch order
// Workgroup id -> pair of the attention launches.  Ids [0, n - T) keep the
// XCD group mapping (xcd_group_remap<G>); the last T ids take the pairs that
// mapping would give them, longest work list first, so the launch ends on
// short workgroups instead of waiting for long ones started last.
constexpr int kOrderMax = 16384;  // largest sorted tail (one workgroup, LDS bitonic sort, 128 KB)

__device__ __forceinline__ int group_remap_rt(int bid, int n, int G) {
  const int full = n / (8 * G) * (8 * G);
  if (bid >= full) return bid;
  const int chunk = bid / (8 * G), xcd = bid & 7, slot = (bid >> 3) % G;
  return chunk * 8 * G + xcd * G + slot;
}

__global__ __launch_bounds__(1024) void pair_order_kernel(const int32_t* __restrict__ ulen, int n, int G, int T,
                                                          int P2, int32_t* __restrict__ order) {
  __shared__ uint64_t key[kOrderMax];  // (~len << 32) | pair: ascending = longest first, then lower pair
  const int k = n - T;
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < k; p += gridDim.x * blockDim.x)
    order[p] = group_remap_rt(p, n, G);
  if (blockIdx.x != 0) return;
  for (int i = threadIdx.x; i < P2; i += blockDim.x) {
    uint64_t v = ~0ull;
    if (i < T) {
      const int pair = group_remap_rt(k + i, n, G);
      v = ((uint64_t)(0xffffffffu - (uint32_t)ulen[pair]) << 32) | (uint32_t)pair;
    }
    key[i] = v;
  }
  __syncthreads();
  for (int size = 2; size <= P2; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < P2; i += blockDim.x) {
        const int j = i ^ stride;
        if (j > i) {
          const bool up = (i & size) == 0;
          const uint64_t x = key[i], y = key[j];
          if ((x > y) == up) {
            key[i] = y;
            key[j] = x;
          }
        }
      }
      __syncthreads();
    }
  for (int i = threadIdx.x; i < T; i += blockDim.x) order[k + i] = (int32_t)(key[i] & 0xffffffffu);
}

// ------------------------------------------------------------------ compact CSR
// offsets[r] = sum of len[0..r) as int32, *total = the int64 sum (so the
// caller can reject a total past int32).  One workgroup: thread t sums a
// contiguous chunk of rows, a block scan places the chunks.
constexpr int kCsrThreads = 1024;

__global__ __launch_bounds__(kCsrThreads) void csr_offsets_kernel(const int32_t* __restrict__ len, int64_t rows,
                                                                  int32_t* __restrict__ offsets,
                                                                  int64_t* __restrict__ total) {
  __shared__ int64_t wsum[kCsrThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t chunk = (rows + kCsrThreads - 1) / kCsrThreads;
  const int64_t r0 = (int64_t)tid * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
  int64_t part = 0;
  for (int64_t r = r0; r < r1; ++r) part += len[r] > 0 ? len[r] : 0;
  // inclusive scan of the 64-bit chunk sums over the workgroup
  int64_t incl = part;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = __shfl_up((uint32_t)incl, off, 64);
    const uint32_t hi = __shfl_up((uint32_t)((uint64_t)incl >> 32), off, 64);
    if (lane >= off) incl += (int64_t)(((uint64_t)hi << 32) | lo);
  }
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  int64_t before = 0, all = 0;
  for (int v = 0; v < kCsrThreads / 64; ++v) {
    before += v < wid ? wsum[v] : 0;
    all += wsum[v];
  }
  int64_t run = before + incl - part;
  for (int64_t r = r0; r < r1; ++r) {
    offsets[r] = (int32_t)run;
    run += len[r] > 0 ? len[r] : 0;
  }
  if (tid == 0) {
    offsets[rows] = (int32_t)all;
    *total = all;
  }
}

// one wave per row: row r's len[r] entries from cols + start[r] to
// out + offsets[r]
__global__ __launch_bounds__(256) void csr_fill_kernel(const int64_t* __restrict__ start,
                                                       const int32_t* __restrict__ len,
                                                       const int32_t* __restrict__ cols, int64_t rows,
                                                       const int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const int32_t n = len[r];
  const int32_t* src = cols + start[r];
  int32_t* dst = out + offsets[r];
  for (int32_t i = lane; i < n; i += 64) dst[i] = src[i];
}

}  // namespace

extern "C" {

int prism_lists_csr_offsets(const int32_t* len, int64_t rows, int32_t* offsets, int64_t* total,
                            hipStream_t stream) {
  PRISM_REQUIRE(offsets && total && (len || rows == 0), "prism_lists_csr_offsets: null pointer");
  PRISM_REQUIRE(rows >= 0, "prism_lists_csr_offsets: negative row count");
  csr_offsets_kernel<<<1, kCsrThreads, 0, stream>>>(len, rows, offsets, total);
  PRISM_LAUNCH_CHECK("prism_lists_csr_offsets");
  return PRISM_OK;
}

int prism_lists_csr_fill(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows,
                         const int32_t* offsets, int32_t* out_cols, hipStream_t stream) {
  PRISM_REQUIRE(rows >= 0 && rows < (1ll << 33), "prism_lists_csr_fill: row count out of range");
  if (rows == 0) return PRISM_OK;
  PRISM_REQUIRE(start && len && cols && offsets && out_cols, "prism_lists_csr_fill: null pointer");
  csr_fill_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, stream>>>(start, len, cols, rows, offsets, out_cols);
  PRISM_LAUNCH_CHECK("prism_lists_csr_fill");
  return PRISM_OK;
}

int prism_pair_union(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, const int32_t* pairmap, const uint64_t* tile_masks, int64_t ucap,
                     int64_t* ustart, int32_t* ulen, int32_t* ucols, hipStream_t stream) {
  PRISM_REQUIRE(start && len && cols && ustart && ulen && ucols, "prism_pair_union: null pointer");
  PRISM_REQUIRE(rows >= 0 && rows % 2 == 0, "prism_pair_union: rows must be even (pairs of tiles)");
  PRISM_REQUIRE(row_tiles > 0 && row_tiles % 2 == 0 && rows % row_tiles == 0,
                "prism_pair_union: rows must be a multiple of an even row_tiles (tiles per head)");
  PRISM_REQUIRE(col_tiles > 0 && col_tiles < (1ll << 28), "prism_pair_union: col_tiles out of range");
  PRISM_REQUIRE(ucap >= col_tiles, "prism_pair_union: ucap must be >= col_tiles");
  const int64_t pairs = rows / 2;
  if (pairs == 0) return PRISM_OK;
  PRISM_REQUIRE(pairs < (1ll << 31), "prism_pair_union: too many pairs");
  if (prism_debug_enabled()) {
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_pair_union", start, len, cols, rows, col_tiles, 0, nullptr,
                                              stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_pair_union", pairmap, rows / row_tiles, row_tiles, nullptr, 0,
                                             stream));
  }
  pair_union_kernel<2><<<(unsigned)pairs, 256, 0, stream>>>(start, len, cols, row_tiles, col_tiles, pairmap, tile_masks,
                                                             ucap, ustart, ulen, ucols);
  PRISM_LAUNCH_CHECK("prism_pair_union");
  return PRISM_OK;
}

int prism_quad_union(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, const int32_t* pairmap, const uint64_t* tile_masks, int64_t ucap,
                     int64_t* ustart, int32_t* ulen, int32_t* ucols, hipStream_t stream) {
  PRISM_REQUIRE(start && len && cols && ustart && ulen && ucols, "prism_quad_union: null pointer");
  PRISM_REQUIRE(rows >= 0 && rows % 4 == 0, "prism_quad_union: rows must be a multiple of 4 (quads of tiles)");
  PRISM_REQUIRE(row_tiles > 0 && row_tiles % 4 == 0 && rows % row_tiles == 0,
                "prism_quad_union: rows must be a multiple of row_tiles (tiles per head), itself a multiple of 4");
  PRISM_REQUIRE(col_tiles > 0 && col_tiles < (1ll << 26), "prism_quad_union: col_tiles out of range");
  PRISM_REQUIRE(ucap >= col_tiles, "prism_quad_union: ucap must be >= col_tiles");
  const int64_t quads = rows / 4;
  if (quads == 0) return PRISM_OK;
  PRISM_REQUIRE(quads < (1ll << 31), "prism_quad_union: too many quads");
  if (prism_debug_enabled()) {
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_quad_union", start, len, cols, rows, col_tiles, 0, nullptr,
                                              stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_quad_union", pairmap, rows / row_tiles, row_tiles, nullptr, 0,
                                             stream));
  }
  pair_union_kernel<4><<<(unsigned)quads, 256, 0, stream>>>(start, len, cols, row_tiles, col_tiles, pairmap, tile_masks,
                                                              ucap, ustart, ulen, ucols);
  PRISM_LAUNCH_CHECK("prism_quad_union");
  return PRISM_OK;
}

int prism_pair_tiles(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, int32_t* pairmap, hipStream_t stream) {
  PRISM_REQUIRE(start && len && cols && pairmap, "prism_pair_tiles: null pointer");
  PRISM_REQUIRE(row_tiles > 0 && row_tiles % 2 == 0 && rows % row_tiles == 0,
                "prism_pair_tiles: rows must be a multiple of an even row_tiles (tiles per head)");
  PRISM_REQUIRE(col_tiles > 0 && col_tiles < (1ll << 30), "prism_pair_tiles: col_tiles out of range");
  if (rows == 0) return PRISM_OK;
  const int64_t groups = (row_tiles + kGroup - 1) / kGroup;
  const int64_t blocks = rows / row_tiles * groups;
  PRISM_REQUIRE(blocks < (1ll << 31), "prism_pair_tiles: too many groups");
  pair_tiles_kernel<<<(unsigned)blocks, 256, 0, stream>>>(start, len, cols, row_tiles, col_tiles, groups, pairmap);
  PRISM_LAUNCH_CHECK("prism_pair_tiles");
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

int prism_pair_order(const int32_t* ulen, int64_t n, int G, int64_t tail, int32_t* order, hipStream_t stream) {
  PRISM_REQUIRE(ulen && order, "prism_pair_order: null pointer");
  PRISM_REQUIRE(n >= 1 && n < (1ll << 31), "prism_pair_order: n out of range");
  PRISM_REQUIRE(G == 32 || G == 64, "prism_pair_order: G must be the attention kernels' group (32 or 64)");
  PRISM_REQUIRE(tail >= 0 && tail <= n && tail <= kOrderMax, "prism_pair_order: tail must be in [0, min(n, %d)]",
                kOrderMax);
  int P2 = 1;
  while (P2 < tail) P2 <<= 1;
  const int64_t head = n - tail;
  const unsigned blocks = (unsigned)(head > 0 ? (head + 1023) / 1024 : 1);
  pair_order_kernel<<<blocks < 1 ? 1 : blocks, 1024, 0, stream>>>(ulen, (int)n, G, (int)tail, P2, order);
  PRISM_LAUNCH_CHECK("prism_pair_order");
  return PRISM_OK;
}

}  // extern "C"
