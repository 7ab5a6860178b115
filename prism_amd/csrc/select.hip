// Block scores, hybrid top-k / cumulative-threshold selection, tile lists and
// their transpose (gfx950).
//
// Reference (hymm/models/modules/block_sparse_attention/):
//   block_scores_kernel  cal_score (bsa_interface.py:203-207) + invalid-key fill
//                        (dynamic_block_attention.py:276-279), fp32 out
//   select_rows_kernel   get_select_indices_topk_from_score (bsa_interface.py:235-248),
//   (select_kernel,      get_select_indices_cdf_from_score (:257-275),
//    select_wide_kernel) get_select_indices_cdf_topk_from_score (:284-304),
//                        fused with the block -> tile expansion
//                        (dynamic_block_attention.py:297-319); one wave per
//                        row up to 6,144 blocks, one workgroup per row beyond
//   tile_rows_kernel     q-tile rows share their q-block's list (:315-318)
//   transpose kernels    create_indices_k_from_indices_q_varlen (bsa_interface.py:147-161)
//                        as a bitmap transpose instead of a dense N_tiles^2 mask + sort
//                        (prism_transpose_lists_noalloc: the same kernels with the
//                        bitmap in a file-scope device workspace)
//
// Canonical arithmetic (compiled with -ffp-contract=off):
//   score   = fmaf chain over d ascending, from +0;
//   softmax = e_j = canon_exp(s_j*scale - max), sum = fl32(sum_j floor(e_j 2^40)) 2^-40,
//             w_j = e_j / sum;
//   cdf     = exact fixed-point prefix sums of floor(w 2^60) in (w desc, index asc)
//             order; "cdf < p" <=> prefix < thr (thr from the host).
// The selection never sorts: the crossing element is found by a radix search
// (four 8-bit digits, LDS histograms) on the fp32 bit pattern of w
// (order-preserving for w >= 0) with exact integer sums, so the result does
// not depend on thread order.
#include <mutex>

#include "common.h"

namespace {

// ------------------------------------------------------------------ scores
constexpr int kSTile = 128, kSChunk = 16;

__global__ __launch_bounds__(256) void block_scores_kernel(const float* __restrict__ qc, const float* __restrict__ kc,
                                                           const int32_t* __restrict__ block_count, int64_t Nq,
                                                           int64_t Nk, int D, float* __restrict__ scores) {
  __shared__ float sA[kSChunk][kSTile + 4];
  __shared__ float sB[kSChunk][kSTile + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t i0 = (int64_t)blockIdx.y * kSTile, j0 = (int64_t)blockIdx.x * kSTile;
  const int bh = blockIdx.z;
  const float* A = qc + (int64_t)bh * Nq * D;
  const float* Bm = kc + (int64_t)bh * Nk * D;
  float acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;

  for (int d0 = 0; d0 < D; d0 += kSChunk) {
    // 128 rows x 16 cols = 512 float4 per operand; 2 per thread
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int idx = tid + u * 256;
      const int row = idx >> 2, c4 = (idx & 3) * 4;
      float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
      if (i0 + row < Nq) va = *reinterpret_cast<const float4*>(A + (i0 + row) * D + d0 + c4);
      if (j0 + row < Nk) vb = *reinterpret_cast<const float4*>(Bm + (j0 + row) * D + d0 + c4);
      sA[c4 + 0][row] = va.x; sA[c4 + 1][row] = va.y; sA[c4 + 2][row] = va.z; sA[c4 + 3][row] = va.w;
      sB[c4 + 0][row] = vb.x; sB[c4 + 1][row] = vb.y; sB[c4 + 2][row] = vb.z; sB[c4 + 3][row] = vb.w;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kSChunk; ++kk) {
      float a[8], b[8];
      const float4 a0 = *reinterpret_cast<const float4*>(&sA[kk][ty * 8]);
      const float4 a1 = *reinterpret_cast<const float4*>(&sA[kk][ty * 8 + 4]);
      const float4 b0 = *reinterpret_cast<const float4*>(&sB[kk][tx * 8]);
      const float4 b1 = *reinterpret_cast<const float4*>(&sB[kk][tx * 8 + 4]);
      a[0] = a0.x; a[1] = a0.y; a[2] = a0.z; a[3] = a0.w; a[4] = a1.x; a[5] = a1.y; a[6] = a1.z; a[7] = a1.w;
      b[0] = b0.x; b[1] = b0.y; b[2] = b0.z; b[3] = b0.w; b[4] = b1.x; b[5] = b1.y; b[6] = b1.z; b[7] = b1.w;
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  const float ninf = -__uint_as_float(0x7f800000u);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = i0 + ty * 8 + i;
    if (row >= Nq) continue;
    float* out = scores + ((int64_t)bh * Nq + row) * Nk;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t col = j0 + tx * 8 + j;
      if (col < Nk) out[col] = (block_count && block_count[col] == 0) ? ninf : acc[i][j];
    }
  }
}

// ------------------------------------------------------------------ block-wide helpers (256 threads)
constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / 64;

template <int NW>
struct SelSharedT {
  uint64_t u64[NW];
  uint32_t u32[NW];
  float f32[NW];
};
using SelShared = SelSharedT<kSelWaves>;

// Workgroup reductions and scans over NW waves; every thread gets the result.
template <int NW>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, SelSharedT<NW>& sh) {
  v = wave_sum_u64(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sh.u64[wid] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += sh.u64[w];
  __syncthreads();
  return t;
}
template <int NW>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, SelSharedT<NW>& sh) {
  v = wave_sum_u32(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sh.u32[wid] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += sh.u32[w];
  __syncthreads();
  return t;
}
template <int NW>
__device__ __forceinline__ float block_max_f32(float v, SelSharedT<NW>& sh) {
  v = wave_max_xor(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sh.f32[wid] = v;
  __syncthreads();
  float t = sh.f32[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) t = fmaxf(t, sh.f32[w]);
  __syncthreads();
  return t;
}
// exclusive scan in thread order; returns the block total in *total
template <int NW>
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, SelSharedT<NW>& sh, uint32_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan_u32(v, lane);
  if (lane == 63) sh.u32[wid] = incl;
  __syncthreads();
  uint32_t before = 0, t = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint32_t x = sh.u32[w];
    before += (w < wid) ? x : 0u;
    t += x;
  }
  __syncthreads();
  *total = t;
  return before + incl - v;
}
template <int NW>
__device__ __forceinline__ uint64_t block_excl_scan_u64(uint64_t v, SelSharedT<NW>& sh, uint64_t* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint64_t incl = v;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = __shfl_up((uint32_t)incl, off, 64);
    const uint32_t hi = __shfl_up((uint32_t)(incl >> 32), off, 64);
    if (lane >= off) incl += ((uint64_t)hi << 32) | lo;
  }
  if (lane == 63) sh.u64[wid] = incl;
  __syncthreads();
  uint64_t before = 0, t = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint64_t x = sh.u64[w];
    before += (w < wid) ? x : 0ull;
    t += x;
  }
  __syncthreads();
  *total = t;
  return before + incl - v;
}

// Wave 0's step of a radix digit: given the histogram hb of the elements that
// match the digits found so far and acc, the weight of the keys whose decided
// digits exceed them, find the largest digit d* whose suffix sum reaches
// thr - acc; sh.u64[0] = weight of the digits above d*, sh.u32[0] = 255 - d*.
// Also clears hn, the histogram buffer of the next digit.
template <int NW>
__device__ __forceinline__ void radix_pick(const unsigned long long* hb, unsigned long long* hn, uint64_t acc,
                                           uint64_t thr, SelSharedT<NW>& sh, int lane) {
  // lane l takes digits 255 - 4 l - i (i = 0..3): inclusive sums over the
  // descending digits; the first t = 4 l + i with acc + incl >= thr is d*
  uint64_t h[4], p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = hb[255 - 4 * lane - i];
  p[0] = h[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) p[i] = p[i - 1] + h[i];
  uint64_t incl = p[3];
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = __shfl_up((uint32_t)incl, off, 64);
    const uint32_t hi = __shfl_up((uint32_t)(incl >> 32), off, 64);
    if (lane >= off) incl += ((uint64_t)hi << 32) | lo;
  }
  const uint64_t base = incl - p[3];
  uint32_t below = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) below += acc + base + p[i] >= thr ? 0u : 1u;
  const uint32_t tstar = min(wave_sum_u32(below), 255u);  // (<= 255: the bins hold >= thr - acc)
  if ((uint32_t)lane == (tstar >> 2)) {
    const int slot = (int)(tstar & 3);
    sh.u64[0] = base + (slot == 0 ? 0ull : slot == 1 ? p[0] : slot == 2 ? p[1] : p[2]);  // weight of digits > d*
    sh.u32[0] = tstar;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) hn[4 * lane + i] = 0ull;
}

// The cdf weight of a key: floor(w 2^60) of the softmax weight w whose fp32
// bits the key is (recomputed where used instead of held beside the key: the
// row kernel then needs 48 fewer VGPRs and keeps more workgroups resident)
__device__ __forceinline__ uint64_t weight_of(uint32_t key) { return fixp(__uint_as_float(key), 60); }

// Radix search over the 32-bit keys of one row (4 digits of 8 bits, most
// significant first): the largest v with S(v) >= thr, where S(v) is the sum
// of wt over present elements with key >= v (wt = weight_of(key[e]), or 1 to count), for
// 0 < thr <= S(0).  *above = S(v + 1), the weight strictly above v.  The
// sums are exact integers, so v is the same as a bisection on S would find.
// Per digit: an LDS histogram of wt over the elements that match the digits
// found so far, then wave 0 alone scans the 256 bins from the top digit down
// and finds the largest digit whose suffix reaches thr, and clears the other
// histogram buffer for the next digit (two buffers alternate), so a digit
// costs two workgroup barriers.  hist: [2][256], buffer 0 zero on entry (and
// again on return).
template <int EPT, bool WEIGHTED>
__device__ __forceinline__ uint32_t radix_search(const uint32_t* key, uint64_t present, uint64_t thr,
                                                 uint64_t* above, SelShared& sh, unsigned long long* hist) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0;
  uint64_t acc = 0;  // weight of keys whose decided digits exceed the prefix
#pragma unroll 1
  for (int level = 0; level < 4; ++level) {
    const int shift = 24 - 8 * level;
    const uint32_t hmask = level == 0 ? 0u : (0xffffffffu << (shift + 8));
    unsigned long long* hb = hist + 256 * (level & 1);
    // A thread's elements are neighbouring blocks, whose weights mostly share
    // a digit (at the first level, all of a row's weights share one or two
    // exponent bytes): runs of one digit are summed in registers and added
    // with one LDS atomic, instead of one atomic per element on the same
    // few bins.  Integer sums, so the histogram is the same.
    uint32_t run_bin = 0xffffffffu;
    uint64_t run_w = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (((present >> e) & 1) && (key[e] & hmask) == prefix) {
        const uint32_t b = (key[e] >> shift) & 255u;
        const uint64_t w = WEIGHTED ? weight_of(key[e]) : 1ull;
        if (b != run_bin) {
          if (run_bin != 0xffffffffu) atomicAdd(&hb[run_bin], (unsigned long long)run_w);
          run_bin = b;
          run_w = 0;
        }
        run_w += w;
      }
    if (run_bin != 0xffffffffu) atomicAdd(&hb[run_bin], (unsigned long long)run_w);
    __syncthreads();
    if (tid < 64) radix_pick(hb, hist + 256 * ((level + 1) & 1), acc, thr, sh, lane);
    __syncthreads();
    acc += sh.u64[0];
    prefix |= (255u - sh.u32[0]) << shift;
  }
  *above = acc;
  return prefix;
}

struct SelArgs {
  const float* scores;            // [rows, N]
  int64_t rows, N;
  int mode;                       // 0 top-k, 1 cdf, 2 cdf + top-k
  int64_t k_lo, ub;
  float scale;
  uint64_t thr;
  const int32_t* block_first_tile;  // [N+1]
  const int32_t* tile_count;        // [Nt] or null (no padded-tile filtering)
  int64_t tcap;
  int32_t* tiles;                 // [rows, tcap]
  int32_t* ntiles;                // [rows]
  int32_t* sel_blocks;            // [rows, bcap] or null
  int64_t bcap;
  int32_t* nsel;                  // [rows] or null
};

// One workgroup per row; element j lives in thread j / EPT, slot j % EPT.
template <int EPT>
__global__ __launch_bounds__(kSelThreads, EPT <= 24 ? 4 : 1) void select_kernel(SelArgs a) {
  static_assert(kSelThreads == 256, "one radix bin per thread");
  __shared__ SelShared sh;
  __shared__ unsigned long long hist[2 * 256];
  const int tid = threadIdx.x;
  hist[tid] = 0ull;  // buffer 0 of the radix searches
  __syncthreads();
  const int64_t row = blockIdx.x;
  const float* s = a.scores + row * a.N;
  const int64_t N = a.N;

  const int64_t j0 = (int64_t)tid * EPT;

  uint32_t key[EPT];
  uint64_t present = 0;  // bit e: slot e holds a real element
  int64_t eff = 0;
  uint32_t v_e = 0;
  uint64_t need = 0;

  if (a.mode == 0) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int64_t j = (int64_t)tid * EPT + e;
      key[e] = 0;
      if (j < N) {
        const uint32_t u = __float_as_uint(s[j]);
        key[e] = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        present |= 1ull << e;
      }
    }
    eff = a.k_lo < N ? a.k_lo : N;
  } else {
    float x[EPT];
    float m = -__uint_as_float(0x7f800000u);
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int64_t j = (int64_t)tid * EPT + e;
      x[e] = m;
      if (j < N) {
        x[e] = s[j] * a.scale;
        m = fmaxf(m, x[e]);
        present |= 1ull << e;
      }
    }
    m = block_max_f32(m, sh);
    if (m == -__uint_as_float(0x7f800000u)) {
      eff = 0;
    } else {
      uint64_t E = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        x[e] = ((present >> e) & 1) ? canon_exp(x[e] - m) : 0.0f;
        E += fixp(x[e], 40);
      }
      E = block_sum_u64(E, sh);
      const float sum = (float)E * 9.094947017729282e-13f;  // 2^-40
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const float w = ((present >> e) & 1) ? x[e] / sum : 0.0f;
        key[e] = __float_as_uint(w);
      }
      // G(v) = sum of W over present elements with key >= v
      auto G = [&](uint32_t v) {
        uint64_t t = 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) t += (((present >> e) & 1) && key[e] >= v) ? weight_of(key[e]) : 0ull;
        return block_sum_u64(t, sh);
      };
      auto Nge = [&](uint32_t v) {
        uint32_t t = 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) t += (((present >> e) & 1) && key[e] >= v) ? 1u : 0u;
        return block_sum_u32(t, sh);
      };
      int64_t c = a.ub;
      bool crossed = false;
      uint32_t vc = 0;
      uint64_t jt = 0;
      if (G(0) >= a.thr) {
        // crossing value vc: G(vc) >= thr > G(vc + 1) = A
        uint64_t A;
        vc = radix_search<EPT, true>(key, present, a.thr, &A, sh, hist);
        const uint32_t ngt = Nge(vc + 1);
        const uint64_t Wv = fixp(__uint_as_float(vc), 60);
        jt = (a.thr - A - 1) / Wv;  // smallest j with A + (j+1) Wv >= thr
        const int64_t k = (int64_t)ngt + (int64_t)jt;
        if (k < a.ub) { c = k; crossed = true; }
      }
      int64_t n = c + 1;
      if (n < a.k_lo) n = a.k_lo;
      if (n > N) n = N;
      eff = n < a.ub ? n : a.ub;
      if (crossed && eff == c + 1) {
        v_e = vc;
        need = jt + 1;
        eff = -eff;  // marks "v_e already known"
      }
    }
  }

  if (eff > 0) {  // count search: largest v with #(key >= v) >= eff (eff <= #present)
    uint64_t above;
    v_e = radix_search<EPT, false>(key, present, (uint64_t)eff, &above, sh, hist);
    need = (uint64_t)eff - above;
  } else {
    eff = -eff;
  }

  // emit selected blocks in ascending index order, expanded to tiles.  Thread
  // t owns blocks [t EPT, t EPT + EPT), so one scan of per-thread tie counts
  // ranks the ties and one scan of per-thread output counts places the lists.
  int32_t* trow = a.tiles + row * a.tcap;
  int32_t* brow = a.sel_blocks ? a.sel_blocks + row * a.bcap : nullptr;
  uint32_t nties = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) nties += (eff > 0 && ((present >> e) & 1) && key[e] == v_e) ? 1u : 0u;
  uint32_t tot;
  uint32_t rank = block_excl_scan_u32(nties, sh, &tot);
  uint64_t selm = 0;  // bit e: block j0 + e is selected
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const bool pres = (present >> e) & 1;
    const bool tie = eff > 0 && pres && key[e] == v_e;
    const bool sel = eff > 0 && pres && (key[e] > v_e || (tie && rank < need));
    rank += tie ? 1u : 0u;
    selm |= sel ? 1ull << e : 0ull;
  }
  // tiles of the selected blocks: all first-tile entries are read at once,
  // then the tile counts of the selected blocks' tiles (two round trips, not
  // two per selected block); bit e of ok0m / ok1m: the first / second tile
  // of block e is listed, of bigm: block e has more than two tiles (counted
  // by a loop)
  int32_t fb[EPT + 1];
#pragma unroll
  for (int e = 0; e <= EPT; ++e) {
    // (first tile of a selected block e, or end of a selected block e - 1)
    const bool need = (e < EPT && ((selm >> e) & 1)) || (e > 0 && ((selm >> (e - 1)) & 1));
    fb[e] = need ? a.block_first_tile[j0 + e] : 0;
  }
  uint64_t ok0m = 0, ok1m = 0, bigm = 0;
  uint64_t packed = 0;  // tiles | blocks << 32 of this thread (32-bit fields: a row may hold any tile count)
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if ((selm >> e) & 1) {
      const int32_t t0 = fb[e], nt = fb[e + 1] - t0;
      uint32_t cnt;
      if (nt <= 2) {
        const bool ok0 = nt >= 1 && (a.tile_count == nullptr || a.tile_count[t0] > 0);
        const bool ok1 = nt >= 2 && (a.tile_count == nullptr || a.tile_count[t0 + 1] > 0);
        ok0m |= ok0 ? 1ull << e : 0ull;
        ok1m |= ok1 ? 1ull << e : 0ull;
        cnt = (ok0 ? 1u : 0u) + (ok1 ? 1u : 0u);
      } else {
        bigm |= 1ull << e;
        cnt = 0;
        for (int32_t t = t0; t < t0 + nt; ++t) cnt += (a.tile_count == nullptr || a.tile_count[t] > 0) ? 1u : 0u;
      }
      packed += (uint64_t)cnt | (1ull << 32);
    }
  }
  uint64_t tot64;
  const uint64_t pos = block_excl_scan_u64(packed, sh, &tot64);
  int64_t p = (int64_t)(pos & 0xffffffffu), q = (int64_t)(pos >> 32);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if ((selm >> e) & 1) {
      const int32_t t0 = fb[e];
      if (!((bigm >> e) & 1)) {
        if ((ok0m >> e) & 1) {
          if (p < a.tcap) trow[p] = t0;
          ++p;
        }
        if ((ok1m >> e) & 1) {
          if (p < a.tcap) trow[p] = t0 + 1;
          ++p;
        }
      } else {
        for (int32_t t = t0; t < fb[e + 1]; ++t)
          if (a.tile_count == nullptr || a.tile_count[t] > 0) {
            if (p < a.tcap) trow[p] = t;
            ++p;
          }
      }
      if (brow && q < a.bcap) brow[q] = (int32_t)(j0 + e);
      ++q;
    }
  }
  if (tid == 0) {
    a.ntiles[row] = (int32_t)(tot64 & 0xffffffffu);
    if (a.nsel) a.nsel[row] = (int32_t)(tot64 >> 32);
  }
}

// ------------------------------------------------------------ one wave per row
// Rows of up to kWaveMaxN blocks: one wave per row, kWaveRows rows per
// workgroup.  Element j lives in lane j % 64, slot j / 64 (coalesced loads;
// slot order is ascending block order, so ballots rank the ties and place the
// outputs).  After the workgroup's set-up there is no workgroup barrier: each
// wave runs its row's chain on its own, and the waves of other rows hide its
// latency (the 256-thread row kernel waits at about twenty barriers per row).
// The arithmetic is select_kernel's (same canonical exp, division and exact
// integer sums), so the selection is identical.  LDS per workgroup: the tile
// flags of every block, built once for the workgroup's rows, and a pair of
// 256-bin histograms per wave.
constexpr int kWaveRows = 4;
constexpr int kWaveMaxN = 6144;

// tile flags of block j: first tile << 3 | second tile listed << 1 | first
// tile listed for blocks of at most two tiles; kBigBlock for others (their
// tiles are counted from block_first_tile in the emit)
constexpr int32_t kBigBlock = 4;

__device__ __forceinline__ int32_t block_tile_flags(const int32_t* first, const int32_t* tile_count, int64_t j) {
  const int32_t f0 = first[j], nt = first[j + 1] - f0;
  if (nt > 2 || nt < 0 || f0 < 0 || f0 >= (1 << 28)) return kBigBlock;
  const bool ok0 = nt >= 1 && (tile_count == nullptr || tile_count[f0] > 0);
  const bool ok1 = nt >= 2 && (tile_count == nullptr || tile_count[f0 + 1] > 0);
  return (f0 << 3) | (ok1 ? 2 : 0) | (ok0 ? 1 : 0);
}

// canon_exp and fixp without branches: the same operations for every input
// in range, the special cases selected at the end (per-slot branch nests
// otherwise serialise the unrolled slots of a lane)
__device__ __forceinline__ float canon_exp_nb(float x) {
#pragma clang fp contract(off)
  const float xc = fminf(fmaxf(x, -87.0f), 88.0f);  // == x wherever the result is computed
  const float t = xc * 1.44269504f;
  const float n = floorf(t + 0.5f);
  float r = __builtin_fmaf(-n, 0.693359375f, xc);
  r = __builtin_fmaf(-n, -2.12194440e-4f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float v = p * __uint_as_float((uint32_t)((int)n + 127) << 23);
  return x != x ? x : x > 88.0f ? __uint_as_float(0x7f800000u) : x < -87.0f ? 0.0f : v;
}
__device__ __forceinline__ uint64_t fixp_nb(float w, int F) {
  const uint32_t u = __float_as_uint(w);
  const int e8 = (int)((u >> 23) & 0xffu);
  const uint64_t m = (u & 0x7fffffu) | (e8 != 0 ? 0x800000u : 0u);
  const int sh = (e8 != 0 ? e8 : 1) - 150 + F;
  const uint64_t left = m << (sh > 0 ? (sh < 63 ? sh : 63) : 0);
  const uint64_t right = sh <= -64 ? 0ull : m >> (-sh > 0 ? -sh : 0);
  return sh >= 0 ? left : right;
}
__device__ __forceinline__ uint64_t weight_of_nb(uint32_t key) { return fixp_nb(__uint_as_float(key), 60); }

// 64-lane reductions and scans through DPP row operations (VALU latency, no
// LDS round trips): rows of 16 lanes by row_shr 1, 2, 4, 8, then the rows
// joined by row_bcast15 (rows 1, 3) and row_bcast31 (rows 2, 3)
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_zero(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xf, true);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t dpp_add_u64(uint64_t v) {
  const uint32_t lo = dpp_zero<CTRL, ROWS>((uint32_t)v), hi = dpp_zero<CTRL, ROWS>((uint32_t)(v >> 32));
  return v + (((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64_dpp(uint64_t v) {
  v = dpp_add_u64<0x111, 0xf>(v);
  v = dpp_add_u64<0x112, 0xf>(v);
  v = dpp_add_u64<0x114, 0xf>(v);
  v = dpp_add_u64<0x118, 0xf>(v);
  v = dpp_add_u64<0x142, 0xa>(v);
  v = dpp_add_u64<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32_dpp(uint32_t v) {
  v += dpp_zero<0x111, 0xf>(v);
  v += dpp_zero<0x112, 0xf>(v);
  v += dpp_zero<0x114, 0xf>(v);
  v += dpp_zero<0x118, 0xf>(v);
  v += dpp_zero<0x142, 0xa>(v);
  v += dpp_zero<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64_dpp(uint64_t v) {
  const uint64_t s = wave_incl_scan_u64_dpp(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)s, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(s >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t wave_sum_u32_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan_u32_dpp(v), 63);
}
// max over the 64 lanes (lanes whose DPP source is out of range keep their own value)
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_max(float v) {
  return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xf,
                                                            false)));
}
__device__ __forceinline__ float wave_max_f32_dpp(float v) {
  v = dpp_max<0x111, 0xf>(v);
  v = dpp_max<0x112, 0xf>(v);
  v = dpp_max<0x114, 0xf>(v);
  v = dpp_max<0x118, 0xf>(v);
  v = dpp_max<0x142, 0xa>(v);
  v = dpp_max<0x143, 0xc>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// LDS accesses of one wave complete in issue order; this keeps the compiler
// from moving them across the point
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// radix_search for one wave: the largest v with S(v) >= thr (S(v) = sum of wt
// over present elements with key >= v, wt = weight_of(key) or 1); *above =
// S(v + 1).  Returns false, with no search, when S(0) < thr (S(0) is the
// total of the first level's histogram).  hist: this wave's two 256-bin
// buffers, buffer 0 zero on entry and on return.
template <int EPL, bool WEIGHTED>
__device__ __forceinline__ bool wave_radix_search(uint32_t* key, int64_t N, int lane, uint64_t thr, uint32_t* value,
                                                  uint64_t* above, unsigned long long (*hist)[256]) {
  uint32_t prefix = 0;
  uint64_t acc = 0;
#pragma unroll 1
  for (int level = 0; level < 4; ++level) {
    // the keys are opaque to the compiler at each level, so the per-element
    // weights are recomputed where used instead of held across the levels
    // (2 EPL more registers)
#pragma unroll
    for (int e = 0; e < EPL; ++e) asm volatile("" : "+v"(key[e]));
    const int shift = 24 - 8 * level;
    const uint32_t hmask = level == 0 ? 0u : (0xffffffffu << (shift + 8));
    unsigned long long* hb = hist[level & 1];
    unsigned long long* hn = hist[(level + 1) & 1];
    int64_t lim = N - lane;  // slot e present: 64 e < lim (opaque: no predicate held across loops)
    asm volatile("" : "+v"(lim));
    // a lane's weights mostly share a digit (at the first level, all of a
    // row's weights share one or two exponent bytes): runs of one digit over
    // a lane's slots are summed in registers and added with one LDS atomic
    uint32_t run_bin = 0xffffffffu;
    uint64_t run_w = 0;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const bool hit = 64 * e < lim && (key[e] & hmask) == prefix;
      const uint32_t b = hit ? (key[e] >> shift) & 255u : run_bin;
      if (b != run_bin) {
        if (run_bin != 0xffffffffu) atomicAdd(&hb[run_bin], (unsigned long long)run_w);
        run_bin = b;
        run_w = 0;
      }
      run_w += hit ? (WEIGHTED ? weight_of_nb(key[e]) : 1ull) : 0ull;
    }
    if (run_bin != 0xffffffffu) atomicAdd(&hb[run_bin], (unsigned long long)run_w);
    wave_lds_order();
    // lane l takes digits 255 - 4 l - i: inclusive sums over the descending
    // digits; the first t = 4 l + i with acc + incl >= thr is d* = 255 - t
    uint64_t h[4], p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = hb[255 - 4 * lane - i];
    p[0] = h[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) p[i] = p[i - 1] + h[i];
    const uint64_t incl = wave_incl_scan_u64_dpp(p[3]);
    const uint64_t base = incl - p[3];
    if (level == 0) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)incl, 63);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(incl >> 32), 63);
      if ((((uint64_t)hi << 32) | lo) < thr) {  // S(0) < thr: no crossing
#pragma unroll
        for (int i = 0; i < 4; ++i) hb[4 * lane + i] = 0ull;
        wave_lds_order();
        return false;
      }
    }
    uint32_t below = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) below += acc + base + p[i] >= thr ? 0u : 1u;
    const int tstar = (int)min(wave_sum_u32_dpp(below), 255u);
    const int slot = tstar & 3;
    const uint64_t mine = base + (slot == 0 ? 0ull : slot == 1 ? p[0] : slot == 2 ? p[1] : p[2]);
    acc += readlane_u64(mine, tstar >> 2);  // weight of the digits above d*
#pragma unroll
    for (int i = 0; i < 4; ++i) hn[4 * lane + i] = 0ull;
    wave_lds_order();
    prefix |= (255u - (uint32_t)tstar) << shift;
  }
  *above = acc;
  *value = prefix;
  return true;
}

template <int EPL>
__global__ __launch_bounds__(64 * kWaveRows) void select_rows_kernel(SelArgs a) {
  static_assert(64 * EPL <= kWaveMaxN, "row too wide for the wave kernel");
  __shared__ int32_t flags[kWaveMaxN];
  __shared__ unsigned long long hist_all[kWaveRows][2][256];
  __shared__ uint64_t selm_all[kWaveRows][kWaveMaxN / 64];
  // the wave index in a scalar register: the row and its score pointer are
  // then scalar, and the score loads take a scalar base + 32-bit lane offset
  // (a 64-bit address per load and slot otherwise: 2 EPL registers)
  const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t N = a.N;
  for (int64_t j = tid; j < N; j += 64 * kWaveRows) flags[j] = block_tile_flags(a.block_first_tile, a.tile_count, j);
#pragma unroll
  for (int i = 0; i < 4; ++i) hist_all[wid][0][4 * lane + i] = 0ull;
  __syncthreads();
  const int64_t row = (int64_t)blockIdx.x * kWaveRows + wid;
  if (row >= a.rows) return;  // wave-uniform; no barrier follows
  unsigned long long(*hist)[256] = hist_all[wid];
  const float* s = a.scores + row * N;
  const float NINF = -__uint_as_float(0x7f800000u);

  uint32_t key[EPL];
  int64_t eff = 0;
  uint32_t v_e = 0;
  uint64_t need = 0;
  // slot e of this lane is present iff 64 e < lim; lim is made opaque in
  // each loop, so the compiler does not keep EPL predicate masks across loops
  int64_t lim = N - lane;
  if (a.mode == 0) {
    asm volatile("" : "+v"(lim));
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      // unconditional loads (absent slots read the row's last score): the
      // loads of all slots are in flight together, not one branch each
      const uint32_t u = __float_as_uint(s[min(64 * e + lane, (int)N - 1)]);
      key[e] = 64 * e < lim ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
    }
    eff = a.k_lo < N ? a.k_lo : N;
  } else {
    float x[EPL];
    float m = NINF;
    asm volatile("" : "+v"(lim));
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float v = s[min(64 * e + lane, (int)N - 1)] * a.scale;  // unconditional load, as above
      x[e] = 64 * e < lim ? v : NINF;
      m = fmaxf(m, x[e]);
    }
    m = wave_max_f32_dpp(m);
    if (m == NINF) {
      eff = 0;
#pragma unroll
      for (int e = 0; e < EPL; ++e) key[e] = 0;
    } else {
      // (the running sums are opaque at each step: integer adds would
      // otherwise be reassociated into a tree over all EPL terms at once, 2 EPL
      // registers more)
      uint64_t E = 0;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        x[e] = canon_exp_nb(x[e] - m);  // absent slots hold -inf: 0
        E += fixp_nb(x[e], 40);
        asm volatile("" : "+v"(E));
      }
      E = wave_sum_u64_dpp(E);
      const float sum = (float)E * 9.094947017729282e-13f;  // 2^-40
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        key[e] = __float_as_uint(x[e] / sum);  // absent slots: 0 / sum = 0
        asm volatile("" : "+v"(key[e]));       // one division at a time (their temporaries otherwise pile up)
      }
      int64_t c = a.ub;
      bool crossed = false;
      uint32_t vc = 0;
      uint64_t jt = 0;
      uint64_t A;
      // crossing value vc: G(vc) >= thr > G(vc + 1) = A (none when G(0) < thr)
      if (wave_radix_search<EPL, true>(key, N, lane, a.thr, &vc, &A, hist)) {
        uint32_t ngt = 0;
        asm volatile("" : "+v"(lim));
#pragma unroll
        for (int e = 0; e < EPL; ++e) ngt += (64 * e < lim && key[e] > vc) ? 1u : 0u;
        ngt = wave_sum_u32_dpp(ngt);
        const uint64_t Wv = fixp(__uint_as_float(vc), 60);
        jt = (a.thr - A - 1) / Wv;  // smallest j with A + (j+1) Wv >= thr
        const int64_t k = (int64_t)ngt + (int64_t)jt;
        if (k < a.ub) { c = k; crossed = true; }
      }
      int64_t n = c + 1;
      if (n < a.k_lo) n = a.k_lo;
      if (n > N) n = N;
      eff = n < a.ub ? n : a.ub;
      if (crossed && eff == c + 1) {
        v_e = vc;
        need = jt + 1;
        eff = -eff;  // marks "v_e already known"
      }
    }
  }
  if (eff > 0) {  // count search: largest v with #(key >= v) >= eff
    uint64_t above;
    (void)wave_radix_search<EPL, false>(key, N, lane, (uint64_t)eff, &v_e, &above, hist);  // (eff <= the count)
    need = (uint64_t)eff - above;
  } else {
    eff = -eff;
  }

  // emit in ascending block order.  Pass 1 (unrolled over the keys): rank
  // the ties and record each slot's selection as a ballot in LDS.  Pass 2 (a
  // plain loop, no key access): place the tiles and blocks slot by slot from
  // the ballots and the tile flags.
  const uint64_t lt = (1ull << lane) - 1ull;
  uint64_t* selm = selm_all[wid];
  {
    int64_t lim = eff > 0 ? N - lane : 0;  // slot e present: 64 e < lim
    asm volatile("" : "+v"(lim));
    uint64_t ties_before = 0;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const bool pres = 64 * e < lim;
      const bool tie = pres && key[e] == v_e;
      const uint64_t tb = __builtin_amdgcn_ballot_w64(tie);
      const uint64_t rank = ties_before + (uint64_t)__popcll(tb & lt);
      ties_before += (uint64_t)__popcll(tb);
      // every lane stores the same value (no branch per slot)
      selm[e] = __builtin_amdgcn_ballot_w64(pres && (key[e] > v_e || (tie && rank < need)));
    }
  }
  wave_lds_order();
  int32_t* trow = a.tiles + row * a.tcap;
  int32_t* brow = a.sel_blocks ? a.sel_blocks + row * a.bcap : nullptr;
  uint64_t tiles_before = 0, blocks_before = 0;
  const int nslots = (int)((N + 63) >> 6);
#pragma unroll 4
  for (int e = 0; e < nslots; ++e) {
    const uint64_t bs = selm[e];
    if (bs == 0) continue;
    const int64_t j = 64 * e + lane;
    const bool sel = (bs >> lane) & 1ull;
    const int32_t f = sel ? flags[j] : 0;
    const bool big = sel && (f & kBigBlock);
    const bool ok0 = f & 1, ok1 = f & 2;  // (neither for a block of more than two tiles)
    const uint64_t b0 = __builtin_amdgcn_ballot_w64(ok0), b1 = __builtin_amdgcn_ballot_w64(ok1);
    if (__builtin_amdgcn_ballot_w64(big) == 0) {
      const int64_t p = (int64_t)(tiles_before + __popcll(b0 & lt) + __popcll(b1 & lt));
      const int32_t t0 = f >> 3;
      if (ok0 && p < a.tcap) trow[p] = t0;
      if (ok1 && p + (ok0 ? 1 : 0) < a.tcap) trow[p + (ok0 ? 1 : 0)] = t0 + 1;
      tiles_before += (uint64_t)(__popcll(b0) + __popcll(b1));
    } else {
      // a block of more than two tiles in this slot: counts by loop, one scan
      int32_t t0 = 0, t1 = 0;
      uint32_t cnt = (ok0 ? 1u : 0u) + (ok1 ? 1u : 0u);
      if (big) {
        t0 = a.block_first_tile[j];
        t1 = a.block_first_tile[j + 1];
        for (int32_t t = t0; t < t1; ++t) cnt += (a.tile_count == nullptr || a.tile_count[t] > 0) ? 1u : 0u;
      }
      const uint32_t incl = wave_incl_scan_u32(cnt, lane);
      int64_t p = (int64_t)tiles_before + (int64_t)(incl - cnt);
      if (big) {
        for (int32_t t = t0; t < t1; ++t)
          if (a.tile_count == nullptr || a.tile_count[t] > 0) {
            if (p < a.tcap) trow[p] = t;
            ++p;
          }
      } else {
        if (ok0) { if (p < a.tcap) trow[p] = f >> 3; ++p; }
        if (ok1 && p < a.tcap) trow[p] = (f >> 3) + 1;
      }
      tiles_before += (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    }
    if (brow && sel) {
      const int64_t q = (int64_t)(blocks_before + __popcll(bs & lt));
      if (q < a.bcap) brow[q] = (int32_t)j;
    }
    blocks_before += (uint64_t)__popcll(bs);
  }
  if (lane == 0) {
    a.ntiles[row] = (int32_t)tiles_before;
    if (a.nsel) a.nsel[row] = (int32_t)blocks_before;
  }
}

// ------------------------------------------------------------ wide rows
// Rows of more than 64 kSelThreads blocks: one 1024-thread workgroup per row;
// element j is taken by thread j mod 1024 in pass j / 1024 (coalesced reads),
// and each pass recomputes the keys and weights from the row's scores (the row
// stays in the L2 / Infinity Cache) instead of holding them in registers.
// The arithmetic is select_kernel's (same canonical exp, same exact integer
// sums), so the selection is identical; the emit phase ranks the ties and
// places the outputs with one ordered workgroup scan per pass and running
// carries.
constexpr int kWideThreads = 1024, kWideWaves = kWideThreads / 64;
constexpr int64_t kWideMaxN = (int64_t)1 << 30;

// Adds w to bin b of hb for the active lanes of a wave: the lanes that share
// the first active lane's bin (a row's keys mostly share their leading
// digits) are summed across the wave and added with one LDS atomic; the other
// active lanes add their own.
__device__ __forceinline__ void hist_add_wave(unsigned long long* hb, bool act, uint32_t b, uint64_t w, int lane) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(act);
  if (m == 0) return;
  const int leader = (int)__builtin_ctzll(m);
  const uint32_t lb = (uint32_t)__builtin_amdgcn_readlane((int)b, leader);
  const bool same = act && b == lb;
  const uint64_t sum = wave_sum_u64(same ? w : 0ull);
  if (lane == leader) atomicAdd(&hb[lb], (unsigned long long)sum);
  if (act && !same) atomicAdd(&hb[b], (unsigned long long)w);
}

// radix_search over the row's N elements, element j's (key, weight) from
// elem(j, key, weight); the passes over the row are wave-uniform
template <bool WEIGHTED, class Elem>
__device__ __forceinline__ uint32_t radix_search_wide(const Elem& elem, int64_t N, uint64_t thr, uint64_t* above,
                                                      SelSharedT<kWideWaves>& sh, unsigned long long* hist) {
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t prefix = 0;
  uint64_t acc = 0;
#pragma unroll 1
  for (int level = 0; level < 4; ++level) {
    const int shift = 24 - 8 * level;
    const uint32_t hmask = level == 0 ? 0u : (0xffffffffu << (shift + 8));
    unsigned long long* hb = hist + 256 * (level & 1);
    for (int64_t base = 0; base < N; base += kWideThreads) {
      const int64_t j = base + tid;
      bool act = false;
      uint32_t b = 0;
      uint64_t w = 0;
      if (j < N) {
        uint32_t k;
        uint64_t wt;
        elem(j, k, wt);
        if ((k & hmask) == prefix) {
          act = true;
          b = (k >> shift) & 255u;
          w = WEIGHTED ? wt : 1ull;
        }
      }
      hist_add_wave(hb, act, b, w, lane);
    }
    __syncthreads();
    if (tid < 64) radix_pick(hb, hist + 256 * ((level + 1) & 1), acc, thr, sh, lane);
    __syncthreads();
    acc += sh.u64[0];
    prefix |= (255u - sh.u32[0]) << shift;
  }
  *above = acc;
  return prefix;
}

__global__ __launch_bounds__(kWideThreads) void select_wide_kernel(SelArgs a) {
  __shared__ SelSharedT<kWideWaves> sh;
  __shared__ unsigned long long hist[2 * 256];
  const int tid = threadIdx.x;
  if (tid < 256) hist[tid] = 0ull;  // buffer 0 of the radix searches
  __syncthreads();
  const int64_t row = blockIdx.x;
  const float* s = a.scores + row * a.N;
  const int64_t N = a.N;
  const float NINF = -__uint_as_float(0x7f800000u);

  // top-k keys: the order-preserving u32 of the score
  auto key_topk = [&](int64_t j, uint32_t& k, uint64_t& w) {
    const uint32_t u = __float_as_uint(s[j]);
    k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    w = 1ull;
  };
  // cdf keys: the fp32 bits of the softmax weight, and its 2^-60 fixed point
  float m = NINF, sum = 1.0f;
  auto key_cdf = [&](int64_t j, uint32_t& k, uint64_t& w) {
    const float x = s[j] * a.scale;
    const float p = canon_exp(x - m) / sum;
    k = __float_as_uint(p);
    w = fixp(p, 60);
  };

  int64_t eff = 0;
  uint32_t v_e = 0;
  uint64_t need = 0;
  if (a.mode == 0) {
    eff = a.k_lo < N ? a.k_lo : N;
  } else {
    float mx = NINF;
    for (int64_t j = tid; j < N; j += kWideThreads) mx = fmaxf(mx, s[j] * a.scale);
    m = block_max_f32(mx, sh);
    if (m == NINF) {
      eff = 0;
    } else {
      uint64_t E = 0;
      for (int64_t j = tid; j < N; j += kWideThreads) {
        const float x = s[j] * a.scale;
        E += fixp(canon_exp(x - m), 40);
      }
      E = block_sum_u64(E, sh);
      sum = (float)E * 9.094947017729282e-13f;  // 2^-40
      uint64_t g0 = 0;
      for (int64_t j = tid; j < N; j += kWideThreads) {
        uint32_t k;
        uint64_t w;
        key_cdf(j, k, w);
        g0 += w;
      }
      g0 = block_sum_u64(g0, sh);
      int64_t c = a.ub;
      bool crossed = false;
      uint32_t vc = 0;
      uint64_t jt = 0;
      if (g0 >= a.thr) {
        // crossing value vc: G(vc) >= thr > G(vc + 1) = A
        uint64_t A;
        vc = radix_search_wide<true>(key_cdf, N, a.thr, &A, sh, hist);
        uint32_t ngt = 0;
        for (int64_t j = tid; j < N; j += kWideThreads) {
          uint32_t k;
          uint64_t w;
          key_cdf(j, k, w);
          ngt += k >= vc + 1 ? 1u : 0u;
        }
        ngt = block_sum_u32(ngt, sh);
        const uint64_t Wv = fixp(__uint_as_float(vc), 60);
        jt = (a.thr - A - 1) / Wv;  // smallest j with A + (j+1) Wv >= thr
        const int64_t k = (int64_t)ngt + (int64_t)jt;
        if (k < a.ub) { c = k; crossed = true; }
      }
      int64_t n = c + 1;
      if (n < a.k_lo) n = a.k_lo;
      if (n > N) n = N;
      eff = n < a.ub ? n : a.ub;
      if (crossed && eff == c + 1) {
        v_e = vc;
        need = jt + 1;
        eff = -eff;  // marks "v_e already known"
      }
    }
  }

  if (eff > 0) {  // count search: largest v with #(key >= v) >= eff
    uint64_t above;
    v_e = a.mode == 0 ? radix_search_wide<false>(key_topk, N, (uint64_t)eff, &above, sh, hist)
                      : radix_search_wide<false>(key_cdf, N, (uint64_t)eff, &above, sh, hist);
    need = (uint64_t)eff - above;
  } else {
    eff = -eff;
  }

  // emit in ascending block order, pass by pass: ties ranked by an ordered
  // scan plus the ties of earlier passes; (tiles | blocks << 32) placed the
  // same way
  int32_t* trow = a.tiles + row * a.tcap;
  int32_t* brow = a.sel_blocks ? a.sel_blocks + row * a.bcap : nullptr;
  uint32_t ties_before = 0;
  uint64_t out_before = 0;
  for (int64_t base = 0; base < N; base += kWideThreads) {
    const int64_t j = base + tid;
    const bool pres = eff > 0 && j < N;
    uint32_t k = 0;
    if (pres) {
      uint64_t w;
      if (a.mode == 0) key_topk(j, k, w);
      else key_cdf(j, k, w);
    }
    const bool tie = pres && k == v_e;
    uint32_t ties_here;
    const uint32_t rank = ties_before + block_excl_scan_u32(tie ? 1u : 0u, sh, &ties_here);
    ties_before += ties_here;
    const bool sel = pres && (k > v_e || (tie && rank < need));
    int32_t t0 = 0, t1 = 0;
    uint32_t cnt = 0;
    if (sel) {
      t0 = a.block_first_tile[j];
      t1 = a.block_first_tile[j + 1];
      for (int32_t t = t0; t < t1; ++t) cnt += (a.tile_count == nullptr || a.tile_count[t] > 0) ? 1u : 0u;
    }
    uint64_t out_here;
    const uint64_t pos =
        out_before + block_excl_scan_u64(sel ? ((uint64_t)cnt | (1ull << 32)) : 0ull, sh, &out_here);
    out_before += out_here;
    if (sel) {
      int64_t p = (int64_t)(pos & 0xffffffffu);
      for (int32_t t = t0; t < t1; ++t)
        if (a.tile_count == nullptr || a.tile_count[t] > 0) {
          if (p < a.tcap) trow[p] = t;
          ++p;
        }
      if (brow && (int64_t)(pos >> 32) < a.bcap) brow[pos >> 32] = (int32_t)j;
    }
  }
  if (tid == 0) {
    a.ntiles[row] = (int32_t)(out_before & 0xffffffffu);
    if (a.nsel) a.nsel[row] = (int32_t)(out_before >> 32);
  }
}

// q tile t of head bh uses the list of its block (shared by the block's tiles);
// with q_tile_count, tiles without a valid query token get an empty list
__global__ void tile_rows_kernel(const int32_t* __restrict__ ntiles, const int32_t* __restrict__ block_id_of_tile,
                                 const int32_t* __restrict__ q_tile_count, int64_t BH, int64_t Nt, int64_t N_b,
                                 int64_t tcap, int64_t* __restrict__ qstart, int32_t* __restrict__ qlen) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= BH * Nt) return;
  const int64_t bh = i / Nt, t = i - bh * Nt;
  const int64_t r = bh * N_b + block_id_of_tile[t];
  qstart[i] = r * tcap;
  qlen[i] = (q_tile_count && q_tile_count[t] == 0) ? 0 : ntiles[r];
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = v;
}

// one 64-lane group per q row: set bit q in the bitmap row of every listed k tile
__global__ __launch_bounds__(64) void set_bits_kernel(const int64_t* __restrict__ qstart, const int32_t* __restrict__ qlen,
                                                      const int32_t* __restrict__ qcols, int64_t Ntq, int64_t Ntk,
                                                      int64_t words, uint32_t* __restrict__ bm) {
  const int64_t row = blockIdx.x;
  const int64_t bh = row / Ntq, t = row - bh * Ntq;
  const int n = qlen[row];
  const int32_t* cols = qcols + qstart[row];
  for (int i = threadIdx.x; i < n; i += 64) {
    const int64_t k = cols[i];
    if (k >= 0 && k < Ntk) atomicOr(&bm[(bh * Ntk + k) * words + (t >> 5)], 1u << (t & 31));
  }
}

// grid (words, BH): workgroup (w, bh) builds bitmap column w (q tiles
// 32 w .. 32 w + 31) of head bh for every k tile in LDS with LDS atomics and
// writes it once (no global atomics, the bitmap needs no clearing)
constexpr int kColMaxTiles = 16384;  // LDS column of up to 16384 k tiles (64 KB of dynamic LDS)
__global__ __launch_bounds__(256) void set_bits_col_kernel(const int64_t* __restrict__ qstart,
                                                           const int32_t* __restrict__ qlen,
                                                           const int32_t* __restrict__ qcols, int64_t Ntq, int64_t Ntk,
                                                           int64_t words, uint32_t* __restrict__ bm) {
  extern __shared__ uint32_t col[];  // [Ntk]
  const int64_t w = blockIdx.x, bh = blockIdx.y;
  for (int64_t k = threadIdx.x; k < Ntk; k += blockDim.x) col[k] = 0u;
  __syncthreads();
  for (int j = 0; j < 32; ++j) {
    const int64_t t = w * 32 + j;
    if (t >= Ntq) break;
    const int64_t row = bh * Ntq + t;
    const int n = qlen[row];
    const int32_t* cols = qcols + qstart[row];
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int32_t k = cols[i];
      if (k >= 0 && k < Ntk) atomicOr(&col[k], 1u << j);
    }
  }
  __syncthreads();
  for (int64_t k = threadIdx.x; k < Ntk; k += blockDim.x) bm[(bh * Ntk + k) * words + w] = col[k];
}

// one wave per k row: emit the set bits (ascending q tiles); bitmap row r is
// output row row0 + r
__global__ __launch_bounds__(256) void emit_bits_kernel(const uint32_t* __restrict__ bm, int64_t rows,
                                                        int64_t words, int64_t kcap, int64_t row0,
                                                        int64_t* __restrict__ kstart, int32_t* __restrict__ klen,
                                                        int32_t* __restrict__ kcols) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const uint32_t* w = bm + r * words;
  const int64_t row = row0 + r;
  int32_t* out = kcols + row * kcap;
  uint32_t carry = 0;
  for (int64_t base = 0; base < words; base += 64) {
    const int64_t wi = base + lane;
    uint32_t word = wi < words ? w[wi] : 0u;
    const uint32_t c = __popc(word);
    const uint32_t incl = wave_incl_scan_u32(c, lane);
    uint32_t pos = carry + incl - c;
    while (word) {
      const int b = __ffs(word) - 1;
      out[pos++] = (int32_t)(wi * 32 + b);
      word &= word - 1;
    }
    carry += __shfl(incl, 63, 64);
  }
  if (lane == 0) {
    kstart[row] = row * kcap;
    klen[row] = (int32_t)carry;
  }
}

// The list transpose of heads [bh0, bh0 + nbh) through the bitmap bm (rows
// of those heads only): bits set per bitmap column in LDS when the key tiles
// fit (nothing to clear), else zero-filled and set with global atomics.
void launch_transpose(const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, int bh0, int nbh,
                      int64_t Ntq, int64_t Ntk, uint32_t* bm, int64_t kcap, int64_t* kstart, int32_t* klen,
                      int32_t* kcols, hipStream_t stream) {
  const int64_t words = (Ntq + 31) / 32, krows = (int64_t)nbh * Ntk;
  const int64_t* qs = qstart + (int64_t)bh0 * Ntq;  // entries of qstart are absolute offsets into qcols
  const int32_t* ql = qlen + (int64_t)bh0 * Ntq;
  if (Ntk <= kColMaxTiles) {
    set_bits_col_kernel<<<dim3((unsigned)words, (unsigned)nbh), 256, (size_t)Ntk * 4, stream>>>(qs, ql, qcols, Ntq,
                                                                                              Ntk, words, bm);
  } else {
    fill_u32_kernel<<<1024, 256, 0, stream>>>(bm, krows * words, 0u);
    set_bits_kernel<<<(unsigned)((int64_t)nbh * Ntq), 64, 0, stream>>>(qs, ql, qcols, Ntq, Ntk, words, bm);
  }
  emit_bits_kernel<<<(unsigned)((krows + 3) / 4), 256, 0, stream>>>(bm, krows, words, kcap, (int64_t)bh0 * Ntk, kstart,
                                                                    klen, kcols);
}

// Workspace of prism_transpose_lists_noalloc: the bitmap of as many heads as
// fit, in a file-scope device array instead of caller memory.  Each GPU the
// library runs on holds its own copy (8 MiB) until the process ends; host
// code reaches it only through the address hipGetSymbolAddress returns for
// the current device (ScratchDevice::ptr), never through the name.
constexpr int64_t kScratchWords = (int64_t)1 << 21;
static __device__ __align__(256) uint32_t scratch[kScratchWords];

constexpr int kMaxDevices = 64;

// Per-device state of `scratch`, set up on the first call on the device:
// its address, and an event recorded on the stream of each call after its
// kernels.  Every later call's stream waits for that event first, so calls
// on different streams of one GPU take the array one after the other
// instead of racing on it (calls under graph capture neither wait nor
// record: the graph's own launch order applies to them).
struct ScratchDevice {
  uint32_t* ptr = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
};
std::mutex g_scratch_mu;  // held by a call from set-up until its event is recorded
ScratchDevice g_scratch[kMaxDevices];

int scratch_device(ScratchDevice** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    prism_set_error("prism_transpose_lists_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return PRISM_EHIP;
  }
  PRISM_REQUIRE(dev >= 0 && dev < kMaxDevices, "prism_transpose_lists_noalloc: device %d out of range", dev);
  ScratchDevice& sd = g_scratch[dev];
  if (!sd.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      prism_set_error("prism_transpose_lists_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return PRISM_EHIP;
    }
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      prism_set_error("prism_transpose_lists_noalloc: hipEventCreateWithFlags failed: %s", hipGetErrorString(e));
      return PRISM_EHIP;
    }
    sd.done = ev;
    sd.ptr = (uint32_t*)p;
  }
  *out = &sd;
  return PRISM_OK;
}

}  // namespace

extern "C" {

int prism_block_scores(const float* qc, const float* kc, const int32_t* block_count, int BH, int64_t Nq, int64_t Nk,
                       int D, float* scores, hipStream_t stream) {
  PRISM_REQUIRE(qc && kc && scores, "prism_block_scores: null pointer");
  PRISM_REQUIRE(D > 0 && D % kSChunk == 0, "prism_block_scores: D=%d must be a multiple of %d", D, kSChunk);
  PRISM_REQUIRE(BH >= 1 && Nq >= 1 && Nk >= 1, "prism_block_scores: empty problem");
  dim3 grid((unsigned)((Nk + kSTile - 1) / kSTile), (unsigned)((Nq + kSTile - 1) / kSTile), BH);
  block_scores_kernel<<<grid, 256, 0, stream>>>(qc, kc, block_count, Nq, Nk, D, scores);
  PRISM_LAUNCH_CHECK("prism_block_scores");
  return PRISM_OK;
}

int prism_select_tiles(const float* scores, int64_t rows, int64_t N, int mode, int64_t k_lo, int64_t ub, float scale,
                       uint64_t thr, const int32_t* block_first_tile, const int32_t* tile_count, int64_t tcap,
                       int32_t* tiles, int32_t* ntiles, int32_t* sel_blocks, int64_t bcap, int32_t* nsel,
                       hipStream_t stream) {
  PRISM_REQUIRE(scores && block_first_tile && tiles && ntiles, "prism_select_tiles: null pointer");
  PRISM_REQUIRE(mode >= 0 && mode <= 2, "prism_select_tiles: mode %d unknown", mode);
  PRISM_REQUIRE(N >= 1 && N <= kWideMaxN, "prism_select_tiles: N=%lld out of range [1, %lld]", (long long)N,
                (long long)kWideMaxN);
  PRISM_REQUIRE(k_lo >= 0 && ub >= 0 && ub <= N, "prism_select_tiles: bad k/ub");
  PRISM_REQUIRE(mode == 0 || thr > 0, "prism_select_tiles: threshold must be positive");
  PRISM_REQUIRE(tcap >= (mode == 0 ? (k_lo < N ? k_lo : N) : ub), "prism_select_tiles: tcap too small");
  PRISM_REQUIRE(sel_blocks == nullptr || bcap >= (mode == 0 ? (k_lo < N ? k_lo : N) : ub),
                "prism_select_tiles: bcap too small");
  if (rows == 0) return PRISM_OK;
  SelArgs a;
  a.scores = scores; a.rows = rows; a.N = N; a.mode = mode; a.k_lo = k_lo; a.ub = ub; a.scale = scale; a.thr = thr;
  a.block_first_tile = block_first_tile; a.tile_count = tile_count; a.tcap = tcap; a.tiles = tiles;
  a.ntiles = ntiles; a.sel_blocks = sel_blocks; a.bcap = bcap; a.nsel = nsel;
  const int64_t need = (N + kSelThreads - 1) / kSelThreads;
  const unsigned wave_grid = (unsigned)((rows + kWaveRows - 1) / kWaveRows);
  // rows of up to 6,144 blocks: one wave per row; up to 16,384: one
  // 256-thread workgroup per row, in registers; wider rows pass by pass (all
  // place tiles and blocks with 32-bit fields)
  if (N <= 1024) select_rows_kernel<16><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (N <= 2048) select_rows_kernel<32><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (N <= 3072) select_rows_kernel<48><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (N <= 4096) select_rows_kernel<64><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (N <= 5120) select_rows_kernel<80><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (N <= 5632) select_rows_kernel<88><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (N <= kWaveMaxN) select_rows_kernel<96><<<wave_grid, 64 * kWaveRows, 0, stream>>>(a);
  else if (need > 64) select_wide_kernel<<<(unsigned)rows, kWideThreads, 0, stream>>>(a);
  else if (need <= 32) select_kernel<32><<<(unsigned)rows, kSelThreads, 0, stream>>>(a);
  else select_kernel<64><<<(unsigned)rows, kSelThreads, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_select_tiles");
  return PRISM_OK;
}

int prism_tile_rows(const int32_t* ntiles, const int32_t* block_id_of_tile, const int32_t* q_tile_count, int BH,
                    int64_t Nt, int64_t N_b, int64_t tcap, int64_t* qstart, int32_t* qlen, hipStream_t stream) {
  PRISM_REQUIRE(ntiles && block_id_of_tile && qstart && qlen, "prism_tile_rows: null pointer");
  const int64_t n = (int64_t)BH * Nt;
  if (n == 0) return PRISM_OK;
  tile_rows_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(ntiles, block_id_of_tile, q_tile_count, BH, Nt, N_b, tcap,
                                                                    qstart, qlen);
  PRISM_LAUNCH_CHECK("prism_tile_rows");
  return PRISM_OK;
}

int prism_transpose_lists(const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, int BH, int64_t Ntq,
                          int64_t Ntk, uint32_t* bitmap, int64_t kcap, int64_t* kstart, int32_t* klen, int32_t* kcols,
                          hipStream_t stream) {
  PRISM_REQUIRE(qstart && qlen && qcols && bitmap && kstart && klen && kcols, "prism_transpose_lists: null pointer");
  PRISM_REQUIRE(Ntq >= 1 && Ntk >= 1, "prism_transpose_lists: empty tile range");
  PRISM_REQUIRE(kcap >= Ntq, "prism_transpose_lists: kcap must be >= Ntq");
  if (BH <= 0) return PRISM_OK;
  launch_transpose(qstart, qlen, qcols, 0, BH, Ntq, Ntk, bitmap, kcap, kstart, klen, kcols, stream);
  PRISM_LAUNCH_CHECK("prism_transpose_lists");
  return PRISM_OK;
}

int prism_transpose_lists_noalloc(const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, int BH,
                                  int64_t Ntq, int64_t Ntk, int64_t kcap, int64_t* kstart, int32_t* klen,
                                  int32_t* kcols, hipStream_t stream) {
  PRISM_REQUIRE(qstart && qlen && qcols && kstart && klen && kcols, "prism_transpose_lists_noalloc: null pointer");
  PRISM_REQUIRE(Ntq >= 1 && Ntk >= 1, "prism_transpose_lists_noalloc: empty tile range");
  PRISM_REQUIRE(kcap >= Ntq, "prism_transpose_lists_noalloc: kcap must be >= Ntq");
  const int64_t per_head = Ntk * ((Ntq + 31) / 32);  // bitmap words of one head
  PRISM_REQUIRE(per_head <= kScratchWords,
                "prism_transpose_lists_noalloc: one head's bitmap (%lld key tiles x %lld words) exceeds the "
                "%lld-word workspace; use prism_transpose_lists with a caller workspace",
                (long long)Ntk, (long long)((Ntq + 31) / 32), (long long)kScratchWords);
  if (BH <= 0) return PRISM_OK;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchDevice* sd = nullptr;
  const int rc = scratch_device(&sd);
  if (rc != PRISM_OK) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) {
    prism_set_error("prism_transpose_lists_noalloc: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
    return PRISM_EHIP;
  }
  const bool ordered = cap == hipStreamCaptureStatusNone;
  if (ordered && sd->recorded && (e = hipStreamWaitEvent(stream, sd->done, 0)) != hipSuccess) {
    prism_set_error("prism_transpose_lists_noalloc: hipStreamWaitEvent failed: %s", hipGetErrorString(e));
    return PRISM_EHIP;
  }
  // heads in batches that fit the workspace, one after the other on `stream`
  const int per_batch = (int)(kScratchWords / per_head < BH ? kScratchWords / per_head : BH);
  for (int bh0 = 0; bh0 < BH; bh0 += per_batch) {
    const int nbh = BH - bh0 < per_batch ? BH - bh0 : per_batch;
    launch_transpose(qstart, qlen, qcols, bh0, nbh, Ntq, Ntk, sd->ptr, kcap, kstart, klen, kcols, stream);
  }
  PRISM_LAUNCH_CHECK("prism_transpose_lists_noalloc");
  if (ordered) {
    if ((e = hipEventRecord(sd->done, stream)) != hipSuccess) {
      prism_set_error("prism_transpose_lists_noalloc: hipEventRecord failed: %s", hipGetErrorString(e));
      return PRISM_EHIP;
    }
    sd->recorded = true;
  }
  return PRISM_OK;
}

}  // extern "C"
