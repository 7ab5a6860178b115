// Zone geometry, fused row gather + block mean pooling, inverse scatter (gfx950).
//
// Reference (hymm/models/modules/block_sparse_attention/):
//   zone_layout_kernel   _build_block_tile_maps (dynamic_block_attention.py:138-170)
//                        in CSR form: block_offset[Nz+1] (block_offset[Nz] = N_b),
//                        block_id_of_tile[N_tiles], block_first_tile[N_b+1]
//                        (block b owns tiles [first[b], first[b+1]))
//   rearrange_kernel     _build_rearrange_index (dynamic_block_attention.py:107-135)
//   gather_pool_kernel   q/k/v.index_select(2, src_idx) (:250-253) fused with
//                        masked_mean_pooling_compression (bsa_interface.py:177-201)
//                        and _logical_block_means (dynamic_block_attention.py:173-188),
//                        plus the transposed-tile copy the MFMA kernels read and,
//                        for the backward, delta = rowsum(o * do) (common.py:110-127)
//   scatter_rows_kernel  o_re.index_select(2, inv_idx) (dynamic_block_attention.py:329)
//
// Tile order: zone z holds rearranged positions [512 z, 512 z + 512); 64-token
// tile t = position / 64.  Block means are fp32 sums over the block's valid
// tokens in rearranged order (sequential per channel), divided by max(count, 1).
#include "common.h"
#include "mfma.h"

namespace {

constexpr int kLayoutThreads = 1024;

__global__ __launch_bounds__(kLayoutThreads) void zone_layout_kernel(
    const int64_t* __restrict__ shape_ids, int Nz, int32_t* __restrict__ block_offset,
    int32_t* __restrict__ block_id_of_tile, int32_t* __restrict__ block_first_tile) {
  __shared__ int32_t sWave[kLayoutThreads / 64];
  __shared__ int32_t sCarry;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) sCarry = 0;
  __syncthreads();
  for (int base = 0; base < Nz; base += kLayoutThreads) {
    const int z = base + tid;
    int tpb = 1, nbz = 0;
    if (z < Nz) {
      const int c = (int)shape_ids[z];
      tpb = (kCand[c][0] * kCand[c][1] * kCand[c][2]) / 64;
      nbz = 8 / tpb;
    }
    const uint32_t incl = wave_incl_scan_u32((uint32_t)nbz, lane);
    if (lane == 63) sWave[wid] = (int32_t)incl;
    __syncthreads();
    int32_t before = sCarry;
    for (int w = 0; w < wid; ++w) before += sWave[w];
    const int32_t excl = before + (int32_t)incl - nbz;
    if (z < Nz) {
      block_offset[z] = excl;
      for (int t = 0; t < 8; ++t) block_id_of_tile[z * 8 + t] = excl + t / tpb;
      for (int j = 0; j < nbz; ++j) block_first_tile[excl + j] = z * 8 + j * tpb;
    }
    __syncthreads();
    if (tid == kLayoutThreads - 1) sCarry = excl + nbz;
    __syncthreads();
  }
  if (tid == 0) {
    block_offset[Nz] = sCarry;
    block_first_tile[sCarry] = Nz * 8;
  }
}

__global__ void rearrange_kernel(const int64_t* __restrict__ shape_ids, int64_t S, int ZH, int ZW, int Hg, int Wg,
                                 int64_t* __restrict__ src_idx, int64_t* __restrict__ inv_idx) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= S) return;
  const int z = (int)(p >> 9), r = (int)(p & 511);
  const int64_t tok = token_of(z, local_of_rearr((int)shape_ids[z], r), ZH, ZW, Hg, Wg);
  src_idx[p] = tok;
  inv_idx[tok] = p;
}

template <typename T, int CPL>
__device__ __forceinline__ void load_row(const T* p, float* x) {
  if (sizeof(T) == 2) {
    if (CPL == 2) {
      const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
      x[0] = __uint_as_float(u << 16);
      x[CPL - 1] = __uint_as_float(u & 0xffff0000u);
    } else {
      x[0] = bf2f(*reinterpret_cast<const uint16_t*>(p));
    }
  } else {
    if (CPL == 2) {
      const float2 f = *reinterpret_cast<const float2*>(p);
      x[0] = f.x;
      x[CPL - 1] = f.y;
    } else {
      x[0] = *reinterpret_cast<const float*>(p);
    }
  }
}

struct GatherArgs {
  const void* x;             // [B,H,S,D] THW order, dtype T
  const uint8_t* valid;      // [S] THW or null
  const int64_t* shape_ids;  // [Nz]
  const int32_t* block_offset;
  int64_t S;
  int64_t N_b;
  int ZH, ZW, Hg, Wg;
  uint16_t* out_rows;        // [B,H,S,D] bf16 tile order, or null
  float* block_mean;         // [B,H,N_b,D] fp32, or null
  int32_t* block_count;      // [N_b] or null
  int32_t* tile_count;       // [Nt] or null
  uint8_t* valid_re;         // [S] tile order, or null
  const uint16_t* dot_with;  // [B,H,S,D] bf16 tile order, or null
  float* rowdot;             // [B,H,S] fp32, or null
};

constexpr int kGatherThreads = 256;  // 4 waves, 128 rearranged rows each
constexpr int kGatherBatch = 8;      // rows loaded per step (loads in flight)

// grid (Nz, B*H).  Wave w covers rearranged rows [128 w, 128 w + 128) of zone z
// (two 64-token blocks or one 128-token block; two tiles); lane l owns
// channels [l*CPL, l*CPL + CPL).
template <int D, typename T>
__global__ __launch_bounds__(kGatherThreads) void gather_pool_kernel(GatherArgs a) {
  constexpr int CPL = D / 64;
  const int z = blockIdx.x;
  const int bh = blockIdx.y;
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = (int)a.shape_ids[z];
  const int bsz = kCand[c][0] * kCand[c][1] * kCand[c][2];
  const int boff = a.block_offset[z];
  const bool first_bh = bh == 0;
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)bh * a.S * D;
  const int64_t rowbase = (int64_t)bh * a.S + (int64_t)z * 512;

  float acc[CPL];
  int cnt = 0, tcnt = 0;
#pragma unroll
  for (int j = 0; j < CPL; ++j) acc[j] = 0.0f;

  for (int o0 = 0; o0 < 128; o0 += kGatherBatch) {
    float xv[kGatherBatch][CPL];
    bool ok[kGatherBatch];
#pragma unroll
    for (int u = 0; u < kGatherBatch; ++u) {
      const int r = wid * 128 + o0 + u;
      const int64_t tok = token_of(z, local_of_rearr(c, r), a.ZH, a.ZW, a.Hg, a.Wg);
      ok[u] = a.valid ? (a.valid[tok] != 0) : true;
      load_row<T, CPL>(x + tok * D + lane * CPL, xv[u]);
    }
#pragma unroll
    for (int u = 0; u < kGatherBatch; ++u) {
      const int r = wid * 128 + o0 + u;
      if (a.out_rows) {
        uint16_t* dst = a.out_rows + (rowbase + r) * D + lane * CPL;
        if (CPL == 2) *reinterpret_cast<uint32_t*>(dst) = (uint32_t)f2bf(xv[u][0]) | ((uint32_t)f2bf(xv[u][CPL - 1]) << 16);
        else dst[0] = f2bf(xv[u][0]);
      }
      if (a.rowdot) {
        const uint16_t* y = a.dot_with + (rowbase + r) * D + lane * CPL;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) part = __builtin_fmaf(xv[u][j], bf2f(y[j]), part);
        part = wave_sum_xor(part);
        if (lane == 0) a.rowdot[rowbase + r] = part;
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] = ok[u] ? acc[j] + xv[u][j] : acc[j];
      cnt += ok[u] ? 1 : 0;
      tcnt += ok[u] ? 1 : 0;
      if (first_bh && lane == 0 && a.valid_re) a.valid_re[(int64_t)z * 512 + r] = ok[u] ? 1 : 0;
      if ((r + 1) % bsz == 0) {  // block complete
        const int blk = r / bsz;
        if (a.block_mean) {
          const float den = (float)(cnt > 0 ? cnt : 1);
          float* dst = a.block_mean + ((int64_t)bh * a.N_b + boff + blk) * D + lane * CPL;
#pragma unroll
          for (int j = 0; j < CPL; ++j) dst[j] = acc[j] / den;
        }
        if (first_bh && lane == 0 && a.block_count) a.block_count[boff + blk] = cnt;
        cnt = 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc[j] = 0.0f;
      }
      if ((r & 63) == 63) {  // tile complete
        if (first_bh && lane == 0 && a.tile_count) a.tile_count[z * 8 + (r >> 6)] = tcnt;
        tcnt = 0;
      }
    }
  }
}

// grid (Nz, B*H): tile-order bf16 rows -> THW rows of dtype TO.
template <int D, typename TO>
__global__ __launch_bounds__(kGatherThreads) void scatter_rows_kernel(
    const uint16_t* __restrict__ in, const int64_t* __restrict__ shape_ids, int64_t S, int ZH, int ZW, int Hg,
    int Wg, TO* __restrict__ out) {
  constexpr int CPL = D / 64;
  const int z = blockIdx.x, bh = blockIdx.y;
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = (int)shape_ids[z];
  for (int o = 0; o < 128; ++o) {
    const int r = wid * 128 + o;
    const int64_t tok = token_of(z, local_of_rearr(c, r), ZH, ZW, Hg, Wg);
    const uint16_t* src = in + ((int64_t)bh * S + (int64_t)z * 512 + r) * D + lane * CPL;
    TO* dst = out + ((int64_t)bh * S + tok) * D + lane * CPL;
    if (sizeof(TO) == 2) {
      if (CPL == 2) *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
      else *reinterpret_cast<uint16_t*>(dst) = src[0];
    } else {
#pragma unroll
      for (int j = 0; j < CPL; ++j) reinterpret_cast<float*>(dst)[j] = bf2f(src[j]);
    }
  }
}

bool grid_ok(int T, int Hg, int Wg) { return T > 0 && Hg > 0 && Wg > 0 && T % 8 == 0 && Hg % 8 == 0 && Wg % 8 == 0; }

}  // namespace

extern "C" {

int prism_zone_layout(const int64_t* shape_ids, int Nz, int32_t* block_offset, int32_t* block_id_of_tile,
                      int32_t* block_first_tile, hipStream_t stream) {
  PRISM_REQUIRE(shape_ids && block_offset && block_id_of_tile && block_first_tile, "prism_zone_layout: null pointer");
  PRISM_REQUIRE(Nz >= 1, "prism_zone_layout: Nz must be >= 1");
  zone_layout_kernel<<<1, kLayoutThreads, 0, stream>>>(shape_ids, Nz, block_offset, block_id_of_tile,
                                                       block_first_tile);
  PRISM_LAUNCH_CHECK("prism_zone_layout");
  return PRISM_OK;
}

int prism_rearrange_index(const int64_t* shape_ids, int T, int Hg, int Wg, int64_t* src_idx, int64_t* inv_idx,
                          hipStream_t stream) {
  PRISM_REQUIRE(shape_ids && src_idx && inv_idx, "prism_rearrange_index: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_rearrange_index: grid must be multiples of 8");
  const int64_t S = (int64_t)T * Hg * Wg;
  rearrange_kernel<<<(unsigned)((S + 255) / 256), 256, 0, stream>>>(shape_ids, S, Hg / 8, Wg / 8, Hg, Wg, src_idx,
                                                                    inv_idx);
  PRISM_LAUNCH_CHECK("prism_rearrange_index");
  return PRISM_OK;
}

int prism_gather_pool(const void* x, int dtype, int B, int H, int64_t S, int D, const uint8_t* valid,
                      const int64_t* shape_ids, const int32_t* block_offset, int T, int Hg, int Wg, int64_t N_b,
                      void* out_rows, float* block_mean, int32_t* block_count, int32_t* tile_count,
                      uint8_t* valid_re, const void* dot_with, float* rowdot, hipStream_t stream) {
  PRISM_REQUIRE(x && shape_ids && block_offset, "prism_gather_pool: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_gather_pool: grid (%d,%d,%d) must be multiples of 8", T, Hg, Wg);
  PRISM_REQUIRE((int64_t)T * Hg * Wg == S, "prism_gather_pool: T*H*W != S");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_gather_pool: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(B >= 1 && H >= 1, "prism_gather_pool: B, H must be >= 1");
  PRISM_REQUIRE(dtype == PRISM_F32 || dtype == PRISM_BF16, "prism_gather_pool: bad dtype");
  PRISM_REQUIRE((dot_with == nullptr) == (rowdot == nullptr), "prism_gather_pool: dot_with and rowdot go together");
  PRISM_REQUIRE(block_mean == nullptr || N_b > 0, "prism_gather_pool: N_b required for pooling");
  GatherArgs a;
  a.x = x; a.valid = valid; a.shape_ids = shape_ids; a.block_offset = block_offset; a.S = S; a.N_b = N_b;
  a.ZH = Hg / 8; a.ZW = Wg / 8; a.Hg = Hg; a.Wg = Wg;
  a.out_rows = (uint16_t*)out_rows; a.block_mean = block_mean;
  a.block_count = block_count; a.tile_count = tile_count; a.valid_re = valid_re;
  a.dot_with = (const uint16_t*)dot_with; a.rowdot = rowdot;
  const int Nz = (int)(S / 512);
  dim3 grid(Nz, B * H);
  if (dtype == PRISM_BF16) {
    if (D == 128) gather_pool_kernel<128, uint16_t><<<grid, kGatherThreads, 0, stream>>>(a);
    else gather_pool_kernel<64, uint16_t><<<grid, kGatherThreads, 0, stream>>>(a);
  } else {
    if (D == 128) gather_pool_kernel<128, float><<<grid, kGatherThreads, 0, stream>>>(a);
    else gather_pool_kernel<64, float><<<grid, kGatherThreads, 0, stream>>>(a);
  }
  PRISM_LAUNCH_CHECK("prism_gather_pool");
  return PRISM_OK;
}

int prism_scatter_rows(const void* in_rows, int B, int H, int64_t S, int D, const int64_t* shape_ids, int T, int Hg,
                       int Wg, void* out, int out_dtype, hipStream_t stream) {
  PRISM_REQUIRE(in_rows && shape_ids && out, "prism_scatter_rows: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_scatter_rows: grid must be multiples of 8");
  PRISM_REQUIRE((int64_t)T * Hg * Wg == S, "prism_scatter_rows: T*H*W != S");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_scatter_rows: head_dim %d unsupported", D);
  PRISM_REQUIRE(out_dtype == PRISM_F32 || out_dtype == PRISM_BF16, "prism_scatter_rows: bad dtype");
  dim3 grid((unsigned)(S / 512), B * H);
  const uint16_t* in = (const uint16_t*)in_rows;
  if (out_dtype == PRISM_BF16) {
    if (D == 128) scatter_rows_kernel<128, uint16_t><<<grid, kGatherThreads, 0, stream>>>(in, shape_ids, S, Hg / 8, Wg / 8, Hg, Wg, (uint16_t*)out);
    else scatter_rows_kernel<64, uint16_t><<<grid, kGatherThreads, 0, stream>>>(in, shape_ids, S, Hg / 8, Wg / 8, Hg, Wg, (uint16_t*)out);
  } else {
    if (D == 128) scatter_rows_kernel<128, float><<<grid, kGatherThreads, 0, stream>>>(in, shape_ids, S, Hg / 8, Wg / 8, Hg, Wg, (float*)out);
    else scatter_rows_kernel<64, float><<<grid, kGatherThreads, 0, stream>>>(in, shape_ids, S, Hg / 8, Wg / 8, Hg, Wg, (float*)out);
  }
  PRISM_LAUNCH_CHECK("prism_scatter_rows");
  return PRISM_OK;
}

}  // extern "C"
