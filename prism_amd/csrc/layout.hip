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
//                        and _logical_block_means (dynamic_block_attention.py:173-188)
//                        and, for the backward, delta = rowsum(o * do)
//                        (common.py:110-127); with the uniform chunk layout it
//                        is rearrange_THW_to_3d_block (bsa_interface.py:1105-1109)
//                        fused with the 3-D / 1-D padding of flash_attn_bsa_cross
//                        (:1263-1273, :1318-1367) and (masked_)mean_pooling_compression
//                        (:164-201)
//   scatter_rows_kernel  o_re.index_select(2, inv_idx) (dynamic_block_attention.py:329),
//                        rearrange_3d_block_to_THW + unpadding (bsa_interface.py:1111-1115,
//                        :1372-1380)
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
  __shared__ int32_t sCarry, sBad;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) sCarry = sBad = 0;
  __syncthreads();
  for (int base = 0; base < Nz; base += kLayoutThreads) {
    const int z = base + tid;
    int tpb = 1, nbz = 0;
    if (z < Nz) {
      const int64_t id = shape_ids[z];
      // an id outside the candidate table is reported through block_offset[Nz]
      // (the caller raises); shape 0 stands in so that no access leaves bounds
      const int c = (id >= 0 && id < PRISM_NCAND) ? (int)id : 0;
      if (c != id) sBad = 1;
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
  __syncthreads();
  if (tid == 0) {
    block_offset[Nz] = sBad ? -1 : sCarry;
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

struct GatherArgs {
  const void* x;             // [B,H,S_in,D] THW order, dtype T
  const uint8_t* valid;      // [S_in] THW or null
  int64_t S_in;              // tokens per head in x
  int64_t S_out;             // rows per head of the tile-order outputs
  int64_t N_b;               // blocks per head
  uint16_t* out_rows;        // [B,H,S_out,D] bf16 tile order, or null
  float* block_mean;         // [B,H,N_b,D] fp32, or null
  int32_t* block_count;      // [N_b] or null
  int32_t* tile_count;       // [S_out/64] or null
  uint8_t* valid_re;         // [S_out] tile order, or null
  const uint16_t* dot_with;  // [B,H,S_out,D] bf16 tile order, or null
  float* rowdot;             // [B,H,S_out] fp32, or null
};

// Rearranged row r (0..511) of work unit u -> source token, for the two
// layouts.  token() is -1 for a padding row (no source token); a block is
// bsz consecutive rows starting at a multiple of bsz.
//
// ZoneMap: the dynamic layout.  Unit = zone z (512 rows); its blocks have the
// zone's candidate shape (local_of_rearr) and are numbered from block_offset[z].
struct ZoneMap {
  const int64_t* shape_ids;
  const int32_t* block_offset;
  int ZH, ZW;
  GridBox box;  // input grid (tokens outside it are padding)
  int z, c, bsz, boff;
  __device__ __forceinline__ void init(int unit) {
    z = unit;
    c = (int)shape_ids[z];
    bsz = kCand[c][0] * kCand[c][1] * kCand[c][2];
    boff = block_offset ? block_offset[z] : 0;  // (the scatter needs no block numbers)
  }
  __device__ __forceinline__ int64_t row(int r) const { return (int64_t)z * 512 + r; }
  __device__ __forceinline__ bool live(int) const { return true; }
  __device__ __forceinline__ int64_t token(int r) const { return token_in(z, local_of_rearr(c, r), ZH, ZW, box); }
  __device__ __forceinline__ int64_t block(int r) const { return boff + r / bsz; }
};

// ChunkMap: the uniform 3-D chunk layout (rearrange_THW_to_3d_block,
// bsa_interface.py:1105-1109): the padded grid Tp x Hp x Wp is cut into
// ct x ch x cw chunks, chunk n = (nt Nh + nh) Nw + nw owns rows
// [n csz, n csz + csz) with offset (it ch + ih) cw + iw.  Tokens outside the
// input grid T x Hg x Wg (the padding of _pad_1d_for_bsa / the 3-D pads of
// flash_attn_bsa_cross, bsa_interface.py:1263-1273, 1318-1331) and rows past
// Tp Hp Wp (tile-pair alignment) are padding.  Unit = 512 consecutive rows.
struct ChunkMap {
  int T, Hg, Wg;    // input grid
  int ct, ch, cw;   // chunk shape
  int Nh, Nw;       // chunks along padded h, w
  int64_t Sp;       // Tp Hp Wp
  int64_t S_out;    // rows per head (>= Sp)
  int bsz;          // ct ch cw
  int64_t base;
  __device__ __forceinline__ void init(int unit) { base = (int64_t)unit * 512; }
  __device__ __forceinline__ int64_t row(int r) const { return base + r; }
  __device__ __forceinline__ bool live(int r) const { return base + r < S_out; }
  __device__ __forceinline__ int64_t token(int r) const {
    const int64_t p = base + r;
    if (p >= Sp) return -1;
    const int64_t n = p / bsz;
    const int off = (int)(p - n * bsz);
    const int64_t nt = n / ((int64_t)Nh * Nw);
    const int nh = (int)((n / Nw) % Nh), nw = (int)(n % Nw);
    const int it = off / (ch * cw), ih = (off / cw) % ch, iw = off % cw;
    const int64_t t = nt * ct + it;
    const int h = nh * ch + ih, w = nw * cw + iw;
    if (t >= T || h >= Hg || w >= Wg) return -1;
    return (t * Hg + h) * Wg + w;
  }
  __device__ __forceinline__ int64_t block(int r) const { return (base + r) / bsz; }
};

constexpr int kGatherThreads = 256;  // 4 waves, 128 rearranged rows each

// 8 channels of one row as floats (16 bytes of bf16 or 32 bytes of fp32)
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* x) {
  if (sizeof(T) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
    const float4 lo = reinterpret_cast<const float4*>(p)[0], hi = reinterpret_cast<const float4*>(p)[1];
    x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
    x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
  }
}

// grid (units, B*H).  Wave w covers rearranged rows [128 w, 128 w + 128) of
// unit u (blocks of 64 or 128 rows: one or two whole blocks, two tiles).  A
// lane moves 8 channels (16 bytes of bf16): D / 8 lanes per row, 64 / (D / 8)
// rows per wave instruction, NB instructions in flight (fewer registers, more
// waves per SIMD beat more loads per wave here).  Block means: row group g
// (rows o of the block with o mod RPI = g, RPI = 512 / D) is summed in fp32
// in row order from +0 by the lanes that load it, and the block sum is
// ((p_0 + p_1) + ...) + p_{RPI-1}, formed by the first group's lanes when the
// block is complete; padding rows are written as zeros, are invalid, and
// belong to no block when they lie past the last block.
template <int D, typename T, typename Map, bool POOL>
__global__ __launch_bounds__(kGatherThreads) void gather_pool_kernel(GatherArgs a, Map m) {
  constexpr int LPR = D / 8;     // lanes per row
  constexpr int RPI = 64 / LPR;  // rows per wave instruction
  // wave instructions in flight: with pooling 2 (2: 0.256 ms, 4: 0.283, 8:
  // 0.326 averaged over the step's launches at C4), without it 4
  constexpr int NB = POOL ? 2 : 4;
  constexpr int RB = RPI * NB;   // rows per batch (inside one block and one tile)
  static_assert(64 % RB == 0, "batches must not straddle tiles");
  const int bh = blockIdx.y;
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane / LPR, cl = lane % LPR, c8 = cl * 8;
  m.init(blockIdx.x);
  if (!m.live(wid * 128)) return;  // rows per head are a multiple of 128
  const bool first_bh = bh == 0;
  const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)bh * a.S_in * D + c8;
  const int64_t rowbase = (int64_t)bh * a.S_out;

  float acc[8];
  int cnt = 0, tcnt = 0;  // (meaningful in the first row group)
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;

  for (int o0 = 0; o0 < 128; o0 += RB) {
    float xv[NB][8];
    bool ok[NB];
    int64_t grow[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int r = wid * 128 + o0 + b * RPI + sub;
      const int64_t tok = m.token(r);
      grow[b] = m.row(r);
      ok[b] = tok >= 0 && (a.valid ? (a.valid[tok] != 0) : true);
      if (tok >= 0) {
        load8<T>(x + tok * D, xv[b]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[b][j] = 0.0f;
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (a.out_rows) {
        uint4 u;
        u.x = (uint32_t)f2bf(xv[b][0]) | ((uint32_t)f2bf(xv[b][1]) << 16);
        u.y = (uint32_t)f2bf(xv[b][2]) | ((uint32_t)f2bf(xv[b][3]) << 16);
        u.z = (uint32_t)f2bf(xv[b][4]) | ((uint32_t)f2bf(xv[b][5]) << 16);
        u.w = (uint32_t)f2bf(xv[b][6]) | ((uint32_t)f2bf(xv[b][7]) << 16);
        *reinterpret_cast<uint4*>(a.out_rows + (rowbase + grow[b]) * D + c8) = u;
      }
      if (a.rowdot) {
        float y[8];
        load8<uint16_t>(a.dot_with + (rowbase + grow[b]) * D + c8, y);
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) part = __builtin_fmaf(xv[b][j], y[j], part);
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
        if (cl == 0) a.rowdot[rowbase + grow[b]] = part;
      }
      if (first_bh && cl == 0 && a.valid_re) a.valid_re[grow[b]] = ok[b] ? 1 : 0;
    }
    if (POOL) {
      // this lane's row of each instruction, in row order within its group;
      // valid rows counted from one ballot per instruction (a lane per row)
      constexpr uint64_t kRowLead = LPR == 16 ? 0x0001000100010001ull : 0x0101010101010101ull;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = ok[b] ? acc[j] + xv[b][j] : acc[j];
        const int nv = __popcll(__ballot(ok[b]) & kRowLead);
        cnt += nv;
        tcnt += nv;
      }
      const int rlast = wid * 128 + o0 + RB - 1;
      if ((rlast + 1) % m.bsz == 0) {  // block complete
        const int64_t blk = m.block(rlast);
        if (blk < a.N_b) {
          if (a.block_mean) {
            float sum[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) sum[j] = acc[j];
#pragma unroll
            for (int g = 1; g < RPI; ++g)
#pragma unroll
              for (int j = 0; j < 8; ++j) sum[j] = sum[j] + __shfl(acc[j], g * LPR + cl, 64);
            if (sub == 0) {
              const float den = (float)(cnt > 0 ? cnt : 1);
              float* dst = a.block_mean + ((int64_t)bh * a.N_b + blk) * D + c8;
#pragma unroll
              for (int j = 0; j < 8; ++j) dst[j] = sum[j] / den;
            }
          }
          if (first_bh && lane == 0 && a.block_count) a.block_count[blk] = cnt;
        }
        cnt = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
      }
      if ((rlast + 1) % 64 == 0) {  // tile complete
        if (first_bh && lane == 0 && a.tile_count) a.tile_count[m.row(rlast) >> 6] = tcnt;
        tcnt = 0;
      }
    }
  }
}

// grid (units, B*H): tile-order bf16 rows (S_out per head) -> THW rows of
// dtype TO (S_in per head); padding rows are dropped.  Each lane moves 16
// bytes (8 channels): a wave instruction covers 64 / (D / 8) rows, and NB
// instructions are in flight per wave.
template <int D, typename TO, typename Map>
__global__ __launch_bounds__(kGatherThreads) void scatter_rows_kernel(const uint16_t* __restrict__ in, int64_t S_in,
                                                                      int64_t S_out, Map m, TO* __restrict__ out) {
  constexpr int LPR = D / 8;     // lanes per row
  constexpr int RPI = 64 / LPR;  // rows per wave instruction
  constexpr int NB = 4;          // wave instructions in flight
  constexpr int RB = RPI * NB;   // rows per batch
  static_assert(128 % RB == 0, "a wave's 128 rows split into whole batches");
  const int bh = blockIdx.y;
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane / LPR, c8 = (lane % LPR) * 8;
  m.init(blockIdx.x);
  if (!m.live(wid * 128)) return;
  const uint16_t* inh = in + (int64_t)bh * S_out * D + c8;
  TO* outh = out + (int64_t)bh * S_in * D + c8;
  for (int o0 = 0; o0 < 128; o0 += RB) {
    uint4 v[NB];
    int64_t tok[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int r = wid * 128 + o0 + b * RPI + sub;
      tok[b] = m.token(r);
      if (tok[b] >= 0) v[b] = *reinterpret_cast<const uint4*>(inh + m.row(r) * D);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (tok[b] < 0) continue;
      TO* dst = outh + tok[b] * D;
      if (sizeof(TO) == 2) {
        *reinterpret_cast<uint4*>(dst) = v[b];
      } else {
        const uint32_t w[4] = {v[b].x, v[b].y, v[b].z, v[b].w};
        float4 lo, hi;
        lo.x = __uint_as_float(w[0] << 16); lo.y = __uint_as_float(w[0] & 0xffff0000u);
        lo.z = __uint_as_float(w[1] << 16); lo.w = __uint_as_float(w[1] & 0xffff0000u);
        hi.x = __uint_as_float(w[2] << 16); hi.y = __uint_as_float(w[2] & 0xffff0000u);
        hi.z = __uint_as_float(w[3] << 16); hi.w = __uint_as_float(w[3] & 0xffff0000u);
        reinterpret_cast<float4*>(dst)[0] = lo;
        reinterpret_cast<float4*>(dst)[1] = hi;
      }
    }
  }
}

template <typename Map, bool POOL>
void launch_gather_t(const GatherArgs& a, const Map& m, int dtype, int D, dim3 grid, hipStream_t stream) {
  if (dtype == PRISM_BF16) {
    if (D == 128) gather_pool_kernel<128, uint16_t, Map, POOL><<<grid, kGatherThreads, 0, stream>>>(a, m);
    else gather_pool_kernel<64, uint16_t, Map, POOL><<<grid, kGatherThreads, 0, stream>>>(a, m);
  } else {
    if (D == 128) gather_pool_kernel<128, float, Map, POOL><<<grid, kGatherThreads, 0, stream>>>(a, m);
    else gather_pool_kernel<64, float, Map, POOL><<<grid, kGatherThreads, 0, stream>>>(a, m);
  }
}
template <typename Map>
void launch_gather(const GatherArgs& a, const Map& m, int dtype, int D, dim3 grid, hipStream_t stream) {
  if (a.block_mean != nullptr || a.block_count != nullptr || a.tile_count != nullptr)
    launch_gather_t<Map, true>(a, m, dtype, D, grid, stream);
  else
    launch_gather_t<Map, false>(a, m, dtype, D, grid, stream);
}

template <typename Map>
void launch_scatter(const void* in_rows, int64_t S_in, int64_t S_out, const Map& m, void* out, int out_dtype, int D,
                    dim3 grid, hipStream_t stream) {
  const uint16_t* in = (const uint16_t*)in_rows;
  if (out_dtype == PRISM_BF16) {
    if (D == 128) scatter_rows_kernel<128, uint16_t, Map><<<grid, kGatherThreads, 0, stream>>>(in, S_in, S_out, m, (uint16_t*)out);
    else scatter_rows_kernel<64, uint16_t, Map><<<grid, kGatherThreads, 0, stream>>>(in, S_in, S_out, m, (uint16_t*)out);
  } else {
    if (D == 128) scatter_rows_kernel<128, float, Map><<<grid, kGatherThreads, 0, stream>>>(in, S_in, S_out, m, (float*)out);
    else scatter_rows_kernel<64, float, Map><<<grid, kGatherThreads, 0, stream>>>(in, S_in, S_out, m, (float*)out);
  }
}

ZoneMap zone_map(const int64_t* shape_ids, const int32_t* block_offset, int Hg, int Wg, GridBox box) {
  ZoneMap m = {};
  m.shape_ids = shape_ids; m.block_offset = block_offset; m.ZH = Hg / 8; m.ZW = Wg / 8; m.box = box;
  return m;
}

// validates a chunk geometry; returns PRISM_OK or sets the error
int chunk_map(int T, int Hg, int Wg, int Tp, int Hp, int Wp, int ct, int ch, int cw, int64_t S_out, const char* who,
              ChunkMap* m) {
  PRISM_REQUIRE(T > 0 && Hg > 0 && Wg > 0 && ct > 0 && ch > 0 && cw > 0, "%s: empty grid or chunk", who);
  PRISM_REQUIRE(Tp >= T && Hp >= Hg && Wp >= Wg && Tp % ct == 0 && Hp % ch == 0 && Wp % cw == 0,
                "%s: padded grid (%d,%d,%d) must cover the grid and be multiples of the chunk (%d,%d,%d)", who, Tp, Hp,
                Wp, ct, ch, cw);
  const int bsz = ct * ch * cw;
  PRISM_REQUIRE(bsz == 64 || bsz == 128, "%s: chunk of %d tokens unsupported (64 or 128)", who, bsz);
  const int64_t Sp = (int64_t)Tp * Hp * Wp;
  PRISM_REQUIRE(S_out >= Sp && S_out % 128 == 0, "%s: rows per head must be a multiple of 128 and >= T*H*W padded",
                who);
  *m = ChunkMap{};
  m->T = T; m->Hg = Hg; m->Wg = Wg; m->ct = ct; m->ch = ch; m->cw = cw; m->Nh = Hp / ch; m->Nw = Wp / cw;
  m->Sp = Sp; m->S_out = S_out; m->bsz = bsz;
  return PRISM_OK;
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
                      const int64_t* shape_ids, const int32_t* block_offset, int T, int Hg, int Wg, int Tin, int Hin,
                      int Win, int64_t N_b, void* out_rows, float* block_mean, int32_t* block_count,
                      int32_t* tile_count, uint8_t* valid_re, const void* dot_with, float* rowdot,
                      hipStream_t stream) {
  PRISM_REQUIRE(x && shape_ids && block_offset, "prism_gather_pool: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_gather_pool: grid (%d,%d,%d) must be multiples of 8", T, Hg, Wg);
  PRISM_REQUIRE(box_ok(T, Hg, Wg, Tin, Hin, Win), "prism_gather_pool: input grid (%d,%d,%d) must fit the zone grid",
                Tin, Hin, Win);
  PRISM_REQUIRE((int64_t)Tin * Hin * Win == S, "prism_gather_pool: Tin*Hin*Win != S");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_gather_pool: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(B >= 1 && H >= 1, "prism_gather_pool: B, H must be >= 1");
  PRISM_REQUIRE(dtype == PRISM_F32 || dtype == PRISM_BF16, "prism_gather_pool: bad dtype");
  PRISM_REQUIRE((dot_with == nullptr) == (rowdot == nullptr), "prism_gather_pool: dot_with and rowdot go together");
  PRISM_REQUIRE((block_mean == nullptr && block_count == nullptr) || N_b > 0,
                "prism_gather_pool: N_b required for pooling and block counts");
  GatherArgs a = {};
  const int64_t S_out = (int64_t)T * Hg * Wg;
  a.x = x; a.valid = valid; a.S_in = S; a.S_out = S_out; a.N_b = N_b;
  a.out_rows = (uint16_t*)out_rows; a.block_mean = block_mean;
  a.block_count = block_count; a.tile_count = tile_count; a.valid_re = valid_re;
  a.dot_with = (const uint16_t*)dot_with; a.rowdot = rowdot;
  launch_gather(a, zone_map(shape_ids, block_offset, Hg, Wg, GridBox{Tin, Hin, Win}), dtype, D,
                dim3((unsigned)(S_out / 512), B * H), stream);
  PRISM_LAUNCH_CHECK("prism_gather_pool");
  return PRISM_OK;
}

int prism_scatter_rows(const void* in_rows, int B, int H, int64_t S, int D, const int64_t* shape_ids, int T, int Hg,
                       int Wg, int Tin, int Hin, int Win, void* out, int out_dtype, hipStream_t stream) {
  PRISM_REQUIRE(in_rows && shape_ids && out, "prism_scatter_rows: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_scatter_rows: grid must be multiples of 8");
  PRISM_REQUIRE(box_ok(T, Hg, Wg, Tin, Hin, Win), "prism_scatter_rows: input grid must fit the zone grid");
  PRISM_REQUIRE((int64_t)Tin * Hin * Win == S, "prism_scatter_rows: Tin*Hin*Win != S");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_scatter_rows: head_dim %d unsupported", D);
  PRISM_REQUIRE(out_dtype == PRISM_F32 || out_dtype == PRISM_BF16, "prism_scatter_rows: bad dtype");
  const int64_t S_out = (int64_t)T * Hg * Wg;
  launch_scatter(in_rows, S, S_out, zone_map(shape_ids, nullptr, Hg, Wg, GridBox{Tin, Hin, Win}), out, out_dtype, D,
                 dim3((unsigned)(S_out / 512), B * H), stream);
  PRISM_LAUNCH_CHECK("prism_scatter_rows");
  return PRISM_OK;
}

int prism_chunk_gather_pool(const void* x, int dtype, int B, int H, int D, const uint8_t* valid, int T, int Hg, int Wg,
                            int Tp, int Hp, int Wp, int ct, int ch, int cw, int64_t S_out, void* out_rows,
                            float* block_mean, int32_t* block_count, int32_t* tile_count, uint8_t* valid_re,
                            const void* dot_with, float* rowdot, hipStream_t stream) {
  PRISM_REQUIRE(x, "prism_chunk_gather_pool: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_chunk_gather_pool: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(B >= 1 && H >= 1, "prism_chunk_gather_pool: B, H must be >= 1");
  PRISM_REQUIRE(dtype == PRISM_F32 || dtype == PRISM_BF16, "prism_chunk_gather_pool: bad dtype");
  PRISM_REQUIRE((dot_with == nullptr) == (rowdot == nullptr), "prism_chunk_gather_pool: dot_with and rowdot go together");
  ChunkMap m;
  int rc = chunk_map(T, Hg, Wg, Tp, Hp, Wp, ct, ch, cw, S_out, "prism_chunk_gather_pool", &m);
  if (rc) return rc;
  GatherArgs a = {};
  a.x = x; a.valid = valid; a.S_in = (int64_t)T * Hg * Wg; a.S_out = S_out; a.N_b = m.Sp / m.bsz;
  a.out_rows = (uint16_t*)out_rows; a.block_mean = block_mean;
  a.block_count = block_count; a.tile_count = tile_count; a.valid_re = valid_re;
  a.dot_with = (const uint16_t*)dot_with; a.rowdot = rowdot;
  launch_gather(a, m, dtype, D, dim3((unsigned)((S_out + 511) / 512), B * H), stream);
  PRISM_LAUNCH_CHECK("prism_chunk_gather_pool");
  return PRISM_OK;
}

int prism_chunk_scatter_rows(const void* in_rows, int B, int H, int D, int T, int Hg, int Wg, int Tp, int Hp, int Wp,
                             int ct, int ch, int cw, int64_t S_out, void* out, int out_dtype, hipStream_t stream) {
  PRISM_REQUIRE(in_rows && out, "prism_chunk_scatter_rows: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_chunk_scatter_rows: head_dim %d unsupported", D);
  PRISM_REQUIRE(out_dtype == PRISM_F32 || out_dtype == PRISM_BF16, "prism_chunk_scatter_rows: bad dtype");
  ChunkMap m;
  int rc = chunk_map(T, Hg, Wg, Tp, Hp, Wp, ct, ch, cw, S_out, "prism_chunk_scatter_rows", &m);
  if (rc) return rc;
  launch_scatter(in_rows, (int64_t)T * Hg * Wg, S_out, m, out, out_dtype, D,
                 dim3((unsigned)((S_out + 511) / 512), B * H), stream);
  PRISM_LAUNCH_CHECK("prism_chunk_scatter_rows");
  return PRISM_OK;
}

}  // extern "C"
