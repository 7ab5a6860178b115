// A2V bridge output projection with the per-token residual norm fused into
// its epilogue (gfx950, bf16 MFMA).
//
// Reference: the a2v bridge residual is ConditionalCrossAttention's output
// projection, delta_h = self.o(x) = x W^T + b (nn.Linear(dim, dim),
// hymm/models/modules/interactionv2.py:225, :348), stored as
// a2v_bridge_residual (hymm/models/modules/mova.py:127-137), whose per-token
// L2 norms drive the audio terms of the shape choice
// (hymm/models/modules/wan_video_dit.py:742-752: residual.norm(dim=-1)).  The
// reference runs the projection and then reads the [S, C] residual again for
// the norms; here the norm is formed while the projection's output tiles are
// still in registers.
//
// Kernels:
//   linear_rownorm_kernel  y[M,N] = x[M,K] W[N,K]^T + b (bf16 out, fp32
//                          accumulate) and, per row m and 256-column tile t,
//                          partial[m][t] = sum over the tile's columns of
//                          bf16(y)^2 (the squares of the stored values)
//   rownorm_finish_kernel  norms[m] = sqrt(sum_t partial[m][t]), t ascending
//
// MI355X design: one 256 x 256 output tile per workgroup of four waves (one
// per SIMD), each wave 128 x 128 = 4 x 4 blocks of v_mfma_f32_32x32x16_bf16
// (256 accumulator registers; the tile computes C^T = W x^T, so each lane owns
// one output row and four consecutive columns per register quad).  K steps of
// 64, double-buffered: the x and W tiles of step k + 1 (2 x 32 KB) are copied
// HBM -> LDS by global_load_lds_dwordx4 while step k is multiplied, the copy
// instructions spread between the step's MFMA groups.  LDS rows are 128
// bytes, unpadded, with the 16-byte chunks of row r XOR-swizzled by
// (r >> 1) & 7, so the row-operand reads (16 consecutive rows, one chunk
// each, per 16 lanes) hit distinct bank groups.  Workgroup
// ids are ordered so that each XCD (own L2) works on about 8 x 4 neighbouring
// output tiles at a time, which share their k-slices of x and W in its L2.
// Deterministic (no atomics).
//
// Measured at the config-4 shape (M = 302,400, N = K = 5,120): 15.3-16.7 ms,
// 1.0 PFLOP/s.  The kernel is bound by streaming its tiles from L2 into LDS:
// a copies-only variant (no MFMAs) takes 11.4 ms (124 GB of tile copies at
// 10.9 TB/s), an MFMA-only variant (no copies) 13 ms; torch's F.linear
// (hipBLASLt) plus prism_a2v_norms takes 11.0 ms for the same outputs.
#include "common.h"
#include "mfma.h"
#include "tile_dma.h"

namespace {

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kStages = 2;                         // the copies of step k + 1 run while step k is multiplied
constexpr int kRowBytes = kBK * 2;                 // 128
constexpr int kTileBytes = kBM * kRowBytes;        // 32 KB (x or W tile of one stage)
constexpr int kStageBytes = 2 * kTileBytes;        // 64 KB
constexpr int kOprojThreads = 256;                 // 4 waves
constexpr int kTileKB = kTileBytes / 1024;         // 32
constexpr int kCopiesPerWave = kStageBytes / 1024 / 4;  // 16 KB-instructions per wave and stage
constexpr int kGroupM = 4;                         // output-tile rows per group of the launch order

struct OprojArgs {
  const uint16_t* x;     // [M, K]
  const uint16_t* w;     // [N, K]
  const uint16_t* bias;  // [N] or null
  int64_t M;
  int N, K;
  int mtiles, ntiles;    // ceil(M / 256), N / 256
  uint16_t* y;           // [M, N]
  float* partial;        // [M, ntiles]
};

// byte offset of logical 16-byte chunk c (0..7) of tile row r: chunks XOR-
// swizzled by (r >> 1) & 7, so that the 16 rows one 16-lane group reads
// (one chunk each) fall in 16 distinct 16-byte bank groups (two rows per
// 256-byte bank line: (r & 1, (r >> 1) & 7) differ for 16 consecutive rows)
__device__ __forceinline__ uint32_t swz(int r, int c) { return (uint32_t)(r * kRowBytes + 16 * (c ^ ((r >> 1) & 7))); }

__global__ __launch_bounds__(kOprojThreads, 1) void linear_rownorm_kernel(OprojArgs a) {
  __shared__ __align__(16) uint8_t smem[kStages * kStageBytes];
  __shared__ float sNorm[2][kBM];  // the two n-halves' row partials

  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const int mh = w & 1, nh = w >> 1;

  // Launch order.  Hardware id b runs on XCD b & 7: each XCD takes a
  // contiguous range of logical ids; logical ids walk groups of kGroupM
  // output-tile rows column by column, so the ~32 workgroups an XCD runs at
  // once cover about 4 x 8 tiles and share each k-slice of x (8 ways) and W
  // (4 ways) in that XCD's L2 (4-row groups measured 4% faster than 8-row
  // groups; plain row order was within 1%).
  const int nwg = (int)gridDim.x;
  const int b = (int)blockIdx.x;
  const int per = nwg / 8;
  const int lid = b < per * 8 ? (b & 7) * per + (b >> 3) : b;
  const int gsize = kGroupM * a.ntiles;
  const int grp = lid / gsize, first_m = grp * kGroupM;
  const int gm = a.mtiles - first_m < kGroupM ? a.mtiles - first_m : kGroupM;
  const int inner = lid - grp * gsize;
  const int mt = first_m + inner % gm, nt = inner / gm;
  const int64_t m0 = (int64_t)mt * kBM;
  const int n0 = nt * kBN;

  // DMA plan: KB-instruction i of a stage covers tile bytes [1024 i', 1024 i' + 1024)
  // of the x tile (i < 32, i' = i) or the W tile (i' = i - 32); lane L of it
  // writes 16 bytes at 16 L: row (1024 i' + 16 L) / 128, stored chunk L % 8,
  // logical chunk (L % 8) ^ ((row >> 1) & 7).  Wave w issues i = w + 4 s.
  uint32_t voff0[kCopiesPerWave];  // byte offset of this lane's 16 bytes at k = 0, from the tensor's base
#pragma unroll
  for (int s = 0; s < kCopiesPerWave; ++s) {
    const int i = w + 4 * s;
    const int tb = (i % kTileKB) * 1024 + 16 * lane;
    const int row = tb / kRowBytes, sc = (tb % kRowBytes) / 16;
    const int c = sc ^ ((row >> 1) & 7);
    int64_t grow;
    if (i < kTileKB) {
      grow = m0 + row;
      if (grow >= a.M) grow = a.M - 1;  // rows past M re-read the last row (never stored)
    } else {
      grow = n0 + row;
    }
    voff0[s] = (uint32_t)((grow * a.K + 8 * c) * 2);
  }
  const uint32_t lds0 = lds_addr(smem);
  const void* xb = uniform_ptr(a.x);
  const void* wb = uniform_ptr(a.w);
  // copies [q0, q1) of this wave for k-step kstep into stage st
  auto issue = [&](int kstep, int st, int q0, int q1) {
    const uint32_t base = lds0 + (uint32_t)(st * kStageBytes);
    const uint32_t kb = (uint32_t)kstep * (uint32_t)kRowBytes;
#pragma unroll
    for (int s = 0; s < kCopiesPerWave; ++s) {
      if (s < q0 || s >= q1) continue;
      const int i = w + 4 * s;
      dma_b128(voff0[s] + kb, i < kTileKB ? xb : wb, base + (uint32_t)i * 1024u);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_zero();

  const int nsteps = a.K / kBK;
  // operand fragments of k-step s: A = W rows 128 nh + 32 i + l32, B = x rows
  // 128 mh + 32 i + l32, logical chunk 2 s + g; chunk 2 s + g of row r sits at
  // the offset of chunk g XOR 32 s (the swizzle XORs the chunk index, and 2 s
  // only touches its upper bit)
  uint32_t offA[4], offB[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    offA[i] = (uint32_t)kTileBytes + swz(nh * 128 + 32 * i + l32, g);
    offB[i] = swz(mh * 128 + 32 * i + l32, g);
  }
  auto load_ops = [&](const uint8_t* st, int s, bf16x8* av, bf16x8* bv) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      av[i] = *reinterpret_cast<const bf16x8*>(st + (offA[i] ^ (uint32_t)(32 * s)));
      bv[i] = *reinterpret_cast<const bf16x8*>(st + (offB[i] ^ (uint32_t)(32 * s)));
    }
  };
  constexpr int KS = kBK / 16;                  // k-steps per stage
  constexpr int QC = kCopiesPerWave / KS;       // copies issued after each k-step's MFMAs
  issue(0, 0, 0, kCopiesPerWave);
  for (int ks = 0; ks < nsteps; ++ks) {
    dma_wait_all();
    __syncthreads();
    const bool more = ks + 1 < nsteps;
    const uint8_t* sp = smem + (ks & 1) * kStageBytes;
    // software pipeline over the stage's k-steps: the fragments of step s + 1
    // are read while the sixteen MFMAs of step s run, and a quarter of the
    // next stage's copies is issued after each step's MFMAs (a wave stalls
    // while its copy instructions queue; spread out, they hide behind MFMAs)
    bf16x8 av[2][4], bv[2][4];
    load_ops(sp, 0, av[0], bv[0]);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if (s + 1 < KS) load_ops(sp, s + 1, av[(s + 1) & 1], bv[(s + 1) & 1]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[s & 1][i], bv[s & 1][j], acc[i][j], 0, 0, 0);
      if (s == 0) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // step 0 reads first
      if (s + 1 < KS) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (more) issue(ks + 1, (ks + 1) & 1, s * QC, s * QC + QC);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // epilogue: acc[i][j] register r holds C^T[n][m] with
  // n = n0 + 128 nh + 32 i + 8 (r >> 2) + 4 g + (r & 3), m = m0 + 128 mh + 32 j + l32
  float ss[4];  // squares of the stored values of this lane's row, per m block
#pragma unroll
  for (int j = 0; j < 4; ++j) ss[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n0 + 128 * nh + 32 * i + 8 * q + 4 * g;
      float bb[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (a.bias) {
        const uint2 u = *reinterpret_cast<const uint2*>(a.bias + n);
        bb[0] = __uint_as_float(u.x << 16); bb[1] = __uint_as_float(u.x & 0xffff0000u);
        bb[2] = __uint_as_float(u.y << 16); bb[3] = __uint_as_float(u.y & 0xffff0000u);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t m = m0 + 128 * mh + 32 * j + l32;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = round_bf(acc[i][j][4 * q + e] + bb[e]);
#pragma unroll
        for (int e = 0; e < 4; ++e) ss[j] = __builtin_fmaf(v[e], v[e], ss[j]);
        if (m < a.M) {
          uint2 o;
          o.x = pack_bf16(v[0], v[1]);
          o.y = pack_bf16(v[2], v[3]);
          *reinterpret_cast<uint2*>(a.y + m * a.N + n) = o;
        }
      }
    }
  }
  // row partial of this wave (its 128 columns): the two lane halves hold
  // different columns of the same row
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float t = xor32_add(ss[j]);
    if (g == 0) sNorm[nh][128 * mh + 32 * j + l32] = t;
  }
  __syncthreads();
  for (int r = tid; r < kBM; r += kOprojThreads) {
    const int64_t m = m0 + r;
    if (m < a.M) a.partial[m * a.ntiles + nt] = sNorm[0][r] + sNorm[1][r];
  }
}

template <typename TO>
__global__ __launch_bounds__(256) void rownorm_finish_kernel(const float* __restrict__ partial, int64_t M, int nt,
                                                              TO* __restrict__ norms) {
  const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (m >= M) return;
  float s = 0.0f;
  for (int t = 0; t < nt; ++t) s = s + partial[m * nt + t];
  const float r = sqrtf(s);
  if (sizeof(TO) == 2) reinterpret_cast<uint16_t*>(norms)[m] = f2bf(r);
  else reinterpret_cast<float*>(norms)[m] = r;
}

}  // namespace

extern "C" {

int prism_linear_rownorm(const void* x, const void* w, const void* bias, int64_t M, int N, int K, void* y, void* norms,
                         int norms_dtype, float* partial, hipStream_t stream) {
  PRISM_REQUIRE(x && w && y && norms && partial, "prism_linear_rownorm: null pointer");
  PRISM_REQUIRE(M >= 1, "prism_linear_rownorm: M must be >= 1");
  PRISM_REQUIRE(N >= kBN && N % kBN == 0, "prism_linear_rownorm: N=%d must be a positive multiple of %d", N, kBN);
  PRISM_REQUIRE(K >= 64 && K % 64 == 0, "prism_linear_rownorm: K=%d must be a positive multiple of 64", K);
  PRISM_REQUIRE(norms_dtype == PRISM_F32 || norms_dtype == PRISM_BF16, "prism_linear_rownorm: bad norms dtype");
  // per-lane source offsets are 32-bit byte offsets from the tensors' bases
  PRISM_REQUIRE(M * (int64_t)K * 2 < (1ll << 32) && (int64_t)N * K * 2 < (1ll << 32),
                "prism_linear_rownorm: x and W must each be smaller than 4 GiB");
  const int64_t mtiles = (M + kBM - 1) / kBM;
  const int ntiles = N / kBN;
  PRISM_REQUIRE(mtiles * ntiles < (1ll << 31), "prism_linear_rownorm: grid too large");
  OprojArgs a;
  a.x = (const uint16_t*)x; a.w = (const uint16_t*)w; a.bias = (const uint16_t*)bias;
  a.M = M; a.N = N; a.K = K; a.mtiles = (int)mtiles; a.ntiles = ntiles; a.y = (uint16_t*)y; a.partial = partial;
  linear_rownorm_kernel<<<(unsigned)(mtiles * ntiles), kOprojThreads, 0, stream>>>(a);
  const unsigned fb = (unsigned)((M + 255) / 256);
  if (norms_dtype == PRISM_BF16) rownorm_finish_kernel<uint16_t><<<fb, 256, 0, stream>>>(partial, M, ntiles, (uint16_t*)norms);
  else rownorm_finish_kernel<float><<<fb, 256, 0, stream>>>(partial, M, ntiles, (float*)norms);
  PRISM_LAUNCH_CHECK("prism_linear_rownorm");
  return PRISM_OK;
}

}  // extern "C"
