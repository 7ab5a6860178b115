// Block-sparse flash attention backward, bf16 MFMA (gfx950).
//
// Reference: attn_bwd_bsa_varlen_triton (bsa_interface.py:387-523):
//   delta = rowsum(O * dO) (common.py:110-127; computed by prism_gather_pool
//   or prism_bwd_preprocess), dK/dV per key tile over the query tiles that
//   selected it (_attn_bwd_dkdv_bsa_varlen_wrapper,
//   flash_attn_bsa_varlen_mask.py:562-704, inner loop :323-402), dQ per query
//   tile over its key tiles (_attn_bwd_dq_bsa_varlen_align_wrapper, :879-1014,
//   inner loop :479-541).  Both passes are deterministic (no atomics), as in the
//   reference.
//
// Layouts (per head, tile order): Q, K, V, dO row-major [S][D]; Q^T, K^T, dO^T
// as transposed 64-row tiles [Nt][D][64] with keys in MFMA k-slot order
// (prism_transpose_tiles).
//
// MI355X design, shared by both kernels:
//  * one workgroup (4 waves) per PAIR of tiles (2p, 2p+1) walking the sorted
//    union of their two lists; waves 0-1 own tile 2p, waves 2-3 tile 2p+1 and
//    skip the math for list entries that are not theirs;
//  * operand tiles are staged HBM -> registers -> LDS with the next tile's
//    loads in flight during the current tile's math (double-buffered LDS,
//    one wave per SIMD); LDS
//    rows are padded so MFMA operand reads are conflict-free 16-byte loads;
//  * workgroup ids are remapped per XCD (contiguous zones per L2).
// dK/dV: wave w owns keys [32w', 32w'+32) of its tile.  S = Q K^T and
// dP = dO V^T keep one key per lane column, so P and dS feed the B operand of
// dV^T = dO^T P and dK^T = Q^T dS straight from the accumulators; the 64 query
// rows are processed in two 32-row halves to bound register pressure.
// dQ: wave w owns 32 queries.  S^T = K Q^T and dP^T = V dO^T keep one query per
// lane column; dQ^T = K^T dS^T.
#include "common.h"
#include "mfma.h"

namespace {

struct BwdArgs {
  const uint16_t *q, *qt, *k, *kt, *v, *do_, *dot;
  const float* lse;         // [BH, S] natural log
  const float* delta;       // [BH, S]
  const uint8_t* kv_valid;  // [S] tile order or null
  const int64_t* start;     // list starts (per key tile for dK/dV, per query tile for dQ)
  const int32_t* len;
  const int32_t* cols;
  int64_t S, Nt;
  int npairs;
  float sm_scale, scale_log2;
  uint16_t *dq, *dk, *dv;
};

constexpr float kLog2e = 1.4426950408889634f;

// merge cursor over two ascending lists (wave-uniform)
struct Union2 {
  const int32_t *A, *B;
  int nA, nB, ia, ib;
  __device__ __forceinline__ bool next(int& t, bool& inA, bool& inB) {
    const int ca = ia < nA ? A[ia] : INT32_MAX;
    const int cb = ib < nB ? B[ib] : INT32_MAX;
    t = ca < cb ? ca : cb;
    inA = ca == t;
    inB = cb == t;
    if (t == INT32_MAX) return false;
    ia += inA;
    ib += inB;
    return true;
  }
};

// Global -> register staging of one bf16 tile of 64*D elements (contiguous in
// HBM) by 256 threads: KCH 16-byte chunks per thread, chunk c = tid + 256 i.
template <int KCH>
__device__ __forceinline__ void stage_load(uint4* r, const uint16_t* __restrict__ g, int tid) {
#pragma unroll
  for (int i = 0; i < KCH; ++i) r[i] = *reinterpret_cast<const uint4*>(g + (tid + i * 256) * 8);
}
// register -> LDS: row-major [64][D] tile with pitch RP
template <int D, int KCH, int RP>
__device__ __forceinline__ void stage_rows(uint16_t* s, const uint4* r, int tid) {
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = tid + i * 256;
    *reinterpret_cast<uint4*>(&s[(c / (D / 8)) * RP + (c % (D / 8)) * 8]) = r[i];
  }
}
// register -> LDS: transposed [D][64] tile with pitch TP
template <int KCH, int TP>
__device__ __forceinline__ void stage_trans(uint16_t* s, const uint4* r, int tid) {
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = tid + i * 256;
    *reinterpret_cast<uint4*>(&s[(c >> 3) * TP + (c & 7) * 8]) = r[i];
  }
}

template <int D>
__global__ __launch_bounds__(256, 1) void bsa_bwd_dkdv_kernel(BwdArgs a) {
  constexpr int RP = D + 8, TP = 64 + 8, NS = D / 16, NDT = D / 32, KCH = 64 * D / 8 / 256;
  __shared__ __align__(16) uint16_t sQ[2][64 * RP];
  __shared__ __align__(16) uint16_t sDO[2][64 * RP];
  __shared__ __align__(16) uint16_t sQT[2][D * TP];
  __shared__ __align__(16) uint16_t sDOT[2][D * TP];
  __shared__ __align__(16) float sM[2][64];
  __shared__ __align__(16) float sDl[2][64];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / a.npairs, pair = logical - bh * a.npairs;
  const int64_t rowA = (int64_t)bh * a.Nt + 2 * pair;
  Union2 u{a.cols + a.start[rowA], a.cols + a.start[rowA + 1], a.len[rowA], a.len[rowA + 1], 0, 0};
  const bool mine_is_b = w >= 2;
  const int64_t hoff = (int64_t)bh * a.S * D;
  const int64_t key = (int64_t)(2 * pair + (w >> 1)) * 64 + 32 * (w & 1) + l32;
  const bool kvalid = a.kv_valid ? a.kv_valid[key] != 0 : true;
  const float NINF = -__builtin_inff();
  const float* lse_h = a.lse + (int64_t)bh * a.S;
  const float* dl_h = a.delta + (int64_t)bh * a.S;

  bf16x8 kf[NS], vf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kf[s] = ld_bf16x8(a.k + hoff + key * D + 16 * s + 8 * g);
    vf[s] = ld_bf16x8(a.v + hoff + key * D + 16 * s + 8 * g);
  }
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) { dk[dt] = f32x16_zero(); dv[dt] = f32x16_zero(); }

  uint4 rq[KCH], rdo[KCH], rqt[KCH], rdot[KCH];
  float rm = 0.0f;
#define PRISM_DKDV_ISSUE(qt_)                                          \
  do {                                                                 \
    const int64_t toff = hoff + (int64_t)(qt_) * 64 * D;               \
    stage_load<KCH>(rq, a.q + toff, tid);                              \
    stage_load<KCH>(rdo, a.do_ + toff, tid);                           \
    stage_load<KCH>(rqt, a.qt + toff, tid);                            \
    stage_load<KCH>(rdot, a.dot + toff, tid);                          \
    if (tid < 64) rm = lse_h[(int64_t)(qt_) * 64 + tid] * kLog2e;      \
    else if (tid < 128) rm = dl_h[(int64_t)(qt_) * 64 + tid - 64];     \
  } while (0)
#define PRISM_DKDV_COMMIT(b)                                           \
  do {                                                                 \
    stage_rows<D, KCH, RP>(sQ[b], rq, tid);                            \
    stage_rows<D, KCH, RP>(sDO[b], rdo, tid);                          \
    stage_trans<KCH, TP>(sQT[b], rqt, tid);                            \
    stage_trans<KCH, TP>(sDOT[b], rdot, tid);                          \
    if (tid < 64) sM[b][tid] = rm;                                     \
    else if (tid < 128) sDl[b][tid - 64] = rm;                         \
  } while (0)

  int qt_cur = 0;
  bool inA = false, inB = false;
  bool more = u.next(qt_cur, inA, inB);
  PRISM_DKDV_ISSUE(more ? qt_cur : 0);
  PRISM_DKDV_COMMIT(0);
  __syncthreads();
  int buf = 0;
  while (more) {
    const bool act = mine_is_b ? inB : inA;
    int qt_nxt = qt_cur;
    bool nA = false, nB = false;
    const bool more_nxt = u.next(qt_nxt, nA, nB);
    PRISM_DKDV_ISSUE(more_nxt ? qt_nxt : qt_cur);
    if (act) {
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        f32x16 sacc = f32x16_zero(), pacc = f32x16_zero();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_bf16x8(&sQ[buf][(32 * qh + l32) * RP + 16 * s + 8 * g]),
                                                         kf[s], sacc, 0, 0, 0);
          pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_bf16x8(&sDO[buf][(32 * qh + l32) * RP + 16 * s + 8 * g]),
                                                         vf[s], pacc, 0, 0, 0);
        }
        // P and dS for rows q = 32qh + 8j + 4g + i (register r = 4j + i), column = this lane's key
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 m4 = *reinterpret_cast<const float4*>(&sM[buf][32 * qh + 8 * j + 4 * g]);
          const float4 d4 = *reinterpret_cast<const float4*>(&sDl[buf][32 * qh + 8 * j + 4 * g]);
          const float mv[4] = {m4.x, m4.y, m4.z, m4.w}, dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * j + i;
            const float p = (kvalid && mv[i] != NINF) ? fast_exp2(__builtin_fmaf(sacc[r], a.scale_log2, -mv[i])) : 0.0f;
            sacc[r] = p;
            pacc[r] = p * (pacc[r] - dv4[i]);
          }
        }
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const int tt = 2 * qh + t2;
          const bf16x8 pb = b_from_acc(&sacc, t2);
          const bf16x8 sb = b_from_acc(&pacc, t2);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_from_t(sDOT[buf], TP, dt, tt, l32, g), pb, dv[dt], 0, 0, 0);
            dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_from_t(sQT[buf], TP, dt, tt, l32, g), sb, dk[dt], 0, 0, 0);
          }
        }
      }
    }
    PRISM_DKDV_COMMIT(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    more = more_nxt;
    qt_cur = qt_nxt;
    inA = nA;
    inB = nB;
  }
#undef PRISM_DKDV_ISSUE
#undef PRISM_DKDV_COMMIT
  uint16_t* dkr = a.dk + hoff + key * D;
  uint16_t* dvr = a.dv + hoff + key * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 o;
      o.x = pack_bf16(dk[dt][4 * j + 0] * a.sm_scale, dk[dt][4 * j + 1] * a.sm_scale);
      o.y = pack_bf16(dk[dt][4 * j + 2] * a.sm_scale, dk[dt][4 * j + 3] * a.sm_scale);
      *reinterpret_cast<uint2*>(dkr + 32 * dt + 8 * j + 4 * g) = o;
      o.x = pack_bf16(dv[dt][4 * j + 0], dv[dt][4 * j + 1]);
      o.y = pack_bf16(dv[dt][4 * j + 2], dv[dt][4 * j + 3]);
      *reinterpret_cast<uint2*>(dvr + 32 * dt + 8 * j + 4 * g) = o;
    }
}

template <int D>
__global__ __launch_bounds__(256, 1) void bsa_bwd_dq_kernel(BwdArgs a) {
  constexpr int RP = D + 8, TP = 64 + 8, NS = D / 16, NDT = D / 32, KCH = 64 * D / 8 / 256;
  __shared__ __align__(16) uint16_t sK[2][64 * RP];
  __shared__ __align__(16) uint16_t sV[2][64 * RP];
  __shared__ __align__(16) uint16_t sKT[2][D * TP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / a.npairs, pair = logical - bh * a.npairs;
  const int64_t rowA = (int64_t)bh * a.Nt + 2 * pair;
  Union2 u{a.cols + a.start[rowA], a.cols + a.start[rowA + 1], a.len[rowA], a.len[rowA + 1], 0, 0};
  const bool mine_is_b = w >= 2;
  const int64_t hoff = (int64_t)bh * a.S * D;
  const int64_t qrow = (int64_t)(2 * pair + (w >> 1)) * 64 + 32 * (w & 1) + l32;
  const bool has_mask = a.kv_valid != nullptr;
  const float NINF = -__builtin_inff();

  bf16x8 qf[NS], df[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = ld_bf16x8(a.q + hoff + qrow * D + 16 * s + 8 * g);
    df[s] = ld_bf16x8(a.do_ + hoff + qrow * D + 16 * s + 8 * g);
  }
  const float mq = a.lse[(int64_t)bh * a.S + qrow] * kLog2e;
  const float dlt = a.delta[(int64_t)bh * a.S + qrow];
  const bool qlive = mq != NINF;
  f32x16 dq[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dq[dt] = f32x16_zero();

  uint4 rk[KCH], rv[KCH], rkt[KCH];
  uint8_t rvalid = 1;
#define PRISM_DQ_ISSUE(kt_)                                                 \
  do {                                                                      \
    const int64_t toff = hoff + (int64_t)(kt_) * 64 * D;                    \
    stage_load<KCH>(rk, a.k + toff, tid);                                   \
    stage_load<KCH>(rv, a.v + toff, tid);                                   \
    stage_load<KCH>(rkt, a.kt + toff, tid);                                 \
    if (has_mask) rvalid = a.kv_valid[(int64_t)(kt_) * 64 + lane];          \
  } while (0)
#define PRISM_DQ_COMMIT(b)                                                  \
  do {                                                                      \
    stage_rows<D, KCH, RP>(sK[b], rk, tid);                                 \
    stage_rows<D, KCH, RP>(sV[b], rv, tid);                                 \
    stage_trans<KCH, TP>(sKT[b], rkt, tid);                                 \
  } while (0)

  int kt_cur = 0;
  bool inA = false, inB = false;
  bool more = u.next(kt_cur, inA, inB);
  PRISM_DQ_ISSUE(more ? kt_cur : 0);
  uint64_t vmask_next = has_mask ? (uint64_t)__ballot(rvalid != 0) : ~0ull;
  PRISM_DQ_COMMIT(0);
  __syncthreads();
  int buf = 0;
  while (more) {
    const bool act = mine_is_b ? inB : inA;
    const uint64_t vmask = vmask_next;
    int kt_nxt = kt_cur;
    bool nA = false, nB = false;
    const bool more_nxt = u.next(kt_nxt, nA, nB);
    PRISM_DQ_ISSUE(more_nxt ? kt_nxt : kt_cur);
    if (act) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        f32x16 sacc = f32x16_zero(), pacc = f32x16_zero();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_bf16x8(&sK[buf][(32 * kh + l32) * RP + 16 * s + 8 * g]),
                                                         qf[s], sacc, 0, 0, 0);
          pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_bf16x8(&sV[buf][(32 * kh + l32) * RP + 16 * s + 8 * g]),
                                                         df[s], pacc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kk = 32 * kh + 8 * (r >> 2) + 4 * g + (r & 3);
          const bool ok = qlive && ((vmask >> kk) & 1ull);
          const float p = ok ? fast_exp2(__builtin_fmaf(sacc[r], a.scale_log2, -mq)) : 0.0f;
          pacc[r] = p * (pacc[r] - dlt);
        }
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const int tt = 2 * kh + t2;
          const bf16x8 sb = b_from_acc(&pacc, t2);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
            dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_from_t(sKT[buf], TP, dt, tt, l32, g), sb, dq[dt], 0, 0, 0);
        }
      }
    }
    vmask_next = has_mask ? (uint64_t)__ballot(rvalid != 0) : ~0ull;
    PRISM_DQ_COMMIT(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    more = more_nxt;
    kt_cur = kt_nxt;
    inA = nA;
    inB = nB;
  }
#undef PRISM_DQ_ISSUE
#undef PRISM_DQ_COMMIT
  uint16_t* dqr = a.dq + hoff + qrow * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 o;
      o.x = pack_bf16(dq[dt][4 * j + 0] * a.sm_scale, dq[dt][4 * j + 1] * a.sm_scale);
      o.y = pack_bf16(dq[dt][4 * j + 2] * a.sm_scale, dq[dt][4 * j + 3] * a.sm_scale);
      *reinterpret_cast<uint2*>(dqr + 32 * dt + 8 * j + 4 * g) = o;
    }
}

// delta[row] = sum_d o[row][d] * do[row][d]: one wave per row, 4 rows per block
template <int D>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(const uint16_t* __restrict__ o, const uint16_t* __restrict__ dO,
                                                             int64_t rows, float* __restrict__ delta) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  float part = 0.0f;
  for (int d = lane; d < D; d += 64) part = __builtin_fmaf(bf2f(o[r * D + d]), bf2f(dO[r * D + d]), part);
  part = wave_sum_xor(part);
  if (lane == 0) delta[r] = part;
}

int check_common(const void* q, const void* k, int BH, int64_t S, int D, const char* who) {
  PRISM_REQUIRE(q && k, "%s: null pointer", who);
  PRISM_REQUIRE(D == 64 || D == 128, "%s: head_dim %d unsupported (64, 128)", who, D);
  PRISM_REQUIRE(S > 0 && S % 128 == 0, "%s: S must be a positive multiple of 128", who);
  PRISM_REQUIRE(BH >= 1 && (int64_t)BH * (S / 128) < (1ll << 31), "%s: BH out of range", who);
  return PRISM_OK;
}

}  // namespace

extern "C" {

int prism_bwd_preprocess(const void* o, const void* do_, int64_t rows, int D, float* delta, hipStream_t stream) {
  PRISM_REQUIRE(o && do_ && delta, "prism_bwd_preprocess: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_bwd_preprocess: head_dim %d unsupported", D);
  if (rows == 0) return PRISM_OK;
  const unsigned blocks = (unsigned)((rows + 3) / 4);
  if (D == 128) bwd_preprocess_kernel<128><<<blocks, 256, 0, stream>>>((const uint16_t*)o, (const uint16_t*)do_, rows, delta);
  else bwd_preprocess_kernel<64><<<blocks, 256, 0, stream>>>((const uint16_t*)o, (const uint16_t*)do_, rows, delta);
  PRISM_LAUNCH_CHECK("prism_bwd_preprocess");
  return PRISM_OK;
}

int prism_bsa_bwd_dkdv(const void* q, const void* qt, const void* k, const void* v, const void* do_, const void* dot,
                       const float* lse, const float* delta, int BH, int64_t S, int D, const uint8_t* kv_valid,
                       const int64_t* kstart, const int32_t* klen, const int32_t* kcols, float sm_scale, void* dk,
                       void* dv, hipStream_t stream) {
  int rc = check_common(q, k, BH, S, D, "prism_bsa_bwd_dkdv");
  if (rc) return rc;
  PRISM_REQUIRE(qt && v && do_ && dot && lse && delta && kstart && klen && kcols && dk && dv,
                "prism_bsa_bwd_dkdv: null pointer");
  BwdArgs a = {};
  a.q = (const uint16_t*)q; a.qt = (const uint16_t*)qt; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v;
  a.do_ = (const uint16_t*)do_; a.dot = (const uint16_t*)dot; a.lse = lse; a.delta = delta; a.kv_valid = kv_valid;
  a.start = kstart; a.len = klen; a.cols = kcols; a.S = S; a.Nt = S / 64; a.npairs = (int)(S / 128);
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
  const unsigned blocks = (unsigned)((int64_t)BH * a.npairs);
  if (D == 128) bsa_bwd_dkdv_kernel<128><<<blocks, 256, 0, stream>>>(a);
  else bsa_bwd_dkdv_kernel<64><<<blocks, 256, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_bwd_dkdv");
  return PRISM_OK;
}

int prism_bsa_bwd_dq(const void* q, const void* k, const void* kt, const void* v, const void* do_, const float* lse,
                     const float* delta, int BH, int64_t S, int D, const uint8_t* kv_valid, const int64_t* qstart,
                     const int32_t* qlen, const int32_t* qcols, float sm_scale, void* dq, hipStream_t stream) {
  int rc = check_common(q, k, BH, S, D, "prism_bsa_bwd_dq");
  if (rc) return rc;
  PRISM_REQUIRE(kt && v && do_ && lse && delta && qstart && qlen && qcols && dq, "prism_bsa_bwd_dq: null pointer");
  BwdArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.kt = (const uint16_t*)kt; a.v = (const uint16_t*)v;
  a.do_ = (const uint16_t*)do_; a.lse = lse; a.delta = delta; a.kv_valid = kv_valid;
  a.start = qstart; a.len = qlen; a.cols = qcols; a.S = S; a.Nt = S / 64; a.npairs = (int)(S / 128);
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dq = (uint16_t*)dq;
  const unsigned blocks = (unsigned)((int64_t)BH * a.npairs);
  if (D == 128) bsa_bwd_dq_kernel<128><<<blocks, 256, 0, stream>>>(a);
  else bsa_bwd_dq_kernel<64><<<blocks, 256, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_bwd_dq");
  return PRISM_OK;
}

}  // extern "C"
