// Block-sparse flash attention backward, bf16 MFMA (gfx950).
//
// Reference: attn_bwd_bsa_varlen_triton (bsa_interface.py:387-523):
//   delta = rowsum(O * dO) (common.py:110-127; computed by prism_gather_pool),
//   dK/dV per key tile over the query tiles that selected it
//   (_attn_bwd_dkdv_bsa_varlen_wrapper, flash_attn_bsa_varlen_mask.py:562-704,
//   inner loop :323-402), dQ per query tile over its key tiles
//   (_attn_bwd_dq_bsa_varlen_align_wrapper, :879-1014, inner loop :479-541).
// Both passes are deterministic (no atomics), as in the reference.
//
// Layouts (per head, tile order): Q, K, V, dO row-major [S][D]; Q^T, K^T, dO^T
// as transposed 64-row tiles [Nt][D][64], so every MFMA operand is read with
// contiguous 8- or 16-byte LDS loads.
//
// dK/dV: workgroup = key tile, wave w owns keys [32w, 32w+32).  S = Q K^T and
// dP = dO V^T keep one key per lane column, so P and dS feed the B operand of
// dV^T = dO^T P and dK^T = Q^T dS straight from the accumulators.
// dQ: workgroup = query tile, wave w owns queries [32w, 32w+32).  S^T = K Q^T and
// dP^T = V dO^T keep one query per lane column; dQ^T = K^T dS^T.
#include "common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const __bf16 x = (__bf16)a, y = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}
// B operand (16 rows x 32 cols) built from a 32x32 accumulator pair: rows
// 16tt + {4g + i, 8 + 4g + i} of the 64-row C block held as acc[tt/2]
__device__ __forceinline__ bf16x8 b_from_acc(const f32x16* acc, int tt) {
  const int h = tt >> 1, j0 = 2 * (tt & 1);
  uint4 pb;
  pb.x = pack_bf16(acc[h][4 * j0 + 0], acc[h][4 * j0 + 1]);
  pb.y = pack_bf16(acc[h][4 * j0 + 2], acc[h][4 * j0 + 3]);
  pb.z = pack_bf16(acc[h][4 * j0 + 4], acc[h][4 * j0 + 5]);
  pb.w = pack_bf16(acc[h][4 * j0 + 6], acc[h][4 * j0 + 7]);
  return as_bf16x8(pb);
}
// A operand (32 rows x 16 k) from a transposed tile [D][pitch]: row 32dt + l32,
// k slots 16tt + {4g .. 4g+3, 8+4g .. 8+4g+3}
__device__ __forceinline__ bf16x8 a_from_t(const uint16_t* sT, int pitch, int dt, int tt, int l32, int g) {
  const uint16_t* p = sT + (32 * dt + l32) * pitch + 16 * tt + 4 * g;
  const uint2 lo = *reinterpret_cast<const uint2*>(p);
  const uint2 hi = *reinterpret_cast<const uint2*>(p + 8);
  return as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
}

struct BwdArgs {
  const uint16_t *q, *qt, *k, *kt, *v, *do_, *dot;
  const float* lse;        // [BH, S] natural log
  const float* delta;      // [BH, S]
  const uint8_t* kv_valid; // [S] tile order or null
  const int64_t* start;    // list starts (per key tile for dK/dV, per query tile for dQ)
  const int32_t* len;
  const int32_t* cols;
  int64_t S, Nt;
  float sm_scale, scale_log2;
  uint16_t *dq, *dk, *dv;
};

constexpr float kLog2e = 1.4426950408889634f;

template <int D>
__global__ __launch_bounds__(128, 1) void bsa_bwd_dkdv_kernel(BwdArgs a) {
  constexpr int RP = D + 8, TP = 68, NS = D / 16, NDT = D / 32, KCH = 64 * D / 8 / 128;
  __shared__ __align__(16) uint16_t sQ[64 * RP];
  __shared__ __align__(16) uint16_t sDO[64 * RP];
  __shared__ __align__(16) uint16_t sQT[D * TP];
  __shared__ __align__(16) uint16_t sDOT[D * TP];
  __shared__ float sM[64], sDl[64];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int kt = blockIdx.x, bh = blockIdx.y;
  const int64_t row = (int64_t)bh * a.Nt + kt;
  const int n = a.len[row];
  const int32_t* cols = a.cols + a.start[row];
  const int64_t hoff = (int64_t)bh * a.S * D;
  const int64_t key = (int64_t)kt * 64 + 32 * w + l32;
  const bool kvalid = a.kv_valid ? a.kv_valid[key] != 0 : true;
  const float NINF = -__uint_as_float(0x7f800000u);

  bf16x8 kf[NS], vf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(a.k + hoff + key * D + 16 * s + 8 * g));
    vf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(a.v + hoff + key * D + 16 * s + 8 * g));
  }
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) { dk[dt][r] = 0.0f; dv[dt][r] = 0.0f; }

  for (int it = 0; it < n; ++it) {
    const int64_t qt = cols[it];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * 128;
      const int r = c / (D / 8), c8 = c % (D / 8);
      const int64_t src = hoff + (qt * 64 + r) * D + c8 * 8;
      *reinterpret_cast<uint4*>(&sQ[r * RP + c8 * 8]) = *reinterpret_cast<const uint4*>(a.q + src);
      *reinterpret_cast<uint4*>(&sDO[r * RP + c8 * 8]) = *reinterpret_cast<const uint4*>(a.do_ + src);
      const int d = c >> 3, k8 = c & 7;
      const int64_t srct = hoff + (qt * D + d) * 64 + k8 * 8;
      *reinterpret_cast<uint4*>(&sQT[d * TP + k8 * 8]) = *reinterpret_cast<const uint4*>(a.qt + srct);
      *reinterpret_cast<uint4*>(&sDOT[d * TP + k8 * 8]) = *reinterpret_cast<const uint4*>(a.dot + srct);
    }
    if (tid < 64) {
      sM[tid] = a.lse[(int64_t)bh * a.S + qt * 64 + tid] * kLog2e;
      sDl[tid] = a.delta[(int64_t)bh * a.S + qt * 64 + tid];
    }
    __syncthreads();

    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
#pragma unroll
      for (int r = 0; r < 16; ++r) { sacc[qh][r] = 0.0f; pacc[qh][r] = 0.0f; }
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bf16x8 qa = as_bf16x8(*reinterpret_cast<const uint4*>(&sQ[(32 * qh + l32) * RP + 16 * s + 8 * g]));
        sacc[qh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kf[s], sacc[qh], 0, 0, 0);
        const bf16x8 da = as_bf16x8(*reinterpret_cast<const uint4*>(&sDO[(32 * qh + l32) * RP + 16 * s + 8 * g]));
        pacc[qh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, vf[s], pacc[qh], 0, 0, 0);
      }
    }
    // P and dS for rows q = 32qh + 8(r/4) + 4g + r%4, column = this lane's key
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int q = 32 * qh + 8 * (r >> 2) + 4 * g + (r & 3);
        const float mq = sM[q];
        const float p = (kvalid && mq != NINF) ? exp2f(__builtin_fmaf(sacc[qh][r], a.scale_log2, -mq)) : 0.0f;
        sacc[qh][r] = p;
        pacc[qh][r] = p * (pacc[qh][r] - sDl[q]);
      }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 pb = b_from_acc(sacc, tt);
      const bf16x8 sb = b_from_acc(pacc, tt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_from_t(sDOT, TP, dt, tt, l32, g), pb, dv[dt], 0, 0, 0);
        dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_from_t(sQT, TP, dt, tt, l32, g), sb, dk[dt], 0, 0, 0);
      }
    }
  }
  uint16_t* dkr = a.dk + hoff + key * D;
  uint16_t* dvr = a.dv + hoff + key * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 u;
      u.x = pack_bf16(dk[dt][4 * j + 0] * a.sm_scale, dk[dt][4 * j + 1] * a.sm_scale);
      u.y = pack_bf16(dk[dt][4 * j + 2] * a.sm_scale, dk[dt][4 * j + 3] * a.sm_scale);
      *reinterpret_cast<uint2*>(dkr + 32 * dt + 8 * j + 4 * g) = u;
      u.x = pack_bf16(dv[dt][4 * j + 0], dv[dt][4 * j + 1]);
      u.y = pack_bf16(dv[dt][4 * j + 2], dv[dt][4 * j + 3]);
      *reinterpret_cast<uint2*>(dvr + 32 * dt + 8 * j + 4 * g) = u;
    }
}

template <int D>
__global__ __launch_bounds__(128, 2) void bsa_bwd_dq_kernel(BwdArgs a) {
  constexpr int RP = D + 8, TP = 68, NS = D / 16, NDT = D / 32, KCH = 64 * D / 8 / 128;
  __shared__ __align__(16) uint16_t sK[64 * RP];
  __shared__ __align__(16) uint16_t sV[64 * RP];
  __shared__ __align__(16) uint16_t sKT[D * TP];
  __shared__ __align__(16) uint8_t sValid[64];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int t = blockIdx.x, bh = blockIdx.y;
  const int64_t row = (int64_t)bh * a.Nt + t;
  const int n = a.len[row];
  const int32_t* cols = a.cols + a.start[row];
  const int64_t hoff = (int64_t)bh * a.S * D;
  const int64_t qrow = (int64_t)t * 64 + 32 * w + l32;
  const bool has_mask = a.kv_valid != nullptr;
  const float NINF = -__uint_as_float(0x7f800000u);

  bf16x8 qf[NS], df[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(a.q + hoff + qrow * D + 16 * s + 8 * g));
    df[s] = as_bf16x8(*reinterpret_cast<const uint4*>(a.do_ + hoff + qrow * D + 16 * s + 8 * g));
  }
  const float mq = a.lse[(int64_t)bh * a.S + qrow] * kLog2e;
  const float dlt = a.delta[(int64_t)bh * a.S + qrow];
  f32x16 dq[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[dt][r] = 0.0f;

  for (int it = 0; it < n; ++it) {
    const int64_t kt = cols[it];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * 128;
      const int r = c / (D / 8), c8 = c % (D / 8);
      const int64_t src = hoff + (kt * 64 + r) * D + c8 * 8;
      *reinterpret_cast<uint4*>(&sK[r * RP + c8 * 8]) = *reinterpret_cast<const uint4*>(a.k + src);
      *reinterpret_cast<uint4*>(&sV[r * RP + c8 * 8]) = *reinterpret_cast<const uint4*>(a.v + src);
      const int d = c >> 3, k8 = c & 7;
      *reinterpret_cast<uint4*>(&sKT[d * TP + k8 * 8]) =
          *reinterpret_cast<const uint4*>(a.kt + hoff + (kt * D + d) * 64 + k8 * 8);
    }
    if (has_mask && tid < 16)
      *reinterpret_cast<uint32_t*>(&sValid[tid * 4]) = *reinterpret_cast<const uint32_t*>(a.kv_valid + kt * 64 + tid * 4);
    __syncthreads();

    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
      for (int r = 0; r < 16; ++r) { sacc[kh][r] = 0.0f; pacc[kh][r] = 0.0f; }
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bf16x8 ka = as_bf16x8(*reinterpret_cast<const uint4*>(&sK[(32 * kh + l32) * RP + 16 * s + 8 * g]));
        sacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[s], sacc[kh], 0, 0, 0);
        const bf16x8 va = as_bf16x8(*reinterpret_cast<const uint4*>(&sV[(32 * kh + l32) * RP + 16 * s + 8 * g]));
        pacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, df[s], pacc[kh], 0, 0, 0);
      }
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = 32 * kh + 8 * (r >> 2) + 4 * g + (r & 3);
        const bool ok = (!has_mask || sValid[kk] != 0) && mq != NINF;
        const float p = ok ? exp2f(__builtin_fmaf(sacc[kh][r], a.scale_log2, -mq)) : 0.0f;
        pacc[kh][r] = p * (pacc[kh][r] - dlt);
      }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 sb = b_from_acc(pacc, tt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
        dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_from_t(sKT, TP, dt, tt, l32, g), sb, dq[dt], 0, 0, 0);
    }
  }
  uint16_t* dqr = a.dq + hoff + qrow * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 u;
      u.x = pack_bf16(dq[dt][4 * j + 0] * a.sm_scale, dq[dt][4 * j + 1] * a.sm_scale);
      u.y = pack_bf16(dq[dt][4 * j + 2] * a.sm_scale, dq[dt][4 * j + 3] * a.sm_scale);
      *reinterpret_cast<uint2*>(dqr + 32 * dt + 8 * j + 4 * g) = u;
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
  PRISM_REQUIRE(S > 0 && S % 64 == 0, "%s: S must be a positive multiple of 64", who);
  PRISM_REQUIRE(BH >= 1 && BH <= 65535, "%s: BH out of range", who);
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
  a.start = kstart; a.len = klen; a.cols = kcols; a.S = S; a.Nt = S / 64;
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
  dim3 grid((unsigned)(S / 64), BH);
  if (D == 128) bsa_bwd_dkdv_kernel<128><<<grid, 128, 0, stream>>>(a);
  else bsa_bwd_dkdv_kernel<64><<<grid, 128, 0, stream>>>(a);
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
  a.start = qstart; a.len = qlen; a.cols = qcols; a.S = S; a.Nt = S / 64;
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dq = (uint16_t*)dq;
  dim3 grid((unsigned)(S / 64), BH);
  if (D == 128) bsa_bwd_dq_kernel<128><<<grid, 128, 0, stream>>>(a);
  else bsa_bwd_dq_kernel<64><<<grid, 128, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_bwd_dq");
  return PRISM_OK;
}

}  // extern "C"
