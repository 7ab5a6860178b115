// Block-sparse flash attention forward, bf16 MFMA (gfx950, v_mfma_f32_32x32x16_bf16).
//
// Reference: _attn_fwd_bsa_varlen_align (flash_attn_bsa_varlen_mask.py:191-319)
// and its host wrapper attn_fwd_bsa_varlen_triton (bsa_interface.py:328-385).
// Semantics kept: per 64-row query tile, online softmax in base 2 over the
// listed 64-key tiles, keys with kv_valid == 0 masked to -inf, l initialised
// to 1 with the all-masked guard alpha = 1 (output 0, lse -inf for rows
// without a valid key), natural-log LSE out.
//
// MI355X design: one workgroup (2 waves) per query tile; wave w owns query rows
// [32w, 32w+32).  Both waves share one K tile [64][D] and one V^T tile [D][64]
// in LDS, refilled from registers prefetched during the previous tile's math.
// S^T = K Q^T puts one query per lane column, so the softmax statistics are
// per lane (one xor-32 shuffle), and the S^T accumulator feeds the B operand
// of O^T = V^T P^T directly (no LDS round trip for P).
#include "common.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct FwdArgs {
  const uint16_t* q;      // [BH, S, D] tile order
  const uint16_t* k;      // [BH, S, D] tile order
  const uint16_t* vt;     // [BH, Nt, D, 64] transposed tiles
  const uint8_t* kv_valid;  // [S] tile order or null
  const int64_t* qstart;  // [BH*Nt]
  const int32_t* qlen;    // [BH*Nt]
  const int32_t* qcols;   // key tile ids
  int64_t S, Nt;
  float scale_log2;       // sm_scale * log2(e)
  uint16_t* o;            // [BH, S, D]
  float* lse;             // [BH, S] natural log
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  const __bf16 x = (__bf16)a, y = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}

template <int D>
__global__ __launch_bounds__(128, 2) void bsa_fwd_kernel(FwdArgs a) {
  constexpr int KP = D + 8;        // K tile pitch (bf16 elements)
  constexpr int VP = 68;           // V^T tile pitch
  constexpr int NS = D / 16;       // MFMA steps over d
  constexpr int NDT = D / 32;      // 32-row d tiles of O^T
  constexpr int KCH = 64 * D / 8 / 128;  // 16-byte chunks per thread per tile
  __shared__ __align__(16) uint16_t sK[64 * KP];
  __shared__ __align__(16) uint16_t sVT[D * VP];
  __shared__ __align__(16) uint8_t sValid[64];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int t = blockIdx.x, bh = blockIdx.y;
  const int64_t row = (int64_t)bh * a.Nt + t;
  const int n = a.qlen[row];
  const int32_t* cols = a.qcols + a.qstart[row];
  const uint16_t* Qh = a.q + (int64_t)bh * a.S * D;
  const uint16_t* Kh = a.k + (int64_t)bh * a.S * D;
  const uint16_t* VTh = a.vt + (int64_t)bh * a.S * D;
  const bool has_mask = a.kv_valid != nullptr;
  const float NINF = -__uint_as_float(0x7f800000u);

  const int64_t qrow = (int64_t)t * 64 + 32 * w + l32;
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(Qh + qrow * D + 16 * s + 8 * g));

  f32x16 acc_o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.0f;
  float m = NINF, l = 1.0f;

  uint4 pk[KCH], pv[KCH];
  uint32_t pvalid = 0xffffffffu;
  auto issue = [&](int kt) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * 128;
      const int r = c / (D / 8), c8 = c % (D / 8);
      pk[i] = *reinterpret_cast<const uint4*>(Kh + ((int64_t)kt * 64 + r) * D + c8 * 8);
      const int d = c >> 3, k8 = c & 7;
      pv[i] = *reinterpret_cast<const uint4*>(VTh + ((int64_t)kt * D + d) * 64 + k8 * 8);
    }
    if (has_mask && tid < 16) pvalid = *reinterpret_cast<const uint32_t*>(a.kv_valid + (int64_t)kt * 64 + tid * 4);
  };
  auto commit = [&]() {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = tid + i * 128;
      const int r = c / (D / 8), c8 = c % (D / 8);
      *reinterpret_cast<uint4*>(&sK[r * KP + c8 * 8]) = pk[i];
      const int d = c >> 3, k8 = c & 7;
      *reinterpret_cast<uint4*>(&sVT[d * VP + k8 * 8]) = pv[i];
    }
    if (has_mask && tid < 16) *reinterpret_cast<uint32_t*>(&sValid[tid * 4]) = pvalid;
  };

  if (n > 0) issue(cols[0]);
  for (int it = 0; it < n; ++it) {
    __syncthreads();
    commit();
    __syncthreads();
    if (it + 1 < n) issue(cols[it + 1]);

    // S^T[key][q] = K Q^T, two 32-key halves
    f32x16 sacc[2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kh][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const bf16x8 ka = as_bf16x8(*reinterpret_cast<const uint4*>(&sK[(32 * kh + l32) * KP + 16 * s + 8 * g]));
        sacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[s], sacc[kh], 0, 0, 0);
      }
    }
    // mask and tile max for this lane's query
    float mx = NINF;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 32 * kh + 8 * (r >> 2) + 4 * g + (r & 3);
        float v = sacc[kh][r];
        if (has_mask && sValid[key] == 0) v = NINF;
        sacc[kh][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx * a.scale_log2);
    const bool dead = m_new == NINF;
    const float alpha = dead ? 1.0f : exp2f(m - m_new);
    float ls = 0.0f;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = dead ? 0.0f : exp2f(__builtin_fmaf(sacc[kh][r], a.scale_log2, -m_new));
        sacc[kh][r] = p;
        ls += p;
      }
    ls += __shfl_xor(ls, 32, 64);
    l = l * alpha + ls;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;

    // O^T[d][q] += V^T P^T over four 16-key steps
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int kh = tt >> 1, j0 = 2 * (tt & 1);
      uint4 pb;
      pb.x = pack_bf16(sacc[kh][4 * j0 + 0], sacc[kh][4 * j0 + 1]);
      pb.y = pack_bf16(sacc[kh][4 * j0 + 2], sacc[kh][4 * j0 + 3]);
      pb.z = pack_bf16(sacc[kh][4 * j0 + 4], sacc[kh][4 * j0 + 5]);
      pb.w = pack_bf16(sacc[kh][4 * j0 + 6], sacc[kh][4 * j0 + 7]);
      const bf16x8 pbv = as_bf16x8(pb);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const uint16_t* vrow = &sVT[(32 * dt + l32) * VP + 16 * tt + 4 * g];
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
        const bf16x8 va = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
        acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pbv, acc_o[dt], 0, 0, 0);
      }
    }
  }

  const float inv = 1.0f / l;
  uint16_t* Oq = a.o + ((int64_t)bh * a.S + qrow) * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 u;
      u.x = pack_bf16(acc_o[dt][4 * j + 0] * inv, acc_o[dt][4 * j + 1] * inv);
      u.y = pack_bf16(acc_o[dt][4 * j + 2] * inv, acc_o[dt][4 * j + 3] * inv);
      *reinterpret_cast<uint2*>(Oq + 32 * dt + 8 * j + 4 * g) = u;
    }
  if (g == 0) a.lse[(int64_t)bh * a.S + qrow] = (m + log2f(l)) * 0.6931471805599453f;
}

}  // namespace

extern "C" {

int prism_bsa_fwd(const void* q, const void* k, const void* vt, int BH, int64_t S, int D, const uint8_t* kv_valid,
                  const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, float sm_scale, void* o, float* lse,
                  hipStream_t stream) {
  PRISM_REQUIRE(q && k && vt && qstart && qlen && qcols && o && lse, "prism_bsa_fwd: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_bsa_fwd: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(S > 0 && S % 64 == 0, "prism_bsa_fwd: S must be a positive multiple of 64");
  PRISM_REQUIRE(BH >= 1 && BH <= 65535, "prism_bsa_fwd: BH out of range");
  FwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.vt = (const uint16_t*)vt; a.kv_valid = kv_valid;
  a.qstart = qstart; a.qlen = qlen; a.qcols = qcols; a.S = S; a.Nt = S / 64;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = (uint16_t*)o; a.lse = lse;
  dim3 grid((unsigned)(S / 64), BH);
  if (D == 128) bsa_fwd_kernel<128><<<grid, 128, 0, stream>>>(a);
  else bsa_fwd_kernel<64><<<grid, 128, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_fwd");
  return PRISM_OK;
}

}  // extern "C"
