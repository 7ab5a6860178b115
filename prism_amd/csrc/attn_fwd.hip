// Block-sparse flash attention forward, bf16 MFMA (gfx950, v_mfma_f32_32x32x16_bf16).
//
// Reference: _attn_fwd_bsa_varlen_align (flash_attn_bsa_varlen_mask.py:191-319)
// and its host wrapper attn_fwd_bsa_varlen_triton (bsa_interface.py:328-385).
// Semantics kept: per 64-row query tile, online softmax in base 2 over the
// listed 64-key tiles, keys with kv_valid == 0 masked to -inf, l initialised
// to 1 with the all-masked guard alpha = 1 (output 0, lse -inf for rows
// without a valid key), natural-log LSE out.
//
// MI355X design:
//  * one workgroup (4 waves) per PAIR of query tiles (2p, 2p+1) of a zone.
//    The two tiles of a 128-token block share one list; neighbouring 64-token
//    blocks share most of theirs.  The workgroup walks the sorted union of the
//    two lists, so each K/V tile it stages in LDS serves up to 128 query rows;
//    waves 0-1 own tile 2p, waves 2-3 tile 2p+1, and a wave whose tile did not
//    list the current key tile skips the math for it.
//  * S^T = K Q^T puts one query per lane column: softmax statistics stay per
//    lane (one xor-32 shuffle), and the S^T accumulator is the B operand of
//    O^T = V^T P^T (no LDS round trip for P).
//  * K [64][D] and V^T [D][64] tiles are double-buffered in LDS (one barrier per
//    key tile); the next tile's global loads are in flight during the math.
//    V^T tiles come from prism_transpose_tiles with the key order inside each
//    16-key group permuted to the MFMA k-slot order, so every operand read is
//    a single 16-byte LDS load.
//  * key validity is a 64-bit ballot per key tile (uniform), applied only to
//    tiles that contain padding.
//  * workgroup ids are remapped so that each XCD (own L2) processes a
//    contiguous range of zones: neighbouring query tiles select overlapping
//    key tiles, which then hit in that XCD's L2.
#include "common.h"
#include "mfma.h"

namespace {

struct FwdArgs {
  const uint16_t* q;        // [BH, S, D] tile order
  const uint16_t* k;        // [BH, S, D] tile order
  const uint16_t* vt;       // [BH, Nt, D, 64] transposed tiles, MFMA key order
  const uint8_t* kv_valid;  // [S] tile order or null
  const int64_t* qstart;    // [BH*Nt]
  const int32_t* qlen;      // [BH*Nt]
  const int32_t* qcols;     // key tile ids, ascending per row
  int64_t S, Nt;
  int npairs, BH;
  float scale_log2;         // sm_scale * log2(e)
  uint16_t* o;              // [BH, S, D]
  float* lse;               // [BH, S] natural log
};

template <int D>
__global__ __launch_bounds__(256, 2) void bsa_fwd_kernel(FwdArgs a) {
  constexpr int KP = D + 8;    // K tile pitch (bf16), 16-byte rows offset by 4 banks
  constexpr int VP = 64 + 8;   // V^T tile pitch
  constexpr int NS = D / 16;   // MFMA k-steps over d
  constexpr int NDT = D / 32;  // 32-row d blocks of O^T
  constexpr int KCH = 64 * D / 8 / 256;  // 16-byte chunks per thread per tile and operand
  __shared__ __align__(16) uint16_t sK[2][64 * KP];
  __shared__ __align__(16) uint16_t sV[2][D * VP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 5, l32 = lane & 31;
  const int logical = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int bh = logical / a.npairs, pair = logical - bh * a.npairs;
  const int64_t rowA = (int64_t)bh * a.Nt + 2 * pair;
  const int32_t* colsA = a.qcols + a.qstart[rowA];
  const int32_t* colsB = a.qcols + a.qstart[rowA + 1];
  const int nA = a.qlen[rowA], nB = a.qlen[rowA + 1];
  const bool mine_is_b = w >= 2;

  const uint16_t* Qh = a.q + (int64_t)bh * a.S * D;
  const uint16_t* Kh = a.k + (int64_t)bh * a.S * D;
  const uint16_t* VTh = a.vt + (int64_t)bh * a.S * D;
  const bool has_mask = a.kv_valid != nullptr;
  const float NINF = -__builtin_inff();

  const int64_t qrow = (int64_t)(2 * pair + (w >> 1)) * 64 + 32 * (w & 1) + l32;
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = ld_bf16x8(Qh + qrow * D + 16 * s + 8 * g);

  f32x16 acc_o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_o[dt] = f32x16_zero();
  float m = NINF, l = 1.0f;

  // merge cursor over the two ascending lists (wave-uniform)
  int ia = 0, ib = 0;
  auto next_union = [&](int& kt, bool& actA, bool& actB) -> bool {
    const int ca = ia < nA ? colsA[ia] : INT32_MAX;
    const int cb = ib < nB ? colsB[ib] : INT32_MAX;
    kt = ca < cb ? ca : cb;
    if (kt == INT32_MAX) return false;
    actA = ca == kt;
    actB = cb == kt;
    ia += actA;
    ib += actB;
    return true;
  };

  // staging registers for the next tile (global -> VGPR -> LDS)
  uint4 pk[KCH], pv[KCH];
  uint8_t pvalid = 1;
#define PRISM_FWD_ISSUE(kt)                                                              \
  do {                                                                                   \
    const uint16_t* ksrc = Kh + (int64_t)(kt) * 64 * D;                                  \
    const uint16_t* vsrc = VTh + (int64_t)(kt) * 64 * D;                                 \
    _Pragma("unroll") for (int i = 0; i < KCH; ++i) {                                    \
      pk[i] = *reinterpret_cast<const uint4*>(ksrc + (tid + i * 256) * 8);               \
      pv[i] = *reinterpret_cast<const uint4*>(vsrc + (tid + i * 256) * 8);               \
    }                                                                                    \
    if (has_mask) pvalid = a.kv_valid[(int64_t)(kt) * 64 + lane];                        \
  } while (0)
#define PRISM_FWD_COMMIT(b)                                                              \
  do {                                                                                   \
    _Pragma("unroll") for (int i = 0; i < KCH; ++i) {                                    \
      const int c = tid + i * 256;                                                       \
      *reinterpret_cast<uint4*>(&sK[b][(c / (D / 8)) * KP + (c % (D / 8)) * 8]) = pk[i]; \
      *reinterpret_cast<uint4*>(&sV[b][(c >> 3) * VP + (c & 7) * 8]) = pv[i];            \
    }                                                                                    \
  } while (0)

  int kt_cur = 0;
  bool actA_cur = false, actB_cur = false;
  bool more = next_union(kt_cur, actA_cur, actB_cur);
  PRISM_FWD_ISSUE(more ? kt_cur : 0);
  uint64_t vmask_next = has_mask ? (uint64_t)__ballot(pvalid != 0) : ~0ull;
  PRISM_FWD_COMMIT(0);
  __syncthreads();
  int buf = 0;
  while (more) {
    const bool act = mine_is_b ? actB_cur : actA_cur;
    const uint64_t vmask = vmask_next;
    int kt_nxt = kt_cur;
    bool actA_nxt = false, actB_nxt = false;
    const bool more_nxt = next_union(kt_nxt, actA_nxt, actB_nxt);
    PRISM_FWD_ISSUE(more_nxt ? kt_nxt : kt_cur);

    if (act) {
      // S^T[key][q] = K Q^T, two 32-key halves as interleaved MFMA chains
      f32x16 sacc[2] = {f32x16_zero(), f32x16_zero()};
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const bf16x8 ka = lds_bf16x8(&sK[buf][(32 * kh + l32) * KP + 16 * s + 8 * g]);
          sacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qf[s], sacc[kh], 0, 0, 0);
        }
      if (vmask != ~0ull) {
        // this lane's keys are 32kh + 8j + 4g + i: bit (32kh + 8j + i) of vmask >> 4g
        const uint64_t mm = vmask >> (4 * g);
        const uint32_t lo = (uint32_t)mm, hi = (uint32_t)(mm >> 32);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int b = 8 * (r >> 2) + (r & 3);
          sacc[0][r] = ((lo >> b) & 1u) ? sacc[0][r] : NINF;
          sacc[1][r] = ((hi >> b) & 1u) ? sacc[1][r] : NINF;
        }
      }
      float mx = fmax_nn(sacc[0][0], sacc[1][0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmax_nn(fmax_nn(mx, sacc[0][r]), sacc[1][r]);
      mx = xor32_max(mx) * a.scale_log2;
      // Lazy rescale: the running reference m only moves when the tile max
      // exceeds it by more than 8 (log2 units), so p <= 2^8 and the O / l
      // rescale is skipped unless some lane of the wave moved.  The final
      // o = acc / l and lse = m + log2 l are unchanged by the choice of m.
      const bool move = mx > m + 8.0f || (m == NINF && mx != NINF);
      const float m_new = move ? mx : m;
      const float alpha = move ? fast_exp2(m - m_new) : 1.0f;
      const float mb = m_new == NINF ? 0.0f : m_new;
      float ls = 0.0f;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = fast_exp2(__builtin_fmaf(sacc[kh][r], a.scale_log2, -mb));
          sacc[kh][r] = p;
          ls += p;
        }
      ls = xor32_add(ls);
      l = __builtin_fmaf(l, alpha, ls);
      m = m_new;
      if (__builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
      }

      // O^T[d][q] += V^T P^T over four 16-key steps
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const bf16x8 pb = b_from_acc(sacc, tt);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const bf16x8 va = lds_bf16x8(&sV[buf][(32 * dt + l32) * VP + 16 * tt + 8 * g]);
          acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, acc_o[dt], 0, 0, 0);
        }
      }
    }
    vmask_next = has_mask ? (uint64_t)__ballot(pvalid != 0) : ~0ull;
    PRISM_FWD_COMMIT(buf ^ 1);
    __syncthreads();
    buf ^= 1;
    more = more_nxt;
    kt_cur = kt_nxt;
    actA_cur = actA_nxt;
    actB_cur = actB_nxt;
  }
#undef PRISM_FWD_ISSUE
#undef PRISM_FWD_COMMIT

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
  if (g == 0) a.lse[(int64_t)bh * a.S + qrow] = (m + __log2f(l)) * 0.6931471805599453f;
}

}  // namespace

extern "C" {

int prism_bsa_fwd(const void* q, const void* k, const void* vt, int BH, int64_t S, int D, const uint8_t* kv_valid,
                  const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, float sm_scale, void* o, float* lse,
                  hipStream_t stream) {
  PRISM_REQUIRE(q && k && vt && qstart && qlen && qcols && o && lse, "prism_bsa_fwd: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_bsa_fwd: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(S > 0 && S % 128 == 0, "prism_bsa_fwd: S must be a positive multiple of 128");
  PRISM_REQUIRE(BH >= 1, "prism_bsa_fwd: BH must be >= 1");
  PRISM_REQUIRE((int64_t)BH * (S / 128) < (1ll << 31), "prism_bsa_fwd: grid too large");
  FwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.vt = (const uint16_t*)vt; a.kv_valid = kv_valid;
  a.qstart = qstart; a.qlen = qlen; a.qcols = qcols; a.S = S; a.Nt = S / 64;
  a.npairs = (int)(S / 128); a.BH = BH;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = (uint16_t*)o; a.lse = lse;
  const unsigned blocks = (unsigned)((int64_t)BH * a.npairs);
  if (D == 128) bsa_fwd_kernel<128><<<blocks, 256, 0, stream>>>(a);
  else bsa_fwd_kernel<64><<<blocks, 256, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_fwd");
  return PRISM_OK;
}

}  // extern "C"
