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
// Layouts (per head, tile order): Q, dO row-major [Sq][D], K, V [Sk][D]
// (Sq = Sk for self-attention); m2 = lse * log2(e) with rows that saw no valid
// key at +inf (prism_lse_to_m2).
//
// MI355X design, shared by both kernels:
//  * a PAIR of tiles (2p, 2p+1) is taken by one workgroup, which walks the
//    sorted union of the two tiles' lists (prism_pair_union);
//  * the operand tiles of list entry j + NST - 1 are copied HBM -> LDS by
//    global_load_lds_dwordx4 while entry j is multiplied (NST = 3 stages for
//    dK/dV, 2 for dQ; one barrier per entry, no VGPR staging);
//  * all operands come from row-major tiles: row reads (ds_read_b128) for the
//    S / dP products, transposing reads (ds_read_b64_tr_b16) for the products
//    that contract over the tile's rows (see RowTile), so no transposed
//    copies of Q, K or dO are made;
//  * pairs in the launch order of prism_pair_order; with a work counter,
//    persistent workgroups take them from an atomic work queue (as in the
//    forward kernel), without one a workgroup per pair with its id remapped
//    per XCD (xcd_group_remap).
// dK/dV: one 8-wave workgroup per CU (two waves per SIMD).  The waves split
// each (tile, tile) product in two halves of the query rows, so every wave
// holds half-size partial accumulators; the two partials are added in a
// fixed order through LDS at the end (deterministic).  Wave w owns keys
// [32 kh, 32 kh + 32) of tile 2p + tk and query rows [32 qh, 32 qh + 32) of
// every listed query tile (kh = w & 1, qh = (w >> 1) & 1, tk = w >> 2).
// Waves w and w + 4 share a SIMD (the hardware places wave i of a workgroup
// on SIMD (i + c) mod 4), so each SIMD holds one wave of each key tile and an
// entry listed by one tile only still keeps all four SIMDs busy.
// S = Q K^T and dP = dO V^T keep one key per lane column, so P
// and dS feed the B operand of dV^T = dO^T P and dK^T = Q^T dS straight from
// the accumulators.
// dQ: two 4-wave workgroups per CU (their phases drift apart, so one's
// exponentials overlap the other's MFMA work); wave w owns query rows
// [32 qh, 32 qh + 32) of tile 2p + tq over all 64 keys of every listed key
// tile (qh = w & 1, tq = w >> 1).  S^T = K Q^T and dP^T = V dO^T keep one
// query per lane column; dQ^T = K^T dS^T.
#include <type_traits>

#include "common.h"
#include "mfma.h"
#include "tile_dma.h"
#include "validate.h"

namespace {

struct BwdArgs {
  const uint16_t *q, *k, *v, *do_;
  const float* m2;          // [BH, Sq] base-2 row max (lse * log2 e, +inf for empty rows)
  const float* delta;       // [BH, Sq]
  const uint8_t* kv_valid;  // [Sk] tile order or null (dK/dV)
  const uint64_t* tmask;    // [Sk/64] per-tile key validity or null (dQ)
  const int64_t* ustart;    // pair-union lists
  const int32_t* ulen;
  const int32_t* ucols;
  const int32_t* pairmap;   // tiles of pair p (of the side the grid walks), or null for 2p, 2p + 1
  const int32_t* order;     // pair of each workgroup id (prism_pair_order), or null: xcd_group_remap
  int64_t Sq, Sk;
  int npairs;               // tile pairs per head of the side the grid walks
  float sm_scale, scale_log2;
  uint16_t *dq, *dk, *dv;
  int total;                // pairs of the launch (BH * npairs)
  int* queue;               // work-queue counter (persistent launch), or null: one pair per workgroup
};

constexpr float kLog2e = 1.4426950408889634f;
// dK/dV: four LDS stages, entry j + 2 copied while entry j is multiplied (the
// waves that run behind still read entry j - 1's stage)
constexpr int kStagesDkdv = 4, kAheadDkdv = 2;
constexpr int kStagesDq = 2;    // two 4-wave workgroups per CU, double-buffered each

template <int D>
struct BwdTiles {
  using RT = RowTile<D>;
  // dQ stage: K, V; dK/dV stage: Q, dO, then the m2 and delta rows (256 B each)
  static constexpr int DQ_STAGE = 2 * RT::BYTES;
  static constexpr int DKDV_STAGE = 2 * RT::BYTES + 512;
  static constexpr int SLOTS = 2 * RT::KB / 8;  // KB-instructions per wave and stage
  static_assert(2 * RT::KB % 8 == 0, "stage must split evenly over 8 waves");
  static constexpr int NDT = D / 32;
  static constexpr int DKDV_RED = 4 * 64 * 2 * NDT * 16 * 4;  // qh = 1 partials of dK and dV
  static constexpr int DKDV_LDS = kStagesDkdv * DKDV_STAGE > DKDV_RED ? kStagesDkdv * DKDV_STAGE : DKDV_RED;
  static_assert(kAheadDkdv + 2 <= kStagesDkdv, "stages of entries j - 1 .. j + kAheadDkdv");
  static constexpr int DQ_LDS = kStagesDq * DQ_STAGE;
  static_assert(DKDV_LDS <= 160 * 1024 && DQ_LDS <= 160 * 1024, "LDS budget");
};

// one pair-union work list: the two key tiles of pair `logical`
template <int D>
__device__ __forceinline__ void bsa_bwd_dkdv_pair(const BwdArgs& a, uint8_t* smem, int logical) {
  using T = BwdTiles<D>;
  using RT = typename T::RT;
  constexpr int NS = D / 16, NDT = D / 32;
  constexpr int SB = T::DKDV_STAGE;

  const int tid = opaque_thread_id(), lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const int kh = w & 1, qh = (w >> 1) & 1, tk = w >> 2;
  const int bh = logical / a.npairs, pair = logical - bh * a.npairs;
  const int32_t* U = a.ucols + a.ustart[logical];
  const int n = a.ulen[logical];
  const int mybit = 1 << tk;
  const int64_t qoff = (int64_t)bh * a.Sq * D, koff = (int64_t)bh * a.Sk * D;
  const float* m2h = a.m2 + (int64_t)bh * a.Sq;
  const float* dlh = a.delta + (int64_t)bh * a.Sq;

  // DMA plan: waves 0-3 (one per SIMD) issue KB-instructions w, w + 4, ...
  // (Q then dO), wave 3 also the m2 row and wave 2 the delta row; waves 4-7
  // issue none and start their MFMAs right after the barrier while the
  // others queue their copies (-2.4% against all eight issuing, A/B on one
  // box).  Instruction w + 4s of a tile reads 4096 s bytes past instruction w.
  constexpr int SL4 = 2 * T::SLOTS, NOFF = RT::KB / 4;
  static_assert(RT::KB % 4 == 0, "tile splits over four waves");
  const uint32_t soff = RT::src_offset(w & 3, lane);
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int qtile, int st) {
    if (w >= 4) return;
    const int64_t toff = qoff + (int64_t)qtile * 64 * D;
    const char* qb = (const char*)uniform_ptr(a.q + toff);
    const char* db = (const char*)uniform_ptr(a.do_ + toff);
    const uint32_t base = lds0 + (uint32_t)(st * SB);
#pragma unroll
    for (int s = 0; s < SL4; ++s) {
      const int i = w + 4 * s;
      dma_b128(soff, (i < RT::KB ? qb : db) + 4096 * (s % NOFF), base + (uint32_t)i * 1024u);
    }
    if (w >= 2) {
      const float* rowsrc = (w == 3 ? m2h : dlh) + (int64_t)qtile * 64;
      dma_b32_rows(uniform_ptr(rowsrc), base + 2u * RT::BYTES + (w == 3 ? 0u : 256u));
    }
  };
  RowOperand rop;                // Q / dO rows 32 qh + l32
  rop.init<RT>(32 * qh, l32, g);
  TrOperand top;                 // Q^T / dO^T over query rows 32 qh .. 32 qh + 31
  top.init<RT>(32 * qh, lane);

  EntryRing<kAheadDkdv + 1> ring;
  ring.init(U, n);
#pragma unroll
  for (int k = 0; k < kAheadDkdv; ++k)
    if (k < n) issue(ring.e[k] >> 3, k);

  const int kslot = 2 * pair + tk;
  const int ktile = a.pairmap ? a.pairmap[(int64_t)bh * 2 * a.npairs + kslot] : kslot;
  const int64_t key = (int64_t)ktile * 64 + 32 * kh + l32;
  bf16x8 kf[NS], vf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    kf[s] = ld_bf16x8(a.k + koff + key * D + 16 * s + 8 * g);
    vf[s] = ld_bf16x8(a.v + koff + key * D + 16 * s + 8 * g);
  }
  const bool kvalid = a.kv_valid ? a.kv_valid[key] != 0 : true;
  const float kbias = kvalid ? 0.0f : -__builtin_inff();
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    consume_regs(kf[s]);
    consume_regs(vf[s]);
  }
  consume_regs(kbias);
  const bool all_valid = __builtin_amdgcn_ballot_w64(!kvalid) == 0;
  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) { dk[dt] = f32x16_zero(); dv[dt] = f32x16_zero(); }

  // S = Q K^T and dP = dO V^T of one entry, then P and dS (bf16 B operands of
  // the dV / dK products, query rows 32qh + 8j + 4g + i in register r = 4j + i,
  // column = this lane's key); allv: std::true_type when every key of this
  // wave is valid
  auto sdp = [&](auto allv, const uint8_t* sQ, bf16x8* pb, bf16x8* sb) {
    constexpr bool AV = decltype(allv)::value;
    const uint8_t* sDO = sQ + RT::BYTES;
    const float* sM = reinterpret_cast<const float*>(sQ + 2 * RT::BYTES);
    const float* sDl = sM + 64;
    f32x16 sacc = f32x16_zero(), pacc = f32x16_zero();
    // The 2 NS row operands (Q and dO of k-steps 0, 0, 1, 1, ...) go through
    // a ring of three registers: operand i + 2 is read while MFMA i runs.
    constexpr int NO = 2 * NS;
    bf16x8 op[3];
    auto rd = [&](int i) { return rop.load((i & 1) ? sDO : sQ, i >> 1); };
    op[0] = rd(0);
    op[1] = rd(1);
#pragma unroll
    for (int i = 0; i < NO; ++i) {
      if (i + 2 < NO) op[(i + 2) % 3] = rd(i + 2);
      if (i & 1) pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % 3], vf[i >> 1], pacc, 0, 0, 0);
      else sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % 3], kf[i >> 1], sacc, 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
    for (int i = 0; i + 3 < NO; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
    // P = 2^(S log2e scale - m2 [+ kbias]) and dS = P (dP - delta); kbias
    // is -inf at this lane's key when it is invalid, else 0; waves whose
    // keys are all valid (AV) skip the add
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float4 m4 = *reinterpret_cast<const float4*>(sM + 32 * qh + 8 * jj + 4 * g);
      const float4 d4 = *reinterpret_cast<const float4*>(sDl + 32 * qh + 8 * jj + 4 * g);
      const float mv[4] = {m4.x, m4.y, m4.z, m4.w}, dl4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * jj + i;
        float x = __builtin_fmaf(sacc[r], a.scale_log2, -mv[i]);
        if constexpr (!AV) x += kbias;
        const float p = fast_exp2(x);
        sacc[r] = p;
        pacc[r] = p * (pacc[r] - dl4[i]);
      }
    }
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      pb[t2] = b_from_acc(&sacc, t2);
      sb[t2] = b_from_acc(&pacc, t2);
    }
  };
  // dV^T += dO^T P and dK^T += Q^T dS of one entry
  auto dvdk = [&](const uint8_t* sQ, const bf16x8* pb, const bf16x8* sb) {
    const uint8_t* sDO = sQ + RT::BYTES;
    constexpr int NO = 4 * NDT, RING = 4;
    // The 4 NDT transposed operands (dO^T for even i, Q^T for odd i, of
    // k-step t2 = i / (2 NDT) and head-dim tile dt = (i / 2) % NDT) go
    // through a ring of four registers: the two ds_read_b64_tr_b16 of
    // operand i + 3 are issued after MFMA i. Left to itself the compiler
    // issued eight reads at a time and waited on them (3.5% slower kernel).
    bf16x8 op[RING];
    auto rd = [&](int i) { return top.load<RT>((i & 1) ? sQ : sDO, i / (2 * NDT), (i >> 1) % NDT); };
#pragma unroll
    for (int i = 0; i + 1 < RING; ++i) op[i] = rd(i);
#pragma unroll
    for (int i = 0; i < NO; ++i) {
      if (i + RING - 1 < NO) op[(i + RING - 1) % RING] = rd(i + RING - 1);
      const int t2 = i / (2 * NDT), dt = (i >> 1) % NDT;
      if (i & 1) dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % RING], sb[t2], dk[dt], 0, 0, 0);
      else dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % RING], pb[t2], dv[dt], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * (RING - 1), 0);
#pragma unroll
    for (int i = 0; i + RING - 1 < NO; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, RING - 1, 0);
  };

  // The two waves of a SIMD (tiles tk = 0 and 1) run half an entry apart: a
  // tk = 0 wave takes entry j as S / dP, exponentials, dV / dK; a tk = 1 wave
  // first does dV / dK of its previous entry, then S / dP and exponentials of
  // entry j.  So each wave's exponentials run while the other wave's MFMAs
  // hold the matrix core, instead of both SIMD waves leaving it idle at once.
  // Each group has a loop of its own (the same barriers per entry), so the
  // P / dS operands the tk = 1 waves carry to the next entry are not live in
  // the tk = 0 loop.  Both loops are instantiated for waves with and without
  // invalid keys (a wave-uniform choice made once).
  auto run = [&](auto allv) {
  if (tk == 0) {
    int st = 0;  // stage of entry j
    for (int j = 0; j < n; ++j) {
      const int e = ring.e[0], enext = ring.e[kAheadDkdv];
      ring.advance(U, n, j);
      if (w >= 2) stage_wait<kAheadDkdv + 1, SL4 + 1>(n - 1 - j);
      else stage_wait<kAheadDkdv + 1, SL4>(n - 1 - j);
      __syncthreads();
      if (j + kAheadDkdv < n) issue(enext >> 3, (st + kAheadDkdv) % kStagesDkdv);
      const uint8_t* sQ = smem + st * SB;
      st = st + 1 == kStagesDkdv ? 0 : st + 1;
      if (!(e & mybit)) continue;
      bf16x8 pb[2], sb[2];
      sdp(allv, sQ, pb, sb);
      // dV / dK of a tk = 0 wave at raised priority: its SIMD partner (a
      // tk = 1 wave, half an entry behind) is then in its S / dP phase
      // (-1% against equal priority; raising the tk = 1 waves instead, or
      // also the exponentials, was slower)
      __builtin_amdgcn_s_setprio(1);
      dvdk(sQ, pb, sb);
      __builtin_amdgcn_s_setprio(0);
    }
  } else {
    int st = 0;
    bool pend = false;          // P / dS of the previous entry wait for their dV / dK
    const uint8_t* sPrev = smem;
    bf16x8 pb[2], sb[2];
    for (int j = 0; j < n; ++j) {
      const int e = ring.e[0];
      ring.advance(U, n, j);
      __syncthreads();
      const uint8_t* sQ = smem + st * SB;
      st = st + 1 == kStagesDkdv ? 0 : st + 1;
      if (pend) dvdk(sPrev, pb, sb);
      pend = (e & mybit) != 0;
      if (pend) {
        sdp(allv, sQ, pb, sb);
        sPrev = sQ;
      }
    }
    if (pend) dvdk(sPrev, pb, sb);
  }

  };
  if (all_valid) run(std::true_type{});
  else run(std::false_type{});

  // add the two query-half partials in a fixed order (qh = 0 + qh = 1)
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  const int slot = kh | tk << 1;  // (kh, tk) of the wave pair
  if (qh == 1) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        red[((slot * 2 * NDT + dt) * 16 + r) * 64 + lane] = dk[dt][r];
        red[((slot * 2 * NDT + NDT + dt) * 16 + r) * 64 + lane] = dv[dt][r];
      }
  }
  __syncthreads();
  if (qh == 0) {
    uint16_t* dkr = a.dk + koff + key * D;
    uint16_t* dvr = a.dv + koff + key * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        dk[dt][r] += red[((slot * 2 * NDT + dt) * 16 + r) * 64 + lane];
        dv[dt][r] += red[((slot * 2 * NDT + NDT + dt) * 16 + r) * 64 + lane];
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        uint2 o;
        o.x = pack_bf16(dk[dt][4 * jj + 0] * a.sm_scale, dk[dt][4 * jj + 1] * a.sm_scale);
        o.y = pack_bf16(dk[dt][4 * jj + 2] * a.sm_scale, dk[dt][4 * jj + 3] * a.sm_scale);
        *reinterpret_cast<uint2*>(dkr + 32 * dt + 8 * jj + 4 * g) = o;
        o.x = pack_bf16(dv[dt][4 * jj + 0], dv[dt][4 * jj + 1]);
        o.y = pack_bf16(dv[dt][4 * jj + 2], dv[dt][4 * jj + 3]);
        *reinterpret_cast<uint2*>(dvr + 32 * dt + 8 * jj + 4 * g) = o;
      }
    }
  }
}

// One workgroup per pair (no work counter), or persistent workgroups that
// take pairs from the work queue (work_queue_take).  The pair body re-reads
// the arguments (kernel_args) and recomputes its lane offsets
// (opaque_thread_id), so nothing stays in registers across pairs.
template <int D>
__global__ __launch_bounds__(512, 1) void bsa_bwd_dkdv_kernel(BwdArgs a) {
  __shared__ __align__(16) uint8_t smem[BwdTiles<D>::DKDV_LDS];
  __shared__ WorkQueueState wq;
  work_queue_init(&wq);
  for (int pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : (int)blockIdx.x; pid >= 0;
       pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : -1) {
    const BwdArgs ap = kernel_args<BwdArgs>();
    bsa_bwd_dkdv_pair<D>(ap, smem, a.order ? a.order[pid] : xcd_group_remap<32>(pid, a.total));
  }
}

// one pair-union work list: the two query tiles of pair `logical`
template <int D>
__device__ __forceinline__ void bsa_bwd_dq_pair(const BwdArgs& a, uint8_t* smem, int logical) {
  using T = BwdTiles<D>;
  using RT = typename T::RT;
  constexpr int NS = D / 16, NDT = D / 32;
  constexpr int SB = T::DQ_STAGE;
  constexpr int SLOTS = 2 * RT::KB / 4;  // KB-instructions per wave and stage (4 waves)

  const int tid = opaque_thread_id(), lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const int qh = w & 1, tq = w >> 1;
  const int bh = logical / a.npairs, pair = logical - bh * a.npairs;
  const int32_t* U = a.ucols + a.ustart[logical];
  const int n = a.ulen[logical];
  const int mybit = 1 << tq;
  const int64_t qoff = (int64_t)bh * a.Sq * D, koff = (int64_t)bh * a.Sk * D;
  const float NINF = -__builtin_inff();

  // DMA plan: wave w issues KB-instructions w, w + 4, ... (K then V);
  // instruction w + 4s of a tile reads 4096 s bytes past instruction w
  constexpr int NOFF = RT::KB / 4;
  const uint32_t soff = RT::src_offset(w, lane);
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int ktile, int st) {
    const int64_t toff = koff + (int64_t)ktile * 64 * D;
    const char* kb = (const char*)uniform_ptr(a.k + toff);
    const char* vb = (const char*)uniform_ptr(a.v + toff);
    const uint32_t base = lds0 + (uint32_t)(st * SB);
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
      const int i = w + 4 * s;
      dma_b128(soff, (i < RT::KB ? kb : vb) + 4096 * (s % NOFF), base + (uint32_t)i * 1024u);
    }
  };
  RowOperand rop;  // K / V rows l32 (+ 32 kh as an immediate)
  rop.init<RT>(0, l32, g);
  TrOperand top;   // K^T over key rows 0 .. 63
  top.init<RT>(0, lane);

  EntryRing<kStagesDq> ring;
  ring.init(U, n);
#pragma unroll
  for (int k = 0; k + 1 < kStagesDq; ++k)
    if (k < n) issue(ring.e[k] >> 3, k);

  const int qslot = 2 * pair + tq;
  const int qtile = a.pairmap ? a.pairmap[(int64_t)bh * 2 * a.npairs + qslot] : qslot;
  const int64_t qrow = (int64_t)qtile * 64 + 32 * qh + l32;
  bf16x8 qf[NS], df[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = ld_bf16x8(a.q + qoff + qrow * D + 16 * s + 8 * g);
    df[s] = ld_bf16x8(a.do_ + qoff + qrow * D + 16 * s + 8 * g);
  }
  const float mq = a.m2[(int64_t)bh * a.Sq + qrow];
  const float dlt = a.delta[(int64_t)bh * a.Sq + qrow];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    consume_regs(qf[s]);
    consume_regs(df[s]);
  }
  consume_regs(mq);
  consume_regs(dlt);
  // -delta of this lane's query in every accumulator slot: the dP^T chains
  // start from it, so they produce dP - delta without a per-element subtract
  f32x16 ndl;
#pragma unroll
  for (int r = 0; r < 16; ++r) ndl[r] = -dlt;
  f32x16 dq[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dq[dt] = f32x16_zero();

  int st = 0;  // stage of entry j
  for (int j = 0; j < n; ++j) {
    const int e = ring.e[0], enext = ring.e[kStagesDq - 1];
    ring.advance(U, n, j);
    stage_wait<kStagesDq, SLOTS>(n - 1 - j);
    __syncthreads();
    if (j + kStagesDq - 1 < n) issue(enext >> 3, stage_ahead<kStagesDq>(st));
    const uint8_t* sK = smem + st * SB;
    st = st + 1 == kStagesDq ? 0 : st + 1;
    if (!(e & mybit)) continue;

    const uint8_t* sV = sK + RT::BYTES;
    f32x16 sacc[2] = {f32x16_zero(), f32x16_zero()}, pacc[2] = {ndl, ndl};
    // the 4 NS row operands (K then V of key half 0, then 1, of k-step 0,
    // then of step 1, ...) go through a ring of four registers: operand
    // i + 3 is read while MFMA i runs
    {
      constexpr int NO = 4 * NS, RING = 4;
      bf16x8 op[RING];
      auto rd = [&](int i) { return rop.load(((i & 1) ? sV : sK) + RT::rows(32 * ((i >> 1) & 1)), i >> 2); };
#pragma unroll
      for (int i = 0; i + 1 < RING; ++i) op[i] = rd(i);
#pragma unroll
      for (int i = 0; i < NO; ++i) {
        if (i + RING - 1 < NO) op[(i + RING - 1) % RING] = rd(i + RING - 1);
        const int kh = (i >> 1) & 1;
        if (i & 1) pacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % RING], df[i >> 2], pacc[kh], 0, 0, 0);
        else sacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % RING], qf[i >> 2], sacc[kh], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, RING - 1, 0);
#pragma unroll
      for (int i = 0; i + RING - 1 < NO; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, RING - 1, 0);
    }
    // the first K^T operands of the dQ product are read before the
    // exponentials, so their LDS latency hides behind them; the rest go
    // through a ring of RQ registers, operand i + RQ - 1 read while MFMA i runs
    constexpr int NQ = 4 * NDT, RQ = 4;
    bf16x8 kt[RQ];
    auto rdk = [&](int i) { return top.load<RT>(sK, i / NDT, i % NDT); };
#pragma unroll
    for (int i = 0; i + 1 < RQ; ++i) kt[i] = rdk(i);
    // exponentials, dS and dQ at raised wave priority (as in the forward
    // kernel; measured 1% faster; the same in dK/dV was 4% slower)
    __builtin_amdgcn_s_setprio(1);
    // element (kh, r): key 32kh + 8(r >> 2) + 4g + (r & 3), query = this lane's column
    if (e & 4) {
      const uint64_t mm = sload_u64(a.tmask + (e >> 3)) >> (4 * g);
      const uint32_t lo = (uint32_t)mm, hi = (uint32_t)(mm >> 32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int b = 8 * (r >> 2) + (r & 3);
        sacc[0][r] = keep_or_ninf(sacc[0][r], lo, b);
        sacc[1][r] = keep_or_ninf(sacc[1][r], hi, b);
      }
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(sacc[kh][r], a.scale_log2, -mq));
        pacc[kh][r] = p * pacc[kh][r];
      }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 sb = b_from_acc(pacc, tt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int i = tt * NDT + dt;
        if (i + RQ - 1 < NQ) kt[(i + RQ - 1) % RQ] = rdk(i + RQ - 1);
        dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kt[i % RQ], sb, dq[dt], 0, 0, 0);
      }
    }
    // one MFMA, then the two transposing reads of the ring's next operand;
    // the exponentials are left to the scheduler (pinning them into groups
    // between the MFMAs measured slower)
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + RQ - 1 < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  }

  uint16_t* dqr = a.dq + qoff + qrow * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      uint2 o;
      o.x = pack_bf16(dq[dt][4 * jj + 0] * a.sm_scale, dq[dt][4 * jj + 1] * a.sm_scale);
      o.y = pack_bf16(dq[dt][4 * jj + 2] * a.sm_scale, dq[dt][4 * jj + 3] * a.sm_scale);
      *reinterpret_cast<uint2*>(dqr + 32 * dt + 8 * jj + 4 * g) = o;
    }
}

// One workgroup per pair (no work counter), or persistent workgroups that
// take pairs from the work queue (work_queue_take).  The pair body re-reads
// the arguments (kernel_args) and recomputes its lane offsets
// (opaque_thread_id), so nothing stays in registers across pairs.
template <int D>
__global__ __launch_bounds__(256, 2) void bsa_bwd_dq_kernel(BwdArgs a) {
  __shared__ __align__(16) uint8_t smem[kStagesDq * BwdTiles<D>::DQ_STAGE];
  __shared__ WorkQueueState wq;
  work_queue_init(&wq);
  for (int pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : (int)blockIdx.x; pid >= 0;
       pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : -1) {
    const BwdArgs ap = kernel_args<BwdArgs>();
    bsa_bwd_dq_pair<D>(ap, smem, a.order ? a.order[pid] : xcd_group_remap<64>(pid, a.total));
  }
}

// ------------------------------------------------------------ dQ over quads
// A QUAD of query tiles (two pairs of a zone) per 8-wave workgroup, one
// workgroup per CU, over the quad's union list (prism_quad_union: entries
// tile << 5 | partial << 4 | member bits), so each staged K / V tile serves up
// to 256 query rows.  Wave w owns query rows [32 qh, 32 qh + 32) of quad tile
// tq (qh = w & 1, tq = w >> 1) with the pair kernel's per-entry arithmetic;
// waves w and w + 4 share a SIMD.  Four stages, the copies of entry j + 2
// issued while entry j is multiplied, an eighth by every wave.  Group 0
// (waves 0-3) takes entry j whole after its barrier (S^T and dP^T, then the
// exponentials, dS and dQ).  Group 1 (waves 4-7) runs half an entry behind:
// after the barrier it first finishes entry j - 1 (exponentials, dS and dQ
// from the accumulators it carried across the barrier and the K tile still in
// entry j - 1's stage), then issues its copies, then S^T and dP^T of entry j,
// so on each SIMD one wave's exponentials run beside the other's MFMAs.
// Every wave walks its own tile's entries in ascending order: dQ is
// bit-identical to the pair kernel's.
constexpr int kStagesDqQuad = 4, kAheadDqQuad = 2;

template <int D>
__device__ __forceinline__ void bsa_bwd_dq_quad(const BwdArgs& a, uint8_t* smem, int logical) {
  using T = BwdTiles<D>;
  using RT = typename T::RT;
  constexpr int NS = D / 16, NDT = D / 32;
  constexpr int SB = T::DQ_STAGE;
  constexpr int PERW = T::SLOTS;  // KB-instructions per wave and stage (8 waves)
  constexpr int NOFF = RT::KB / 4;

  const int tid = opaque_thread_id(), lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const int qh = w & 1, tq = w >> 1;
  const int bh = logical / a.npairs, quad = logical - bh * a.npairs;  // npairs: quads per head
  const int32_t* U = a.ucols + a.ustart[logical];
  const int n = a.ulen[logical];
  const int mybit = 1 << tq;
  const int64_t qoff = (int64_t)bh * a.Sq * D, koff = (int64_t)bh * a.Sk * D;

  // DMA plan: wave w issues KB-instructions w, w + 8, ... of each stage (K
  // then V); instruction i + 4m of a tile reads 4096 m bytes past
  // instruction i, so one lane offset serves all
  const uint32_t soff = RT::src_offset(w & 3, lane);
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int ktile, int st) {
    const int64_t toff = koff + (int64_t)ktile * 64 * D;
    const char* kb = (const char*)uniform_ptr(a.k + toff);
    const char* vb = (const char*)uniform_ptr(a.v + toff);
    const uint32_t base = lds0 + (uint32_t)(st * SB);
#pragma unroll
    for (int s = 0; s < PERW; ++s) {
      const int i = w + 8 * s;
      const int t = i < RT::KB ? i : i - RT::KB;
      dma_b128(soff, (i < RT::KB ? kb : vb) + 4096 * ((t >> 2) % NOFF), base + (uint32_t)i * 1024u);
    }
  };
  RowOperand rop;  // K / V rows l32 (+ 32 kh as an immediate)
  rop.init<RT>(0, l32, g);
  TrOperand top;   // K^T over key rows 0 .. 63
  top.init<RT>(0, lane);

  EntryRing<kAheadDqQuad + 1> ring;
  ring.init(U, n);
#pragma unroll
  for (int k = 0; k < kAheadDqQuad; ++k)
    if (k < n) issue(ring.e[k] >> 5, k);

  const int qslot = 4 * quad + tq;
  const int qtile = a.pairmap ? a.pairmap[(int64_t)bh * 4 * a.npairs + qslot] : qslot;
  const int64_t qrow = (int64_t)qtile * 64 + 32 * qh + l32;
  bf16x8 qf[NS], df[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    qf[s] = ld_bf16x8(a.q + qoff + qrow * D + 16 * s + 8 * g);
    df[s] = ld_bf16x8(a.do_ + qoff + qrow * D + 16 * s + 8 * g);
  }
  const float mq = a.m2[(int64_t)bh * a.Sq + qrow];
  const float dlt = a.delta[(int64_t)bh * a.Sq + qrow];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    consume_regs(qf[s]);
    consume_regs(df[s]);
  }
  consume_regs(mq);
  consume_regs(dlt);
  f32x16 ndl;  // -delta: the dP^T chains start from it (dP - delta)
#pragma unroll
  for (int r = 0; r < 16; ++r) ndl[r] = -dlt;
  f32x16 dq[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dq[dt] = f32x16_zero();

  // S^T = K Q^T and dP^T - delta = V dO^T - delta (the pair kernel's ring of
  // four row operands)
  auto sdp_phase = [&](const uint8_t* sK, f32x16 (&sacc)[2], f32x16 (&pacc)[2]) {
    const uint8_t* sV = sK + RT::BYTES;
    sacc[0] = f32x16_zero();
    sacc[1] = f32x16_zero();
    pacc[0] = ndl;
    pacc[1] = ndl;
    constexpr int NO = 4 * NS, RING = 4;
    bf16x8 op[RING];
    auto rd = [&](int i) { return rop.load(((i & 1) ? sV : sK) + RT::rows(32 * ((i >> 1) & 1)), i >> 2); };
#pragma unroll
    for (int i = 0; i + 1 < RING; ++i) op[i] = rd(i);
#pragma unroll
    for (int i = 0; i < NO; ++i) {
      if (i + RING - 1 < NO) op[(i + RING - 1) % RING] = rd(i + RING - 1);
      const int kh = (i >> 1) & 1;
      if (i & 1) pacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % RING], df[i >> 2], pacc[kh], 0, 0, 0);
      else sacc[kh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[i % RING], qf[i >> 2], sacc[kh], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, RING - 1, 0);
#pragma unroll
    for (int i = 0; i + RING - 1 < NO; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, RING - 1, 0);
  };
  // key mask of a partial tile, P, dS = P (dP - delta) and dQ^T += K^T dS^T
  // (the pair kernel's arithmetic and K^T operand ring)
  auto ds_phase = [&](int e, const uint8_t* sK, f32x16 (&sacc)[2], f32x16 (&pacc)[2]) {
    constexpr int NQ = 4 * NDT, RQ = 4;
    bf16x8 kt[RQ];
    auto rdk = [&](int i) { return top.load<RT>(sK, i / NDT, i % NDT); };
#pragma unroll
    for (int i = 0; i + 1 < RQ; ++i) kt[i] = rdk(i);
    __builtin_amdgcn_s_setprio(1);
    if (e & 16) {
      const uint64_t mm = sload_u64(a.tmask + (e >> 5)) >> (4 * g);
      const uint32_t lo = (uint32_t)mm, hi = (uint32_t)(mm >> 32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int b = 8 * (r >> 2) + (r & 3);
        sacc[0][r] = keep_or_ninf(sacc[0][r], lo, b);
        sacc[1][r] = keep_or_ninf(sacc[1][r], hi, b);
      }
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(__builtin_fmaf(sacc[kh][r], a.scale_log2, -mq));
        pacc[kh][r] = p * pacc[kh][r];
      }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const bf16x8 sb = b_from_acc(pacc, tt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int i = tt * NDT + dt;
        if (i + RQ - 1 < NQ) kt[(i + RQ - 1) % RQ] = rdk(i + RQ - 1);
        dq[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kt[i % RQ], sb, dq[dt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + RQ - 1 < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  if (w < 4) {
    int st = 0;  // stage of entry j
    for (int j = 0; j < n; ++j) {
      const int e = ring.e[0], enext = ring.e[kAheadDqQuad];
      ring.advance(U, n, j);
      stage_wait<kAheadDqQuad + 1, PERW>(n - 1 - j);
      __syncthreads();
      if (j + kAheadDqQuad < n) issue(enext >> 5, (st + kAheadDqQuad) % kStagesDqQuad);
      const uint8_t* sK = smem + st * SB;
      st = st + 1 == kStagesDqQuad ? 0 : st + 1;
      if (!(e & mybit)) continue;
      f32x16 sacc[2], pacc[2];
      sdp_phase(sK, sacc, pacc);
      ds_phase(e, sK, sacc, pacc);
    }
  } else {
    int st = 0;
    int epend = 0;  // entry j - 1 if it waits for its dS and dQ, else 0
    const uint8_t* spend = smem;
    f32x16 sacc[2], pacc[2];
    for (int j = 0; j < n; ++j) {
      const int e = ring.e[0], enext = ring.e[kAheadDqQuad];
      ring.advance(U, n, j);
      stage_wait<kAheadDqQuad + 1, PERW>(n - 1 - j);
      __syncthreads();
      const int snext = (st + kAheadDqQuad) % kStagesDqQuad;
      const uint8_t* sK = smem + st * SB;
      st = st + 1 == kStagesDqQuad ? 0 : st + 1;
      if (epend) ds_phase(epend, spend, sacc, pacc);
      if (j + kAheadDqQuad < n) issue(enext >> 5, snext);
      epend = (e & mybit) ? e : 0;
      spend = sK;
      if (epend) sdp_phase(sK, sacc, pacc);
    }
    if (epend) ds_phase(epend, spend, sacc, pacc);
  }

  uint16_t* dqr = a.dq + qoff + qrow * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      uint2 o;
      o.x = pack_bf16(dq[dt][4 * jj + 0] * a.sm_scale, dq[dt][4 * jj + 1] * a.sm_scale);
      o.y = pack_bf16(dq[dt][4 * jj + 2] * a.sm_scale, dq[dt][4 * jj + 3] * a.sm_scale);
      *reinterpret_cast<uint2*>(dqr + 32 * dt + 8 * jj + 4 * g) = o;
    }
}

template <int D>
__global__ __launch_bounds__(512, 1) void bsa_bwd_dq_quad_kernel(BwdArgs a) {
  __shared__ __align__(16) uint8_t smem[kStagesDqQuad * BwdTiles<D>::DQ_STAGE];
  __shared__ WorkQueueState wq;
  work_queue_init(&wq);
  for (int pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : (int)blockIdx.x; pid >= 0;
       pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : -1) {
    const BwdArgs ap = kernel_args<BwdArgs>();
    bsa_bwd_dq_quad<D>(ap, smem, a.order ? a.order[pid] : xcd_group_remap<32>(pid, a.total));
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

int check_common(const void* q, const void* k, int BH, int64_t Sq, int64_t Sk, int D, const char* who) {
  PRISM_REQUIRE(q && k, "%s: null pointer", who);
  PRISM_REQUIRE(D == 64 || D == 128, "%s: head_dim %d unsupported (64, 128)", who, D);
  PRISM_REQUIRE(Sq > 0 && Sq % 128 == 0 && Sk > 0 && Sk % 128 == 0, "%s: Sq and Sk must be positive multiples of 128",
                who);
  PRISM_REQUIRE(BH >= 1 && (int64_t)BH * ((Sq > Sk ? Sq : Sk) / 128) < (1ll << 31), "%s: BH out of range", who);
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

int prism_bsa_bwd_dkdv(const void* q, const void* k, const void* v, const void* do_, const float* m2,
                       const float* delta, int BH, int64_t Sq, int64_t Sk, int D, const uint8_t* kv_valid,
                       const int64_t* ustart, const int32_t* ulen, const int32_t* ucols, const int32_t* pairmap,
                       const int32_t* order, float sm_scale, void* dk, void* dv, int32_t* work_counter,
                       hipStream_t stream) {
  int rc = check_common(q, k, BH, Sq, Sk, D, "prism_bsa_bwd_dkdv");
  if (rc) return rc;
  PRISM_REQUIRE(v && do_ && m2 && delta && ustart && ulen && ucols && dk && dv, "prism_bsa_bwd_dkdv: null pointer");
  if (prism_debug_enabled()) {
    // per-key-tile query lists: entries are query tiles, built without tile masks
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_bsa_bwd_dkdv", ustart, ulen, ucols, (int64_t)BH * (Sk / 128),
                                              Sq / 64, 1, nullptr, stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_bsa_bwd_dkdv", pairmap, BH, Sk / 64, order,
                                             (int64_t)BH * (Sk / 128), stream));
  }
  BwdArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.do_ = (const uint16_t*)do_;
  a.m2 = m2; a.delta = delta; a.kv_valid = kv_valid;
  a.ustart = ustart; a.ulen = ulen; a.ucols = ucols; a.pairmap = pairmap; a.order = order; a.Sq = Sq; a.Sk = Sk;
  a.npairs = (int)(Sk / 128);
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dk = (uint16_t*)dk; a.dv = (uint16_t*)dv;
  a.total = (int)((int64_t)BH * a.npairs);
  a.queue = work_counter;
  if (a.queue) zero_counter_kernel<<<1, kQueueLanes, 0, stream>>>(a.queue);
  const int res = !a.queue ? 0 : D == 128 ? resident_workgroups<bsa_bwd_dkdv_kernel<128>>(512)
                                          : resident_workgroups<bsa_bwd_dkdv_kernel<64>>(512);
  const unsigned blocks = (unsigned)(a.queue && res < a.total ? res : a.total);
  if (D == 128) bsa_bwd_dkdv_kernel<128><<<blocks, 512, 0, stream>>>(a);
  else bsa_bwd_dkdv_kernel<64><<<blocks, 512, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_bwd_dkdv");
  return PRISM_OK;
}

int prism_bsa_bwd_dq(const void* q, const void* k, const void* v, const void* do_, const float* m2, const float* delta,
                     int BH, int64_t Sq, int64_t Sk, int D, const uint64_t* tile_masks, const int64_t* ustart, const int32_t* ulen,
                     const int32_t* ucols, const int32_t* pairmap, const int32_t* order, float sm_scale, void* dq,
                     int32_t* work_counter, hipStream_t stream) {
  int rc = check_common(q, k, BH, Sq, Sk, D, "prism_bsa_bwd_dq");
  if (rc) return rc;
  PRISM_REQUIRE(v && do_ && m2 && delta && ustart && ulen && ucols && dq, "prism_bsa_bwd_dq: null pointer");
  if (prism_debug_enabled()) {
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_bsa_bwd_dq", ustart, ulen, ucols, (int64_t)BH * (Sq / 128),
                                              Sk / 64, 1, tile_masks, stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_bsa_bwd_dq", pairmap, BH, Sq / 64, order,
                                             (int64_t)BH * (Sq / 128), stream));
  }
  BwdArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.do_ = (const uint16_t*)do_;
  a.m2 = m2; a.delta = delta; a.tmask = tile_masks;
  a.ustart = ustart; a.ulen = ulen; a.ucols = ucols; a.pairmap = pairmap; a.order = order; a.Sq = Sq; a.Sk = Sk;
  a.npairs = (int)(Sq / 128);
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dq = (uint16_t*)dq;
  a.total = (int)((int64_t)BH * a.npairs);
  a.queue = work_counter;
  if (a.queue) zero_counter_kernel<<<1, kQueueLanes, 0, stream>>>(a.queue);
  const int res = !a.queue ? 0 : D == 128 ? resident_workgroups<bsa_bwd_dq_kernel<128>>(256)
                                          : resident_workgroups<bsa_bwd_dq_kernel<64>>(256);
  const unsigned blocks = (unsigned)(a.queue && res < a.total ? res : a.total);
  if (D == 128) bsa_bwd_dq_kernel<128><<<blocks, 256, 0, stream>>>(a);
  else bsa_bwd_dq_kernel<64><<<blocks, 256, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_bwd_dq");
  return PRISM_OK;
}

int prism_bsa_bwd_dq_quad(const void* q, const void* k, const void* v, const void* do_, const float* m2,
                          const float* delta, int BH, int64_t Sq, int64_t Sk, int D, const uint64_t* tile_masks,
                          const int64_t* ustart, const int32_t* ulen, const int32_t* ucols, const int32_t* quadmap,
                          const int32_t* order, float sm_scale, void* dq, int32_t* work_counter, hipStream_t stream) {
  int rc = check_common(q, k, BH, Sq, Sk, D, "prism_bsa_bwd_dq_quad");
  if (rc) return rc;
  PRISM_REQUIRE(v && do_ && m2 && delta && ustart && ulen && ucols && dq, "prism_bsa_bwd_dq_quad: null pointer");
  PRISM_REQUIRE(Sq % 256 == 0, "prism_bsa_bwd_dq_quad: Sq must be a multiple of 256");
  if (prism_debug_enabled()) {
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_bsa_bwd_dq_quad", ustart, ulen, ucols, (int64_t)BH * (Sq / 256),
                                              Sk / 64, 2, tile_masks, stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_bsa_bwd_dq_quad", quadmap, BH, Sq / 64, order,
                                             (int64_t)BH * (Sq / 256), stream));
  }
  BwdArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.do_ = (const uint16_t*)do_;
  a.m2 = m2; a.delta = delta; a.tmask = tile_masks;
  a.ustart = ustart; a.ulen = ulen; a.ucols = ucols; a.pairmap = quadmap; a.order = order; a.Sq = Sq; a.Sk = Sk;
  a.npairs = (int)(Sq / 256);  // quads per head
  a.sm_scale = sm_scale; a.scale_log2 = sm_scale * kLog2e; a.dq = (uint16_t*)dq;
  a.total = (int)((int64_t)BH * a.npairs);
  a.queue = work_counter;
  if (a.queue) zero_counter_kernel<<<1, kQueueLanes, 0, stream>>>(a.queue);
  const int res = !a.queue ? 0 : D == 128 ? resident_workgroups<bsa_bwd_dq_quad_kernel<128>>(512)
                                          : resident_workgroups<bsa_bwd_dq_quad_kernel<64>>(512);
  const unsigned blocks = (unsigned)(a.queue && res < a.total ? res : a.total);
  if (D == 128) bsa_bwd_dq_quad_kernel<128><<<blocks, 512, 0, stream>>>(a);
  else bsa_bwd_dq_quad_kernel<64><<<blocks, 512, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_bwd_dq_quad");
  return PRISM_OK;
}

}  // extern "C"
