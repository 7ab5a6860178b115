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
//  * a PAIR of query tiles (2p, 2p+1) of a zone is taken by one workgroup
//    (4 waves), two workgroups per CU (two waves per SIMD).  The two tiles of a
//    128-token block share one list and neighbouring 64-token blocks share
//    most of theirs; the workgroup walks the sorted union of the two lists
//    (prism_pair_union), so each K/V tile it stages in LDS serves up to 128
//    query rows.  Waves 0-1 own tile 2p, waves 2-3 tile 2p+1; a wave whose
//    tile did not list the current key tile skips the math for it.
//  * K and V tiles [64][D] are copied HBM -> LDS by global_load_lds_dwordx4
//    (no VGPR staging), double-buffered: the copy of key tile j+1 is in
//    flight while tile j is multiplied; one barrier per key tile publishes
//    the next stage.  (Two independent workgroups per CU drift out of phase,
//    so one's softmax overlaps the other's MFMA work; a single 8-wave
//    workgroup with a deeper pipeline runs its waves in lock-step and was
//    slower.)
//  * S^T = K Q^T puts one query per lane column: softmax statistics stay per
//    lane (one xor-32 lane swap), and the S^T accumulator is the B operand
//    of O^T = V^T P^T (no LDS round trip for P).  K is read as row operands
//    (ds_read_b128), V^T straight from the row-major V tile by transposing
//    reads (ds_read_b64_tr_b16, see RowTile), so V needs no transposed copy.
//  * key validity: union entries flag tiles that contain padding; only those
//    load their 64-bit validity word and mask.
//  * pairs are taken in the launch order of prism_pair_order (one head region
//    at a time GPU-wide, so K/V stay in the Infinity Cache; the longest lists
//    of the last quarter first).  With a work counter the launch is
//    persistent: as many workgroups as the GPU holds, each taking the next
//    pair from an atomic work queue, so the work spreads over the XCDs as
//    they free up (without one, the hardware hands workgroup ids to the XCDs
//    round-robin whatever their load, and xcd_group_remap gives each XCD runs
//    of neighbouring pairs).
#include "common.h"
#include "mfma.h"
#include "tile_dma.h"
#include "validate.h"

namespace {

struct FwdArgs {
  const uint16_t* q;       // [BH, Sq, D] tile order
  const uint16_t* k;       // [BH, Sk, D] tile order
  const uint16_t* v;       // [BH, Sk, D] tile order
  const uint64_t* tmask;   // [Sk/64] key validity per tile, or null
  const int64_t* ustart;   // [BH * Sq/128] pair-union list starts
  const int32_t* ulen;     // [BH * Sq/128]
  const int32_t* ucols;    // entries tile << 3 | partial << 2 | in_b << 1 | in_a
  const int32_t* pairmap;  // [BH * Sq/64]: tiles of pair p are pairmap[2p], pairmap[2p + 1] (or 2p, 2p + 1)
  const int32_t* order;    // [BH * Sq/128] pair of each workgroup id (prism_pair_order), or null: xcd_group_remap
  int64_t Sq, Sk;
  int npairs;              // query-tile pairs per head
  float scale_log2;        // sm_scale * log2(e)
  uint16_t* o;             // [BH, Sq, D]
  float* lse;              // [BH, Sq] natural log
  int total;               // pairs of the launch (BH * npairs)
  int* queue;              // work-queue counter (persistent launch), or null: one pair per workgroup
};

constexpr int kStages = 2;  // two workgroups per CU: 2 x 2 stages of K and V fill the LDS

template <int D>
struct FwdTiles {
  using RT = RowTile<D>;
  static constexpr int STAGE = 2 * RT::BYTES;  // K, V
  static constexpr int STAGE_KB = 2 * RT::KB;
  static_assert(STAGE_KB % 2 == 0, "stage must split evenly over 2 waves");
};

// one pair-union work list: the two query tiles of pair `logical`
template <int D>
__device__ __forceinline__ void bsa_fwd_pair(const FwdArgs& a, uint8_t* smem, int logical) {
  using T = FwdTiles<D>;
  using RT = typename T::RT;
  constexpr int NS = D / 16;   // MFMA k-steps over d
  constexpr int NDT = D / 32;  // 32-row d blocks of O^T

  const int tid = opaque_thread_id(), lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const int bh = logical / a.npairs, pair = logical - bh * a.npairs;
  const int32_t* U = a.ucols + a.ustart[logical];
  const int n = a.ulen[logical];
  const int mybit = 1 << (w >> 1);

  const uint16_t* Qh = a.q + (int64_t)bh * a.Sq * D;
  const uint16_t* Kh = a.k + (int64_t)bh * a.Sk * D;
  const uint16_t* Vh = a.v + (int64_t)bh * a.Sk * D;
  const float NINF = -__builtin_inff();

  // DMA plan: waves 0 and 1 issue KB-instructions w, w + 2, ... of each
  // stage (K then V); waves 2 and 3 issue none.  A wave stalls while the
  // CU's address path takes its copy instructions, so the two waves that
  // issue none start their MFMAs right after the barrier (-1% against four
  // waves issuing ten each, A/B on one box).  Instruction i + 4m of a tile
  // reads 4096 m bytes past instruction i, so two lane offsets serve all.
  constexpr int SL2 = T::STAGE_KB / 2, NOFF = RT::KB / 4;
  static_assert(RT::KB % 4 == 0, "tile splits into fours");
  const uint32_t soff0 = RT::src_offset(w & 1, lane), soff1 = RT::src_offset((w & 1) + 2, lane);
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int kt, int st) {
    if (w >= 2) return;
    const char* kb = (const char*)uniform_ptr(Kh + (int64_t)kt * 64 * D);
    const char* vb = (const char*)uniform_ptr(Vh + (int64_t)kt * 64 * D);
    const uint32_t base = lds0 + (uint32_t)(st * T::STAGE);
#pragma unroll
    for (int s = 0; s < SL2; ++s) {
      const int i = w + 2 * s;                  // instruction of the stage
      const int t = i < RT::KB ? i : i - RT::KB;  // instruction of its tile
      dma_b128((s & 1) ? soff1 : soff0, (i < RT::KB ? kb : vb) + 4096 * ((t >> 2) % NOFF), base + (uint32_t)i * 1024u);
    }
  };
  RowOperand kop;
  kop.init<RT>(0, l32, g);
  TrOperand vop;
  vop.init<RT>(0, lane);

  EntryRing<kStages> ring;
  ring.init(U, n);
#pragma unroll
  for (int k = 0; k + 1 < kStages; ++k)
    if (k < n) issue(ring.e[k] >> 3, k);

  const int slot2 = 2 * pair + (w >> 1);
  const int qtile = a.pairmap ? a.pairmap[(int64_t)bh * 2 * a.npairs + slot2] : slot2;
  const int64_t qrow = (int64_t)qtile * 64 + 32 * (w & 1) + l32;
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = ld_bf16x8(Qh + qrow * D + 16 * s + 8 * g);
#pragma unroll
  for (int s = 0; s < NS; ++s) consume_regs(qf[s]);

  f32x16 acc_o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_o[dt] = f32x16_zero();
  float m = NINF, l = 1.0f;

  int st = 0;  // stage of entry j
  for (int j = 0; j < n; ++j) {
    const int e = ring.e[0], enext = ring.e[kStages - 1];
    ring.advance(U, n, j);
    stage_wait<kStages, SL2>(n - 1 - j);
    __syncthreads();
    if (j + kStages - 1 < n) issue(enext >> 3, stage_ahead<kStages>(st));
    const uint8_t* sK = smem + st * T::STAGE;
    st = st + 1 == kStages ? 0 : st + 1;
    if (!(e & mybit)) continue;

    const uint8_t* sV = sK + RT::BYTES;
    // S^T[key][q] = K Q^T, two 32-key halves as interleaved MFMA chains; the
    // 2 NS K operands (half 0, 1 of k-step 0, then of step 1, ...) go through
    // a ring of four registers: operand i + 3 is read while MFMA i runs
    f32x16 sacc[2] = {f32x16_zero(), f32x16_zero()};
    {
      constexpr int NO = 2 * NS, RING = 4;
      bf16x8 kfr[RING];
      auto rd = [&](int i) { return kop.load(sK + RT::rows(32 * (i & 1)), i >> 1); };
#pragma unroll
      for (int i = 0; i + 1 < RING; ++i) kfr[i] = rd(i);
#pragma unroll
      for (int i = 0; i < NO; ++i) {
        if (i + RING - 1 < NO) kfr[(i + RING - 1) % RING] = rd(i + RING - 1);
        sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[i % RING], qf[i >> 1], sacc[i & 1], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, RING - 1, 0);
#pragma unroll
      for (int i = 0; i + RING - 1 < NO; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, RING - 1, 0);
    }
    // V^T operands of the P V product, in flight while the softmax runs
    bf16x8 vfr[4][NDT];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) vfr[tt][dt] = vop.load<RT>(sV, tt, dt);
    if (e & 4) {
      // this lane's keys are 32kh + 8j + 4g + i: bit (32kh + 8j + i) of vmask >> 4g
      const uint64_t mm = sload_u64(a.tmask + (e >> 3)) >> (4 * g);
      const uint32_t lo = (uint32_t)mm, hi = (uint32_t)(mm >> 32);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int b = 8 * (r >> 2) + (r & 3);
        sacc[0][r] = keep_or_ninf(sacc[0][r], lo, b);
        sacc[1][r] = keep_or_ninf(sacc[1][r], hi, b);
      }
    }
    // softmax and P V at raised wave priority: when both waves of a SIMD are
    // ready, this phase's VALU work issues first and the other wave's S
    // MFMAs fill the matrix core behind it (measured 1% faster than equal
    // priority; raising it for the S MFMAs instead was slower).  The row max
    // and rescale, which no MFMA of this wave can overlap, run one level
    // higher still (-0.8% against one level for the whole phase)
    __builtin_amdgcn_s_setprio(2);
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
    if (__builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
    }
    // P and O^T[d][q] += V^T P^T one 16-key step at a time: the exponentials
    // of step tt + 1 run on the VALU while the MFMAs of step tt execute
    __builtin_amdgcn_s_setprio(1);  // exponentials interleaved with the P V MFMAs
    float ls = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int h = tt >> 1, r0 = 8 * (tt & 1);
#pragma unroll
      for (int r = r0; r < r0 + 8; ++r) {
        const float p = fast_exp2(__builtin_fmaf(sacc[h][r], a.scale_log2, -mb));
        sacc[h][r] = p;
        ls += p;
      }
      const bf16x8 pb = b_from_acc(sacc, tt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[tt][dt], pb, acc_o[dt], 0, 0, 0);
    }
    // scheduling: first step's VALU, then alternate one MFMA with the next
    // step's VALU work
    __builtin_amdgcn_sched_group_barrier(0x002, 28, 0);
#pragma unroll
    for (int i = 0; i < 3 * NDT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 28 / NDT, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NDT, 0);
    ls = xor32_add(ls);
    l = __builtin_fmaf(l, alpha, ls);
    m = m_new;
    __builtin_amdgcn_s_setprio(0);
  }

  const float inv = 1.0f / l;
  uint16_t* Oq = a.o + ((int64_t)bh * a.Sq + qrow) * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 u;
      u.x = pack_bf16(acc_o[dt][4 * j + 0] * inv, acc_o[dt][4 * j + 1] * inv);
      u.y = pack_bf16(acc_o[dt][4 * j + 2] * inv, acc_o[dt][4 * j + 3] * inv);
      *reinterpret_cast<uint2*>(Oq + 32 * dt + 8 * j + 4 * g) = u;
    }
  if (g == 0) a.lse[(int64_t)bh * a.Sq + qrow] = (m + __log2f(l)) * 0.6931471805599453f;
}

// ------------------------------------------------------------ quads
// A QUAD of query tiles (two pairs of a zone) per 8-wave workgroup, one
// workgroup per CU, over the quad's union list (prism_quad_union: entries
// tile << 5 | partial << 4 | member bits), so each staged K / V tile serves up
// to 256 query rows.  Wave w owns 32 queries of quad tile w >> 1; waves w and
// w + 4 share a SIMD.  Every wave issues an eighth of the copies of entry
// j + 2 (four stages).  Group 0 (waves 0-3) issues them right after the
// barrier of entry j and takes entry j as the pair kernel does (S, row max,
// exponentials with P V).  Group 1 (waves 4-7) runs half an entry behind:
// after the barrier it first finishes entry j - 1 (rescale, exponentials with
// P V, from the S accumulators and V operands it carried across the barrier),
// then issues its copies, then S and the row max of entry j, so on each SIMD
// one wave's exponentials run beside the other's MFMAs (group 1 issuing
// right after the barrier too measured 4% slower, group 0 issuing all
// copies 1% slower).  Every wave walks its own tile's entries in
// ascending order with the pair kernel's arithmetic: results are bit-identical.
constexpr int kStagesQuad = 4, kAheadQuad = 2;

template <int D>
__device__ __forceinline__ void bsa_fwd_quad(const FwdArgs& a, uint8_t* smem, int logical) {
  using T = FwdTiles<D>;
  using RT = typename T::RT;
  constexpr int NS = D / 16;   // MFMA k-steps over d
  constexpr int NDT = D / 32;  // 32-row d blocks of O^T
  constexpr int NOFF = RT::KB / 4, PERW = T::STAGE_KB / 8;

  const int tid = opaque_thread_id(), lane = tid & 63, g = lane >> 5, l32 = lane & 31;
  const int w = (int)uniform_u32((uint32_t)tid >> 6);
  const int slot = w >> 1;  // quad tile of this wave
  const int bh = logical / a.npairs, quad = logical - bh * a.npairs;  // npairs: quads per head
  const int32_t* U = a.ucols + a.ustart[logical];
  const int n = a.ulen[logical];
  const int mybit = 1 << slot;

  const uint16_t* Qh = a.q + (int64_t)bh * a.Sq * D;
  const uint16_t* Kh = a.k + (int64_t)bh * a.Sk * D;
  const uint16_t* Vh = a.v + (int64_t)bh * a.Sk * D;
  const float NINF = -__builtin_inff();

  // DMA plan: every wave issues KB-instructions w, w + 8, ... of each stage
  // (K then V); instruction i + 4m of a tile reads 4096 m bytes past
  // instruction i, so one lane offset serves all
  static_assert(RT::KB % 4 == 0 && T::STAGE_KB % 8 == 0, "tile splits into fours");
  const uint32_t soff = RT::src_offset(w & 3, lane);
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int kt, int st) {
    const char* kb = (const char*)uniform_ptr(Kh + (int64_t)kt * 64 * D);
    const char* vb = (const char*)uniform_ptr(Vh + (int64_t)kt * 64 * D);
    const uint32_t base = lds0 + (uint32_t)(st * T::STAGE);
#pragma unroll
    for (int s = 0; s < PERW; ++s) {
      const int i = w + 8 * s;
      const int t = i < RT::KB ? i : i - RT::KB;
      dma_b128(soff, (i < RT::KB ? kb : vb) + 4096 * ((t >> 2) % NOFF), base + (uint32_t)i * 1024u);
    }
  };
  RowOperand kop;
  kop.init<RT>(0, l32, g);
  TrOperand vop;
  vop.init<RT>(0, lane);

  EntryRing<kAheadQuad + 1> ring;
  ring.init(U, n);
#pragma unroll
  for (int k = 0; k < kAheadQuad; ++k)
    if (k < n) issue(ring.e[k] >> 5, k);

  const int qtile = a.pairmap ? a.pairmap[(int64_t)bh * 4 * a.npairs + 4 * quad + slot] : 4 * quad + slot;
  const int64_t qrow = (int64_t)qtile * 64 + 32 * (w & 1) + l32;
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = ld_bf16x8(Qh + qrow * D + 16 * s + 8 * g);
#pragma unroll
  for (int s = 0; s < NS; ++s) consume_regs(qf[s]);

  f32x16 acc_o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc_o[dt] = f32x16_zero();
  float m = NINF, l = 1.0f;

  // S^T[key][q] = K Q^T (the pair kernel's S phase: operand ring of four)
  auto s_phase = [&](const uint8_t* sK, f32x16 (&sacc)[2]) {
    sacc[0] = f32x16_zero();
    sacc[1] = f32x16_zero();
    constexpr int NO = 2 * NS, RING = 4;
    bf16x8 kfr[RING];
    auto rd = [&](int i) { return kop.load(sK + RT::rows(32 * (i & 1)), i >> 1); };
#pragma unroll
    for (int i = 0; i + 1 < RING; ++i) kfr[i] = rd(i);
#pragma unroll
    for (int i = 0; i < NO; ++i) {
      if (i + RING - 1 < NO) kfr[(i + RING - 1) % RING] = rd(i + RING - 1);
      sacc[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[i % RING], qf[i >> 1], sacc[i & 1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, RING - 1, 0);
#pragma unroll
    for (int i = 0; i + RING - 1 < NO; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, RING - 1, 0);
  };
  // key mask of a partial tile, then the tile's row max and the lazy
  // reference move (the pair kernel's arithmetic)
  auto mask_max = [&](int e, f32x16 (&sacc)[2], float& m_new, float& alpha, float& mb, bool& move) {
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
    float mx = fmax_nn(sacc[0][0], sacc[1][0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmax_nn(fmax_nn(mx, sacc[0][r]), sacc[1][r]);
    mx = xor32_max(mx) * a.scale_log2;
    move = mx > m + 8.0f || (m == NINF && mx != NINF);
    m_new = move ? mx : m;
    alpha = move ? fast_exp2(m - m_new) : 1.0f;
    mb = m_new == NINF ? 0.0f : m_new;
  };
  // rescale, then P and O^T += V^T P^T one 16-key step at a time, the
  // exponentials of step tt + 1 beside the MFMAs of step tt
  auto pv_phase = [&](f32x16 (&sacc)[2], bf16x8 (&vfr)[4][NDT], float m_new, float alpha, float mb, bool move) {
    if (__builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
    }
    float ls = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int h = tt >> 1, r0 = 8 * (tt & 1);
#pragma unroll
      for (int r = r0; r < r0 + 8; ++r) {
        const float p = fast_exp2(__builtin_fmaf(sacc[h][r], a.scale_log2, -mb));
        sacc[h][r] = p;
        ls += p;
      }
      const bf16x8 pb = b_from_acc(sacc, tt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[tt][dt], pb, acc_o[dt], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x002, 28, 0);
#pragma unroll
    for (int i = 0; i < 3 * NDT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 28 / NDT, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NDT, 0);
    ls = xor32_add(ls);
    l = __builtin_fmaf(l, alpha, ls);
    m = m_new;
  };
  auto v_reads = [&](const uint8_t* sV, bf16x8 (&vfr)[4][NDT]) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) vfr[tt][dt] = vop.load<RT>(sV, tt, dt);
  };

  if (w < 4) {
    int st = 0;  // stage of entry j
    for (int j = 0; j < n; ++j) {
      const int e = ring.e[0], enext = ring.e[kAheadQuad];
      ring.advance(U, n, j);
      stage_wait<kAheadQuad + 1, PERW>(n - 1 - j);
      __syncthreads();
      if (j + kAheadQuad < n) issue(enext >> 5, (st + kAheadQuad) % kStagesQuad);
      const uint8_t* sK = smem + st * T::STAGE;
      st = st + 1 == kStagesQuad ? 0 : st + 1;
      if (!(e & mybit)) continue;
      f32x16 sacc[2];
      s_phase(sK, sacc);
      bf16x8 vfr[4][NDT];
      v_reads(sK + RT::BYTES, vfr);
      float m_new, alpha, mb;
      bool move;
      __builtin_amdgcn_s_setprio(2);
      mask_max(e, sacc, m_new, alpha, mb, move);
      __builtin_amdgcn_s_setprio(1);
      pv_phase(sacc, vfr, m_new, alpha, mb, move);
      __builtin_amdgcn_s_setprio(0);
    }
  } else {
    int st = 0;
    bool pend = false;  // entry j - 1 waits for its exponentials and P V
    f32x16 sacc[2];
    bf16x8 vfr[4][NDT];
    float m_new = NINF, alpha = 1.0f, mb = 0.0f;
    bool move = false;
    for (int j = 0; j < n; ++j) {
      const int e = ring.e[0], enext = ring.e[kAheadQuad];
      ring.advance(U, n, j);
      stage_wait<kAheadQuad + 1, PERW>(n - 1 - j);
      __syncthreads();
      const int snext = (st + kAheadQuad) % kStagesQuad;
      const uint8_t* sK = smem + st * T::STAGE;
      st = st + 1 == kStagesQuad ? 0 : st + 1;
      if (pend) {
        __builtin_amdgcn_s_setprio(1);
        pv_phase(sacc, vfr, m_new, alpha, mb, move);
        __builtin_amdgcn_s_setprio(0);
      }
      if (j + kAheadQuad < n) issue(enext >> 5, snext);
      pend = (e & mybit) != 0;
      if (pend) {
        s_phase(sK, sacc);
        __builtin_amdgcn_s_setprio(2);  // the row max as in group 0 (-0.3%; no priorities at all: +5%)
        mask_max(e, sacc, m_new, alpha, mb, move);
        __builtin_amdgcn_s_setprio(0);
        v_reads(sK + RT::BYTES, vfr);
      }
    }
    if (pend) pv_phase(sacc, vfr, m_new, alpha, mb, move);
  }

  const float inv = 1.0f / l;
  uint16_t* Oq = a.o + ((int64_t)bh * a.Sq + qrow) * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 u;
      u.x = pack_bf16(acc_o[dt][4 * j + 0] * inv, acc_o[dt][4 * j + 1] * inv);
      u.y = pack_bf16(acc_o[dt][4 * j + 2] * inv, acc_o[dt][4 * j + 3] * inv);
      *reinterpret_cast<uint2*>(Oq + 32 * dt + 8 * j + 4 * g) = u;
    }
  if (g == 0) a.lse[(int64_t)bh * a.Sq + qrow] = (m + __log2f(l)) * 0.6931471805599453f;
}

template <int D>
__global__ __launch_bounds__(512, 1) void bsa_fwd_quad_kernel(FwdArgs a) {
  __shared__ __align__(16) uint8_t smem[kStagesQuad * FwdTiles<D>::STAGE];
  __shared__ WorkQueueState wq;
  work_queue_init(&wq);
  for (int pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : (int)blockIdx.x; pid >= 0;
       pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : -1) {
    const FwdArgs ap = kernel_args<FwdArgs>();
    bsa_fwd_quad<D>(ap, smem, a.order ? a.order[pid] : xcd_group_remap<32>(pid, a.total));
  }
}

// One workgroup per pair (no work counter), or persistent workgroups that
// take pairs from the work queue (work_queue_take).  The pair body re-reads
// the arguments (kernel_args) and recomputes its lane offsets
// (opaque_thread_id), so nothing stays in registers across pairs.
template <int D>
__global__ __launch_bounds__(256, 2) void bsa_fwd_kernel(FwdArgs a) {
  __shared__ __align__(16) uint8_t smem[kStages * FwdTiles<D>::STAGE];
  __shared__ WorkQueueState wq;
  work_queue_init(&wq);
  for (int pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : (int)blockIdx.x; pid >= 0;
       pid = a.queue ? work_queue_take(a.queue, a.total, &wq) : -1) {
    const FwdArgs ap = kernel_args<FwdArgs>();
    bsa_fwd_pair<D>(ap, smem, a.order ? a.order[pid] : xcd_group_remap<64>(pid, a.total));
  }
}

}  // namespace

extern "C" {

int prism_bsa_fwd(const void* q, const void* k, const void* v, int BH, int64_t Sq, int64_t Sk, int D,
                  const uint64_t* tile_masks,
                  const int64_t* ustart, const int32_t* ulen, const int32_t* ucols, const int32_t* pairmap,
                  const int32_t* order, float sm_scale, void* o, float* lse, int32_t* work_counter,
                  hipStream_t stream) {
  PRISM_REQUIRE(q && k && v && ustart && ulen && ucols && o && lse, "prism_bsa_fwd: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_bsa_fwd: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(Sq > 0 && Sq % 128 == 0 && Sk > 0 && Sk % 128 == 0,
                "prism_bsa_fwd: Sq and Sk must be positive multiples of 128");
  PRISM_REQUIRE(BH >= 1, "prism_bsa_fwd: BH must be >= 1");
  PRISM_REQUIRE((int64_t)BH * (Sq / 128) < (1ll << 31), "prism_bsa_fwd: grid too large");
  if (prism_debug_enabled()) {
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_bsa_fwd", ustart, ulen, ucols, (int64_t)BH * (Sq / 128), Sk / 64,
                                              1, tile_masks, stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_bsa_fwd", pairmap, BH, Sq / 64, order, (int64_t)BH * (Sq / 128),
                                             stream));
  }
  FwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.tmask = tile_masks;
  a.ustart = ustart; a.ulen = ulen; a.ucols = ucols; a.pairmap = pairmap; a.order = order; a.Sq = Sq; a.Sk = Sk;
  a.npairs = (int)(Sq / 128);
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = (uint16_t*)o; a.lse = lse;
  a.total = (int)((int64_t)BH * a.npairs);
  a.queue = work_counter;
  if (a.queue) zero_counter_kernel<<<1, kQueueLanes, 0, stream>>>(a.queue);
  const int res = !a.queue ? 0 : D == 128 ? resident_workgroups<bsa_fwd_kernel<128>>(256)
                                          : resident_workgroups<bsa_fwd_kernel<64>>(256);
  const unsigned blocks = (unsigned)(a.queue && res < a.total ? res : a.total);
  if (D == 128) bsa_fwd_kernel<128><<<blocks, 256, 0, stream>>>(a);
  else bsa_fwd_kernel<64><<<blocks, 256, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_fwd");
  return PRISM_OK;
}

int prism_bsa_fwd_quad(const void* q, const void* k, const void* v, int BH, int64_t Sq, int64_t Sk, int D,
                       const uint64_t* tile_masks, const int64_t* ustart, const int32_t* ulen, const int32_t* ucols,
                       const int32_t* quadmap, const int32_t* order, float sm_scale, void* o, float* lse,
                       int32_t* work_counter, hipStream_t stream) {
  PRISM_REQUIRE(q && k && v && ustart && ulen && ucols && o && lse, "prism_bsa_fwd_quad: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_bsa_fwd_quad: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(Sq > 0 && Sq % 256 == 0 && Sk > 0 && Sk % 128 == 0,
                "prism_bsa_fwd_quad: Sq must be a positive multiple of 256, Sk of 128");
  PRISM_REQUIRE(BH >= 1, "prism_bsa_fwd_quad: BH must be >= 1");
  PRISM_REQUIRE((int64_t)BH * (Sq / 256) < (1ll << 31), "prism_bsa_fwd_quad: grid too large");
  if (prism_debug_enabled()) {
    PRISM_DEBUG_CHECK(prism_debug_check_lists("prism_bsa_fwd_quad", ustart, ulen, ucols, (int64_t)BH * (Sq / 256),
                                              Sk / 64, 2, tile_masks, stream));
    PRISM_DEBUG_CHECK(prism_debug_check_maps("prism_bsa_fwd_quad", quadmap, BH, Sq / 64, order,
                                             (int64_t)BH * (Sq / 256), stream));
  }
  FwdArgs a;
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.tmask = tile_masks;
  a.ustart = ustart; a.ulen = ulen; a.ucols = ucols; a.pairmap = quadmap; a.order = order; a.Sq = Sq; a.Sk = Sk;
  a.npairs = (int)(Sq / 256);  // quads per head
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.o = (uint16_t*)o; a.lse = lse;
  a.total = (int)((int64_t)BH * a.npairs);
  a.queue = work_counter;
  if (a.queue) zero_counter_kernel<<<1, kQueueLanes, 0, stream>>>(a.queue);
  const int res = !a.queue ? 0 : D == 128 ? resident_workgroups<bsa_fwd_quad_kernel<128>>(512)
                                          : resident_workgroups<bsa_fwd_quad_kernel<64>>(512);
  const unsigned blocks = (unsigned)(a.queue && res < a.total ? res : a.total);
  if (D == 128) bsa_fwd_quad_kernel<128><<<blocks, 512, 0, stream>>>(a);
  else bsa_fwd_quad_kernel<64><<<blocks, 512, 0, stream>>>(a);
  PRISM_LAUNCH_CHECK("prism_bsa_fwd_quad");
  return PRISM_OK;
}

}  // extern "C"
