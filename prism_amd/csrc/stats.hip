// Macro-zone statistics and per-zone block-shape assignment (gfx950).
//
// Kernels (reference: hymm/models/modules/block_sparse_attention/):
//   zone_stats_kernel      compute_zone_aggregates (dynamic_block_shape.py:68-129)
//                          fused with the batch-0 head mean of V
//                          (dynamic_block_attention.py:236)
//   audio_zone_kernel      compute_audio_directional (dynamic_block_shape.py:189-245)
//   zone_gradient_kernel   compute_effective_gradient (dynamic_block_shape.py:248-289)
//   zone_shapes_kernel     rho / a_bar normalisation, g, select_shapes_ivpq /
//                          select_shapes_penalty (dynamic_block_shape.py:280-355)
//   a2v_norms_kernel       residual.norm(dim=-1) (wan_video_dit.py:742-752)
//
// Floating-point order is canonical (this file is compiled with
// -ffp-contract=off; fused operations are explicit):
//   * head mean: sequential fp32 sum over heads, times fl(1/H), rounded to V's
//     dtype;
//   * zone sums: r[lt][lh] = sum_lw, c[lt][lw] = sum_lh (valid tokens only),
//     frame = sum_lh r, hsum = sum_lt r, wsum = sum_lt c, total = sum_lt frame,
//     each sequential from +0; mean = sum / max(count, 1);
//   * channel reductions: lane l holds channels l (+ l+64), 64-lane xor
//     butterfly, times 1/D;
//   * norms: lane l owns 8-element chunks l, l+64, ..., fmaf(x, x, acc) in
//     element order, xor butterfly, sqrtf.
#include "common.h"

namespace {

constexpr int kZoneThreads = 512;  // 8 waves: wave index = frame lt

// One workgroup per zone.  Wave lt walks frame lt row by row; lane l owns
// channels [l*CPL, l*CPL + CPL).
// Raw loads of CPL channels (kept unconverted until they are added, so a
// load's wait is at its use) and their conversion to float
template <typename T, int CPL>
struct ChanRaw;
template <>
struct ChanRaw<uint16_t, 2> {
  using type = uint32_t;
  static __device__ __forceinline__ type load(const uint16_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
  static __device__ __forceinline__ void unpack(type u, float* x) {
    x[0] = __uint_as_float(u << 16);
    x[1] = __uint_as_float(u & 0xffff0000u);
  }
};
template <>
struct ChanRaw<uint16_t, 1> {
  using type = uint32_t;
  static __device__ __forceinline__ type load(const uint16_t* p) { return *p; }
  static __device__ __forceinline__ void unpack(type u, float* x) { x[0] = __uint_as_float(u << 16); }
};
template <>
struct ChanRaw<float, 2> {
  using type = float2;
  static __device__ __forceinline__ type load(const float* p) { return *reinterpret_cast<const float2*>(p); }
  static __device__ __forceinline__ void unpack(type f, float* x) {
    x[0] = f.x;
    x[1] = f.y;
  }
};
template <>
struct ChanRaw<float, 1> {
  using type = float;
  static __device__ __forceinline__ type load(const float* p) { return *p; }
  static __device__ __forceinline__ void unpack(type f, float* x) { x[0] = f; }
};

template <int D, typename T>
__global__ __launch_bounds__(kZoneThreads, sizeof(T) == 2 ? 6 : 4) void zone_stats_kernel(
    const T* __restrict__ v, int H, int64_t S, const uint8_t* __restrict__ valid,
    int ZH, int ZW, GridBox box, float invH, float* __restrict__ packed,
    uint8_t* __restrict__ axis_valid) {
  constexpr int CPL = D / 64;
  __shared__ float sRC[8][8][D];  // row sums r[lt][lh][d], later col sums c[lt][lw][d]
  __shared__ float sF[8][D];      // frame sums
  __shared__ uint8_t sValid[512];
  __shared__ int sCnt[25];        // cT[8], cH[8], cW[8], call

  const int z = blockIdx.x;
  const int tid = threadIdx.x;
  const int lt = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // (lt is wave-uniform)

  __shared__ int sPart[8][17];    // per frame t: valid tokens, per h, per w
  {
    const int64_t tok = token_in(z, tid, ZH, ZW, box);
    const uint8_t ok = tok < 0 ? (uint8_t)0 : valid ? valid[tok] : (uint8_t)1;
    sValid[tid] = ok;
    // wave lt holds frame lt: lane 8 h + w is token (lt, h, w)
    const uint64_t m = __ballot(ok != 0);
    if (lane < 17) {
      const uint64_t sel = lane == 0 ? ~0ull : lane <= 8 ? (0xffull << (8 * (lane - 1)))
                                                         : (0x0101010101010101ull << (lane - 9));
      sPart[lt][lane] = __popcll(m & sel);
    }
  }
  __syncthreads();
  if (tid < 25) {
    int cnt = 0;
    if (tid < 8) {
      cnt = sPart[tid][0];
    } else {
      const int col = tid < 24 ? tid - 7 : 0;  // h = tid - 8 -> column 1 + h; w = tid - 16 -> column 9 + w
      for (int t = 0; t < 8; ++t) cnt += sPart[t][col];
    }
    sCnt[tid] = cnt;
  }

  float cacc[8][CPL];
  float frame[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    frame[j] = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; ++w) cacc[w][j] = 0.0f;
  }
  // Steps k = 0 .. 8 NP - 1 (NP head pairs): row lh = k / NP, heads 2 hp and
  // 2 hp + 1 of its eight tokens (hp = k mod NP).  The sixteen loads of step
  // k + 1 are issued before step k is added, so a wave always has a step in
  // flight; every step issues all sixteen loads (positions outside the input
  // grid, or past the last head, re-read a valid address and are added as
  // zero), so the waits count loads statically.  Each token's head sum runs
  // over h in order from +0.
  using Raw = typename ChanRaw<T, CPL>::type;
  const int NP = (H + 1) >> 1, K = 8 * NP;
  const int nw_in = min(8, box.W - (z % ZW) * 8);  // tokens of a row inside the grid (if the row is)
  float acc[8][CPL];
#pragma unroll
  for (int lw = 0; lw < 8; ++lw)
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc[lw][j] = 0.0f;
  float r[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) r[j] = 0.0f;
  auto load_step = [&](int k, Raw (&b)[8][2]) {
    const int lh = k / NP, h = 2 * (k - lh * NP);
    const int64_t t0 = token_in(z, (lt * 8 + lh) * 8, ZH, ZW, box);
    const int nw = t0 < 0 ? 0 : nw_in;
    const int h1 = h + 1 < H ? h + 1 : h;
    // wave-uniform row bases of the two heads, plus this lane's channels
    const T* r0 = v + ((int64_t)h * S + (t0 < 0 ? 0 : t0)) * D;
    const T* r1 = v + ((int64_t)h1 * S + (t0 < 0 ? 0 : t0)) * D;
#pragma unroll
    for (int lw = 0; lw < 8; ++lw) {
      const int c = lw < nw ? lw : 0;
      b[lw][0] = ChanRaw<T, CPL>::load(r0 + c * D + lane * CPL);
      b[lw][1] = ChanRaw<T, CPL>::load(r1 + c * D + lane * CPL);
    }
  };
  auto add_step = [&](int k, const Raw (&b)[8][2]) {
    const int lh = k / NP, hp = k - lh * NP;
    const bool two = 2 * hp + 1 < H;
    const int nw = token_in(z, (lt * 8 + lh) * 8, ZH, ZW, box) < 0 ? 0 : nw_in;
#pragma unroll
    for (int lw = 0; lw < 8; ++lw) {
      float x0[CPL], x1[CPL];
      ChanRaw<T, CPL>::unpack(b[lw][0], x0);
      ChanRaw<T, CPL>::unpack(b[lw][1], x1);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const float y0 = lw < nw ? x0[j] : 0.0f, y1 = lw < nw ? x1[j] : 0.0f;
        acc[lw][j] = acc[lw][j] + y0;
        if (two) acc[lw][j] = acc[lw][j] + y1;
      }
    }
    if (hp == NP - 1) {  // row lh complete
#pragma unroll
      for (int lw = 0; lw < 8; ++lw) {
        const bool ok = sValid[(lt * 8 + lh) * 8 + lw] != 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          float a = acc[lw][j] * invH;
          if (sizeof(T) == 2) a = round_bf(a);
          r[j] = ok ? r[j] + a : r[j];
          cacc[lw][j] = ok ? cacc[lw][j] + a : cacc[lw][j];
          acc[lw][j] = 0.0f;
        }
      }
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        frame[j] = frame[j] + r[j];
        sRC[lt][lh][lane * CPL + j] = r[j];
        r[j] = 0.0f;
      }
    }
  };
  // (K is even; the loop has no branch around a load, so each add waits for
  // exactly its own step: the last iteration re-reads step K - 1 as a dummy)
  Raw b0[8][2], b1[8][2];
  load_step(0, b0);
  for (int k = 0; k < K; k += 2) {
    load_step(k + 1, b1);
    add_step(k, b0);
    load_step(k + 2 < K ? k + 2 : K - 1, b0);
    add_step(k + 1, b1);
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j) sF[lt][lane * CPL + j] = frame[j];
  __syncthreads();

  // packed[z] = channel(D) | frame(8D) | h(8D) | w(8D)
  float* out = packed + (int64_t)z * 25 * D;
  for (int o = tid; o < 17 * D; o += kZoneThreads) {
    const int sect = o / D, d = o - sect * D;
    float s = 0.0f;
    int cnt;
    if (sect == 0) {
      for (int t = 0; t < 8; ++t) s = s + sF[t][d];
      cnt = sCnt[24];
    } else if (sect <= 8) {
      s = sF[sect - 1][d];
      cnt = sCnt[sect - 1];
    } else {
      const int hh = sect - 9;
      for (int t = 0; t < 8; ++t) s = s + sRC[t][hh][d];
      cnt = sCnt[8 + hh];
    }
    out[o] = s / (float)(cnt > 0 ? cnt : 1);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int w = 0; w < 8; ++w) sRC[lt][w][lane * CPL + j] = cacc[w][j];
  __syncthreads();
  for (int o = tid; o < 8 * D; o += kZoneThreads) {
    const int ww = o / D, d = o - ww * D;
    float s = 0.0f;
    for (int t = 0; t < 8; ++t) s = s + sRC[t][ww][d];
    const int cnt = sCnt[16 + ww];
    out[17 * D + o] = s / (float)(cnt > 0 ? cnt : 1);
  }
  if (tid < 24) axis_valid[z * 24 + tid] = sCnt[tid] > 0;
}

// masked population variance over 8 positions (stride apart)
__device__ __forceinline__ float masked_var8(const float* a, int stride, const uint8_t* vflag) {
  float n = 0.0f, s = 0.0f, q = 0.0f;
  for (int p = 0; p < 8; ++p) n = n + (float)vflag[p];
  n = fmaxf(n, 1.0f);
  for (int p = 0; p < 8; ++p) s = s + a[p * stride] * (float)vflag[p];
  const float mean = s / n;
  for (int p = 0; p < 8; ++p) {
    const float dl = a[p * stride] - mean;
    q = q + (dl * dl) * (float)vflag[p];
  }
  return q / n;
}

// One 64-lane workgroup per zone.
template <typename T>
__global__ __launch_bounds__(64) void audio_zone_kernel(
    const T* __restrict__ norms, const uint8_t* __restrict__ valid, int ZH, int ZW, GridBox box,
    float* __restrict__ abar, float* __restrict__ vhat) {
  __shared__ float sA[512];
  __shared__ uint8_t sV[512];
  __shared__ float sRow[8][8], sCol[8][8];
  const int z = blockIdx.x, lane = threadIdx.x;
  for (int lf = lane; lf < 512; lf += 64) {
    const int64_t tok = token_in(z, lf, ZH, ZW, box);
    sA[lf] = tok < 0 ? 0.0f : ldf(norms, sizeof(T) == 2 ? PRISM_BF16 : PRISM_F32, tok);
    sV[lf] = tok < 0 ? (uint8_t)0 : valid ? valid[tok] : (uint8_t)1;
  }
  __syncthreads();
  {
    const int a = lane >> 3, b = lane & 7;
    float r = 0.0f, c = 0.0f;
    for (int i = 0; i < 8; ++i) {
      const int lr = (a * 8 + b) * 8 + i;   // (lt=a, lh=b, lw=i)
      r = sV[lr] ? r + sA[lr] : r;
      const int lc = (a * 8 + i) * 8 + b;   // (lt=a, lh=i, lw=b)
      c = sV[lc] ? c + sA[lc] : c;
    }
    sRow[a][b] = r;
    sCol[a][b] = c;
  }
  __syncthreads();
  // valid-token counts per frame, row and column from one ballot per frame
  // (lane 8 h + w of ballot t is token (t, h, w))
  uint64_t vb[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) vb[t] = __ballot(sV[t * 64 + lane] != 0);
  if (lane == 0) {
    int cT[8], cH[8], cW[8], call = 0;
    for (int i = 0; i < 8; ++i) cT[i] = cH[i] = cW[i] = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      cT[t] = __popcll(vb[t]);
      call += cT[t];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        cH[i] += __popcll(vb[t] & (0xffull << (8 * i)));
        cW[i] += __popcll(vb[t] & (0x0101010101010101ull << i));
      }
    }
    float frame[8], hs[8], ws[8], total = 0.0f;
    for (int t = 0; t < 8; ++t) {
      frame[t] = 0.0f;
      for (int h = 0; h < 8; ++h) frame[t] = frame[t] + sRow[t][h];
    }
    for (int i = 0; i < 8; ++i) {
      hs[i] = 0.0f; ws[i] = 0.0f;
      for (int t = 0; t < 8; ++t) { hs[i] = hs[i] + sRow[t][i]; ws[i] = ws[i] + sCol[t][i]; }
    }
    for (int t = 0; t < 8; ++t) total = total + frame[t];
    abar[z] = total / (float)(call > 0 ? call : 1);
    float m[3][8];
    uint8_t vv[3][8];
    for (int i = 0; i < 8; ++i) {
      m[0][i] = frame[i] / (float)(cT[i] > 0 ? cT[i] : 1); vv[0][i] = cT[i] > 0;
      m[1][i] = hs[i] / (float)(cH[i] > 0 ? cH[i] : 1);    vv[1][i] = cH[i] > 0;
      m[2][i] = ws[i] / (float)(cW[i] > 0 ? cW[i] : 1);    vv[2][i] = cW[i] > 0;
    }
    float var[3];
    for (int a = 0; a < 3; ++a) var[a] = masked_var8(m[a], 1, vv[a]);
    const float den = fmaxf((var[0] + var[1]) + var[2], 1e-6f);
    for (int a = 0; a < 3; ++a) vhat[z * 3 + a] = var[a] / den;
  }
}

// One wave per zone; lane l owns channels l and l + 64 (D = 128) or l (D = 64).
template <int D>
__global__ __launch_bounds__(64) void zone_gradient_kernel(
    const float* __restrict__ packed, const uint8_t* __restrict__ axis_valid,
    float* __restrict__ rho_raw, float* __restrict__ aniso) {
  constexpr int CPL = D / 64;
  const int z = blockIdx.x, lane = threadIdx.x;
  const float* cm = packed + (int64_t)z * 25 * D;
  const float* fr = cm + D;
  const float* hm = cm + 9 * D;
  const float* wm = cm + 17 * D;
  __shared__ uint8_t av[24];
  if (lane < 24) av[lane] = axis_valid[z * 24 + lane];
  __syncthreads();
  const float invD = 1.0f / (float)D;

  auto lane_pair = [&](float a0, float a1) { return CPL == 2 ? a0 + a1 : a0; };

  float c0 = cm[lane], c1 = CPL == 2 ? cm[lane + 64] : 0.0f;
  const float gcm = wave_sum_xor(lane_pair(c0, c1)) * invD;
  float t0 = c0 - gcm, t1 = c1 - gcm;
  const float sv = wave_sum_xor(lane_pair(t0 * t0, t1 * t1)) * invD;

  float bv[7], np = 0.0f;
  for (int t = 0; t < 7; ++t) { bv[t] = (float)(av[t] && av[t + 1]); np = np + bv[t]; }
  np = fmaxf(np, 1.0f);
  float tvv[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int d = lane + 64 * j;
    float acc = 0.0f;
    for (int t = 0; t < 7; ++t) {
      const float df = fr[(t + 1) * D + d] - fr[t * D + d];
      acc = acc + (df * df) * bv[t];
    }
    tvv[j] = acc / np;
  }
  const float tv = wave_sum_xor(lane_pair(tvv[0], CPL == 2 ? tvv[CPL - 1] : 0.0f)) * invD;

  float var[3];
  const float* axes[3] = {fr, hm, wm};
  for (int a = 0; a < 3; ++a) {
    float vv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) vv[j] = masked_var8(axes[a] + lane + 64 * j, D, av + 8 * a);
    var[a] = wave_sum_xor(lane_pair(vv[0], CPL == 2 ? vv[CPL - 1] : 0.0f)) * invD;
  }
  if (lane == 0) {
    rho_raw[z] = sv + tv;
    const float asum = fmaxf((var[0] + var[1]) + var[2], 1e-6f);
    for (int a = 0; a < 3; ++a) aniso[z * 3 + a] = var[a] / asum;
  }
}

constexpr int kShapeThreads = 256;

// Shape decision for one zone: select_shapes_ivpq (method 0) /
// select_shapes_penalty (method 1); first index wins ties.
__device__ __forceinline__ int decide_shape(const float* g, float rho, int method, float tau_128, float lambda_128) {
  const bool forbid128 = rho >= tau_128;
  float best = __uint_as_float(0x7f800000u);
  int bi = 0;
  if (method == 0) {
    float l[3];
    for (int a = 0; a < 3; ++a) l[a] = -0.666666686534881591796875f * canon_log2(g[a]);
    const float cc = (6.0f - ((l[0] + l[1]) + l[2])) / 3.0f;
    const float ideal[3] = {l[0] + cc, l[1] + cc, l[2] + cc};
    for (int c = 0; c < PRISM_NCAND; ++c) {
      float dd[3];
      for (int a = 0; a < 3; ++a) {
        const float ls = (float)(31 - __builtin_clz((unsigned)kCand[c][a]));
        const float t = ls - ideal[a];
        dd[a] = t * t;
      }
      float dist = (dd[0] + dd[1]) + dd[2];
      if (c >= 7 && forbid128) dist = __uint_as_float(0x7f800000u);
      if (dist < best) { best = dist; bi = c; }
    }
  } else {
    const float bonus = lambda_128 * (1.0f - rho);
    for (int c = 0; c < PRISM_NCAND; ++c) {
      float pen = (g[0] * (float)kCand[c][0] + g[1] * (float)kCand[c][1]) + g[2] * (float)kCand[c][2];
      pen = pen - (c >= 7 ? bonus : 0.0f);
      if (c >= 7 && forbid128) pen = __uint_as_float(0x7f800000u);
      if (pen < best) { best = pen; bi = c; }
    }
  }
  return bi;
}

// Single workgroup: maxima over zones, then one thread per zone.
__global__ __launch_bounds__(kShapeThreads) void zone_shapes_kernel(
    const float* __restrict__ rho_raw, const float* __restrict__ aniso, const float* __restrict__ abar,
    const float* __restrict__ vhat, int Nz, int method, float lambda_a, float tau_128, float lambda_128,
    float* __restrict__ g_out, float* __restrict__ rho_out, int64_t* __restrict__ shape_ids) {
  __shared__ float sMax[2][kShapeThreads / 64];
  const int tid = threadIdx.x;
  float mr = -__uint_as_float(0x7f800000u), ma = mr;
  for (int z = tid; z < Nz; z += kShapeThreads) {
    mr = fmaxf(mr, rho_raw[z]);
    if (abar) ma = fmaxf(ma, abar[z]);
  }
  mr = wave_max_xor(mr);
  ma = wave_max_xor(ma);
  if ((tid & 63) == 0) { sMax[0][tid >> 6] = mr; sMax[1][tid >> 6] = ma; }
  __syncthreads();
  mr = sMax[0][0]; ma = sMax[1][0];
  for (int w = 1; w < kShapeThreads / 64; ++w) { mr = fmaxf(mr, sMax[0][w]); ma = fmaxf(ma, sMax[1][w]); }
  const float rden = fmaxf(mr, 1e-6f);
  const float aden = abar ? fmaxf(ma, 1e-6f) : 1.0f;

  for (int z = tid; z < Nz; z += kShapeThreads) {
    const float rho = rho_raw[z] / rden;
    const float an = abar ? abar[z] / aden : 0.0f;
    float g[3];
    for (int a = 0; a < 3; ++a) {
      const float vh = abar ? vhat[z * 3 + a] : 0.0f;
      g[a] = fmaxf(aniso[z * 3 + a] + (lambda_a * an) * vh, 1e-4f);
      g_out[z * 3 + a] = g[a];
    }
    rho_out[z] = rho;
    shape_ids[z] = decide_shape(g, rho, method, tau_128, lambda_128);
  }
}

__global__ void assign_shapes_kernel(const float* __restrict__ g, const float* __restrict__ rho, int Nz, int method,
                                     float tau_128, float lambda_128, int64_t* __restrict__ shape_ids) {
  const int z = blockIdx.x * blockDim.x + threadIdx.x;
  if (z >= Nz) return;
  const float gz[3] = {g[z * 3 + 0], g[z * 3 + 1], g[z * 3 + 2]};
  shape_ids[z] = decide_shape(gz, rho[z], method, tau_128, lambda_128);
}

// One wave per token, 4 tokens per workgroup.
template <typename T, typename TO>
__global__ __launch_bounds__(256) void a2v_norms_kernel(const T* __restrict__ res, int64_t S, int C,
                                                        TO* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= S) return;
  const T* row = res + s * C;
  const int nch = C / 8;
  float acc = 0.0f;
  for (int j = lane; j < nch; j += 64) {
    float x[8];
    if (sizeof(T) == 2) {
      const uint4 u = *reinterpret_cast<const uint4*>(row + j * 8);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = __uint_as_float(w[e] << 16);
        x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
      }
    } else {
      const float4 a = *reinterpret_cast<const float4*>(row + j * 8);
      const float4 b = *reinterpret_cast<const float4*>(row + j * 8 + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(x[e], x[e], acc);
  }
  const float n = sqrtf(wave_sum_xor(acc));
  if (lane == 0) {
    if (sizeof(TO) == 2) reinterpret_cast<uint16_t*>(out)[s] = f2bf(n);
    else reinterpret_cast<float*>(out)[s] = n;
  }
}

bool grid_ok(int T, int Hg, int Wg) { return T > 0 && Hg > 0 && Wg > 0 && T % 8 == 0 && Hg % 8 == 0 && Wg % 8 == 0; }

}  // namespace

extern "C" {

int prism_zone_stats(const void* v, int dtype, int H, int64_t S, int D, const uint8_t* valid, int T,
                     int Hg, int Wg, int Tin, int Hin, int Win, float* packed, uint8_t* axis_valid,
                     hipStream_t stream) {
  PRISM_REQUIRE(v && packed && axis_valid, "prism_zone_stats: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_zone_stats: grid (%d,%d,%d) must be multiples of 8", T, Hg, Wg);
  PRISM_REQUIRE(box_ok(T, Hg, Wg, Tin, Hin, Win), "prism_zone_stats: input grid (%d,%d,%d) must fit the zone grid",
                Tin, Hin, Win);
  PRISM_REQUIRE((int64_t)Tin * Hin * Win == S, "prism_zone_stats: Tin*Hin*Win != S");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_zone_stats: head_dim %d unsupported (64, 128)", D);
  PRISM_REQUIRE(H >= 1, "prism_zone_stats: H must be >= 1");
  PRISM_REQUIRE(dtype == PRISM_F32 || dtype == PRISM_BF16, "prism_zone_stats: bad dtype");
  const int ZH = Hg / 8, ZW = Wg / 8, Nz = (T / 8) * ZH * ZW;
  const float invH = 1.0f / (float)H;
  const GridBox box{Tin, Hin, Win};
  dim3 grid(Nz), block(kZoneThreads);
  if (dtype == PRISM_BF16) {
    if (D == 128) zone_stats_kernel<128, uint16_t><<<grid, block, 0, stream>>>((const uint16_t*)v, H, S, valid, ZH, ZW, box, invH, packed, axis_valid);
    else zone_stats_kernel<64, uint16_t><<<grid, block, 0, stream>>>((const uint16_t*)v, H, S, valid, ZH, ZW, box, invH, packed, axis_valid);
  } else {
    if (D == 128) zone_stats_kernel<128, float><<<grid, block, 0, stream>>>((const float*)v, H, S, valid, ZH, ZW, box, invH, packed, axis_valid);
    else zone_stats_kernel<64, float><<<grid, block, 0, stream>>>((const float*)v, H, S, valid, ZH, ZW, box, invH, packed, axis_valid);
  }
  PRISM_LAUNCH_CHECK("prism_zone_stats");
  return PRISM_OK;
}

int prism_audio_zone_stats(const void* norms, int dtype, const uint8_t* valid, int T, int Hg, int Wg, int Tin,
                           int Hin, int Win, float* abar, float* vhat, hipStream_t stream) {
  PRISM_REQUIRE(norms && abar && vhat, "prism_audio_zone_stats: null pointer");
  PRISM_REQUIRE(grid_ok(T, Hg, Wg), "prism_audio_zone_stats: grid must be multiples of 8");
  PRISM_REQUIRE(box_ok(T, Hg, Wg, Tin, Hin, Win), "prism_audio_zone_stats: input grid must fit the zone grid");
  const GridBox box{Tin, Hin, Win};
  PRISM_REQUIRE(dtype == PRISM_F32 || dtype == PRISM_BF16, "prism_audio_zone_stats: bad dtype");
  const int ZH = Hg / 8, ZW = Wg / 8, Nz = (T / 8) * ZH * ZW;
  if (dtype == PRISM_BF16)
    audio_zone_kernel<uint16_t><<<Nz, 64, 0, stream>>>((const uint16_t*)norms, valid, ZH, ZW, box, abar, vhat);
  else
    audio_zone_kernel<float><<<Nz, 64, 0, stream>>>((const float*)norms, valid, ZH, ZW, box, abar, vhat);
  PRISM_LAUNCH_CHECK("prism_audio_zone_stats");
  return PRISM_OK;
}

int prism_zone_gradient(const float* packed, const uint8_t* axis_valid, int Nz, int D, float* rho_raw,
                        float* aniso, hipStream_t stream) {
  PRISM_REQUIRE(packed && axis_valid && rho_raw && aniso, "prism_zone_gradient: null pointer");
  PRISM_REQUIRE(D == 64 || D == 128, "prism_zone_gradient: head_dim %d unsupported", D);
  PRISM_REQUIRE(Nz >= 1, "prism_zone_gradient: Nz must be >= 1");
  if (D == 128) zone_gradient_kernel<128><<<Nz, 64, 0, stream>>>(packed, axis_valid, rho_raw, aniso);
  else zone_gradient_kernel<64><<<Nz, 64, 0, stream>>>(packed, axis_valid, rho_raw, aniso);
  PRISM_LAUNCH_CHECK("prism_zone_gradient");
  return PRISM_OK;
}

int prism_zone_shapes(const float* rho_raw, const float* aniso, const float* abar, const float* vhat, int Nz,
                      int method, float lambda_a, float tau_128, float lambda_128, float* g, float* rho,
                      int64_t* shape_ids, hipStream_t stream) {
  PRISM_REQUIRE(rho_raw && aniso && g && rho && shape_ids, "prism_zone_shapes: null pointer");
  PRISM_REQUIRE((abar == nullptr) == (vhat == nullptr), "prism_zone_shapes: abar and vhat go together");
  PRISM_REQUIRE(method == 0 || method == 1, "prism_zone_shapes: unknown method %d", method);
  PRISM_REQUIRE(Nz >= 1, "prism_zone_shapes: Nz must be >= 1");
  zone_shapes_kernel<<<1, kShapeThreads, 0, stream>>>(rho_raw, aniso, abar, vhat, Nz, method, lambda_a, tau_128,
                                                      lambda_128, g, rho, shape_ids);
  PRISM_LAUNCH_CHECK("prism_zone_shapes");
  return PRISM_OK;
}

int prism_assign_shapes(const float* g, const float* rho, int Nz, int method, float tau_128, float lambda_128,
                        int64_t* shape_ids, hipStream_t stream) {
  PRISM_REQUIRE(g && rho && shape_ids, "prism_assign_shapes: null pointer");
  PRISM_REQUIRE(method == 0 || method == 1, "prism_assign_shapes: unknown method %d", method);
  PRISM_REQUIRE(Nz >= 1, "prism_assign_shapes: Nz must be >= 1");
  assign_shapes_kernel<<<(Nz + 255) / 256, 256, 0, stream>>>(g, rho, Nz, method, tau_128, lambda_128, shape_ids);
  PRISM_LAUNCH_CHECK("prism_assign_shapes");
  return PRISM_OK;
}

int prism_a2v_norms(const void* res, int dtype, int64_t S, int C, void* out, int out_dtype, hipStream_t stream) {
  PRISM_REQUIRE(res && out, "prism_a2v_norms: null pointer");
  PRISM_REQUIRE(C > 0 && C % 8 == 0, "prism_a2v_norms: C=%d must be a positive multiple of 8", C);
  PRISM_REQUIRE(S >= 0, "prism_a2v_norms: S < 0");
  PRISM_REQUIRE(dtype == PRISM_F32 || dtype == PRISM_BF16, "prism_a2v_norms: bad dtype");
  PRISM_REQUIRE(out_dtype == PRISM_F32 || out_dtype == PRISM_BF16, "prism_a2v_norms: bad out dtype");
  if (S == 0) return PRISM_OK;
  const int64_t blocks = (S + 3) / 4;
  if (dtype == PRISM_BF16) {
    if (out_dtype == PRISM_BF16) a2v_norms_kernel<uint16_t, uint16_t><<<blocks, 256, 0, stream>>>((const uint16_t*)res, S, C, (uint16_t*)out);
    else a2v_norms_kernel<uint16_t, float><<<blocks, 256, 0, stream>>>((const uint16_t*)res, S, C, (float*)out);
  } else {
    if (out_dtype == PRISM_BF16) a2v_norms_kernel<float, uint16_t><<<blocks, 256, 0, stream>>>((const float*)res, S, C, (uint16_t*)out);
    else a2v_norms_kernel<float, float><<<blocks, 256, 0, stream>>>((const float*)res, S, C, (float*)out);
  }
  PRISM_LAUNCH_CHECK("prism_a2v_norms");
  return PRISM_OK;
}

}  // extern "C"
