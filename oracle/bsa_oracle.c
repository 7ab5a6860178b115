/*
 * bsa_oracle.c -- CPU restatement of Prism's dynamic block-sparse attention
 * selection path (TEST INFRASTRUCTURE ONLY).
 *
 * This file is the parity oracle.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it, and only as the checker.  The product
 * (prism_amd/) never links, imports or calls it.
 *
 * Every function follows a reference function (file:line under the reference
 * tree hymm/models/modules/...) and fixes one canonical floating-point
 * evaluation order for it.  The HIP kernels in prism_amd/csrc/ implement the
 * same order independently, so parity is bit-exact.  Canonical choices that
 * differ from "whatever torch happened to do" are listed at each function and
 * are pinned against independent mathematics in tests/test_oracle_*.py.
 *
 * Arithmetic rules used throughout (compile with -ffp-contract=off):
 *   - every add/mul/div is one IEEE fp32 operation, round-to-nearest-even;
 *   - fused multiply-adds are written explicitly as fmaf();
 *   - "sum_lanes" is the 64-lane xor butterfly defined in sum_lanes64();
 *   - exp / log2 are canon_exp / canon_log2 below (not libm), so the device
 *     code can reproduce them exactly.
 *
 * Parity status per function (see the test that pins each one):
 *   canon_exp, canon_log2 ............ pinned vs libm (ulp bound, exact cases)
 *   oc_zone_stats .................... pinned vs float64 numpy means
 *   oc_zone_gradient, oc_zone_shapes . pinned by closed-form grids
 *   oc_audio_zone_stats .............. pinned vs float64 numpy
 *   oc_a2v_norms ..................... pinned vs float64 norms
 *   oc_rearrange_index, oc_tile_maps . pinned by brute-force invariants
 *   oc_block_pool .................... pinned vs float64 numpy
 *   oc_block_scores .................. pinned vs float64 matmul
 *   oc_select ........................ pinned vs brute-force exact-rational
 *                                      selection and torch semantics (margin)
 *   oc_expand_tiles, oc_transpose_lists pinned by brute force
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ZS 8          /* macro-zone edge: dynamic_block_shape.py:31 */
#define TILE 64       /* kernel tile: dynamic_block_attention.py:15 */
#define NCAND 13      /* dynamic_block_shape.py:6-29 */

/* Candidate block shapes, table order of dynamic_block_shape.py:6-27. */
static const int CAND[NCAND][3] = {
    {4, 4, 4}, {8, 2, 4}, {8, 4, 2}, {2, 4, 8}, {2, 8, 4}, {4, 2, 8}, {4, 8, 2},
    {2, 8, 8}, {8, 2, 8}, {8, 8, 2}, {4, 4, 8}, {4, 8, 4}, {8, 4, 4},
};

int oc_num_candidates(void) { return NCAND; }
void oc_candidates(int *out) { memcpy(out, CAND, sizeof(CAND)); }

/* ------------------------------------------------------------------ */
/* scalar helpers                                                      */
/* ------------------------------------------------------------------ */
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bf2f(uint16_t h) { return u2f((uint32_t)h << 16); }
static inline uint16_t f2bf(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static inline float round_bf(float f) { return bf2f(f2bf(f)); }
/* dtype codes shared with the product's C-ABI: 0 = fp32, 1 = bf16 */
static inline float ld(const void *p, int dtype, int64_t i) {
    return dtype ? bf2f(((const uint16_t *)p)[i]) : ((const float *)p)[i];
}
static inline float fmax_(float a, float b) { return a > b ? a : b; }

/* canon_exp: Cody-Waite reduction with the Cephes split of ln 2
 * (C1 = 0.693359375, C2 = -2.12194440e-4), then the degree-7 Taylor
 * polynomial of e^r on |r| <= ln2/2 in Horner form with fmaf, then an exact
 * power-of-two scale.  Inputs below -87 return 0 (no subnormal results). */
float canon_exp(float x) {
    if (x != x) return x;
    if (x > 88.0f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    float t = x * 1.44269504f;
    float n = floorf(t + 0.5f);
    float r = fmaf(-n, 0.693359375f, x);
    r = fmaf(-n, -2.12194440e-4f, r);
    float p = 1.98412698e-4f;          /* 1/7! */
    p = fmaf(p, r, 1.38888889e-3f);    /* 1/6! */
    p = fmaf(p, r, 8.33333333e-3f);    /* 1/5! */
    p = fmaf(p, r, 4.16666667e-2f);    /* 1/4! */
    p = fmaf(p, r, 1.66666667e-1f);    /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    return p * u2f((uint32_t)(ni + 127) << 23);
}

/* canon_log2 for positive, finite, normal x: x = m 2^e with m in
 * [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s), s = (m-1)/(m+1), odd series to
 * s^11 (Horner in s^2 with fmaf), log2 x = e + ln(m) * log2(e). */
float canon_log2(float x) {
    uint32_t u = f2u(x);
    int e = (int)((u >> 23) & 0xffu) - 127;
    float m = u2f((u & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
    float s = (m - 1.0f) / (m + 1.0f);
    float z = s * s;
    float p = 0.0909090909f;           /* 1/11 */
    p = fmaf(p, z, 0.111111111f);      /* 1/9 */
    p = fmaf(p, z, 0.142857143f);      /* 1/7 */
    p = fmaf(p, z, 0.2f);              /* 1/5 */
    p = fmaf(p, z, 0.333333333f);      /* 1/3 */
    float s2 = s + s;
    float lnm = fmaf(s2 * z, p, s2);
    return fmaf(lnm, 1.44269504f, (float)e);
}

/* 64-lane xor butterfly sum.  vals has n entries, n in {64, 128}; lane l
 * first forms vals[l] (+ vals[l+64]), then for off = 32..1 adds its xor
 * partner.  All lanes end equal; lane 0's value is returned. */
static float sum_lanes64(const float *vals, int n) {
    float p[64], q[64];
    for (int l = 0; l < 64; ++l) p[l] = (n == 128) ? vals[l] + vals[l + 64] : vals[l];
    for (int off = 32; off >= 1; off >>= 1) {
        for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ off];
        memcpy(p, q, sizeof(p));
    }
    return p[0];
}
float oc_sum_lanes64(const float *vals, int n) { return sum_lanes64(vals, n); }

/* exact floor(w * 2^F) of a finite w >= 0 (w * 2^F < 2^63) */
static inline uint64_t fixp(float w, int F) {
    uint32_t u = f2u(w);
    int e = (int)((u >> 23) & 0xffu);
    uint64_t m = u & 0x7fffffu;
    if (e == 0) e = 1; else m |= 0x800000u;
    int sh = e - 150 + F;
    if (sh >= 0) return m << sh;
    sh = -sh;
    return sh >= 64 ? 0 : (m >> sh);
}

/* ------------------------------------------------------------------ */
/* (a4) zone aggregates                                                */
/* ------------------------------------------------------------------ */
/* Head average of batch 0 (dynamic_block_attention.py:236,
 * v[0].mean(dim=0)): sequential fp32 sum over heads, times fl(1/H), rounded
 * to V's dtype.  Then the masked zone means of compute_zone_aggregates
 * (dynamic_block_shape.py:68-129) with the canonical order:
 *   r[lt][lh] = sum over lw, c[lt][lw] = sum over lh (valid tokens only),
 *   frame[lt] = sum_lh r, hsum[lh] = sum_lt r, wsum[lw] = sum_lt c,
 *   total = sum_lt frame, each sequential from 0.0f; mean = sum / max(cnt,1).
 * packed[z] = [chan(D) | frame(8D) | hmean(8D) | wmean(8D)], axis_valid[z] =
 * [t(8) | h(8) | w(8)] "has >= 1 valid token" flags. */
void oc_zone_stats(const void *v, int dtype, int H, int64_t S, int D,
                   const uint8_t *valid, int T, int Hg, int Wg,
                   float *packed, uint8_t *axis_valid) {
    (void)T;
    int ZH = Hg / ZS, ZW = Wg / ZS, ZT = T / ZS;
    int Nz = ZT * ZH * ZW;
    float invH = 1.0f / (float)H;
    float *x = (float *)malloc(sizeof(float) * 512 * D);
    for (int z = 0; z < Nz; ++z) {
        int zt = z / (ZH * ZW), zh = (z / ZW) % ZH, zw = z % ZW;
        int vmask[512];
        for (int lt = 0; lt < 8; ++lt)
            for (int lh = 0; lh < 8; ++lh)
                for (int lw = 0; lw < 8; ++lw) {
                    int64_t tok = ((int64_t)(zt * 8 + lt) * Hg + zh * 8 + lh) * Wg + zw * 8 + lw;
                    int li = (lt * 8 + lh) * 8 + lw;
                    vmask[li] = valid ? (valid[tok] != 0) : 1;
                    for (int d = 0; d < D; ++d) {
                        float acc = 0.0f;
                        for (int h = 0; h < H; ++h) acc = acc + ld(v, dtype, ((int64_t)h * S + tok) * D + d);
                        float a = acc * invH;
                        x[li * D + d] = dtype ? round_bf(a) : a;
                    }
                }
        int cT[8] = {0}, cH[8] = {0}, cW[8] = {0}, call = 0;
        for (int li = 0; li < 512; ++li)
            if (vmask[li]) { cT[li / 64]++; cH[(li / 8) % 8]++; cW[li % 8]++; call++; }
        float *out = packed + (int64_t)z * 25 * D;
        for (int d = 0; d < D; ++d) {
            float r[8][8], c[8][8], frame[8], hs[8], ws[8], total = 0.0f;
            for (int lt = 0; lt < 8; ++lt) {
                for (int i = 0; i < 8; ++i) { r[lt][i] = 0.0f; c[lt][i] = 0.0f; }
                for (int lh = 0; lh < 8; ++lh)
                    for (int lw = 0; lw < 8; ++lw) {
                        int li = (lt * 8 + lh) * 8 + lw;
                        if (!vmask[li]) continue;
                        float xv = x[li * D + d];
                        r[lt][lh] = r[lt][lh] + xv;
                        c[lt][lw] = c[lt][lw] + xv;
                    }
                frame[lt] = 0.0f;
                for (int lh = 0; lh < 8; ++lh) frame[lt] = frame[lt] + r[lt][lh];
            }
            for (int i = 0; i < 8; ++i) {
                hs[i] = 0.0f; ws[i] = 0.0f;
                for (int lt = 0; lt < 8; ++lt) { hs[i] = hs[i] + r[lt][i]; ws[i] = ws[i] + c[lt][i]; }
            }
            for (int lt = 0; lt < 8; ++lt) total = total + frame[lt];
            out[d] = total / (float)(call > 0 ? call : 1);
            for (int i = 0; i < 8; ++i) {
                out[D + i * D + d] = frame[i] / (float)(cT[i] > 0 ? cT[i] : 1);
                out[9 * D + i * D + d] = hs[i] / (float)(cH[i] > 0 ? cH[i] : 1);
                out[17 * D + i * D + d] = ws[i] / (float)(cW[i] > 0 ? cW[i] : 1);
            }
        }
        for (int i = 0; i < 8; ++i) {
            axis_valid[z * 24 + i] = cT[i] > 0;
            axis_valid[z * 24 + 8 + i] = cH[i] > 0;
            axis_valid[z * 24 + 16 + i] = cW[i] > 0;
        }
    }
    free(x);
}

/* masked population variance over 8 positions (one channel):
 * _axis_var / _masked_var_1d (dynamic_block_shape.py:165-186). */
static float masked_var8(const float *a, int stride, const uint8_t *valid) {
    float n = 0.0f, s = 0.0f, q = 0.0f;
    for (int p = 0; p < 8; ++p) n = n + (float)valid[p];
    n = fmax_(n, 1.0f);
    for (int p = 0; p < 8; ++p) s = s + a[p * stride] * (float)valid[p];
    float mean = s / n;
    for (int p = 0; p < 8; ++p) { float dlt = a[p * stride] - mean; q = q + (dlt * dlt) * (float)valid[p]; }
    return q / n;
}

/* (a5) per-zone part of compute_effective_gradient
 * (dynamic_block_shape.py:248-289): rho_raw = spatial + temporal variance and
 * the anisotropy ratios.  Channel means use sum_lanes64 and * (1/D).
 * out: rho_raw[Nz], aniso[Nz*3]. */
void oc_zone_gradient(const float *packed, const uint8_t *axis_valid, int Nz, int D,
                      float *rho_raw, float *aniso) {
    float invD = 1.0f / (float)D;
    float *tmp = (float *)malloc(sizeof(float) * D);
    for (int z = 0; z < Nz; ++z) {
        const float *cm = packed + (int64_t)z * 25 * D;
        const float *fr = cm + D, *hm = cm + 9 * D, *wm = cm + 17 * D;
        const uint8_t *av = axis_valid + z * 24;
        float gcm = sum_lanes64(cm, D) * invD;
        for (int d = 0; d < D; ++d) { float t = cm[d] - gcm; tmp[d] = t * t; }
        float sv = sum_lanes64(tmp, D) * invD;
        float bv[7], np = 0.0f;
        for (int t = 0; t < 7; ++t) { bv[t] = (float)(av[t] && av[t + 1]); np = np + bv[t]; }
        np = fmax_(np, 1.0f);
        for (int d = 0; d < D; ++d) {
            float acc = 0.0f;
            for (int t = 0; t < 7; ++t) { float df = fr[(t + 1) * D + d] - fr[t * D + d]; acc = acc + (df * df) * bv[t]; }
            tmp[d] = acc / np;
        }
        float tv = sum_lanes64(tmp, D) * invD;
        rho_raw[z] = sv + tv;
        float var[3];
        const float *axes[3] = {fr, hm, wm};
        for (int a = 0; a < 3; ++a) {
            for (int d = 0; d < D; ++d) tmp[d] = masked_var8(axes[a] + d, D, av + 8 * a);
            var[a] = sum_lanes64(tmp, D) * invD;
        }
        float asum = fmax_((var[0] + var[1]) + var[2], 1e-6f);
        for (int a = 0; a < 3; ++a) aniso[z * 3 + a] = var[a] / asum;
    }
    free(tmp);
}

/* (a6) per-zone part of compute_audio_directional
 * (dynamic_block_shape.py:189-245): masked mean a_bar (not yet
 * max-normalised) and the normalised directional variances.  The canonical
 * sum order is the one of oc_zone_stats with D = 1, and the masked variance
 * formula is used also when no mask is given.  out: abar[Nz], vhat[Nz*3]. */
void oc_audio_zone_stats(const void *norms, int dtype, const uint8_t *valid,
                         int T, int Hg, int Wg, float *abar, float *vhat) {
    int ZT = T / ZS, ZH = Hg / ZS, ZW = Wg / ZS, Nz = ZT * ZH * ZW;
    for (int z = 0; z < Nz; ++z) {
        int zt = z / (ZH * ZW), zh = (z / ZW) % ZH, zw = z % ZW;
        float r[8][8], c[8][8], frame[8], hs[8], ws[8], total = 0.0f;
        int cT[8] = {0}, cH[8] = {0}, cW[8] = {0}, call = 0;
        for (int lt = 0; lt < 8; ++lt) {
            for (int i = 0; i < 8; ++i) { r[lt][i] = 0.0f; c[lt][i] = 0.0f; }
            for (int lh = 0; lh < 8; ++lh)
                for (int lw = 0; lw < 8; ++lw) {
                    int64_t tok = ((int64_t)(zt * 8 + lt) * Hg + zh * 8 + lh) * Wg + zw * 8 + lw;
                    if (valid && !valid[tok]) continue;
                    float a = ld(norms, dtype, tok);
                    r[lt][lh] = r[lt][lh] + a;
                    c[lt][lw] = c[lt][lw] + a;
                    cT[lt]++; cH[lh]++; cW[lw]++; call++;
                }
            frame[lt] = 0.0f;
            for (int lh = 0; lh < 8; ++lh) frame[lt] = frame[lt] + r[lt][lh];
        }
        for (int i = 0; i < 8; ++i) {
            hs[i] = 0.0f; ws[i] = 0.0f;
            for (int lt = 0; lt < 8; ++lt) { hs[i] = hs[i] + r[lt][i]; ws[i] = ws[i] + c[lt][i]; }
        }
        for (int lt = 0; lt < 8; ++lt) total = total + frame[lt];
        abar[z] = total / (float)(call > 0 ? call : 1);
        float m[3][8]; uint8_t vv[3][8];
        for (int i = 0; i < 8; ++i) {
            m[0][i] = frame[i] / (float)(cT[i] > 0 ? cT[i] : 1); vv[0][i] = cT[i] > 0;
            m[1][i] = hs[i] / (float)(cH[i] > 0 ? cH[i] : 1);    vv[1][i] = cH[i] > 0;
            m[2][i] = ws[i] / (float)(cW[i] > 0 ? cW[i] : 1);    vv[2][i] = cW[i] > 0;
        }
        float var[3];
        for (int a = 0; a < 3; ++a) var[a] = masked_var8(m[a], 1, vv[a]);
        float den = fmax_((var[0] + var[1]) + var[2], 1e-6f);
        for (int a = 0; a < 3; ++a) vhat[z * 3 + a] = var[a] / den;
    }
}

/* (a5 tail + a7) normalisation over zones and the per-zone shape decision:
 * compute_effective_gradient (dynamic_block_shape.py:280, :297-300),
 * compute_audio_directional (:244), select_shapes_ivpq (:303-327) and
 * select_shapes_penalty (:330-355).  method 0 = ivpq, 1 = penalty.
 * abar/vhat may be NULL (no audio).  Ties in argmin go to the first index. */
void oc_zone_shapes(const float *rho_raw, const float *aniso, const float *abar,
                    const float *vhat, int Nz, int method, float lambda_a,
                    float tau_128, float lambda_128, float *g_out, float *rho_out,
                    int64_t *shape_ids) {
    float mr = -INFINITY, ma = -INFINITY;
    for (int z = 0; z < Nz; ++z) mr = fmax_(mr, rho_raw[z]);
    float rden = fmax_(mr, 1e-6f);
    float aden = 1.0f;
    if (abar) { for (int z = 0; z < Nz; ++z) ma = fmax_(ma, abar[z]); aden = fmax_(ma, 1e-6f); }
    for (int z = 0; z < Nz; ++z) {
        float rho = rho_raw[z] / rden;
        float an = abar ? abar[z] / aden : 0.0f;
        float g[3];
        for (int a = 0; a < 3; ++a) {
            float vh = abar ? vhat[z * 3 + a] : 0.0f;
            g[a] = fmax_(aniso[z * 3 + a] + (lambda_a * an) * vh, 1e-4f);
            g_out[z * 3 + a] = g[a];
        }
        rho_out[z] = rho;
        int forbid128 = rho >= tau_128;
        float best = INFINITY; int bi = 0;
        if (method == 0) {
            float l[3];
            for (int a = 0; a < 3; ++a) l[a] = -0.666666686534881591796875f * canon_log2(g[a]);
            float cc = (6.0f - ((l[0] + l[1]) + l[2])) / 3.0f;
            float ideal[3] = {l[0] + cc, l[1] + cc, l[2] + cc};
            for (int c = 0; c < NCAND; ++c) {
                float dd[3];
                for (int a = 0; a < 3; ++a) { float ls = (float)(31 - __builtin_clz(CAND[c][a])); float t = ls - ideal[a]; dd[a] = t * t; }
                float dist = (dd[0] + dd[1]) + dd[2];
                if (c >= 7 && forbid128) dist = INFINITY;
                if (dist < best) { best = dist; bi = c; }
            }
        } else {
            float bonus = lambda_128 * (1.0f - rho);
            for (int c = 0; c < NCAND; ++c) {
                float pen = ((g[0] * (float)CAND[c][0] + g[1] * (float)CAND[c][1]) + g[2] * (float)CAND[c][2]);
                pen = pen - (c >= 7 ? bonus : 0.0f);
                if (c >= 7 && forbid128) pen = INFINITY;
                if (pen < best) { best = pen; bi = c; }
            }
        }
        shape_ids[z] = bi;
    }
}

/* (a2) A2V token norms, wan_video_dit.py:742-752 (residual.norm(dim=-1),
 * batch 0): lane l of a 64-lane group owns the 8-element chunks l, l+64, ...
 * and accumulates x*x with fmaf in element order; lanes are combined with
 * sum_lanes64; then sqrtf and a rounding to the residual dtype. */
void oc_a2v_norms(const void *res, int dtype, int64_t S, int C, void *out, int out_dtype) {
    float acc[64];
    int nch = C / 8;
    for (int64_t s = 0; s < S; ++s) {
        for (int l = 0; l < 64; ++l) acc[l] = 0.0f;
        for (int j = 0; j < nch; ++j) {
            int l = j % 64;
            for (int e = 0; e < 8; ++e) { float x = ld(res, dtype, s * C + j * 8 + e); acc[l] = fmaf(x, x, acc[l]); }
        }
        float n = sqrtf(sum_lanes64(acc, 64));
        if (out_dtype) ((uint16_t *)out)[s] = f2bf(n); else ((float *)out)[s] = n;
    }
}

/* ------------------------------------------------------------------ */
/* (a8) geometry                                                       */
/* ------------------------------------------------------------------ */
/* rearranged position r (0..511) of a zone with shape c -> local flat
 * (lt*64 + lh*8 + lw): _precompute_local_orders, dynamic_block_attention.py:21-63 */
static int local_of_rearr(int c, int r) {
    int bt = CAND[c][0], bh = CAND[c][1], bw = CAND[c][2];
    int bsz = bt * bh * bw, Nh = ZS / bh, Nw = ZS / bw;
    int blk = r / bsz, off = r % bsz;
    int nt = blk / (Nh * Nw), nh = (blk / Nw) % Nh, nw = blk % Nw;
    int it = off / (bh * bw), ih = (off / bw) % bh, iw = off % bw;
    return ((nt * bt + it) * ZS + (nh * bh + ih)) * ZS + (nw * bw + iw);
}
int oc_local_of_rearr(int c, int r) { return local_of_rearr(c, r); }

/* _build_rearrange_index (dynamic_block_attention.py:107-135) */
void oc_rearrange_index(const int64_t *shape_ids, int T, int Hg, int Wg,
                        int64_t *src_idx, int64_t *inv_idx) {
    int ZT = T / ZS, ZH = Hg / ZS, ZW = Wg / ZS, Nz = ZT * ZH * ZW;
    for (int z = 0; z < Nz; ++z) {
        int zt = z / (ZH * ZW), zh = (z / ZW) % ZH, zw = z % ZW;
        for (int r = 0; r < 512; ++r) {
            int lf = local_of_rearr((int)shape_ids[z], r);
            int lt = lf / 64, lh = (lf / 8) % 8, lw = lf % 8;
            int64_t g = ((int64_t)(zt * 8 + lt) * Hg + zh * 8 + lh) * Wg + zw * 8 + lw;
            src_idx[(int64_t)z * 512 + r] = g;
            inv_idx[g] = (int64_t)z * 512 + r;
        }
    }
}

/* _build_block_tile_maps (dynamic_block_attention.py:138-170).  Returns N_b;
 * block_id_of_tile[N_tiles], kblock_tiles[(N_b+1)*2] (sentinel N_tiles),
 * block_offset[Nz].  kblock_tiles may be NULL to query N_b. */
int64_t oc_tile_maps(const int64_t *shape_ids, int Nz, int64_t *block_id_of_tile,
                     int64_t *kblock_tiles, int64_t *block_offset) {
    int64_t nb = 0, Nt = (int64_t)Nz * 8;
    for (int z = 0; z < Nz; ++z) {
        int c = (int)shape_ids[z];
        int tpb = (CAND[c][0] * CAND[c][1] * CAND[c][2]) / TILE;
        if (block_offset) block_offset[z] = nb;
        if (block_id_of_tile)
            for (int t = 0; t < 8; ++t) block_id_of_tile[z * 8 + t] = nb + t / tpb;
        nb += 8 / tpb;
    }
    if (kblock_tiles) {
        for (int64_t i = 0; i < (nb + 1) * 2; ++i) kblock_tiles[i] = Nt;
        for (int z = 0; z < Nz; ++z) {
            int c = (int)shape_ids[z];
            int tpb = (CAND[c][0] * CAND[c][1] * CAND[c][2]) / TILE;
            for (int t = 0; t < 8; ++t) kblock_tiles[block_id_of_tile[z * 8 + t] * 2 + t % tpb] = (int64_t)z * 8 + t;
        }
    }
    return nb;
}

/* ------------------------------------------------------------------ */
/* (a9/a10) block pooling                                               */
/* ------------------------------------------------------------------ */
/* Masked block means of the rearranged q (or k): masked_mean_pooling_compression
 * (bsa_interface.py:177-201) + _logical_block_means
 * (dynamic_block_attention.py:173-188).  Canonical: the block's valid tokens
 * in rearranged order o = 0 .. bsz-1 fall into RPI = 512 / D row groups
 * (o mod RPI); each group is summed in fp32 from +0 in row order, the block
 * sum is ((p_0 + p_1) + ...) + p_{RPI-1}, divided by max(count,1) (the
 * reference evaluates the same quantity as a count-weighted mean of tile
 * means in q's dtype).  x: [B,H,S,D] in THW order (padded grid).
 * out: [B,H,N_b,D] fp32; block_count[N_b]; tile_count[N_tiles]. */
void oc_block_pool(const void *x, int dtype, int B, int H, int64_t S, int D,
                   const uint8_t *valid, const int64_t *shape_ids, int T, int Hg, int Wg,
                   float *out, int32_t *block_count, int32_t *tile_count) {
    int ZT = T / ZS, ZH = Hg / ZS, ZW = Wg / ZS, Nz = ZT * ZH * ZW;
    int64_t *src = (int64_t *)malloc(sizeof(int64_t) * S);
    int64_t *inv = (int64_t *)malloc(sizeof(int64_t) * S);
    oc_rearrange_index(shape_ids, T, Hg, Wg, src, inv);
    int64_t nb = oc_tile_maps(shape_ids, Nz, NULL, NULL, NULL);
    const int rpi = 512 / D;
    float *acc = (float *)malloc(sizeof(float) * D * rpi);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            int64_t blk = 0;
            for (int z = 0; z < Nz; ++z) {
                int c = (int)shape_ids[z];
                int bsz = CAND[c][0] * CAND[c][1] * CAND[c][2];
                for (int j = 0; j < 512 / bsz; ++j, ++blk) {
                    int cnt = 0;
                    for (int d = 0; d < D * rpi; ++d) acc[d] = 0.0f;
                    for (int o = 0; o < bsz; ++o) {
                        int64_t rpos = (int64_t)z * 512 + j * bsz + o;
                        int64_t g = src[rpos];
                        if (valid && !valid[g]) continue;
                        cnt++;
                        const int64_t base = (((int64_t)b * H + h) * S + g) * D;
                        float *part = acc + (o % rpi) * D;
                        for (int d = 0; d < D; ++d) part[d] = part[d] + ld(x, dtype, base + d);
                    }
                    for (int r = 1; r < rpi; ++r)
                        for (int d = 0; d < D; ++d) acc[d] = acc[d] + acc[r * D + d];
                    float den = (float)(cnt > 0 ? cnt : 1);
                    float *o = out + (((int64_t)b * H + h) * nb + blk) * D;
                    for (int d = 0; d < D; ++d) o[d] = acc[d] / den;
                    if (b == 0 && h == 0 && block_count) block_count[blk] = cnt;
                }
            }
        }
    if (tile_count)
        for (int64_t t = 0; t < (int64_t)Nz * 8; ++t) {
            int cnt = 0;
            for (int o = 0; o < TILE; ++o) cnt += valid ? (valid[src[t * TILE + o]] != 0) : 1;
            tile_count[t] = cnt;
        }
    free(acc); free(src); free(inv);
}

/* (a11) cal_score (bsa_interface.py:203-207) with the invalid-key fill of
 * dynamic_block_attention.py:278-279.  Canonical: fp32 fmaf chain over d in
 * increasing order from +0.  scores: [BH, N, N]. */
void oc_block_scores(const float *qc, const float *kc, const int32_t *block_count,
                     int BH, int64_t Nq, int64_t Nk, int D, float *scores) {
    for (int bh = 0; bh < BH; ++bh)
        for (int64_t i = 0; i < Nq; ++i) {
            const float *q = qc + ((int64_t)bh * Nq + i) * D;
            for (int64_t j = 0; j < Nk; ++j) {
                float s;
                if (block_count && block_count[j] == 0) s = -INFINITY;
                else {
                    const float *k = kc + ((int64_t)bh * Nk + j) * D;
                    s = 0.0f;
                    for (int d = 0; d < D; ++d) s = fmaf(q[d], k[d], s);
                }
                scores[((int64_t)bh * Nq + i) * Nk + j] = s;
            }
        }
}

/* ------------------------------------------------------------------ */
/* (a12) selection                                                     */
/* ------------------------------------------------------------------ */
/* smallest X with fl32(X) * 2^-60 >= p: the fixed-point form of the test
 * "cumsum < p" of bsa_interface.py:265/:296 (used by both modes with p) */
uint64_t oc_cdf_threshold(float p) {
    uint64_t lo = 0, hi = (uint64_t)1 << 62;
    while (lo < hi) {
        uint64_t mid = lo + (hi - lo) / 2;
        float f = (float)mid * 8.673617379884035e-19f; /* 2^-60, exact */
        if (f >= p) hi = mid; else lo = mid + 1;
    }
    return lo;
}

typedef struct { float w; int64_t i; } wi_t;
static int cmp_desc(const void *a, const void *b) {
    const wi_t *x = (const wi_t *)a, *y = (const wi_t *)b;
    if (x->w > y->w) return -1;
    if (x->w < y->w) return 1;
    return (x->i < y->i) ? -1 : (x->i > y->i);
}
static int cmp_i64(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return (x > y) - (x < y);
}

/* Per-row block selection.
 *   mode 0 (top-k, get_select_indices_topk_from_score, bsa_interface.py:235-248):
 *     the k largest scores;
 *   mode 1 (cdf, get_select_indices_cdf_from_score, :257-275) and mode 2
 *     (hybrid, get_select_indices_cdf_topk_from_score, :284-304): softmax
 *     weights w of score*scale, descending order, n = clamp(#(cdf<p among the
 *     first ub)+1, lo, N), the first min(n, ub) blocks.
 * Canonical arithmetic: x = s*scale (fp32), e = canon_exp(x - max x),
 * sum = fl32(sum_j floor(e_j 2^40)) 2^-40, w = e / sum,
 * cdf_k < p  <=>  sum_{j<=k} floor(w_(j) 2^60) < thr (oc_cdf_threshold(p)).
 * Order: value descending, index ascending on ties.
 * Output: sel[row*cap ...] ascending block ids, nsel[row]. */
void oc_select(const float *scores, int64_t rows, int64_t N, int mode, int64_t k_lo,
               int64_t ub, float scale, uint64_t thr, int64_t cap,
               int64_t *sel, int32_t *nsel) {
    wi_t *a = (wi_t *)malloc(sizeof(wi_t) * N);
    float *e = (float *)malloc(sizeof(float) * N);
    for (int64_t row = 0; row < rows; ++row) {
        const float *s = scores + row * N;
        int64_t eff;
        if (mode == 0) {
            for (int64_t j = 0; j < N; ++j) { a[j].w = s[j]; a[j].i = j; }
            qsort(a, N, sizeof(wi_t), cmp_desc);
            eff = k_lo < N ? k_lo : N;
        } else {
            float m = -INFINITY;
            for (int64_t j = 0; j < N; ++j) { float x = s[j] * scale; e[j] = x; m = fmax_(m, x); }
            if (m == -INFINITY) { nsel[row] = 0; continue; }
            uint64_t E = 0;
            for (int64_t j = 0; j < N; ++j) { e[j] = canon_exp(e[j] - m); E += fixp(e[j], 40); }
            float sum = (float)E * 9.094947017729282e-13f; /* 2^-40 */
            for (int64_t j = 0; j < N; ++j) { a[j].w = e[j] / sum; a[j].i = j; }
            qsort(a, N, sizeof(wi_t), cmp_desc);
            int64_t c = ub;
            uint64_t P = 0;
            for (int64_t k = 0; k < ub; ++k) {
                P += fixp(a[k].w, 60);
                if (P >= thr) { c = k; break; }
            }
            int64_t n = c + 1;
            if (n < k_lo) n = k_lo;
            if (n > N) n = N;
            eff = n < ub ? n : ub;
        }
        int64_t *o = sel + row * cap;
        for (int64_t k = 0; k < eff; ++k) o[k] = a[k].i;
        qsort(o, eff, sizeof(int64_t), cmp_i64);
        nsel[row] = (int32_t)eff;
    }
    free(a); free(e);
}

/* (a13) block -> tile expansion (dynamic_block_attention.py:297-319):
 * selected blocks (ascending) -> their 1-2 tiles, tiles with zero valid
 * tokens dropped when tile_count is given.  Output per block row. */
void oc_expand_tiles(const int64_t *sel, const int32_t *nsel, int64_t rows, int64_t cap,
                     const int64_t *kblock_tiles, int64_t Nt, const int32_t *tile_count,
                     int64_t tcap, int32_t *tiles, int32_t *ntiles) {
    for (int64_t row = 0; row < rows; ++row) {
        int32_t n = 0;
        for (int k = 0; k < nsel[row]; ++k) {
            int64_t b = sel[row * cap + k];
            for (int t = 0; t < 2; ++t) {
                int64_t tile = kblock_tiles[b * 2 + t];
                if (tile >= Nt) continue;
                if (tile_count && tile_count[tile] == 0) continue;
                tiles[row * tcap + n++] = (int32_t)tile;
            }
        }
        ntiles[row] = n;
    }
}

/* Transposed lists for the dK/dV pass: create_indices_k_from_indices_q_varlen
 * (bsa_interface.py:147-161) as a list transpose.  Input: per q tile
 * (row = bh*Nt + t) a list at qstart[row], length qlen[row].  Output: per k
 * tile the ascending q tiles at row*Nt, klen[row]. */
/* rows bh*Ntq + t list key tiles < Ntk; output rows bh*Ntk + k, stride Ntq */
void oc_transpose_lists(const int64_t *qstart, const int32_t *qlen, const int32_t *qcols,
                        int BH, int64_t Ntq, int64_t Ntk, int32_t *kcols, int32_t *klen) {
    for (int64_t i = 0; i < (int64_t)BH * Ntk; ++i) klen[i] = 0;
    for (int bh = 0; bh < BH; ++bh)
        for (int64_t t = 0; t < Ntq; ++t) {
            int64_t row = (int64_t)bh * Ntq + t;
            for (int i = 0; i < qlen[row]; ++i) {
                int64_t kr = (int64_t)bh * Ntk + qcols[qstart[row] + i];
                kcols[kr * Ntq + klen[kr]++] = (int32_t)t;
            }
        }
}
