/*
 * prism_bsa.h -- C-ABI of libprism_bsa.so, the MI355X (gfx950) implementation
 * of Prism's dynamic block-sparse attention path.
 *
 * Plain pointers and sizes only.  Every pointer argument is a device pointer
 * (HIP) unless stated otherwise; every call is asynchronous on `stream` and
 * returns 0 on success, 1 for an invalid argument, 2 for a HIP launch error;
 * prism_last_error() then holds the message (per host thread).
 *
 * Citations name the reference function (file:line under
 * hymm/models/modules/block_sparse_attention/ unless another path is given)
 * whose behaviour the entry point provides.  The reference is Python/Triton;
 * its host layer reaches these functions through the torch.ops.prism
 * operators (prism_amd/csrc/torch_ops.cpp) or through ctypes.
 *
 * dtype codes: PRISM_F32 = 0, PRISM_BF16 = 1.
 * Layouts: "THW order" = the reference's flattened (t, h, w) token order of a
 * padded grid T x Hg x Wg (all multiples of 8); "tile order" = the per-zone
 * anisotropic rearrangement of _build_rearrange_index
 * (dynamic_block_attention.py:107-135): zone z owns positions
 * [512 z, 512 z + 512), tile t = position / 64.
 */
#ifndef PRISM_BSA_H_
#define PRISM_BSA_H_

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PRISM_F32 0
#define PRISM_BF16 1

/* Message of the last failed call on this host thread ("" if none). */
const char* prism_last_error(void);
/* ABI version of this library. */
int prism_abi_version(void);

/* ------------------------------------------------------------------ zone statistics */

/* Input grid and zone grid.  Entry points of the dynamic path take the zone
 * grid T x Hg x Wg (multiples of 8) and the input grid Tin x Hin x Win inside
 * it (the caller's unpadded video; Tin = T, Hin = Hg, Win = Wg when the input
 * is already padded).  Inputs hold S = Tin*Hin*Win tokens per head; zone-grid
 * positions outside the input grid read as zero, invalid tokens: this is the
 * zero padding plus valid mask of wan_video_dit.py:342-400 without the padded
 * copies.  Tile-order rows always cover the zone grid (T*Hg*Wg per head). */

/* compute_zone_aggregates (dynamic_block_shape.py:68-129) applied to the
 * batch-0 head mean of V (dynamic_block_attention.py:236).
 * v: [B,H,S,D] THW order of the input grid (only batch 0 is read), valid: [S]
 * uint8 or NULL.  packed: [Nz, 25*D] fp32 = channel(D) | frame means(8D) |
 * h means(8D) | w means(8D); axis_valid: [Nz, 24] uint8 (t, h, w "has a
 * valid token" flags). */
int prism_zone_stats(const void* v, int dtype, int H, int64_t S, int D, const uint8_t* valid,
                     int T, int Hg, int Wg, int Tin, int Hin, int Win, float* packed, uint8_t* axis_valid,
                     hipStream_t stream);

/* compute_audio_directional (dynamic_block_shape.py:189-245) before the
 * max-normalisation of a_bar.  norms: [S] THW order of the input grid.
 * abar: [Nz]; vhat: [Nz,3]. */
int prism_audio_zone_stats(const void* norms, int dtype, const uint8_t* valid, int T, int Hg, int Wg, int Tin,
                           int Hin, int Win, float* abar, float* vhat, hipStream_t stream);

/* Per-zone part of compute_effective_gradient (dynamic_block_shape.py:248-289):
 * rho_raw = spatial + temporal variance, aniso = axis variances / their sum. */
int prism_zone_gradient(const float* packed, const uint8_t* axis_valid, int Nz, int D,
                        float* rho_raw, float* aniso, hipStream_t stream);

/* Zone normalisation, g = aniso + lambda_a * a_bar * v_hat (clamped >= 1e-4)
 * (dynamic_block_shape.py:280, :297-300) and the shape decision of
 * select_shapes_ivpq (method 0, :303-327) or select_shapes_penalty (method 1,
 * :330-355).  abar/vhat NULL = no audio.  Outputs g [Nz,3], rho [Nz],
 * shape_ids [Nz] int64 (index into the 13-entry candidate table :6-27). */
int prism_zone_shapes(const float* rho_raw, const float* aniso, const float* abar, const float* vhat,
                      int Nz, int method, float lambda_a, float tau_128, float lambda_128,
                      float* g, float* rho, int64_t* shape_ids, hipStream_t stream);

/* select_shapes_ivpq (method 0, dynamic_block_shape.py:303-327) /
 * select_shapes_penalty (method 1, :330-355) on given g [Nz,3] and rho [Nz]. */
int prism_assign_shapes(const float* g, const float* rho, int Nz, int method, float tau_128, float lambda_128,
                        int64_t* shape_ids, hipStream_t stream);

/* Per-token L2 norm of the A->V bridge residual, batch 0
 * (hymm/models/modules/wan_video_dit.py:742-752).  res: [S, C]; out: [S]. */
int prism_a2v_norms(const void* res, int dtype, int64_t S, int C, void* out, int out_dtype,
                    hipStream_t stream);

/* The a2v bridge's output projection with the residual norms of
 * wan_video_dit.py:742-752 fused into its epilogue: y = x W^T + b
 * (nn.Linear, ConditionalCrossAttention.o, interactionv2.py:225, :348; the
 * a2v_bridge_residual of mova.py:127-137) and norms[m] = ||y[m, :]||_2 of the
 * stored bf16 values.  x: [M, K] bf16, w: [N, K] bf16, bias: [N] bf16 or NULL;
 * y: [M, N] bf16; norms: [M] of norms_dtype; partial: workspace of
 * M * (N / 256) floats (per-row sums of squares of each 256-column tile,
 * added in tile order).  N must be a multiple of 256, K of 64; x and w each
 * below 4 GiB. */
int prism_linear_rownorm(const void* x, const void* w, const void* bias, int64_t M, int N, int K, void* y,
                         void* norms, int norms_dtype, float* partial, hipStream_t stream);

/* ------------------------------------------------------------------ geometry */

/* _build_block_tile_maps (dynamic_block_attention.py:138-170) in CSR form.
 * block_offset: [Nz+1] (block_offset[Nz] = N_b), block_id_of_tile: [Nz*8],
 * block_first_tile: [Nz*8+1] (block b owns tiles [first[b], first[b+1]);
 * entry N_b is the sentinel N_tiles, as kblock_tiles row N_b).
 * A shape id outside 0..12 sets block_offset[Nz] = -1 (the other outputs are
 * then meaningless): the caller checks it before passing the ids to any other
 * entry point, which all take valid ids (the reference raises an IndexError
 * from local_orders[shape_ids] in the same case, dynamic_block_attention.py:130). */
int prism_zone_layout(const int64_t* shape_ids, int Nz, int32_t* block_offset, int32_t* block_id_of_tile,
                      int32_t* block_first_tile, hipStream_t stream);

/* _build_rearrange_index (dynamic_block_attention.py:107-135): src_idx[S]
 * (tile position -> THW index) and inv_idx[S]. */
int prism_rearrange_index(const int64_t* shape_ids, int T, int Hg, int Wg, int64_t* src_idx, int64_t* inv_idx,
                          hipStream_t stream);

/* x.index_select(2, src_idx) (dynamic_block_attention.py:250-253) fused with
 * masked_mean_pooling_compression + _logical_block_means
 * (bsa_interface.py:177-201, dynamic_block_attention.py:173-188).
 * x: [B,H,S,D] THW order of the input grid.  With Sz = T*Hg*Wg zone-grid
 * rows, optional outputs (NULL to skip):
 *   out_rows [B,H,Sz,D] bf16 tile order; block_mean [B,H,N_b,D] fp32;
 *   block_count [N_b], tile_count [Sz/64] int32; valid_re [Sz] uint8 tile order;
 *   rowdot [B,H,Sz] fp32 = rowsum(x_re * dot_with) with dot_with [B,H,Sz,D] bf16
 *   tile order (the delta of common.py:110-127 when x = dO, dot_with = O). */
int prism_gather_pool(const void* x, int dtype, int B, int H, int64_t S, int D, const uint8_t* valid,
                      const int64_t* shape_ids, const int32_t* block_offset, int T, int Hg, int Wg, int Tin,
                      int Hin, int Win, int64_t N_b, void* out_rows, float* block_mean, int32_t* block_count,
                      int32_t* tile_count, uint8_t* valid_re, const void* dot_with, float* rowdot,
                      hipStream_t stream);

/* o_re.index_select(2, inv_idx) (dynamic_block_attention.py:329) plus the
 * unpadding of wan_video_dit.py:429-431: tile-order bf16 rows [B,H,T*Hg*Wg,D]
 * -> rows of out_dtype [B,H,S,D] in THW order of the input grid. */
int prism_scatter_rows(const void* in_rows, int B, int H, int64_t S, int D, const int64_t* shape_ids, int T,
                       int Hg, int Wg, int Tin, int Hin, int Win, void* out, int out_dtype, hipStream_t stream);

/* Uniform chunk layout (the fixed-shape BSA of flash_attn_bsa_3d and
 * flash_attn_bsa_cross, bsa_interface.py:1123-1176, 1276-1392):
 * rearrange_THW_to_3d_block (bsa_interface.py:1105-1109) fused with the
 * padding of the grid to a multiple of the chunk (:1263-1273, :1318-1367) and
 * with (masked_)mean_pooling_compression (:164-201).
 * x: [B,H,T*Hg*Wg,D] THW order over the input grid; the padded grid Tp x Hp x Wp
 * (multiples of ct x ch x cw, chunk of 64 or 128 tokens) is cut into chunks
 * n = (nt*Nh + nh)*Nw + nw, each owning rows [n*csz, (n+1)*csz) in
 * (it*ch + ih)*cw + iw order; tokens outside the input grid and rows in
 * [Tp*Hp*Wp, S_out) are padding (zero rows, invalid).  S_out: rows per head of
 * the outputs, a multiple of 128.  valid: [T*Hg*Wg] uint8 or NULL.  Outputs as
 * prism_gather_pool with N_b = Tp*Hp*Wp / csz blocks (means over the valid
 * tokens of each chunk, count clamped to 1). */
int prism_chunk_gather_pool(const void* x, int dtype, int B, int H, int D, const uint8_t* valid, int T, int Hg,
                            int Wg, int Tp, int Hp, int Wp, int ct, int ch, int cw, int64_t S_out, void* out_rows,
                            float* block_mean, int32_t* block_count, int32_t* tile_count, uint8_t* valid_re,
                            const void* dot_with, float* rowdot, hipStream_t stream);

/* rearrange_3d_block_to_THW (bsa_interface.py:1111-1115) plus the unpadding
 * slice (:1372-1380): tile-order bf16 rows [B,H,S_out,D] of the chunk layout
 * above -> [B,H,T*Hg*Wg,D] THW rows of out_dtype (padding rows dropped). */
int prism_chunk_scatter_rows(const void* in_rows, int B, int H, int D, int T, int Hg, int Wg, int Tp, int Hp, int Wp,
                             int ct, int ch, int cw, int64_t S_out, void* out, int out_dtype, hipStream_t stream);

/* ------------------------------------------------------------------ selection */

/* cal_score (bsa_interface.py:203-207) in fp32 with the invalid-key fill of
 * dynamic_block_attention.py:276-279 (block_count[j] == 0 -> -inf; NULL = none,
 * as in the uniform path, bsa_interface.py:611-631).
 * qc: [BH, Nq, D], kc: [BH, Nk, D] fp32; scores: [BH, Nq, Nk] fp32. */
int prism_block_scores(const float* qc, const float* kc, const int32_t* block_count, int BH, int64_t Nq, int64_t Nk,
                       int D, float* scores, hipStream_t stream);

/* Per-row block selection fused with the block -> tile expansion:
 *   mode 0: get_select_indices_topk_from_score (bsa_interface.py:235-248), k = k_lo;
 *   mode 1: get_select_indices_cdf_from_score (:257-275), k_lo = 1;
 *   mode 2: get_select_indices_cdf_topk_from_score (:284-304), k_lo = k_t;
 * ub as the reference derives it; thr = cumulative threshold in 2^-60 fixed
 * point (smallest X with fl32(X) 2^-60 >= p).  Expansion and padded-tile
 * filtering: dynamic_block_attention.py:297-319 (tile_count NULL = keep all).
 * tiles: [rows, tcap] ascending tile ids (tcap >= the tiles of the widest
 * selection: tiles per block x selected blocks), ntiles: [rows];
 * sel_blocks: [rows, bcap] ascending block ids (NULL to skip), nsel: [rows].
 * 1 <= N <= 2^30 (rows of more than 16384 blocks take a slower pass-by-pass
 * kernel with the same results). */
int prism_select_tiles(const float* scores, int64_t rows, int64_t N, int mode, int64_t k_lo, int64_t ub,
                       float scale, uint64_t thr, const int32_t* block_first_tile, const int32_t* tile_count,
                       int64_t tcap, int32_t* tiles, int32_t* ntiles, int32_t* sel_blocks, int64_t bcap,
                       int32_t* nsel, hipStream_t stream);

/* q tile rows share their q block's list (tile_sel.index_select(2,
 * block_id_of_tile), dynamic_block_attention.py:315-318):
 * qstart[bh*Nt + t] = (bh*N_b + block_id_of_tile[t]) * tcap, qlen likewise.
 * q_tile_count [Nt] (or NULL): tiles with no valid query token get qlen 0
 * (their rows are padding that the caller slices away, wan_video_dit.py:429-431;
 * the reference still computes them). */
int prism_tile_rows(const int32_t* ntiles, const int32_t* block_id_of_tile, const int32_t* q_tile_count, int BH,
                    int64_t Nt, int64_t N_b, int64_t tcap, int64_t* qstart, int32_t* qlen, hipStream_t stream);

/* create_indices_k_from_indices_q_varlen (bsa_interface.py:147-161) as a
 * bitmap transpose.  Input rows bh*Ntq + t list key tiles < Ntk.
 * bitmap: workspace of BH*Ntk*ceil(Ntq/32) uint32.  Output per key tile
 * (row bh*Ntk + k): kstart = row*kcap (kcap >= Ntq), klen, kcols ascending
 * query tiles. */
int prism_transpose_lists(const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, int BH, int64_t Ntq,
                          int64_t Ntk, uint32_t* bitmap, int64_t kcap, int64_t* kstart, int32_t* klen,
                          int32_t* kcols, hipStream_t stream);

/* prism_transpose_lists without the bitmap argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * bitmap lives in a library-owned device workspace of 2^21 uint32 words (8 MiB
 * per GPU, held until the process ends); heads are processed in batches that
 * fit it, and one head's bitmap (Ntk * ceil(Ntq / 32) words) must fit
 * (else PRISM_EINVAL).  The call allocates nothing (its first call on a GPU
 * looks up the workspace's address and creates one event there).  Every call
 * on a GPU uses that GPU's one workspace; the library orders the calls made
 * outside graph capture, whatever their streams or threads: each call's
 * stream waits for the event the previous call recorded after its kernels.
 * Calls captured into a graph neither wait nor record, so a graph replay
 * that overlaps another call on the same GPU races with it.  Outputs as
 * prism_transpose_lists. */
int prism_transpose_lists_noalloc(const int64_t* qstart, const int32_t* qlen, const int32_t* qcols, int BH,
                                  int64_t Ntq, int64_t Ntk, int64_t kcap, int64_t* kstart, int32_t* klen,
                                  int32_t* kcols, hipStream_t stream);

/* ------------------------------------------------------------------ attention */

/* Work lists of the paired-tile attention kernels.  Every attention kernel runs
 * one workgroup per pair of tiles (2p, 2p+1) and walks the sorted union of the
 * two tiles' lists.  For pair p (rows 2p, 2p+1 of a per-row list, or the
 * rows pairmap[2p], pairmap[2p+1] of the pair's head when pairmap is given; rows =
 * BH*row_tiles, row_tiles even; entries are tiles < col_tiles):
 * ucols[ustart[p] .. + ulen[p]) ascending entries
 * tile << 3 | partial << 2 | in_row_2p+1 << 1 | in_row_2p, where partial =
 * (tile_masks != NULL && tile_masks[tile] != all ones), tile_masks from
 * prism_tile_masks.  ustart[p] = p * ucap, ucap >= col_tiles.  Used on the per-query-tile key lists (forward, dQ; the
 * reference's block_indices, bsa_interface.py:328-385) and on the per-key-tile
 * query lists of prism_transpose_lists (dK/dV; bsa_interface.py:437-447).
 * No counterpart routine in the reference: its kernels take one list per tile. */
int prism_pair_union(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, const int32_t* pairmap, const uint64_t* tile_masks, int64_t ucap,
                     int64_t* ustart, int32_t* ulen, int32_t* ucols, hipStream_t stream);

/* Quad unions for prism_bsa_fwd_quad and prism_bsa_bwd_dq_quad (no
 * counterpart in the reference; its forward and dQ kernels walk one query
 * tile's list): rows of four tiles, quad q of a
 * head being pairmap[4 q + k], k < 4 (four consecutive entries of a
 * prism_pair_tiles map: two pairs of a group), or rows 4 q + k.  Entries
 * tile << 5 | partial << 4 | member bits (bit k: row k lists the tile); rows %
 * 4 == 0, row_tiles % 4 == 0; otherwise as prism_pair_union. */
int prism_quad_union(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, const int32_t* pairmap, const uint64_t* tile_masks, int64_t ucap,
                     int64_t* ustart, int32_t* ulen, int32_t* ucols, hipStream_t stream);

/* Compact CSR of per-row lists (the select and list-transpose output form of
 * the drop-in operators: offsets int32 [rows + 1], entries int32 [nnz]) from the
 * (start, len, cols) lists the other entry points produce, whose rows sit
 * anywhere in cols (prism_select_tiles + prism_tile_rows: bsa_interface.py
 * :235-304 with dynamic_block_attention.py:297-319; prism_transpose_lists:
 * create_indices_k_from_indices_q_varlen, bsa_interface.py:147-161;
 * prism_pair_union).  Two calls so that the caller can allocate the entries:
 * prism_lists_csr_offsets writes offsets[r] = sum of len[0..r) (negative
 * lengths count as 0) and the int64 total to *total (one int64 on the
 * device; a total past 2^31 - 1 does not fit the offsets); then
 * prism_lists_csr_fill copies row r's len[r] entries from cols + start[r] to
 * out_cols + offsets[r].  The attention kernels take the result as lists
 * with start = offsets[r], len = offsets[r + 1] - offsets[r]; they reject a
 * null entry pointer, so a caller allocates at least one entry even when the
 * total is 0 (the torch operators do). */
int prism_lists_csr_offsets(const int32_t* len, int64_t rows, int32_t* offsets, int64_t* total,
                            hipStream_t stream);
int prism_lists_csr_fill(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows,
                         const int32_t* offsets, int32_t* out_cols, hipStream_t stream);

/* Pairing of the tiles that the paired kernels process together: inside each
 * group of 8 consecutive tiles of a head (fewer at a head's end), the perfect
 * matching with the largest summed list overlap |A n B| over its pairs (ties:
 * the lowest matching index, where matching m pairs the first free tile with
 * the (m mod (free - 1))-th other free tile, m /= (free - 1), and so on).
 * Lists as for prism_pair_union.  pairmap [rows]: pair p of a head is the
 * tiles pairmap[2p], pairmap[2p+1] (indices inside the head), listed by
 * their first tile.  Pairing changes no result: every tile still walks its
 * own list in ascending order.  No counterpart in the reference (its kernels
 * take one tile per program). */
int prism_pair_tiles(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t row_tiles,
                     int64_t col_tiles, int32_t* pairmap, hipStream_t stream);

/* Launch order of an attention kernel: order[id] = the pair (index into the
 * prism_pair_union arrays, n = BH * pairs per head) that work id processes
 * (workgroup id without a work counter, work-queue position with one).  Ids [0, n - tail) keep the XCD group mapping the kernel uses
 * without an order (G = 64 for prism_bsa_fwd and prism_bsa_bwd_dq, 32 for
 * prism_bsa_bwd_dkdv); the last tail ids (tail <= 16384) take the pairs that
 * mapping gives them, longest union list (ulen) first, so the launch does not
 * end waiting for long workgroups started last.  Changes no result.  No
 * counterpart in the reference (its launch order is the hardware's). */
int prism_pair_order(const int32_t* ulen, int64_t n, int G, int64_t tail, int32_t* order, hipStream_t stream);

/* Key validity per 64-token tile (the reference's kv_valid_mask,
 * bsa_interface.py:328-385, flash_attn_bsa_varlen_mask.py:263-295) packed as
 * masks[t] bit j = valid[64 t + j] != 0.  valid: [Nt*64] uint8 tile order. */
int prism_tile_masks(const uint8_t* valid, int64_t Nt, uint64_t* masks, hipStream_t stream);

/* Base-2 row maximum of the backward (bsa_interface.py:405-416: M = lse / ln 2):
 * m2[i] = lse[i] * log2(e), with lse = -inf (a row that saw no valid key)
 * mapped to +inf so that its probabilities are exactly 0. */
int prism_lse_to_m2(const float* lse, int64_t n, float* m2, hipStream_t stream);

/* Work counters of the attention kernels (work_counter argument): 8 int32 of
 * device memory (one per XCD), which the call zeroes on its stream before the
 * launch.  With them, the launch is persistent: as many workgroups as the GPU
 * holds at once, each taking pairs of `order` from atomic work queues until
 * none is left: first the positions b = 8 k + x of its own XCD x (the pairs a
 * one-workgroup-per-pair launch would run there, since the hardware hands
 * workgroup ids to the XCDs round-robin), then the remaining positions of
 * slower XCDs.  The work spreads over the XCDs as they free up.  Calls that
 * may overlap need counters of their own.  NULL: one workgroup per pair.
 * Without an `order`, position b runs the pair the same fixed XCD grouping
 * gives workgroup id b (runs of neighbouring pairs per XCD) in both launch
 * forms.  The results are bit-identical either way.  No counterpart in the reference (a
 * Triton launch of one program per tile). */

/* attn_fwd_bsa_varlen_triton (bsa_interface.py:328-385) with
 * _attn_fwd_bsa_varlen_align (flash_attn_bsa_varlen_mask.py:191-319), on
 * 64-token tiles (larger chunks are lists of their tiles).  Sq, Sk (query and
 * key rows per head; equal for self-attention) must be multiples of 128
 * (tiles are processed in pairs).  q: [BH,Sq,D], k, v: [BH,Sk,D] bf16 tile
 * order; ustart/ulen/ucols: prism_pair_union of the per-query-tile key lists
 * with the same tile_masks (prism_tile_masks of the key validity, or NULL when
 * no key is padded) and the same pairmap (prism_pair_tiles of those lists, or
 * NULL for tiles 2p, 2p+1).  order: prism_pair_order of ulen with G = 64, or
 * NULL.  o: [BH,Sq,D] bf16; lse: [BH,Sq] fp32 natural log (-inf for rows
 * without a valid key; their o is 0). */
int prism_bsa_fwd(const void* q, const void* k, const void* v, int BH, int64_t Sq, int64_t Sk, int D,
                  const uint64_t* tile_masks, const int64_t* ustart, const int32_t* ulen, const int32_t* ucols,
                  const int32_t* pairmap, const int32_t* order, float sm_scale, void* o, float* lse,
                  int32_t* work_counter, hipStream_t stream);

/* prism_bsa_fwd over quad unions (prism_quad_union): one 8-wave workgroup per
 * four query tiles, so each staged K / V tile serves up to 256 query rows;
 * quadmap: the pairmap the quad unions were built with (or NULL).  Same
 * outputs, bit for bit, as prism_bsa_fwd over the pair unions of the same
 * lists (every query row walks its own list in the same order with the same
 * arithmetic).  Sq a multiple of 256; order (or NULL) a permutation of the
 * BH * Sq/256 quads; work_counter as for prism_bsa_fwd. */
int prism_bsa_fwd_quad(const void* q, const void* k, const void* v, int BH, int64_t Sq, int64_t Sk, int D,
                       const uint64_t* tile_masks, const int64_t* ustart, const int32_t* ulen, const int32_t* ucols,
                       const int32_t* quadmap, const int32_t* order, float sm_scale, void* o, float* lse,
                       int32_t* work_counter, hipStream_t stream);

/* _attn_bwd_preprocess (common.py:110-127): delta[r] = sum_d o[r][d] * do[r][d]
 * over rows of bf16 [rows, D] tensors; fp32 out. */
int prism_bwd_preprocess(const void* o, const void* do_, int64_t rows, int D, float* delta, hipStream_t stream);

/* dK, dV of attn_bwd_bsa_varlen_triton (bsa_interface.py:387-487;
 * _attn_bwd_dkdv_bsa_varlen_wrapper, flash_attn_bsa_varlen_mask.py:562-704).
 * q, do_: [BH,Sq,D], k, v: [BH,Sk,D] bf16 tile order; m2 [BH,Sq] from
 * prism_lse_to_m2; delta [BH,Sq] from prism_gather_pool or
 * prism_bwd_preprocess; kv_valid: [Sk] uint8 tile order or NULL;
 * ustart/ulen/ucols: prism_pair_union of the per-key-tile query lists of
 * prism_transpose_lists (tile_masks NULL), built with the key-tile pairing
 * pairmap (prism_pair_tiles of those lists, or NULL for tiles 2p, 2p+1);
 * order: prism_pair_order of ulen with G = 32, or NULL.
 * dk, dv: [BH,Sk,D] bf16. */
int prism_bsa_bwd_dkdv(const void* q, const void* k, const void* v, const void* do_, const float* m2,
                       const float* delta, int BH, int64_t Sq, int64_t Sk, int D, const uint8_t* kv_valid,
                       const int64_t* ustart, const int32_t* ulen, const int32_t* ucols, const int32_t* pairmap,
                       const int32_t* order, float sm_scale, void* dk, void* dv, int32_t* work_counter,
                       hipStream_t stream);

/* dQ of attn_bwd_bsa_varlen_triton (bsa_interface.py:489-523;
 * _attn_bwd_dq_bsa_varlen_align_wrapper, flash_attn_bsa_varlen_mask.py:879-1014).
 * Shapes as for prism_bsa_bwd_dkdv; lists, tile_masks and order as for
 * prism_bsa_fwd; dq: [BH,Sq,D] bf16. */
int prism_bsa_bwd_dq(const void* q, const void* k, const void* v, const void* do_, const float* m2, const float* delta,
                     int BH, int64_t Sq, int64_t Sk, int D, const uint64_t* tile_masks, const int64_t* ustart,
                     const int32_t* ulen, const int32_t* ucols, const int32_t* pairmap, const int32_t* order,
                     float sm_scale, void* dq, int32_t* work_counter, hipStream_t stream);

/* prism_bsa_bwd_dq over quad unions (prism_quad_union of the per-query-tile
 * key lists; no counterpart in the reference, whose dQ kernel walks one query
 * tile's list): one 8-wave workgroup per four query tiles, so each staged K /
 * V tile serves up to 256 query rows.  quadmap: the pairmap the quad unions
 * were built with (or NULL).  The same dq, bit for bit, as prism_bsa_bwd_dq
 * over the pair unions of the same lists.  Sq a multiple of 256; order (or
 * NULL) a permutation of the BH * Sq/256 quads; work_counter as for
 * prism_bsa_bwd_dq. */
int prism_bsa_bwd_dq_quad(const void* q, const void* k, const void* v, const void* do_, const float* m2,
                          const float* delta, int BH, int64_t Sq, int64_t Sk, int D, const uint64_t* tile_masks,
                          const int64_t* ustart, const int32_t* ulen, const int32_t* ucols, const int32_t* quadmap,
                          const int32_t* order, float sm_scale, void* dq, int32_t* work_counter, hipStream_t stream);

/* ------------------------------------------------------------------ measured ceilings */

/* Measurement aids of the benchmark's roofline (no counterpart in the
 * reference).  prism_mfma_peak: two 4-wave workgroups per CU, each wave
 * running iters x 4 independent v_mfma_f32_32x32x16_bf16 on register operands
 * (no memory traffic): the bf16 MFMA rate the chip sustains at full load.
 * *flops (host) = the launch's FLOPs; sink: >= 512 x CUs floats; clocks[0],
 * clocks[1] (device) = shader-clock and 100 MHz constant-clock ticks of one
 * wave over the launch (their ratio x 100 MHz is the engine clock it ran at).
 * prism_copy_peak: dst = src over `bytes` (a multiple of 16) with 16-byte
 * lanes, the HBM rate of a read + write stream. */
int prism_mfma_peak(int64_t iters, float* sink, int64_t sink_len, uint64_t* clocks, int64_t* flops,
                    hipStream_t stream);
int prism_copy_peak(const void* src, void* dst, int64_t bytes, hipStream_t stream);
/* prism_tile_stream_peak: the attention kernels' tile stream without their
 * math.  Two workgroups per CU each copy `steps` stages of two 16 KB tiles of
 * src (`bytes`, a multiple of 16384; tiles drawn by a per-workgroup LCG) into
 * LDS with global_load_lds_dwordx4, one stage in flight, a barrier per stage.
 * *moved (host) = the bytes copied; sink: >= 2 x CUs words (the first word of
 * each workgroup's last stage).  Over a buffer that the Infinity Cache holds
 * but the L2s do not (~190 MB), the rate the forward's K/V stream can reach. */
int prism_tile_stream_peak(const void* src, int64_t bytes, int64_t steps, uint32_t* sink, int64_t sink_len,
                           int64_t* moved, hipStream_t stream);

/* ------------------------------------------------------------------ list checks (debug) */

/* Work-list validation on HOST memory (no counterpart in the reference, whose
 * Triton kernels read the lists unchecked).  rows lists (start[r], len[r]) into
 * cols[0, ncols): each len in [0, ntiles], each row inside cols, entries
 * strictly ascending in [0, ntiles); with unions == 1 the entries are
 * prism_pair_union entries (tile = entry >> 3, two member bits, partial bit
 * 4), with unions == 2 prism_quad_union entries (tile = entry >> 5, four
 * member bits, partial bit 16): flagged for at least one tile of the pair or
 * quad, and flagged partial exactly where tile_masks[tile] is not all ones
 * (never when tile_masks is NULL).  Returns 1 (invalid argument) naming the
 * first violation.  With PRISM_DEBUG=1 in the environment, prism_bsa_fwd,
 * prism_bsa_fwd_quad, prism_bsa_bwd_dkdv, prism_bsa_bwd_dq,
 * prism_bsa_bwd_dq_quad, prism_pair_union and prism_quad_union run these checks on host copies of their lists
 * (synchronising their stream) before launching anything, and return 1
 * without a launch when one fails. */
int prism_check_lists(const int64_t* start, const int32_t* len, const int32_t* cols, int64_t rows, int64_t ncols,
                      int64_t ntiles, int unions, const uint64_t* tile_masks);

/* Launch maps on HOST memory: pairmap [heads, tiles_per_head] (if not NULL)
 * a permutation of each head's tiles (prism_pair_tiles), order [n_order] (if
 * not NULL) a permutation of [0, n_order) (prism_pair_order).  No counterpart
 * in the reference. */
int prism_check_launch_maps(const int32_t* pairmap, int64_t heads, int64_t tiles_per_head, const int32_t* order,
                            int64_t n_order);

#ifdef __cplusplus
}
#endif

#endif /* PRISM_BSA_H_ */
