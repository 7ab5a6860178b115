"""GPU parity of the uniform (fixed chunk shape) BSA path against the CPU oracle:
flash_attn_bsa_3d (bsa_interface.py:1123-1176), flash_attn_bsa_cross
(:1276-1392) and flash_attn_bsa (:597-683).

Bit-exact: chunk rearrangement with padding, chunk means, counts, validity,
the inverse scatter, rectangular scores, list transpose and pair unions, and
the per-query-tile key lists of the whole selection.  Tolerance (bf16 MFMA vs
the float64 oracle on the oracle's own lists): O, dQ, dK, dV with max-abs
2e-2 and mean-abs 2e-3.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import bf16
from tests.test_gpu_parity import DEV, _tol, bits_equal, dev, host, say

pytestmark = pytest.mark.gpu


def _f(x_bits_or_f32):
    return O.bf16_bits_to_f32(x_bits_or_f32) if x_bits_or_f32.dtype == np.uint16 else x_bits_or_f32


# ------------------------------------------------------------------ layout kernels
LAYOUTS = [
    # (name, grid, chunk, D, dtype, masked)
    ("444_f32_d64", (8, 8, 8), (4, 4, 4), 64, "f32", False),
    ("448_bf16_pad_mask", (5, 9, 12), (4, 4, 8), 128, "bf16", True),
    ("1d_200", (1, 1, 200), (1, 1, 64), 128, "bf16", False),
    ("1d_130_rowpad", (1, 1, 130), (1, 1, 64), 64, "f32", True),
]


@pytest.mark.parametrize("lcase", LAYOUTS, ids=[c[0] for c in LAYOUTS])
def test_chunk_gather_pool_scatter_bitexact(lcase):
    from prism_amd import ops
    name, grid, chunk, D, dt, masked = lcase
    say("chunk layout", lcase)
    rng = np.random.default_rng(11)
    S = int(np.prod(grid))
    x = rng.standard_normal((1, 2, S, D)).astype(np.float32)
    xh = bf16(x) if dt == "bf16" else x
    valid = (rng.random(S) > 0.25).astype(np.uint8) if masked else None
    lay = ops.ChunkLayout(grid, chunk, DEV)
    assert lay.pgrid == O.padded_grid(grid, chunk)
    src = O.chunk_source_index(grid, lay.pgrid, chunk, lay.rows)
    csz = int(np.prod(chunk))
    do = bf16(rng.standard_normal((1, 2, lay.rows, D)).astype(np.float32))
    g = ops.chunk_gather_pool(dev(xh), lay, None if valid is None else dev(valid), rows=True, pool=True, counts=True,
                              dot_with=dev(do))
    xf = _f(xh)
    rows_ref = O.chunk_rows(bf16(xf), src)
    assert bits_equal(host(g["rows"]), rows_ref)
    mean, cnt = O.chunk_pool(xf, src, valid, csz, lay.N_b)
    assert bits_equal(host(g["block_mean"]), mean)
    assert np.array_equal(host(g["block_count"]), cnt)
    ok = src >= 0
    if valid is not None:
        ok &= valid.astype(bool)[np.maximum(src, 0)]
    assert np.array_equal(host(g["valid_re"]), ok.astype(np.uint8))
    assert np.array_equal(host(g["tile_count"]), ok.reshape(-1, 64).sum(1))
    # rowdot multiplies the input values (fp32 inputs are not rounded first)
    rd = (O.chunk_rows(xf, src).astype(np.float64) * O.bf16_bits_to_f32(do)).sum(-1)
    np.testing.assert_allclose(host(g["rowdot"]), rd, rtol=1e-5, atol=1e-4)
    back = ops.chunk_scatter_rows(g["rows"], lay, torch.bfloat16)
    assert bits_equal(host(back), bf16(xf))


def test_rect_scores_transpose_pair_union_bitexact():
    from prism_amd import ops
    rng = np.random.default_rng(12)
    qc = rng.standard_normal((3, 37, 128)).astype(np.float32)
    kc = rng.standard_normal((3, 150, 128)).astype(np.float32)
    assert bits_equal(host(ops.block_scores(dev(qc), dev(kc), None)), O.block_scores(qc, kc, None))
    BH, Ntq, Ntk = 3, 6, 14
    qlen = rng.integers(0, Ntk + 1, BH * Ntq).astype(np.int32)
    qstart = np.arange(BH * Ntq, dtype=np.int64) * Ntk
    qcols = np.full(BH * Ntq * Ntk, -1, np.int32)
    for r in range(BH * Ntq):
        qcols[r * Ntk: r * Ntk + qlen[r]] = np.sort(rng.choice(Ntk, qlen[r], replace=False))
    ks, kl, kcol = ops.transpose_lists(dev(qstart), dev(qlen), dev(qcols), BH, Ntq, Ntk)
    ref_c, ref_l = O.transpose_lists(qstart, qlen, qcols, BH, Ntq, Ntk)
    assert np.array_equal(host(kl), ref_l)
    kc_h, ks_h = host(kcol), host(ks)
    for r in range(BH * Ntk):
        assert np.array_equal(kc_h[ks_h[r]: ks_h[r] + ref_l[r]], ref_c[r, : ref_l[r]])
    valid = (rng.random(Ntk * 64) > 0.05).astype(np.uint8)
    tm = ops.tile_masks(dev(valid))
    for lists, rows_per, cols, masks in (((qstart, qlen, qcols), Ntq, Ntk, O.tile_masks(valid)),
                                         ((ks_h, host(kl), kc_h), Ntk, Ntq, None)):
        u = ops.pair_union(*(dev(np.ascontiguousarray(a)) for a in lists), rows_per,
                           tm if masks is not None else None, col_tiles=cols)
        ref = O.pair_union(*lists, cols, masks)
        us, ul, uc = (host(a) for a in u)
        for p, want in enumerate(ref):
            assert np.array_equal(uc[us[p]: us[p] + ul[p]], want), p


# ------------------------------------------------------------------ end to end
def _oracle_attention(qh, kh, vh, do, ref, B, H, sm, k_masked):
    """O (THW of q), dQ (THW of q), dK, dV (THW of k) from the float64 oracle
    on the oracle's lists."""
    sq, sk = ref["q"], ref["k"]
    D = qh.shape[-1]
    qre = O.chunk_rows(bf16(_f(qh)), sq["src"])
    kre = O.chunk_rows(bf16(_f(kh)), sk["src"])
    vre = O.chunk_rows(bf16(_f(vh)), sk["src"])
    qf, kf, vf = (O.bf16_bits_to_f32(a).reshape(B * H, -1, D) for a in (qre, kre, vre))
    kv = sk["valid_re"] if k_masked else None
    o_ref, lse_ref = O.attn_fwd(qf, kf, vf, ref["qstart"], ref["qlen"], ref["qcols"], kv, sm)
    o_bf = O.bf16_bits_to_f32(bf16(o_ref.astype(np.float32)))
    do_re = O.bf16_bits_to_f32(O.chunk_rows(bf16(do), sq["src"])).reshape(B * H, -1, D)
    dq, dk, dv = O.attn_bwd(qf, kf, vf, o_bf, do_re, lse_ref, ref["qstart"], ref["qlen"], ref["qcols"], kv, sm)

    def thw(rows, src, S):
        out = np.zeros((B * H, S, D))
        ok = src >= 0
        out[:, src[ok]] = rows[:, ok]
        return out
    Sq, Sk = qh.shape[2], kh.shape[2]
    return (thw(o_ref, sq["src"], Sq), thw(dq, sq["src"], Sq), thw(dk, sk["src"], Sk), thw(dv, sk["src"], Sk))


def _check_lists(plan, ref, BH):
    Ntq = ref["q"]["Nt"]
    qs, ql, qc = host(plan.qstart), host(plan.qlen), host(plan.qcols)
    assert np.array_equal(ql, ref["qlen"])
    for r in range(BH * Ntq):
        assert np.array_equal(qc[qs[r]: qs[r] + ql[r]], ref["qcols"][ref["qstart"][r]: ref["qstart"][r] + ql[r]]), r


def _run_and_compare(q_np, k_np, v_np, fn, ref, B, H, k_masked):
    """fn(q, k, v) -> out; forward + backward vs the oracle."""
    D = q_np.shape[-1]
    sm = 1 / math.sqrt(D)
    tdt = torch.bfloat16 if q_np.dtype == np.uint16 else torch.float32
    q, k, v = (dev(a).requires_grad_(True) for a in (q_np, k_np, v_np))
    out = fn(q, k, v)
    assert out.dtype == tdt and out.shape == q.shape
    rng = np.random.default_rng(21)
    do = O.bf16_bits_to_f32(bf16(rng.standard_normal(q_np.shape).astype(np.float32)))
    o_r, dq_r, dk_r, dv_r = _oracle_attention(q_np, k_np, v_np, do, ref, B, H, sm, k_masked)
    _tol(out.detach().float().cpu().numpy().reshape(B * H, -1, D), o_r, "O")
    out.backward(torch.from_numpy(do).to(DEV).to(tdt))
    for name, t, r in (("dQ", q, dq_r), ("dK", k, dk_r), ("dV", v, dv_r)):
        _tol(t.grad.float().cpu().numpy().reshape(B * H, -1, D), r, name)


UNIFORM = [
    # (name, seed, B, H, grid, valid box or None, chunk_q, chunk_k, D, dtype, sparsity, cdf)
    ("444_d128_topk", 0, 1, 2, (8, 8, 16), None, (4, 4, 4), (4, 4, 4), 128, "bf16", 0.75, None),
    ("448_d64_pad_hybrid", 1, 1, 2, (8, 12, 16), (7, 10, 13), (4, 4, 8), (4, 4, 8), 64, "f32", 0.5, 0.9),
    ("mixed_chunks_cdf", 2, 2, 1, (8, 8, 16), (6, 8, 16), (4, 4, 4), (2, 4, 8), 128, "bf16", None, 0.8),
]


@pytest.mark.parametrize("ucase", UNIFORM, ids=[c[0] for c in UNIFORM])
def test_flash_attn_bsa_3d_vs_oracle(ucase):
    from prism_amd import ops
    from prism_amd.uniform_block_attention import flash_attn_bsa_3d, plan_chunked
    name, seed, B, H, grid, box, cq, ck, D, dt, sp, cdf = ucase
    say("uniform 3d", ucase)
    rng = np.random.default_rng(seed)
    S = int(np.prod(grid))
    valid = None
    if box is not None:
        t, h, w = np.meshgrid(*(np.arange(g) for g in grid), indexing="ij")
        valid = ((t < box[0]) & (h < box[1]) & (w < box[2])).reshape(-1).astype(np.uint8)
    qkv = []
    for _ in range(3):
        x = rng.standard_normal((B, H, S, D)).astype(np.float32)
        if valid is not None:
            x *= valid[None, None, :, None]
        qkv.append(bf16(x) if dt == "bf16" else x)
    qh, kh, vh = qkv
    # flash_attn_bsa_3d attends for fully padded query tiles by default, as the reference does
    ref = O.uniform_pipeline(_f(qh), _f(kh), grid, grid, cq, ck, sparsity=sp, cdf_threshold_p=cdf, q_valid=valid,
                             k_valid=valid, skip_padded_queries=False)
    vm = None if valid is None else dev(valid).bool()
    lq, lk = ops.ChunkLayout(grid, cq, DEV), ops.ChunkLayout(grid, ck, DEV)
    plan = plan_chunked(dev(qh), dev(kh), dev(vh), lq, lk, sparsity=sp, cdf_threshold=cdf, sm_scale=1 / math.sqrt(D),
                        q_valid=vm, k_valid=vm, compute_padded_queries=True, keep_scores=True)
    assert bits_equal(host(plan.scores), ref["scores"])
    _check_lists(plan, ref, B * H)
    _run_and_compare(qh, kh, vh, lambda q, k, v: flash_attn_bsa_3d(q, k, v, grid, grid, sparsity=sp, cdf_threshold=cdf,
                                                                   chunk_3d_shape_q=cq, chunk_3d_shape_k=ck,
                                                                   valid_mask=vm),
                     ref, B, H, k_masked=valid is not None)


CROSS = [
    # (name, q_structure, q_len or grid, k_structure, k_len or grid, chunk_q(3d) / size(1d), chunk_k, sparsity)
    ("audio_q_over_video_k", "1d", 200, "3d", (5, 8, 8), 64, (4, 4, 4), 0.5),
    ("video_q_over_audio_k_qrowpad", "3d", (4, 4, 10), "1d", 250, (4, 4, 4), 64, 0.5),
    ("audio_1d_krowpad", "1d", 100, "1d", 300, 64, 64, 0.6),
]


@pytest.mark.parametrize("ccase", CROSS, ids=[c[0] for c in CROSS])
def test_flash_attn_bsa_cross_vs_oracle(ccase):
    from prism_amd import ops
    from prism_amd.uniform_block_attention import flash_attn_bsa_cross, plan_chunked
    name, qs, qshape, ks, kshape, cq, ck, sp = ccase
    say("cross", ccase)
    B, H, D = 1, 2, 128
    rng = np.random.default_rng(31)
    qgrid = qshape if qs == "3d" else (1, 1, qshape)
    kgrid = kshape if ks == "3d" else (1, 1, kshape)
    chq = cq if qs == "3d" else (1, 1, cq)
    chk = ck if ks == "3d" else (1, 1, ck)
    qh, kh, vh = (bf16(rng.standard_normal((B, H, int(np.prod(g)), D)).astype(np.float32))
                  for g in (qgrid, kgrid, kgrid))
    lq, lk = ops.ChunkLayout(qgrid, chq, DEV), ops.ChunkLayout(kgrid, chk, DEV)
    ref = O.uniform_pipeline(_f(qh), _f(kh), qgrid, kgrid, chq, chk, sparsity=sp, q_pad_rows=lq.rows,
                             k_pad_rows=lk.rows, skip_padded_queries=True)
    plan = plan_chunked(dev(qh), dev(kh), dev(vh), lq, lk, sparsity=sp, cdf_threshold=None,
                        sm_scale=1 / math.sqrt(D), keep_scores=True)
    assert bits_equal(host(plan.scores), ref["scores"])
    _check_lists(plan, ref, B * H)
    kw = dict(q_grid_size=qshape if qs == "3d" else None, k_grid_size=kshape if ks == "3d" else None, sparsity=sp)
    if qs == "3d":
        kw["chunk_3d_shape_q"] = cq
    else:
        kw["chunk_size_q"] = cq
    if ks == "3d":
        kw["chunk_3d_shape_k"] = ck
    else:
        kw["chunk_size_k"] = ck
    _run_and_compare(qh, kh, vh, lambda q, k, v: flash_attn_bsa_cross(q, k, v, qs, ks, **kw), ref, B, H,
                     k_masked=lk.padded)


def test_flash_attn_bsa_block_order_chunk128_kvmask():
    """The autograd op on chunk-ordered tensors (bsa_interface.py:597-683),
    128-token chunks, queries pooled with the key mask (Sq == Sk)."""
    from prism_amd.uniform_block_attention import flash_attn_bsa
    B, H, S, D = 1, 2, 1024, 128
    rng = np.random.default_rng(41)
    qh, kh, vh = (bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    kv = (rng.random(S) > 0.1).astype(np.uint8)
    kv[256:384] = 0  # one fully padded chunk
    ref = O.uniform_pipeline(_f(qh), _f(kh), (1, 1, S), (1, 1, S), (1, 1, 128), (1, 1, 128), sparsity=0.5,
                             cdf_threshold_p=0.85, q_valid=kv, k_valid=kv, skip_padded_queries=False)
    sm = 1 / math.sqrt(D)
    _run_and_compare(qh, kh, vh, lambda q, k, v: flash_attn_bsa(q, k, v, 128, 128, 0.5, 0.85, sm,
                                                                kv_valid_mask=dev(kv).bool()),
                     ref, B, H, k_masked=True)


def test_uniform_errors():
    from prism_amd.uniform_block_attention import flash_attn_bsa_3d, flash_attn_bsa_cross, flash_attn_bsa
    q = torch.zeros((1, 1, 512, 64), device=DEV, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        flash_attn_bsa_3d(q, q, q, (8, 8, 6), (8, 8, 6))          # T*H*W != S
    with pytest.raises(AssertionError):
        flash_attn_bsa_3d(q, q, q, (8, 8, 8), (8, 8, 8), chunk_3d_shape_q=(4, 4, 3))
    with pytest.raises(ValueError, match="64 or 128"):
        flash_attn_bsa_3d(q, q, q, (8, 8, 8), (8, 8, 8), chunk_3d_shape_q=(2, 2, 8), chunk_3d_shape_k=(2, 2, 8))
    with pytest.raises(ValueError, match="sparsity or cdf_threshold"):
        flash_attn_bsa_3d(q, q, q, (8, 8, 8), (8, 8, 8), sparsity=None)
    with pytest.raises(ValueError, match="structure"):
        flash_attn_bsa_cross(q, q, q, "2d", "1d")
    with pytest.raises(NotImplementedError):
        flash_attn_bsa(q, q, q, 64, 64, 0.5, None, 0.125, score_modifier=torch.ones(1, device=DEV))


def test_run_bsa_uniform_matches_padded_reference_flow():
    """run_bsa_uniform (fused padding) equals the reference's flow of
    _run_bsa: F.pad to whole chunks + valid mask + flash_attn_bsa_3d + slice
    (wan_video_dit.py:470-507, :674-692), bit for bit, gradients included."""
    import torch.nn.functional as F
    from prism_amd.adapter import run_bsa_uniform
    from prism_amd.uniform_block_attention import flash_attn_bsa_3d
    B, H, D = 1, 2, 128
    grid = (5, 10, 14)
    pg = (8, 12, 16)
    S = int(np.prod(grid))
    rng = np.random.default_rng(51)
    qh, kh, vh, doh = (bf16(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(4))
    params = {"sparsity": 0.6, "cdf_threshold": 0.9, "chunk_3d_shape_q": [4, 4, 4], "chunk_3d_shape_k": [4, 4, 4],
              "variance_boost_gamma": 1.0}
    q1, k1, v1 = (dev(a).requires_grad_(True) for a in (qh, kh, vh))
    o1 = run_bsa_uniform(q1, k1, v1, grid, params)
    o1.backward(dev(doh))
    q2, k2, v2 = (dev(a).requires_grad_(True) for a in (qh, kh, vh))
    pad = lambda t: F.pad(t.view(B, H, *grid, D), (0, 0, 0, pg[2] - grid[2], 0, pg[1] - grid[1], 0, pg[0] - grid[0])
                          ).reshape(B, H, -1, D)
    t_, h_, w_ = torch.meshgrid(*(torch.arange(g, device=DEV) for g in pg), indexing="ij")
    vm = ((t_ < grid[0]) & (h_ < grid[1]) & (w_ < grid[2])).reshape(-1)
    o2p = flash_attn_bsa_3d(pad(q2), pad(k2), pad(v2), pg, pg, sparsity=0.6, cdf_threshold=0.9,
                            chunk_3d_shape_q=(4, 4, 4), chunk_3d_shape_k=(4, 4, 4), valid_mask=vm)
    o2 = o2p.view(B, H, *pg, D)[:, :, :grid[0], :grid[1], :grid[2]].reshape(B, H, S, D)
    o2.backward(dev(doh))
    assert bits_equal(host(o1), host(o2))
    for a, b in ((q1, q2), (k1, k2), (v1, v2)):
        assert bits_equal(host(a.grad), host(b.grad))
