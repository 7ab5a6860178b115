"""Seeded random sweep of the uniform-chunk entry points end to end:
flash_attn_bsa_3d (bsa_interface.py:1123-1176) and flash_attn_bsa_cross
(:1276-1392), forward and backward through autograd, against the oracle's
uniform selection (per-query-tile key lists, bit for bit) and its float64
attention on those lists.  Each case draws the entry point, the structure of
each side (3-D grid or 1-D sequence), grids and lengths (whole chunks or not
for the cross path, which pads internally), chunk shapes of 64 or 128
tokens, a valid box (self path), batch, heads, head dim, dtype and the
selection mode with its parameters.  O / dQ / dK / dV within the bound of the
dynamic sweep (tests/test_gpu_random.py): the north-star bound on the error
beyond a per-element bf16 allowance (the value's storage rounding, and for
the gradients the rounding of the reference backward's bf16 operands, 2^-8
times the sum of the magnitudes of the element's terms).  Cross cases with
few queries per key have |dK|, |dV| ~ 1 on average; there the reference's
own bf16 arithmetic has a mean-abs error of 2.0e-3 to 2.5e-3 (seeds 37 and
175 of a longer sweep)."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import bf16
from tests.test_gpu_parity import DEV, _tol, dev, host, say

pytestmark = pytest.mark.gpu

N_CASES = 48
# cross cases of a longer sweep whose gradients average |dK|, |dV| ~ 1
REGRESSION_SEEDS = (37, 175)

# chunk shapes of 64 and 128 tokens (t, h, w)
CHUNKS_3D = [(4, 4, 4), (2, 4, 8), (2, 8, 4), (1, 8, 8), (4, 2, 8), (4, 4, 8), (2, 8, 8), (4, 8, 4), (8, 4, 4)]


def _draw(seed):
    rng = np.random.default_rng(7000 + seed)
    mode = ("topk", "hybrid", "cdf")[seed % 3]
    sparsity = None if mode == "cdf" else float(rng.uniform(0.3, 0.9))
    cdf = None if mode == "topk" else float(rng.uniform(0.5, 0.97))
    c = dict(rng=rng, mode=mode, sparsity=sparsity, cdf=cdf, B=int(rng.integers(1, 3)), H=int(rng.integers(1, 3)),
             D=(64, 128)[(seed // 3) % 2], dtype=("bf16", "f32")[(seed // 6) % 2])
    if seed % 2 == 0:
        # self path: one grid of whole chunks on both sides, optional valid box
        cq = CHUNKS_3D[int(rng.integers(len(CHUNKS_3D)))]
        ck = CHUNKS_3D[int(rng.integers(len(CHUNKS_3D)))] if rng.random() < 0.5 else cq
        unit = tuple(int(np.lcm(a, b)) for a, b in zip(cq, ck))
        grid = tuple(u * int(rng.integers(1, 3 if u >= 8 else 4)) for u in unit)
        box = tuple(int(rng.integers(max(1, g - 3), g + 1)) for g in grid) if rng.random() < 0.5 else None
        c.update(kind="3d", grid=grid, cq=cq, ck=ck, box=box)
    else:
        qs, ks = ("1d", "3d"), ("1d", "3d")
        q_st, k_st = qs[int(rng.integers(2))], ks[int(rng.integers(2))]

        def side(st):
            if st == "1d":
                return int(rng.integers(20, 400)), int((64, 128)[int(rng.integers(2))])
            chunk = CHUNKS_3D[int(rng.integers(len(CHUNKS_3D)))]
            grid = tuple(int(rng.integers(max(1, x // 2), 3 * x)) for x in chunk)
            return grid, chunk
        qg, qc = side(q_st)
        kg, kc = side(k_st)
        c.update(kind="cross", q_st=q_st, k_st=k_st, qg=qg, qc=qc, kg=kg, kc=kc)
    return c


def _oracle_attention(qh, kh, vh, do, ref, B, H, sm, k_masked):
    """O, dQ (THW of q), dK, dV (THW of k) and the term magnitudes of the
    gradients, float64 oracle on the oracle's lists."""
    sq, sk = ref["q"], ref["k"]
    D = qh.shape[-1]
    f = lambda a: O.bf16_bits_to_f32(a) if a.dtype == np.uint16 else a
    qre = O.chunk_rows(bf16(f(qh)), sq["src"])
    kre = O.chunk_rows(bf16(f(kh)), sk["src"])
    vre = O.chunk_rows(bf16(f(vh)), sk["src"])
    qf, kf, vf = (O.bf16_bits_to_f32(a).reshape(B * H, -1, D) for a in (qre, kre, vre))
    kv = sk["valid_re"] if k_masked else None
    o_ref, lse_ref = O.attn_fwd(qf, kf, vf, ref["qstart"], ref["qlen"], ref["qcols"], kv, sm)
    o_bf = O.bf16_bits_to_f32(bf16(o_ref.astype(np.float32)))
    do_re = O.bf16_bits_to_f32(O.chunk_rows(bf16(do), sq["src"])).reshape(B * H, -1, D)
    args = (qf, kf, vf, o_bf, do_re, lse_ref, ref["qstart"], ref["qlen"], ref["qcols"], kv, sm)
    dq, dk, dv = O.attn_bwd(*args)
    mq, mk, mv = O.attn_bwd_term_magnitudes(*args)

    def thw(rows, src, S):
        out = np.zeros((B * H, S, D))
        ok = src >= 0
        out[:, src[ok]] = rows[:, ok]
        return out
    Sq, Sk = qh.shape[2], kh.shape[2]
    return (thw(o_ref, sq["src"], Sq), [thw(dq, sq["src"], Sq), thw(dk, sk["src"], Sk), thw(dv, sk["src"], Sk)],
            [thw(mq, sq["src"], Sq), thw(mk, sk["src"], Sk), thw(mv, sk["src"], Sk)])


@pytest.mark.parametrize("seed", sorted(set(range(N_CASES)) | set(REGRESSION_SEEDS)))
def test_random_uniform_end_to_end(seed):
    from prism_amd import ops
    from prism_amd.uniform_block_attention import flash_attn_bsa_3d, flash_attn_bsa_cross, plan_chunked
    c = _draw(seed)
    rng, B, H, D = c["rng"], c["B"], c["H"], c["D"]
    say("random uniform case", seed, {k: v for k, v in c.items() if k != "rng"})
    sm = 1.0 / math.sqrt(D)
    if c["kind"] == "3d":
        qgrid = kgrid = c["grid"]
        chq, chk = c["cq"], c["ck"]
    else:
        qgrid = c["qg"] if c["q_st"] == "3d" else (1, 1, c["qg"])
        kgrid = c["kg"] if c["k_st"] == "3d" else (1, 1, c["kg"])
        chq = c["qc"] if c["q_st"] == "3d" else (1, 1, c["qc"])
        chk = c["kc"] if c["k_st"] == "3d" else (1, 1, c["kc"])
    Sq, Sk = int(np.prod(qgrid)), int(np.prod(kgrid))
    valid = None
    if c["kind"] == "3d" and c["box"] is not None:
        t, h, w = np.meshgrid(*(np.arange(g) for g in qgrid), indexing="ij")
        b = c["box"]
        valid = ((t < b[0]) & (h < b[1]) & (w < b[2])).reshape(-1).astype(np.uint8)
    xs = [rng.standard_normal((B, H, S, D)).astype(np.float32) for S in (Sq, Sk, Sk)]
    if valid is not None:
        xs = [x * valid[None, None, :, None] for x in xs]
    ins = [bf16(x) if c["dtype"] == "bf16" else x for x in xs]
    qh, kh, vh = ins
    tdt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    lq, lk = ops.ChunkLayout(qgrid, chq, DEV), ops.ChunkLayout(kgrid, chk, DEV)
    f = lambda a: O.bf16_bits_to_f32(a) if a.dtype == np.uint16 else a
    if c["kind"] == "3d":
        ref = O.uniform_pipeline(f(qh), f(kh), qgrid, kgrid, chq, chk, sparsity=c["sparsity"],
                                 cdf_threshold_p=c["cdf"], q_valid=valid, k_valid=valid, skip_padded_queries=False)
        vm = None if valid is None else dev(valid).bool()
        plan = plan_chunked(dev(qh), dev(kh), dev(vh), lq, lk, sparsity=c["sparsity"], cdf_threshold=c["cdf"],
                            sm_scale=sm, q_valid=vm, k_valid=vm, compute_padded_queries=True)
        fn = lambda q, k, v: flash_attn_bsa_3d(q, k, v, qgrid, kgrid, sparsity=c["sparsity"],
                                               cdf_threshold=c["cdf"], chunk_3d_shape_q=chq, chunk_3d_shape_k=chk,
                                               valid_mask=vm)
        k_masked = valid is not None or ref["k"]["masked"]
    else:
        ref = O.uniform_pipeline(f(qh), f(kh), qgrid, kgrid, chq, chk, sparsity=c["sparsity"],
                                 cdf_threshold_p=c["cdf"], q_pad_rows=lq.rows, k_pad_rows=lk.rows,
                                 skip_padded_queries=True)
        plan = plan_chunked(dev(qh), dev(kh), dev(vh), lq, lk, sparsity=c["sparsity"], cdf_threshold=c["cdf"],
                            sm_scale=sm)
        kw = dict(sparsity=c["sparsity"], cdf_threshold=c["cdf"])
        if c["q_st"] == "3d":
            kw.update(q_grid_size=qgrid, chunk_3d_shape_q=chq)
        else:
            kw.update(chunk_size_q=c["qc"])
        if c["k_st"] == "3d":
            kw.update(k_grid_size=kgrid, chunk_3d_shape_k=chk)
        else:
            kw.update(chunk_size_k=c["kc"])
        fn = lambda q, k, v: flash_attn_bsa_cross(q, k, v, c["q_st"], c["k_st"], **kw)
        k_masked = lk.padded
    say("N_b", ref["q"]["nb"], ref["k"]["nb"], "kept tile pairs", int(ref["qlen"].sum()))
    # the selection, bit for bit: per-query-tile key lists
    Ntq = ref["q"]["Nt"]
    qs_, ql_, qc_ = host(plan.qstart), host(plan.qlen), host(plan.qcols)
    assert np.array_equal(ql_, ref["qlen"])
    for r in range(B * H * Ntq):
        want = ref["qcols"][ref["qstart"][r]: ref["qstart"][r] + ql_[r]]
        assert np.array_equal(qc_[qs_[r]: qs_[r] + ql_[r]], want), r
    del plan
    # attention, forward + backward
    q, k, v = (dev(a).requires_grad_(True) for a in ins)
    out = fn(q, k, v)
    assert out.dtype == tdt and out.shape == q.shape
    # the inference path (no autograd) gives the same output bits
    with torch.no_grad():
        out_ng = fn(*(dev(a) for a in ins))
    iv = torch.int16 if tdt == torch.bfloat16 else torch.int32
    assert torch.equal(out_ng.view(iv), out.detach().view(iv))
    do = O.bf16_bits_to_f32(bf16(rng.standard_normal((B, H, Sq, D)).astype(np.float32)))
    o_r, grads, mags = _oracle_attention(qh, kh, vh, do, ref, B, H, sm, k_masked)
    _tol(out.detach().float().cpu().numpy().reshape(B * H, -1, D), o_r, "O")
    out.backward(torch.from_numpy(do).to(DEV).to(tdt))
    for name, t, r, m in zip(("dQ", "dK", "dV"), (q, k, v), grads, mags):
        _tol(t.grad.float().cpu().numpy().reshape(B * H, -1, D), r, name, slack=2.0 ** -8 * m)
