"""The torch float32 restatement of the reference's CPU path (oracle/torch_path.py,
the timed CPU baseline of bench.py) computes what the C / float64 oracle
computes: the same shape ids, the same per-tile key lists (except rows whose
cumulative-threshold decision lies within float32 rounding of p, counted),
and the same attention outputs and gradients within float32 tolerance."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle import torch_path as TP
from tests.cases import padded_case

TILE = 64


def _case(seed, grid_real, H, D, audio):
    c = padded_case(seed, 1, H, grid_real, D, lowrank=True, audio_tokens=audio)
    t = {n: torch.from_numpy(c[n]) for n in ("q", "k", "v")}
    t["norms"] = None if c["norms"] is None else torch.from_numpy(c["norms"])
    t["valid"] = torch.from_numpy(c["valid"]).bool()
    return c, t


@pytest.mark.parametrize("method", ["ivpq", "penalty"])
def test_shape_ids_match_oracle(method):
    for seed, gr in ((0, (4, 16, 16)), (1, (13, 20, 24))):
        c, t = _case(seed, gr, 3, 64, 32)
        ref = O.select_zone_shapes(c["v"], c["norms"], c["grid"], method, valid=c["valid"])
        got = TP.zone_shapes(t["v"], t["norms"], c["grid"], t["valid"], method)
        assert np.array_equal(got.numpy(), ref), (seed, method)


def test_geometry_matches_oracle():
    rng = np.random.default_rng(3)
    grid = (16, 16, 24)
    sid = rng.integers(0, 13, size=(2 * 2 * 3)).astype(np.int64)
    src, inv = TP.rearrange_index(torch.from_numpy(sid), grid)
    rsrc, rinv = O.rearrange_index(sid, grid)
    assert np.array_equal(src.numpy(), rsrc) and np.array_equal(inv.numpy(), rinv)
    bid, kbt, nb = TP.block_maps(torch.from_numpy(sid))
    rbid, rkbt, rnb, _ = O.tile_maps(sid)
    assert nb == rnb and np.array_equal(bid.numpy(), rbid) and np.array_equal(kbt.numpy(), rkbt)


def test_selection_and_attention_match_oracle():
    """Config 1's parameters: top-8 blocks + p = 0.9, fp32, D = 64, grid
    4x16x16 padded to 8x16x16, audio norms."""
    c, t = _case(0, (4, 16, 16), 4, 64, 64)
    grid, valid = c["grid"], c["valid"]
    sid = O.select_zone_shapes(c["v"], c["norms"], grid, "ivpq", valid=valid)
    _, _, N_b, _ = O.tile_maps(sid)
    sp = 1.0 - (8 + 0.5) / N_b
    ref = O.select_pipeline(c["q"], c["k"], c["v"], grid, sparsity=sp, cdf_threshold_p=0.9, audio_norms=c["norms"],
                            valid=valid, shape_ids=sid)
    rng = np.random.default_rng(5)
    do = rng.standard_normal(c["q"].shape).astype(np.float32)
    out, dq, dk, dv, pl = TP.forward_backward(t["q"], t["k"], t["v"], torch.from_numpy(do), grid, sparsity=sp,
                                              cdf_threshold=0.9, norms=t["norms"], valid=t["valid"])
    assert np.array_equal(pl["shape_ids"].numpy(), sid)
    B, H, S, D = c["q"].shape
    Nt = S // TILE
    tiles = pl["tiles"].reshape(B * H * Nt, -1).numpy()
    lens = pl["lens"].reshape(-1).numpy()
    differ = 0
    for r in range(B * H * Nt):
        a = ref["qcols"][ref["qstart"][r]: ref["qstart"][r] + ref["qlen"][r]]
        b = tiles[r, : lens[r]]
        differ += not np.array_equal(a, b)
    assert differ <= B * H * Nt // 50, differ  # rows decided within float32 rounding of p
    # attention on the torch path's own lists vs the float64 oracle on the same lists
    src, inv = pl["src"].numpy(), pl["inv"].numpy()
    qf, kf, vf = (c[n][:, :, src].reshape(B * H, S, D) for n in ("q", "k", "v"))
    qstart = np.arange(B * H * Nt, dtype=np.int64) * tiles.shape[1]
    o_ref, lse_ref = O.attn_fwd(qf, kf, vf, qstart, lens.astype(np.int32), tiles.reshape(-1).astype(np.int32),
                                valid[src], 1 / math.sqrt(D))
    grads = O.attn_bwd(qf, kf, vf, o_ref, do.reshape(B * H, S, D)[:, src], lse_ref, qstart, lens.astype(np.int32),
                       tiles.reshape(-1).astype(np.int32), valid[src], 1 / math.sqrt(D))
    for name, got, want in (("O", out, o_ref), ("dQ", dq, grads[0]), ("dK", dk, grads[1]), ("dV", dv, grads[2])):
        g = got.numpy().reshape(B * H, S, D)[:, src]
        assert np.abs(g - want).max() < 1e-4, name


def test_selection_agreement_counts_only_rounding_differences():
    """The checker the GPU tests and the benchmark use (selection_agreement):
    against the C oracle's selection of the same scores it finds no untied
    row decided away from p, and it counts every row of a planted mistake
    (the oracle run at p = 0.8 against the sequence at p = 0.9)."""
    import numpy as np
    import torch
    from oracle import oracle as O
    from oracle.torch_path import selection_agreement
    rng = np.random.default_rng(4)
    R, N = 96, 700
    s = (rng.standard_normal((R, N)) * 3).astype(np.float32)
    sp = 1 - 20.5 / N
    for p_ours, planted in ((0.9, False), (0.8, True)):
        sel, nsel = O.select(s, sp, p_ours, 0.125)
        sel_t = torch.from_numpy(np.where(sel < 0, 0, sel))
        out = selection_agreement(torch.from_numpy(s), sel_t, torch.from_numpy(nsel), sp, 0.9, 0.125)
        for c in out.values():
            if planted:
                assert c["rows_differing"] - c["of_them_tied"] >= R // 2
            else:
                assert c["max_untied_margin"] <= 4e-6, c
                assert c["rows_differing"] - c["of_them_tied"] <= R // 20, c
