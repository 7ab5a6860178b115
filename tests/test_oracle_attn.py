"""Pins the float64 attention oracle (oracle.attn_fwd / oracle.attn_bwd) to
an independent formulation: dense softmax attention in torch float64 with a
token mask, differentiated by torch autograd.

The dense mask is built the way the reference builds it:
  * create_mask_from_indices_varlen (bsa_interface.py:127-145): query tile i
    attends key tile j iff j is one of the first lens[i] entries of i's list;
  * the kernels' key-validity mask (flash_attn_bsa_varlen_mask.py:263-302):
    invalid keys get s = -inf and p = 0;
  * a row with no valid key at all has O = 0 and LSE = -inf (l_i starts at
    1.0 and m_i at -inf, :256-257 and :310-311), and no gradient.
LSE is the natural log (bsa_interface.py:383: M * ln 2 of the base-2 value).

Cases: empty lists, a fully masked key tile, rows whose first listed tile
is fully masked, Sq != Sk, D = 64 and 128.  Planted mistakes (made from the
oracle's own outputs or inputs: LSE in base 2, dK without sm_scale, a wrong
delta) must fail the same comparison.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

TILE = 64


def _lists(rng, BH, Ntq, Ntk, empty_rows=(), first_tiles=None):
    """Random ascending key-tile lists per query tile (row bh*Ntq + t)."""
    cap = Ntk
    qstart = np.arange(BH * Ntq, dtype=np.int64) * cap
    qlen = np.zeros(BH * Ntq, np.int32)
    qcols = np.zeros(BH * Ntq * cap, np.int32)
    for r in range(BH * Ntq):
        if r in empty_rows:
            continue
        n = int(rng.integers(1, Ntk + 1))
        cols = np.sort(rng.choice(Ntk, n, replace=False))
        if first_tiles is not None and r in first_tiles:
            cols = np.union1d(cols, [first_tiles[r]])  # the smallest tile id, so listed first
        qlen[r] = len(cols)
        qcols[r * cap: r * cap + len(cols)] = cols
    return qstart, qlen, qcols


def _dense_reference(q, k, v, do, qstart, qlen, qcols, kv_valid, sm):
    """float64 torch: masked softmax attention + autograd -> o, lse, dq, dk, dv."""
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    Ntq, Ntk = Sq // TILE, Sk // TILE
    tmask = torch.zeros((BH, Ntq, Ntk), dtype=torch.bool)
    for r in range(BH * Ntq):
        bh, t = divmod(r, Ntq)
        cols = qcols[qstart[r]: qstart[r] + qlen[r]]
        tmask[bh, t, torch.as_tensor(cols, dtype=torch.long)] = True
    mask = tmask.repeat_interleave(TILE, 1).repeat_interleave(TILE, 2)
    if kv_valid is not None:
        mask &= torch.as_tensor(kv_valid.astype(bool))[None, None, :]
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    s = qt @ kt.transpose(1, 2) * sm
    row_ok = mask.any(-1)
    s = torch.where(mask, s, torch.tensor(-math.inf, dtype=torch.float64))
    s = torch.where(row_ok[..., None], s, torch.zeros((), dtype=torch.float64))  # finite rows for autograd
    lse = torch.logsumexp(s, -1)
    p = torch.softmax(s, -1) * row_ok[..., None]
    o = p @ vt
    (o * torch.tensor(do, dtype=torch.float64)).sum().backward()
    lse = torch.where(row_ok, lse, torch.tensor(-math.inf, dtype=torch.float64))
    return (o.detach().numpy(), lse.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy())


def _close(a, b, what):
    fa, fb = np.isfinite(a), np.isfinite(b)
    assert np.array_equal(fa, fb), f"{what}: non-finite entries differ"
    assert np.array_equal(a[~fa], b[~fb]), f"{what}: infinities differ"
    err = np.abs(a[fa] - b[fb]).max() if fa.any() else 0.0
    scale = max(1.0, np.abs(b[fb]).max() if fb.any() else 0.0)
    assert err <= 1e-10 * scale, f"{what}: max error {err}"


def _case(seed, BH, Sq, Sk, D, masked_tiles=(), empty_rows=(), first_masked=False):
    rng = np.random.default_rng(seed)
    Ntq, Ntk = Sq // TILE, Sk // TILE
    kv = (rng.random(Sk) > 0.2).astype(np.uint8)
    for t in masked_tiles:
        kv[t * TILE:(t + 1) * TILE] = 0
    first = None
    if first_masked and masked_tiles:
        # rows whose smallest listed tile is the fully masked one (the
        # reference's all-(-inf) first-block guard, flash_attn_bsa_varlen_mask.py:295-302)
        m0 = min(masked_tiles)
        first = {r: m0 for r in range(0, BH * Ntq, 2)}
    qstart, qlen, qcols = _lists(rng, BH, Ntq, Ntk, empty_rows, first)
    if first is not None:
        for r in first:
            if qlen[r]:
                assert qcols[qstart[r]] == min(masked_tiles)
    q = rng.standard_normal((BH, Sq, D)).astype(np.float32)
    k = rng.standard_normal((BH, Sk, D)).astype(np.float32)
    v = rng.standard_normal((BH, Sk, D)).astype(np.float32)
    do = rng.standard_normal((BH, Sq, D)).astype(np.float32)
    return q, k, v, do, qstart, qlen, qcols, kv


CASES = [
    # seed, BH, Sq, Sk, D, fully masked key tiles, empty rows, first listed tile fully masked
    (0, 2, 256, 256, 64, (), (), False),
    (1, 2, 256, 256, 128, (1,), (3,), False),
    (2, 1, 192, 384, 64, (0, 4), (0, 2), True),   # Sq != Sk, more key tiles
    (3, 2, 384, 128, 128, (0,), (5,), True),      # Sq != Sk, more query tiles; tile 0 masked and first
]


@pytest.mark.parametrize("seed,BH,Sq,Sk,D,masked,empty,first", CASES)
def test_oracle_attention_vs_dense_autograd(seed, BH, Sq, Sk, D, masked, empty, first):
    q, k, v, do, qstart, qlen, qcols, kv = _case(seed, BH, Sq, Sk, D, masked, empty, first)
    sm = 1.0 / math.sqrt(D)
    o, lse = O.attn_fwd(q, k, v, qstart, qlen, qcols, kv, sm)
    dq, dk, dv = O.attn_bwd(q, k, v, o, do, lse, qstart, qlen, qcols, kv, sm)
    ro, rlse, rdq, rdk, rdv = _dense_reference(q, k, v, do, qstart, qlen, qcols, kv, sm)
    _close(o, ro, "O")
    _close(lse, rlse, "LSE")
    _close(dq, rdq, "dQ")
    _close(dk, rdk, "dK")
    _close(dv, rdv, "dV")
    # special cases the reference kernel defines
    Ntq = Sq // TILE
    for r in empty:
        bh, t = divmod(r, Ntq)
        rows = slice(t * TILE, (t + 1) * TILE)
        assert np.all(o[bh, rows] == 0) and np.all(np.isneginf(lse[bh, rows]))
        assert np.all(dq[bh, rows] == 0)
    assert np.isfinite(o).all() and np.isfinite(dq).all() and np.isfinite(dk).all() and np.isfinite(dv).all()


def test_oracle_attention_no_key_mask():
    """kv_valid = None (no padded key) agrees with an all-true mask."""
    q, k, v, do, qstart, qlen, qcols, _ = _case(7, 1, 128, 256, 64)
    sm = 1.0 / 8.0
    o, lse = O.attn_fwd(q, k, v, qstart, qlen, qcols, None, sm)
    dq, dk, dv = O.attn_bwd(q, k, v, o, do, lse, qstart, qlen, qcols, None, sm)
    ref = _dense_reference(q, k, v, do, qstart, qlen, qcols, np.ones(256, np.uint8), sm)
    for got, want, what in zip((o, lse, dq, dk, dv), ref, ("O", "LSE", "dQ", "dK", "dV")):
        _close(got, want, what)


def test_oracle_attention_dense_point_is_plain_softmax():
    """Every list full and every key valid: the oracle is textbook softmax
    attention (torch.nn.functional.scaled_dot_product_attention, float64)."""
    rng = np.random.default_rng(11)
    BH, S, D = 2, 256, 64
    q, k, v = (rng.standard_normal((BH, S, D)) for _ in range(3))
    Nt = S // TILE
    qstart = np.arange(BH * Nt, dtype=np.int64) * Nt
    qlen = np.full(BH * Nt, Nt, np.int32)
    qcols = np.tile(np.arange(Nt, dtype=np.int32), BH * Nt)
    o, lse = O.attn_fwd(q, k, v, qstart, qlen, qcols, None, 1 / 8.0)
    ref = torch.nn.functional.scaled_dot_product_attention(*(torch.tensor(x) for x in (q, k, v)))
    assert np.abs(o - ref.numpy()).max() < 1e-12
    s = np.einsum("bqd,bkd->bqk", q, k) / 8.0
    ref_lse = np.log(np.exp(s - s.max(-1, keepdims=True)).sum(-1)) + s.max(-1)
    assert np.abs(lse - ref_lse).max() < 1e-12


def _fails(fn):
    try:
        fn()
    except AssertionError:
        return True
    return False


def test_oracle_attention_planted_mistakes_fail():
    """Mistakes a restatement could make must fail the comparison above:
    the LSE stored in base 2, dK missing its sm_scale, and a wrong delta
    (rowsum of O * dO computed from a perturbed O)."""
    q, k, v, do, qstart, qlen, qcols, kv = _case(1, 2, 256, 256, 128, (1,), (3,), False)
    sm = 1.0 / math.sqrt(128)
    o, lse = O.attn_fwd(q, k, v, qstart, qlen, qcols, kv, sm)
    dq, dk, dv = O.attn_bwd(q, k, v, o, do, lse, qstart, qlen, qcols, kv, sm)
    ro, rlse, rdq, rdk, rdv = _dense_reference(q, k, v, do, qstart, qlen, qcols, kv, sm)
    _close(lse, rlse, "LSE")
    _close(dk, rdk, "dK")
    assert _fails(lambda: _close(lse / math.log(2.0), rlse, "LSE in log2"))
    assert _fails(lambda: _close(dk / sm, rdk, "dK without sm_scale"))
    # attn_bwd reads O only through delta = rowsum(O * dO)
    bad_o = o * 1.01
    bdq, bdk, bdv = O.attn_bwd(q, k, v, bad_o, do, lse, qstart, qlen, qcols, kv, sm)
    _close(bdv, rdv, "dV does not depend on delta")
    assert _fails(lambda: _close(bdq, rdq, "dQ with a wrong delta"))
    assert _fails(lambda: _close(bdk, rdk, "dK with a wrong delta"))
    # a key mask that is ignored
    o2, _ = O.attn_fwd(q, k, v, qstart, qlen, qcols, None, sm)
    assert _fails(lambda: _close(o2, ro, "O without the key mask"))
