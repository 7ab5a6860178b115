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


def test_oracle_bf16_operands_closed_form():
    """attn_bwd(bf16_operands=True) rounds P before dV = P^T dO and dS =
    P (dP - delta), formed from the unrounded P, before dK and dQ
    (flash_attn_bsa_varlen_mask.py:382-399, :462-470).  Inputs with a closed
    form: keys 0-2 valid (the rest masked), K = 0 except k_0 = 2 e_1, queries
    with q[:, 1] = 0, so every score is 0 and P = 1/3 over the valid keys
    (LSE = ln 3); v_0 = 5 e_0, the rest 0; dO rows e_0; O = 0, so delta = 0.
    Then dP = 5 on key 0 and 0 elsewhere, dS = 5/3 on key 0.  bf16(1/3) =
    0.333984375 and bf16(5/3) = 1.6640625 (8 significant bits, nearest);
    rounding P inside dS as well would give bf16(0.333984375 * 5) = 1.671875,
    and leaving dS unrounded 5/3."""
    rng = np.random.default_rng(5)
    S, D = 64, 64
    sm = 1.0 / 8.0
    q = rng.standard_normal((1, S, D))
    q[:, :, 1] = 0.0
    k = np.zeros((1, S, D)); k[0, 0, 1] = 2.0
    v = np.zeros((1, S, D)); v[0, 0, 0] = 5.0
    do = np.zeros((1, S, D)); do[:, :, 0] = 1.0
    o = np.zeros((1, S, D))
    lse = np.full((1, S), math.log(3.0))
    kv = np.zeros(S, np.uint8); kv[:3] = 1
    qstart, qlen, qcols = np.zeros(1, np.int64), np.ones(1, np.int32), np.zeros(1, np.int32)
    qsum = q[0].sum(0)
    for bf, p_bf, ds_bf in ((False, 1.0 / 3.0, 5.0 / 3.0), (True, 0.333984375, 1.6640625)):
        dq, dk, dv = O.attn_bwd(q, k, v, o, do, lse, qstart, qlen, qcols, kv, sm, bf16_operands=bf)
        want_dv = np.zeros((S, D)); want_dv[:3, 0] = S * p_bf
        want_dk = np.zeros((S, D)); want_dk[0] = ds_bf * sm * qsum
        want_dq = np.zeros((S, D)); want_dq[:, 1] = ds_bf * 2.0 * sm
        for got, want, what in ((dv[0], want_dv, "dV"), (dk[0], want_dk, "dK"), (dq[0], want_dq, "dQ")):
            assert np.abs(got - want).max() <= 1e-12 * max(1.0, np.abs(want).max()), (bf, what)
    # the three roundings are distinguishable at these values
    r = lambda x: float(O._round_bf16(np.array([x]))[0])
    assert r(1.0 / 3.0) == 0.333984375 and r(5.0 / 3.0) == 1.6640625 and r(0.333984375 * 5.0) == 1.671875


def test_oracle_bf16_operands_within_rounding_bound():
    """On random lists the bf16-operand backward differs from the float64 one
    by at most the rounding bound 2^-9 * sum |terms| per element
    (attn_bwd_term_magnitudes), and by more than nothing.  The magnitudes are
    at least |float64 result| (triangle inequality) and equal it where every
    term has one sign (the closed-form case: one nonzero dS per row, q >= 0)."""
    q, k, v, do, qstart, qlen, qcols, kv = _case(1, 2, 256, 256, 128, (1,), (3,), False)
    sm = 1.0 / math.sqrt(128)
    o, lse = O.attn_fwd(q, k, v, qstart, qlen, qcols, kv, sm)
    args = (q, k, v, o, do, lse, qstart, qlen, qcols, kv, sm)
    exact = O.attn_bwd(*args)
    rounded = O.attn_bwd(*args, bf16_operands=True)
    mags = O.attn_bwd_term_magnitudes(*args)
    for e, rr, m, what in zip(exact, rounded, mags, ("dQ", "dK", "dV")):
        diff = np.abs(rr - e)
        assert (diff <= 2.0 ** -9 * m + 1e-12).all(), what
        assert diff.max() > 0, what
        assert (np.abs(e) <= m * (1 + 1e-12) + 1e-12).all(), what
    # one sign: the closed-form inputs with q >= 0
    S, D = 64, 64
    qq = np.abs(np.random.default_rng(5).standard_normal((1, S, D))); qq[:, :, 1] = 0.0
    kk = np.zeros((1, S, D)); kk[0, 0, 1] = 2.0
    vv = np.zeros((1, S, D)); vv[0, 0, 0] = 5.0
    dd = np.zeros((1, S, D)); dd[:, :, 0] = 1.0
    kv1 = np.zeros(S, np.uint8); kv1[:3] = 1
    a1 = (qq, kk, vv, np.zeros((1, S, D)), dd, np.full((1, S), math.log(3.0)), np.zeros(1, np.int64),
          np.ones(1, np.int32), np.zeros(1, np.int32), kv1, 0.125)
    for e, m in zip(O.attn_bwd(*a1), O.attn_bwd_term_magnitudes(*a1)):
        assert np.abs(np.abs(e) - m).max() <= 1e-12
