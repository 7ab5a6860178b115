"""Pin the oracle's statistics and shape functions against independent
mathematics: libm / numpy float64 routines, closed-form grids and
known-answer shape decisions.  CPU only."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.cases import bf16


# ------------------------------------------------------------------ canonical exp / log2 / sums
def _ulp_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref) / np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)


def test_canon_exp_matches_exp_within_one_ulp():
    xs = np.concatenate([np.linspace(-87, 0, 40001), np.linspace(0, 88, 4001), [-1e-7, 1e-7]]).astype(np.float32)
    got = np.array([O.canon_exp(float(x)) for x in xs], np.float32)
    assert _ulp_err(got, np.exp(xs.astype(np.float64))).max() <= 1.0
    assert np.all(np.diff(got[:40001]) >= 0)  # monotone on the softmax range


def test_canon_exp_special_values():
    assert O.canon_exp(0.0) == 1.0
    assert O.canon_exp(float("-inf")) == 0.0
    assert O.canon_exp(-87.5) == 0.0
    assert math.isinf(O.canon_exp(89.0))
    assert math.isnan(O.canon_exp(float("nan")))


def test_canon_log2_accuracy_and_powers_of_two():
    gs = np.exp(np.linspace(np.log(1e-4), np.log(4.0), 30001)).astype(np.float32)
    got = np.array([O.canon_log2(float(g)) for g in gs], np.float32)
    ref = np.log2(gs.astype(np.float64))
    err = np.abs(got - ref)
    assert (err <= 3 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-7).all()
    for e in range(-14, 3):
        assert O.canon_log2(2.0 ** e) == float(e)


def test_sum_lanes64_exact_on_integers_and_close_otherwise():
    rng = np.random.default_rng(0)
    ints = rng.integers(-1000, 1000, 128).astype(np.float32)
    assert O.sum_lanes64(ints) == float(ints.sum())
    x = rng.standard_normal(128).astype(np.float32)
    assert abs(O.sum_lanes64(x) - x.astype(np.float64).sum()) < 1e-5
    x64 = rng.standard_normal(64).astype(np.float32)
    assert abs(O.sum_lanes64(x64) - x64.astype(np.float64).sum()) < 1e-5


@pytest.mark.parametrize("p", [0.9, 0.2, 0.5, 0.999, 1e-3])
def test_cdf_threshold_is_the_rounding_boundary(p):
    thr = O.cdf_threshold(p)
    pf = np.float32(p)
    f = lambda X: np.float32(np.uint64(X)) * np.float32(2.0 ** -60)
    assert f(thr) >= pf and f(thr - 1) < pf


# ------------------------------------------------------------------ zone aggregates
def _np_zone_means(x, grid, valid):
    """float64 masked zone means via numpy (independent of the oracle's order)."""
    T, Hg, Wg = grid
    D = x.shape[-1]
    ZT, ZH, ZW = T // 8, Hg // 8, Wg // 8
    xz = x.reshape(ZT, 8, ZH, 8, ZW, 8, D).transpose(0, 2, 4, 1, 3, 5, 6).reshape(-1, 8, 8, 8, D).astype(np.float64)
    m = valid.reshape(ZT, 8, ZH, 8, ZW, 8).transpose(0, 2, 4, 1, 3, 5).reshape(-1, 8, 8, 8, 1).astype(np.float64)
    cm = (xz * m).sum((1, 2, 3)) / np.maximum(m.sum((1, 2, 3)), 1)
    fT = (xz * m).sum((2, 3)) / np.maximum(m.sum((2, 3)), 1)
    aH = (xz * m).sum((1, 3)) / np.maximum(m.sum((1, 3)), 1)
    aW = (xz * m).sum((1, 2)) / np.maximum(m.sum((1, 2)), 1)
    Nz = xz.shape[0]
    return np.concatenate([cm, fT.reshape(Nz, -1), aH.reshape(Nz, -1), aW.reshape(Nz, -1)], 1)


@pytest.mark.parametrize("D", [64, 128])
def test_zone_stats_vs_float64(D):
    rng = np.random.default_rng(1)
    grid = (8, 16, 24)
    S = 8 * 16 * 24
    v = rng.standard_normal((1, 3, S, D)).astype(np.float32)
    valid = (rng.random(S) > 0.2).astype(np.uint8)
    packed, av = O.zone_stats(v, grid, valid)
    havg = (v[0].astype(np.float64).sum(0) * np.float32(1 / 3)).astype(np.float32)
    ref = _np_zone_means(havg, grid, valid)
    assert np.allclose(packed, ref, rtol=1e-5, atol=1e-6)
    vz = valid.reshape(1, 8, 2, 8, 3, 8).transpose(0, 2, 4, 1, 3, 5).reshape(-1, 8, 8, 8)
    assert np.array_equal(av[:, :8], vz.any((2, 3)))
    assert np.array_equal(av[:, 8:16], vz.any((1, 3)))
    assert np.array_equal(av[:, 16:], vz.any((1, 2)))


def test_zone_stats_bf16_head_mean_rounds_to_bf16():
    rng = np.random.default_rng(2)
    grid = (8, 8, 8)
    v = rng.standard_normal((1, 5, 512, 64)).astype(np.float32)
    vb = bf16(v)
    packed, _ = O.zone_stats(vb, grid, None)
    havg = O.bf16_bits_to_f32(vb)[0].astype(np.float64).sum(0)
    hb = O.bf16_bits_to_f32(bf16((havg * np.float32(0.2)).astype(np.float32)))
    ref = _np_zone_means(hb, grid, np.ones(512, np.uint8))
    assert np.allclose(packed, ref, rtol=1e-5, atol=1e-6)


def test_zone_gradient_constant_field_is_zero():
    grid = (8, 8, 16)
    D = 64
    v = np.broadcast_to(np.float32(1.5), (1, 2, 8 * 8 * 16, D)).copy()
    packed, av = O.zone_stats(v, grid, None)
    rho_raw, aniso = O.zone_gradient(packed, av, D)
    assert np.all(rho_raw == 0) and np.all(aniso == 0)


def test_zone_gradient_linear_in_t_closed_form():
    """x[t,h,w,d] = a_d * t: var_H = var_W = 0, aniso_T = 1,
    temporal var = mean(a^2), spatial var = var_d(3.5 a_d)."""
    D = 64
    a = np.linspace(-1, 1, D).astype(np.float32)
    t = np.arange(8, dtype=np.float32)
    x = (t[:, None, None, None] * a[None, None, None, :]) * np.ones((8, 8, 8, D), np.float32)
    v = x.reshape(1, 1, 512, D)
    packed, av = O.zone_stats(v, (8, 8, 8), None)
    rho_raw, aniso = O.zone_gradient(packed, av, D)
    assert np.allclose(aniso[0], [1, 0, 0], atol=1e-6)
    cm = 3.5 * a.astype(np.float64)
    expect = np.var(cm) + np.mean(a.astype(np.float64) ** 2)
    assert abs(rho_raw[0] - expect) < 1e-5 * expect


def test_zone_gradient_vs_float64_formulas():
    """Spatial/temporal variance and masked axis variances against numpy
    np.var / np.mean on random aggregates with random validity."""
    rng = np.random.default_rng(4)
    Nz, D = 6, 128
    packed = rng.standard_normal((Nz, 25 * D)).astype(np.float32)
    av = (rng.random((Nz, 24)) > 0.3).astype(np.uint8)
    av[0] = 1
    rho_raw, aniso = O.zone_gradient(packed, av, D)
    for z in range(Nz):
        p = packed[z].astype(np.float64)
        cm, fr = p[:D], p[D:9 * D].reshape(8, D)
        axes = [fr, p[9 * D:17 * D].reshape(8, D), p[17 * D:].reshape(8, D)]
        tv = av[z, :8].astype(bool)
        bv = tv[1:] & tv[:-1]
        temporal = (((fr[1:] - fr[:-1]) ** 2)[bv].sum(0) / max(bv.sum(), 1)).mean()
        assert abs(rho_raw[z] - (np.var(cm) + temporal)) < 1e-5 * (1 + rho_raw[z])
        var = []
        for i, A in enumerate(axes):
            m = av[z, 8 * i:8 * i + 8].astype(bool)
            var.append(np.var(A[m], axis=0).mean() if m.any() else 0.0)
        s = max(sum(var), 1e-6)
        assert np.allclose(aniso[z], np.array(var) / s, rtol=1e-5, atol=1e-7)


def test_audio_zone_stats_vs_float64():
    rng = np.random.default_rng(5)
    grid = (8, 16, 8)
    S = 8 * 16 * 8
    n = rng.random(S).astype(np.float32)
    valid = (rng.random(S) > 0.25).astype(np.uint8)
    abar, vhat = O.audio_zone_stats(n, grid, valid)
    means = _np_zone_means(n[:, None], grid, valid)  # [Nz, 25]
    assert np.allclose(abar, means[:, 0], rtol=1e-6)
    vz = valid.reshape(1, 8, 2, 8, 1, 8).transpose(0, 2, 4, 1, 3, 5).reshape(-1, 8, 8, 8)
    for z in range(2):
        var = []
        for i, flags in enumerate((vz[z].any((1, 2)), vz[z].any((0, 2)), vz[z].any((0, 1)))):
            vals = means[z, 1 + 8 * i:9 + 8 * i]
            var.append(np.var(vals[flags]) if flags.any() else 0.0)
        assert np.allclose(vhat[z], np.array(var) / max(sum(var), 1e-6), rtol=1e-5, atol=1e-7)


def test_a2v_norms_vs_float64():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((50, 5120)).astype(np.float32)
    got = O.a2v_norms(x, False)
    assert np.allclose(got, np.linalg.norm(x.astype(np.float64), axis=1), rtol=2e-6)
    gb = O.bf16_bits_to_f32(O.a2v_norms(bf16(x), True))
    ref = np.linalg.norm(O.bf16_bits_to_f32(bf16(x)).astype(np.float64), axis=1)
    assert np.allclose(gb, ref, rtol=2 ** -8)


# ------------------------------------------------------------------ shape decisions (known answers)
CAND = O.CANDIDATES


@pytest.mark.parametrize("cid", range(7))
def test_ivpq_exact_hit_selects_that_candidate(cid):
    """g_a = 2^(-1.5 log2 b_a) makes the ideal block exactly candidate b."""
    lb = np.log2(np.array(CAND[cid], np.float64))
    g = (2.0 ** (-1.5 * lb)).astype(np.float32)[None]
    rho_raw = np.array([1.0], np.float32)  # rho = 1 >= tau: 64-token pool
    _, _, sid = O.zone_shapes(rho_raw, g, None, None, "ivpq", tau_128=0.15)
    assert sid[0] == cid


def test_ivpq_128_pool_gating():
    """ideal = (2/3, 8/3, 8/3): (2,8,8) is nearest (dist 1/3) when the 128
    pool is open, a 64-token shape at dist 2/3 when rho >= tau."""
    g = (2.0 ** (-1.5 * np.array([2 / 3, 8 / 3, 8 / 3]))).astype(np.float32)[None]
    rho_raw = np.array([0.1], np.float32)
    # rho = rho_raw / max(rho_raw) = 1 for a single zone: add a second zone to control rho
    rr = np.array([0.1, 1.0], np.float32)
    gg = np.concatenate([g, np.full((1, 3), 1 / 3, np.float32)])
    _, rho, sid = O.zone_shapes(rr, gg, None, None, "ivpq", tau_128=0.15)
    assert rho[0] == np.float32(0.1) and sid[0] == 7 and sid[1] == 0
    _, _, sid2 = O.zone_shapes(rr, gg, None, None, "ivpq", tau_128=0.05)
    assert sid2[0] in (3, 4)


def test_penalty_known_answers():
    g = np.array([[1.0, 0.5, 1e-4]], np.float32)
    rr = np.array([0.0], np.float32)  # rho_raw max 0 -> rho = 0 / 1e-6 = 0 < tau
    _, _, sid = O.zone_shapes(rr, g, None, None, "penalty", tau_128=0.15, lambda_128=1.0)
    assert sid[0] == 3  # (2,4,8): 2 + 2 + 0.0008
    _, _, sid = O.zone_shapes(rr, g, None, None, "penalty", tau_128=0.15, lambda_128=3.0)
    assert sid[0] == 7  # (2,8,8): 2 + 4 + 0.0008 - 3
    rr1 = np.array([1.0], np.float32)  # rho = 1 >= tau: 128 pool closed
    _, _, sid = O.zone_shapes(rr1, g, None, None, "penalty", tau_128=0.15, lambda_128=3.0)
    assert sid[0] == 3


def test_audio_term_enters_g():
    """g = aniso + lambda_a * a_bar_norm * v_hat with a_bar max-normalised."""
    aniso = np.array([[0.2, 0.3, 0.5], [0.2, 0.3, 0.5]], np.float32)
    abar = np.array([2.0, 4.0], np.float32)
    vhat = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]], np.float32)
    g, _, _ = O.zone_shapes(np.ones(2, np.float32), aniso, abar, vhat, "ivpq", lambda_a=0.5)
    assert np.allclose(g[0], [0.2 + 0.5 * 0.5, 0.3, 0.5], rtol=1e-6)
    assert np.allclose(g[1], [0.2, 0.3, 0.5 + 0.5], rtol=1e-6)
    g2, _, _ = O.zone_shapes(np.ones(2, np.float32), np.zeros((2, 3), np.float32), None, None, "ivpq")
    assert np.all(g2 == np.float32(1e-4))  # clamp


def test_unknown_method_raises():
    with pytest.raises(ValueError):
        O.zone_shapes(np.ones(1, np.float32), np.ones((1, 3), np.float32), method="nope")
