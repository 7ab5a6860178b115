"""Pin the oracle's uniform chunk layout (flash_attn_bsa_3d / flash_attn_bsa_cross
geometry, padding and pooling) and its rectangular scores / list transpose
against brute force: per-token chunk arithmetic written from the reference's
definition of the 3-D block order (bsa_interface.py:1105-1121), float64
masked means, float64 matmuls and set transposes.  CPU only.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.cases import bf16


def _brute_src(grid, pgrid, chunk):
    """For every padded-grid token: its chunk n = (nt Nh + nh) Nw + nw and
    offset (it ch + ih) cw + iw, written out per token."""
    T, H, W = grid
    Tp, Hp, Wp = pgrid
    ct, ch, cw = chunk
    Nh, Nw = Hp // ch, Wp // cw
    csz = ct * ch * cw
    src = np.full(Tp * Hp * Wp, -7, np.int64)
    for t in range(Tp):
        for h in range(Hp):
            for w in range(Wp):
                n = ((t // ct) * Nh + h // ch) * Nw + w // cw
                off = ((t % ct) * ch + h % ch) * cw + w % cw
                src[n * csz + off] = (t * H + h) * W + w if (t < T and h < H and w < W) else -1
    return src


@pytest.mark.parametrize("grid,chunk", [((8, 8, 8), (4, 4, 4)), ((5, 9, 12), (4, 4, 8)), ((3, 7, 10), (2, 4, 8)),
                                        ((1, 1, 200), (1, 1, 64)), ((4, 8, 16), (4, 4, 8))])
def test_chunk_source_index_brute_force(grid, chunk):
    pg = O.padded_grid(grid, chunk)
    assert all(p % c == 0 and p >= g and p - g < c for p, g, c in zip(pg, grid, chunk))
    src = O.chunk_source_index(grid, pg, chunk)
    assert np.array_equal(src, _brute_src(grid, pg, chunk))
    S = int(np.prod(grid))
    assert np.array_equal(np.sort(src[src >= 0]), np.arange(S))  # every token exactly once
    # every chunk is a ct x ch x cw box of the padded grid
    csz = int(np.prod(chunk))
    T, H, W = grid
    for n in range(src.size // csz):
        toks = src[n * csz:(n + 1) * csz]
        toks = toks[toks >= 0]
        if toks.size:
            t, h, w = toks // (H * W), (toks // W) % H, toks % W
            assert t.max() - t.min() < chunk[0] and h.max() - h.min() < chunk[1] and w.max() - w.min() < chunk[2]
    # rows past the padded grid are padding
    more = O.chunk_source_index(grid, pg, chunk, rows=src.size + 64)
    assert np.array_equal(more[: src.size], src) and (more[src.size:] == -1).all()


def test_chunk_pool_masked_mean_and_order():
    rng = np.random.default_rng(5)
    grid, chunk = (5, 6, 8), (4, 4, 4)
    pg = O.padded_grid(grid, chunk)
    S = int(np.prod(grid))
    x = O.bf16_bits_to_f32(bf16(rng.standard_normal((1, 2, S, 64)).astype(np.float32)))
    valid = (rng.random(S) > 0.3).astype(np.uint8)
    src = O.chunk_source_index(grid, pg, chunk)
    nb = src.size // 64
    mean, cnt = O.chunk_pool(x, src, valid, 64, nb)
    for n in range(nb):
        rows = src[n * 64:(n + 1) * 64]
        ok = [r for r in rows if r >= 0 and valid[r]]
        assert cnt[n] == len(ok)
        want = x[:, :, ok].astype(np.float64).sum(2) / max(len(ok), 1)
        np.testing.assert_allclose(mean[:, :, n], want, rtol=2e-6, atol=1e-7)
        # the fp32 sum is taken per row group (chunk row j mod 512 / D) in row
        # order, then over the groups in order (the order the HIP kernel uses)
        rpi = 512 // 64
        part = np.zeros((rpi, 1, 2, 64), np.float32)
        for j, r in enumerate(rows):
            if r >= 0 and valid[r]:
                part[j % rpi] = (part[j % rpi] + x[:, :, r]).astype(np.float32)
        acc = part[0]
        for g in range(1, rpi):
            acc = (acc + part[g]).astype(np.float32)
        assert np.array_equal(mean[:, :, n], (acc / np.float32(max(len(ok), 1))).astype(np.float32))
    # unmasked pooling of an unpadded grid is the plain chunk mean (mean_pooling_compression)
    g2 = (4, 4, 8)
    x2 = rng.standard_normal((1, 1, 128, 64)).astype(np.float32)
    s2 = O.chunk_source_index(g2, g2, (4, 4, 4))
    m2, c2 = O.chunk_pool(x2, s2, None, 64, 2)
    assert (c2 == 64).all()
    np.testing.assert_allclose(m2[0, 0], x2[0, 0][s2].reshape(2, 64, 64).astype(np.float64).mean(1), rtol=1e-5,
                               atol=1e-6)


def test_rect_scores_and_transpose():
    rng = np.random.default_rng(6)
    qc = rng.standard_normal((2, 7, 64)).astype(np.float32)
    kc = rng.standard_normal((2, 11, 64)).astype(np.float32)
    s = O.block_scores(qc, kc, None)
    assert s.shape == (2, 7, 11)
    np.testing.assert_allclose(s, np.einsum("bid,bjd->bij", qc.astype(np.float64), kc.astype(np.float64)),
                               rtol=1e-5, atol=1e-5)
    # a row block of the rectangular product equals the square product's rows
    sq = O.block_scores(qc[:, :7], kc[:, :7], None)
    assert np.array_equal(s[:, :, :7], sq)
    BH, Ntq, Ntk = 2, 6, 10
    qlen = rng.integers(0, Ntk + 1, BH * Ntq).astype(np.int32)
    qstart = np.arange(BH * Ntq, dtype=np.int64) * Ntk
    qcols = np.full(BH * Ntq * Ntk, -1, np.int32)
    lists = []
    for r in range(BH * Ntq):
        li = np.sort(rng.choice(Ntk, qlen[r], replace=False))
        qcols[r * Ntk: r * Ntk + qlen[r]] = li
        lists.append(set(li.tolist()))
    kcols, klen = O.transpose_lists(qstart, qlen, qcols, BH, Ntq, Ntk)
    assert kcols.shape == (BH * Ntk, Ntq)
    for bh in range(BH):
        for kt in range(Ntk):
            want = [t for t in range(Ntq) if kt in lists[bh * Ntq + t]]
            row = bh * Ntk + kt
            assert kcols[row, : klen[row]].tolist() == want


def test_uniform_pipeline_lists():
    """Tile lists of the uniform pipeline: each query tile carries the tiles
    of its chunk's selected key chunks (fully padded key tiles dropped), row
    padding tiles carry nothing."""
    rng = np.random.default_rng(8)
    qg, kg = (1, 1, 200), (5, 8, 8)  # 1-D queries (padded to 256) over 3-D keys (padded to 8x8x8)
    q = rng.standard_normal((1, 2, 200, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 320, 64)).astype(np.float32)
    r = O.uniform_pipeline(q, k, qg, kg, (1, 1, 64), (4, 4, 8), sparsity=0.5, q_pad_rows=256)
    sq, sk = r["q"], r["k"]
    assert sq["Nt"] == 4 and sk["Nt"] == 8 and sk["nb"] == 4
    assert sk["masked"] and sq["masked"]
    for bh in range(2):
        for t in range(sq["Nt"]):
            row = bh * sq["Nt"] + t
            got = r["qcols"][r["qstart"][row]: r["qstart"][row] + r["qlen"][row]].tolist()
            blocks = r["sel"][bh * sq["nb"] + t, : r["nsel"][bh * sq["nb"] + t]]
            want = sorted(tt for b in blocks for tt in (2 * b, 2 * b + 1) if sk["tile_count"][tt] > 0)
            assert got == want
