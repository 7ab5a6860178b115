"""prism_transpose_lists_noalloc (the allocation-free variant of the list
transpose: bitmap in the library's device workspace) against
prism_transpose_lists (caller workspace), through the C-ABI: bit-identical
lengths, starts and lists on consecutive calls of decreasing size, covering
the batched-heads path (a head's bitmap is half the workspace), the
LDS-column path and the zero-filled global-atomic path (more than 16,384 key
tiles), and the size check."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lists(rng, BH, Ntq, Ntk, density):
    """Random ascending key-tile lists per query tile: (qstart, qlen, qcols)
    on the GPU, row r at offset r * Ntk (some rows empty)."""
    qlen = np.zeros(BH * Ntq, np.int32)
    qcols = np.zeros(BH * Ntq * Ntk, np.int32)
    for r in range(BH * Ntq):
        if r % 17 == 3:
            continue  # an empty list
        cols = np.nonzero(rng.random(Ntk) < density)[0].astype(np.int32)
        qlen[r] = len(cols)
        qcols[r * Ntk: r * Ntk + len(cols)] = cols
    qstart = np.arange(BH * Ntq, dtype=np.int64) * Ntk
    to = lambda a: torch.from_numpy(a).to(DEV)
    return to(qstart), to(qlen), to(qcols)


def _transpose(name, lists, BH, Ntq, Ntk):
    from prism_amd import ops
    qstart, qlen, qcols = lists
    kstart = torch.full((BH * Ntk,), -1, device=DEV, dtype=torch.int64)
    klen = torch.full((BH * Ntk,), -1, device=DEV, dtype=torch.int32)
    kcols = torch.full((BH * Ntk * Ntq,), -1, device=DEV, dtype=torch.int32)
    if name == "prism_transpose_lists":
        words = (Ntq + 31) // 32
        bitmap = torch.empty(BH * Ntk * words, device=DEV, dtype=torch.int32)
        ops._lib.call(name, qstart.data_ptr(), qlen.data_ptr(), qcols.data_ptr(), BH, Ntq, Ntk, bitmap.data_ptr(),
                      Ntq, kstart.data_ptr(), klen.data_ptr(), kcols.data_ptr(), ops._stream())
    else:
        ops._lib.call(name, qstart.data_ptr(), qlen.data_ptr(), qcols.data_ptr(), BH, Ntq, Ntk, Ntq,
                      kstart.data_ptr(), klen.data_ptr(), kcols.data_ptr(), ops._stream())
    torch.cuda.synchronize()
    return kstart.cpu().numpy(), klen.cpu().numpy(), kcols.cpu().numpy().reshape(BH * Ntk, Ntq)


def test_transpose_lists_noalloc_matches_workspace_variant():
    rng = np.random.default_rng(0)
    # (BH, Ntq, Ntk, density): decreasing sizes; the first needs two heads per
    # workspace batch (5760 x 180 words per head), the last has more than
    # 16,384 key tiles (zero-filled bitmap, global atomics)
    for BH, Ntq, Ntk, dens in ((5, 5760, 5760, 0.03), (2, 640, 512, 0.2), (1, 64, 20000, 0.01)):
        print("[case] noalloc transpose", BH, Ntq, Ntk, dens, flush=True)
        lists = _lists(rng, BH, Ntq, Ntk, dens)
        ks_a, kl_a, kc_a = _transpose("prism_transpose_lists", lists, BH, Ntq, Ntk)
        ks_b, kl_b, kc_b = _transpose("prism_transpose_lists_noalloc", lists, BH, Ntq, Ntk)
        assert np.array_equal(kl_a, kl_b) and np.array_equal(ks_a, ks_b)
        assert int(kl_a.sum()) == int(lists[1].sum())
        for r in range(BH * Ntk):
            assert np.array_equal(kc_a[r, : kl_a[r]], kc_b[r, : kl_b[r]]), r
        # a second call on the same (reused) workspace gives the same lists
        ks_c, kl_c, kc_c = _transpose("prism_transpose_lists_noalloc", lists, BH, Ntq, Ntk)
        assert np.array_equal(kl_c, kl_a) and np.array_equal(ks_c, ks_a)
        live = np.arange(Ntq)[None, :] < kl_a[:, None]
        assert np.array_equal(np.where(live, kc_c, 0), np.where(live, kc_a, 0))


def test_transpose_lists_noalloc_rejects_oversized_heads():
    from prism_amd import ops
    x = torch.zeros(4, device=DEV, dtype=torch.int64)
    # one head of 20,000 x 20,000 tiles needs 20,000 * 625 words > 2^21
    with pytest.raises(ValueError, match="workspace"):
        ops._lib.call("prism_transpose_lists_noalloc", x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 20000, 20000,
                      20000, x.data_ptr(), x.data_ptr(), x.data_ptr(), ops._stream())
