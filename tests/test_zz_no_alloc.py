"""prism_transpose_lists_noalloc (the allocation-free variant of the list
transpose: bitmap in the library's device workspace) against
prism_transpose_lists (caller workspace), through the C-ABI: bit-identical
lengths, starts and lists on consecutive calls of decreasing size, covering
the batched-heads path (a head's bitmap is half the workspace), the
LDS-column path and the zero-filled global-atomic path (more than 16,384 key
tiles); on two calls issued back to back on two streams (the library orders
them on the workspace); on replays of a captured graph with eager calls in
between; and the size check."""
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


def _outputs(BH, Ntq, Ntk):
    """kstart, klen, kcols filled with -1 on the current stream."""
    return (torch.full((BH * Ntk,), -1, device=DEV, dtype=torch.int64),
            torch.full((BH * Ntk,), -1, device=DEV, dtype=torch.int32),
            torch.full((BH * Ntk * Ntq,), -1, device=DEV, dtype=torch.int32))


def _call(name, lists, outs, BH, Ntq, Ntk):
    """Enqueue one transpose on the current stream (the workspace variant
    allocates its bitmap there)."""
    from prism_amd import ops
    qstart, qlen, qcols = lists
    kstart, klen, kcols = outs
    if name == "prism_transpose_lists":
        words = (Ntq + 31) // 32
        bitmap = torch.empty(BH * Ntk * words, device=DEV, dtype=torch.int32)
        ops._lib.call(name, qstart.data_ptr(), qlen.data_ptr(), qcols.data_ptr(), BH, Ntq, Ntk, bitmap.data_ptr(),
                      Ntq, kstart.data_ptr(), klen.data_ptr(), kcols.data_ptr(), ops._stream())
    else:
        ops._lib.call(name, qstart.data_ptr(), qlen.data_ptr(), qcols.data_ptr(), BH, Ntq, Ntk, Ntq,
                      kstart.data_ptr(), klen.data_ptr(), kcols.data_ptr(), ops._stream())


def _fetch(outs, BH, Ntq, Ntk):
    torch.cuda.synchronize()
    kstart, klen, kcols = outs
    return kstart.cpu().numpy(), klen.cpu().numpy(), kcols.cpu().numpy().reshape(BH * Ntk, Ntq)


def _transpose(name, lists, BH, Ntq, Ntk):
    outs = _outputs(BH, Ntq, Ntk)
    _call(name, lists, outs, BH, Ntq, Ntk)
    return _fetch(outs, BH, Ntq, Ntk)


def _assert_same(ref, got):
    """Equal lengths and starts, equal live entries of every list."""
    ks_a, kl_a, kc_a = ref
    ks_b, kl_b, kc_b = got
    assert np.array_equal(kl_a, kl_b) and np.array_equal(ks_a, ks_b)
    live = np.arange(kc_a.shape[1])[None, :] < kl_a[:, None]
    assert np.array_equal(np.where(live, kc_a, 0), np.where(live, kc_b, 0))


def test_transpose_lists_noalloc_matches_workspace_variant():
    rng = np.random.default_rng(0)
    # (BH, Ntq, Ntk, density): decreasing sizes; the first needs two heads per
    # workspace batch (5760 x 180 words per head), the last has more than
    # 16,384 key tiles (zero-filled bitmap, global atomics)
    for BH, Ntq, Ntk, dens in ((5, 5760, 5760, 0.03), (2, 640, 512, 0.2), (1, 64, 20000, 0.01)):
        print("[case] noalloc transpose", BH, Ntq, Ntk, dens, flush=True)
        lists = _lists(rng, BH, Ntq, Ntk, dens)
        ref = _transpose("prism_transpose_lists", lists, BH, Ntq, Ntk)
        assert int(ref[1].sum()) == int(lists[1].sum())
        _assert_same(ref, _transpose("prism_transpose_lists_noalloc", lists, BH, Ntq, Ntk))
        # a second call on the same (reused) workspace gives the same lists
        _assert_same(ref, _transpose("prism_transpose_lists_noalloc", lists, BH, Ntq, Ntk))


def test_transpose_lists_noalloc_rejects_oversized_heads():
    from prism_amd import ops
    x = torch.zeros(4, device=DEV, dtype=torch.int64)
    # one head of 20,000 x 20,000 tiles needs 20,000 * 625 words > 2^21
    with pytest.raises(ValueError, match="workspace"):
        ops._lib.call("prism_transpose_lists_noalloc", x.data_ptr(), x.data_ptr(), x.data_ptr(), 1, 20000, 20000,
                      20000, x.data_ptr(), x.data_ptr(), x.data_ptr(), ops._stream())


def test_transpose_lists_noalloc_orders_calls_on_two_streams():
    """Two calls enqueued back to back on two streams, with different inputs
    (the first takes three workspace batches): the second call's stream waits
    for the first call's event, so neither overwrites the other's bitmap."""
    rng = np.random.default_rng(1)
    cases = ((5, 5760, 5760, 0.03), (3, 1440, 4000, 0.1))
    lists = [_lists(rng, *c) for c in cases]
    refs = [_transpose("prism_transpose_lists", li, *c[:3]) for li, c in zip(lists, cases)]
    streams = (torch.cuda.Stream(), torch.cuda.Stream())
    torch.cuda.synchronize()
    outs = []
    for li, c, st in zip(lists, cases, streams):
        print("[case] noalloc transpose on a second stream", c, flush=True)
        with torch.cuda.stream(st):
            o = _outputs(*c[:3])
            _call("prism_transpose_lists_noalloc", li, o, *c[:3])
        outs.append(o)
    for ref, o, c in zip(refs, outs, cases):
        _assert_same(ref, _fetch(o, *c[:3]))


def test_transpose_lists_noalloc_graph_replays():
    """The call captured into a graph (no event wait or record inside the
    capture) and replayed three times, with an eager call on other inputs
    and a synchronisation between replays: every replay equals the
    workspace variant's lists."""
    rng = np.random.default_rng(2)
    shape, other = (2, 640, 512), (1, 320, 900)
    lists, lists_o = _lists(rng, *shape, 0.2), _lists(rng, *other, 0.1)
    ref = _transpose("prism_transpose_lists", lists, *shape)
    ref_o = _transpose("prism_transpose_lists", lists_o, *other)
    _assert_same(ref, _transpose("prism_transpose_lists_noalloc", lists, *shape))  # set-up outside the capture
    outs = _outputs(*shape)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call("prism_transpose_lists_noalloc", lists, outs, *shape)
    for rep in range(3):
        print("[case] noalloc transpose graph replay", rep, flush=True)
        for t in outs:
            t.fill_(-1)
        g.replay()
        _assert_same(ref, _fetch(outs, *shape))
        _assert_same(ref_o, _transpose("prism_transpose_lists_noalloc", lists_o, *other))
