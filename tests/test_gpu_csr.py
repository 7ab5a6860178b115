"""Compact CSR work lists on the GPU (prism_lists_csr_offsets /
prism_lists_csr_fill, ops.lists_to_csr, ops.select_csr, ops.transpose_csr and
plan_dynamic(compact_lists=True)).

Bit-exact: CSR rows equal the source lists (rows anywhere in the source
buffer, empty rows, a row past the others' capacity); select_csr equals the
oracle's selection expanded to tiles per query tile; transpose_csr equals the
oracle's transpose.  A compact plan gives bit-identical attention outputs and
gradients to a dense one, and after its forward keeps only the two pair
unions, in CSR form, with the dense unions' rows."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.cases import bf16, padded_case
from tests.test_gpu_parity import dev, host, say

pytestmark = pytest.mark.gpu


def test_lists_to_csr_equals_lists():
    from prism_amd import ops
    rng = np.random.default_rng(3)
    rows = 3000
    cap = 50
    buf = rng.integers(0, 1 << 20, rows * cap + 77).astype(np.int32)
    length = rng.integers(0, cap + 1, rows).astype(np.int32)
    length[::7] = 0
    start = (rng.permutation(rows) * cap).astype(np.int64)
    start[5], length[5] = rows * cap, 77  # a row in the buffer's tail
    say("lists_to_csr", rows)
    off, ent = ops.lists_to_csr(dev(start), dev(length), dev(buf))
    off_h, ent_h = host(off), host(ent)
    assert off_h.dtype == np.int32 and off_h[0] == 0 and off_h[-1] == ent_h.size == int(length.sum())
    assert np.array_equal(np.diff(off_h), length)
    for r in range(rows):
        assert np.array_equal(ent_h[off_h[r]: off_h[r + 1]], buf[start[r]: start[r] + length[r]]), r
    s2, l2 = ops.csr_lists(off)
    assert s2.dtype == torch.int64 and np.array_equal(host(l2), length)
    # no rows, and rows that are all empty
    off0, ent0 = ops.lists_to_csr(dev(np.zeros(0, np.int64)), dev(np.zeros(0, np.int32)), dev(buf))
    # (a one-element entry buffer, never read: a non-null pointer for the kernels)
    assert host(off0).tolist() == [0] and ent0.numel() == 1
    off1, ent1 = ops.lists_to_csr(dev(start[:9]), dev(np.zeros(9, np.int32)), dev(buf))
    assert host(off1).tolist() == [0] * 10 and ent1.numel() == 1


@pytest.fixture(scope="module")
def plan_case():
    c = padded_case(4, 1, 3, (13, 20, 24), 128, lowrank=True, audio_tokens=32)
    return c


def test_select_and_transpose_csr_bitexact(plan_case):
    from prism_amd import ops, plan_dynamic
    c = plan_case
    q, k, v = (dev(bf16(c[n])) for n in ("q", "k", "v"))
    p = plan_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.75, cdf_threshold=0.9,
                     audio_token_norms=dev(c["norms"]), valid_mask=dev(c["valid"]).bool(), keep_scores=True)
    lay = p.lay
    BH = p.B * p.H
    sm = 1 / math.sqrt(q.shape[-1])
    say("select_csr")
    off, tiles = ops.select_csr(p.scores, 0.75, 0.9, sm, lay, p.tile_count)
    # the reference lists: the oracle's selection on the same scores, expanded to tiles
    sel, nsel = O.select(host(p.scores).reshape(-1, lay.N_b), 0.75, 0.9, sm)
    bot, kbt, nb, _ = O.tile_maps(host(lay.shape_ids))
    assert nb == lay.N_b
    etiles, ent = O.expand_tiles(sel, nsel, kbt, lay.Nt, host(p.tile_count))
    off_h, tiles_h = host(off), host(tiles)
    assert off_h.size == BH * lay.Nt + 1
    for bh in range(BH):
        for t in range(lay.Nt):
            r = bh * lay.N_b + bot[t]
            got = tiles_h[off_h[bh * lay.Nt + t]: off_h[bh * lay.Nt + t + 1]]
            assert np.array_equal(got, etiles[r, : ent[r]]), (bh, t)
    say("transpose_csr")
    koff, kq = ops.transpose_csr(off, tiles, BH, lay.Nt)
    qs, ql = ops.csr_lists(off)
    ref_c, ref_l = O.transpose_lists(host(qs), host(ql), tiles_h, BH, lay.Nt)
    koff_h, kq_h = host(koff), host(kq)
    assert np.array_equal(np.diff(koff_h), ref_l)
    for r in range(BH * lay.Nt):
        assert np.array_equal(kq_h[koff_h[r]: koff_h[r + 1]], ref_c[r, : ref_l[r]]), r


def test_compact_plan_identical_and_smaller(plan_case):
    from prism_amd import flash_attn_bsa_3d_dynamic, plan_dynamic
    c = plan_case
    outs = []
    for compact in (False, True):
        say("compact_lists", compact)
        q, k, v = (dev(bf16(c[n])).requires_grad_(True) for n in ("q", "k", "v"))
        o = flash_attn_bsa_3d_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.75, cdf_threshold=0.9,
                                      audio_token_norms=dev(c["norms"]), valid_mask=dev(c["valid"]).bool(),
                                      compact_lists=compact)
        g = torch.randn_like(o, generator=torch.Generator(device="cuda").manual_seed(9))
        o.backward(g)
        outs.append([host(t) for t in (o, q.grad, k.grad, v.grad)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    # list memory the plan keeps from the forward to the backward (after
    # settle(), as the forward leaves it): the per-tile lists are released,
    # the pair unions stay as dense buffers or compact CSR with the same rows
    q, k, v = (dev(bf16(c[n])) for n in ("q", "k", "v"))
    sizes, unions = [], []
    for compact in (False, True):
        p = plan_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.75, cdf_threshold=0.9,
                         audio_token_norms=dev(c["norms"]), valid_mask=dev(c["valid"]).bool(), compact_lists=compact)
        p.build_key_lists()
        peak = p.list_bytes()
        p.settle()
        assert p.qcols is None and p.klists is None and "tiles" not in p.sel
        sizes.append(p.list_bytes())
        assert sizes[-1] < peak
        unions.append([[host(t) for t in u] for u in (p.qunion, p.kunion)])
        if compact:
            # O(nnz): every kept union buffer holds exactly its entries
            assert p.qunion[2].numel() == int(p.qunion[1].sum().item())
            assert p.kunion[2].numel() == int(p.kunion[1].sum().item())
    for (s0, l0, c0), (s1, l1, c1) in zip(*unions):
        assert np.array_equal(l0, l1)
        for r in range(l0.size):
            assert np.array_equal(c0[s0[r]: s0[r] + l0[r]], c1[s1[r]: s1[r] + l1[r]]), r
    say("list bytes kept: dense", sizes[0], "compact", sizes[1])
    assert sizes[1] < sizes[0]


def test_compact_uniform_identical(plan_case):
    """The uniform-shape branch (run_bsa_uniform) with compact lists: same
    output and gradients as with the dense lists."""
    from prism_amd.adapter import run_bsa_uniform
    c = plan_case
    outs = []
    for compact in (False, True):
        say("uniform compact_lists", compact)
        q, k, v = (dev(bf16(c[n])).requires_grad_(True) for n in ("q", "k", "v"))
        o = run_bsa_uniform(q, k, v, c["grid"], {"sparsity": 0.75, "cdf_threshold": 0.9,
                                                      "compact_lists": compact})
        o.backward(torch.ones_like(o) * 0.01)
        outs.append([host(t) for t in (o, q.grad, k.grad, v.grad)])
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def test_autograd_forward_keeps_only_compact_unions(plan_case):
    """Through autograd (flash_attn_bsa_3d_dynamic with gradients), the plan
    the backward holds has released its per-tile lists and keeps the two pair
    unions as CSR (each entry buffer exactly the union sizes), by default."""
    from prism_amd import flash_attn_bsa_3d_dynamic
    c = plan_case
    q, k, v = (dev(bf16(c[n])).requires_grad_(True) for n in ("q", "k", "v"))
    o = flash_attn_bsa_3d_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.75, cdf_threshold=0.9,
                                  audio_token_norms=dev(c["norms"]), valid_mask=dev(c["valid"]).bool())
    plan = o.grad_fn.plan
    assert plan.qcols is None and plan.klists is None and "tiles" not in plan.sel
    for u in (plan.qunion, plan.kunion):
        assert u[2].numel() == int(u[1].sum().item())
    o.backward(torch.ones_like(o))
    assert all(bool(torch.isfinite(t.grad).all()) for t in (q, k, v))
