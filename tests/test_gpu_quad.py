"""The quad forward (prism_bsa_fwd_quad over prism_quad_union lists, one
8-wave workgroup per four query tiles) against the pair forward
(prism_bsa_fwd over prism_pair_union lists) on the same per-query-tile key
lists: every query row walks its own list in the same order with the same
arithmetic, so O and LSE must agree bit for bit.  Cases: D = 64 and 128,
padded grids (partial key tiles) and unpadded, a launch order and none,
lists with empty rows, and config 4's full-size lists."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.test_gpu_parity import CASES, bits_equal, dev, host, make, say

pytestmark = pytest.mark.gpu


def _quad_vs_pair(plan, D, with_order=True):
    from prism_amd import ops
    sm = 1.0 / math.sqrt(D)
    o1, l1 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    quad = ops.quad_union(plan.qstart, plan.qlen, plan.qcols, plan.lay.Nt, plan.tmasks, pairmap=plan.qpair)
    order = ops.pair_order(quad[1], 32) if with_order else None
    o2, l2 = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, order)
    torch.cuda.synchronize()
    assert bits_equal(host(o2), host(o1)), "O"
    assert bits_equal(host(l2), host(l1)), "LSE"
    return quad


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_quad_forward_bitexact_vs_pair(case):
    from prism_amd import plan_dynamic
    c = make(case)
    say("quad", case)
    valid = c["valid"] if c["pad"] else None
    D = c["q"].shape[-1]
    plan = plan_dynamic(dev(c["qh"]), dev(c["kh"]), dev(c["vh"]), c["grid"], method="ivpq", sparsity=0.6,
                        cdf_threshold=0.9, valid_mask=None if valid is None else dev(valid).bool())
    quad = _quad_vs_pair(plan, D)
    _quad_vs_pair(plan, D, with_order=False)
    # the quad lists are the unions of the quads' four tile lists, member bits
    # and partial flags as the oracle's pair unions of the two pairs
    qs, ql, qc = (host(t) for t in quad)
    pm = host(plan.qpair)
    st, ln, cl = host(plan.qstart), host(plan.qlen), host(plan.qcols)
    Nt = plan.lay.Nt
    masks = None if plan.tmasks is None else host(plan.tmasks).view(np.uint64)
    for qd in range(min(ql.size, 64)):
        bh, qq = divmod(qd, Nt // 4)
        tiles = [bh * Nt + int(pm[bh * Nt + 4 * qq + k]) for k in range(4)]
        want = {}
        for k, r in enumerate(tiles):
            for t in cl[st[r]: st[r] + ln[r]]:
                want[int(t)] = want.get(int(t), 0) | (1 << k)
        ents = qc[qs[qd]: qs[qd] + ql[qd]]
        assert [int(e) >> 5 for e in ents] == sorted(want), qd
        for e in ents:
            t = int(e) >> 5
            assert int(e) & 15 == want[t], (qd, t)
            partial = masks is not None and masks[t] != np.uint64(0xFFFFFFFFFFFFFFFF)
            assert bool(int(e) & 16) == bool(partial), (qd, t)


def test_quad_forward_bitexact_fullsize_c4():
    """Config 4's lists (as benchmarked): the quad and pair forwards agree bit
    for bit over all 14,400 pairs."""
    import bench
    from prism_amd import ops, plan_dynamic, a2v_token_norms
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import _gradient_and_shapes
    from tests.test_gpu_fullsize import _sparsity
    say("quad fullsize c4: inputs")
    inp = bench.make_inputs("c4")
    grid = inp["grid"]
    gp, _ = padded_grid(grid)
    with torch.no_grad():
        norms = a2v_token_norms(inp["res"])
        sid = _gradient_and_shapes(inp["v"], norms, gp, "ivpq", 0.5, 0.15, 1.0, None, grid)[2]
        sp, cdf = _sparsity(inp, ops.ZoneLayout(sid, gp, grid).N_b)
        plan = plan_dynamic(inp["q"], inp["k"], inp["v"], gp, method="ivpq", sparsity=sp, cdf_threshold=cdf,
                            audio_token_norms=norms, input_grid=grid)
    say("quad fullsize c4: attention")
    _quad_vs_pair(plan, inp["D"])
