"""The quad kernels (prism_bsa_fwd_quad and prism_bsa_bwd_dq_quad over
prism_quad_union lists, one 8-wave workgroup per four query tiles) against
the pair kernels (prism_bsa_fwd, prism_bsa_bwd_dq over prism_pair_union
lists) on the same per-query-tile key lists: every query row walks its own
list in the same order with the same arithmetic, so O, LSE and dQ must agree
bit for bit.  Cases: D = 64 and 128, padded grids (partial key tiles) and
unpadded, a launch order and none, lists with empty rows, config 4's
full-size lists, and the autograd path with quads on and off."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.test_gpu_parity import CASES, bits_equal, dev, host, make, say

pytestmark = pytest.mark.gpu


def _quad_vs_pair(plan, D, with_order=True, seed=5):
    from prism_amd import ops
    sm = 1.0 / math.sqrt(D)
    o1, l1 = ops.bsa_fwd(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, plan.qunion, sm, plan.qpair, plan.qorder)
    quad = ops.quad_union(plan.qstart, plan.qlen, plan.qcols, plan.lay.Nt, plan.tmasks, pairmap=plan.qpair)
    order = ops.pair_order(quad[1], 32) if with_order else None
    o2, l2 = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, order)
    torch.cuda.synchronize()
    assert bits_equal(host(o2), host(o1)), "O"
    assert bits_equal(host(l2), host(l1)), "LSE"
    # dQ over the quads against dQ over the pairs (dK / dV: the same launch)
    plan.build_key_lists()
    do = torch.randn(plan.q_re.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(seed))
    do = do.to(torch.bfloat16)
    m2, delta = ops.lse_to_m2(l1), ops.bwd_preprocess(o1, do)
    g1 = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do, m2, delta, plan.kv_valid, plan.tmasks, plan.qunion,
                     plan.kunion, sm, plan.qpair, plan.kpair, plan.qorder, plan.korder)
    g2 = ops.bsa_bwd(plan.q_re, plan.k_re, plan.v_re, do, m2, delta, plan.kv_valid, plan.tmasks, quad,
                     plan.kunion, sm, plan.qpair, plan.kpair, order, plan.korder, q_quads=True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), g2, g1):
        assert bits_equal(host(a), host(b)), name
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


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4"])
def test_quad_forward_bitexact_fullsize(cfg):
    """Configs 2-4 at full size (the benchmark's inputs and lists): the quad
    and pair forwards and dQ agree bit for bit over every quad."""
    import bench
    from prism_amd import ops, plan_dynamic, a2v_token_norms
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import _gradient_and_shapes
    from tests.test_gpu_fullsize import _sparsity
    say("quad fullsize", cfg, "inputs")
    inp = bench.make_inputs(cfg)
    grid = inp["grid"]
    gp, _ = padded_grid(grid)
    with torch.no_grad():
        norms = a2v_token_norms(inp["res"])
        sid = _gradient_and_shapes(inp["v"], norms, gp, "ivpq", 0.5, 0.15, 1.0, None, grid)[2]
        sp, cdf = _sparsity(inp, ops.ZoneLayout(sid, gp, grid).N_b)
        plan = plan_dynamic(inp["q"], inp["k"], inp["v"], gp, method="ivpq", sparsity=sp, cdf_threshold=cdf,
                            audio_token_norms=norms, input_grid=grid)
    say("quad fullsize", cfg, "attention")
    _quad_vs_pair(plan, inp["D"])


# (ops.QUADS, ops.DQ_QUADS); None: the path's default (dQ on quads on the
# dynamic-shape path, on pairs on the uniform and cross paths)
SWITCHES = ((False, False), (True, False), (True, True), (True, None))


@pytest.mark.parametrize("case", [CASES[0], CASES[-1]], ids=[CASES[0][0], CASES[-1][0]])
def test_quads_autograd_identical(case, monkeypatch):
    """flash_attn_bsa_3d_dynamic with the forward on pairs, on quads, the
    forward and dQ on quads, and the defaults: the same output and q, k, v
    gradients, bit for bit."""
    from prism_amd import flash_attn_bsa_3d_dynamic, ops
    c = make(case)
    say("quads autograd", case)
    valid = dev(c["valid"]).bool() if c["pad"] else None
    outs = []
    for quads, dq_quads in SWITCHES:
        monkeypatch.setattr(ops, "QUADS", quads)
        monkeypatch.setattr(ops, "DQ_QUADS", dq_quads)
        q, k, v = (dev(c[n]).requires_grad_(True) for n in ("qh", "kh", "vh"))
        o = flash_attn_bsa_3d_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.6, cdf_threshold=0.9,
                                      valid_mask=valid)
        plan = o.grad_fn.plan
        want_dq = quads and dq_quads is not False
        assert plan.lay.Nt % 4 == 0 and plan.quads == quads and plan.dq_quads == want_dq
        assert (plan.qquad is not None) == want_dq  # kept for the backward only when dQ walks it
        o.backward(torch.randn(o.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(3))
                   .to(o.dtype))
        outs.append([host(t) for t in (o, q.grad, k.grad, v.grad)])
    for other in outs[1:]:
        for name, a, b in zip(("O", "dQ", "dK", "dV"), outs[0], other):
            assert bits_equal(a, b), name


def test_quads_uniform_and_cross_identical(monkeypatch):
    """The uniform-shape branch (run_bsa_uniform, padded grid) and the
    cross-modal BSA (flash_attn_bsa_cross, audio queries over video keys)
    with the forward on pairs, on quads, and the forward and dQ on quads: the
    same output and gradients, bit for bit."""
    from prism_amd import ops
    from prism_amd.adapter import run_bsa_uniform
    from prism_amd.uniform_block_attention import flash_attn_bsa_cross
    from tests.cases import bf16 as to_bf16
    rng = np.random.default_rng(23)
    D = 128
    grid = (7, 16, 16)
    qh, kh, vh = (to_bf16(rng.standard_normal((1, 2, int(np.prod(grid)), D)).astype(np.float32)) for _ in range(3))
    aq = to_bf16(rng.standard_normal((1, 2, 460, D)).astype(np.float32))  # 8 query tiles, the last partial
    calls = {
        "uniform": (lambda q, k, v: run_bsa_uniform(q, k, v, grid, {"sparsity": 0.6, "cdf_threshold": 0.9}),
                    (qh, kh, vh)),
        "cross": (lambda q, k, v: flash_attn_bsa_cross(q, k, v, "1d", "3d", k_grid_size=grid, chunk_size_q=64,
                                                       chunk_3d_shape_k=(4, 4, 4), sparsity=0.5),
                  (aq, kh, vh)),
    }
    for name, (fn, arrays) in calls.items():
        outs = []
        for quads, dq_quads in SWITCHES:
            say("quads", name, quads, dq_quads)
            monkeypatch.setattr(ops, "QUADS", quads)
            monkeypatch.setattr(ops, "DQ_QUADS", dq_quads)
            q, k, v = (dev(a).requires_grad_(True) for a in arrays)
            o = fn(q, k, v)
            assert o.grad_fn.plan.quads == quads and o.grad_fn.plan.dq_quads == (quads and dq_quads is True), name
            o.backward(torch.randn(o.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(4))
                       .to(o.dtype))
            outs.append([host(t) for t in (o, q.grad, k.grad, v.grad)])
        for other in outs[1:]:
            for what, a, b in zip(("O", "dQ", "dK", "dV"), outs[0], other):
                assert bits_equal(a, b), (name, what)


def test_quad_debug_mode_checks_lists(monkeypatch):
    """PRISM_DEBUG=1: prism_bsa_fwd_quad and prism_bsa_bwd_dq_quad check their
    quad unions and maps on the host before launching.  Valid lists give the
    same bits as without the checks; corrupted ones (kept inside the operands'
    bounds) raise ValueError naming the defect."""
    from prism_amd import ops, plan_dynamic
    case = CASES[1]
    c = make(case)
    say("quad debug", case)
    D = c["q"].shape[-1]
    sm = 1.0 / math.sqrt(D)
    plan = plan_dynamic(dev(c["qh"]), dev(c["kh"]), dev(c["vh"]), c["grid"], method="ivpq", sparsity=0.6,
                        cdf_threshold=0.9, valid_mask=dev(c["valid"]).bool() if c["pad"] else None)
    quad = ops.quad_union(plan.qstart, plan.qlen, plan.qcols, plan.lay.Nt, plan.tmasks, pairmap=plan.qpair)
    order = ops.pair_order(quad[1], 32)
    o, lse = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, order)
    do = torch.randn(plan.q_re.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(8))
    do = do.to(torch.bfloat16)
    m2, delta = ops.lse_to_m2(lse), ops.bwd_preprocess(o, do)
    dq_args = lambda u, om: (plan.q_re, plan.k_re, plan.v_re, do, m2, delta, plan.tmasks, *u, plan.qpair, om, sm)
    dq = torch.ops.prism.bsa_bwd_dq_quad(*dq_args(quad, order))
    monkeypatch.setenv("PRISM_DEBUG", "1")
    say("quad debug: valid lists")
    o2, lse2 = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, order)
    dq2 = torch.ops.prism.bsa_bwd_dq_quad(*dq_args(quad, order))
    assert bits_equal(host(o), host(o2)) and bits_equal(host(lse), host(lse2)) and bits_equal(host(dq), host(dq2))
    us, ul, uc = quad
    r = int(torch.nonzero(ul >= 2)[0, 0])
    s = int(us[r])
    bad = uc.clone()
    bad[s] = bad[s] & ~15  # an entry that belongs to no tile of its quad
    say("quad debug: entry without member bits")
    with pytest.raises(ValueError, match="belongs to no tile of its quad"):
        ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, (us, ul, bad), sm, plan.qpair, order)
    bad = uc.clone()
    bad[s], bad[s + 1] = uc[s + 1], uc[s]
    say("quad debug: descending entries in dQ")
    with pytest.raises(ValueError, match="not above"):
        torch.ops.prism.bsa_bwd_dq_quad(*dq_args((us, ul, bad), order))
    bad_order = order.clone()
    bad_order[1] = bad_order[0]
    say("quad debug: launch order with a repeated quad")
    with pytest.raises(ValueError, match="twice"):
        ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, bad_order)
    torch.cuda.synchronize()


@pytest.mark.parametrize("case", [CASES[0], CASES[-1]], ids=[CASES[0][0], CASES[-1][0]])
def test_quad_work_queue_bit_identical(case):
    """prism_bsa_fwd_quad and prism_bsa_bwd_dq_quad through the C-ABI with
    work_counter = NULL (one workgroup per quad) and with a counter
    (persistent workgroups over the per-XCD work queues; the counter starts
    with garbage, which the call clears, and is reused by the next call):
    the same bits as the operators."""
    from prism_amd import ops, plan_dynamic
    c = make(case)
    say("quad work queue", case)
    q = dev(c["qh"])
    B, H, S, D = q.shape
    BH, sm = B * H, 1.0 / math.sqrt(D)
    plan = plan_dynamic(q, dev(c["kh"]), dev(c["vh"]), c["grid"], method="ivpq", sparsity=0.6, cdf_threshold=0.9,
                        valid_mask=dev(c["valid"]).bool() if c["pad"] else None)
    Sp = plan.q_re.shape[2]
    quad = ops.quad_union(plan.qstart, plan.qlen, plan.qcols, plan.lay.Nt, plan.tmasks, pairmap=plan.qpair)
    order = ops.pair_order(quad[1], 32)
    o, lse = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, order)
    do = torch.randn(plan.q_re.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(9))
    do = do.to(plan.q_re.dtype)
    m2, delta = ops.lse_to_m2(lse), ops.bwd_preprocess(o, do)
    dq = torch.ops.prism.bsa_bwd_dq_quad(plan.q_re, plan.k_re, plan.v_re, do, m2, delta, plan.tmasks, *quad,
                                         plan.qpair, order, sm)
    ptr = lambda t: None if t is None else t.data_ptr()
    stream = torch.cuda.current_stream().cuda_stream
    counter = torch.full((8,), 12345, dtype=torch.int32, device="cuda")
    for ctr in (None, counter, counter):
        say("quad work queue: counter", ctr is not None)
        o2, lse2, dq2 = torch.empty_like(o), torch.empty_like(lse), torch.empty_like(dq)
        ops._lib.call("prism_bsa_fwd_quad", ptr(plan.q_re), ptr(plan.k_re), ptr(plan.v_re), BH, Sp, Sp, D,
                      ptr(plan.tmasks), *(ptr(t) for t in quad), ptr(plan.qpair), ptr(order), sm, ptr(o2), ptr(lse2),
                      ptr(ctr), stream)
        if ctr is not None:
            counter.fill_(-7)  # garbage again: the dQ call clears it too
        ops._lib.call("prism_bsa_bwd_dq_quad", ptr(plan.q_re), ptr(plan.k_re), ptr(plan.v_re), ptr(do), ptr(m2),
                      ptr(delta), BH, Sp, Sp, D, ptr(plan.tmasks), *(ptr(t) for t in quad), ptr(plan.qpair),
                      ptr(order), sm, ptr(dq2), ptr(ctr), stream)
        torch.cuda.synchronize()
        assert bits_equal(host(o), host(o2)) and bits_equal(host(lse), host(lse2)) and bits_equal(host(dq), host(dq2))


def test_quad_graph_capture_replays():
    """The quad forward and dQ over a prebuilt plan, captured in one HIP graph
    (persistent launches with their counter-zeroing kernels, outputs and
    counters from the graph's memory pool): three replays, with eager work
    and synchronisations between them, each give the eager bits."""
    from prism_amd import ops, plan_dynamic
    c = make(CASES[-1])
    say("quad graph capture")
    D = c["q"].shape[-1]
    sm = 1.0 / math.sqrt(D)
    plan = plan_dynamic(dev(c["qh"]), dev(c["kh"]), dev(c["vh"]), c["grid"], method="ivpq", sparsity=0.6,
                        cdf_threshold=0.9)
    quad = ops.quad_union(plan.qstart, plan.qlen, plan.qcols, plan.lay.Nt, plan.tmasks, pairmap=plan.qpair)
    order = ops.pair_order(quad[1], 32)
    do = torch.randn(plan.q_re.shape, device="cuda", generator=torch.Generator(device="cuda").manual_seed(10))
    do = do.to(plan.q_re.dtype)

    def step():
        o, lse = ops.bsa_fwd_quad(plan.q_re, plan.k_re, plan.v_re, plan.tmasks, quad, sm, plan.qpair, order)
        m2, delta = ops.lse_to_m2(lse), ops.bwd_preprocess(o, do)
        dq = torch.ops.prism.bsa_bwd_dq_quad(plan.q_re, plan.k_re, plan.v_re, do, m2, delta, plan.tmasks, *quad,
                                             plan.qpair, order, sm)
        return o, lse, dq

    ref = [host(t) for t in step()]
    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        step()
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for rep in range(3):
        say("quad graph replay", rep)
        junk = torch.full((1 << 20,), float(rep), device="cuda").cumsum(0)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, t, r in zip(("O", "LSE", "dQ"), outs, ref):
            assert bits_equal(host(t), r), (rep, name)
        del junk
