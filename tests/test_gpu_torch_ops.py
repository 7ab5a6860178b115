"""torch.library.opcheck of the prism operators (TORCH_LIBRARY(prism)) on the
GPU: schema (no input mutated or aliased) and fake-tensor agreement (the fake
implementation's shapes, dtypes and strides equal the kernels' outputs), on
the arguments of a small dynamic-path plan."""
import math

import pytest
import torch

from tests.cases import bf16, padded_case
from tests.test_gpu_parity import dev

pytestmark = pytest.mark.gpu
UTILS = ("test_schema", "test_faketensor")


@pytest.fixture(scope="module")
def plan():
    from prism_amd import plan_dynamic
    c = padded_case(3, 1, 2, (13, 20, 24), 128, lowrank=True, audio_tokens=32)
    q, k, v = (dev(bf16(c[n])) for n in ("q", "k", "v"))
    p = plan_dynamic(q, k, v, c["grid"], method="ivpq", sparsity=0.6, cdf_threshold=0.9,
                     audio_token_norms=dev(c["norms"]), valid_mask=dev(c["valid"]).bool(), keep_scores=True)
    return c, p


def _check(op, *args):
    print("[case] opcheck", op, flush=True)
    torch.library.opcheck(getattr(torch.ops.prism, op).default, args, test_utils=UTILS)


def test_opcheck_statistics_and_geometry(plan):
    c, p = plan
    lay = p.lay
    grid = list(lay.grid)
    v = dev(bf16(c["v"]))
    valid = dev(c["valid"])
    _check("zone_stats", v, valid, grid, grid)
    packed, av = torch.ops.prism.zone_stats(v, valid, grid, grid)
    _check("audio_zone_stats", dev(c["norms"]), valid, grid, grid)
    _check("zone_gradient", packed, av, 128)
    rho_raw, aniso = torch.ops.prism.zone_gradient(packed, av, 128)
    _check("zone_shapes", rho_raw, aniso, None, None, 0, 0.5, 0.15, 1.0)
    g, rho, _ = torch.ops.prism.zone_shapes(rho_raw, aniso, None, None, 0, 0.5, 0.15, 1.0)
    _check("assign_shapes", g, rho, 1, 0.15, 1.0)
    _check("a2v_norms", torch.randn(300, 256, device="cuda", dtype=torch.bfloat16))
    xb = torch.randn(300, 128, device="cuda", dtype=torch.bfloat16)
    wt = torch.randn(256, 128, device="cuda", dtype=torch.bfloat16)
    _check("linear_rownorm", xb, wt, torch.randn(256, device="cuda", dtype=torch.bfloat16), 0)
    _check("linear_rownorm", xb, wt, None, 1)
    _check("zone_layout", lay.shape_ids)
    _check("rearrange_index", lay.shape_ids, grid)
    _check("gather_pool", v, valid, lay.shape_ids, lay.block_offset, grid, grid, lay.N_b, True, True, True, None)
    _check("gather_pool", v, None, lay.shape_ids, lay.block_offset, grid, grid, lay.N_b, True, False, False, p.q_re)
    _check("scatter_rows", p.q_re, lay.shape_ids, grid, grid, 0)
    x = torch.randn(1, 2, 200, 128, device="cuda", dtype=torch.bfloat16)
    _check("chunk_gather_pool", x, None, [1, 1, 200], [1, 1, 256], [1, 1, 64], 256, True, True, True, None)
    rows = torch.ops.prism.chunk_gather_pool(x, None, [1, 1, 200], [1, 1, 256], [1, 1, 64], 256, True, False, False,
                                             None)[0]
    _check("chunk_scatter_rows", rows, [1, 1, 200], [1, 1, 256], [1, 1, 64], 1)


def test_opcheck_selection_and_lists(plan):
    from prism_amd import ops
    _, p = plan
    lay = p.lay
    BH = p.B * p.H
    qc = torch.randn(BH, lay.N_b, 128, device="cuda")
    _check("block_scores", qc, qc, p.block_count)
    mode, k_lo, ub = ops.selection_params(lay.N_b, 0.6, 0.9)
    thr = ops.cdf_threshold_fixed(0.9)
    tcap = p.sel["tcap"]
    _check("select_tiles", p.scores, mode, k_lo, ub, 1 / math.sqrt(128), thr, lay.block_first_tile, p.tile_count,
           tcap, ub, True)
    _check("tile_rows", p.sel["ntiles"], lay.block_id_of_tile, p.tile_count, BH, lay.Nt, lay.N_b, tcap)
    _check("transpose_lists", p.qstart, p.qlen, p.qcols, BH, lay.Nt, lay.Nt)
    _check("pair_tiles", p.qstart, p.qlen, p.qcols, lay.Nt, lay.Nt)
    _check("pair_union", p.qstart, p.qlen, p.qcols, lay.Nt, lay.Nt, p.qpair, p.tmasks)
    _check("pair_order", p.qunion[1], 64, 8)
    assert lay.Nt % 4 == 0
    _check("quad_union", p.qstart, p.qlen, p.qcols, lay.Nt, lay.Nt, p.qpair, p.tmasks)
    _check("lists_csr_offsets", p.qlen)
    off, total = torch.ops.prism.lists_csr_offsets(p.qlen)
    _check("lists_csr_fill", p.qstart, p.qlen, p.qcols, off, int(total.item()))
    # (data-dependent output length: schema check; the fake's symbolic size is
    # covered on the CPU)
    print("[case] opcheck lists_to_csr", flush=True)
    torch.library.opcheck(torch.ops.prism.lists_to_csr.default, (p.qstart, p.qlen, p.qcols),
                          test_utils=("test_schema",))
    _check("tile_masks", p.kv_valid)


def test_opcheck_attention(plan):
    from prism_amd import ops
    _, p = plan
    sm = 1 / math.sqrt(128)
    args = (p.q_re, p.k_re, p.v_re, p.tmasks, *p.qunion, p.qpair, p.qorder, sm)
    _check("bsa_fwd", *args)
    o, lse = torch.ops.prism.bsa_fwd(*args)
    do = torch.randn_like(o)
    _check("bwd_preprocess", o, do)
    _check("lse_to_m2", lse)
    m2 = torch.ops.prism.lse_to_m2(lse)
    delta = torch.ops.prism.bwd_preprocess(o, do)
    BH, Nt = p.B * p.H, p.lay.Nt
    kl = ops.transpose_lists(p.qstart, p.qlen, p.qcols, BH, Nt)
    ku = ops.pair_union(*kl, Nt)
    _check("bsa_bwd_dkdv", p.q_re, p.k_re, p.v_re, do, m2, delta, p.kv_valid, *ku, None, None, sm)
    _check("bsa_bwd_dq", p.q_re, p.k_re, p.v_re, do, m2, delta, p.tmasks, *p.qunion, p.qpair, p.qorder, sm)
    quad = ops.quad_union(p.qstart, p.qlen, p.qcols, Nt, p.tmasks, pairmap=p.qpair)
    qorder = ops.pair_order(quad[1], 32)
    _check("bsa_fwd_quad", p.q_re, p.k_re, p.v_re, p.tmasks, *quad, p.qpair, qorder, sm)
    _check("bsa_bwd_dq_quad", p.q_re, p.k_re, p.v_re, do, m2, delta, p.tmasks, *quad, p.qpair, qorder, sm)


def test_errors_come_back_as_python_exceptions():
    x = torch.zeros((1, 1, 512, 64), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="multiples of 8"):
        torch.ops.prism.zone_stats(x, None, [8, 8, 12], [8, 8, 8])
    with pytest.raises(TypeError):
        torch.ops.prism.bsa_fwd(x.float(), x, x, None, torch.zeros(1, device="cuda", dtype=torch.int64),
                                torch.zeros(1, device="cuda", dtype=torch.int32),
                                torch.zeros(1, device="cuda", dtype=torch.int32), None, None, 0.1)
