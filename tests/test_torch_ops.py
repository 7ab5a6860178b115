"""The PyTorch operator registration (TORCH_LIBRARY(prism), libprism_torch.so):
every C-ABI entry point the path uses is an operator of torch.ops.prism with a
schema, and every operator has a fake (meta) implementation whose output
shapes and dtypes follow the C-ABI's contract.  Runs without a GPU (fake
tensors); tests/test_gpu_torch_ops.py runs torch.library.opcheck on the GPU."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

OPS = ["zone_stats", "audio_zone_stats", "zone_gradient", "zone_shapes", "assign_shapes", "a2v_norms", "zone_layout",
       "rearrange_index", "gather_pool", "scatter_rows", "chunk_gather_pool", "chunk_scatter_rows", "block_scores",
       "select_tiles", "tile_rows", "transpose_lists", "pair_tiles", "pair_union", "pair_order", "tile_masks",
       "lse_to_m2", "bsa_fwd", "bwd_preprocess", "bsa_bwd_dkdv", "bsa_bwd_dq", "linear_rownorm", "lists_to_csr",
       "lists_csr_offsets", "lists_csr_fill"]


@pytest.fixture(scope="module")
def prism():
    from prism_amd import _torch_ops
    return _torch_ops.load()


def test_every_operator_registered(prism):
    for name in OPS:
        op = getattr(prism, name)
        assert op.default._schema.name == f"prism::{name}"


def _t(shape, dtype):
    return torch.empty(shape, device="cuda", dtype=dtype)


def test_fake_shapes(prism):
    bf, f32, i32, i64, u8 = torch.bfloat16, torch.float32, torch.int32, torch.int64, torch.uint8
    B, H, D, grid, box = 1, 2, 128, [8, 16, 24], [7, 16, 20]
    S, Sin, Nz, Nt, N_b = 8 * 16 * 24, 7 * 16 * 20, 6, 48, 40
    with FakeTensorMode():
        v = _t((B, H, Sin, D), bf)
        packed, av = prism.zone_stats(v, None, grid, box)
        assert packed.shape == (Nz, 25 * D) and av.shape == (Nz, 24) and av.dtype == u8
        a, vh = prism.audio_zone_stats(_t((Sin,), f32), None, grid, box)
        assert a.shape == (Nz,) and vh.shape == (Nz, 3)
        g, rho, sid = prism.zone_shapes(_t((Nz,), f32), _t((Nz, 3), f32), None, None, 0, 0.5, 0.15, 1.0)
        assert g.shape == (Nz, 3) and sid.dtype == i64
        assert prism.a2v_norms(_t((Sin, 256), bf)).dtype == bf
        yb, nb = prism.linear_rownorm(_t((Sin, 128), bf), _t((256, 128), bf), None, 0)
        assert yb.shape == (Sin, 256) and yb.dtype == bf and nb.shape == (Sin,) and nb.dtype == f32
        boff, bot, bft = prism.zone_layout(_t((Nz,), i64))
        assert boff.shape == (Nz + 1,) and bot.shape == (Nt,) and bft.shape == (Nt + 1,)
        out = prism.gather_pool(v, None, _t((Nz,), i64), boff, grid, box, N_b, True, True, True, None)
        assert out[0].shape == (B, H, S, D) and out[0].dtype == bf and out[1].shape == (B, H, N_b, D)
        assert out[2].shape == (N_b,) and out[3].shape == (Nt,) and out[4].shape == (S,) and out[5].numel() == 0
        out = prism.gather_pool(v, None, _t((Nz,), i64), boff, grid, box, N_b, True, False, False,
                                _t((B, H, S, D), bf))
        assert out[1].numel() == 0 and out[5].shape == (B, H, S)
        assert prism.scatter_rows(_t((B, H, S, D), bf), _t((Nz,), i64), grid, box, 0).shape == (B, H, Sin, D)
        sc = prism.block_scores(_t((B * H, N_b, D), f32), _t((B * H, N_b, D), f32), None)
        assert sc.shape == (B * H, N_b, N_b)
        t, n, s_, ns = prism.select_tiles(sc, 2, 4, 30, 0.1, 7, bft, None, 60, 30, True)
        assert t.shape == (B * H * N_b, 60) and n.shape == (B * H * N_b,) and s_.shape == (B * H * N_b, 30)
        qs, ql = prism.tile_rows(n, bot, None, B * H, Nt, N_b, 60)
        assert qs.dtype == i64 and ql.shape == (B * H * Nt,)
        ks, kl, kc = prism.transpose_lists(qs, ql, t.view(-1), B * H, Nt, Nt)
        assert kc.shape == (B * H * Nt * Nt,)
        pm = prism.pair_tiles(qs, ql, t.view(-1), Nt, Nt)
        us, ul, uc = prism.pair_union(qs, ql, t.view(-1), Nt, Nt, pm, _t((Nt,), i64))
        assert us.shape == (B * H * Nt // 2,) and uc.shape == (B * H * Nt // 2 * Nt,)
        assert prism.pair_order(ul, 64, 10).shape == ul.shape
        assert prism.tile_masks(_t((S,), u8)).shape == (Nt,)
        q = _t((B, H, S, D), bf)
        o, lse = prism.bsa_fwd(q, q, q, None, us, ul, uc, pm, None, 0.1)
        assert o.shape == q.shape and o.dtype == bf and lse.shape == (B, H, S) and lse.dtype == f32
        assert prism.lse_to_m2(lse).shape == lse.shape
        assert prism.bwd_preprocess(o, q).shape == (B, H, S)
        dk, dv = prism.bsa_bwd_dkdv(q, q, q, q, lse, lse, None, us, ul, uc, None, None, 0.1)
        assert dk.shape == q.shape and dv.dtype == bf
        assert prism.bsa_bwd_dq(q, q, q, q, lse, lse, None, us, ul, uc, None, None, 0.1).shape == q.shape
        r = prism.chunk_gather_pool(_t((B, H, 200, D), bf), None, [1, 1, 200], [1, 1, 256], [1, 1, 64], 256, True,
                                    True, True, None)
        assert r[0].shape == (B, H, 256, D) and r[1].shape == (B, H, 4, D) and r[3].shape == (4,)
        assert prism.chunk_scatter_rows(r[0], [1, 1, 200], [1, 1, 256], [1, 1, 64], 1).shape == (B, H, 200, D)


def test_fake_csr_has_a_data_dependent_size(prism):
    """lists_to_csr's entry count is data-dependent: under a shape
    environment its fake output has an unbacked symbolic length."""
    from torch.fx.experimental.symbolic_shapes import ShapeEnv
    i32, i64 = torch.int32, torch.int64
    with FakeTensorMode(shape_env=ShapeEnv()):
        off, cols = prism.lists_to_csr(_t((10,), i64), _t((10,), i32), _t((100,), i32))
        assert off.shape == (11,) and off.dtype == i32 and cols.dtype == i32
        assert isinstance(cols.shape[0], torch.SymInt)


def test_operators_reject_cpu_tensors(prism):
    """A CPU tensor has no kernel here: the call fails loudly (no fallback)."""
    x = torch.zeros((1, 1, 512, 64), dtype=torch.bfloat16)
    with pytest.raises(Exception):
        prism.zone_stats(x, None, [8, 8, 8], [8, 8, 8])


def test_fake_split_csr(prism):
    """lists_csr_offsets keeps the total on the device; lists_csr_fill takes
    the caller's nnz (no data-dependent size)."""
    with FakeTensorMode():
        off, tot = prism.lists_csr_offsets(_t((100,), torch.int32))
        assert off.shape == (101,) and off.dtype == torch.int32 and tot.shape == (1,) and tot.dtype == torch.int64
        ent = prism.lists_csr_fill(_t((100,), torch.int64), _t((100,), torch.int32), _t((5000,), torch.int32), off, 777)
        assert ent.shape == (777,) and ent.dtype == torch.int32
        # no entries: still a one-element buffer (a valid pointer for the kernels)
        ent = prism.lists_csr_fill(_t((100,), torch.int64), _t((100,), torch.int32), _t((5000,), torch.int32), off, 0)
        assert ent.shape == (1,)
