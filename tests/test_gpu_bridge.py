"""The a2v bridge output projection with the residual norms fused into its
epilogue (prism_linear_rownorm; interactionv2.py:225/:348, mova.py:127-137,
wan_video_dit.py:742-752), against float64 restatements:
  * y = x W^T + b: every entry within bf16 rounding of the float64 product
    (|y - ref| <= 2^-7 |ref| + 1e-3 max(|ref|)), and close to torch's bf16
    F.linear;
  * norms = ||y_stored[m, :]||_2: within 1e-5 relative of the float64 norm of
    the kernel's own bf16 output, and of prism_a2v_norms on that output;
  * tail rows (M not a multiple of 256), no bias, fp32 norms, the argument
    checks, and the config-4 shape (302,400 x 5,120 x 5,120) on sampled rows.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(M, N, K, bias=True, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=DEV) / K ** 0.5).to(torch.bfloat16)
    b = (0.1 * torch.randn(N, generator=g, device=DEV)).to(torch.bfloat16) if bias else None
    return x, w, b


def _check_rows(x, w, b, y, norms, rows):
    xr = x[rows].double()
    ref = xr @ w.double().T + (0 if b is None else b.double())
    got = y[rows].double()
    err = (got - ref).abs()
    bound = 2.0 ** -7 * ref.abs() + 1e-3 * float(ref.abs().max())
    print("[case] y max-abs", float(err.max()), "rel", float((got - ref).norm() / ref.norm()), flush=True)
    assert bool((err <= bound).all())
    own = got.norm(dim=-1)
    rel = ((norms[rows].double() - own).abs() / own.clamp_min(1e-30)).max()
    print("[case] norms rel vs own output", float(rel), flush=True)
    tol = 1e-5 if norms.dtype == torch.float32 else 2.0 ** -8
    assert float(rel) <= tol


@pytest.mark.parametrize("M,N,K,bias", [(1000, 512, 320, True), (256, 256, 64, False), (777, 768, 1024, True)])
def test_linear_rownorm_small(M, N, K, bias):
    from prism_amd import ops
    x, w, b = _inputs(M, N, K, bias)
    y, n32 = ops.linear_rownorm(x, w, b, torch.float32)
    _, n16 = ops.linear_rownorm(x, w, b)
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == torch.bfloat16 and n16.dtype == torch.bfloat16
    rows = torch.arange(M, device=DEV)
    _check_rows(x, w, b, y, n32, rows)
    _check_rows(x, w, b, y, n16, rows)
    ref = torch.nn.functional.linear(x, w, b)
    assert float((y.double() - ref.double()).abs().max()) <= 4e-2 * float(ref.abs().max())
    # the same norms from the unfused kernel on the fused kernel's output
    assert float(((ops.a2v_norms(y.float()).double() - n32.double()).abs() / n32.double()).max()) <= 1e-5


def test_bridge_projection_api_batch0():
    from prism_amd import a2v_bridge_projection, a2v_token_norms
    x, w, b = _inputs(2 * 300, 256, 128)
    res, norms = a2v_bridge_projection(x.view(2, 300, 128), w, b)
    assert res.shape == (2, 300, 256) and norms.shape == (300,)
    ref = a2v_token_norms(res)
    assert float(((norms.double() - ref.double()).abs() / ref.double()).max()) <= 2.0 ** -8


def test_linear_rownorm_errors():
    from prism_amd import ops
    x, w, b = _inputs(64, 256, 64)
    with pytest.raises(ValueError, match="multiple of 256"):
        ops.linear_rownorm(x, w[:200], None)
    with pytest.raises(ValueError, match="multiple of 64"):
        ops.linear_rownorm(x[:, :48].contiguous(), w[:, :48].contiguous(), None)
    with pytest.raises(TypeError):
        ops.linear_rownorm(x.float(), w, None)


def test_linear_rownorm_config4_shape():
    """Config 4's video tokens and C = 5,120 (the a2v bridge of the 2K
    model): sampled rows against float64, all norms against prism_a2v_norms
    of the stored output."""
    from prism_amd import ops
    M, C = 302400, 5120
    x, w, b = _inputs(M, C, C, seed=3)
    y, norms = ops.linear_rownorm(x, w, b, torch.float32)
    torch.cuda.synchronize()
    rows = torch.as_tensor(np.random.default_rng(0).choice(M, 64, replace=False), device=DEV)
    rows = torch.cat([rows, torch.tensor([0, M - 1], device=DEV)])
    _check_rows(x, w, b, y, norms, rows)
    ref = ops.a2v_norms(y.float())
    rel = float(((norms.double() - ref.double()).abs() / ref.double()).max())
    print("[case] config-4 norms vs unfused, max rel", rel, flush=True)
    assert rel <= 1e-5
