"""The reference's pure-PyTorch dynamic block-sparse attention path, restated
in torch float32 for the CPU.

TEST INFRASTRUCTURE ONLY: this is the timed CPU baseline of ``bench.py``
(``cpu_baseline``) and a cross-check in ``tests/``; the product package
``prism_amd`` never imports it.  Only the selection checker
(selection_rows_with_margins, selection_agreement) also runs torch's GPU
kernels, as the second float32 evaluation of the reference's sequence.

It restates, with torch operations in the reference's order of steps (paths
relative to hymm/models/modules/block_sparse_attention/):
  * zone statistics and shape choice: compute_zone_aggregates,
    compute_effective_gradient, compute_audio_directional, select_shapes_ivpq
    / select_shapes_penalty (dynamic_block_shape.py:55-355), on the batch-0
    head mean of V (dynamic_block_attention.py:236);
  * the per-zone rearrangement and block/tile maps
    (dynamic_block_attention.py:21-63, 107-170) and the gathers (:250-253);
  * masked tile mean pooling and logical-block means (bsa_interface.py:177-201,
    dynamic_block_attention.py:173-188, :259-268);
  * block scores with the invalid-key fill (bsa_interface.py:203-207,
    dynamic_block_attention.py:270-279) and the top-k / cdf / hybrid selection
    (bsa_interface.py:235-304);
  * the block -> tile expansion (dynamic_block_attention.py:297-319);
  * the token mask of the selected tiles (create_mask_from_indices_varlen,
    bsa_interface.py:127-145, expanded to tokens and AND'ed with the key
    validity) and masked scaled-dot-product attention
    (torch.nn.functional.scaled_dot_product_attention with a boolean mask,
    the SDPA fallback of flash_attention, wan_video_dit.py:77-110), whose
    autograd is the backward.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

ZONE = 8
TILE = 64
EPS = 1e-6
CANDIDATES = [
    (4, 4, 4), (8, 2, 4), (8, 4, 2), (2, 4, 8), (2, 8, 4), (4, 2, 8), (4, 8, 2),
    (2, 8, 8), (8, 2, 8), (8, 8, 2), (4, 4, 8), (4, 8, 4), (8, 4, 4),
]


# ---------------------------------------------------------------- zone statistics and shapes
def _zones(x: torch.Tensor, grid) -> torch.Tensor:
    """[T, Hg, Wg, *rest] -> [Nz, 8, 8, 8, *rest], zones in (zt, zh, zw) order."""
    T, Hg, Wg = grid
    rest = x.shape[3:]
    y = x.reshape(T // ZONE, ZONE, Hg // ZONE, ZONE, Wg // ZONE, ZONE, *rest)
    perm = (0, 2, 4, 1, 3, 5) + tuple(range(6, 6 + len(rest)))
    return y.permute(*perm).reshape(-1, ZONE, ZONE, ZONE, *rest)


def _masked_axis_means(xz: torch.Tensor, mz: torch.Tensor):
    """Masked means of xz [Nz,8,8,8,D] (mask mz [Nz,8,8,8,1]) over all tokens,
    per t (over h, w), per h and per w, plus the axis validity flags."""
    def mean(dims):
        return (xz * mz).sum(dim=dims) / mz.sum(dim=dims).clamp(min=1.0)
    m = mz[..., 0]
    valid = tuple(m.sum(dim=d) > 0 for d in ((2, 3), (1, 3), (1, 2)))
    return mean((1, 2, 3)), mean((2, 3)), mean((1, 3)), mean((1, 2)), valid


def _var_over_valid(vals: torch.Tensor, valid: torch.Tensor) -> torch.Tensor:
    """Population variance over dim 1 restricted to valid positions; a trailing
    channel dim (if any) is averaged afterwards."""
    vf = valid.to(vals.dtype)
    if vals.dim() == 3:
        vf = vf[..., None]
    n = vf.sum(dim=1, keepdim=True).clamp(min=1.0)
    mu = (vals * vf).sum(dim=1, keepdim=True) / n
    var = (((vals - mu) ** 2) * vf).sum(dim=1, keepdim=True) / n
    var = var.squeeze(1)
    return var.mean(dim=-1) if vals.dim() == 3 else var


def zone_shapes(v: torch.Tensor, norms: Optional[torch.Tensor], grid, valid: Optional[torch.Tensor],
                method: str = "ivpq", lambda_a: float = 0.5, tau_128: float = 0.15,
                lambda_128: float = 1.0) -> torch.Tensor:
    """Shape id per zone (int64 [Nz]) from V [B,H,S,D] THW over the padded grid."""
    T, Hg, Wg = grid
    D = v.shape[-1]
    vh = v[0].mean(dim=0).reshape(T, Hg, Wg, D).float()
    m = (torch.ones(T * Hg * Wg) if valid is None else valid.float()).reshape(T, Hg, Wg, 1)
    xz, mz = _zones(vh, grid), _zones(m, grid)
    cm, fT, aH, aW, (tv, hv, wv) = _masked_axis_means(xz, mz)
    # information density rho (dynamic_block_shape.py:274-282)
    spatial = ((cm - cm.mean(dim=-1, keepdim=True)) ** 2).mean(dim=-1)
    pair = (tv[:, 1:] & tv[:, :-1]).to(fT.dtype)[..., None]
    temporal = (((fT[:, 1:] - fT[:, :-1]) ** 2 * pair).sum(dim=1) / pair.sum(dim=1).clamp(min=1.0)).mean(dim=-1)
    rho_raw = spatial + temporal
    rho = rho_raw / rho_raw.max().clamp(min=EPS)
    # anisotropy (:284-291)
    var = torch.stack([_var_over_valid(fT, tv), _var_over_valid(aH, hv), _var_over_valid(aW, wv)], dim=-1)
    aniso = var / var.sum(dim=-1, keepdim=True).clamp(min=EPS)
    # audio directional term (:189-245)
    if norms is not None:
        az = _zones(norms.float().reshape(T, Hg, Wg, 1), grid)
        abar, nT, nH, nW, (atv, ahv, awv) = _masked_axis_means(az, mz)
        avar = torch.stack([_var_over_valid(nT[..., 0], atv), _var_over_valid(nH[..., 0], ahv),
                            _var_over_valid(nW[..., 0], awv)], dim=-1)
        vhat = avar / avar.sum(dim=-1, keepdim=True).clamp(min=EPS)
        abar = abar[:, 0] / abar[:, 0].max().clamp(min=EPS)
        g = aniso + lambda_a * abar[:, None] * vhat
    else:
        g = aniso.clone()
    g = g.clamp(min=1e-4)
    shapes = torch.tensor(CANDIDATES, dtype=torch.float32)
    is128 = shapes.prod(dim=-1) > 64.5
    if method == "ivpq":   # select_shapes_ivpq (:303-327)
        lr = (-2.0 / 3.0) * torch.log2(g)
        ideal = lr + (6.0 - lr.sum(dim=-1, keepdim=True)) / 3.0
        cost = ((torch.log2(shapes)[None] - ideal[:, None]) ** 2).sum(dim=-1)
    elif method == "penalty":  # select_shapes_penalty (:330-355)
        cost = (g[:, None] * shapes[None]).sum(dim=-1) - (lambda_128 * (1.0 - rho))[:, None] * is128[None].float()
    else:
        raise ValueError(f"unknown dynamic-block method: {method!r}")
    cost = cost.masked_fill((rho[:, None] >= tau_128) & is128[None], float("inf"))
    return cost.argmin(dim=-1)


# ---------------------------------------------------------------- geometry
def rearrange_index(shape_ids: torch.Tensor, grid):
    """src[r] = THW index of rearranged position r; inv its inverse."""
    T, Hg, Wg = grid
    ZH, ZW = Hg // ZONE, Wg // ZONE
    lf = torch.arange(512)
    lt, lh, lw = lf // 64, (lf // 8) % 8, lf % 8
    orders = []
    for bt, bh, bw in CANDIDATES:
        pos = (((lt // bt) * (8 // bh) + lh // bh) * (8 // bw) + lw // bw) * (bt * bh * bw) \
            + ((lt % bt) * bh + lh % bh) * bw + lw % bw
        o = torch.empty(512, dtype=torch.long)
        o[pos] = lf
        orders.append(o)
    lo = torch.stack(orders)[shape_ids]                       # [Nz, 512] local flat coordinate
    z = torch.arange(len(shape_ids))
    zt, zh, zw = z // (ZH * ZW), (z // ZW) % ZH, z % ZW
    src = (((zt[:, None] * 8 + lo // 64) * Hg + zh[:, None] * 8 + (lo // 8) % 8) * Wg
           + zw[:, None] * 8 + lo % 8).reshape(-1)
    inv = torch.empty_like(src)
    inv[src] = torch.arange(src.numel())
    return src, inv


def block_maps(shape_ids: torch.Tensor):
    """(block_id_of_tile [Nt], kblock_tiles [N_b + 1, 2] with sentinel Nt, N_b)."""
    tpb = torch.tensor([b[0] * b[1] * b[2] // TILE for b in CANDIDATES])[shape_ids]
    nbz = 8 // tpb
    Nt = len(shape_ids) * 8
    N_b = int(nbz.sum())
    first = torch.cumsum(nbz, 0) - nbz
    t = torch.arange(Nt)
    zt, loc = t // 8, t % 8
    bid = first[zt] + loc // tpb[zt]
    kbt = torch.full((N_b + 1, 2), Nt, dtype=torch.long)
    kbt[bid, loc % tpb[zt]] = t
    return bid, kbt, N_b


# ---------------------------------------------------------------- pooling, scores, selection
def block_means(x_re: torch.Tensor, valid_re: Optional[torch.Tensor], bid: torch.Tensor, N_b: int):
    """Masked tile means, then count-weighted logical-block means (fp32)."""
    B, H, S, D = x_re.shape
    Nt = S // TILE
    m = torch.ones(S) if valid_re is None else valid_re.float()
    mt = m.view(1, 1, Nt, TILE, 1)
    cnt = mt.sum(dim=3).clamp(min=1.0)
    tile_mean = (x_re.float().view(B, H, Nt, TILE, D) * mt).sum(dim=3) / cnt
    tcount = m.view(Nt, TILE).sum(dim=1)
    bsum = torch.zeros(B, H, N_b, D).index_add_(2, bid, tile_mean * tcount.view(1, 1, Nt, 1))
    bcount = torch.zeros(N_b).index_add_(0, bid, tcount)
    return bsum / bcount.clamp(min=1.0).view(1, 1, N_b, 1), bcount, tcount


def select_blocks(score: torch.Tensor, sparsity: Optional[float], p: Optional[float], sm_scale: float):
    """[R, N] scores -> selected block ids [R, r] ascending, sentinel N past the
    selection (bsa_interface.py:235-304)."""
    N = score.shape[-1]
    if sparsity is not None and p is None:
        k = int((1 - sparsity) * N)
        return torch.sort(torch.topk(score, k, dim=-1).indices, dim=-1).values
    w = torch.softmax(score * sm_scale, dim=-1)
    lo = 1 if sparsity is None else max(1, int((1 - sparsity) * N))
    if sparsity is None and p is None:
        raise ValueError("Either sparsity or cdf_threshold must be provided")
    ub = min(N, max(lo, int(p * N) + 1))
    vals, idx = torch.topk(w, k=ub, dim=-1, largest=True, sorted=True)
    n = ((torch.cumsum(vals, dim=-1) < p).sum(dim=-1, keepdim=True) + 1).clamp(min=lo, max=N)
    idx = idx.masked_fill(torch.arange(ub)[None, :] >= n, N)
    return torch.sort(idx, dim=-1).values


def selection_rows_with_margins(scores: torch.Tensor, sparsity, p, sm: float):
    """The reference's selection (bsa_interface.py:235-304) as the same torch
    op sequence in float32 on the device that holds `scores` (the GPU, or the
    host for torch's CPU kernels).  scores: [R, N].  Returns the selected
    sets as a [R, N] bool mask, the decision margin |exact cumsum - p| at the
    crossing (float64 cumsum of the float32 weights; inf for top-k rows) and
    the boundary-tie flags (the weight or score at the cut equals the next)."""
    R, N = scores.shape
    dev = scores.device
    if p is None:
        k = int((1 - sparsity) * N)
        _, idx = torch.topk(scores, k, dim=-1)
        mask = torch.zeros((R, N), dtype=torch.bool, device=dev).scatter_(1, idx, True)
        srt = torch.sort(scores, dim=-1, descending=True).values
        tie = (srt[:, k - 1] == srt[:, k]) if k < N else torch.zeros(R, dtype=torch.bool, device=dev)
        return mask, torch.full((R,), float("inf"), device=dev, dtype=torch.float64), tie
    w = torch.softmax(scores * sm, dim=-1)
    lo = 1 if sparsity is None else max(1, int((1 - sparsity) * N))
    ub = min(N, max(lo, int(p * N) + 1))
    vals, idx = torch.topk(w, k=ub, dim=-1, largest=True, sorted=True)
    cdf = torch.cumsum(vals, dim=-1)
    n = ((cdf < p).to(torch.int32).sum(dim=-1, keepdim=True) + 1).clamp(min=lo, max=N)
    pos = torch.arange(ub, device=dev)
    idx = idx.masked_fill(pos >= n, N)
    mask = torch.zeros((R, N + 1), dtype=torch.bool, device=dev).scatter_(1, idx, True)[:, :N]
    c = (cdf < p).to(torch.int64).sum(dim=-1)
    cdf64 = torch.cumsum(vals.double(), dim=-1)
    near = torch.stack([(cdf64.gather(1, (c - d).clamp(0, ub - 1)[:, None])[:, 0] - p).abs() for d in (0, 1)])
    margin = near.min(dim=0).values
    e = torch.clamp(n.squeeze(-1), max=ub).long()
    srt = torch.sort(w, dim=-1, descending=True).values
    nxt = torch.clamp(e, max=N - 1)
    tie = (e < N) & (srt.gather(1, (e - 1)[:, None])[:, 0] == srt.gather(1, nxt[:, None])[:, 0])
    return mask, margin, tie


def selection_agreement(scores: torch.Tensor, sel_blocks: torch.Tensor, nsel: torch.Tensor, sparsity, p,
                        sm: float, chunk: int = 2048):
    """Rows whose selected block set (sel_blocks [R, width] ascending, nsel
    [R] live entries) differs from the reference's torch sequence in float32,
    run on the scores' device and with torch's CPU kernels.  Returns
    {"gpu" | "cpu": {"rows_differing", "of_them_tied", "max_untied_margin"}}
    (margins and ties from the device run; a row is tied if either run finds a
    tie at its cut)."""
    R, N = scores.shape
    dev = scores.device
    width = sel_blocks.shape[1]
    out = {"gpu": [0, 0, 0.0], "cpu": [0, 0, 0.0]}
    for r0 in range(0, R, chunk):
        s = scores[r0:r0 + chunk]
        sel = sel_blocks[r0:r0 + chunk].long()
        live = torch.arange(width, device=dev)[None, :] < nsel[r0:r0 + chunk, None]
        sel = torch.where(live, sel, torch.full_like(sel, N))
        mine = torch.zeros((len(s), N + 1), dtype=torch.bool, device=dev).scatter_(1, sel, True)[:, :N]
        ref_dev = selection_rows_with_margins(s, sparsity, p, sm)
        ref_cpu = selection_rows_with_margins(s.cpu(), sparsity, p, sm)
        margin, tie = ref_dev[1], ref_dev[2] | ref_cpu[2].to(dev)
        for name, ref_mask in (("gpu", ref_dev[0]), ("cpu", ref_cpu[0].to(dev))):
            diff = (mine != ref_mask).any(dim=1)
            if bool(diff.any()):
                dm, dt = margin[diff], tie[diff]
                out[name][0] += int(diff.sum())
                out[name][1] += int(dt.sum())
                untied = dm[~dt]
                if untied.numel():
                    out[name][2] = max(out[name][2], float(untied.max()))
    return {k: {"rows_differing": v[0], "of_them_tied": v[1], "max_untied_margin": v[2]} for k, v in out.items()}


def tile_lists(sel: torch.Tensor, kbt: torch.Tensor, tcount: Optional[torch.Tensor], Nt: int):
    """Selected blocks [..., r] -> ascending key-tile lists [..., 2r] (sentinel
    Nt; padded tiles dropped) and their lengths."""
    tiles = torch.cat([kbt[:, 0][sel], kbt[:, 1][sel]], dim=-1)
    if tcount is not None:
        ok = (tiles < Nt) & (tcount > 0)[tiles.clamp(max=Nt - 1)]
        tiles = torch.where(ok, tiles, torch.full_like(tiles, Nt))
    tiles = torch.sort(tiles, dim=-1).values
    return tiles, (tiles < Nt).sum(dim=-1)


def plan(q, k, v, grid, *, sparsity, cdf_threshold, norms=None, valid=None, shape_ids=None, method="ivpq"):
    """Steps (1)-(5) of flash_attn_bsa_3d_dynamic on the CPU.  q, k, v:
    [B,H,S,D] THW over the padded grid.  Returns a dict with the shape ids,
    the rearranged q, k, v, the key validity and per-query-tile tile lists."""
    B, H, S, D = q.shape
    sm = 1.0 / math.sqrt(D)
    if shape_ids is None:
        shape_ids = zone_shapes(v, norms, grid, valid, method)
    src, inv = rearrange_index(shape_ids, grid)
    bid, kbt, N_b = block_maps(shape_ids)
    Nt = S // TILE
    q_re, k_re, v_re = (x.index_select(2, src) for x in (q, k, v))
    valid_re = None if valid is None else valid[src]
    qm, _, tcount = block_means(q_re, valid_re, bid, N_b)
    km, bcount, _ = block_means(k_re, valid_re, bid, N_b)
    tiles, lens = [], []
    for h in range(H):  # per head, as the reference loops (dynamic_block_attention.py:276-289)
        s = qm[:, h] @ km[:, h].transpose(-1, -2)
        if valid is not None:
            s = s.masked_fill((bcount == 0)[None, None, :], float("-inf"))
        sel = select_blocks(s.reshape(-1, N_b), sparsity, cdf_threshold, sm).clamp(max=N_b)
        t, n = tile_lists(sel, kbt, tcount if valid is not None else None, Nt)
        tiles.append(t.view(B, N_b, -1)[:, bid])   # each query tile takes its block's row
        lens.append(n.view(B, N_b)[:, bid])
    return dict(shape_ids=shape_ids, src=src, inv=inv, q_re=q_re, k_re=k_re, v_re=v_re, valid_re=valid_re,
                tiles=torch.stack(tiles, 1), lens=torch.stack(lens, 1), N_b=N_b, Nt=Nt)


# ---------------------------------------------------------------- masked attention
def token_mask(tiles: torch.Tensor, lens: torch.Tensor, Nt: int, valid_re: Optional[torch.Tensor]):
    """Boolean [..., 64, Nt*64] key mask of query tiles from their tile lists
    (create_mask_from_indices_varlen, bsa_interface.py:127-145, per token) and
    the key validity."""
    lead = tiles.shape[:-1]
    tm = torch.zeros(*lead, Nt + 1, dtype=torch.bool)
    live = torch.arange(tiles.shape[-1]) < lens[..., None]
    tm.scatter_(-1, torch.where(live, tiles, torch.full_like(tiles, Nt)), True)
    km = tm[..., :Nt].repeat_interleave(TILE, dim=-1)
    if valid_re is not None:
        km = km & valid_re.bool()
    return km[..., None, :].expand(*lead, TILE, Nt * TILE)


def masked_attention(q, k, v, mask, do=None):
    """Masked SDPA in fp32 (+ backward by autograd when do is given).  Rows
    whose mask is empty give 0 (the reference kernel's O = 0, LSE = -inf)."""
    q = q.float().detach().requires_grad_(do is not None)
    k = k.float().detach().requires_grad_(do is not None)
    v = v.float().detach().requires_grad_(do is not None)
    any_key = mask.any(dim=-1, keepdim=True)
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask | ~any_key)
    o = torch.where(any_key, o, torch.zeros_like(o))
    if do is None:
        return o.detach(), None
    o.backward(do.float())
    return o.detach(), (q.grad, k.grad, v.grad)


def forward_backward(q, k, v, do, grid, *, sparsity, cdf_threshold, norms=None, valid=None, shape_ids=None):
    """The whole CPU path, forward and backward, in THW order: out, dq, dk, dv, plan."""
    pl = plan(q, k, v, grid, sparsity=sparsity, cdf_threshold=cdf_threshold, norms=norms, valid=valid,
              shape_ids=shape_ids)
    B, H, S, D = q.shape
    Nt = pl["Nt"]
    mask = token_mask(pl["tiles"], pl["lens"], Nt, pl["valid_re"]).reshape(B, H, S, S)
    do_re = do.index_select(2, pl["src"])
    o, (dq, dk, dv) = masked_attention(pl["q_re"], pl["k_re"], pl["v_re"], mask, do_re)
    inv = pl["inv"]
    return (o.index_select(2, inv), dq.index_select(2, inv), dk.index_select(2, inv), dv.index_select(2, inv), pl)
