"""Benchmark of the dynamic block-sparse attention path on one MI355X.

Default workload = BASELINE config 4 ("2K fwd+bwd, one GPU's head share"):
B=1, H=5, D=128, bf16, latent grid 21x90x160 (302,400 video tokens, padded
to 24x96x160) plus 2,000 audio tokens; hybrid top-48 + cumulative 0.9.
A step = A2V token norms + SelfAttention._run_bsa_dynamic forward (zone
stats, shapes, gather + pooling, scores, selection, attention, scatter; the
caller's padding to multiples of 8 and unpadding happen inside the gather and
scatter kernels) + its backward, on synthetic inputs already resident in HBM.

Prints ONE JSON line.  value = kept-block algorithmic FLOP/s of the step
((4 + 10) * 64 * 64 * D * sum_lens per step, FA convention).
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "sparse-attn fwd+bwd ms & effective TFLOP/s at 2K shape; MFMA util %"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (B, H, D, grid_real, audio_tokens, C, topk, cdf, sparsity_only, struct_scale, field_amp, field_ell)
    "c4": (1, 5, 128, (21, 90, 160), 2000, 5120, 48, 0.9, None, 2.0, 2.45, 16.0),
    "c3": (1, 24, 128, (21, 68, 120), 2000, 3072, 32, 0.9, None, 2.0, 2.45, 16.0),
    "c2": (1, 24, 128, (21, 45, 80), 2000, 3072, None, None, 0.75, 2.0, 2.45, 16.0),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ synthetic inputs (GPU, seeded)
def lowrank_zone_field(gen, H, grid_pad, D, rank, scale, device):
    """[H, T, Hg, Wg, D] per-zone rank-`rank` structure with smooth t/h/w
    modulation and Dirichlet axis weights (zone variances differ)."""
    import torch
    T, Hg, Wg = grid_pad
    ZT, ZH, ZW = T // 8, Hg // 8, Wg // 8
    Nz = ZT * ZH * ZW
    w = -torch.log(torch.rand(Nz, 3, generator=gen, device=device).clamp_min(1e-12))
    w = w / w.sum(1, keepdim=True)
    f = 0.5 + 2.5 * torch.rand(Nz, rank, 3, generator=gen, device=device)
    ph = 2 * math.pi * torch.rand(Nz, rank, 3, generator=gen, device=device)
    x = torch.linspace(0, 1, 8, device=device)
    ct = torch.sin(f[..., 0, None] * math.pi * x + ph[..., 0, None])  # [Nz, r, 8]
    ch = torch.sin(f[..., 1, None] * math.pi * x + ph[..., 1, None])
    cw = torch.sin(f[..., 2, None] * math.pi * x + ph[..., 2, None])
    coef = (w[:, None, 0, None, None, None] * ct[..., :, None, None]
            + w[:, None, 1, None, None, None] * ch[..., None, :, None]
            + w[:, None, 2, None, None, None] * cw[..., None, None, :]).reshape(Nz, rank, 512)
    amp = scale * torch.rand(Nz, 1, 1, generator=gen, device=device)
    out = torch.empty((H, T, Hg, Wg, D), device=device, dtype=torch.float32)
    for h in range(H):
        basis = torch.randn(Nz, rank, D, generator=gen, device=device)
        s = amp * torch.bmm(coef.transpose(1, 2).contiguous(), basis)  # [Nz, 512, D]
        s = s.view(ZT, ZH, ZW, 8, 8, 8, D).permute(0, 3, 1, 4, 2, 5, 6).reshape(T, Hg, Wg, D)
        out[h] = s
    return out


def shared_field(gen, grid_pad, D, ell, device):
    """Random Fourier features F [T*Hg*Wg, D] of the token coordinates with a
    Gaussian kernel of length scale `ell` tokens, F(x).F(x') ~ D exp(-|x-x'|^2 /
    (2 ell^2)).  Added to both q and k of a head, it makes block scores decay
    with distance, so the hybrid selection keeps a local neighbourhood (the
    amplitude sets the realized density)."""
    import torch
    T, Hg, Wg = grid_pad
    om = torch.randn(D, 3, generator=gen, device=device) / ell
    ph = 2 * math.pi * torch.rand(D, generator=gen, device=device)
    R = torch.linalg.qr(torch.randn(D, D, generator=gen, device=device))[0]
    t = torch.arange(T, device=device, dtype=torch.float32)
    h = torch.arange(Hg, device=device, dtype=torch.float32)
    w = torch.arange(Wg, device=device, dtype=torch.float32)
    arg = t[:, None, None, None] * om[:, 0] + h[None, :, None, None] * om[:, 1] + w[None, None, :, None] * om[:, 2] + ph
    return (math.sqrt(2.0) * torch.cos(arg)).reshape(-1, D) @ R.T.contiguous()


def make_inputs(cfg_name, seed=0, device="cuda"):
    """Seeded synthetic inputs of a BASELINE config: q, k, v [B,H,S,D] bf16 THW
    order (noise + per-zone rank-8 structure; q and k also share a per-head
    smooth field), the A2V bridge residual [B,S,C] bf16 with audio coupling in
    ~10% of the zones, and dO."""
    import torch
    B, H, D, grid, audio, C, topk, cdf, sp_only, scale, famp, fell = CONFIGS[cfg_name]
    T, Hg, Wg = grid
    gp = tuple((x + 7) // 8 * 8 for x in grid)
    gen = torch.Generator(device=device).manual_seed(seed)
    S = T * Hg * Wg
    fields = torch.stack([shared_field(gen, gp, D, fell, device).view(*gp, D)[:T, :Hg, :Wg].reshape(S, D)
                          for _ in range(H)])
    qkv = []
    for i in range(3):
        low = lowrank_zone_field(gen, H, gp, D, 8, scale, device)[:, :T, :Hg, :Wg].reshape(H, S, D)
        x = torch.randn((B, H, S, D), generator=gen, device=device) + low[None]
        if i < 2:
            x += famp * fields[None]
        x = x / x.std()  # unit marginal variance; the structure keeps its scale relative to the noise
        qkv.append(x.to(torch.bfloat16).contiguous())
        del low, x
    del fields
    # A2V bridge residual [B, S, C]: audio coupling concentrated in ~10% of
    # the zones.  There each channel is correlated with the token's keys at
    # rho = 0.8 (rho * a fixed random projection of the heads' keys, unit
    # variance, + sqrt(1 - rho^2) * noise) and the amplitude is 3; elsewhere
    # the residual is unit noise.
    zone_amp = torch.zeros(gp[0] // 8, gp[1] // 8, gp[2] // 8, device=device)
    zone_amp.view(-1)[torch.randperm(zone_amp.numel(), generator=gen, device=device)[: max(1, zone_amp.numel() // 10)]] = 2.0
    amp = zone_amp.repeat_interleave(8, 0).repeat_interleave(8, 1).repeat_interleave(8, 2)[:T, :Hg, :Wg].reshape(S, 1)
    rho = 0.8
    proj = torch.randn((H * D, C), generator=gen, device=device) / math.sqrt(H * D)
    res = torch.empty((B, S, C), device=device, dtype=torch.bfloat16)
    for b in range(B):
        z = qkv[1][b].float().permute(1, 0, 2).reshape(S, H * D) @ proj
        z /= z.std()
        eps = torch.randn((S, C), generator=gen, device=device)
        res[b] = (torch.where(amp > 0, rho * z + math.sqrt(1 - rho * rho) * eps, eps) * (1.0 + amp)).to(torch.bfloat16)
        del z, eps
    do = torch.randn((B, H, S, D), generator=gen, device=device).to(torch.bfloat16)
    if str(device).startswith("cuda"):
        torch.cuda.synchronize()
    return dict(q=qkv[0], k=qkv[1], v=qkv[2], res=res, do=do, grid=grid, grid_pad=gp, topk=topk, cdf=cdf,
                sp_only=sp_only, B=B, H=H, D=D, S=S)


# ------------------------------------------------------------------ timing helpers
def time_region(fn, steps, warmup):
    """warmup untimed calls, then steps timed calls each bracketed by HIP
    events on the current stream.  Returns (mean ms, median ms, wall ms per
    call)."""
    import statistics
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    gc.collect()
    gc.disable()  # no cyclic garbage collection inside the timed region
    t0 = time.perf_counter()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in ev:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gc.enable()
    per = [a.elapsed_time(b) for a, b in ev]
    return sum(per) / steps, statistics.median(per), wall / steps * 1e3


DENSE_STEPS, DENSE_WARMUP = 10, 3  # torch SDPA comparison: median of 10 after 3 warm-ups


# ------------------------------------------------------------------ CPU baseline
def _host_threads() -> int:
    """Host threads for the CPU baseline: every core this process may use
    (the CPU share OMP_NUM_THREADS states on a GPU box, else os.cpu_count)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        pass
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _pad_host(x, grid, gp):
    """[B,H,S,D] (or [S]) THW of grid on the GPU -> float32 host tensor over
    the zero-padded zone grid gp (the padding of wan_video_dit.py:342-400)."""
    import torch
    T, Hg, Wg = grid
    if x.dim() == 1:
        out = torch.zeros(gp, device=x.device, dtype=torch.float32)
        out[:T, :Hg, :Wg] = x.view(T, Hg, Wg).float()
        return out.reshape(-1).cpu()
    B, H, S, D = x.shape
    out = torch.zeros((B, H, *gp, D), device=x.device, dtype=torch.float32)
    out[:, :, :T, :Hg, :Wg] = x.view(B, H, T, Hg, Wg, D).float()
    return out.view(B, H, -1, D).cpu()


def cpu_c1_end_to_end(seed=0):
    """Config 1 through the whole CPU path (oracle/torch_path.py), forward and
    backward: B=1, H=4, D=64, fp32, grid 4x16x16 padded to 8x16x16, 64 audio
    tokens, top-8 blocks + p = 0.9.  Returns (ms, kept tile pairs)."""
    import torch
    from oracle import torch_path as TP
    g = torch.Generator().manual_seed(seed)
    grid, gp, H, D = (4, 16, 16), (8, 16, 16), 4, 64
    S, Sp = 4 * 16 * 16, 8 * 16 * 16
    valid = torch.zeros(gp, dtype=torch.bool)
    valid[:4] = True
    valid = valid.reshape(-1)
    pad = lambda x: torch.cat([x, torch.zeros(*x.shape[:-2], Sp - S, x.shape[-1])], dim=-2)
    q, k, v, do = (pad(torch.randn(1, H, S, D, generator=g)) for _ in range(4))
    # A2V residual of 64 audio tokens: cross-attention of the video queries
    # (heads concatenated, C = 256) over audio keys/values; its per-token norms
    qv = q[0, :, :S].transpose(0, 1).reshape(S, H * D)
    ka, va = torch.randn(64, H * D, generator=g), torch.randn(64, H * D, generator=g)
    res = torch.softmax(qv @ ka.T / math.sqrt(H * D), dim=-1) @ va
    norms = torch.cat([res.norm(dim=-1), torch.zeros(Sp - S)])
    sid = TP.zone_shapes(v, norms, gp, valid)
    N_b = TP.block_maps(sid)[2]
    sp = 1.0 - (8 + 0.5) / N_b
    t0 = time.perf_counter()
    out = TP.forward_backward(q, k, v, do, gp, sparsity=sp, cdf_threshold=0.9, norms=norms, valid=valid)
    ms = (time.perf_counter() - t0) * 1e3
    return ms, int(out[4]["lens"].sum())


def cpu_baseline(inp, sparsity, cdf, budget_s=12.0, step_pairs=None):
    """The reference's pure-PyTorch path (block-mask selection + masked SDPA)
    restated in torch float32 (oracle/torch_path.py), timed on the host cores
    on the same inputs: zone statistics and shapes, rearrangement + pooling,
    and scores + selection + tile lists at full size; the masked SDPA forward
    + backward (dense over every key of the head, as masked SDPA computes it)
    on seeded query tiles for about budget_s seconds, extrapolated to every
    query tile; config 1 end to end.  value = the kept-block FLOPs of the
    GPU step ((4 + 10) 64 64 D step_pairs, the GPU line's convention; the CPU
    path's own count when step_pairs is None) / the extrapolated CPU step
    time, i.e. the rate at which the host completes the same step."""
    import torch
    from oracle import torch_path as TP
    from prism_amd import a2v_token_norms
    from prism_amd.adapter import padded_grid, valid_mask_for
    threads = _host_threads()
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        grid = inp["grid"]
        gp, _ = padded_grid(grid)
        B, H, D = inp["B"], inp["H"], inp["D"]
        with torch.no_grad():
            q, k, v, do = (_pad_host(inp[n], grid, gp) for n in ("q", "k", "v", "do"))
            norms = _pad_host(a2v_token_norms(inp["res"]), grid, gp)
        valid = valid_mask_for(grid, "cpu")
        sm = 1.0 / math.sqrt(D)
        st = {}
        t0 = time.perf_counter()
        sid = TP.zone_shapes(v, norms, gp, valid)
        st["zone_stats_shapes"] = time.perf_counter() - t0
        t0 = time.perf_counter()
        src, _ = TP.rearrange_index(sid, gp)
        bid, kbt, N_b = TP.block_maps(sid)
        q_re, k_re, v_re = (x.index_select(2, src) for x in (q, k, v))
        do_re = do.index_select(2, src)
        valid_re = None if valid is None else valid[src]
        qm, _, tcount = TP.block_means(q_re, valid_re, bid, N_b)
        km, bcount, _ = TP.block_means(k_re, valid_re, bid, N_b)
        st["rearrange_pool"] = time.perf_counter() - t0
        Nt = q.shape[2] // 64
        t0 = time.perf_counter()
        tiles, lens = [], []
        for h in range(H):
            s = qm[:, h] @ km[:, h].transpose(-1, -2)
            if valid is not None:
                s = s.masked_fill((bcount == 0)[None, None, :], float("-inf"))
            sel = TP.select_blocks(s.reshape(-1, N_b), sparsity, cdf, sm).clamp(max=N_b)
            t, n = TP.tile_lists(sel, kbt, tcount if valid is not None else None, Nt)
            tiles.append(t.view(B, N_b, -1)[:, bid])
            lens.append(n.view(B, N_b)[:, bid])
            del s, sel
        tiles, lens = torch.stack(tiles, 1), torch.stack(lens, 1)
        st["scores_select_lists"] = time.perf_counter() - t0
        sum_lens = int(lens.sum())
        # masked SDPA on seeded query tiles of the same plan
        gen = torch.Generator().manual_seed(0)
        order = torch.randperm(B * H * Nt, generator=gen)
        used, n_tiles, pairs = 0.0, 0, 0
        for r in order.tolist():
            b, rem = divmod(r, H * Nt)
            h, t = divmod(rem, Nt)
            rows = slice(t * 64, (t + 1) * 64)
            t0 = time.perf_counter()
            mask = TP.token_mask(tiles[b, h, t], lens[b, h, t], Nt, valid_re)
            TP.masked_attention(q_re[b, h, rows][None], k_re[b, h][None], v_re[b, h][None], mask[None],
                                do_re[b, h, rows][None])
            used += time.perf_counter() - t0
            n_tiles += 1
            pairs += int(lens[b, h, t])
            if used > budget_s:
                break
        attn_s = used / n_tiles * (B * H * Nt)
        total_s = sum(st.values()) + attn_s
        c1_ms, c1_pairs = cpu_c1_end_to_end()
    finally:
        torch.set_num_threads(prev_threads)
    flops = 14 * 64 * 64 * D * (sum_lens if step_pairs is None else step_pairs)
    return {"value": flops / total_s / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(),
            "ms_per_step_extrapolated": round(total_s * 1e3, 1),
            "stages_ms": {k_: round(v_ * 1e3, 1) for k_, v_ in st.items()},
            "attention_ms_extrapolated": round(attn_s * 1e3, 1),
            "cpu_path_kept_tile_pairs": sum_lens,  # includes the padded query tiles the reference attends for
            "c1_end_to_end_ms": round(c1_ms, 1), "c1_kept_tile_pairs": c1_pairs,
            "sample": (f"torch float32 restatement of the reference's CPU path on {threads} host threads: zone "
                       f"statistics + shapes, rearrangement + pooling, scores + selection + tile lists at full "
                       f"size (measured); masked SDPA fwd+bwd dense over all {q.shape[2]} keys of the head for "
                       f"{n_tiles} random query tiles ({pairs} kept tile pairs, {used:.1f} s), extrapolated to all "
                       f"{B * H * Nt} query tiles (extrapolated); config 1 end to end {c1_ms:.0f} ms")}


# ------------------------------------------------------------------ HBM traffic
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_c4.json")
COPY_BYTES = 2 << 30


def copy_calibration():
    """One device-to-device copy of COPY_BYTES (reads and writes exactly that
    many bytes): the reference dispatch that scales the rocprofv3 FETCH_SIZE /
    WRITE_SIZE counters to bytes."""
    import torch
    x = torch.empty(COPY_BYTES // 4, device="cuda", dtype=torch.float32).fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES}), flush=True)


def _counter_means(csv_path: str, counter: str):
    """kernel name -> mean counter value per dispatch (rocprofv3 --output-format csv)."""
    import csv
    acc = {}
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            acc.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}


def summarize_counters(fetch_csv, write_csv, calib_fetch_csv, calib_write_csv):
    """Write TRAFFIC_FILE: HBM bytes per launch of each prism kernel from the
    FETCH_SIZE and WRITE_SIZE runs, each scaled so that the calibration copy of
    COPY_BYTES reads and writes exactly COPY_BYTES."""
    names = {"bsa_fwd_kernel": "prism_bsa_fwd", "bsa_bwd_dkdv_kernel": "prism_bsa_bwd_dkdv",
             "bsa_bwd_dq_kernel": "prism_bsa_bwd_dq", "bsa_fwd_quad_kernel": "prism_bsa_fwd_quad",
             "bsa_bwd_dq_quad_kernel": "prism_bsa_bwd_dq_quad", "select_kernel": "prism_select_tiles",
             "gather_pool_kernel": "prism_gather_pool", "scatter_rows_kernel": "prism_scatter_rows",
             "block_scores_kernel": "prism_block_scores", "a2v_norms_kernel": "prism_a2v_norms",
             "zone_stats_kernel": "prism_zone_stats", "pair_union_kernel": "prism_pair_union"}
    cf = [v for k, v in _counter_means(calib_fetch_csv, "FETCH_SIZE").items() if "copy" in k]
    cw = [v for k, v in _counter_means(calib_write_csv, "WRITE_SIZE").items() if "copy" in k]
    f_scale = COPY_BYTES / (max(cf) * 1024.0)
    w_scale = COPY_BYTES / (max(cw) * 1024.0)
    fetch = _counter_means(fetch_csv, "FETCH_SIZE")
    write = _counter_means(write_csv, "WRITE_SIZE")
    out = {"copy_bytes": COPY_BYTES, "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
           "unit": "bytes per launch", "kernels": {}}
    for k, fv in fetch.items():
        entry = next((v for sub, v in names.items() if sub in k), None)
        if entry is None or k not in write:
            continue
        fb, wb = fv * 1024.0 * f_scale, write[k] * 1024.0 * w_scale
        out["kernels"][entry] = {"fetch_bytes": round(fb), "write_bytes": round(wb),
                                 "hbm_bytes_per_launch": round(fb + wb)}
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out), flush=True)


def staged_tile_bytes(plan, D: int) -> dict:
    """Bytes the attention kernels copy into LDS per launch: one 64 x D bf16
    tile of each operand per union entry (forward and dQ: K and V over the
    query-side pair or quad unions; dK/dV: Q and dO plus the m2 and delta rows
    over the key-side unions), whether the copy hits in L2 or not."""
    tile = 64 * D * 2
    q_entries = int(plan.qunion[1].sum().item())
    out = {"prism_bsa_fwd": 2 * tile * q_entries, "prism_bsa_bwd_dq": 2 * tile * q_entries}
    quad = getattr(plan, "qquad", None)
    if quad is not None:
        quad_entries = int(quad[1].sum().item())
        out.update({"prism_bsa_fwd_quad": 2 * tile * quad_entries, "prism_bsa_bwd_dq_quad": 2 * tile * quad_entries})
    if plan.kunion is not None:
        out["prism_bsa_bwd_dkdv"] = (2 * tile + 2 * 64 * 4) * int(plan.kunion[1].sum().item())
    return out


def slot_efficiency(plan, sum_lens: int) -> dict:
    """Fraction of the wave-tile slots of the forward and dQ kernels that do
    math: Σlens over (tiles per union) x (union entries), for the pair unions
    and, when the plan has them, the quad unions; and which unions the
    forward and dQ launches of the plan walk."""
    pair = sum_lens / max(1, 2 * int(plan.qunion[1].sum().item()))
    quad = getattr(plan, "qquad", None)
    qeff = None if quad is None else sum_lens / max(1, 4 * int(quad[1].sum().item()))
    walk = {"forward": "quad" if getattr(plan, "quads", False) else "pair",
            "dq": "quad" if getattr(plan, "dq_quads", False) else "pair"}
    return {"union_slot_efficiency": round(pair, 4),
            "quad_union_slot_efficiency": None if qeff is None else round(qeff, 4), "query_unions": walk}


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by the copy calibration),
    or None when no summary for it exists."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


# ------------------------------------------------------------------ measured ceilings
WALL_CLOCK_HZ = 100e6   # s_memrealtime (wall_clock64) counts at a constant 100 MHz
MFMA_FLOPS_PER_CU_CYCLE = 4 * 2 * 32 * 32 * 16 / 32  # one 32x32x16 bf16 MFMA per 32 cycles per SIMD


def measured_ceilings():
    """The device's measured bf16 MFMA, GEMM and HBM rates, beside the
    datasheet's 2.5 PFLOP/s and 8 TB/s:
      mfma_loop  prism_mfma_peak: four chains of v_mfma_f32_32x32x16_bf16 per
                 wave on register operands, two waves per SIMD on every CU,
                 ~0.25 s per launch (no memory traffic): the MFMA rate at the
                 clock the chip holds under full matrix load; best of 3;
      gemm       torch.matmul bf16 8192^3 and F.linear at the A2V bridge shape
                 (302,400 x 5,120 x 5,120) (hipBLASLt), median of 20 and of 5;
      copy       prism_copy_peak over 4 GiB (read + write bytes), best of 10;
      tile stream  prism_tile_stream_peak: the attention kernels' LDS tile
                 copies without their math, over one config-4 head's K and V
                 (189 MB: the Infinity Cache holds it, the L2s do not) and over
                 4 GiB (HBM), ~50 ms per launch after a warm-up, best of 3."""
    import ctypes
    import statistics
    import torch
    from prism_amd import _lib
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    sink = torch.empty(512 * cus, device="cuda", dtype=torch.float32)
    clocks = torch.zeros(2, device="cuda", dtype=torch.int64)
    flops = ctypes.c_int64(0)

    def timed(fn, reps):
        out = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            out.append(a.elapsed_time(b))
        return out

    def mfma(iters):
        _lib.call("prism_mfma_peak", iters, sink.data_ptr(), sink.numel(), clocks.data_ptr(),
                  ctypes.addressof(flops), stream)

    t_probe = timed(lambda: mfma(20000), 2)[-1]
    iters = max(20000, int(20000 * 250.0 / max(t_probe, 1e-3)))
    best = None
    for t in timed(lambda: mfma(iters), 3):
        rate = flops.value / (t * 1e-3) / 1e12
        if best is None or rate > best[0]:
            c = clocks.cpu().tolist()
            best = (rate, t, c[0] / max(c[1], 1) * WALL_CLOCK_HZ / 1e9)
    mfma_tflops, mfma_ms, clk = best
    a = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
    timed(lambda: torch.matmul(a, b), 3)
    g_ms = statistics.median(timed(lambda: torch.matmul(a, b), 20))
    del a, b
    x = torch.randn(302400, 5120, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(5120, 5120, device="cuda", dtype=torch.bfloat16)
    timed(lambda: torch.nn.functional.linear(x, w), 2)
    l_ms = statistics.median(timed(lambda: torch.nn.functional.linear(x, w), 5))
    del x, w
    nbytes = 4 << 30
    src = torch.ones(nbytes // 4, device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)

    def copy():
        _lib.call("prism_copy_peak", src.data_ptr(), dst.data_ptr(), nbytes, stream)

    c_ms = min(timed(copy, 12)[2:])
    assert bool((dst[:: 1 << 20] == 1).all())
    del dst
    ssink = torch.empty(2 * cus, device="cuda", dtype=torch.int32)
    moved = ctypes.c_int64(0)

    def tile_stream(buf, nbytes):
        def run(steps):
            _lib.call("prism_tile_stream_peak", buf.data_ptr(), nbytes, steps, ssink.data_ptr(), ssink.numel(),
                      ctypes.addressof(moved), stream)
        t_probe = timed(lambda: run(1000), 2)[-1]
        steps = max(1000, int(1000 * 50.0 / max(t_probe, 1e-3)))
        t = min(timed(lambda: run(steps), 4)[1:])
        return moved.value / (t * 1e-3) / 1e12
    cache_bytes = 11520 * 16384  # 2 x 5,760 tiles of 64 x 128 bf16: one config-4 head's K and V
    cache_buf = torch.zeros(cache_bytes // 4, device="cuda", dtype=torch.float32)
    stream_cache = tile_stream(cache_buf, cache_bytes)
    stream_hbm = tile_stream(src, nbytes)
    del src, cache_buf
    torch.cuda.empty_cache()
    return {
        "mfma_loop_tflops": round(mfma_tflops, 1), "mfma_loop_ms": round(mfma_ms, 1),
        "mfma_loop_clock_ghz": round(clk, 3),
        "mfma_loop_issue_clock_ghz": round(mfma_tflops * 1e12 / (cus * MFMA_FLOPS_PER_CU_CYCLE) / 1e9, 3),
        "gemm_tflops": round(max(2 * 8192 ** 3 / (g_ms * 1e-3), 2 * 302400 * 5120 * 5120 / (l_ms * 1e-3)) / 1e12, 1),
        "gemm_8192_tflops": round(2 * 8192 ** 3 / (g_ms * 1e-3) / 1e12, 1),
        "gemm_bridge_tflops": round(2 * 302400 * 5120 * 5120 / (l_ms * 1e-3) / 1e12, 1),
        "gemm": "hipBLASLt bf16 (torch.matmul 8192^3, F.linear 302400x5120x5120): the faster of the two",
        "copy_GBps": round(2 * nbytes / (c_ms * 1e-3) / 1e9, 1), "copy": "prism_copy_peak, 4 GiB read + 4 GiB written",
        "tile_stream_TBps": round(stream_cache, 2), "tile_stream_hbm_TBps": round(stream_hbm, 2),
        "tile_stream": "prism_tile_stream_peak: 32 KB stages of two random 16 KB tiles into LDS, the forward's copy "
                       "plan, no math; over 189 MB (Infinity Cache) and over 4 GiB (HBM)",
        "cus": cus,
    }


# ------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--path", default="dynamic", choices=("dynamic", "uniform"),
                    help="dynamic: _run_bsa_dynamic (the headline); uniform: the fixed 4x4x4-chunk branch of "
                         "_run_bsa (flash_attn_bsa_3d) on the same inputs and selection parameters")
    ap.add_argument("--sweep", action="store_true",
                    help="C5: density sweep on the config's shapes (one JSON line of its own, not the headline)")
    ap.add_argument("--bridge", action="store_true",
                    help="the a2v bridge o-projection with fused residual norms (prism_linear_rownorm) at the "
                         "config's tokens and C, against torch F.linear + the norm kernel (one JSON line)")
    ap.add_argument("--dense-lists", action="store_true",
                    help="keep the pair unions as dense pairs x Nt buffers until the backward (bsa_params "
                         "compact_lists=False) instead of compact CSR; reported in config")
    ap.add_argument("--forward-only", action="store_true",
                    help="time the forward alone (inference, no autograd), as BASELINE config 2 is quoted; one JSON "
                         "line of its own, not the headline")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-ceilings", action="store_true", help="skip the measured MFMA / GEMM / copy ceilings")
    ap.add_argument("--cpu-budget", type=float, default=8.0,
                    help="seconds of sampled masked-SDPA work in the CPU baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run one plain device copy of 2 GiB (reference dispatch for the HBM counters)")
    ap.add_argument("--summarize-counters", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "CALIB_FETCH_CSV", "CALIB_WRITE_CSV"),
                    help="write the HBM traffic summary from rocprofv3 counter CSVs and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.summarize_counters:
        summarize_counters(*args.summarize_counters)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path shards by "
              "head across GPUs and is not run multi-GPU here", file=sys.stderr)
        sys.exit(2)

    import torch
    from prism_amd import DynamicBlockSparseAttention, a2v_token_norms, plan_dynamic
    from prism_amd import ops
    from prism_amd.adapter import padded_grid

    torch.backends.cuda.matmul.allow_tf32 = False
    log(f"[bench] config {args.config}: generating inputs")
    inp = make_inputs(args.config)
    if args.sweep:
        run_sweep(args, inp)
        return
    if args.bridge:
        run_bridge(args, inp)
        return
    if args.path == "uniform":
        run_uniform(args, inp)
        return
    B, H, D, S = inp["B"], inp["H"], inp["D"], inp["S"]
    grid = inp["grid"]
    gp, _ = padded_grid(grid)

    # N_b from the shape decision on these inputs -> sparsity giving top-k exactly
    norms0 = a2v_token_norms(inp["res"])
    dyn = DynamicBlockSparseAttention("ivpq", {"dynamic_block_tau_128": 0.15})
    q0 = inp["q"]
    with torch.no_grad():
        from prism_amd.dynamic_block_shape import _gradient_and_shapes
        sid = _gradient_and_shapes(inp["v"], norms0, gp, "ivpq", 0.5, 0.15, 1.0, None, grid)[2]
        N_b = ops.ZoneLayout(sid, gp, grid).N_b
    if inp["sp_only"] is not None:
        sparsity, cdf = inp["sp_only"], None
    else:
        sparsity, cdf = 1.0 - (inp["topk"] + 0.5) / N_b, inp["cdf"]
    compact = not args.dense_lists
    dyn.bsa_params.update({"sparsity": sparsity, "cdf_threshold": cdf, "compact_lists": compact})
    log(f"[bench] N_b={N_b} sparsity={sparsity:.6f} cdf={cdf}")

    fwd_only = bool(args.forward_only)
    q = inp["q"].clone().requires_grad_(not fwd_only)
    k = inp["k"].clone().requires_grad_(not fwd_only)
    v = inp["v"].clone().requires_grad_(not fwd_only)
    do = inp["do"]

    def step():
        if fwd_only:
            with torch.no_grad():
                dyn(q, k, v, grid, a2v_token_norms(inp["res"]))
            return
        q.grad = k.grad = v.grad = None
        norms = a2v_token_norms(inp["res"])
        out = dyn(q, k, v, grid, norms)
        out.backward(do)

    log("[bench] warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log("[bench] timed steps")
    # no cyclic garbage collection inside the timed region (a collection of
    # the earlier steps' plans and events stalled the host for ~50 ms, long
    # enough to leave the GPU idle in a 25 ms forward-only step)
    gc.collect()
    gc.disable()
    # timed region: every C-ABI launch is bracketed by HIP events on its stream
    with ops.kernel_timing() as tm:
        st = torch.cuda.Event(enable_timing=True)
        en = torch.cuda.Event(enable_timing=True)
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        t0 = time.perf_counter()
        st.record()
        marks[0].record()
        for i in range(args.steps):
            step()
            marks[i + 1].record()
        en.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) / args.steps * 1e3
    gc.enable()
    ms = st.elapsed_time(en) / args.steps
    import statistics
    ms_median = statistics.median(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    kt = ops.summarize(tm)  # name -> (launches, average ms per launch)

    # the plan of these inputs (deterministic: identical to the one inside each step)
    with torch.no_grad():
        plan = plan_dynamic(q.detach(), k.detach(), v.detach(), gp, method="ivpq", sparsity=sparsity,
                            cdf_threshold=cdf, audio_token_norms=norms0, input_grid=grid,
                            compact_lists=compact, keep_scores=True)
        plan.build_key_lists()
    # bytes of work lists at their peak (all lists of the call) and those the
    # step keeps from its forward to its backward (the two pair unions, after
    # the forward's settle(), as _DynBSA.forward does)
    list_bytes_peak = plan.list_bytes()
    sum_lens = plan.sum_lens()
    Nt, Nb, Sp = plan.lay.Nt, plan.lay.N_b, plan.S
    density = sum_lens / (B * H * Nt * Nt)
    n_qvalid = int((plan.tile_count > 0).sum().item()) if plan.tile_count is not None else Nt
    density_valid = sum_lens / (B * H * n_qvalid * Nt)  # over query tiles holding a valid token
    # fraction of (wave, key tile) slots of the forward and dQ kernels that do math (slot_efficiency, below)
    fl = 64 * 64 * D * sum_lens  # one 64x64xD product over all kept tile pairs
    kept_flops = (4 if fwd_only else 14) * fl  # FA convention: fwd 4, bwd 10

    # attention kernels: algorithmic FLOPs per launch (executed in parentheses)
    attn = {"prism_bsa_fwd": (4 * fl, 4 * fl), "prism_bsa_bwd_dkdv": (8 * fl, 8 * fl),
            "prism_bsa_bwd_dq": (2 * fl, 6 * fl)}
    attn.update({n + "_quad": attn[n] for n in ("prism_bsa_fwd", "prism_bsa_bwd_dq")})
    X = B * H * Sp * D * 2   # one bf16 [B,H,S_p,D] tile-order tensor (zone grid)
    Xin = B * H * S * D * 2  # one bf16 [B,H,S,D] THW tensor (input grid)
    nnz_tiles = int(plan.sel["ntiles"].sum().item())
    slots = slot_efficiency(plan, sum_lens)
    staged = staged_tile_bytes(plan, D)
    with torch.no_grad():
        plan.settle()
    list_bytes = plan.list_bytes()
    hbm = {  # algorithmic bytes per launch (average over the step's launches of that entry point)
        "prism_zone_stats": H * S * D * 2 + plan.lay.Nz * 25 * D * 4,
        "prism_a2v_norms": S * inp["res"].shape[-1] * 2 + S * 2,
        "prism_gather_pool": (4 * (Xin + X) + X) / 4,  # q, k, v, dO: read THW + write rows; dO also reads O
        "prism_scatter_rows": 2 * Xin,
        "prism_block_scores": 2 * B * H * Nb * D * 4 + B * H * Nb * Nb * 4,
        "prism_select_tiles": B * H * Nb * Nb * 4 + 4 * nnz_tiles + 4 * B * H * Nb,
    }
    breakdown, side = {}, {}
    for name, (n, t) in sorted(kt.items(), key=lambda x: -x[1][0] * x[1][1]):
        if name.endswith(" (side stream)"):
            # launches beside the forward kernel: their events also time the
            # wait for CUs the forward holds, so they are no kernel durations
            side[name[: -len(" (side stream)")]] = {"launches_per_step": n // args.steps,
                                                     "event_ms_incl_wait": round(t, 4)}
            continue
        e = {"launches_per_step": n // args.steps, "ms": round(t, 4)}
        if name in attn:
            alg, exe = attn[name]
            e.update(tflops=round(alg / (t * 1e-3) / 1e12, 1), executed_tflops=round(exe / (t * 1e-3) / 1e12, 1),
                     mfma_frac=round(alg / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4))
            if name in staged:
                e.update(staged_tile_GB=round(staged[name] / 1e9, 2),
                         staged_tile_TBps=round(staged[name] / (t * 1e-3) / 1e12, 2))
        elif name in hbm:
            e.update(GBps=round(hbm[name] / (t * 1e-3) / 1e9, 1),
                     hbm_frac=round(hbm[name] / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))
        breakdown[name] = e
    dom = max((n for n in kt if n in attn), key=lambda n: kt[n][1])
    dom_ms = kt[dom][1]
    roof = {"kernel": dom, "bound": "mfma", "achieved": round(attn[dom][0] / (dom_ms * 1e-3) / 1e12, 2),
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(attn[dom][0] / (dom_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            # the committed counter summary is of config 4's launches
            "traffic": measured_traffic(dom) if args.config == "c4" else None}
    att_ms = sum(kt[n][1] for n in attn if n in kt)

    ceil = None
    if not args.no_ceilings:
        log("[bench] measured ceilings (MFMA loop, hipBLASLt GEMM, copy)")
        ceil = measured_ceilings()
        pm, pg, ph = ceil["mfma_loop_tflops"], ceil["gemm_tflops"], ceil["copy_GBps"]
        roof.update(peak_measured=pm, frac_measured=round(roof["achieved"] / pm, 4),
                    peak_measured_kind="MFMA loop at the sustained clock (prism_mfma_peak)",
                    gemm_peak_measured=pg, frac_gemm=round(roof["achieved"] / pg, 4),
                    clock_ghz_mfma_loop=ceil["mfma_loop_clock_ghz"])
        for name, e in breakdown.items():
            if "mfma_frac" in e:
                e["mfma_frac_measured"] = round(e["tflops"] / pm, 4)
            if "hbm_frac" in e:
                e["hbm_frac_measured"] = round(e["GBps"] / ph, 4)
            if "staged_tile_TBps" in e:
                e["tile_stream_frac_measured"] = round(e["staged_tile_TBps"] / ceil["tile_stream_TBps"], 4)

    dense = None
    if not args.no_dense:
        log("[bench] dense SDPA comparison")
        qd = inp["q"].clone().requires_grad_(True)
        kd = inp["k"].clone().requires_grad_(True)
        vd = inp["v"].clone().requires_grad_(True)

        def dstep():
            if fwd_only:
                with torch.no_grad():
                    torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)
                return
            qd.grad = kd.grad = vd.grad = None
            o = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)
            o.backward(do)

        try:
            dmean, dms, _ = time_region(dstep, DENSE_STEPS, DENSE_WARMUP)
            dense = {"impl": f"torch SDPA (ROCm) {'forward' if fwd_only else 'fwd+bwd'}, same shape, unpadded",
                     "ms": round(dms, 2),
                     "ms_mean": round(dmean, 2), "timing": f"median of {DENSE_STEPS} after {DENSE_WARMUP} warm-ups",
                     "tflops": round((4 if fwd_only else 14) * S * S * D * B * H / (dms * 1e-3) / 1e12, 1),
                     "speedup_sparse_vs_dense": round(dms / ms_median, 2)}
        except Exception as e:  # report, do not fail the bench
            dense = {"error": repr(e)[:200]}
        del qd, kd, vd
        if not fwd_only:
            log("[bench] own kernels at 100% density (every tile listed)")
            dense.update(own_dense_point(inp, grid, gp, ms_median, q, k, v, do))

    cpu = None
    sel_agree = None
    if not args.no_cpu and not fwd_only:
        log("[bench] CPU baseline (the reference's torch path, float32, host cores)")
        cpu = cpu_baseline(inp, sparsity, cdf, args.cpu_budget, step_pairs=sum_lens)
        log("[bench] selection vs the reference's torch sequence (GPU and CPU kernels, same scores)")
        sel_agree = selection_vs_torch(plan, sparsity, cdf, 1 / math.sqrt(D))
    plan.scores = None

    value = kept_flops / (ms * 1e-3) / 1e12
    rec = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.config}: BASELINE config {'4 (2K fwd+bwd)' if args.config == 'c4' else args.config}"
                               + (" forward only" if fwd_only else ""),
                   "B": B, "H": H, "D": D, "grid": list(grid), "grid_padded": list(gp),
                   "audio_tokens": CONFIGS[args.config][4], "topk": inp["topk"], "cdf_threshold": cdf,
                   "sparsity": sparsity, "N_b": Nb, "sum_lens": sum_lens, "density": round(density, 4),
                   "density_valid_q": round(density_valid, 4), **slots,
                   "mfma_util_step": round(value / PEAK_BF16_TFLOPS, 4), "wall_ms_per_step": round(wall_ms, 3),
                   "ms_per_step_median": round(ms_median, 3),
                   "compact_lists": compact, "list_bytes": list_bytes, "list_bytes_peak": list_bytes_peak,
                   "attention_ms": round(att_ms, 3),
                   "attention_mfma_util": round(kept_flops / (att_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                   "selection_vs_reference_torch": sel_agree},
        "roofline": roof, "cpu_baseline": cpu, "dense": dense, "breakdown": breakdown,
        "side_stream": {"note": "key-side list builds launched beside the forward kernel on a second stream; "
                                "event times include waiting for the CUs the forward holds (kernel durations: "
                                "rocprofv3 kernel trace)", "launches": side},
    }
    if ceil is not None:
        rec["config"]["mfma_util_step_measured"] = round(value / ceil["mfma_loop_tflops"], 4)
        rec["hbm_peak_measured"] = {"GBps": ceil["copy_GBps"], "kernel": ceil["copy"],
                                    "frac_of_nominal": round(ceil["copy_GBps"] / PEAK_HBM_GBS, 4)}
        rec["ceilings"] = ceil
    print(json.dumps(rec), flush=True)


def own_dense_point(inp, grid, gp, sparse_ms, q, k, v, do):
    """The same step with every block selected (sparsity 0: every query tile
    lists every key tile that holds a valid token, i.e. dense attention
    through these kernels), median of 3 after 1 warm-up."""
    import torch
    from prism_amd import DynamicBlockSparseAttention, a2v_token_norms, plan_dynamic
    B, H, D, S = inp["B"], inp["H"], inp["D"], inp["S"]
    full = DynamicBlockSparseAttention("ivpq", {"dynamic_block_tau_128": 0.15})
    full.bsa_params.update({"sparsity": 0.0, "cdf_threshold": None})

    def step():
        q.grad = k.grad = v.grad = None
        out = full(q, k, v, grid, a2v_token_norms(inp["res"]))
        out.backward(do)

    _, oms, _ = time_region(step, 3, 1)
    with torch.no_grad():
        plan = plan_dynamic(q.detach(), k.detach(), v.detach(), gp, method="ivpq", sparsity=0.0,
                            cdf_threshold=None, audio_token_norms=a2v_token_norms(inp["res"]), input_grid=grid)
        pairs = plan.sum_lens()
        Nt = plan.lay.Nt
    del plan
    torch.cuda.empty_cache()
    return {"own_kernel_impl": "this path with sparsity 0 (every key tile with a valid token listed), fwd+bwd",
            "own_kernel_ms": round(oms, 2), "own_kernel_density": round(pairs / (B * H * Nt * Nt), 4),
            "own_kernel_kept_block_tflops": round(14 * 64 * 64 * D * pairs / (oms * 1e-3) / 1e12, 1),
            "own_kernel_dense_equivalent_tflops": round(14 * S * S * D * B * H / (oms * 1e-3) / 1e12, 1),
            "speedup_sparse_vs_own_dense": round(oms / sparse_ms, 2),
            "crossover_note": "vs torch SDPA the sparse step wins at every density including 100% (bench.py "
                              "--sweep); vs the own dense point it wins below 100%, where it is the same "
                              "computation"}


def selection_vs_torch(plan, sparsity, cdf, sm):
    """Rows whose selected block set differs from the reference's torch op
    sequence (bsa_interface.py:235-304) in float32 on the same scores, with
    torch's GPU and CPU kernels (the checker of oracle/torch_path.py)."""
    from oracle import torch_path as TP
    from prism_amd import ops
    N_b = plan.lay.N_b
    scores = plan.scores.view(-1, N_b)
    ours = ops.select_tiles(scores, sparsity, cdf, sm, plan.lay.block_first_tile, plan.tile_count, want_blocks=True)
    out = TP.selection_agreement(scores, ours["sel_blocks"], ours["nsel"], sparsity, cdf, sm)
    out["rows"] = int(scores.shape[0])
    return out


SWEEP_DENSITIES = (0.05, 0.10, 0.25, 0.50, 1.00)


def run_sweep(args, inp):
    """C5: density sweep on the C4 shapes.  Shape ids uniform over the 13
    candidates (seeded) and passed as shape_ids=; top-k only with
    k = round(d N_b) for d in SWEEP_DENSITIES (sparsity = 1 - (k + 0.5) / N_b,
    so that int((1 - s) N_b) = k, bsa_interface.py:289; s = 0 for k = N_b);
    fwd + bwd of flash_attn_bsa_3d_dynamic per density against torch SDPA
    fwd + bwd on the same unpadded shape.  Prints one JSON line with the
    per-density step time, kept-block TFLOP/s and realised density, the dense
    time, and the density at which the sparse step stops being faster."""
    import torch
    from prism_amd import flash_attn_bsa_3d_dynamic, ops, plan_dynamic
    from prism_amd.adapter import padded_grid
    from prism_amd.dynamic_block_shape import ALL_CANDIDATE_SHAPES
    B, H, D, S = inp["B"], inp["H"], inp["D"], inp["S"]
    grid = inp["grid"]
    gp, _ = padded_grid(grid)
    Nz = (gp[0] // 8) * (gp[1] // 8) * (gp[2] // 8)
    gen = torch.Generator(device="cuda").manual_seed(5)
    sid = torch.randint(0, len(ALL_CANDIDATE_SHAPES), (Nz,), generator=gen, device="cuda", dtype=torch.int64)
    N_b = ops.ZoneLayout(sid, gp, grid).N_b
    q = inp["q"].clone().requires_grad_(True)
    k = inp["k"].clone().requires_grad_(True)
    v = inp["v"].clone().requires_grad_(True)
    do = inp["do"]
    rows = []
    for d in SWEEP_DENSITIES:
        kk = max(1, min(N_b, round(d * N_b)))
        sp = 0.0 if kk == N_b else 1.0 - (kk + 0.5) / N_b

        def step():
            q.grad = k.grad = v.grad = None
            out = flash_attn_bsa_3d_dynamic(q, k, v, gp, method="ivpq", sparsity=sp, cdf_threshold=None,
                                            shape_ids=sid, input_grid=grid)
            out.backward(do)

        log(f"[sweep] density {d}: k={kk} of N_b={N_b}")
        ms, _, _ = time_region(step, args.steps, args.warmup)
        with torch.no_grad():
            plan = plan_dynamic(q.detach(), k.detach(), v.detach(), gp, method="ivpq", sparsity=sp,
                                cdf_threshold=None, shape_ids=sid, input_grid=grid)
        sum_lens = plan.sum_lens()
        Nt = plan.lay.Nt
        fl = 64 * 64 * D * sum_lens
        rows.append({"target_density": d, "k": kk, "density": round(sum_lens / (B * H * Nt * Nt), 4),
                     "ms_per_step": round(ms, 2), "tflops": round(14 * fl / (ms * 1e-3) / 1e12, 1)})
        del plan
        torch.cuda.empty_cache()
    qd = inp["q"].clone().requires_grad_(True)
    kd = inp["k"].clone().requires_grad_(True)
    vd = inp["v"].clone().requires_grad_(True)

    def dstep():
        qd.grad = kd.grad = vd.grad = None
        o = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)
        o.backward(do)

    log("[sweep] dense SDPA")
    _, dms, _ = time_region(dstep, DENSE_STEPS, DENSE_WARMUP)
    # the sparse step's time grows with density; first density where it is no
    # longer faster than dense, linearly interpolated (None: faster everywhere)
    def crossover(dense_ms):
        for a_, b_ in zip(rows, rows[1:]):
            if a_["ms_per_step"] < dense_ms <= b_["ms_per_step"]:
                t = (dense_ms - a_["ms_per_step"]) / (b_["ms_per_step"] - a_["ms_per_step"])
                return round(a_["density"] + t * (b_["density"] - a_["density"]), 4)
        return None

    cross = crossover(dms)
    # k = N_b: every tile with a valid token listed, the same kernels run dense;
    # against it the sparse step is faster at every lower density (the times
    # rise monotonically) and equal at that density
    own = rows[-1]
    monotonic = all(a_["ms_per_step"] < b_["ms_per_step"] for a_, b_ in zip(rows, rows[1:]))
    cross_own = own["density"] if monotonic else crossover(own["ms_per_step"])
    print(json.dumps({
        "metric": "C5 density sweep: sparse fwd+bwd ms per step vs dense SDPA fwd+bwd",
        "config": {"workload": "c5: C4 shapes, seeded uniform shape ids, top-k only", "B": B, "H": H, "D": D,
                   "grid": list(grid), "grid_padded": list(gp), "N_b": N_b},
        "steps": args.steps, "warmup": args.warmup, "dtype": "bf16", "data": "synthetic",
        "sweep": rows,
        "dense": {"impl": "torch SDPA (ROCm) fwd+bwd, same shape, unpadded", "ms": round(dms, 2),
                  "tflops": round(14 * S * S * D * B * H / (dms * 1e-3) / 1e12, 1),
                  "own_kernel_ms": own["ms_per_step"], "own_kernel_density": own["density"],
                  "own_kernel_dense_equivalent_tflops": round(14 * S * S * D * B * H / (own["ms_per_step"] * 1e-3)
                                                              / 1e12, 1)},
        "crossover_density": cross,
        "crossover_note": ("vs torch SDPA: " + ("sparse wins at every density, including 100%" if cross is None
                                                 else f"crossover at density {cross}")
                           + f"; vs the own dense point (k = N_b, density {own['density']}): crossover at "
                           f"{cross_own}, i.e. sparse wins at every lower density"),
        "crossover_density_vs_own_dense": cross_own}))


def run_bridge(args, inp):
    """The a2v bridge output projection of the config (residual = x W^T + b,
    interactionv2.py:348; M = video tokens, N = K = C) with the per-token
    residual norms (wan_video_dit.py:742-752): fused into this build's GEMM
    epilogue (prism_linear_rownorm) and unfused (torch's F.linear, i.e.
    hipBLASLt, followed by prism_a2v_norms): median ms of each, the GEMM
    alone, and the fused kernel's bf16 MFMA rate (2 M N K flop)."""
    import torch
    from prism_amd import ops
    S, C = inp["S"], CONFIGS[args.config][5]
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(S, C, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(C, C, generator=g, device="cuda") / C ** 0.5).to(torch.bfloat16)
    b = (0.1 * torch.randn(C, generator=g, device="cuda")).to(torch.bfloat16)
    del inp
    torch.cuda.empty_cache()
    steps, warm = max(args.steps, 10), max(args.warmup, 3)
    with ops.kernel_timing() as tm:
        fmean, fmed, _ = time_region(lambda: ops.linear_rownorm(x, w, b), steps, warm)
    kt = ops.summarize(tm)
    umean, umed, _ = time_region(lambda: ops.a2v_norms(torch.nn.functional.linear(x, w, b)), steps, warm)
    gmean, gmed, _ = time_region(lambda: torch.nn.functional.linear(x, w, b), steps, warm)
    flop = 2.0 * S * C * C
    print(json.dumps({
        "metric": "a2v bridge o-projection + residual norms (fused epilogue) ms",
        "config": {"workload": f"{args.config}: M={S} video tokens, N=K=C={C}, bf16, bias"},
        "steps": steps, "warmup": warm, "dtype": "bf16", "data": "synthetic",
        "fused_ms": round(fmed, 3), "fused_ms_mean": round(fmean, 3),
        "fused_tflops": round(flop / (fmed * 1e-3) / 1e12, 1),
        "fused_mfma_frac": round(flop / (fmed * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "unfused_torch_linear_plus_norms_ms": round(umed, 3),
        "speedup_fused_vs_unfused": round(umed / fmed, 3),
        "torch_linear_alone_ms": round(gmed, 3),
        "breakdown": {k: {"launches": n // steps, "ms": round(t, 4)} for k, (n, t) in kt.items()}}), flush=True)


def run_uniform(args, inp):
    """The uniform-shape branch of _run_bsa (4x4x4 chunks, flash_attn_bsa_3d
    with the grid padded to whole chunks) fwd + bwd on the config's inputs,
    top-k + cumulative threshold as the headline.  Prints one JSON line of the
    headline schema with workload "<config>-uniform"."""
    import torch
    from prism_amd import ops
    from prism_amd.adapter import run_bsa_uniform
    from prism_amd.uniform_block_attention import plan_chunked
    B, H, D, S = inp["B"], inp["H"], inp["D"], inp["S"]
    grid = inp["grid"]
    chunk = (4, 4, 4)
    lq = ops.ChunkLayout(grid, chunk, "cuda")
    N_b = lq.N_b
    if inp["sp_only"] is not None:
        sparsity, cdf = inp["sp_only"], None
    else:
        sparsity, cdf = 1.0 - (inp["topk"] + 0.5) / N_b, inp["cdf"]
    params = {"sparsity": sparsity, "cdf_threshold": cdf, "chunk_3d_shape_q": list(chunk),
              "chunk_3d_shape_k": list(chunk)}
    log(f"[bench] uniform: padded grid {lq.pgrid} N_b={N_b} sparsity={sparsity:.6f} cdf={cdf}")
    q = inp["q"].clone().requires_grad_(True)
    k = inp["k"].clone().requires_grad_(True)
    v = inp["v"].clone().requires_grad_(True)
    do = inp["do"]

    def step():
        q.grad = k.grad = v.grad = None
        out = run_bsa_uniform(q, k, v, grid, params)
        out.backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log("[bench] timed steps")
    gc.collect()
    gc.disable()  # no cyclic garbage collection inside the timed region
    with ops.kernel_timing() as tm:
        st = torch.cuda.Event(enable_timing=True)
        en = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        st.record()
        for _ in range(args.steps):
            step()
        en.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) / args.steps * 1e3
    gc.enable()
    ms = st.elapsed_time(en) / args.steps
    kt = ops.summarize(tm)
    with torch.no_grad():
        plan = plan_chunked(q.detach(), k.detach(), v.detach(), lq, lq, sparsity=sparsity, cdf_threshold=cdf,
                            sm_scale=1 / math.sqrt(D))
    sum_lens = plan.sum_lens()
    slots = slot_efficiency(plan, sum_lens)
    with torch.no_grad():
        plan.key_lists()
    staged = staged_tile_bytes(plan, D)
    fl = 64 * 64 * D * sum_lens
    kept_flops = 14 * fl
    attn = {"prism_bsa_fwd": (4 * fl, 4 * fl), "prism_bsa_bwd_dkdv": (8 * fl, 8 * fl),
            "prism_bsa_bwd_dq": (2 * fl, 6 * fl)}
    attn.update({n + "_quad": attn[n] for n in ("prism_bsa_fwd", "prism_bsa_bwd_dq")})
    X_in, X_rows = B * H * S * D * 2, B * H * lq.rows * D * 2
    hbm = {"prism_chunk_gather_pool": (4 * (X_in + X_rows) + X_rows) / 4,  # q, k, v, dO (+ O for delta)
           "prism_chunk_scatter_rows": X_rows + X_in,
           "prism_block_scores": 2 * B * H * N_b * D * 4 + B * H * N_b * N_b * 4,
           "prism_select_tiles": B * H * N_b * N_b * 4 + 4 * int(plan.sel["ntiles"].sum().item()) + 4 * B * H * N_b}
    breakdown = {}
    for name, (n, t) in sorted(kt.items(), key=lambda x: -x[1][0] * x[1][1]):
        if name.endswith(" (side stream)"):
            continue  # event times that include waiting beside the forward kernel
        e = {"launches_per_step": n // args.steps, "ms": round(t, 4)}
        if name in attn:
            alg, exe = attn[name]
            e.update(tflops=round(alg / (t * 1e-3) / 1e12, 1), executed_tflops=round(exe / (t * 1e-3) / 1e12, 1),
                     mfma_frac=round(alg / (t * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4))
            if name in staged:
                e.update(staged_tile_GB=round(staged[name] / 1e9, 2),
                         staged_tile_TBps=round(staged[name] / (t * 1e-3) / 1e12, 2))
        elif name in hbm:
            e.update(GBps=round(hbm[name] / (t * 1e-3) / 1e9, 1),
                     hbm_frac=round(hbm[name] / (t * 1e-3) / 1e9 / PEAK_HBM_GBS, 4))
        breakdown[name] = e
    dom = max((n for n in kt if n in attn), key=lambda n: kt[n][1])
    dom_ms = kt[dom][1]
    att_ms = sum(kt[n][1] for n in attn if n in kt)
    value = kept_flops / (ms * 1e-3) / 1e12
    rec = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.config}-uniform: flash_attn_bsa_3d, 4x4x4 chunks (_run_bsa uniform branch)",
                   "B": B, "H": H, "D": D, "grid": list(grid), "grid_padded": list(lq.pgrid), "chunk": list(chunk),
                   "topk": inp["topk"], "cdf_threshold": cdf, "sparsity": sparsity, "N_b": N_b,
                   "cpu_path_kept_tile_pairs": sum_lens,  # includes the padded query tiles the reference attends for "density": round(sum_lens / (B * H * lq.Nt * lq.Nt), 4),
                   **slots, "wall_ms_per_step": round(wall_ms, 3),
                   "attention_ms": round(att_ms, 3),
                   "attention_mfma_util": round(kept_flops / (att_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)},
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(attn[dom][0] / (dom_ms * 1e-3) / 1e12, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(attn[dom][0] / (dom_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4), "traffic": None},
        "cpu_baseline": None, "breakdown": breakdown,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
