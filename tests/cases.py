"""Seeded synthetic inputs shared by the tests (small versions of the
BASELINE configs).  Everything is generated on the CPU with numpy so the
oracle and the GPU see identical bits."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16)."""
    return O.f32_to_bf16_bits(x)


def lowrank_zone_tensor(rng, B, H, grid, D, rank=8, scale=2.0, noise=1.0):
    """N(0, noise^2) plus a per-zone rank-`rank` structure with smooth
    t/h/w modulation, so zone variances and anisotropies differ."""
    T, Hg, Wg = grid
    x = rng.standard_normal((B, H, T, Hg, Wg, D)).astype(np.float32) * noise
    ZT, ZH, ZW = T // 8, Hg // 8, Wg // 8
    for zt in range(ZT):
        for zh in range(ZH):
            for zw in range(ZW):
                basis = rng.standard_normal((rank, D)).astype(np.float32)
                amp = rng.uniform(0, scale)
                wt, wh, ww = rng.dirichlet([1.0, 1.0, 1.0])
                t = np.linspace(0, 1, 8)[:, None, None]
                h = np.linspace(0, 1, 8)[None, :, None]
                w = np.linspace(0, 1, 8)[None, None, :]
                coef = []
                for r in range(rank):
                    f = rng.uniform(0.5, 3.0, size=3)
                    ph = rng.uniform(0, 2 * np.pi, size=3)
                    c = (wt * np.sin(f[0] * np.pi * t + ph[0]) + wh * np.sin(f[1] * np.pi * h + ph[1])
                         + ww * np.sin(f[2] * np.pi * w + ph[2]))
                    coef.append(c)
                coef = np.stack(coef, -1).astype(np.float32)  # [8,8,8,rank]
                blockv = amp * (coef @ basis)                 # [8,8,8,D]
                x[:, :, zt * 8:(zt + 1) * 8, zh * 8:(zh + 1) * 8, zw * 8:(zw + 1) * 8, :] += blockv[None, None]
    return x.reshape(B, H, T * Hg * Wg, D)


def padded_case(seed, B, H, grid_real, D, *, lowrank=False, audio_tokens=0, C=None):
    """Inputs of _run_bsa_dynamic after its padding: q, k, v [B,H,S_p,D]
    float32 (zeros in padding), valid mask [S_p] uint8, audio norms [S_p]
    float32 or None, padded grid."""
    rng = np.random.default_rng(seed)
    T, Hg, Wg = grid_real
    Tp, Hp, Wp = [(x + 7) // 8 * 8 for x in grid_real]
    S = T * Hg * Wg
    if lowrank:
        full = [lowrank_zone_tensor(rng, B, H, (Tp, Hp, Wp), D) for _ in range(3)]
        qkv = [f.reshape(B, H, Tp, Hp, Wp, D)[:, :, :T, :Hg, :Wg].reshape(B, H, S, D) for f in full]
        # unit marginal variance (q/k of the model are RMS-normalised): the
        # structure keeps its scale relative to the noise
        qkv = [(x / x.std()).astype(np.float32) for x in qkv]
    else:
        qkv = [rng.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(3)]
    out = []
    for x in qkv:
        p = np.zeros((B, H, Tp, Hp, Wp, D), np.float32)
        p[:, :, :T, :Hg, :Wg] = x.reshape(B, H, T, Hg, Wg, D)
        out.append(p.reshape(B, H, -1, D))
    valid = np.zeros((Tp, Hp, Wp), np.uint8)
    valid[:T, :Hg, :Wg] = 1
    norms = None
    if audio_tokens:
        # A2V residual: cross-attention of video queries (head-concatenated)
        # over audio keys/values, as the bridge produces it
        C = C or H * D
        qv = qkv[0][0].transpose(1, 0, 2).reshape(S, H * D)[:, :C]
        ka = rng.standard_normal((audio_tokens, C)).astype(np.float32)
        va = rng.standard_normal((audio_tokens, C)).astype(np.float32)
        s = qv @ ka.T / np.sqrt(C)
        s -= s.max(1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(1, keepdims=True)
        res = (p @ va).astype(np.float32)
        n = np.sqrt((res.astype(np.float64) ** 2).sum(1)).astype(np.float32)
        pn = np.zeros((Tp, Hp, Wp), np.float32)
        pn[:T, :Hg, :Wg] = n.reshape(T, Hg, Wg)
        norms = pn.reshape(-1)
    return dict(q=out[0], k=out[1], v=out[2], valid=valid.reshape(-1), norms=norms, grid=(Tp, Hp, Wp),
                grid_real=grid_real)
