"""Deterministic synthetic inputs for the five benchmark configurations.

All draws use torch generators (on the target device for large sizes); values
are drawn in fp32 and cast to fp16.  d = 128 everywhere.

  c1  B1  H32       S4096    Q/K/V ~ N(0, 1/128), seed 0
  c2  B8  H32       S32768   K ~ N(0, 1/128); per (b,h) a random 5% of keys are
                             k = 0.3 q + sqrt(0.91) z (correlation 0.3 with q); seed 1
  c3  B8  H32       S65536   Q/K/V ~ N(0, 1/128), K and V rows scaled by a
                             per-(b,h,s) LogNormal(0, 0.25) factor; seed 2
  c4  B4  Hq32/Hkv8 S16384 prefill + 256 decode steps, N(0, 1/128); seed 3
  c5  B16 Hq32/Hkv8 S131072  K/V ~ N(0, 1/128) with 4 seeded outlier channels
                             per kv head scaled x10; seed 4; top 10% residual
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

D = 128
SIGMA = 1.0 / math.sqrt(128.0)


@dataclass(frozen=True)
class Config:
    name: str
    batch: int
    n_heads: int
    n_kv_heads: int
    seq_len: int
    seed: int
    head_dim: int = D


CONFIGS = {
    "c1": Config("c1", 1, 32, 32, 4096, 0),
    "c2": Config("c2", 8, 32, 32, 32768, 1),
    "c3": Config("c3", 8, 32, 32, 65536, 2),
    "c4": Config("c4", 4, 32, 8, 16384, 3),
    "c5": Config("c5", 16, 32, 8, 131072, 4),
}
C4_DECODE_STEPS = 256


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal(shape, gen, device, std=SIGMA):
    return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std)


def make_qkv(cfg: Config, device="cuda", seq_len=None):
    """Q [B, Hq, d], K/V [B, Hkv, S, d] fp16 for c1/c3/c4/c5 (c2: see make_c2)."""
    S = cfg.seq_len if seq_len is None else seq_len
    g = _gen(device, cfg.seed)
    B, Hq, Hkv, d = cfg.batch, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    q = normal((B, Hq, d), g, device)
    k = normal((B, Hkv, S, d), g, device)
    v = normal((B, Hkv, S, d), g, device)
    if cfg.name == "c3":
        sk = torch.exp(normal((B, Hkv, S, 1), g, device, std=0.25))
        sv = torch.exp(normal((B, Hkv, S, 1), g, device, std=0.25))
        k = k * sk
        v = v * sv
    if cfg.name == "c5":
        # 4 outlier channels per kv head, chosen with a seeded permutation
        ch = torch.stack([torch.randperm(d, generator=g, device=device)[:4] for _ in range(Hkv)])
        scale = torch.ones((Hkv, d), device=device)
        scale.scatter_(1, ch, 10.0)
        k = k * scale[None, :, None, :]
        v = v * scale[None, :, None, :]
    return q.half(), k.half().contiguous(), v.half().contiguous()


def make_c2(cfg: Config = CONFIGS["c2"], device="cuda", seq_len=None):
    """Binary-scoring workload: Q, K [B, H, S, d]; 5% of keys per (b,h)
    correlated with q at rho = 0.3.  Returns (q, k, correlated_mask)."""
    S = cfg.seq_len if seq_len is None else seq_len
    g = _gen(device, cfg.seed)
    B, H, d = cfg.batch, cfg.n_heads, cfg.head_dim
    q = normal((B, H, d), g, device)
    k = normal((B, H, S, d), g, device)
    z = normal((B, H, S, d), g, device)
    mask = torch.rand((B, H, S), generator=g, device=device) < 0.05
    corr = 0.3 * q[:, :, None, :] + math.sqrt(1 - 0.09) * z
    k = torch.where(mask[..., None], corr, k)
    return q.half(), k.half().contiguous(), mask


def make_c2_values(cfg: Config = CONFIGS["c2"], device="cuda", seq_len=None):
    """V [B, H, S, d] for c2's binary attention: N(0, 1/128), seed cfg.seed + 10
    (the configuration names no V distribution; scoring does not depend on it)."""
    S = cfg.seq_len if seq_len is None else seq_len
    g = _gen(device, cfg.seed + 10)
    return normal((cfg.batch, cfg.n_heads, S, cfg.head_dim), g, device).half().contiguous()


def algorithmic_bytes_per_key(d=D, residual=True):
    """Bytes of one K or V vector that attention must read: d/8 + 2 (+ d/2 + 2)."""
    return d // 8 + 2 + ((d // 2 + 2) if residual else 0)


def kendall_tau_ab(x, y):
    """Kendall tau-a and tau-b of two score vectors (numpy, one head), in
    O(n log n).  tau-a = (C - D) / (n (n - 1) / 2) with tied pairs counted as
    neither concordant nor discordant: the reference's own statistic
    (tests/test_correctness.cu:58-71); tau-b divides C - D by
    sqrt((n0 - n1)(n0 - n2)) instead (n1, n2: pairs tied in x, in y)."""
    import numpy as np
    from scipy.stats import kendalltau

    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    n = x.size
    n0 = n * (n - 1) / 2.0
    if n0 == 0:
        return 1.0, 1.0

    def tied_pairs(a):
        _, c = np.unique(a, return_counts=True)
        return float((c * (c - 1) / 2.0).sum())

    tb = float(kendalltau(x, y).statistic)
    cd = tb * np.sqrt((n0 - tied_pairs(x)) * (n0 - tied_pairs(y)))
    return float(cd / n0), tb
