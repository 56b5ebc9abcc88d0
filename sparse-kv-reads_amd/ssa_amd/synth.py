"""Synthetic Qwen3-shaped decode caches whose keys cluster by direction.

The reference has no generator for this (its tests draw ``randn + offset`` keys); the benchmark
configurations describe one, fixed here once:

  per (sequence, KV head):
    mu      ~ N(0, I_d) * S_MU                          shared mean of the keys
    c_i     uniform on the unit sphere, i < centers     cluster centres
    pi      ~ Dirichlet(ALPHA)                          ragged cluster popularity
  per key j:  i ~ pi,  u = unit(KAPPA * c_i + N(0, I_d)),  r = R0 * exp(SIGMA * N(0, 1)),
              k_j = mu + r * u
  values ~ N(0, 1); each query head q = Q_NORM * unit(KAPPA * c_i* + N(0, I_d)) near one centre.

KAPPA = 20 gives a mean cosine of about KAPPA / sqrt(KAPPA^2 + d - 1) = 0.87 to the centre
(a tangent-normal approximation of a von Mises-Fisher draw). Sequence ``b`` of a batch uses
seed ``1000 * seed + b``; generation runs in float64 on a seeded CPU generator when the cache is
small (bit-identical on every machine with this torch build) and in float32 on the GPU otherwise.
"""

from __future__ import annotations

import torch

S_MU, R0, SIGMA, KAPPA, ALPHA, Q_NORM = 1.0, 10.0, 0.3, 20.0, 1.0, 10.0   # ALPHA is fixed at 1
CONSTANTS = dict(s_mu=S_MU, r0=R0, sigma=SIGMA, kappa=KAPPA, alpha=ALPHA, q_norm=Q_NORM)
_CPU_LIMIT = 1 << 26      # elements per sequence generated on the CPU


def _unit(x):
    return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def _sequence(H_kv, H, n, d, centers, seed, gen_device, fdt):
    g = torch.Generator(device=gen_device).manual_seed(seed)
    kw = dict(device=gen_device, dtype=fdt, generator=g)
    mu = torch.randn(H_kv, 1, d, **kw) * S_MU
    cen = _unit(torch.randn(H_kv, centers, d, **kw))
    # Dirichlet(1) weights from the seeded generator: -log(U) is Gamma(1)
    pi = -torch.log(torch.rand(H_kv, centers, **kw).clamp_min(1e-30))
    pi = pi / pi.sum(-1, keepdim=True)
    which = torch.multinomial(pi.to(gen_device), n, replacement=True, generator=g)          # [H_kv, n]
    u = _unit(KAPPA * torch.gather(cen, 1, which.unsqueeze(-1).expand(H_kv, n, d)) + torch.randn(H_kv, n, d, **kw))
    r = R0 * torch.exp(SIGMA * torch.randn(H_kv, n, 1, **kw))
    K = mu + r * u
    V = torch.randn(H_kv, n, d, **kw)
    G = H // H_kv
    qc = torch.randint(0, centers, (H_kv, G), device=gen_device, generator=g)
    q = Q_NORM * _unit(KAPPA * torch.gather(cen, 1, qc.unsqueeze(-1).expand(H_kv, G, d))
                       + torch.randn(H_kv, G, d, **kw))
    return K, V, q.reshape(H, d), which


def make_cache(B: int, H_kv: int, n: int, d: int = 128, *, H: int | None = None, centers: int = 256,
               capacity: int | None = None, seed: int = 0, dtype=torch.bfloat16, device="cpu",
               gen_device: str | None = None):
    """Keys, values and one decode query per head: ``K, V [B, H_kv, capacity, d]`` (positions
    ``>= n`` zero), ``q [B, H, d]``, and each key's true centre ``which [B, H_kv, n]``."""
    H = 2 * H_kv if H is None else H
    cap = n if capacity is None else capacity
    K = torch.zeros(B, H_kv, cap, d, dtype=dtype, device=device)
    V = torch.zeros_like(K)
    q = torch.empty(B, H, d, dtype=dtype, device=device)
    which = torch.empty(B, H_kv, n, dtype=torch.int64, device=device)
    for b in range(B):
        gd = gen_device or ("cpu" if H_kv * n * d <= _CPU_LIMIT else str(device))
        fdt = torch.float64 if gd == "cpu" else torch.float32
        k, v, qq, wh = _sequence(H_kv, H, n, d, centers, 1000 * seed + b, gd, fdt)
        K[b, :, :n] = k.to(device=device, dtype=dtype)
        V[b, :, :n] = v.to(device=device, dtype=dtype)
        q[b] = qq.to(device=device, dtype=dtype)
        which[b] = wh.to(device)
    return K, V, q, which
