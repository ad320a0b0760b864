"""Deterministic synthetic attention inputs.

``structured_qkv`` restates the clustered generator of the reference's test
suite (``tests/synthetic.py:8-52``) with torch's RNG: the same structure
(cluster centres x1.2, one key cluster per block, query runs of
``block_size // 8`` positions, noise), different random draws.

``baseline_qkv`` is the benchmark generator: i.i.d. N(0, 1) Q/K/V plus a
planted unit direction ``u`` per KV head, added to the keys of block 0 and of
a random fraction of the other key blocks (scaled by ``planted``) and to every
query (scaled by ``query_shift``).  Draw order per KV head: u, K, V, heavy
blocks, then the head group's Q.
"""

from __future__ import annotations

import math

import torch


def structured_qkv(
    *,
    length: int = 2_048,
    query_heads: int = 8,
    kv_heads: int = 2,
    head_dim: int = 64,
    block_size: int = 128,
    clusters: int = 16,
    noise: float = 0.3,
    dtype: torch.dtype = torch.float32,
    seed: int = 0,
    device: str | torch.device = "cpu",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Clustered ``q, k, v`` shaped ``[heads, length, dim]``."""
    if length <= 0 or head_dim <= 0 or block_size <= 0 or clusters <= 0:
        raise ValueError("length, head_dim, block_size, and clusters must be positive")
    if query_heads <= 0 or kv_heads <= 0 or query_heads % kv_heads:
        raise ValueError("query_heads must be divisible by positive kv_heads")
    gen = torch.Generator(device="cpu").manual_seed(seed)
    centers = 1.2 * torch.randn((kv_heads, clusters, head_dim), generator=gen)
    num_blocks = (length + block_size - 1) // block_size
    kv_block_clusters = torch.randint(0, clusters, (kv_heads, num_blocks), generator=gen)
    block_ids = torch.arange(length) // block_size
    kv_cluster_ids = kv_block_clusters[:, block_ids]
    head_ids = torch.arange(kv_heads)[:, None]
    keys = centers[head_ids, kv_cluster_ids]
    keys = keys + noise * torch.randn(keys.shape, generator=gen)
    group = query_heads // kv_heads
    q_kv_ids = torch.arange(query_heads) // group
    run = max(1, block_size // 8)
    run_ids = torch.arange(length) // run
    q_run_clusters = torch.randint(0, clusters, (query_heads, (length + run - 1) // run),
                                   generator=gen)
    q_cluster_ids = q_run_clusters[:, run_ids]
    queries = centers[q_kv_ids[:, None], q_cluster_ids]
    queries = queries + noise * torch.randn(queries.shape, generator=gen)
    values = torch.randn((kv_heads, length, head_dim), generator=gen)
    return tuple(x.to(dtype).to(device) for x in (queries, keys, values))


def baseline_qkv(
    seq: int,
    *,
    query_heads: int = 32,
    kv_heads: int = 8,
    head_dim: int = 128,
    block_k: int = 128,
    heavy_fraction: float = 0.06,
    planted: float = 3.0,
    query_shift: float = 0.5,
    seed: int = 0,
    dtype: torch.dtype = torch.bfloat16,
    device: str | torch.device = "cpu",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Benchmark inputs ``q [Hq, L, D]``, ``k, v [Hkv, L, D]`` in ``dtype``.

    Built in float32 with a torch generator on ``device`` and rounded once to
    ``dtype`` (round-to-nearest-even).  Generation on the CPU is
    device-independent; on a GPU it is fast and reproducible per device type.
    """
    device = torch.device(device)
    gen = torch.Generator(device=device).manual_seed(seed)
    group = query_heads // kv_heads
    num_blocks = seq // block_k
    heavy_count = int(round(heavy_fraction * (num_blocks - 1)))
    q = torch.empty((query_heads, seq, head_dim), dtype=dtype, device=device)
    k = torch.empty((kv_heads, seq, head_dim), dtype=dtype, device=device)
    v = torch.empty((kv_heads, seq, head_dim), dtype=dtype, device=device)
    for h in range(kv_heads):
        u = torch.randn(head_dim, generator=gen, device=device)
        u = u / u.norm()
        kh = torch.randn((seq, head_dim), generator=gen, device=device)
        vh = torch.randn((seq, head_dim), generator=gen, device=device)
        others = torch.randperm(num_blocks - 1, generator=gen, device=device)[:heavy_count] + 1
        heavy = torch.cat([torch.zeros(1, dtype=others.dtype, device=device), others])
        kb = kh[: num_blocks * block_k].view(num_blocks, block_k, head_dim)
        kb[heavy] += planted * u
        k[h] = kh.to(dtype)
        v[h] = vh.to(dtype)
        for g in range(group):
            qh = torch.randn((seq, head_dim), generator=gen, device=device) + query_shift * u
            q[h * group + g] = qh.to(dtype)
    return q, k, v


def contrast_planted(head_dim: int = 128) -> float:
    """Planted key scale of the supplementary high-contrast variant (3 * sqrt(D))."""
    return 3.0 * math.sqrt(head_dim)
