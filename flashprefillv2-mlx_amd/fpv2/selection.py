"""Block scoring and selection for FlashPrefill V2 on MI355X.

Same interface as the reference's ``fpv2/selection.py``: keys are mean-pooled
into blocks, ``k_bar[b] = mean(k[b])``; for every query row and pooled key the
index stage computes ``s[q, b] = scale * q @ k_bar[b]``.  Rows are grouped by
KV head and query tile; a block's tile energy is the sum of ``exp(s - max(s))``
across the tile and all query heads sharing that KV head, and the block is
selected when its energy is at least ``alpha`` times the largest fully visible
block energy.  Sink, local-window and dense-tail blocks are then forced, and
everything is limited to causally visible blocks.

Tensors are torch tensors on a ROCm device; the work runs in hand-written
gfx950 kernels (``libfpv2_hip.so``): block pooling is one HBM-bound kernel,
scoring + selection one MFMA kernel per (KV head, query tile) that never
materialises the ``[Hkv, G, N, Nb]`` score tensor unless it is asked for.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from fpv2 import _lib


@dataclass(frozen=True)
class FPV2Config:
    """Parameters controlling block selection and mean correction.

    Fields, defaults and validation follow ``FPV2Config`` in the reference
    (``fpv2/selection.py:30-65``).
    """

    block_k: int = 128
    tile_q: int = 128
    alpha: float = 0.1
    sink_tokens: int = 256
    window_tokens: int = 384
    # Request-level only when the input contains the complete request.
    last_n_blocks: int = 2
    mean_correction: bool = True
    score_chunk_tiles: int | None = None
    pack_gqa: bool = False

    def __post_init__(self) -> None:
        if self.block_k <= 0 or self.tile_q <= 0:
            raise ValueError("block_k and tile_q must be positive")
        if self.alpha < 0:
            raise ValueError("alpha must be non-negative")
        if self.sink_tokens < 0 or self.window_tokens < 0:
            raise ValueError("sink_tokens and window_tokens must be non-negative")
        if (
            not isinstance(self.last_n_blocks, int)
            or isinstance(self.last_n_blocks, bool)
            or self.last_n_blocks < 0
        ):
            raise ValueError("last_n_blocks must be a non-negative integer")
        if self.score_chunk_tiles is not None and (
            not isinstance(self.score_chunk_tiles, int)
            or isinstance(self.score_chunk_tiles, bool)
            or self.score_chunk_tiles <= 0
        ):
            raise ValueError("score_chunk_tiles must be a positive integer or None")
        if not isinstance(self.pack_gqa, bool):
            raise ValueError("pack_gqa must be a boolean")


_POOL_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def pool_blocks(x: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """Mean-pool the penultimate (sequence) axis into fixed-size blocks.

    Mirrors ``pool_blocks`` (reference ``fpv2/selection.py:68-80``): output
    ``[..., L / block_size, D]`` in the input dtype.  The block mean is
    accumulated in float64 on the device and rounded once.
    """
    if x.ndim < 2:
        raise ValueError("x must have at least sequence and feature dimensions")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    length, head_dim = x.shape[-2:]
    if length % block_size:
        raise ValueError(
            f"sequence length {length} must be divisible by block_size {block_size}"
        )
    if x.dtype not in _POOL_DTYPES:
        raise ValueError("pool_blocks supports float32, float16 and bfloat16")
    device = _lib.require_device(x)
    lib = _lib.load()
    num_blocks = length // block_size
    out = torch.empty((*x.shape[:-2], num_blocks, head_dim), dtype=x.dtype, device=device)
    if out.numel() == 0:
        return out
    if x.stride(-1) != 1:
        x = x.contiguous()
    flat = x.reshape(-1, length, head_dim)
    with torch.cuda.device(device):
        status = lib.fpv2_pool_blocks(
            flat.data_ptr(), out.data_ptr(), _lib.dtype_code(x.dtype), flat.shape[0],
            length, num_blocks, head_dim, block_size, flat.stride(0), flat.stride(1),
            num_blocks * head_dim, _lib.stream_ptr(device))
    _lib.check(status, "pool_blocks")
    return out


def _validate_inputs(
    q: torch.Tensor,
    pooled_k: torch.Tensor,
    config: FPV2Config,
    offset: int,
    query_length: int,
) -> tuple[int, int, int, int]:
    """Shape checks of the reference (``fpv2/selection.py:83-106``)."""
    if q.ndim != 3 or pooled_k.ndim != 3:
        raise ValueError("q and pooled_k must have shape [heads, sequence, dim]")
    query_heads, padded_length, head_dim = q.shape
    kv_heads, num_blocks, key_dim = pooled_k.shape
    if not kv_heads or query_heads % kv_heads:
        raise ValueError("query heads must be divisible by KV heads")
    if head_dim != key_dim:
        raise ValueError("q and pooled_k head dimensions must match")
    if padded_length % config.tile_q:
        raise ValueError("query length must be padded to a multiple of tile_q")
    if not 0 < query_length <= padded_length:
        raise ValueError("query_length must be in (0, q.shape[-2]]")
    if offset < 0:
        raise ValueError("offset must be non-negative")
    if offset + query_length > num_blocks * config.block_k:
        raise ValueError("queries extend beyond the represented key sequence")
    return query_heads, kv_heads, padded_length, num_blocks


def _select_params(q: torch.Tensor, num_blocks: int, *, kv_heads: int, scale: float,
                   config: FPV2Config, offset: int, query_length: int,
                   padded_length: int, key_length: int,
                   pooled_head_stride: int | None = None) -> _lib.SelectParams:
    return _lib.SelectParams(
        query_heads=q.shape[0], kv_heads=kv_heads, head_dim=q.shape[-1],
        padded_query_length=padded_length, query_length=query_length,
        num_blocks=num_blocks, key_length=key_length, offset=offset,
        block_k=config.block_k, tile_q=config.tile_q,
        sink_tokens=config.sink_tokens, window_tokens=config.window_tokens,
        last_n_blocks=config.last_n_blocks, scale=float(scale), alpha=float(config.alpha),
        q_head_stride=q.stride(0), q_row_stride=q.stride(1),
        pooled_head_stride=(num_blocks * q.shape[-1] if pooled_head_stride is None
                            else pooled_head_stride))


def _operands(q: torch.Tensor, pooled_k: torch.Tensor):
    """Same 16-bit dtype -> MFMA path; anything else is scored in float32."""
    if q.dtype == pooled_k.dtype and q.dtype in (torch.float16, torch.bfloat16):
        dtype = q.dtype
    else:
        dtype = torch.float32
        q = q.to(dtype)
        pooled_k = pooled_k.to(dtype)
    if q.stride(-1) != 1 or q.stride(1) % 8 or q.stride(0) % 8:
        q = q.contiguous()
    return q, pooled_k.contiguous(), dtype


def block_scores_and_select(
    q: torch.Tensor,
    pooled_k: torch.Tensor,
    *,
    scale: float,
    config: FPV2Config = FPV2Config(),
    offset: int = 0,
    query_length: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Return selection ``[Hkv, Nt, Nb]`` (bool) and optional raw scores.

    Interface of the reference (``fpv2/selection.py:109-201``).  ``offset`` is
    the absolute key position of query row zero; ``q`` is tile-padded and
    ``query_length`` excludes padded rows (padded rows are treated as zeros
    and never read).  Raw scores ``[Hkv, G, N, Nb]`` (float32) are returned
    only when ``config.score_chunk_tiles`` is None; the kernel works one
    query tile at a time, so grouping tiles never changes the selection.
    """
    valid_length = q.shape[-2] if query_length is None else query_length
    query_heads, kv_heads, padded_length, num_blocks = _validate_inputs(
        q, pooled_k, config, offset, valid_length
    )
    device = _lib.require_device(q, pooled_k)
    lib = _lib.load()
    group = query_heads // kv_heads
    num_tiles = padded_length // config.tile_q
    qk, pk, dtype = _operands(q, pooled_k)
    selected = torch.empty((kv_heads, num_tiles, num_blocks), dtype=torch.bool, device=device)
    scores = None
    if config.score_chunk_tiles is None:
        scores = torch.empty((kv_heads, group, padded_length, num_blocks),
                             dtype=torch.float32, device=device)
    params = _select_params(qk, num_blocks, kv_heads=kv_heads, scale=scale, config=config,
                            offset=offset, query_length=valid_length,
                            padded_length=padded_length,
                            key_length=num_blocks * config.block_k)
    with torch.cuda.device(device):
        status = lib.fpv2_score_select(
            qk.data_ptr(), pk.data_ptr(), _lib.dtype_code(dtype), params,
            selected.data_ptr(), _lib.ptr(scores), None, None, None, None,
            _lib.stream_ptr(device))
    _lib.check(status, "block_scores_and_select")
    return selected, scores


def density(
    selected: torch.Tensor,
    *,
    config: FPV2Config = FPV2Config(),
    offset: int = 0,
    query_length: int | None = None,
) -> torch.Tensor:
    """Retained causal block work as a scalar fraction (0-d float32 tensor).

    ``sum(selected) / (visible (tile, block) pairs * Hkv)`` as in the
    reference (``fpv2/selection.py:204-229``); the visible count is a closed
    form of the tile geometry.
    """
    if selected.ndim != 3:
        raise ValueError("selected must have shape [KV heads, tiles, blocks]")
    kv_heads, num_tiles, num_blocks = selected.shape
    if offset < 0:
        raise ValueError("offset must be non-negative")
    valid_length = num_tiles * config.tile_q if query_length is None else query_length
    if not 0 < valid_length <= num_tiles * config.tile_q:
        raise ValueError("query_length is inconsistent with selected tiles")
    visible = 0
    for tile in range(num_tiles):
        last = min(offset + (tile + 1) * config.tile_q, offset + valid_length) - 1
        visible += min(last // config.block_k + 1, num_blocks)
    denominator = float(visible * kv_heads)
    return selected.sum(dtype=torch.float32) / denominator
