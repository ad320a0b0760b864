"""Block-sparse attention with mean correction on MI355X (gfx950).

Interface of the reference's ``fpv2/kernel.py``: ``compact_block_indices``
turns a selection mask into fixed-width padded ascending block lists (selected
and safely pruned) with per-row counts, and ``sparse_attention`` runs the
FlashAttention-2 online softmax over the selected blocks, then appends the
pooled representatives of the pruned blocks to the same softmax with a
``+log2(block_k)`` logit shift.

The device work is the ``fpv2_sparse_attention`` HIP kernel: one workgroup per
(KV head, query tile, 128 packed rows) so the G query heads of a KV head share
every K/V load (what the reference calls PackGQA is always on here; the flag
is validated and accepted for interface parity), Q held in VGPRs, K/V
sub-tiles double-buffered in LDS, QK^T and PV on bf16/f16 MFMA with float32
accumulation and base-2 exponentials.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from fpv2 import _lib
from fpv2.selection import FPV2Config

SUPPORTED_HEAD_DIMS = (64, 96, 128, 256)


@dataclass(frozen=True)
class TileConfig:
    """A tile request: ``bq`` query rows, ``bk`` keys, ``wm`` warps
    (the names of ``kernel.py:30-40``).

    The gfx950 kernel's tiling is fixed per head dimension (128 packed query
    rows per workgroup, 32-key sub-tiles, 4 waves; 8 for head_dim 256), so a
    tile changes neither the launch nor the output.  ``sparse_attention``
    accepts one for interface parity, checks that it is well formed, and
    uses its ``bq`` in the PackGQA alignment rule (``kernel.py:505-510``).
    """

    bq: int
    bk: int
    wm: int

    @property
    def threads(self) -> int:
        return 32 * self.wm

    def check(self, head_dim: int, *, block_k: int = 128, tile_q: int = 128) -> None:
        """Well-formedness only: positive integer dimensions and a head
        dimension the kernel is built for.  (The reference's threadgroup
        memory and simdgroup fragment rules describe Apple GPUs and do not
        apply to this kernel.)"""
        dims = (self.bq, self.bk, self.wm)
        if any(isinstance(x, bool) or not isinstance(x, int) or x <= 0 for x in dims):
            raise ValueError("tile dimensions must be positive")
        if head_dim not in SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head dimension must be one of {SUPPORTED_HEAD_DIMS}")


_DEFAULT_TILES = {
    64: TileConfig(32, 32, 4),
    96: TileConfig(32, 32, 4),
    128: TileConfig(64, 32, 8),
    256: TileConfig(32, 16, 4),
}


def default_tile(head_dim: int) -> TileConfig:
    """Default tile per supported head dimension (reference table)."""
    try:
        return _DEFAULT_TILES[head_dim]
    except KeyError as error:
        raise ValueError(f"head dimension must be one of {SUPPORTED_HEAD_DIMS}") from error


def _tile_for_config(head_dim: int, config: FPV2Config) -> TileConfig:
    """The tile named for a configuration (``kernel.py:76-88``): the
    head-dimension default when it divides ``tile_q`` and ``block_k``,
    otherwise ``(min(tile_q, 32), min(block_k, 16), bq / 8)`` (at least one
    warp).  Any positive ``tile_q`` and ``block_k`` resolve: the kernel
    takes them all."""
    tile = default_tile(head_dim)
    if (
        config.tile_q >= tile.bq
        and config.tile_q % tile.bq == 0
        and config.block_k % tile.bk == 0
    ):
        return tile
    bq = min(config.tile_q, 32)
    bk = min(config.block_k, 16)
    return TileConfig(bq, bk, max(1, bq // 8))


def compact_block_indices(
    selected: torch.Tensor,
    *,
    config: FPV2Config = FPV2Config(),
    offset: int = 0,
    query_length: int | None = None,
    key_length: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Padded selected/pruned block lists and per-row counts.

    Same contract as the reference (``kernel.py:141-184``): ``selected_ids``
    holds the selected blocks ascending followed by the unselected blocks
    ascending (a stable ``argsort(-mask)``); ``pruned`` = not selected and
    ending (clipped to ``key_length``) at or before the tile's first query.
    Returns int32 ``ids [Hkv, Nt, Nb]``, ``counts [Hkv, Nt]``,
    ``pruned_ids``, ``pruned_counts``.
    """
    if selected.ndim != 3:
        raise ValueError("selected must have shape [KV heads, tiles, blocks]")
    if selected.dtype != torch.bool:
        raise ValueError("selected must have boolean dtype")
    kv_heads, num_tiles, num_blocks = selected.shape
    padded_query_length = num_tiles * config.tile_q
    valid_query_length = padded_query_length if query_length is None else query_length
    represented_key_length = num_blocks * config.block_k
    valid_key_length = represented_key_length if key_length is None else key_length
    if offset < 0:
        raise ValueError("offset must be non-negative")
    if not 0 < valid_query_length <= padded_query_length:
        raise ValueError("query_length is inconsistent with selected tiles")
    if not 0 < valid_key_length <= represented_key_length:
        raise ValueError("key_length is inconsistent with selected blocks")
    if offset + valid_query_length > valid_key_length:
        raise ValueError("queries extend beyond key_length")
    device = _lib.require_device(selected)
    lib = _lib.load()
    mask = selected.contiguous()
    ids = torch.empty((kv_heads, num_tiles, num_blocks), dtype=torch.int32, device=device)
    pruned_ids = torch.empty_like(ids)
    counts = torch.empty((kv_heads, num_tiles), dtype=torch.int32, device=device)
    pruned_counts = torch.empty_like(counts)
    with torch.cuda.device(device):
        status = lib.fpv2_compact_block_indices(
            mask.data_ptr(), kv_heads, num_tiles, num_blocks, config.tile_q,
            config.block_k, offset, valid_key_length, ids.data_ptr(), counts.data_ptr(),
            pruned_ids.data_ptr(), pruned_counts.data_ptr(), _lib.stream_ptr(device))
    _lib.check(status, "compact_block_indices")
    return ids, counts, pruned_ids, pruned_counts


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Last dim contiguous, 8-element strides, 16-byte base; else copy.

    A view that is contiguous but starts off a 16-byte boundary (a view a
    few elements into its storage) is cloned: its ``contiguous()`` would
    return the same misaligned view."""
    if (t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1])
            or t.data_ptr() % 16):
        t = t.clone(memory_format=torch.contiguous_format)
    return t


def sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    pooled_k: torch.Tensor,
    pooled_v: torch.Tensor,
    selected_ids: torch.Tensor,
    selected_counts: torch.Tensor,
    pruned_ids: torch.Tensor,
    pruned_counts: torch.Tensor,
    *,
    scale: float,
    config: FPV2Config = FPV2Config(),
    offset: int = 0,
    query_length: int | None = None,
    key_length: int | None = None,
    tile: TileConfig | None = None,
    pack_gqa: bool = False,
) -> torch.Tensor:
    """Run block-sparse attention with optional mean correction.

    Arguments, validation messages and output (``[Hq, Lq_pad, D]`` in the
    query dtype) follow the reference (``kernel.py:441-590``).  Padded query
    rows (at or beyond ``query_length``) come back as zeros.
    """
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k, and v must have shape [heads, sequence, dim]")
    if k.shape != v.shape:
        raise ValueError("k and v must have identical shapes")
    if (q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype
            or v.dtype != q.dtype):
        raise ValueError("q, k, and v must share float16 or bfloat16 dtype")
    query_heads, padded_query_length, head_dim = q.shape
    kv_heads, padded_key_length, key_dim = k.shape
    if head_dim != key_dim or head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head dimension must be one of {SUPPORTED_HEAD_DIMS}")
    if not kv_heads or query_heads % kv_heads:
        raise ValueError("query heads must be divisible by KV heads")
    if padded_query_length % config.tile_q or padded_key_length % config.block_k:
        raise ValueError("q and k/v sequence lengths must be tile/block aligned")
    valid_query_length = padded_query_length if query_length is None else query_length
    valid_key_length = padded_key_length if key_length is None else key_length
    if not 0 < valid_query_length <= padded_query_length:
        raise ValueError("query_length must fit within padded q")
    if not 0 < valid_key_length <= padded_key_length:
        raise ValueError("key_length must fit within padded k/v")
    num_tiles = padded_query_length // config.tile_q
    num_blocks = padded_key_length // config.block_k
    expected_lists = (kv_heads, num_tiles, num_blocks)
    expected_counts = (kv_heads, num_tiles)
    if tuple(selected_ids.shape) != expected_lists or tuple(pruned_ids.shape) != expected_lists:
        raise ValueError(f"block lists must have shape {expected_lists}")
    if (tuple(selected_counts.shape) != expected_counts
            or tuple(pruned_counts.shape) != expected_counts):
        raise ValueError(f"block counts must have shape {expected_counts}")
    if any(t.dtype != torch.int32 for t in (selected_ids, pruned_ids, selected_counts,
                                             pruned_counts)):
        raise ValueError("block lists and counts must have int32 dtype")
    if (tuple(pooled_k.shape) != (kv_heads, num_blocks, head_dim)
            or pooled_v.shape != pooled_k.shape):
        raise ValueError("pooled k/v shapes do not match padded k/v")
    if offset < 0 or offset + valid_query_length > valid_key_length:
        raise ValueError("offset does not align queries within the key sequence")
    tile = _tile_for_config(head_dim, config) if tile is None else tile
    tile.check(head_dim, block_k=config.block_k, tile_q=config.tile_q)
    group_size = query_heads // kv_heads
    if pack_gqa and (tile.bq % group_size or (config.tile_q * group_size) % tile.bq):
        raise ValueError("PackGQA tile must align with complete GQA groups")

    device = _lib.require_device(q, k, v, pooled_k, pooled_v, selected_ids,
                                 selected_counts, pruned_ids, pruned_counts)
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    _launch_attention(
        q, k, v, pooled_k.to(q.dtype), pooled_v.to(q.dtype), selected_ids,
        selected_counts, pruned_ids, pruned_counts, out, device=device, scale=scale,
        config=config, offset=offset, query_length=valid_query_length,
        key_length=valid_key_length, num_blocks=num_blocks,
        padded_query_length=padded_query_length, out_rows=padded_query_length)
    return out


def _pooled_ready(pooled_k: torch.Tensor, pooled_v: torch.Tensor):
    """Pooled K/V as the kernel reads them: blocks and D contiguous, one head
    stride shared by both (a pooled cache with spare capacity is used in
    place)."""
    def ok(p):
        return (p.stride(-1) == 1 and p.stride(-2) == p.shape[-1] and p.stride(0) % 8 == 0
                and p.data_ptr() % 16 == 0)
    if not (ok(pooled_k) and ok(pooled_v) and pooled_k.stride(0) == pooled_v.stride(0)):
        pooled_k = pooled_k.clone(memory_format=torch.contiguous_format)
        pooled_v = pooled_v.clone(memory_format=torch.contiguous_format)
    return pooled_k, pooled_v


# Sub-tiles (32 keys each) per segment of a split tile: 4096 keys, about
# the walk of a typical tile of a sparse long-context layer.
SPLIT_SEG_STEPS = 128


def _launch_attention(q, k, v, pooled_k, pooled_v, selected_ids, selected_counts,
                      pruned_ids, pruned_counts, out, *, device, scale, config, offset,
                      query_length, key_length, num_blocks, padded_query_length,
                      out_rows, split_tiles=0, seg_steps=SPLIT_SEG_STEPS) -> None:
    """Enqueue ``fpv2_sparse_attention`` on the current stream.

    ``q``/``k``/``v``/``out`` are ``[H, L, D]`` views (any head and row
    strides with a contiguous last dimension); rows past the valid lengths
    are never read.  ``split_tiles``: run the last ``split_tiles`` query
    tiles as key-range segments of ``seg_steps`` sub-tiles, merged after the
    kernel (``fpv2_sparse_attention_split``), with a workspace from the
    caching allocator.
    """
    lib = _lib.load()
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    pooled_k, pooled_v = _pooled_ready(pooled_k, pooled_v)
    ids, counts = selected_ids.contiguous(), selected_counts.contiguous()
    pids, pcounts = pruned_ids.contiguous(), pruned_counts.contiguous()
    params = _lib.AttnParams(
        query_heads=q.shape[0], kv_heads=k.shape[0], head_dim=q.shape[-1],
        padded_query_length=padded_query_length, query_length=query_length,
        out_rows=out_rows, key_length=key_length, num_blocks=num_blocks, offset=offset,
        block_k=config.block_k, tile_q=config.tile_q,
        mean_correction=1 if config.mean_correction else 0, scale=float(scale),
        q_head_stride=q.stride(0), q_row_stride=q.stride(1),
        k_head_stride=k.stride(0), k_row_stride=k.stride(1),
        v_head_stride=v.stride(0), v_row_stride=v.stride(1),
        o_head_stride=out.stride(0), o_row_stride=out.stride(1),
        pooled_head_stride=pooled_k.stride(0))
    with torch.cuda.device(device):
        if split_tiles:
            need = lib.fpv2_sparse_attention_split_workspace_bytes(params, split_tiles,
                                                                   seg_steps)
            if need < 0:
                _lib.check(int(need), "sparse_attention_split")
            workspace = torch.empty(max(int(need), 1), dtype=torch.uint8, device=device)
            status = lib.fpv2_sparse_attention_split(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), pooled_k.data_ptr(),
                pooled_v.data_ptr(), ids.data_ptr(), counts.data_ptr(), pids.data_ptr(),
                pcounts.data_ptr(), out.data_ptr(), _lib.dtype_code(q.dtype), params,
                split_tiles, seg_steps, workspace.data_ptr(), int(need),
                _lib.stream_ptr(device))
        else:
            status = lib.fpv2_sparse_attention(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), pooled_k.data_ptr(),
                pooled_v.data_ptr(), ids.data_ptr(), counts.data_ptr(), pids.data_ptr(),
                pcounts.data_ptr(), out.data_ptr(), _lib.dtype_code(q.dtype), params,
                _lib.stream_ptr(device))
    _lib.check(status, "sparse_attention")

