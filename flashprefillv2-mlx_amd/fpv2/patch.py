"""Model-independent, conservative hook for torch scaled-dot-product attention.

Counterpart of the reference's ``fpv2/patch.py`` (which wraps MLX's
``mx.fast.scaled_dot_product_attention``): ``enable`` replaces
``torch.nn.functional.scaled_dot_product_attention`` with a wrapper that sends
a call to FPV2 only when it is a batch-one, bottom-right causal prefill on a
ROCm device with matching float16/bfloat16 Q/K/V, a supported head dimension,
grouped-query-compatible head counts, at least one full query tile, and a key
length meeting ``min_tokens``.  Everything else goes to the original function
unchanged.

Bottom-right causal in torch terms: ``is_causal=True`` with ``Lq == Lk`` (the
top-left and bottom-right diagonals coincide), or ``attn_mask`` a
``torch.nn.attention.bias.CausalBias`` of variant ``LOWER_RIGHT`` (or
``UPPER_LEFT`` when square).  ``is_causal=True`` with ``Lq < Lk`` is top-left
in torch and therefore passed through.

For eligible calls ``offset = key_length - query_length`` places the query
chunk in the causal key prefix.  An eligible call whose key range needs more
blocks than the selection kernel holds (``FPV2_MAX_BLOCKS``, 1 048 576 keys
at ``block_k`` 128) goes to the original function too, and counts as dense
in ``block_sparsity`` as a call below ``min_tokens`` does.  Nothing is padded
or copied: the kernels take head/row strides and valid lengths, treat rows
past them as zeros, and write the ``[1, Hq, Lq, D]`` output directly.
``disable`` restores the original.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Any

import torch
import torch.nn.functional as F

from fpv2 import _lib
from fpv2.kernel import SPLIT_SEG_STEPS, SUPPORTED_HEAD_DIMS, _kernel_ready, _launch_attention
from fpv2.selection import FPV2Config, _select_params

try:  # torch >= 2.3
    from torch.nn.attention.bias import CausalBias, CausalVariant
except ImportError:  # pragma: no cover - older torch
    CausalBias = CausalVariant = None

_ORIGINAL_SDPA = F.scaled_dot_product_attention
_enabled = False
_collect_stats = False
_forwarding = False  # inside a pass-through's CausalBias dispatch


class SelectedBlockCounter:
    """Sum of the selected-block counts of FPV2 calls on one device.

    A call's ``counts`` tensor (a fresh ``[Hkv, Nt]`` int32 allocation) is
    kept rather than reduced: every ``fold_every`` calls the kept tensors are
    summed by one concatenation and one reduction into a 0-d int64 device
    total, so a call launches no kernel and nothing synchronises until
    ``value()`` is read.  Each kept tensor remembers the stream that wrote
    it; the stream that folds waits for those streams first.
    """

    def __init__(self, fold_every: int = 64) -> None:
        self.fold_every = fold_every
        self._pending: list[torch.Tensor] = []
        self._streams: list[torch.cuda.Stream] = []
        self._total: torch.Tensor | None = None

    def add(self, counts: torch.Tensor) -> None:
        self._pending.append(counts)
        if counts.is_cuda:
            stream = torch.cuda.current_stream(counts.device)
            if all(stream != s for s in self._streams):
                self._streams.append(stream)
        if len(self._pending) >= self.fold_every:
            self._fold()

    def _fold(self) -> None:
        if not self._pending:
            return
        if self._streams:
            current = torch.cuda.current_stream(self._pending[0].device)
            for stream in self._streams:
                if stream != current:
                    current.wait_stream(stream)
            # the allocator must not reuse a kept tensor's memory, nor the
            # previous total's (allocated on an earlier fold's stream), on its
            # own stream before this stream has read it
            for c in self._pending:
                c.record_stream(current)
            if self._total is not None and self._total.is_cuda:
                self._total.record_stream(current)
        part = torch.cat([c.reshape(-1) for c in self._pending]).sum(dtype=torch.int64)
        self._total = part if self._total is None else self._total + part
        self._pending.clear()
        self._streams = [torch.cuda.current_stream(part.device)] if part.is_cuda else []

    def device_total(self) -> torch.Tensor | None:
        """The sum so far as a 0-d int64 device tensor (None if nothing was
        added), without synchronising."""
        self._fold()
        return self._total

    def value(self) -> int:
        """The sum so far (synchronises once)."""
        total = self.device_total()
        return 0 if total is None else int(total.item())

    def reset(self) -> None:
        self._pending.clear()
        self._streams.clear()
        self._total = None


# Selected blocks of FPV2 calls, per device; block_sparsity() reads them once.
_selected_totals: dict[torch.device, SelectedBlockCounter] = {}
_selected_dense_blocks = 0
_visible_blocks = 0
_PACKED_TILE_ROWS = 128


def _effective_config(
    config: FPV2Config, query_heads: int, kv_heads: int
) -> FPV2Config | None:
    """Resolve the default 128 packed rows into query positions (tile_q = 128 / G)."""
    if config.tile_q != _PACKED_TILE_ROWS:
        return config
    if not kv_heads or query_heads % kv_heads:
        return None
    group_size = query_heads // kv_heads
    if _PACKED_TILE_ROWS % group_size:
        return None
    return replace(config, tile_q=_PACKED_TILE_ROWS // group_size)


def _request_config(
    config: FPV2Config, key_length: int, total_tokens: int | None
) -> FPV2Config:
    """Apply the dense tail only when this call reaches the request boundary."""
    if config.last_n_blocks and (total_tokens is None or key_length < total_tokens):
        return replace(config, last_n_blocks=0)
    return config


def _causal_block_count(kv_heads: int, query_length: int, offset: int,
                        config: FPV2Config) -> int:
    count = 0
    for start in range(0, query_length, config.tile_q):
        end = offset + min(start + config.tile_q, query_length)
        count += (end + config.block_k - 1) // config.block_k
    return count * kv_heads


def block_sparsity() -> float:
    """Fraction of visible causal blocks skipped since ``enable``.

    Selected counts stay on the device until this call, which synchronises
    once to read their sum.
    """
    if not _visible_blocks:
        return 0.0
    selected = _selected_dense_blocks
    for total in _selected_totals.values():
        selected += total.value()
    return 1.0 - selected / _visible_blocks


def _num_blocks(query_length: int, key_length: int, config: FPV2Config) -> int:
    """Key blocks of a call: ``ceil(max(Lk, offset + Lq_pad) / block_k)``
    (``patch.py:123-131``)."""
    padded_query_length = -(-query_length // config.tile_q) * config.tile_q
    required = max(key_length, key_length - query_length + padded_query_length)
    return -(-required // config.block_k)


def _within_block_limit(query_length: int, key_length: int, config: FPV2Config) -> bool:
    """Whether the selection kernel holds the call's key blocks."""
    return _num_blocks(query_length, key_length, config) <= _lib.MAX_BLOCKS


def fpv2_sdpa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: float,
    config: FPV2Config = FPV2Config(),
) -> torch.Tensor:
    """Apply FPV2 to a batch-one, bottom-right causal attention ``[1, H, L, D]``.

    Data flow of the reference (``fpv2/patch.py:102-174``) without the
    padding copies: pool K/V (one launch), score/select/compact (one launch),
    sparse attention (one launch), all on the current stream, no host sync.
    """
    return _fpv2_sdpa(q, k, v, scale=scale, config=config)


@dataclass(frozen=True)
class _Geometry:
    """Sizes of one hook call (``patch.py:116-136`` without the padding copies)."""

    config: FPV2Config
    query_heads: int
    kv_heads: int
    head_dim: int
    query_length: int
    key_length: int
    offset: int
    padded_query_length: int
    num_tiles: int
    num_blocks: int


def _geometry(q, k, v, config: FPV2Config, *, capped: bool = True) -> _Geometry:
    """The reference hook's validation (``patch.py:102-124``) and the block
    grid: Q padded to a ``tile_q`` multiple, keys to ``ceil(max(Lk, off +
    Lq_pad) / block_k)`` blocks, as index arithmetic only.  ``capped``:
    refuse more blocks than the selection kernel holds."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have shape [batch, heads, sequence, dim]")
    if q.shape[0] != 1 or k.shape[0] != 1 or v.shape[0] != 1:
        raise ValueError("FPV2 currently supports batch size 1")
    effective_config = _effective_config(config, q.shape[1], k.shape[1])
    if effective_config is None:
        raise ValueError("GQA group size must divide 128 packed query rows")
    config = effective_config
    query_length = q.shape[-2]
    key_length = k.shape[-2]
    if query_length > key_length:
        raise ValueError("query length cannot exceed key length for causal attention")
    if k.shape != v.shape or q.shape[-1] != k.shape[-1]:
        raise ValueError("q, k, and v head dimensions must match")
    if q.shape[-1] not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head dimension must be one of {SUPPORTED_HEAD_DIMS}")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, and v must share float16 or bfloat16 dtype")
    offset = key_length - query_length
    padded_query_length = -(-query_length // config.tile_q) * config.tile_q
    num_blocks = _num_blocks(query_length, key_length, config)
    if capped and num_blocks > _lib.MAX_BLOCKS:
        raise ValueError(f"key length needs {num_blocks} blocks; at most {_lib.MAX_BLOCKS}")
    return _Geometry(config=config, query_heads=q.shape[1], kv_heads=k.shape[1],
                     head_dim=q.shape[-1], query_length=query_length, key_length=key_length,
                     offset=offset, padded_query_length=padded_query_length,
                     num_tiles=padded_query_length // config.tile_q, num_blocks=num_blocks)


def _pool_into(lib, k3, v3, pooled_k, pooled_v, *, dtype, valid_rows, num_blocks,
               block_k, stream) -> None:
    """Pool ``num_blocks`` blocks of ``k3``/``v3`` (``[Hkv, rows, D]`` views;
    rows >= ``valid_rows`` count as zeros) into ``pooled_k``/``pooled_v``
    (``[Hkv, >=num_blocks, D]`` views, any head stride)."""
    kv_heads, _, head_dim = k3.shape
    if k3.stride() == v3.stride() and pooled_k.stride() == pooled_v.stride():
        status = lib.fpv2_pool_kv(
            k3.data_ptr(), v3.data_ptr(), pooled_k.data_ptr(), pooled_v.data_ptr(),
            dtype, kv_heads, valid_rows, num_blocks, head_dim, block_k,
            k3.stride(0), k3.stride(1), pooled_k.stride(0), stream)
        _lib.check(status, "pool_kv")
        return
    for src, dst in ((k3, pooled_k), (v3, pooled_v)):
        status = lib.fpv2_pool_blocks(
            src.data_ptr(), dst.data_ptr(), dtype, kv_heads, valid_rows, num_blocks,
            head_dim, block_k, src.stride(0), src.stride(1), dst.stride(0), stream)
        _lib.check(status, "pool_blocks")


# Whole-tile workgroups of a call from which on the dense tail is not split:
# the launch is long enough to absorb the tail's walk (16 per workgroup slot
# of the chip); measured on the 128k layer (32768 workgroups), splitting
# gains nothing there and costs a launch.
SPLIT_MAX_WORKGROUPS = 8192


def _dense_tail_split(geo: _Geometry) -> int:
    """Query tiles of the call to split by key range: the dense tail (the
    last ``last_n_blocks`` tiles select every visible block,
    ``selection.py:191-195``) when its walk spans more than two segments and
    the call has few enough tiles that the tail, which otherwise walks the
    whole key range in one workgroup per tile, can be its critical path
    (chunked prefill, one GPU's share of a sharded layer)."""
    config = geo.config
    tail = min(config.last_n_blocks, geo.num_tiles)
    if not tail:
        return 0
    rows = geo.query_heads // geo.kv_heads * config.tile_q
    workgroups = geo.kv_heads * geo.num_tiles * -(-rows // 128)
    if workgroups >= SPLIT_MAX_WORKGROUPS:
        return 0
    last_row = geo.offset + geo.query_length - 1
    visible = min(geo.num_blocks, last_row // config.block_k + 1)
    steps = visible * -(-config.block_k // 32)
    return tail if steps > 2 * SPLIT_SEG_STEPS else 0


def _select_attend(q3, k3, v3, pooled_k, pooled_v, geo: _Geometry, *, scale, out=None,
                   marks=None, keep=None, hook_stats=True, split=None):
    """Selection and block-sparse attention of one hook call, given the
    pooled K/V (``[Hkv, >=Nb, D]`` views sharing one head stride).  Writes
    ``out`` (``[Hq, Lq, D]``, allocated when None) and returns it.
    ``hook_stats``: count the call in the hook's ``block_sparsity`` while
    statistics are on (``patch.py:150-155``); callers with counters of
    their own pass False.  ``split``: tiles to split by key range (None: the
    dense tail when it is long, ``_dense_tail_split``)."""
    config = geo.config
    device = q3.device
    lib = _lib.load()
    stream = _lib.stream_ptr(device)
    dtype = _lib.dtype_code(q3.dtype)
    kv_heads, num_tiles, num_blocks = geo.kv_heads, geo.num_tiles, geo.num_blocks
    ids = torch.empty((kv_heads, num_tiles, num_blocks), dtype=torch.int32, device=device)
    pruned_ids = torch.empty_like(ids)
    counts = torch.empty((kv_heads, num_tiles), dtype=torch.int32, device=device)
    pruned_counts = torch.empty_like(counts)
    with torch.cuda.device(device):
        params = _select_params(q3, num_blocks, kv_heads=kv_heads, scale=scale,
                                config=config, offset=geo.offset,
                                query_length=geo.query_length,
                                padded_length=geo.padded_query_length,
                                key_length=geo.key_length,
                                pooled_head_stride=pooled_k.stride(0))
        if marks is not None:
            marks("select")
        status = lib.fpv2_score_select(
            q3.data_ptr(), pooled_k.data_ptr(), dtype, params, None, None, ids.data_ptr(),
            counts.data_ptr(), pruned_ids.data_ptr(), pruned_counts.data_ptr(), stream)
        _lib.check(status, "score_select")
    if _collect_stats and hook_stats:
        global _visible_blocks
        total = _selected_totals.get(counts.device)
        if total is None:
            total = _selected_totals[counts.device] = SelectedBlockCounter()
        total.add(counts)
        _visible_blocks += _causal_block_count(kv_heads, geo.query_length, geo.offset, config)
    if out is None:
        out = torch.empty((geo.query_heads, geo.query_length, geo.head_dim),
                          dtype=q3.dtype, device=device)
    if marks is not None:
        marks("attention")
    split_tiles = _dense_tail_split(geo) if split is None else split
    _launch_attention(
        q3, k3, v3, pooled_k, pooled_v, ids, counts, pruned_ids, pruned_counts, out,
        device=device, scale=scale, config=config, offset=geo.offset,
        query_length=geo.query_length, key_length=geo.key_length, num_blocks=num_blocks,
        padded_query_length=geo.padded_query_length, out_rows=geo.query_length,
        split_tiles=split_tiles)
    if marks is not None:
        marks("done")
    if keep is not None:
        keep.update(config=config, offset=geo.offset, pooled_k=pooled_k, pooled_v=pooled_v,
                    lists=(ids, counts, pruned_ids, pruned_counts), split_tiles=split_tiles)
    return out


def _fpv2_sdpa(q, k, v, *, scale, config, marks=None, keep=None, split=None):
    """``fpv2_sdpa`` body.  ``marks(name)`` (optional) is called on the host
    between the launches ("pool", "select", "attention", "done") so a caller
    can record stream events around each kernel; ``keep`` (optional dict)
    receives the pooled tensors and block lists of the call."""
    geo = _geometry(q, k, v, config)
    device = _lib.require_device(q, k, v)
    lib = _lib.load()
    q3, k3, v3 = _kernel_ready(q[0]), _kernel_ready(k[0]), _kernel_ready(v[0])
    pooled_k = torch.empty((geo.kv_heads, geo.num_blocks, geo.head_dim), dtype=q.dtype,
                           device=device)
    pooled_v = torch.empty_like(pooled_k)
    with torch.cuda.device(device):
        if marks is not None:
            marks("pool")
        _pool_into(lib, k3, v3, pooled_k, pooled_v, dtype=_lib.dtype_code(q.dtype),
                   valid_rows=geo.key_length, num_blocks=geo.num_blocks,
                   block_k=geo.config.block_k, stream=_lib.stream_ptr(device))
    out = torch.empty((1, geo.query_heads, geo.query_length, geo.head_dim), dtype=q.dtype,
                      device=device)
    _select_attend(q3, k3, v3, pooled_k, pooled_v, geo, scale=scale, out=out[0],
                   marks=marks, keep=keep, split=split)
    return out


def _bottom_right_causal(q, k, attn_mask, is_causal) -> bool:
    query_length, key_length = q.shape[-2], k.shape[-2]
    if attn_mask is None:
        return bool(is_causal) and query_length == key_length
    if is_causal or CausalBias is None or not isinstance(attn_mask, CausalBias):
        return False
    if attn_mask.seq_len_q != query_length or attn_mask.seq_len_kv != key_length:
        return False
    if attn_mask.variant == CausalVariant.LOWER_RIGHT:
        return True
    return attn_mask.variant == CausalVariant.UPPER_LEFT and query_length == key_length


def _eligible(q, k, v, attn_mask, dropout_p, is_causal, enable_gqa, kwargs,
              config: FPV2Config, min_tokens: int) -> bool:
    if kwargs or dropout_p:
        return False
    if not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
        return False
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        return False
    if q.shape[0] != 1 or k.shape[0] != 1 or v.shape[0] != 1:
        return False
    if k.shape != v.shape or q.shape[-1] != k.shape[-1]:
        return False
    if q.shape[-2] > k.shape[-2] or q.shape[-2] < config.tile_q:
        return False
    if k.shape[-2] < min_tokens:
        return False
    if q.shape[-1] not in SUPPORTED_HEAD_DIMS:
        return False
    if q.dtype not in (torch.float16, torch.bfloat16):
        return False
    if k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    if not (q.device.type == "cuda" and k.device == q.device and v.device == q.device):
        return False
    if q.requires_grad or k.requires_grad or v.requires_grad:
        return False  # forward-only kernel
    if not k.shape[1] or q.shape[1] % k.shape[1]:
        return False
    if q.shape[1] != k.shape[1] and not enable_gqa:
        return False
    return _bottom_right_causal(q, k, attn_mask, is_causal)


def _call_original(query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa,
                   kwargs):
    """The original function on a passed-through call's arguments.

    torch routes a ``CausalBias`` mask through the bias's own dispatch only
    while ``F.scaled_dot_product_attention`` is the original function
    (``CausalBias.__torch_function__``); with the hook installed that test
    fails and the bias would reach the kernel as a plain tensor.  Such calls
    therefore take the bias's dispatch here, as the original would; the
    calls it makes back into ``F.scaled_dot_product_attention`` (a square
    causal call, or the materialised mask) go straight to the original."""
    global _forwarding
    if (CausalBias is not None and isinstance(attn_mask, CausalBias) and not kwargs
            and not _forwarding):
        _forwarding = True
        try:
            return CausalBias._dispatch(query, key, value, attn_mask, dropout_p=dropout_p,
                                        is_causal=is_causal, scale=scale, enable_gqa=enable_gqa)
        finally:
            _forwarding = False
    return _ORIGINAL_SDPA(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                          is_causal=is_causal, scale=scale, enable_gqa=enable_gqa, **kwargs)


def enable(
    config: FPV2Config | None = None,
    *,
    min_tokens: int = 4_096,
    collect_stats: bool = False,
    total_tokens: int | None = None,
    **config_fields: Any,
) -> None:
    """Replace torch SDPA with an FPV2-gated, request-aware wrapper."""
    global _collect_stats, _enabled, _selected_dense_blocks, _visible_blocks
    if min_tokens <= 0:
        raise ValueError("min_tokens must be positive")
    if not isinstance(collect_stats, bool):
        raise ValueError("collect_stats must be a boolean")
    if total_tokens is not None and (
        not isinstance(total_tokens, int)
        or isinstance(total_tokens, bool)
        or total_tokens <= 0
    ):
        raise ValueError("total_tokens must be a positive integer or None")
    if config is not None and config_fields:
        config = replace(config, **config_fields)
    elif config is None:
        config = FPV2Config(**config_fields)
    _collect_stats = collect_stats
    _selected_totals.clear()
    _selected_dense_blocks = 0
    _visible_blocks = 0

    def wrapped(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                scale=None, enable_gqa=False, **kwargs):
        if _forwarding:  # a call made by a pass-through's CausalBias dispatch
            return _ORIGINAL_SDPA(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                                  is_causal=is_causal, scale=scale, enable_gqa=enable_gqa,
                                  **kwargs)
        four_d = all(isinstance(t, torch.Tensor) and t.ndim == 4 for t in (query, key))
        call_config = _effective_config(config, query.shape[1], key.shape[1]) if four_d else None
        if call_config is not None:
            call_config = _request_config(call_config, key.shape[-2], total_tokens)
        if call_config is not None and _eligible(
            query, key, value, attn_mask, dropout_p, is_causal, enable_gqa, kwargs,
            call_config, min_tokens
        ) and _within_block_limit(query.shape[-2], key.shape[-2], call_config):
            call_scale = query.shape[-1] ** -0.5 if scale is None else scale
            return fpv2_sdpa(query, key, value, scale=call_scale, config=call_config)
        # dense calls: below min_tokens, or more key blocks than selection holds
        if _collect_stats and call_config is not None and _eligible(
            query, key, value, attn_mask, dropout_p, is_causal, enable_gqa, kwargs,
            call_config, 1
        ):
            global _selected_dense_blocks, _visible_blocks
            visible = _causal_block_count(
                key.shape[1], query.shape[-2], key.shape[-2] - query.shape[-2], call_config
            )
            _selected_dense_blocks += visible
            _visible_blocks += visible
        return _call_original(query, key, value, attn_mask, dropout_p, is_causal, scale,
                              enable_gqa, kwargs)

    F.scaled_dot_product_attention = wrapped
    _enabled = True


def disable() -> None:
    """Restore torch's original scaled dot-product attention."""
    global _collect_stats, _enabled
    F.scaled_dot_product_attention = _ORIGINAL_SDPA
    _collect_stats = False
    _enabled = False


def is_enabled() -> bool:
    """Whether the FPV2 SDPA hook is installed."""
    return _enabled
