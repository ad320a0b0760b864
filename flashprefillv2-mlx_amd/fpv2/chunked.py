"""Chunked prefill of one attention layer over a growing KV cache, with an
incremental pooled K/V cache.

The reference serves chunked prefill through its hook: the model appends each
chunk's K/V to its cache and calls attention with the chunk's queries against
the whole prefix, and the hook pads K/V to the block grid and re-pools the
whole prefix on every call (``fpv2/patch.py:125-138``, driven by
``fpv2/generate.py:97-110``).  ``ChunkedPrefill`` owns the layer's KV cache and
a pooled cache of the same capacity.  Each call pools only the blocks that
gained rows since the previous one (completed blocks once, the trailing
partial block again), then runs the hook's selection and block-sparse
attention on views of the two caches, read in place through their head
strides.

The output equals ``fpv2_sdpa`` on the same prefix, bit for bit: a block's
mean is computed exactly and rounded once, so a block pooled on its own equals
the same block pooled as part of the prefix, and the selection and attention
kernels see identical values.

Request rules follow the hook: with ``total_tokens`` known, the dense tail
applies only once the cache reaches it (``patch.py:55-63``); below
``min_tokens`` keys, or with fewer queries than one selection tile, the hook
hands the call to the original attention (``patch.py:177-205``), and here the
same kernels run exact causal attention instead (``alpha = 0`` selects every
visible block, and with no pruned block the correction is empty).  A prefix
longer than the selection kernel holds (more than ``FPV2_MAX_BLOCKS`` key
blocks), which the hook also hands to the original attention, runs exact
causal attention too: the attention kernel walks every visible block of
lists built without the selection kernel.

With ``collect_stats`` the layer counts selected and visible blocks as the
hook's ``block_sparsity`` does (``patch.py:66-88``): selected counts are kept
on the device and summed in batches (``SelectedBlockCounter``), and
``block_sparsity()`` synchronises once to read them.  Exact calls count as
dense, and a chunk of fewer queries than one tile is not counted, as the
hook's accounting rule leaves such calls out (``patch.py:255-266``).  These
counts are the layer's own: the calls do not enter the hook's
``fpv2.block_sparsity()``.

Every call runs on the current stream.  As with a module's buffers, the KV
and pooled caches are not synchronised across streams: a caller that moves
between streams orders the calls itself (``wait_stream``).
"""

from __future__ import annotations

from dataclasses import replace

import torch

from fpv2 import _lib
from fpv2.kernel import SUPPORTED_HEAD_DIMS, _launch_attention
from fpv2.patch import (SelectedBlockCounter, _causal_block_count, _effective_config, _geometry,
                        _pool_into, _request_config, _select_attend)
from fpv2.selection import FPV2Config


class ChunkedPrefill:
    """One attention layer's KV cache, pooled cache and chunked FPV2 attention.

    ``step(q, k, v)`` appends a chunk's keys/values (``[Hkv, L, D]`` or
    ``[1, Hkv, L, D]``) and attends the chunk's queries (``[Hq, L, D]`` or
    ``[1, Hq, L, D]``, the last ``L`` positions of the prefix) against the
    whole cache; it returns ``[1, Hq, L, D]``.
    """

    def __init__(self, query_heads: int, kv_heads: int, head_dim: int, capacity: int, *,
                 dtype: torch.dtype = torch.bfloat16, device: torch.device | str | None = None,
                 config: FPV2Config | None = None, total_tokens: int | None = None,
                 min_tokens: int = 4_096, collect_stats: bool = False) -> None:
        if kv_heads <= 0 or query_heads <= 0 or query_heads % kv_heads:
            raise ValueError("query heads must be divisible by KV heads")
        if head_dim not in SUPPORTED_HEAD_DIMS:
            raise ValueError(f"head dimension must be one of {SUPPORTED_HEAD_DIMS}")
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("q, k, and v must share float16 or bfloat16 dtype")
        if capacity <= 0:
            raise ValueError("capacity must be positive")
        if min_tokens <= 0:
            raise ValueError("min_tokens must be positive")
        if total_tokens is not None and (not isinstance(total_tokens, int)
                                         or isinstance(total_tokens, bool) or total_tokens <= 0):
            raise ValueError("total_tokens must be a positive integer or None")
        base = config if config is not None else FPV2Config()
        effective = _effective_config(base, query_heads, kv_heads)
        if effective is None:
            raise ValueError("GQA group size must divide 128 packed query rows")
        device = torch.device(device if device is not None else "cuda")
        if device.type != "cuda":
            raise RuntimeError("FPV2 kernels run on ROCm devices only (there is no CPU fallback)")
        self.config = effective
        self.query_heads, self.kv_heads, self.head_dim = query_heads, kv_heads, head_dim
        self.capacity = capacity
        self.total_tokens = total_tokens
        self.min_tokens = min_tokens
        self.dtype = dtype
        self.device = device
        bk = effective.block_k
        # Room for the query padding of the last chunk: keys are padded to
        # ceil(max(Lk, offset + Lq_pad) / block_k) blocks.
        self.block_capacity = -(-(capacity + effective.tile_q) // bk)
        self.k = torch.empty((kv_heads, capacity, head_dim), dtype=dtype, device=device)
        self.v = torch.empty_like(self.k)
        # Blocks that hold no key yet must pool to zero.
        self.pooled_k = torch.zeros((kv_heads, self.block_capacity, head_dim), dtype=dtype,
                                    device=device)
        self.pooled_v = torch.zeros_like(self.pooled_k)
        self.length = 0
        self._complete = 0  # leading blocks pooled with all their rows
        self.pooled_rows = 0  # rows read by pooling so far (for accounting)
        self.collect_stats = collect_stats
        self._selected = SelectedBlockCounter()
        self._visible = 0

    def reset(self) -> None:
        """Empty the caches (a new prompt)."""
        self.pooled_k.zero_()
        self.pooled_v.zero_()
        self.length = 0
        self._complete = 0
        self.pooled_rows = 0
        self._selected.reset()
        self._visible = 0

    def block_sparsity(self) -> float:
        """Fraction of visible causal blocks skipped by the ``attend`` calls
        since construction or ``reset`` (0 when nothing was counted)."""
        if not self._visible:
            return 0.0
        return 1.0 - self._selected.value() / self._visible

    @staticmethod
    def _three_d(x: torch.Tensor, name: str) -> torch.Tensor:
        if x.ndim == 4:
            if x.shape[0] != 1:
                raise ValueError("FPV2 currently supports batch size 1")
            x = x[0]
        if x.ndim != 3:
            raise ValueError(f"{name} must have shape [heads, sequence, dim] or [1, heads, sequence, dim]")
        return x

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append a chunk's keys and values to the cache."""
        k, v = self._three_d(k, "k"), self._three_d(v, "v")
        if k.shape != v.shape or k.shape[0] != self.kv_heads or k.shape[-1] != self.head_dim:
            raise ValueError("k and v must be [kv_heads, L, head_dim] of the cache's geometry")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise ValueError("q, k, and v must share float16 or bfloat16 dtype")
        k_rows, v_rows = self.reserve(k.shape[1])
        k_rows.copy_(k)
        v_rows.copy_(v)

    def reserve(self, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Append ``n`` rows without copying: returns the cache's next ``n``
        rows as ``[kv_heads, n, head_dim]`` views of K and V, for a producer
        that writes them in place (e.g. the kernel that normalises and
        rotates K).  They count as appended: fill them before ``attend``."""
        if n < 0 or self.length + n > self.capacity:
            raise ValueError("the KV cache capacity is exceeded")
        a, self.length = self.length, self.length + n
        return self.k[:, a:self.length], self.v[:, a:self.length]

    def _pool_new_blocks(self, device, lib) -> None:
        bk = self.config.block_k
        dtype = _lib.dtype_code(self.dtype)
        stream = _lib.stream_ptr(device)
        full = self.length // bk
        if full > self._complete:
            b0 = self._complete
            _pool_into(lib, self.k[:, b0 * bk:full * bk], self.v[:, b0 * bk:full * bk],
                       self.pooled_k[:, b0:full], self.pooled_v[:, b0:full], dtype=dtype,
                       valid_rows=(full - b0) * bk, num_blocks=full - b0, block_k=bk,
                       stream=stream)
            self.pooled_rows += (full - b0) * bk
            self._complete = full
        tail = self.length - full * bk
        if tail:  # the partial block, re-pooled until it completes
            _pool_into(lib, self.k[:, full * bk:self.length], self.v[:, full * bk:self.length],
                       self.pooled_k[:, full:full + 1], self.pooled_v[:, full:full + 1],
                       dtype=dtype, valid_rows=tail, num_blocks=1, block_k=bk, stream=stream)
            self.pooled_rows += tail

    def request_config(self, query_length: int | None = None) -> FPV2Config:
        """The configuration the next ``attend`` uses for the current cache
        (and, when given, a chunk of ``query_length`` queries).

        The hook sends a call to the original attention when the keys are
        fewer than ``min_tokens`` or the queries fewer than one tile
        (``patch.py:177-205``); those calls run exact causal attention here
        (``alpha = 0``)."""
        config = _request_config(self.config, self.length, self.total_tokens)
        if self.length < self.min_tokens or (
                query_length is not None and query_length < config.tile_q):
            config = replace(config, alpha=0.0)
        return config

    def attend(self, q: torch.Tensor, *, scale: float | None = None, marks=None,
               keep: dict | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """Attend ``q`` (the last ``L`` positions of the cached prefix).

        ``out``: optional ``[Hq, L, D]`` destination with any head and row
        stride (D contiguous), e.g. a transposed view of an ``[L, Hq * D]``
        buffer; the result is written there and returned as ``out[None]``."""
        q3 = self._three_d(q, "q")
        if q3.shape[0] != self.query_heads or q3.shape[-1] != self.head_dim:
            raise ValueError("q must be [query_heads, L, head_dim] of the cache's geometry")
        if q3.dtype != self.dtype:
            raise ValueError("q, k, and v must share float16 or bfloat16 dtype")
        if q3.shape[1] > self.length:
            raise ValueError("query length cannot exceed key length for causal attention")
        device = _lib.require_device(q3, self.k)
        lib = _lib.load()
        k3, v3 = self.k[:, :self.length], self.v[:, :self.length]
        geo = _geometry(q3[None], k3[None], v3[None], self.request_config(q3.shape[1]),
                        capped=False)
        with torch.cuda.device(device):
            if marks is not None:
                marks("pool")
            self._pool_new_blocks(device, lib)
        if q3.stride(-1) != 1:
            q3 = q3.contiguous()
        if out is None:
            out = torch.empty((self.query_heads, q3.shape[1], self.head_dim), dtype=self.dtype,
                              device=device)
        elif (out.shape != (self.query_heads, q3.shape[1], self.head_dim)
              or out.dtype != self.dtype or out.stride(-1) != 1):
            raise ValueError("out must be [query_heads, L, head_dim] of q's dtype with a "
                             "contiguous last dimension")
        _lib.require_device(out, q3)
        call_scale = self.head_dim ** -0.5 if scale is None else scale
        if self.collect_stats and keep is None:
            keep = {}
        pooled_k = self.pooled_k[:, :geo.num_blocks]
        pooled_v = self.pooled_v[:, :geo.num_blocks]
        if geo.num_blocks <= _lib.MAX_BLOCKS:
            _select_attend(q3, k3, v3, pooled_k, pooled_v, geo, scale=call_scale, out=out,
                           marks=marks, keep=keep, hook_stats=False)
        else:
            self._exact_attend(q3, k3, v3, pooled_k, pooled_v, geo, scale=call_scale,
                               out=out, marks=marks, keep=keep)
        if self.collect_stats and geo.query_length >= geo.config.tile_q:
            self._selected.add(keep["lists"][1])
            self._visible += _causal_block_count(self.kv_heads, geo.query_length, geo.offset,
                                                 geo.config)
        return out[None]

    @staticmethod
    def _exact_attend(q3, k3, v3, pooled_k, pooled_v, geo, *, scale, out, marks, keep):
        """Exact causal attention for a prefix past the selection kernel's
        block limit: the lists the selection would give at ``alpha = 0``
        (every block that starts at or before the tile's last row, in
        ascending order; nothing pruned), built here, then the attention
        kernel."""
        config, device = geo.config, q3.device
        hkv, nt, nb = geo.kv_heads, geo.num_tiles, geo.num_blocks
        if marks is not None:
            marks("select")
        ids = torch.arange(nb, dtype=torch.int32, device=device).expand(hkv, nt, nb).contiguous()
        tiles = torch.arange(nt, dtype=torch.int64, device=device)
        tile_last = geo.offset + torch.clamp((tiles + 1) * config.tile_q, max=geo.query_length) - 1
        counts = torch.clamp(tile_last // config.block_k + 1, max=nb).to(torch.int32)
        counts = counts.expand(hkv, nt).contiguous()
        pruned_counts = torch.zeros_like(counts)
        if marks is not None:
            marks("attention")
        _launch_attention(
            q3, k3, v3, pooled_k, pooled_v, ids, counts, ids, pruned_counts, out,
            device=device, scale=scale, config=config, offset=geo.offset,
            query_length=geo.query_length, key_length=geo.key_length, num_blocks=nb,
            padded_query_length=geo.padded_query_length, out_rows=geo.query_length)
        if marks is not None:
            marks("done")
        if keep is not None:
            keep.update(config=config, offset=geo.offset, pooled_k=pooled_k, pooled_v=pooled_v,
                        lists=(ids, counts, ids, pruned_counts))

    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, **kwargs) -> torch.Tensor:
        """Append the chunk's K/V, then attend its queries."""
        self.append(k, v)
        return self.attend(q, **kwargs)
