"""CPU oracle for FlashPrefill V2 — TEST INFRASTRUCTURE ONLY.

This module restates the reference's algorithm for the FPV2 hot path in numpy
so the HIP implementation can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker; the product package never does.

Reference files (``/root/reference``, MLX, not importable here):
  * ``fpv2/selection.py``  pooling, scoring/selection, density
  * ``fpv2/kernel.py``     block-list compaction, kernel numerics
  * ``fpv2/reference.py``  dense float32 FPV2 attention
  * ``fpv2/patch.py``      hook data flow (padding, tile rewrite, dense tail)

Numerics.  Arrays are numpy; a bfloat16 tensor is carried as a float32 array
whose values are bfloat16-representable.  Where the reference computes in
float32 through MLX (whose summation order is not pinned), the oracle
computes the same quantity in float64, i.e. the value the float32 paths
approximate:
  * pooling: exact float64 block mean, rounded once to the output dtype;
  * scores/energies: float64, so block decisions are those of exact
    arithmetic (implementations agree except within ~1e-4 of alpha);
  * attention: float32 (as ``reference.py``) or float64 on request.

How each function is pinned (tests/test_oracle_*.py):
  pool_blocks            closed form on arange / integer data, brute force
  block_scores_and_select  the reference's boolean KATs
                         (tests/test_selection.py:19-87), chunked ==
                         unchunked, brute-force loop restatement, alpha
                         monotonicity
  compact_block_indices  KAT (tests/test_kernel.py:66-72), permutation and
                         stable-order invariants, brute force
  fpv2_attention_*       exact causal attention at alpha=0 (textbook softmax
                         via torch SDPA in float64), explicit-entry float64
                         brute force, correction-improves-error property
  hook helpers           KATs from tests/test_patch.py:27-41,180-207
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

LOG2E = 1.4426950408889634


# --------------------------------------------------------------------------
# Rounding helpers
# --------------------------------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), as float32."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    out = rounded.view(np.float32).copy()
    out[nan] = np.nan
    return out


def f64_to_f32_odd(x) -> np.ndarray:
    """Round float64 to float32 with round-to-odd (sticky) semantics.

    Rounding the result once more to a format with at least two fewer
    significand bits (bfloat16, float16) then equals a single correct
    rounding of the float64 value.
    """
    x = np.asarray(x, dtype=np.float64)
    f = x.astype(np.float32)
    over = np.abs(f.astype(np.float64)) > np.abs(x)
    f = np.where(over, np.nextafter(f, np.float32(0)), f).astype(np.float32)
    inexact = f.astype(np.float64) != x
    bits = f.view(np.uint32).copy()
    bits[inexact & np.isfinite(x)] |= np.uint32(1)
    return bits.view(np.float32)


def round_f64(x, dtype: str) -> np.ndarray:
    """Correctly round float64 values to ``dtype`` ('bf16', 'f16', 'f32')."""
    if dtype == "f32":
        return np.asarray(x, dtype=np.float64).astype(np.float32)
    odd = f64_to_f32_odd(x)
    if dtype == "bf16":
        return f32_to_bf16(odd)
    if dtype == "f16":
        return odd.astype(np.float16).astype(np.float32)
    raise ValueError(dtype)


# --------------------------------------------------------------------------
# Configuration (duck-typed: any object with these attributes works)
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class OracleConfig:
    """Field-for-field copy of FPV2Config's defaults, selection.py:30-43."""

    block_k: int = 128
    tile_q: int = 128
    alpha: float = 0.1
    sink_tokens: int = 256
    window_tokens: int = 384
    last_n_blocks: int = 2
    mean_correction: bool = True
    score_chunk_tiles: int | None = None
    pack_gqa: bool = False


def _replace(config, **changes):
    fields = {name: getattr(config, name) for name in OracleConfig.__dataclass_fields__}
    fields.update(changes)
    return OracleConfig(**fields)


# --------------------------------------------------------------------------
# selection.py
# --------------------------------------------------------------------------

def pool_blocks(x, block_size: int = 128, *, valid_rows: int | None = None,
                out_dtype: str = "f32") -> np.ndarray:
    """Block mean over the penultimate axis (selection.py:68-80).

    The mean is exact in float64 (sum of the block's rows, rows at or beyond
    ``valid_rows`` counting as zero as the hook's zero padding does,
    patch.py:125-138) and rounded once to ``out_dtype``.
    """
    x = np.asarray(x, dtype=np.float64)
    if x.ndim < 2:
        raise ValueError("x must have at least sequence and feature dimensions")
    length, head_dim = x.shape[-2:]
    if length % block_size:
        raise ValueError(
            f"sequence length {length} must be divisible by block_size {block_size}"
        )
    if valid_rows is not None and valid_rows < length:
        x = x.copy()
        x[..., valid_rows:, :] = 0.0
    shape = (*x.shape[:-2], length // block_size, block_size, head_dim)
    mean = x.reshape(shape).sum(axis=-2) / block_size
    return round_f64(mean, out_dtype)


def block_scores_and_select(q, pooled_k, *, scale: float, config=OracleConfig(),
                            offset: int = 0, query_length: int | None = None,
                            return_ratio: bool = False):
    """Selection mask ``[Hkv, Nt, Nb]`` (selection.py:109-201), float64.

    Returns ``(selected, scores)`` like the reference — ``scores`` is the raw
    ``[Hkv, G, N, Nb]`` score tensor when ``config.score_chunk_tiles`` is
    None — plus, if ``return_ratio``, the energy/max-energy ratio
    ``[Hkv, Nt, Nb]`` used to exclude near-alpha decisions from bit-exact
    comparisons.
    """
    q = np.asarray(q, dtype=np.float64)
    pooled_k = np.asarray(pooled_k, dtype=np.float64)
    query_heads, padded_length, head_dim = q.shape
    kv_heads, num_blocks, key_dim = pooled_k.shape
    valid_length = padded_length if query_length is None else query_length
    # _validate_inputs, selection.py:83-106
    if not kv_heads or query_heads % kv_heads:
        raise ValueError("query heads must be divisible by KV heads")
    if head_dim != key_dim:
        raise ValueError("q and pooled_k head dimensions must match")
    if padded_length % config.tile_q:
        raise ValueError("query length must be padded to a multiple of tile_q")
    if not 0 < valid_length <= padded_length:
        raise ValueError("query_length must be in (0, q.shape[-2]]")
    if offset < 0:
        raise ValueError("offset must be non-negative")
    if offset + valid_length > num_blocks * config.block_k:
        raise ValueError("queries extend beyond the represented key sequence")

    group = query_heads // kv_heads
    tq = config.tile_q
    num_tiles = padded_length // tq
    grouped_q = q.reshape(kv_heads, group, padded_length, head_dim)
    block_starts = np.arange(num_blocks, dtype=np.int64) * config.block_k
    block_ends = block_starts + config.block_k
    sink = block_starts < config.sink_tokens
    chunk = config.score_chunk_tiles or num_tiles
    chunks, ratios = [], []
    raw_scores = None
    for tile_start in range(0, num_tiles, chunk):
        tile_end = min(tile_start + chunk, num_tiles)
        rows = np.arange(tile_start * tq, tile_end * tq, dtype=np.int64)
        tile_ids = np.arange(tile_start, tile_end, dtype=np.int64)
        tile_first = offset + tile_ids * tq
        tile_last = np.minimum(tile_first + tq, offset + valid_length) - 1
        # Blocks starting after the chunk's last valid row are invisible to
        # every tile of the chunk (not selected, zero energy): only the
        # leading `nbv` blocks are evaluated (the unchunked call, whose raw
        # scores are returned, evaluates all of them).
        nbv = num_blocks
        if config.score_chunk_tiles is not None:
            nbv = min(num_blocks, int(tile_last.max()) // config.block_k + 1)
        # s[h, g, n, b] = q[h, g, n] . k̄[h, b] (selection.py:154-158), as a
        # batched float64 BLAS product
        scores = np.matmul(grouped_q[:, :, rows[0]:rows[-1] + 1],
                           np.swapaxes(pooled_k[:, :nbv], -1, -2)[:, None]) * scale
        starts, ends = block_starts[:nbv], block_ends[:nbv]
        positions = offset + rows
        row_visible = (starts[None, :] <= positions[:, None]) & (rows[:, None] < valid_length)
        tiles = np.where(row_visible[None, None], scores, -np.inf).reshape(
            kv_heads, group, tile_end - tile_start, tq, nbv)
        fully_visible = ends[None, :] <= tile_last[:, None] + 1
        tiles = np.where(fully_visible[None, None, :, None, :], tiles, -np.inf)
        tile_max = tiles.max(axis=(1, 3, 4), keepdims=True)
        # exp(s - m) on the visible entries, 0 elsewhere (-inf -> 0)
        finite = tiles > -np.inf
        weights = np.zeros(tiles.shape)
        with np.errstate(invalid="ignore"):
            np.exp(np.subtract(tiles, tile_max, where=finite, out=weights), where=finite,
                   out=weights)
        energies = np.zeros((kv_heads, tile_end - tile_start, num_blocks))
        energies[..., :nbv] = weights.sum(axis=(1, 3))
        max_energy = energies.max(axis=-1, keepdims=True)
        selected = energies >= config.alpha * max_energy
        with np.errstate(invalid="ignore", divide="ignore"):
            ratios.append(np.where(max_energy > 0, energies / np.where(
                max_energy > 0, max_energy, 1.0), np.inf))
        visible = block_starts[None, :] <= tile_last[:, None]
        local = block_ends[None, :] > (tile_first[:, None] - config.window_tokens)
        dense_tail = tile_ids >= max(num_tiles - config.last_n_blocks, 0)
        forced = sink[None, :] | local | dense_tail[:, None]
        chunks.append((selected | forced[None]) & visible[None])
        if config.score_chunk_tiles is None:
            raw_scores = scores
    selected = np.concatenate(chunks, axis=1)
    scores_out = raw_scores if len(chunks) == 1 else None
    if return_ratio:
        return selected, scores_out, np.concatenate(ratios, axis=1)
    return selected, scores_out


def density(selected, *, config=OracleConfig(), offset: int = 0,
            query_length: int | None = None) -> float:
    """Retained fraction of causally visible blocks (selection.py:204-229)."""
    selected = np.asarray(selected, dtype=bool)
    kv_heads, num_tiles, num_blocks = selected.shape
    valid = num_tiles * config.tile_q if query_length is None else query_length
    tile_last = np.minimum(
        offset + (np.arange(num_tiles) + 1) * config.tile_q, offset + valid) - 1
    block_starts = np.arange(num_blocks) * config.block_k
    visible = block_starts[None, :] <= tile_last[:, None]
    return float(selected.sum()) / float(visible.sum() * kv_heads)


# --------------------------------------------------------------------------
# kernel.py
# --------------------------------------------------------------------------

def compact_block_indices(selected, *, config=OracleConfig(), offset: int = 0,
                          query_length: int | None = None,
                          key_length: int | None = None):
    """Padded ascending block lists and counts (kernel.py:141-184).

    ``argsort(-mask)`` with a stable sort: the selected blocks ascending,
    then the remaining blocks ascending.
    """
    selected = np.asarray(selected)
    if selected.dtype != np.bool_:
        raise ValueError("selected must have boolean dtype")
    _, num_tiles, num_blocks = selected.shape
    valid_key = num_blocks * config.block_k if key_length is None else key_length
    sel_i = selected.astype(np.int32)
    ids = np.argsort(-sel_i, axis=-1, kind="stable").astype(np.int32)
    counts = sel_i.sum(axis=-1).astype(np.int32)
    tile_first = offset + np.arange(num_tiles) * config.tile_q
    block_ends = np.minimum((np.arange(num_blocks) + 1) * config.block_k, valid_key)
    fully_past = block_ends[None, :] <= tile_first[:, None]
    pruned = (~selected) & fully_past[None]
    pr_i = pruned.astype(np.int32)
    pruned_ids = np.argsort(-pr_i, axis=-1, kind="stable").astype(np.int32)
    pruned_counts = pr_i.sum(axis=-1).astype(np.int32)
    return ids, counts, pruned_ids, pruned_counts


# --------------------------------------------------------------------------
# reference.py — dense FPV2 attention
# --------------------------------------------------------------------------

def fpv2_attention_reference(q, k, v, *, scale: float, config=OracleConfig(),
                             offset: int = 0, dtype=np.float32):
    """Literal restatement of ``fpv2_attention_reference`` (reference.py:10-90).

    Materialises ``[Hkv, G, Lq, Lk]``; use for small shapes only.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    if k.shape != v.shape:
        raise ValueError("k and v must have identical shapes")
    if q.shape[1] % config.tile_q or k.shape[1] % config.block_k:
        raise ValueError("q and k/v sequence lengths must be tile/block aligned")
    if offset < 0 or offset + q.shape[1] > k.shape[1]:
        raise ValueError("offset does not align queries within the key sequence")
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    g = hq // hkv
    nt = lq // config.tile_q
    nb = lk // config.block_k
    gq = q.astype(dtype).reshape(hkv, g, lq, d)
    k32 = k.astype(dtype)
    v32 = v.astype(dtype)
    pooled_k = pool_blocks(k32, config.block_k, out_dtype="f32").astype(dtype)
    pooled_v = pool_blocks(v32, config.block_k, out_dtype="f32").astype(dtype)
    selected, _ = block_scores_and_select(q, pooled_k, scale=scale, config=config,
                                          offset=offset)
    pooled_scores = np.einsum("hgnd,hbd->hgnb", gq, pooled_k) * dtype(scale)
    token_scores = np.einsum("hgnd,hmd->hgnm", gq, k32) * dtype(scale)
    qpos = offset + np.arange(lq)
    kpos = np.arange(lk)
    causal = kpos[None, :] <= qpos[:, None]
    sel_tok = np.repeat(np.repeat(selected, config.tile_q, axis=1),
                        config.block_k, axis=2)[:, :lq, :lk]
    kept = sel_tok[:, None] & causal[None, None]
    exact = np.where(kept, token_scores, -np.inf)
    if config.mean_correction:
        tile_first = offset + np.arange(nt) * config.tile_q
        block_ends = (np.arange(nb) + 1) * config.block_k
        corrected = (~selected) & (block_ends[None, :] <= tile_first[:, None])[None]
        corr_rows = np.repeat(corrected, config.tile_q, axis=1)
        corr = np.where(corr_rows[:, None], pooled_scores + dtype(math.log(config.block_k)),
                        -np.inf)
    else:
        corr = np.full_like(pooled_scores, -np.inf)
    row_max = np.maximum(exact.max(axis=-1, keepdims=True), corr.max(axis=-1, keepdims=True))
    we = np.exp(exact - row_max)
    wc = np.exp(corr - row_max)
    num = np.einsum("hgnm,hmd->hgnd", we, v32) + np.einsum("hgnb,hbd->hgnd", wc, pooled_v)
    den = we.sum(axis=-1, keepdims=True) + wc.sum(axis=-1, keepdims=True)
    return (num / den).reshape(hq, lq, d)


def fpv2_attention_blockwise(q, k, v, *, scale: float, selected, pooled_k,
                             pooled_v, config=OracleConfig(), offset: int = 0,
                             query_length: int | None = None,
                             key_length: int | None = None,
                             dtype=np.float32, tiles=None, row_block: int = 256):
    """Row-blockwise restatement of reference.py:55-90 with explicit inputs.

    Rows are independent, so evaluating query rows in blocks is exact up to
    summation order.  ``selected`` / ``pooled_k`` / ``pooled_v`` are given
    explicitly so a test can supply the same selection and pooled values the
    device used (the hook path casts pooled K/V to the query dtype,
    kernel.py:553-554).  Key padding beyond ``key_length`` is masked, and the
    correction uses the clipped block end as compact_block_indices does
    (kernel.py:174-180).  ``tiles`` restricts evaluation to a subset of
    query tiles (used for bounded CPU timing); other rows are left at zero.
    Returns float ``[Hq, Lq_pad, D]``.
    """
    q = np.asarray(q)
    hq, lq_pad, d = q.shape
    hkv, lk_pad, _ = np.asarray(k).shape
    g = hq // hkv
    tq, bk = config.tile_q, config.block_k
    nb = np.asarray(pooled_k).shape[1]
    valid_q = lq_pad if query_length is None else query_length
    valid_k = lk_pad if key_length is None else key_length
    selected = np.asarray(selected, dtype=bool)
    out = np.zeros((hq, lq_pad, d), dtype=dtype)
    kpos = np.arange(lk_pad)
    log_bk = dtype(math.log(bk))
    tile_list = range(lq_pad // tq) if tiles is None else tiles
    rows_per = max(tq, (row_block // tq) * tq)
    tile_list = list(tile_list)
    for h in range(hkv):
        kh = np.asarray(k[h], dtype=dtype)
        vh = np.asarray(v[h], dtype=dtype)
        pk = np.asarray(pooled_k[h], dtype=dtype)
        pv = np.asarray(pooled_v[h], dtype=dtype)
        qh = np.asarray(q[h * g:(h + 1) * g], dtype=dtype)
        i = 0
        while i < len(tile_list):
            # group consecutive tiles up to rows_per rows
            group_tiles = [tile_list[i]]
            while (i + len(group_tiles) < len(tile_list)
                   and tile_list[i + len(group_tiles)] == group_tiles[-1] + 1
                   and len(group_tiles) * tq < rows_per):
                group_tiles.append(tile_list[i + len(group_tiles)])
            i += len(group_tiles)
            r0 = group_tiles[0] * tq
            r1 = (group_tiles[-1] + 1) * tq
            last_pos = offset + min(r1, valid_q) - 1
            kmax = min(valid_k, last_pos + 1)
            if r0 >= valid_q:
                continue
            rows = np.arange(r0, r1)
            qpos = offset + rows
            sel_rows = np.repeat(selected[h, group_tiles], tq, axis=0)  # [R, Nb]
            sel_tok = np.repeat(sel_rows, bk, axis=1)[:, :kmax]
            kept = sel_tok & (kpos[None, :kmax] <= qpos[:, None])
            qs = qh[:, r0:r1]
            logits = np.matmul(qs, kh[:kmax].T) * dtype(scale)  # BLAS
            logits = np.where(kept[None], logits, -np.inf)
            if config.mean_correction:
                tfirst = offset + np.asarray(group_tiles) * tq
                bend = np.minimum((np.arange(nb) + 1) * bk, valid_k)
                corr = (~selected[h, group_tiles]) & (bend[None, :] <= tfirst[:, None])
                corr_rows = np.repeat(corr, tq, axis=0)
                cl = np.matmul(qs, pk.T) * dtype(scale) + log_bk
                cl = np.where(corr_rows[None], cl, -np.inf)
            else:
                cl = np.full((g, r1 - r0, nb), -np.inf, dtype=dtype)
            with np.errstate(invalid="ignore"):
                m = np.maximum(logits.max(axis=-1, keepdims=True),
                               cl.max(axis=-1, keepdims=True))
                m = np.where(np.isfinite(m), m, 0)
                we = np.exp(logits - m)
                wc = np.exp(cl - m)
            num = np.matmul(we, vh[:kmax]) + np.matmul(wc, pv)
            den = we.sum(axis=-1, keepdims=True) + wc.sum(axis=-1, keepdims=True)
            with np.errstate(invalid="ignore", divide="ignore"):
                res = np.where(den > 0, num / np.where(den > 0, den, 1), 0)
            res[:, rows >= valid_q] = 0
            out[h * g:(h + 1) * g, r0:r1] = res
    return out


def exact_causal_attention(q, k, v, scale: float, offset: int = 0):
    """Plain causal softmax attention in float64 (tests/test_reference.py:10-26)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    gq = q.reshape(hkv, hq // hkv, lq, d)
    s = np.einsum("hgnd,hmd->hgnm", gq, k) * scale
    causal = np.arange(lk)[None, :] <= (offset + np.arange(lq))[:, None]
    s = np.where(causal[None, None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return np.einsum("hgnm,hmd->hgnd", w, v).reshape(hq, lq, d)


# --------------------------------------------------------------------------
# patch.py — hook data flow
# --------------------------------------------------------------------------

PACKED_TILE_ROWS = 128


def effective_config(config, query_heads: int, kv_heads: int):
    """tile_q 128 -> 128 / G (patch.py:41-52)."""
    if config.tile_q != PACKED_TILE_ROWS:
        return config
    if not kv_heads or query_heads % kv_heads:
        return None
    group = query_heads // kv_heads
    if PACKED_TILE_ROWS % group:
        return None
    return _replace(config, tile_q=PACKED_TILE_ROWS // group)


def request_config(config, key_length: int, total_tokens):
    """Dense tail only at the request boundary (patch.py:55-63)."""
    if config.last_n_blocks and (total_tokens is None or key_length < total_tokens):
        return _replace(config, last_n_blocks=0)
    return config


def causal_block_count(kv_heads: int, query_length: int, offset: int, config) -> int:
    """Visible (tile, block) pairs times KV heads (patch.py:66-76)."""
    count = 0
    for start in range(0, query_length, config.tile_q):
        end = offset + min(start + config.tile_q, query_length)
        count += (end + config.block_k - 1) // config.block_k
    return count * kv_heads


def hook_plan(query_heads, kv_heads, query_length, key_length, config):
    """Padded geometry of fpv2_sdpa (patch.py:115-136)."""
    cfg = effective_config(config, query_heads, kv_heads)
    offset = key_length - query_length
    lq_pad = -(-query_length // cfg.tile_q) * cfg.tile_q
    need = max(key_length, offset + lq_pad)
    lk_pad = -(-need // cfg.block_k) * cfg.block_k
    return cfg, offset, lq_pad, lk_pad


def fpv2_sdpa_oracle(q, k, v, *, scale: float, config=OracleConfig(),
                     dtype: str = "bf16", return_plan: bool = False, tiles=None,
                     score_chunk_tiles: int = 16):
    """The hook's data flow (patch.py:102-174) on ``[Hq, Lq, D]`` inputs.

    Pads Q/K/V with zeros, pools K/V in the input dtype (bf16 on the hook
    path), selects on those pooled keys, compacts with the valid key length
    and evaluates attention with the kernel's semantics (pooled values in the
    input dtype).  Returns float32 ``[Hq, Lq, D]``; with ``tiles`` only
    those query tiles are evaluated (other rows stay zero).
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    cfg, offset, lq_pad, lk_pad = hook_plan(hq, hkv, lq, lk, config)
    qp = np.zeros((hq, lq_pad, d), np.float32)
    qp[:, :lq] = q
    kp = np.zeros((hkv, lk_pad, d), np.float32)
    kp[:, :lk] = k
    vp = np.zeros((hkv, lk_pad, d), np.float32)
    vp[:, :lk] = v
    pk = pool_blocks(kp, cfg.block_k, out_dtype=dtype)
    pv = pool_blocks(vp, cfg.block_k, out_dtype=dtype)
    selected, _, ratio = block_scores_and_select(
        qp, pk, scale=scale, config=_replace(cfg, score_chunk_tiles=score_chunk_tiles),
        offset=offset, query_length=lq, return_ratio=True)
    lists = compact_block_indices(selected, config=cfg, offset=offset,
                                  query_length=lq, key_length=lk)
    out = fpv2_attention_blockwise(qp, kp, vp, scale=scale, selected=selected,
                                   pooled_k=pk, pooled_v=pv, config=cfg, offset=offset,
                                   query_length=lq, key_length=lk, tiles=tiles)[:, :lq]
    if return_plan:
        return out, dict(config=cfg, offset=offset, selected=selected, ratio=ratio,
                         pooled_k=pk, pooled_v=pv, lists=lists)
    return out


# --------------------------------------------------------------------------
# Whole calls over tile ranges (parallel threads)
# --------------------------------------------------------------------------

def _tile_ranges(num_tiles, tile_q, offset, parts, last_n):
    """Contiguous tile ranges of about equal causal work (a tile's keys grow
    with its position); the last range keeps at least ``last_n`` tiles, so
    the dense tail is decided within one range."""
    work = offset + (np.arange(num_tiles) + 1) * tile_q
    cum = np.cumsum(work)
    bounds = np.searchsorted(cum, cum[-1] * np.arange(1, parts) / parts, side="left") + 1
    edges = sorted({0, num_tiles, *[int(b) for b in bounds if 0 < b < num_tiles]})
    ranges = [[a, b] for a, b in zip(edges[:-1], edges[1:])]
    if len(ranges) > 1 and ranges[-1][1] - ranges[-1][0] < last_n:
        last = ranges.pop()
        ranges[-1][1] = last[1]
    return ranges


def _map_ranges(fn, ranges, workers):
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits
    if workers <= 1:
        return [fn(r) for r in ranges]
    # numpy releases the GIL in its ufuncs and BLAS calls; BLAS runs
    # single-threaded per range (the limit is process-wide: set once)
    with threadpool_limits(limits=1), ThreadPoolExecutor(max_workers=workers) as pool:
        return list(pool.map(fn, ranges))


def select_tile_ranges(q, pooled_k, *, scale, config=OracleConfig(), offset: int = 0,
                       query_length: int | None = None, workers: int = 1,
                       chunk_tiles: int = 32):
    """``block_scores_and_select`` of a whole call, evaluated as calls of
    contiguous tile ranges (each at its own offset, the dense tail kept only
    in the range that ends the call) on ``workers`` threads.  Tiles are
    independent (selection.py:144-201 scores them in any grouping), so the
    result equals the one-call selection.  Returns ``(selected, ratio)``."""
    q = np.asarray(q)
    tq = config.tile_q
    lq_pad = q.shape[1]
    valid = lq_pad if query_length is None else query_length
    nt = lq_pad // tq  # (every tile holds a valid row: lq_pad = ceil(valid / tq) * tq)
    ranges = _tile_ranges(nt, tq, offset, max(1, 4 * workers), config.last_n_blocks)

    def one(r):
        t0, t1 = r
        sub = config if t1 == nt else _replace(config, last_n_blocks=0)
        rows0, rows1 = t0 * tq, t1 * tq
        sel, _, ratio = block_scores_and_select(
            q[:, rows0:rows1], pooled_k, scale=scale,
            config=_replace(sub, score_chunk_tiles=chunk_tiles), offset=offset + rows0,
            query_length=min(rows1, valid) - rows0, return_ratio=True)
        return sel, ratio

    parts = _map_ranges(one, ranges, workers)
    return (np.concatenate([p[0] for p in parts], axis=1),
            np.concatenate([p[1] for p in parts], axis=1))


def attention_tile_ranges(q, k, v, *, scale: float, selected, pooled_k, pooled_v,
                          config=OracleConfig(), offset: int = 0,
                          query_length: int | None = None, key_length: int | None = None,
                          workers: int = 1, dtype=np.float32, row_block: int = 256):
    """``fpv2_attention_blockwise`` of a whole call, evaluated over
    contiguous tile ranges on ``workers`` threads.  Rows are independent, so
    the result equals the one-call evaluation.  Returns ``[Hq, Lq_pad, D]``."""
    q = np.asarray(q)
    tq = config.tile_q
    hq, lq_pad, d = q.shape
    valid = lq_pad if query_length is None else query_length
    nt = lq_pad // tq
    selected = np.asarray(selected, dtype=bool)
    out = np.zeros((hq, lq_pad, d), dtype=dtype)
    ranges = _tile_ranges(nt, tq, offset, max(1, 4 * workers), 0)

    def one(r):
        t0, t1 = r
        rows0, rows1 = t0 * tq, t1 * tq
        if rows0 >= valid:
            return
        out[:, rows0:rows1] = fpv2_attention_blockwise(
            q[:, rows0:rows1], k, v, scale=scale, selected=selected[:, t0:t1],
            pooled_k=pooled_k, pooled_v=pooled_v, config=config, offset=offset + rows0,
            query_length=min(rows1, valid) - rows0, key_length=key_length, dtype=dtype,
            row_block=row_block)

    _map_ranges(one, ranges, workers)
    return out
