"""Parity at BASELINE's full sizes on a sample of query tiles.

The hook runs the whole layer (Qwen3-4B geometry, BASELINE generator) on the
GPU at seq 32768 and 131072; the oracle then evaluates the last few query
tiles from the same inputs and the device's pooled keys:
  * block lists of those tiles bit-exact against the oracle's selection,
    excluding blocks whose energy ratio lies within 1e-4 of alpha;
  * their attention rows within max-abs 2e-2 / mean-abs 2e-3 of the oracle's
    blockwise float32 evaluation on the device's selection.
Rows are independent, so the last tiles (the longest rows, the dense tail
and the most blocks) check the full-length walk without evaluating the whole
layer on the CPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import attention_errors, to_np
from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config
from fpv2.patch import _fpv2_sdpa
from fpv2.synthetic import baseline_qkv

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS, BAND = 2e-2, 2e-3, 1e-4


def _device_mask(ids, counts, tiles, num_blocks):
    ids, counts = to_np(ids[:, tiles]), to_np(counts[:, tiles])
    mask = np.zeros(ids.shape[:2] + (num_blocks,), dtype=bool)
    for h in range(ids.shape[0]):
        for t in range(ids.shape[1]):
            mask[h, t, ids[h, t, :counts[h, t]]] = True
    return mask


@pytest.mark.parametrize(("seq", "heavy", "planted", "n_tiles", "skip"), [
    (32768, 0.06, 3.0, 6, 0),
    (131072, 0.03, 3.0, 3, 0),
    # the bench's contrast variant: planted x 3*sqrt(D) prunes most blocks, so
    # the correction phase carries hundreds of pooled rows per tile; the tiles
    # just before the dense tail (the last 2 tiles) are sampled
    (131072, 0.03, 3.0 * 128 ** 0.5, 3, 2),
])
def test_last_tiles_match_oracle_at_full_size(cuda, seq, heavy, planted, n_tiles, skip):
    q, k, v = baseline_qkv(seq, planted=planted, heavy_fraction=heavy, seed=0, device=cuda)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    keep = {}
    out = _fpv2_sdpa(q[None], k[None], v[None], scale=128 ** -0.5, config=config, keep=keep)
    torch.cuda.synchronize()
    cfg = keep["config"]
    tq = cfg.tile_q
    nt = seq // tq
    rows0 = seq - (n_tiles + skip) * tq
    ids, counts, _, _ = keep["lists"]
    num_blocks = ids.shape[-1]
    dev_sel = _device_mask(ids, counts, slice(nt - n_tiles - skip, nt - skip), num_blocks)

    ocfg = orc.OracleConfig(**{f: getattr(cfg, f) for f in orc.OracleConfig.__dataclass_fields__})
    if skip:  # the sampled tiles are not the call's last ones: no dense tail among them
        ocfg = orc._replace(ocfg, last_n_blocks=0)
    pooled_k = to_np(keep["pooled_k"])
    pooled_v = to_np(keep["pooled_v"])
    qs = to_np(q[:, rows0:rows0 + n_tiles * tq])
    sel, _, ratio = orc.block_scores_and_select(
        qs, pooled_k, scale=128 ** -0.5, config=orc._replace(ocfg, score_chunk_tiles=1),
        offset=rows0, query_length=n_tiles * tq, return_ratio=True)
    decided = np.abs(ratio - cfg.alpha) > BAND
    assert np.array_equal(sel[decided], dev_sel[decided])
    assert dev_sel.sum() > 0
    if planted > 3.0:
        assert dev_sel.mean() < 0.5  # sparse: the correction phase is exercised

    ref = orc.fpv2_attention_blockwise(
        qs, to_np(k), to_np(v), scale=128 ** -0.5, selected=dev_sel, pooled_k=pooled_k,
        pooled_v=pooled_v, config=ocfg, offset=rows0, row_block=tq)
    err = attention_errors(to_np(out[0, :, rows0:rows0 + n_tiles * tq]), ref)
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err


def test_maximum_block_count(cuda):
    """The largest key range the scoring kernel accepts (FPV2_MAX_BLOCKS =
    8192 blocks, 1 048 576 keys): the last 256 query positions (8 tiles, the
    last 2 dense) against the whole prefix, high-contrast generator so the
    correction phase walks thousands of pooled rows per tile."""
    from fpv2 import _lib
    seq, lq = _lib.MAX_BLOCKS * 128, 256
    q, k, v = baseline_qkv(seq, query_heads=8, kv_heads=2, head_dim=128,
                           planted=3.0 * 128 ** 0.5, heavy_fraction=0.03, seed=1, device=cuda)
    q = q[:, seq - lq:].contiguous()
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    keep = {}
    out = _fpv2_sdpa(q[None], k[None], v[None], scale=128 ** -0.5, config=config, keep=keep)
    torch.cuda.synchronize()
    cfg = keep["config"]
    ids, counts, _, _ = keep["lists"]
    num_blocks = ids.shape[-1]
    assert num_blocks == _lib.MAX_BLOCKS
    dev_sel = _device_mask(ids, counts, slice(0, lq // cfg.tile_q), num_blocks)

    ocfg = orc.OracleConfig(**{f: getattr(cfg, f) for f in orc.OracleConfig.__dataclass_fields__})
    pooled_k, pooled_v = to_np(keep["pooled_k"]), to_np(keep["pooled_v"])
    qs = to_np(q)
    sel, _, ratio = orc.block_scores_and_select(
        qs, pooled_k, scale=128 ** -0.5, config=orc._replace(ocfg, score_chunk_tiles=1),
        offset=seq - lq, query_length=lq, return_ratio=True)
    decided = np.abs(ratio - cfg.alpha) > BAND
    assert np.array_equal(sel[decided], dev_sel[decided])
    assert dev_sel[:, :-2].mean() < 0.5  # sparse outside the dense tail

    ref = orc.fpv2_attention_blockwise(
        qs, to_np(k), to_np(v), scale=128 ** -0.5, selected=dev_sel, pooled_k=pooled_k,
        pooled_v=pooled_v, config=ocfg, offset=seq - lq, row_block=cfg.tile_q)
    err = attention_errors(to_np(out[0]), ref)
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err
