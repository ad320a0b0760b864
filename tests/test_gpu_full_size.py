"""Parity at BASELINE's full sizes.

The hook runs the whole layer (Qwen3-4B geometry, BASELINE generator) on the
GPU at seq 32768 and 131072; the oracle then checks, from the same inputs:
  * the pooled K/V of the whole layer, bit-exact against the oracle's pooling
    of the full K/V;
  * the block lists of every query tile bit-exact against the oracle's
    selection (scored on the host's cores over tile ranges), excluding
    blocks whose energy ratio lies within 1e-4 of alpha, and the full
    padded selected/pruned lists against the oracle's compaction;
  * the attention rows of the sampled tiles within max-abs 2e-2 / mean-abs
    2e-3 of the oracle's blockwise float32 evaluation on the device's
    selection.
Rows are independent, so sampled tiles check the full-length walk without
evaluating the whole layer on the CPU.  Also: the 32k layer without
correction (BASELINE config 2's ablation) and a bitwise re-run of the 32k
layer (determinism).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import attention_errors, oracle_select_parallel, to_np
from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config
from fpv2.patch import _fpv2_sdpa
from fpv2.synthetic import baseline_qkv

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS, BAND = 2e-2, 2e-3, 1e-4
SCALE = 128 ** -0.5


def _device_mask(ids, counts, tiles, num_blocks):
    ids, counts = to_np(ids[:, tiles]), to_np(counts[:, tiles])
    mask = np.zeros(ids.shape[:2] + (num_blocks,), dtype=bool)
    for h in range(ids.shape[0]):
        for t in range(ids.shape[1]):
            mask[h, t, ids[h, t, :counts[h, t]]] = True
    return mask


def _oracle_config(cfg):
    return orc.OracleConfig(**{f: getattr(cfg, f) for f in orc.OracleConfig.__dataclass_fields__})


def _check_tiles(q, kn, vn, out, keep, seq, samples, *, sparse=False):
    """Oracle comparison of tile groups ``(first_tile, n_tiles)`` of one call
    whose queries are the last ``seq`` positions of ``kn``/``vn``."""
    cfg = keep["config"]
    tq = cfg.tile_q
    nt = -(-seq // tq)
    off = kn.shape[1] - seq
    ids, counts, _, _ = keep["lists"]
    num_blocks = ids.shape[-1]
    ocfg = _oracle_config(cfg)
    pooled_k, pooled_v = to_np(keep["pooled_k"]), to_np(keep["pooled_v"])
    for t0, n in samples:
        rows0 = t0 * tq
        # the sampled tiles as a call of their own: the dense tail belongs to
        # the last tiles of the real call only
        sub = ocfg if t0 + n == nt else orc._replace(ocfg, last_n_blocks=0)
        dev_sel = _device_mask(ids, counts, slice(t0, t0 + n), num_blocks)
        qs = to_np(q[:, rows0:rows0 + n * tq])
        sel, _, ratio = orc.block_scores_and_select(
            qs, pooled_k, scale=SCALE, config=orc._replace(sub, score_chunk_tiles=1),
            offset=off + rows0, query_length=n * tq, return_ratio=True)
        decided = np.abs(ratio - cfg.alpha) > BAND
        assert np.array_equal(sel[decided], dev_sel[decided]), (t0, n)
        assert dev_sel.sum() > 0
        if sparse and t0 > 0 and t0 + n < nt - cfg.last_n_blocks:
            assert dev_sel.mean() < 0.5  # the correction phase is exercised
        ref = orc.fpv2_attention_blockwise(
            qs, kn, vn, scale=SCALE, selected=dev_sel, pooled_k=pooled_k, pooled_v=pooled_v,
            config=sub, offset=off + rows0, row_block=tq)
        err = attention_errors(to_np(out[0, :, rows0:rows0 + n * tq]), ref)
        assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, (t0, n, err)


def _check_every_list(q, keep, seq):
    """Every tile x KV head of a call whose queries start at key 0: lists
    outside the 1e-4 band against the oracle's selection, and the full padded
    lists (selected ascending, then the rest), counts and pruned lists equal
    to the oracle's compaction of the device's mask."""
    cfg = keep["config"]
    ids, counts, pids, pcounts = keep["lists"]
    nb, nt = ids.shape[-1], ids.shape[1]
    dev_sel = _device_mask(ids, counts, slice(0, nt), nb)
    sel, ratio = oracle_select_parallel(to_np(q), to_np(keep["pooled_k"]), scale=SCALE,
                                        config=_oracle_config(cfg), offset=0, query_length=seq)
    decided = np.abs(ratio - cfg.alpha) > BAND
    assert np.array_equal(sel[decided], dev_sel[decided])
    o_ids, o_counts, o_pids, o_pcounts = orc.compact_block_indices(
        dev_sel, config=_oracle_config(cfg), offset=0, query_length=seq, key_length=seq)
    assert np.array_equal(to_np(ids), o_ids) and np.array_equal(to_np(counts), o_counts)
    assert np.array_equal(to_np(pcounts), o_pcounts)
    head = np.arange(nb)[None, None, :] < o_pcounts[..., None]  # the defined entries
    assert np.array_equal(np.where(head, to_np(pids), -1), np.where(head, o_pids, -1))
    return int(decided.sum())


def _samples(nt, n_end):
    """Tile groups from the start, the middle and the end of the call."""
    return ((0, 2), (nt // 2, 2), (nt - n_end, n_end))


@pytest.mark.parametrize(("seq", "heavy", "planted", "alpha", "n_end"), [
    (32768, 0.06, 3.0, 0.1, 6),
    # alpha in {0.05, 0.1, 0.2} at 131072, 3% heavy blocks
    (131072, 0.03, 3.0, 0.05, 3),
    (131072, 0.03, 3.0, 0.1, 3),
    (131072, 0.03, 3.0, 0.2, 3),
    # the bench's contrast variant: planted x 3*sqrt(D) prunes most blocks, so
    # the correction phase carries hundreds of pooled rows per tile
    (131072, 0.03, 3.0 * 128 ** 0.5, 0.1, 4),
])
def test_sampled_tiles_match_oracle_at_full_size(cuda, seq, heavy, planted, alpha, n_end):
    q, k, v = baseline_qkv(seq, planted=planted, heavy_fraction=heavy, seed=0, device=cuda)
    config = FPV2Config(alpha=alpha, sink_tokens=128)
    keep = {}
    out = _fpv2_sdpa(q[None], k[None], v[None], scale=SCALE, config=config, keep=keep)
    torch.cuda.synchronize()
    kn, vn = to_np(k), to_np(v)
    # pooling of the whole layer, bit-exact
    assert np.array_equal(to_np(keep["pooled_k"]), orc.pool_blocks(kn, 128, out_dtype="bf16"))
    assert np.array_equal(to_np(keep["pooled_v"]), orc.pool_blocks(vn, 128, out_dtype="bf16"))
    nt = seq // keep["config"].tile_q
    _check_tiles(q, kn, vn, out, keep, seq, _samples(nt, n_end), sparse=planted > 3.0)
    assert _check_every_list(q, keep, seq) > 0.99 * 8 * nt * (nt * 32 // 128 + 1) / 2


def test_every_tile_list_at_32k_matches_oracle(cuda):
    """All 1024 tiles x 8 KV heads of the 32k layer (config 2): block lists
    bit-exact against the oracle's chunked scoring, outside the 1e-4 band,
    and the full padded lists (selected ascending, then the rest) and pruned
    lists equal to the oracle's compaction of the device's mask."""
    seq = 32768
    q, k, v = baseline_qkv(seq, planted=3.0, heavy_fraction=0.06, seed=0, device=cuda)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    keep = {}
    _fpv2_sdpa(q[None], k[None], v[None], scale=SCALE, config=config, keep=keep)
    torch.cuda.synchronize()
    cfg = keep["config"]
    ids, counts, pids, pcounts = keep["lists"]
    nb = ids.shape[-1]
    nt = ids.shape[1]
    dev_sel = _device_mask(ids, counts, slice(0, nt), nb)
    sel, _, ratio = orc.block_scores_and_select(
        to_np(q), to_np(keep["pooled_k"]), scale=SCALE,
        config=orc._replace(_oracle_config(cfg), score_chunk_tiles=128), offset=0,
        query_length=seq, return_ratio=True)
    decided = np.abs(ratio - cfg.alpha) > BAND
    assert np.array_equal(sel[decided], dev_sel[decided])
    o_ids, o_counts, o_pids, o_pcounts = orc.compact_block_indices(
        dev_sel, config=_oracle_config(cfg), offset=0, query_length=seq, key_length=seq)
    assert np.array_equal(to_np(ids), o_ids) and np.array_equal(to_np(counts), o_counts)
    assert np.array_equal(to_np(pcounts), o_pcounts)
    for h in range(ids.shape[0]):  # pruned lists: the first count entries are defined
        for t in range(nt):
            c = o_pcounts[h, t]
            assert np.array_equal(to_np(pids[h, t, :c]), o_pids[h, t, :c])


def test_32k_without_correction(cuda):
    """BASELINE config 2's no-corr ablation: ``mean_correction=False`` at 32k
    against the oracle (start, middle and end tiles), and bit-identical to the
    corrected layer on every tile that prunes no block (the correction phase
    adds nothing there)."""
    seq = 32768
    q, k, v = baseline_qkv(seq, planted=3.0, heavy_fraction=0.06, seed=0, device=cuda)
    keep_nc, keep_c = {}, {}
    out_nc = _fpv2_sdpa(q[None], k[None], v[None], scale=SCALE,
                        config=FPV2Config(alpha=0.1, sink_tokens=128, mean_correction=False),
                        keep=keep_nc)
    out_c = _fpv2_sdpa(q[None], k[None], v[None], scale=SCALE,
                       config=FPV2Config(alpha=0.1, sink_tokens=128), keep=keep_c)
    torch.cuda.synchronize()
    for a, b in zip(keep_nc["lists"][:2], keep_c["lists"][:2]):
        assert torch.equal(a, b)  # selection does not depend on the correction flag
    kn, vn = to_np(k), to_np(v)
    nt = seq // keep_nc["config"].tile_q
    _check_tiles(q, kn, vn, out_nc, keep_nc, seq, _samples(nt, 6))
    tq = keep_c["config"].tile_q
    unpruned = (keep_c["lists"][3] == 0).all(dim=0)  # [Nt]: no head prunes a block
    assert bool(unpruned.any())
    rows = unpruned.repeat_interleave(tq)[:seq]
    assert torch.equal(out_nc[0][:, rows], out_c[0][:, rows])


def test_32k_layer_is_bitwise_deterministic(cuda):
    """Two runs of the 32k hook give identical pooled blocks, block lists,
    counts and outputs, bit for bit (no atomics or order-dependent sums)."""
    seq = 32768
    q, k, v = baseline_qkv(seq, planted=3.0 * 128 ** 0.5, heavy_fraction=0.06, seed=2,
                           device=cuda)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    runs = []
    for _ in range(2):
        keep = {}
        out = _fpv2_sdpa(q[None], k[None], v[None], scale=SCALE, config=config, keep=keep)
        runs.append((out, keep))
    torch.cuda.synchronize()
    (o1, k1), (o2, k2) = runs
    assert torch.equal(o1, o2)
    assert torch.equal(k1["pooled_k"], k2["pooled_k"]) and torch.equal(k1["pooled_v"], k2["pooled_v"])
    for a, b in zip(k1["lists"], k2["lists"]):
        assert torch.equal(a, b)
    assert float((k1["lists"][3] > 0).float().mean()) > 0.5  # most tiles run the correction


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
    out = _fpv2_sdpa(q[None], k[None], v[None], scale=SCALE, config=config, keep=keep)
    torch.cuda.synchronize()
    cfg = keep["config"]
    ids, counts, _, _ = keep["lists"]
    num_blocks = ids.shape[-1]
    assert num_blocks == _lib.MAX_BLOCKS
    dev_sel = _device_mask(ids, counts, slice(0, lq // cfg.tile_q), num_blocks)

    ocfg = _oracle_config(cfg)
    pooled_k, pooled_v = to_np(keep["pooled_k"]), to_np(keep["pooled_v"])
    qs = to_np(q)
    sel, _, ratio = orc.block_scores_and_select(
        qs, pooled_k, scale=SCALE, config=orc._replace(ocfg, score_chunk_tiles=1),
        offset=seq - lq, query_length=lq, return_ratio=True)
    decided = np.abs(ratio - cfg.alpha) > BAND
    assert np.array_equal(sel[decided], dev_sel[decided])
    assert dev_sel[:, :-2].mean() < 0.5  # sparse outside the dense tail

    ref = orc.fpv2_attention_blockwise(
        qs, to_np(k), to_np(v), scale=SCALE, selected=dev_sel, pooled_k=pooled_k,
        pooled_v=pooled_v, config=ocfg, offset=seq - lq, row_block=cfg.tile_q)
    err = attention_errors(to_np(out[0]), ref)
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err
