"""Pins the oracle's compaction and attention (no GPU).

Compaction: the reference KAT (``tests/test_kernel.py:66-72``) plus
permutation/order invariants and a loop formulation of the pruned rule.
Attention: alpha=0 with no forced blocks and no correction must equal plain
causal softmax attention computed by a textbook routine (torch SDPA in
float64), the correction must not increase the error on clustered data
(``tests/test_reference.py:29-89``), and an explicit per-row float64
enumeration of the exact and pooled entries pins the correction term.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import fpv2_oracle as orc
from fpv2.synthetic import structured_qkv

Cfg = orc.OracleConfig


def _np(x):
    return x.float().numpy()


def test_compaction_preserves_ascending_selected_indices():
    ids, counts, _, _ = orc.compact_block_indices(np.array([[[True, False, True, False]]]),
                                                  config=Cfg(block_k=16, tile_q=16))
    assert counts.item() == 2
    assert ids[0, 0, :2].tolist() == [0, 2]
    assert ids[0, 0].tolist() == [0, 2, 1, 3]


def test_compaction_rejects_non_boolean_mask():
    with pytest.raises(ValueError, match="boolean"):
        orc.compact_block_indices(np.ones((1, 1, 1), np.int32))


def test_compaction_invariants_and_pruned_rule():
    rng = np.random.default_rng(9)
    cfg = Cfg(block_k=16, tile_q=8)
    sel = rng.random((3, 12, 10)) < 0.4
    offset, key_length = 40, 150
    ids, counts, pids, pcounts = orc.compact_block_indices(
        sel, config=cfg, offset=offset, query_length=90, key_length=key_length)
    for h in range(3):
        for t in range(12):
            row = ids[h, t]
            assert sorted(row.tolist()) == list(range(10))  # permutation
            c = counts[h, t]
            assert c == sel[h, t].sum()
            assert row[:c].tolist() == sorted(np.flatnonzero(sel[h, t]).tolist())
            assert row[c:].tolist() == sorted(np.flatnonzero(~sel[h, t]).tolist())
            first = offset + t * cfg.tile_q
            pruned = [b for b in range(10)
                      if not sel[h, t, b] and min((b + 1) * 16, key_length) <= first]
            assert pcounts[h, t] == len(pruned)
            assert pids[h, t, :len(pruned)].tolist() == pruned


def _textbook_causal(q, k, v, scale, offset=0):
    """torch SDPA on CPU in float64 with an explicit bottom-right mask."""
    q = torch.as_tensor(q, dtype=torch.float64)
    k = torch.as_tensor(k, dtype=torch.float64)
    v = torch.as_tensor(v, dtype=torch.float64)
    g = q.shape[0] // k.shape[0]
    k = k.repeat_interleave(g, dim=0)
    v = v.repeat_interleave(g, dim=0)
    lq, lk = q.shape[1], k.shape[1]
    mask = torch.arange(lk)[None, :] <= (offset + torch.arange(lq))[:, None]
    out = torch.nn.functional.scaled_dot_product_attention(
        q[None], k[None], v[None], attn_mask=mask, scale=scale)
    return out[0].numpy()


def test_dense_selection_matches_exact_causal_attention():
    # tests/test_reference.py:29-51
    cfg = Cfg(block_k=32, tile_q=32, alpha=0, sink_tokens=0, window_tokens=0,
              mean_correction=False)
    q, k, v = (_np(x) for x in structured_qkv(length=256, block_size=32))
    scale = 64 ** -0.5
    actual = orc.fpv2_attention_reference(q, k, v, scale=scale, config=cfg)
    expected = _textbook_causal(q, k, v, scale)
    rel = np.abs(actual - expected).max() / max(np.abs(expected).max(), 1e-8)
    assert rel < 1e-5
    # the oracle's own textbook helper agrees too
    assert np.allclose(orc.exact_causal_attention(q, k, v, scale), expected, atol=1e-12)


def test_dense_selection_matches_exact_attention_with_offset():
    # tests/test_reference.py:71-89
    cfg = Cfg(block_k=128, tile_q=128, alpha=0, sink_tokens=0, window_tokens=0,
              mean_correction=False)
    q, k, v = (_np(x) for x in structured_qkv(length=2048, block_size=128, seed=13))
    offset = 1024
    scale = 64 ** -0.5
    actual = orc.fpv2_attention_reference(q[:, offset:], k, v, scale=scale, config=cfg,
                                          offset=offset)
    expected = _textbook_causal(q[:, offset:], k, v, scale, offset)
    assert np.allclose(actual, expected, rtol=1e-5, atol=1e-6)


def test_mean_correction_improves_sparse_approximation():
    # tests/test_reference.py:54-68
    base = dict(block_k=32, tile_q=32, alpha=0.6, sink_tokens=32, window_tokens=32)
    q, k, v = (_np(x) for x in structured_qkv(length=512, block_size=32, noise=0.01))
    expected = _textbook_causal(q, k, v, 3.0)
    trunc = orc.fpv2_attention_reference(q, k, v, scale=3.0,
                                         config=Cfg(**base, mean_correction=False))
    corr = orc.fpv2_attention_reference(q, k, v, scale=3.0,
                                        config=Cfg(**base, mean_correction=True))
    assert np.abs(corr - expected).max() <= np.abs(trunc - expected).max()


def test_all_selected_makes_correction_a_no_op():
    cfg = Cfg(block_k=32, tile_q=32, alpha=0.0, sink_tokens=0, window_tokens=0)
    q, k, v = (_np(x) for x in structured_qkv(length=256, block_size=32, seed=4))
    a = orc.fpv2_attention_reference(q, k, v, scale=0.125, config=cfg)
    b = orc.fpv2_attention_reference(q, k, v, scale=0.125,
                                     config=Cfg(block_k=32, tile_q=32, alpha=0.0, sink_tokens=0,
                                                window_tokens=0, mean_correction=False))
    assert np.array_equal(a, b)


def _explicit_entries(q, k, v, selected, pk, pv, cfg, scale, offset, row, qh, valid_k):
    """float64 softmax over an explicit list of (logit, value) entries for one row."""
    q, k, v, pk, pv = (np.asarray(x, np.float64) for x in (q, k, v, pk, pv))
    hkv = k.shape[0]
    g = q.shape[0] // hkv
    h = qh // g
    t = row // cfg.tile_q
    first = offset + t * cfg.tile_q
    entries = []
    for b in range(pk.shape[1]):
        if selected[h, t, b]:
            for j in range(b * cfg.block_k, min((b + 1) * cfg.block_k, valid_k)):
                if j <= offset + row:
                    entries.append((scale * float(np.dot(q[qh, row], k[h, j])), v[h, j]))
        elif cfg.mean_correction and min((b + 1) * cfg.block_k, valid_k) <= first:
            entries.append((scale * float(np.dot(q[qh, row], pk[h, b])) + math.log(cfg.block_k),
                            pv[h, b]))
    m = max(x for x, _ in entries)
    w = np.array([math.exp(x - m) for x, _ in entries])
    vals = np.stack([val for _, val in entries]).astype(np.float64)
    return (w[:, None] * vals).sum(0) / w.sum()


@pytest.mark.parametrize("offset,qlen", [(0, 128), (64, 96)])
def test_blockwise_matches_explicit_entry_enumeration(offset, qlen):
    cfg = Cfg(block_k=16, tile_q=16, alpha=0.3, sink_tokens=16, window_tokens=16)
    q, k, v = (_np(x) for x in structured_qkv(length=192, query_heads=4, kv_heads=2,
                                              block_size=16, seed=offset + 1))
    valid_k = offset + qlen
    lq_pad = -(-qlen // 16) * 16
    qs = np.zeros((4, lq_pad, 64), np.float32)
    qs[:, :qlen] = q[:, offset:offset + qlen]
    lk_pad = -(-max(valid_k, offset + lq_pad) // 16) * 16
    kp = np.zeros((2, lk_pad, 64), np.float32)
    vp = np.zeros((2, lk_pad, 64), np.float32)
    kp[:, :valid_k] = k[:, :valid_k]
    vp[:, :valid_k] = v[:, :valid_k]
    pk = orc.pool_blocks(kp, 16)
    pv = orc.pool_blocks(vp, 16)
    sel, _ = orc.block_scores_and_select(qs, pk, scale=0.125, config=cfg, offset=offset,
                                         query_length=qlen)
    out = orc.fpv2_attention_blockwise(qs, kp, vp, scale=0.125, selected=sel, pooled_k=pk,
                                       pooled_v=pv, config=cfg, offset=offset,
                                       query_length=qlen, key_length=valid_k,
                                       dtype=np.float64)
    assert not np.any(out[:, qlen:])  # padded rows stay zero
    rng = np.random.default_rng(0)
    for _ in range(24):
        qh = int(rng.integers(4))
        row = int(rng.integers(qlen))
        want = _explicit_entries(qs, kp, vp, sel, pk, pv, cfg, 0.125, offset, row, qh, valid_k)
        assert np.allclose(out[qh, row], want, rtol=1e-10, atol=1e-12)


def test_blockwise_equals_literal_reference():
    cfg = Cfg(block_k=32, tile_q=32, alpha=0.4, sink_tokens=32, window_tokens=32)
    q, k, v = (_np(x) for x in structured_qkv(length=384, query_heads=4, kv_heads=2,
                                              block_size=32, seed=21))
    lit = orc.fpv2_attention_reference(q, k, v, scale=0.125, config=cfg, dtype=np.float64)
    pk = orc.pool_blocks(k, 32)
    pv = orc.pool_blocks(v, 32)
    sel, _ = orc.block_scores_and_select(q, pk, scale=0.125, config=cfg)
    blk = orc.fpv2_attention_blockwise(q, k, v, scale=0.125, selected=sel, pooled_k=pk,
                                       pooled_v=pv, config=cfg, dtype=np.float64, row_block=64)
    assert np.allclose(lit, blk, rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize(("offset", "qlen", "workers"), [(0, 1024, 3), (200, 937, 4), (0, 64, 2)])
def test_tile_range_evaluation_equals_one_call(offset, qlen, workers):
    """Selection and attention of a whole call, evaluated as calls of tile
    ranges on several threads, equal the one-call oracle: the selection bit
    for bit (the dense tail, last 2 tiles, stays with the call's end; offsets
    and the partial last tile carry over), the attention up to float32
    summation order (rows are grouped into different BLAS products)."""
    rng = np.random.default_rng(offset + qlen)
    hq, hkv, d, tq, bk = 4, 2, 32, 32, 64
    lq_pad = -(-qlen // tq) * tq
    nb = -(-(offset + lq_pad) // bk)
    q = rng.standard_normal((hq, lq_pad, d)).astype(np.float32)
    q[:, qlen:] = 0
    k = rng.standard_normal((hkv, nb * bk, d)).astype(np.float32)
    v = rng.standard_normal((hkv, nb * bk, d)).astype(np.float32)
    k[:, :bk] += 2.0
    lk = offset + qlen
    k[:, lk:] = 0
    v[:, lk:] = 0
    cfg = orc.OracleConfig(block_k=bk, tile_q=tq, alpha=0.2, sink_tokens=bk, window_tokens=bk)
    pk = orc.pool_blocks(k, bk, out_dtype="bf16")
    pv = orc.pool_blocks(v, bk, out_dtype="bf16")
    one, _, ratio = orc.block_scores_and_select(
        q, pk, scale=d ** -0.5, config=orc._replace(cfg, score_chunk_tiles=5), offset=offset,
        query_length=qlen, return_ratio=True)
    sel, ratio2 = orc.select_tile_ranges(q, pk, scale=d ** -0.5, config=cfg, offset=offset,
                                         query_length=qlen, workers=workers)
    assert np.array_equal(sel, one) and np.array_equal(ratio, ratio2)
    if nb > 4:
        assert sel[:, -1].sum() > sel[:, 0].sum()  # the dense tail is present
    want = orc.fpv2_attention_blockwise(q, k, v, scale=d ** -0.5, selected=one, pooled_k=pk,
                                        pooled_v=pv, config=cfg, offset=offset,
                                        query_length=qlen, key_length=lk)
    got = orc.attention_tile_ranges(q, k, v, scale=d ** -0.5, selected=one, pooled_k=pk,
                                    pooled_v=pv, config=cfg, offset=offset, query_length=qlen,
                                    key_length=lk, workers=workers)
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    assert not np.array_equal(got[:, :qlen], 0)
