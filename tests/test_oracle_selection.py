"""Pins the CPU oracle's pooling and selection (no GPU).

Known-answer tests are the reference's own (``tests/test_selection.py``);
the remaining checks use closed forms, a brute-force loop formulation and
invariants chosen so that a dropped term, wrong comparison or index slip in
the oracle fails at least one of them.
"""

from __future__ import annotations

import math
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import fpv2_oracle as orc
from fpv2.synthetic import structured_qkv

Cfg = orc.OracleConfig


def _np(x):
    return x.float().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)


# --------------------------------------------------------------------------
# rounding helpers
# --------------------------------------------------------------------------

def _bf16_brute(x: float) -> float:
    """Nearest bfloat16 by enumerating the two float32-truncation neighbours."""
    if x == 0.0 or not math.isfinite(x):
        return x
    f = np.float32(x)
    bits = int(np.array([f], np.float32).view(np.uint32)[0])
    lo = bits & 0xFFFF0000
    cands = []
    for c in (lo - 0x10000, lo, lo + 0x10000, lo + 0x20000):
        if 0 <= c <= 0xFFFFFFFF:
            val = float(np.array([c], np.uint32).view(np.float32)[0])
            if math.isfinite(val):
                cands.append((abs(val - x), (c >> 16) & 1, val))
    cands.sort(key=lambda t: (t[0], t[1]))
    return cands[0][2]


def test_round_f64_to_bf16_matches_brute_force():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(2000) * 10.0 ** rng.integers(-6, 6, 2000),
        # exact halfway cases between bf16 neighbours, both parities
        (np.arange(1, 400) * 2 + 1) / 512.0 + 1.0,
        (np.arange(1, 400) * 2 + 1) / 512.0 * 3.0,
    ])
    got = orc.round_f64(xs, "bf16")
    want = np.array([_bf16_brute(float(x)) for x in xs], np.float32)
    assert np.array_equal(got, want)


def test_round_f64_odd_then_f16_is_single_rounding():
    rng = np.random.default_rng(1)
    xs = rng.standard_normal(3000) * 10.0 ** rng.integers(-3, 3, 3000)
    got = orc.round_f64(xs, "f16")
    # float16 has 11 significant bits: exact reference via Python's round on scaled ints
    for x, g in zip(xs[:300], got[:300]):
        e = math.frexp(x)[1]
        scale = 2.0 ** (11 - e)
        want = round(x * scale) / scale  # Python round() is ties-to-even
        assert np.float32(want) == g or abs(x) < 2 ** -14


# --------------------------------------------------------------------------
# pool_blocks  (selection.py:68-80)
# --------------------------------------------------------------------------

def test_pool_blocks_closed_form_on_arange():
    # reference KAT shape (tests/test_selection.py:12-16): x[n, r, d] = 16n + 2r + d
    x = np.arange(32, dtype=np.float32).reshape(2, 8, 2)
    pooled = orc.pool_blocks(x, 4, out_dtype="f32")
    n, b, d = np.meshgrid(np.arange(2), np.arange(2), np.arange(2), indexing="ij")
    assert np.array_equal(pooled, (16 * n + 8 * b + 3 + d).astype(np.float32))


def test_pool_blocks_rejects_unaligned_length():
    with pytest.raises(ValueError, match="divisible"):
        orc.pool_blocks(np.zeros((2, 7, 4)), 4)


def test_pool_blocks_zero_padding_and_bf16_rounding():
    rng = np.random.default_rng(2)
    x = rng.integers(-300, 300, size=(3, 256, 8)).astype(np.float64)
    pooled = orc.pool_blocks(x, 128, valid_rows=200, out_dtype="bf16")
    exact0 = x[:, :128].sum(axis=1) / 128
    exact1 = x[:, 128:200].sum(axis=1) / 128  # rows >= 200 count as zeros
    assert np.array_equal(pooled[:, 0], orc.round_f64(exact0, "bf16"))
    assert np.array_equal(pooled[:, 1], orc.round_f64(exact1, "bf16"))


# --------------------------------------------------------------------------
# block_scores_and_select  (selection.py:109-201)
# --------------------------------------------------------------------------

def test_alpha_zero_selects_exactly_visible_blocks():
    # tests/test_selection.py:19-32
    config = Cfg(block_k=32, tile_q=32, alpha=0, sink_tokens=0, window_tokens=0)
    q, k, _ = structured_qkv(length=256, query_heads=8, kv_heads=2, block_size=32)
    selected, _ = orc.block_scores_and_select(
        _np(q), orc.pool_blocks(_np(k), 32), scale=q.shape[-1] ** -0.5, config=config)
    expected = np.arange(8)[None, None, :] <= np.arange(8)[None, :, None]
    assert np.array_equal(selected, np.broadcast_to(expected, selected.shape))
    assert orc.density(selected, config=config) == 1.0


def test_partially_visible_block_does_not_set_tile_energy_scale():
    # tests/test_selection.py:40-57
    config = Cfg(block_k=4, tile_q=2, alpha=0.5, sink_tokens=0, window_tokens=0,
                 last_n_blocks=0)
    q = np.ones((1, 2, 1))
    pooled_k = np.array([[[0.0], [10.0]]])
    selected, _ = orc.block_scores_and_select(q, pooled_k, scale=1.0, config=config, offset=4)
    assert selected.tolist() == [[[True, True]]]


def test_last_n_blocks_are_fully_dense_for_complete_request():
    # tests/test_selection.py:60-81
    config = Cfg(block_k=4, tile_q=4, alpha=1e9, sink_tokens=0, window_tokens=0,
                 last_n_blocks=2)
    selected, _ = orc.block_scores_and_select(np.ones((1, 16, 1)), np.ones((1, 4, 1)),
                                              scale=1.0, config=config)
    assert selected.tolist() == [[
        [True, False, False, False],
        [False, True, False, False],
        [True, True, True, False],
        [True, True, True, True],
    ]]


def test_defaults():
    # tests/test_selection.py:84-87
    config = Cfg()
    assert config.window_tokens == 384 and config.last_n_blocks == 2


def test_chunked_scoring_matches_unchunked_selection():
    # tests/test_selection.py:90-112
    config = Cfg(block_k=16, tile_q=16, alpha=0.35, sink_tokens=16, window_tokens=32)
    q, k, _ = structured_qkv(length=160, query_heads=8, kv_heads=2, block_size=16, seed=7)
    pk = orc.pool_blocks(_np(k), 16)
    expected, scores = orc.block_scores_and_select(_np(q), pk, scale=64 ** -0.5, config=config)
    actual, chunked = orc.block_scores_and_select(
        _np(q), pk, scale=64 ** -0.5, config=replace(config, score_chunk_tiles=3))
    assert scores is not None and chunked is None
    assert np.array_equal(actual, expected)


def test_chunked_scoring_preserves_offset_and_padded_query_semantics():
    # tests/test_selection.py:114-144
    config = Cfg(block_k=16, tile_q=16, alpha=0.4, sink_tokens=16, window_tokens=16)
    q, k, _ = structured_qkv(length=160, query_heads=4, kv_heads=2, block_size=16, seed=11)
    offset, qlen = 37, 55
    padded = np.zeros((4, 64, 64), np.float32)
    padded[:, :qlen] = _np(q)[:, offset:offset + qlen]
    pk = orc.pool_blocks(_np(k), 16)
    expected, _ = orc.block_scores_and_select(padded, pk, scale=64 ** -0.5, config=config,
                                              offset=offset, query_length=qlen)
    actual, scores = orc.block_scores_and_select(
        padded, pk, scale=64 ** -0.5, config=replace(config, score_chunk_tiles=2),
        offset=offset, query_length=qlen)
    assert scores is None
    assert np.array_equal(actual, expected)


def _brute_select(q, pk, scale, cfg, offset, qlen):
    """Loop formulation of the selection rule, written independently."""
    hq, lq_pad, d = q.shape
    hkv, nb, _ = pk.shape
    g = hq // hkv
    nt = lq_pad // cfg.tile_q
    out = np.zeros((hkv, nt, nb), bool)
    for h in range(hkv):
        for t in range(nt):
            first = offset + t * cfg.tile_q
            last = min(first + cfg.tile_q, offset + qlen) - 1
            entries = {}
            for b in range(nb):
                if (b + 1) * cfg.block_k > last + 1:
                    continue  # only fully visible blocks carry energy
                vals = []
                for gg in range(g):
                    for r in range(t * cfg.tile_q, (t + 1) * cfg.tile_q):
                        if r >= qlen or b * cfg.block_k > offset + r:
                            continue
                        vals.append(scale * float(np.dot(q[h * g + gg, r], pk[h, b])))
                entries[b] = vals
            allv = [x for vs in entries.values() for x in vs]
            m = max(allv) if allv else None
            energy = [sum(math.exp(x - m) for x in entries.get(b, [])) if m is not None else 0.0
                      for b in range(nb)]
            emax = max(energy)
            for b in range(nb):
                start, end = b * cfg.block_k, (b + 1) * cfg.block_k
                forced = (start < cfg.sink_tokens or end > first - cfg.window_tokens
                          or t >= max(nt - cfg.last_n_blocks, 0))
                out[h, t, b] = (energy[b] >= cfg.alpha * emax or forced) and start <= last
    return out


@pytest.mark.parametrize("offset,qlen,alpha", [(0, 64, 0.3), (40, 45, 0.5), (16, 17, 0.05)])
def test_selection_matches_brute_force_loops(offset, qlen, alpha):
    rng = np.random.default_rng(offset + qlen)
    cfg = Cfg(block_k=8, tile_q=8, alpha=alpha, sink_tokens=8, window_tokens=8, last_n_blocks=1)
    lq_pad = -(-qlen // 8) * 8
    q = rng.standard_normal((4, lq_pad, 16))
    q[:, qlen:] = 0.0
    pk = rng.standard_normal((2, (offset + lq_pad + 7) // 8 + 1, 16))
    got, _ = orc.block_scores_and_select(q, pk, scale=0.7, config=cfg, offset=offset,
                                         query_length=qlen)
    assert np.array_equal(got, _brute_select(q, pk, 0.7, cfg, offset, qlen))


def test_selection_shrinks_monotonically_with_alpha():
    q, k, _ = structured_qkv(length=512, query_heads=8, kv_heads=2, block_size=32, seed=5)
    pk = orc.pool_blocks(_np(k), 32)
    prev = None
    for alpha in (0.0, 0.05, 0.2, 0.5, 0.9, 1.0):
        cfg = Cfg(block_k=32, tile_q=32, alpha=alpha, sink_tokens=0, window_tokens=0,
                  last_n_blocks=0)
        sel, _ = orc.block_scores_and_select(_np(q), pk, scale=0.125, config=cfg)
        if prev is not None:
            assert not np.any(sel & ~prev)
        prev = sel
    # alpha = 1 keeps the max-energy block (plus the diagonal) only
    assert prev.sum(axis=-1).max() <= 2


def test_energy_ratio_is_one_for_max_block():
    q, k, _ = structured_qkv(length=256, query_heads=4, kv_heads=2, block_size=32, seed=3)
    cfg = Cfg(block_k=32, tile_q=32, alpha=0.1, sink_tokens=0, window_tokens=0)
    _, _, ratio = orc.block_scores_and_select(_np(q), orc.pool_blocks(_np(k), 32),
                                              scale=0.125, config=cfg, return_ratio=True)
    finite = ratio[:, 1:]  # tile 0 has no fully visible block
    assert np.allclose(finite.max(axis=-1), 1.0)


def test_density_counts_visible_pairs():
    cfg = Cfg(block_k=4, tile_q=4)
    sel = np.zeros((2, 4, 4), bool)
    sel[:, np.arange(4), np.arange(4)] = True  # diagonal only
    assert orc.density(sel, config=cfg) == pytest.approx(4 / 10)
