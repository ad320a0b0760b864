"""Pins the oracle's hook-level helpers with the reference's KATs
(``tests/test_patch.py:27-41,180-201``)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fpv2_oracle as orc
from fpv2.synthetic import structured_qkv

Cfg = orc.OracleConfig


def test_default_tile_uses_128_packed_gqa_rows():
    eff = orc.effective_config(Cfg(), query_heads=32, kv_heads=8)
    assert eff.tile_q == 32
    custom = Cfg(tile_q=64)
    assert orc.effective_config(custom, query_heads=32, kv_heads=8) is custom
    assert orc.effective_config(Cfg(), query_heads=6, kv_heads=2) is None  # 3 does not divide 128


def test_dense_tail_is_applied_only_at_known_request_end():
    config = Cfg(last_n_blocks=2)
    assert orc.request_config(config, 2048, 8192).last_n_blocks == 0
    assert orc.request_config(config, 8192, 8192) is config
    assert orc.request_config(config, 8192, None).last_n_blocks == 0


def test_sparsity_accounting_matches_reference_fractions():
    # tests/test_patch.py:180-201: 256 keys, 4 q heads / 2 kv heads -> tile 32;
    # alpha huge, no sink/window: only the diagonal block per tile survives.
    cfg = orc.effective_config(Cfg(alpha=1e9, sink_tokens=0, window_tokens=0, last_n_blocks=0),
                               4, 2)
    q, k, _ = structured_qkv(length=256, query_heads=4, kv_heads=2, head_dim=64, seed=7)
    sel, _ = orc.block_scores_and_select(q.numpy(), orc.pool_blocks(k.numpy(), 128),
                                         scale=0.125, config=cfg)
    visible = orc.causal_block_count(2, 256, 0, cfg)
    assert 1 - sel.sum() / visible == pytest.approx(1 / 3)
    # a second, dense-gated 128-token call adds 4 visible and 4 selected blocks
    dense = orc.causal_block_count(2, 128, 0, cfg)
    assert 1 - (sel.sum() + dense) / (visible + dense) == pytest.approx(1 / 4)


def test_hook_plan_padding():
    cfg, offset, lq_pad, lk_pad = orc.hook_plan(4, 2, 130, 130, Cfg())
    assert (cfg.tile_q, offset, lq_pad, lk_pad) == (64, 0, 192, 256)
    cfg, offset, lq_pad, lk_pad = orc.hook_plan(4, 2, 128, 190, Cfg())
    assert (offset, lq_pad, lk_pad) == (62, 128, 256)


def test_alpha_zero_hook_oracle_equals_exact_attention():
    # tests/test_patch.py:44-73 with the oracle as the hook
    q, k, v = structured_qkv(length=190, query_heads=4, kv_heads=2, head_dim=64, seed=3)
    q = q[:, 62:]
    cfg = Cfg(alpha=0, sink_tokens=0, window_tokens=0)
    out = orc.fpv2_sdpa_oracle(q.numpy(), k.numpy(), v.numpy(), scale=0.125, config=cfg,
                               dtype="f32")
    exact = orc.exact_causal_attention(q.numpy(), k.numpy(), v.numpy(), 0.125, offset=62)
    assert np.abs(out - exact).max() < 1e-5
