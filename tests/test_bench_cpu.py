"""bench.py's contract and its FLOP accounting, on the CPU.

The dense-equivalent FLOP counts are pinned by the figures computed
independently from the shapes (4*D*Hq*sum of visible keys; 5.498e11,
8.796e12 and 1.407e14 at 8k, 32k and 128k for Hq 32, D 128), and the
retained-FLOP count by two closed forms: every visible block selected gives
exactly the dense count, and each pruned block with correction adds one
pooled entry per valid row.
"""

from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused(bench, capsys, monkeypatch):
    assert bench.main(["--gpus", "2"]) == 2
    assert "single MI355X" in capsys.readouterr().err
    monkeypatch.setenv("WORLD_SIZE", "2")
    assert bench.main([]) == 2


@pytest.mark.parametrize(("seq", "want"), [(8192, 5.498e11), (32768, 8.796e12), (131072, 1.407e14)])
def test_dense_flops_match_the_shape_figures(bench, seq, want):
    got = bench.dense_flops(seq)
    assert got == 4 * 128 * 32 * seq * (seq + 1) // 2
    assert abs(got - want) / want < 5e-4
    assert bench.dense_flops(seq, query_heads=4) * 8 == got  # one KV head's share


def _keep(selected, *, tile_q, block_k, seq, corr):
    config = FPV2Config(block_k=block_k, tile_q=tile_q, mean_correction=corr)
    ocfg = orc.OracleConfig(**{f: getattr(config, f) for f in orc.OracleConfig.__dataclass_fields__})
    lists = orc.compact_block_indices(selected, config=ocfg, offset=0, query_length=seq,
                                      key_length=seq)
    return {"lists": tuple(torch.from_numpy(x) for x in lists), "config": config, "offset": 0}


def _visible(nt, nb, tile_q, block_k):
    t = np.arange(nt)[:, None]
    b = np.arange(nb)[None, :]
    return b * block_k <= (t + 1) * tile_q - 1  # the block starts at or before the tile's last row


def test_all_visible_blocks_selected_gives_the_dense_count(bench):
    seq, tq, bk = 1024, 32, 128  # the hook's tile for G = 4
    nt, nb = seq // tq, seq // bk
    selected = np.broadcast_to(_visible(nt, nb, tq, bk), (8, nt, nb)).copy()
    got, frac = bench.retained_flops(_keep(selected, tile_q=tq, block_k=bk, seq=seq, corr=True),
                                     seq, torch)
    assert got == bench.dense_flops(seq)
    assert frac == selected.mean()


def test_each_pruned_block_adds_one_pooled_entry_per_row(bench):
    seq, tq, bk = 1024, 32, 128
    nt, nb = seq // tq, seq // bk
    vis = _visible(nt, nb, tq, bk)
    selected = np.broadcast_to(vis, (8, nt, nb)).copy()
    selected[:, -1, 0] = False  # the last tile drops block 0, wholly before the tile
    dense = bench.dense_flops(seq)
    exact_lost = 4 * 128 * 4 * 8 * tq * bk  # 4*D*G per (row, key): 32 rows x 128 keys, 8 heads
    with_corr, _ = bench.retained_flops(_keep(selected, tile_q=tq, block_k=bk, seq=seq, corr=True),
                                        seq, torch)
    without, _ = bench.retained_flops(_keep(selected, tile_q=tq, block_k=bk, seq=seq, corr=False),
                                      seq, torch)
    assert without == dense - exact_lost
    assert with_corr == without + 4 * 128 * 4 * 8 * tq  # one pooled entry per row, 8 heads
