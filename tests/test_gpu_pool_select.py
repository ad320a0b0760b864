"""GPU parity: pooling, scoring/selection and list compaction vs the oracle.

Bars (integer/bool work bit-exact, floating point within a stated tolerance):
  * pooled blocks: bit-exact against the oracle's correctly rounded mean;
  * selection masks: bit-exact on every (head, tile, block) whose oracle
    energy/max ratio lies farther than 1e-4 from alpha (the band in which a
    float32 and a float64 evaluation may legitimately disagree);
  * block lists and counts: bit-exact (ids compared in full, including the
    unselected tail, which a stable argsort fixes);
  * raw scores: |gpu - oracle| <= 1e-5 * max(1, |oracle|).
"""

from __future__ import annotations

import ctypes
from dataclasses import replace

import numpy as np
import pytest
import torch

from conftest import to_np
from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config, pool_blocks
from fpv2 import _lib
from fpv2.kernel import compact_block_indices
from fpv2.selection import block_scores_and_select, density
from fpv2.synthetic import baseline_qkv, structured_qkv

pytestmark = pytest.mark.gpu

BAND = 1e-4
_DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _cfg(c: FPV2Config) -> orc.OracleConfig:
    return orc.OracleConfig(**{f: getattr(c, f) for f in orc.OracleConfig.__dataclass_fields__})


# ---------------------------------------------------------------- pooling ----

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 96, 128, 256, 40])
def test_pool_blocks_bit_exact(cuda, dtype, head_dim):
    gen = torch.Generator().manual_seed(head_dim)
    x = (torch.randn((3, 512, head_dim), generator=gen) * 2.0).to(dtype)
    got = pool_blocks(x.to(cuda), 128)
    want = orc.pool_blocks(to_np(x), 128, out_dtype=_DT[dtype])
    assert got.dtype == dtype and got.shape == (3, 4, head_dim)
    assert np.array_equal(to_np(got), want)


@pytest.mark.parametrize(("head_dim", "block"), [(8, 128), (16, 48), (32, 16), (512, 128), (520, 64), (256, 200)])
def test_pool_lane_layouts(cuda, head_dim, block):
    """Head dims and block sizes across the 16-byte kernel's lane layouts
    (R = 8 row groups per wave with 1, 2 or 4 of 8 padded columns in use;
    R = 1 at D = 512), the generic kernel past D = 512, and blocks that are
    not a multiple of the row-group count: whole blocks (``pool_blocks``) and
    a partial last block (``fpv2_pool_kv``, missing rows counted as zeros)."""
    gen = torch.Generator().manual_seed(head_dim + block)
    x = (torch.randn((2, 3 * block, head_dim), generator=gen) * 3.0).bfloat16()
    got = pool_blocks(x.to(cuda), block)
    assert got.shape == (2, 3, head_dim)
    assert np.array_equal(to_np(got), orc.pool_blocks(to_np(x), block, out_dtype="bf16"))
    valid = 3 * block - 5
    kd = x.to(cuda)
    vd = (x * -0.5).to(cuda)
    pk = torch.empty((2, 3, head_dim), dtype=torch.bfloat16, device=cuda)
    pv = torch.empty_like(pk)
    lib = _lib.load()
    status = lib.fpv2_pool_kv(kd.data_ptr(), vd.data_ptr(), pk.data_ptr(), pv.data_ptr(),
                              _lib.BF16, 2, valid, 3, head_dim, block, kd.stride(0), kd.stride(1),
                              pk.stride(0), _lib.stream_ptr(cuda))
    _lib.check(status, "pool_kv")
    for src, pooled in ((kd, pk), (vd, pv)):
        pad = to_np(src).copy()
        pad[:, valid:] = 0.0
        assert np.array_equal(to_np(pooled), orc.pool_blocks(pad, block, out_dtype="bf16"))


def test_pool_blocks_leading_dims_and_strided_input(cuda):
    x = torch.randn((2, 3, 384, 64), generator=torch.Generator().manual_seed(1)).bfloat16()
    xs = x.to(cuda).transpose(1, 2).contiguous().transpose(1, 2)  # head-strided view
    got = pool_blocks(xs, 128)
    want = orc.pool_blocks(to_np(x), 128, out_dtype="bf16")
    assert np.array_equal(to_np(got), want)


def test_pool_kv_partial_last_block_counts_zeros(cuda):
    lib = _lib.load()
    gen = torch.Generator().manual_seed(5)
    k = torch.randn((4, 300, 128), generator=gen).bfloat16()
    v = torch.randn((4, 300, 128), generator=gen).bfloat16()
    kd, vd = k.to(cuda), v.to(cuda)
    pk = torch.empty((4, 3, 128), dtype=torch.bfloat16, device=cuda)
    pv = torch.empty_like(pk)
    status = lib.fpv2_pool_kv(kd.data_ptr(), vd.data_ptr(), pk.data_ptr(), pv.data_ptr(),
                              _lib.BF16, 4, 300, 3, 128, 128, kd.stride(0), kd.stride(1),
                              pk.stride(0), _lib.stream_ptr(cuda))
    _lib.check(status, "pool_kv")
    pad = np.zeros((4, 384, 128), np.float32)
    pad[:, :300] = to_np(k)
    assert np.array_equal(to_np(pk), orc.pool_blocks(pad, 128, out_dtype="bf16"))
    pad[:, :300] = to_np(v)
    assert np.array_equal(to_np(pv), orc.pool_blocks(pad, 128, out_dtype="bf16"))


# ------------------------------------------------------------- selection ----

def test_alpha_zero_selects_exactly_visible_blocks(cuda):
    # tests/test_selection.py:19-32
    config = FPV2Config(block_k=32, tile_q=32, alpha=0, sink_tokens=0, window_tokens=0)
    q, k, _ = structured_qkv(length=256, query_heads=8, kv_heads=2, block_size=32,
                             dtype=torch.bfloat16, device=cuda)
    selected, _ = block_scores_and_select(q, pool_blocks(k, 32), scale=64 ** -0.5, config=config)
    expected = torch.arange(8)[None, None, :] <= torch.arange(8)[None, :, None]
    assert torch.equal(selected.cpu(), expected.expand(selected.shape))
    assert density(selected, config=config).item() == 1.0


def test_partially_visible_block_does_not_set_tile_energy_scale(cuda):
    # tests/test_selection.py:40-57 (head_dim 1: generic float path)
    config = FPV2Config(block_k=4, tile_q=2, alpha=0.5, sink_tokens=0, window_tokens=0,
                        last_n_blocks=0)
    q = torch.ones((1, 2, 1), device=cuda)
    pooled_k = torch.tensor([[[0.0], [10.0]]], device=cuda)
    selected, _ = block_scores_and_select(q, pooled_k, scale=1.0, config=config, offset=4)
    assert selected.cpu().tolist() == [[[True, True]]]


def test_last_n_blocks_are_fully_dense_for_complete_request(cuda):
    # tests/test_selection.py:60-81
    config = FPV2Config(block_k=4, tile_q=4, alpha=1e9, sink_tokens=0, window_tokens=0,
                        last_n_blocks=2)
    selected, _ = block_scores_and_select(torch.ones((1, 16, 1), device=cuda),
                                          torch.ones((1, 4, 1), device=cuda), scale=1.0,
                                          config=config)
    assert selected.cpu().tolist() == [[
        [True, False, False, False],
        [False, True, False, False],
        [True, True, True, False],
        [True, True, True, True],
    ]]


def test_chunked_scoring_matches_unchunked_selection(cuda):
    # tests/test_selection.py:90-112
    config = FPV2Config(block_k=16, tile_q=16, alpha=0.35, sink_tokens=16, window_tokens=32)
    q, k, _ = structured_qkv(length=160, query_heads=8, kv_heads=2, block_size=16, seed=7,
                             dtype=torch.bfloat16, device=cuda)
    pk = pool_blocks(k, 16)
    expected, scores = block_scores_and_select(q, pk, scale=64 ** -0.5, config=config)
    actual, chunked = block_scores_and_select(q, pk, scale=64 ** -0.5,
                                              config=replace(config, score_chunk_tiles=3))
    assert scores is not None and chunked is None
    assert torch.equal(actual, expected)


def _assert_selection_parity(sel_gpu, sel_orc, ratio, alpha):
    near = np.abs(ratio - alpha) <= BAND
    mismatch = (sel_gpu != sel_orc) & ~near
    assert not mismatch.any(), f"{int(mismatch.sum())} block decisions differ outside the band"
    return near


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 96, 128, 256])
@pytest.mark.parametrize("offset,qlen", [(0, 512), (77, 300)])
def test_selection_and_scores_match_oracle(cuda, dtype, head_dim, offset, qlen):
    config = FPV2Config(block_k=32, tile_q=16, alpha=0.2, sink_tokens=32, window_tokens=64,
                        last_n_blocks=1)
    q, k, _ = structured_qkv(length=offset + qlen + 40, query_heads=8, kv_heads=2,
                             head_dim=head_dim, block_size=32, seed=head_dim + offset,
                             dtype=dtype)
    lq_pad = -(-qlen // 16) * 16
    qp = torch.zeros((8, lq_pad, head_dim), dtype=dtype)
    qp[:, :qlen] = q[:, offset:offset + qlen]
    nb = -(-(offset + lq_pad) // 32)
    kp = torch.zeros((2, nb * 32, head_dim), dtype=dtype)
    n = min(k.shape[1], nb * 32)
    kp[:, :n] = k[:, :n]
    pk = pool_blocks(kp.to(cuda), 32)
    pk_orc = orc.pool_blocks(to_np(kp), 32, out_dtype=_DT[dtype])
    assert np.array_equal(to_np(pk), pk_orc)
    sel, scores = block_scores_and_select(qp.to(cuda), pk, scale=head_dim ** -0.5,
                                          config=config, offset=offset, query_length=qlen)
    sel_o, scores_o, ratio = orc.block_scores_and_select(
        to_np(qp), pk_orc, scale=head_dim ** -0.5, config=_cfg(config), offset=offset,
        query_length=qlen, return_ratio=True)
    _assert_selection_parity(to_np(sel), sel_o, ratio, config.alpha)
    got = to_np(scores)
    assert np.all(np.abs(got - scores_o) <= 1e-5 * np.maximum(1.0, np.abs(scores_o)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 96, 128, 256])
@pytest.mark.parametrize("offset,qlen,tile_q", [(0, 512, 16), (77, 300, 16), (40, 700, 64)])
def test_mask_only_selection_matches_oracle(cuda, dtype, head_dim, offset, qlen, tile_q):
    # A mask without lists and without scores runs the score-output kernel's
    # selection.  tile_q = 64 gives 256 packed rows per tile (two passes).
    config = FPV2Config(block_k=32, tile_q=tile_q, alpha=0.2, sink_tokens=32, window_tokens=64,
                        last_n_blocks=1, score_chunk_tiles=4)
    q, k, _ = structured_qkv(length=offset + qlen + 100, query_heads=8, kv_heads=2,
                             head_dim=head_dim, block_size=32, seed=head_dim + offset + 1,
                             dtype=dtype)
    lq_pad = -(-qlen // tile_q) * tile_q
    qp = torch.zeros((8, lq_pad, head_dim), dtype=dtype)
    qp[:, :qlen] = q[:, offset:offset + qlen]
    nb = -(-(offset + lq_pad) // 32)
    kp = torch.zeros((2, nb * 32, head_dim), dtype=dtype)
    n = min(k.shape[1], nb * 32)
    kp[:, :n] = k[:, :n]
    pk = pool_blocks(kp.to(cuda), 32)
    pk_orc = orc.pool_blocks(to_np(kp), 32, out_dtype=_DT[dtype])
    sel, scores = block_scores_and_select(qp.to(cuda), pk, scale=head_dim ** -0.5,
                                          config=config, offset=offset, query_length=qlen)
    assert scores is None
    sel_o, _, ratio = orc.block_scores_and_select(
        to_np(qp), pk_orc, scale=head_dim ** -0.5, config=_cfg(config), offset=offset,
        query_length=qlen, return_ratio=True)
    _assert_selection_parity(to_np(sel), sel_o, ratio, config.alpha)
    assert to_np(sel).any(axis=-1).all()  # every tile keeps at least one block


def test_float32_selection_path_matches_oracle(cuda):
    config = FPV2Config(block_k=16, tile_q=16, alpha=0.3, sink_tokens=0, window_tokens=16)
    q, k, _ = structured_qkv(length=256, query_heads=4, kv_heads=2, head_dim=48,
                             block_size=16, seed=2)
    pk = orc.pool_blocks(k.numpy(), 16)
    sel, _ = block_scores_and_select(q.to(cuda), torch.from_numpy(pk).to(cuda), scale=0.2,
                                     config=config)
    sel_o, _, ratio = orc.block_scores_and_select(q.numpy(), pk, scale=0.2, config=_cfg(config),
                                                  return_ratio=True)
    _assert_selection_parity(to_np(sel), sel_o, ratio, config.alpha)


# ------------------------------------------------------------ compaction ----

def test_compaction_preserves_ascending_selected_indices(cuda):
    selected = torch.tensor([[[True, False, True, False]]], device=cuda)
    ids, counts, _, _ = compact_block_indices(selected, config=FPV2Config(block_k=16, tile_q=16))
    assert counts.item() == 2
    assert ids[0, 0].tolist() == [0, 2, 1, 3]


@pytest.mark.parametrize("nb", [1, 7, 256, 300, 1024, 4097])
def test_compaction_matches_oracle_bit_exact(cuda, nb):
    rng = np.random.default_rng(nb)
    mask = rng.random((3, 5, nb)) < 0.3
    cfg = FPV2Config(block_k=16, tile_q=32)
    offset = max(16 * nb - 5 * 32, 0)
    key_length = min(16 * nb, offset + 5 * 32 + 3)
    qlen = min(5 * 32 - 7, key_length - offset)
    got = compact_block_indices(torch.from_numpy(mask).to(cuda), config=cfg, offset=offset,
                                query_length=qlen, key_length=key_length)
    want = orc.compact_block_indices(mask, config=_cfg(cfg), offset=offset,
                                     query_length=qlen, key_length=key_length)
    for g, w in zip(got, want):
        assert np.array_equal(to_np(g), w)


# --------------------------------------------- fused hook-path selection ----

def _hook_select(q, k, config, *, total_tokens=None):
    """Run the hook's pool + score/select/compact launches; return everything."""
    from fpv2.patch import _effective_config, _request_config
    lib = _lib.load()
    dev = q.device
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    cfg = _request_config(_effective_config(config, hq, hkv), lk, total_tokens)
    offset = lk - lq
    lq_pad = -(-lq // cfg.tile_q) * cfg.tile_q
    lk_pad = -(-max(lk, offset + lq_pad) // cfg.block_k) * cfg.block_k
    nt, nb = lq_pad // cfg.tile_q, lk_pad // cfg.block_k
    pk = torch.empty((hkv, nb, d), dtype=q.dtype, device=dev)
    status = lib.fpv2_pool_blocks(k.data_ptr(), pk.data_ptr(), _lib.dtype_code(q.dtype), hkv,
                                  lk, nb, d, cfg.block_k, k.stride(0), k.stride(1),
                                  pk.stride(0), _lib.stream_ptr(dev))
    _lib.check(status, "pool")
    from fpv2.selection import _select_params
    ids = torch.empty((hkv, nt, nb), dtype=torch.int32, device=dev)
    pids = torch.empty_like(ids)
    cnt = torch.empty((hkv, nt), dtype=torch.int32, device=dev)
    pcnt = torch.empty_like(cnt)
    mask = torch.empty((hkv, nt, nb), dtype=torch.bool, device=dev)
    params = _select_params(q, nb, kv_heads=hkv, scale=d ** -0.5, config=cfg, offset=offset,
                            query_length=lq, padded_length=lq_pad, key_length=lk)
    status = lib.fpv2_score_select(q.data_ptr(), pk.data_ptr(), _lib.dtype_code(q.dtype),
                                   params, mask.data_ptr(), None, ids.data_ptr(),
                                   cnt.data_ptr(), pids.data_ptr(), pcnt.data_ptr(),
                                   _lib.stream_ptr(dev))
    _lib.check(status, "score_select")
    return cfg, offset, pk, mask, (ids, cnt, pids, pcnt)


@pytest.mark.parametrize("seq,planted", [(2048, 3.0), (4096, 3.0 * 128 ** 0.5), (8192, 3.0)])
def test_fused_selection_lists_match_oracle(cuda, seq, planted):
    q, k, _ = baseline_qkv(seq, planted=planted, heavy_fraction=0.06, seed=1)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    qd, kd = q.to(cuda), k.to(cuda)
    cfg, offset, pk, mask, lists = _hook_select(qd, kd, config, total_tokens=seq)
    pk_o = orc.pool_blocks(to_np(k), 128, out_dtype="bf16")
    assert np.array_equal(to_np(pk), pk_o)
    sel_o, _, ratio = orc.block_scores_and_select(
        to_np(q), pk_o, scale=128 ** -0.5, config=_cfg(replace(cfg, score_chunk_tiles=32)),
        offset=offset, query_length=seq, return_ratio=True)
    near = _assert_selection_parity(to_np(mask), sel_o, ratio, config.alpha)
    want = orc.compact_block_indices(to_np(mask).astype(bool), config=_cfg(cfg), offset=offset,
                                     query_length=seq, key_length=seq)
    for g, w in zip(lists, want):
        assert np.array_equal(to_np(g), w)
    if not near.any():
        want_o = orc.compact_block_indices(sel_o, config=_cfg(cfg), offset=offset,
                                           query_length=seq, key_length=seq)
        for g, w in zip(lists, want_o):
            assert np.array_equal(to_np(g), w)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 96, 128, 256])
@pytest.mark.parametrize("lq,lk,tile_q", [(512, 512, 16), (300, 377, 16), (700, 740, 64), (300, 300, 6)])
def test_hook_lists_match_oracle(cuda, dtype, head_dim, lq, lk, tile_q):
    # Lists requested, no score output: the hook's selection.  head_dim <= 128
    # runs the streaming kernel (swizzled Q rows when tile_q is a multiple of
    # a fill's rows, padded rows for tile_q = 6 and head_dim 96; tile_q = 64
    # gives two 128-row units per tile), head_dim 256 the owner kernel.
    config = FPV2Config(block_k=32, tile_q=tile_q, alpha=0.2, sink_tokens=32, window_tokens=64,
                        last_n_blocks=1)
    q_all, k, _ = structured_qkv(length=lk, query_heads=8, kv_heads=2, head_dim=head_dim,
                                 block_size=32, seed=head_dim + lq + tile_q, dtype=dtype)
    q = q_all[:, lk - lq:].contiguous()
    cfg, offset, pk, mask, lists = _hook_select(q.to(cuda), k.to(cuda), config, total_tokens=lk)
    assert offset == lk - lq
    lq_pad = -(-lq // tile_q) * tile_q
    nb = pk.shape[1]
    qp = torch.zeros((8, lq_pad, head_dim), dtype=dtype)
    qp[:, :lq] = q
    kp = torch.zeros((2, nb * 32, head_dim), dtype=dtype)
    kp[:, :lk] = k
    pk_o = orc.pool_blocks(to_np(kp), 32, out_dtype=_DT[dtype])
    assert np.array_equal(to_np(pk), pk_o)
    sel_o, _, ratio = orc.block_scores_and_select(
        to_np(qp), pk_o, scale=head_dim ** -0.5, config=_cfg(cfg), offset=offset,
        query_length=lq, return_ratio=True)
    near = _assert_selection_parity(to_np(mask), sel_o, ratio, config.alpha)
    want = orc.compact_block_indices(to_np(mask).astype(bool), config=_cfg(cfg), offset=offset,
                                     query_length=lq, key_length=lk)
    for g, w in zip(lists, want):
        assert np.array_equal(to_np(g), w)
    if not near.any():
        want_o = orc.compact_block_indices(sel_o, config=_cfg(cfg), offset=offset,
                                           query_length=lq, key_length=lk)
        for g, w in zip(lists, want_o):
            assert np.array_equal(to_np(g), w)


def test_full_size_lists_are_consistent_at_32k(cuda):
    """Size-independent properties at BASELINE config 2 (seq 32768)."""
    seq = 32768
    q, k, _ = baseline_qkv(seq, device=cuda, seed=0)
    cfg, offset, _, mask, (ids, cnt, pids, pcnt) = _hook_select(
        q, k, FPV2Config(alpha=0.1, sink_tokens=128), total_tokens=seq)
    m = mask.cpu()
    assert torch.equal(cnt.cpu(), m.sum(-1, dtype=torch.int32))
    ids_c = ids.cpu().long()
    nb = ids_c.shape[-1]
    # every row is a permutation whose first `count` entries are the mask, ascending
    assert torch.equal(ids_c.sort(-1).values, torch.arange(nb).expand_as(ids_c))
    pos = torch.arange(nb).expand_as(ids_c)
    head = pos < cnt.cpu().long()[..., None]
    assert torch.equal(torch.gather(m, -1, ids_c), head)
    diffs = ids_c[..., 1:] - ids_c[..., :-1]
    boundary = pos[..., 1:] == cnt.cpu().long()[..., None]
    assert bool(((diffs > 0) | boundary).all())
    # visible-only, forced sink/local/diagonal present, pruned strictly in the past
    nt = m.shape[1]
    tile_last = offset + torch.minimum((torch.arange(nt) + 1) * cfg.tile_q, torch.tensor(seq)) - 1
    visible = (torch.arange(nb) * cfg.block_k)[None, :] <= tile_last[:, None]
    assert not bool((m & ~visible).any())
    assert bool(m[:, :, 0].all())
    diag = tile_last // cfg.block_k
    assert bool(m[:, torch.arange(nt), diag].all())
    pc = pcnt.cpu().long()
    first = offset + torch.arange(nt) * cfg.tile_q
    past = ((torch.arange(nb) + 1) * cfg.block_k)[None, :] <= first[:, None]
    assert torch.equal(pc, ((~m) & past).sum(-1))
