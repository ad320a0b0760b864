"""GPU parity of the SDPA hook (``fpv2/patch.py`` counterpart).

Reference tests restated (``tests/test_patch.py``): alpha=0 equals stock
attention for padded, unaligned-chunk and real shapes; ineligible calls are
bit-identical; tile-aligned chunks equal single-shot FPV2; sparsity accounting.
"Stock attention" is computed on the CPU in float32 (a textbook softmax),
never with bf16 batched products on the GPU.  BASELINE config 1 (8k, Qwen3-4B
geometry) and its high-contrast variant are checked end to end against the
oracle's hook data flow on a subset of query tiles.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import attention_errors, to_np
from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config, block_sparsity, disable, enable, fpv2_sdpa
from fpv2.patch import _ORIGINAL_SDPA, _fpv2_sdpa, _request_config
from fpv2.synthetic import baseline_qkv, structured_qkv

pytestmark = pytest.mark.gpu

try:
    from torch.nn.attention.bias import causal_lower_right
except ImportError:  # pragma: no cover
    causal_lower_right = None

MAX_ABS, MEAN_ABS, REL = 2e-2, 2e-3, 2e-2


@pytest.fixture(autouse=True)
def restore_sdpa():
    disable()
    yield
    disable()


def _inputs(length, query_length=None, *, heads=(4, 2), dim=64, seed=7):
    g = torch.Generator().manual_seed(seed)
    query_length = length if query_length is None else query_length
    q = torch.randn((1, heads[0], query_length, dim), generator=g).bfloat16()
    k = torch.randn((1, heads[1], length, dim), generator=g).bfloat16()
    v = torch.randn((1, heads[1], length, dim), generator=g).bfloat16()
    return q, k, v


def _stock(q, k, v, scale):
    """Bottom-right causal softmax attention on the CPU in float32."""
    q, k, v = (x.float().cpu() for x in (q, k, v))
    g = q.shape[1] // k.shape[1]
    k, v = k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
    lq, lk = q.shape[-2], k.shape[-2]
    mask = torch.arange(lk)[None, :] <= (lk - lq + torch.arange(lq))[:, None]
    return _ORIGINAL_SDPA(q, k, v, attn_mask=mask, scale=scale).numpy()


def _hook_call(q, k, v, scale):
    lq, lk = q.shape[-2], k.shape[-2]
    if lq == lk:
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale,
                                              enable_gqa=True)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=causal_lower_right(lq, lk),
                                          scale=scale, enable_gqa=True)


@pytest.mark.parametrize(("length", "query_length"), [(130, 130), (190, 128)])
def test_alpha_zero_padded_and_unaligned_calls_match_stock(cuda, length, query_length):
    # tests/test_patch.py:44-73
    q, k, v = _inputs(length, query_length)
    expected = _stock(q, k, v, 0.125)
    enable(FPV2Config(alpha=0, sink_tokens=0, window_tokens=0), min_tokens=1)
    actual = _hook_call(q.to(cuda), k.to(cuda), v.to(cuda), 0.125)
    assert F.scaled_dot_product_attention is not _ORIGINAL_SDPA
    assert attention_errors(to_np(actual), expected)["rel"] < REL


@pytest.mark.parametrize(("key_length", "query_length"),
                         [(4096, 4096), (4100, 4100), (8192, 2048), (4100, 1000), (6000, 128)])
def test_real_shape_alpha_zero_matches_stock(cuda, key_length, query_length):
    # tests/test_patch.py:110-133
    g = torch.Generator().manual_seed(17)
    q = torch.randn((1, 8, query_length, 128), generator=g).bfloat16()
    k = torch.randn((1, 2, key_length, 128), generator=g).bfloat16()
    v = torch.randn((1, 2, key_length, 128), generator=g).bfloat16()
    expected = _stock(q, k, v, 128 ** -0.5)
    enable(FPV2Config(alpha=0, sink_tokens=0, window_tokens=0), min_tokens=1)
    actual = to_np(_hook_call(q.to(cuda), k.to(cuda), v.to(cuda), 128 ** -0.5))
    err = attention_errors(actual, expected)
    assert err["rel"] < REL and err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err


@pytest.mark.parametrize(("length", "query_length", "kind"),
                         [(64, 64, "causal"), (128, 1, "causal"), (128, 32, "causal"),
                          (128, 128, "none"), (128, 128, "array")])
def test_ineligible_calls_are_bit_identical(cuda, length, query_length, kind):
    # tests/test_patch.py:76-107
    q, k, v = (x.to(cuda) for x in _inputs(length, query_length))
    kwargs = dict(scale=0.125, enable_gqa=True)
    if kind == "causal":
        kwargs["is_causal"] = True
    elif kind == "array":
        kwargs["attn_mask"] = torch.zeros((query_length, length), dtype=torch.bfloat16,
                                          device=cuda)
    expected = _ORIGINAL_SDPA(q, k, v, **kwargs)
    enable(min_tokens=128)
    actual = F.scaled_dot_product_attention(q, k, v, **kwargs)
    assert torch.equal(actual, expected)


def test_tile_aligned_chunks_match_single_shot_fpv2(cuda):
    # tests/test_patch.py:136-166
    q, k, v = structured_qkv(length=8192, query_heads=8, kv_heads=2, head_dim=128,
                             dtype=torch.bfloat16, seed=23, device=cuda)
    q, k, v = q[None], k[None], v[None]
    config = FPV2Config(alpha=0.15, mean_correction=True)
    scale = 128 ** -0.5
    expected = fpv2_sdpa(q, k, v, scale=scale, config=config)
    chunks = []
    for end in range(2048, 8193, 2048):
        cfg = _request_config(config, end, q.shape[-2])
        chunks.append(fpv2_sdpa(q[:, :, end - 2048:end], k[:, :, :end], v[:, :, :end],
                                scale=scale, config=cfg))
    actual = torch.cat(chunks, dim=2)
    assert attention_errors(to_np(actual), to_np(expected))["rel"] < 1e-2


def test_block_sparsity_includes_dense_gated_prefill(cuda):
    # tests/test_patch.py:180-201
    q, k, v = (x.to(cuda) for x in _inputs(256))
    enable(FPV2Config(alpha=1e9, sink_tokens=0, window_tokens=0, last_n_blocks=0),
           min_tokens=256, collect_stats=True)
    F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.125, enable_gqa=True)
    assert block_sparsity() == pytest.approx(1 / 3)
    q, k, v = (x.to(cuda) for x in _inputs(128))
    F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.125, enable_gqa=True)
    assert block_sparsity() == pytest.approx(1 / 4)


def test_strided_model_layout_is_read_in_place(cuda):
    """[B, L, H, D] activations transposed to [B, H, L, D] views (no copy)."""
    g = torch.Generator().manual_seed(29)
    x = torch.randn((1, 4096, 8 + 2 + 2, 128), generator=g).bfloat16().to(cuda)
    q, k, v = (x[:, :, :8].transpose(1, 2), x[:, :, 8:10].transpose(1, 2),
               x[:, :, 10:].transpose(1, 2))
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    a = fpv2_sdpa(q, k, v, scale=128 ** -0.5, config=config)
    b = fpv2_sdpa(q.contiguous(), k.contiguous(), v.contiguous(), scale=128 ** -0.5,
                  config=config)
    assert torch.equal(a, b)


def _baseline_parity(cuda, seq, planted, tiles):
    q, k, v = baseline_qkv(seq, planted=planted, heavy_fraction=0.06, seed=0)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    scale = 128 ** -0.5
    enable(config, min_tokens=1, total_tokens=seq)
    out = _hook_call(q[None].to(cuda), k[None].to(cuda), v[None].to(cuda), scale)[0]
    want, plan = orc.fpv2_sdpa_oracle(to_np(q), to_np(k), to_np(v), scale=scale,
                                      config=orc.OracleConfig(alpha=0.1, sink_tokens=128),
                                      return_plan=True, tiles=tiles)
    tq = plan["config"].tile_q
    rows = np.concatenate([np.arange(t * tq, (t + 1) * tq) for t in tiles])
    got = to_np(out)[:, rows]
    err = attention_errors(got, want[:, rows])
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err
    return plan


def test_baseline_config1_8k_matches_oracle(cuda):
    """BASELINE config 1 through the hook: sampled rows against the oracle's
    hook data flow, and every tile's block lists (256 tiles x 8 KV heads)
    against the oracle's selection and compaction, bit for bit outside the
    1e-4 band."""
    nt = 8192 // 32
    tiles = sorted({0, 1, 2, 3, 100, 177, nt // 2, nt - 3, nt - 2, nt - 1})
    _baseline_parity(cuda, 8192, 3.0, tiles)
    q, k, v = baseline_qkv(8192, planted=3.0, heavy_fraction=0.06, seed=0)
    keep = {}
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    _fpv2_sdpa(q[None].to(cuda), k[None].to(cuda), v[None].to(cuda), scale=128 ** -0.5,
               config=config, keep=keep)
    torch.cuda.synchronize()
    ids, counts, pids, pcounts = (to_np(x) for x in keep["lists"])
    plan_cfg = orc.OracleConfig(**{f: getattr(keep["config"], f)
                                   for f in orc.OracleConfig.__dataclass_fields__})
    sel, _, ratio = orc.block_scores_and_select(
        to_np(q), to_np(keep["pooled_k"]), scale=128 ** -0.5,
        config=orc._replace(plan_cfg, score_chunk_tiles=32), return_ratio=True)
    dev_sel = np.zeros(sel.shape, dtype=bool)
    for h in range(ids.shape[0]):
        for t in range(ids.shape[1]):
            dev_sel[h, t, ids[h, t, :counts[h, t]]] = True
    decided = np.abs(ratio - 0.1) > 1e-4
    assert decided.sum() > 0.99 * decided.size
    assert np.array_equal(sel[decided], dev_sel[decided])
    o_ids, o_counts, o_pids, o_pcounts = orc.compact_block_indices(
        dev_sel, config=plan_cfg, query_length=8192, key_length=8192)
    assert np.array_equal(ids, o_ids) and np.array_equal(counts, o_counts)
    assert np.array_equal(pcounts, o_pcounts)
    head = np.arange(ids.shape[-1])[None, None, :] < o_pcounts[..., None]
    assert np.array_equal(np.where(head, pids, -1), np.where(head, o_pids, -1))


def test_baseline_contrast_variant_exercises_pruning(cuda):
    nt = 8192 // 32
    tiles = sorted({2, 40, 129, nt - 40, nt - 3, nt - 1})
    plan = _baseline_parity(cuda, 8192, 3.0 * 128 ** 0.5, tiles)
    dens = orc.density(plan["selected"], config=plan["config"])
    assert dens < 0.6  # real pruning, so the pooled correction is active
    assert int(plan["lists"][3].max()) > 0


def test_block_counter_waits_for_the_stream_that_wrote_the_counts(cuda):
    """Counts written on a side stream (behind a long matmul) are summed on
    the default stream: the fold waits for the side stream.  Folds happen on
    two different streams, so the running total itself moves between them."""
    from fpv2.patch import SelectedBlockCounter
    counter = SelectedBlockCounter(fold_every=4)
    side = torch.cuda.Stream(device=cuda)
    other = torch.cuda.Stream(device=cuda)
    a = torch.randn((4096, 4096), device=cuda)
    torch.cuda.synchronize()
    expected = 0
    for stream in (side, other, side):
        with torch.cuda.stream(stream):
            for i in range(6):
                b = a @ a  # keeps the stream busy before each count is written
                counts = torch.full((2, 8), i + 1, dtype=torch.int32, device=cuda)
                counts += (b[0, :1] * 0).to(torch.int32)  # written after the matmul
                counter.add(counts)  # folds every 4 calls, on this stream
                expected += 16 * (i + 1)
            # memory the allocator may hand to the next counts on this stream
            junk = torch.full((1 << 20,), -7, dtype=torch.int64, device=cuda)
            del junk
    assert counter.value() == expected


def test_calls_past_the_block_limit_reach_the_original_sdpa(cuda):
    """An otherwise eligible call whose keys need 8193 blocks (one more than
    the selection kernel holds) is served by the original SDPA, bit for bit,
    and counted as dense; the reference's hook has no such limit and serves
    every eligible call (patch.py:237-271), so the call is not refused."""
    from fpv2 import _lib
    lq, lk = 32, _lib.MAX_BLOCKS * 128 + 1
    g = torch.Generator(device=cuda).manual_seed(5)
    q = torch.randn((1, 4, lq, 64), generator=g, device=cuda).bfloat16()
    k = torch.randn((1, 1, lk, 64), generator=g, device=cuda).bfloat16()
    v = torch.randn((1, 1, lk, 64), generator=g, device=cuda).bfloat16()
    kwargs = dict(attn_mask=causal_lower_right(lq, lk), scale=0.125, enable_gqa=True)
    expected = _ORIGINAL_SDPA(q, k, v, **kwargs)
    enable(min_tokens=1, collect_stats=True)
    actual = F.scaled_dot_product_attention(q, k, v, **kwargs)
    torch.cuda.synchronize()
    assert torch.equal(actual, expected)
    assert block_sparsity() == 0.0
    from fpv2 import patch
    assert patch._visible_blocks == patch._selected_dense_blocks == _lib.MAX_BLOCKS + 1


@pytest.mark.parametrize(("heads", "dim"), [((32, 2), 128), ((64, 2), 64), ((32, 1), 128)])
def test_large_gqa_groups_match_oracle(cuda, heads, dim):
    """G = 16 and 32 query heads per KV head: the hook's 128 packed rows
    become tiles of 8 and 4 query positions (patch.py:41-52)."""
    hq, hkv = heads
    lq = lk = 1536
    q, k, v = structured_qkv(length=lk, query_heads=hq, kv_heads=hkv, head_dim=dim, seed=hq + dim,
                             dtype=torch.bfloat16)
    config = FPV2Config(alpha=0.15, sink_tokens=128, window_tokens=128)
    scale = dim ** -0.5
    # the whole request in one call: the dense tail applies (patch.py:55-63)
    enable(config, min_tokens=1, total_tokens=lk)
    out = _hook_call(q[None].to(cuda), k[None].to(cuda), v[None].to(cuda), scale)[0]
    torch.cuda.synchronize()
    want, plan = orc.fpv2_sdpa_oracle(to_np(q), to_np(k), to_np(v), scale=scale,
                                      config=orc.OracleConfig(alpha=0.15, sink_tokens=128,
                                                              window_tokens=128),
                                      return_plan=True)
    assert plan["config"].tile_q == 128 // (hq // hkv)
    tq = plan["config"].tile_q
    near = (np.abs(plan["ratio"] - 0.15) <= 1e-4).any(axis=(0, 2))
    rows = np.ones(lq, dtype=bool)
    for t in np.nonzero(near)[0]:
        rows[t * tq:(t + 1) * tq] = False
    err = attention_errors(to_np(out)[:, rows], want[:, rows])
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err
