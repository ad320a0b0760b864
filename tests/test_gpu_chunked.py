"""Chunked prefill over a growing KV cache (fpv2.chunked.ChunkedPrefill).

Against the hook on the same prefix (``fpv2_sdpa``, which re-pools the whole
prefix per call as ``patch.py:137-138`` does): outputs and pooled blocks are
bit-identical, chunk by chunk, including chunks that end inside a block.  The
pooled cache is also checked against the oracle's pooling of the zero-padded
prefix, and the below-``min_tokens`` path against exact causal attention.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import attention_errors, to_np
from oracle import fpv2_oracle as orc
from fpv2 import ChunkedPrefill, FPV2Config, fpv2_sdpa
from fpv2.synthetic import structured_qkv

pytestmark = pytest.mark.gpu


def _inputs(cuda, length, *, hq=8, hkv=2, d=128, seed=11):
    q, k, v = structured_qkv(length=length, query_heads=hq, kv_heads=hkv, head_dim=d, seed=seed)
    return (x.bfloat16().to(cuda) for x in (q, k, v))


@pytest.mark.parametrize(("total", "chunk"), [(3000, 1000), (2304, 256), (1100, 700)])
def test_chunked_matches_hook_bit_exact(cuda, total, chunk):
    q, k, v = _inputs(cuda, total)
    config = FPV2Config(alpha=0.15, sink_tokens=128, window_tokens=256)
    cp = ChunkedPrefill(8, 2, 128, total, config=config, total_tokens=total, min_tokens=1,
                        device=cuda)
    for start in range(0, total, chunk):
        end = min(start + chunk, total)
        out = cp.step(q[:, start:end], k[:, start:end], v[:, start:end])
        ref = fpv2_sdpa(q[None, :, start:end], k[None, :, :end], v[None, :, :end],
                        scale=128 ** -0.5, config=cp.request_config())
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (start, end)
        nb = -(-end // 128)
        pad = np.zeros((2, nb * 128, 128), np.float32)
        pad[:, :end] = to_np(k[:, :end])
        assert np.array_equal(to_np(cp.pooled_k[:, :nb]), orc.pool_blocks(pad, 128, out_dtype="bf16"))
        pad[:, :end] = to_np(v[:, :end])
        assert np.array_equal(to_np(cp.pooled_v[:, :nb]), orc.pool_blocks(pad, 128, out_dtype="bf16"))
    # every row pooled once, plus the re-pooled partial blocks
    partial = sum(min(s + chunk, total) % 128 for s in range(0, total, chunk))
    assert cp.pooled_rows == total - total % 128 + partial


@pytest.mark.parametrize(("dtype", "d", "heads"), [(torch.float16, 128, (8, 2)),
                                                  (torch.bfloat16, 64, (16, 2)),
                                                  (torch.float16, 256, (4, 1)),
                                                  (torch.bfloat16, 96, (6, 3))])
def test_chunked_other_dtypes_and_head_dims_match_hook_bit_exact(cuda, dtype, d, heads):
    hq, hkv = heads
    total, chunk = 2304, 700
    q, k, v = structured_qkv(length=total, query_heads=hq, kv_heads=hkv, head_dim=d, seed=d + hq)
    q, k, v = (x.to(dtype).to(cuda) for x in (q, k, v))
    config = FPV2Config(alpha=0.15, sink_tokens=128, window_tokens=256)
    cp = ChunkedPrefill(hq, hkv, d, total, config=config, total_tokens=total, min_tokens=1,
                        dtype=dtype, device=cuda)
    for start in range(0, total, chunk):
        end = min(start + chunk, total)
        out = cp.step(q[:, start:end], k[:, start:end], v[:, start:end])
        ref = fpv2_sdpa(q[None, :, start:end], k[None, :, :end], v[None, :, :end],
                        scale=d ** -0.5, config=cp.request_config())
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (start, end)


def test_dense_tail_only_at_total_tokens(cuda):
    cp = ChunkedPrefill(8, 2, 128, 4096, total_tokens=4096, min_tokens=1, device=cuda)
    q, k, v = _inputs(cuda, 4096)
    tails = []
    for start in range(0, 4096, 1024):
        cp.append(k[:, start:start + 1024], v[:, start:start + 1024])
        tails.append(cp.request_config().last_n_blocks)
        cp.attend(q[:, start:start + 1024])
    assert tails == [0, 0, 0, FPV2Config().last_n_blocks]


def test_below_min_tokens_is_exact_causal(cuda):
    q, k, v = _inputs(cuda, 1536, seed=5)
    cp = ChunkedPrefill(8, 2, 128, 1536, min_tokens=4096, device=cuda)
    outs = [cp.step(q[:, s:s + 512], k[:, s:s + 512], v[:, s:s + 512]) for s in range(0, 1536, 512)]
    torch.cuda.synchronize()
    got = np.concatenate([to_np(o[0]) for o in outs], axis=1)
    exact = orc.exact_causal_attention(to_np(q), to_np(k), to_np(v), 128 ** -0.5)
    err = attention_errors(got, exact)
    assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, err


def test_reset_and_capacity(cuda):
    q, k, v = _inputs(cuda, 512)
    cp = ChunkedPrefill(8, 2, 128, 512, min_tokens=1, device=cuda)
    first = cp.step(q, k, v)
    with pytest.raises(ValueError, match="capacity"):
        cp.append(k[:, :1], v[:, :1])
    cp.reset()
    again = cp.step(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(first, again)


def test_reserve_then_fill_equals_append(cuda):
    """``reserve`` hands out the cache rows ``append`` would copy into."""
    from fpv2 import ChunkedPrefill
    g = torch.Generator().manual_seed(5)
    k = torch.randn((2, 300, 64), generator=g).bfloat16().to(cuda)
    v = torch.randn((2, 300, 64), generator=g).bfloat16().to(cuda)
    q = torch.randn((8, 300, 64), generator=g).bfloat16().to(cuda)
    a = ChunkedPrefill(8, 2, 64, 512, device=cuda, min_tokens=1)
    b = ChunkedPrefill(8, 2, 64, 512, device=cuda, min_tokens=1)
    outs = []
    for s0, s1 in ((0, 200), (200, 300)):
        a.append(k[:, s0:s1], v[:, s0:s1])
        kr, vr = b.reserve(s1 - s0)
        kr.copy_(k[:, s0:s1])
        vr.copy_(v[:, s0:s1])
        outs.append((a.attend(q[:, s0:s1]), b.attend(q[:, s0:s1])))
    torch.cuda.synchronize()
    for x, y in outs:
        assert torch.equal(x, y)
    with pytest.raises(ValueError, match="capacity"):
        b.reserve(213)


def test_chunk_shorter_than_a_tile_is_exact_causal(cuda):
    """A chunk with fewer queries than one selection tile (here 20 < 32 at
    G = 4) is sent to the original attention by the hook (``patch.py:177-205``);
    the chunked layer attends it exactly, also when it is not the last chunk
    and no ``total_tokens`` is known."""
    q, k, v = _inputs(cuda, 1320, seed=9)
    config = FPV2Config(alpha=0.5, sink_tokens=128, window_tokens=128)
    cp = ChunkedPrefill(8, 2, 128, 1320, config=config, min_tokens=1, device=cuda,
                        collect_stats=True)
    cp.step(q[:, :1280], k[:, :1280], v[:, :1280])
    assert cp.block_sparsity() > 0  # the long chunk prunes
    sparsity, visible = cp.block_sparsity(), cp._visible
    short = cp.step(q[:, 1280:1300], k[:, 1280:1300], v[:, 1280:1300])
    torch.cuda.synchronize()
    # the hook's accounting leaves such a call out (patch.py:255-266)
    assert cp._visible == visible and cp.block_sparsity() == sparsity
    exact = orc.exact_causal_attention(to_np(q[:, 1280:1300]), to_np(k[:, :1300]),
                                       to_np(v[:, :1300]), 128 ** -0.5, offset=1280)
    err = attention_errors(to_np(short[0]), exact)
    assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, err


def test_prefix_past_the_block_limit_is_exact_causal(cuda):
    """A prefix of 8193 key blocks (past the selection kernel's limit, where
    the hook hands the call to the original attention) runs exact causal
    attention: every visible block, in order, through the attention kernel.
    Checked against float32 attention on the GPU (float32 products only)
    and counted as dense.  The chunked calls stay out of the hook's
    ``block_sparsity``."""
    from fpv2 import _lib, block_sparsity, disable, enable
    lq = 32
    total = _lib.MAX_BLOCKS * 128 + lq
    cp = ChunkedPrefill(4, 1, 64, total, config=FPV2Config(alpha=0.5), min_tokens=1,
                        device=cuda, collect_stats=True)
    g = torch.Generator(device=cuda).manual_seed(3)
    k_rows, v_rows = cp.reserve(total - lq)
    k_rows.copy_(torch.randn(k_rows.shape, generator=g, device=cuda))
    v_rows.copy_(torch.randn(v_rows.shape, generator=g, device=cuda))
    q = torch.randn((4, lq, 64), generator=g, device=cuda).bfloat16()
    k = torch.randn((1, lq, 64), generator=g, device=cuda).bfloat16()
    v = torch.randn((1, lq, 64), generator=g, device=cuda).bfloat16()
    enable(min_tokens=1, collect_stats=True)
    try:
        keep = {}
        cp.append(k, v)
        out = cp.attend(q, keep=keep)[0]
        torch.cuda.synchronize()
        assert block_sparsity() == 0.0  # nothing counted by the hook
    finally:
        disable()
    assert keep["lists"][0].shape[-1] == _lib.MAX_BLOCKS + 1
    assert cp.block_sparsity() == 0.0 and cp._visible == _lib.MAX_BLOCKS + 1
    kf, vf = cp.k[0].float(), cp.v[0].float()  # [total, 64]
    s = (q.float() @ kf.T) * 0.125  # float32 on the GPU
    mask = torch.arange(total, device=cuda)[None, :] <= (total - lq + torch.arange(lq, device=cuda))[:, None]
    s = s.masked_fill(~mask[None], float("-inf"))
    want = torch.softmax(s, dim=-1) @ vf
    err = attention_errors(to_np(out), to_np(want))
    assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, err


def test_config4_chunked_65536_in_2048_token_chunks(cuda):
    """one layer, 65536 tokens of the BASELINE generator in
    2048-token chunks over a growing bf16 KV cache, ``total_tokens`` known.
    Every chunk equals the hook (``fpv2_sdpa``, which re-pools the whole
    prefix) bit for bit, the dense tail appears only on the last chunk, and
    sampled tiles of the last chunk and of a middle chunk match the oracle on
    their full prefixes: block lists outside the 1e-4 band and rows within
    2e-2 / 2e-3."""
    from fpv2.synthetic import baseline_qkv
    total, chunk = 65536, 2048
    q, k, v = baseline_qkv(total, planted=3.0, heavy_fraction=0.06, seed=0, device=cuda)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    cp = ChunkedPrefill(32, 8, 128, total, config=config, total_tokens=total, min_tokens=2048,
                        device=cuda)
    keep = None
    middle = None
    for s0 in range(0, total, chunk):
        s1 = s0 + chunk
        cp.append(k[:, s0:s1], v[:, s0:s1])
        tail = cp.request_config(chunk).last_n_blocks
        assert tail == (2 if s1 == total else 0)
        keep = {}
        out = cp.attend(q[:, s0:s1], keep=keep)
        ref = fpv2_sdpa(q[None, :, s0:s1], k[None, :, :s1], v[None, :, :s1], scale=128 ** -0.5,
                        config=cp.request_config(chunk))
        assert torch.equal(out, ref), (s0, s1)
        if s1 == total // 2:
            middle = (keep, out, s0)
    torch.cuda.synchronize()
    kn, vn = to_np(k), to_np(v)
    nb = keep["lists"][0].shape[-1]
    pooled_k = to_np(cp.pooled_k[:, :nb])
    pooled_v = to_np(cp.pooled_v[:, :nb])
    assert np.array_equal(pooled_k, orc.pool_blocks(kn, 128, out_dtype="bf16"))
    assert np.array_equal(pooled_v, orc.pool_blocks(vn, 128, out_dtype="bf16"))
    # the last chunk (dense tail) and a middle one (chunk 15 of 32, keys up
    # to 32768, no tail: total_tokens not reached) against the oracle on
    # their full prefixes; blocks pooled once are the same in both caches
    for keep_c, out_c, off in ((keep, out, total - chunk), middle):
        _check_chunk_tiles(q, kn, vn, keep_c, out_c, off, chunk, pooled_k, pooled_v)


def _check_chunk_tiles(q, kn, vn, keep, out, off, chunk, pooled_k, pooled_v):
    """Start, middle and end tiles of one chunk's call (queries at ``off``)
    against the oracle: lists outside the 1e-4 band, rows on the device's
    selection."""
    cfg = keep["config"]
    tq = cfg.tile_q
    ids, counts, _, _ = keep["lists"]
    nb = ids.shape[-1]
    pooled_k, pooled_v = pooled_k[:, :nb], pooled_v[:, :nb]
    ocfg = orc.OracleConfig(**{f: getattr(cfg, f) for f in orc.OracleConfig.__dataclass_fields__})
    nt = chunk // tq
    for t0, n in ((0, 2), (nt // 2, 2), (nt - 3, 3)):  # start, middle, end
        rows0 = t0 * tq
        qs = to_np(q[:, off + rows0:off + rows0 + n * tq])
        # the sampled tiles as their own call at offset off + rows0; the dense
        # tail counts tiles from the end of the real call
        sub_cfg = ocfg if t0 + n == nt else orc._replace(ocfg, last_n_blocks=0)
        sel, _, ratio = orc.block_scores_and_select(
            qs, pooled_k, scale=128 ** -0.5, config=orc._replace(sub_cfg, score_chunk_tiles=1),
            offset=off + rows0, query_length=n * tq, return_ratio=True)
        idn, cn = to_np(ids[:, t0:t0 + n]), to_np(counts[:, t0:t0 + n])
        dev_sel = np.zeros(idn.shape, dtype=bool)
        for h in range(idn.shape[0]):
            for t in range(n):
                dev_sel[h, t, idn[h, t, :cn[h, t]]] = True
        decided = np.abs(ratio - cfg.alpha) > 1e-4
        assert np.array_equal(sel[decided], dev_sel[decided]), (off, t0)
        ref = orc.fpv2_attention_blockwise(
            qs, kn[:, :off + chunk], vn[:, :off + chunk], scale=128 ** -0.5, selected=dev_sel,
            pooled_k=pooled_k, pooled_v=pooled_v, config=sub_cfg, offset=off + rows0,
            row_block=tq, key_length=off + chunk)
        err = attention_errors(to_np(out[0, :, rows0:rows0 + n * tq]), ref)
        assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, (off, t0, err)
