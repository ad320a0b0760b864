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
