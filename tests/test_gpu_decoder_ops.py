"""Decoder-layer kernels of the end-to-end harness (include/fpv2_decoder.h)
against float32 PyTorch references of the same operations.

The residual add is one float32 add rounded once, as torch's bf16 add, so the
updated residual must match bit for bit; the norm, rotation and gate outputs
must match to bf16 rounding (one ulp plus float32 reduction-order noise).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from fpv2.prefill_harness import (DecoderShape, _add_rms_norm, _qk_norm_rope, _silu_mul,
                                  rope_tables)

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _close(got, ref):
    # bf16 keeps 8 significant bits: one ulp is 2^-8 relative
    torch.testing.assert_close(got.float(), ref.float(), rtol=2 ** -7, atol=1e-3)


def _norm_ref(x, w):
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS) * w.float()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(37, 2560), (5, 8), (3, 16384), (64, 136)])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rms_norm(cuda, dtype, rows, cols, with_delta):
    g = torch.Generator(device=cuda).manual_seed(rows * cols)
    # a wider parent buffer: the row stride differs from cols
    x = (torch.randn((rows, cols + 8), generator=g, device=cuda) * 3).to(dtype)[:, :cols]
    delta = torch.randn((rows, cols), generator=g, device=cuda).to(dtype) if with_delta else None
    w = (1 + 0.1 * torch.randn(cols, generator=g, device=cuda)).to(dtype)
    x0 = x.clone()
    y = _add_rms_norm(x, delta, w, EPS)
    torch.cuda.synchronize()
    expect_x = (x0.float() + delta.float()).to(dtype) if with_delta else x0
    assert torch.equal(x, expect_x)
    _close(y, _norm_ref(expect_x, w).to(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim,qh,kh", [(128, 32, 8), (64, 4, 2), (256, 2, 1), (96, 6, 3)])
@pytest.mark.parametrize("into_cache", [False, True])
def test_qk_norm_rope(cuda, dtype, head_dim, qh, kh, into_cache):
    shape = DecoderShape(query_heads=qh, kv_heads=kh, head_dim=head_dim)
    rows = 19
    g = torch.Generator(device=cuda).manual_seed(head_dim + qh)
    qkv = (torch.randn((rows, (qh + 2 * kh) * head_dim), generator=g, device=cuda) * 2).to(dtype)
    qw = (1 + 0.2 * torch.randn(head_dim, generator=g, device=cuda)).to(dtype)
    kw = (1 + 0.2 * torch.randn(head_dim, generator=g, device=cuda)).to(dtype)
    cos, sin = rope_tables(shape, torch.arange(1000, 1000 + rows, device=cuda))
    if into_cache:  # rows 5..23 of [kv_heads, 40, D] caches, V copied too
        kc = torch.zeros((kh, 40, head_dim), dtype=dtype, device=cuda)
        vc = torch.zeros_like(kc)
        q, k = _qk_norm_rope(qkv, qw, kw, cos, sin, shape, k_out=kc[:, 5:5 + rows],
                             v_out=vc[:, 5:5 + rows])
    else:
        q, k = _qk_norm_rope(qkv, qw, kw, cos, sin, shape)
    torch.cuda.synchronize()

    def ref(x, w):  # [rows, H, D]: norm stored in dtype, then rotate-half RoPE
        n = _norm_ref(x, w).to(dtype).float()
        half = head_dim // 2
        rot = torch.cat([-n[..., half:], n[..., :half]], dim=-1)
        return (n * cos[:, None] + rot * sin[:, None]).to(dtype)

    qd, kd = qh * head_dim, kh * head_dim
    assert q.shape == (qh, rows, head_dim) and k.shape == (kh, rows, head_dim)
    _close(q.transpose(0, 1), ref(qkv[:, :qd].view(rows, qh, head_dim), qw))
    _close(k.transpose(0, 1), ref(qkv[:, qd:qd + kd].view(rows, kh, head_dim), kw))
    if into_cache:
        v = qkv[:, qd + kd:].view(rows, kh, head_dim).transpose(0, 1)
        assert torch.equal(vc[:, 5:5 + rows], v)
        assert torch.equal(kc[:, 5:5 + rows], k)
        # rows outside the written range are untouched
        assert not kc[:, :5].any() and not kc[:, 5 + rows:].any()
        assert not vc[:, :5].any() and not vc[:, 5 + rows:].any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,cols", [(33, 9728), (1, 8), (300, 136)])
def test_silu_mul(cuda, dtype, rows, cols):
    g = torch.Generator(device=cuda).manual_seed(cols)
    gu = (torch.randn((rows, 2 * cols), generator=g, device=cuda) * 4).to(dtype)
    out = _silu_mul(gu, cols)
    torch.cuda.synchronize()
    ref = (F.silu(gu[:, :cols].float()) * gu[:, cols:].float()).to(dtype)
    _close(out, ref)


def test_decoder_ops_reject_bad_shapes(cuda):
    x = torch.zeros((4, 12), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="multiple of 8"):
        _add_rms_norm(x, None, torch.ones(12, dtype=torch.bfloat16, device=cuda), EPS)
    with pytest.raises(ValueError, match="multiples of 8"):
        _silu_mul(torch.zeros((4, 24), dtype=torch.bfloat16, device=cuda), 12)
    shape = DecoderShape(query_heads=2, kv_heads=1, head_dim=64)
    cos, sin = rope_tables(shape, torch.arange(4, device=cuda))
    short = torch.zeros((4, 128), dtype=torch.bfloat16, device=cuda)  # q heads only
    w = torch.ones(64, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(ValueError, match="shorter"):
        _qk_norm_rope(short, w, w, cos, sin, shape)
