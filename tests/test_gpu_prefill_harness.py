"""End-to-end prefill harness (fpv2.prefill_harness) on a tiny decoder.

The chunked GPU prefill (bf16, ChunkedPrefill per layer, strided Q/K/V views,
RoPE per chunk) is compared with a one-shot float32 CPU forward of the same
weights using full causal attention: dense mode must match it to bf16
accuracy, and FPV2 mode with alpha = 0 must equal dense exactly.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from fpv2 import FPV2Config
from fpv2.prefill_harness import ChunkedPrefillRunner, DecoderShape, RandomDecoder, rope_tables

pytestmark = pytest.mark.gpu

SHAPE = DecoderShape(layers=2, hidden=256, query_heads=8, kv_heads=2, head_dim=128,
                     intermediate=512, vocab=512)


def _cpu_forward(model: RandomDecoder, tokens: torch.Tensor) -> torch.Tensor:
    """Full-sequence float32 forward on the CPU with exact causal attention."""
    s = model.shape
    f32 = lambda t: t.detach().float().cpu()  # noqa: E731
    tok = tokens.cpu()
    L = tok.numel()
    cos, sin = rope_tables(s, torch.arange(L))

    def norm(x, w):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + s.rms_eps) * w

    def rope(x):  # [L, H, D]
        half = s.head_dim // 2
        rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
        return x * cos[:, None] + rot * sin[:, None]

    x = f32(model.embed)[tok]
    qd, kd = s.query_heads * s.head_dim, s.kv_heads * s.head_dim
    g = s.query_heads // s.kv_heads
    for p in model.layers:
        p = {k: f32(v) for k, v in p.items()}
        h = norm(x, p["attn_norm"])
        qkv = h @ p["qkv"].T
        q = rope(norm(qkv[:, :qd].view(L, s.query_heads, s.head_dim), p["q_norm"]))
        k = rope(norm(qkv[:, qd:qd + kd].view(L, s.kv_heads, s.head_dim), p["k_norm"]))
        v = qkv[:, qd + kd:].view(L, s.kv_heads, s.head_dim)
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
        att = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1),
                                             v.transpose(0, 1), is_causal=True)
        x = x + att.transpose(0, 1).reshape(L, qd) @ p["o"].T
        h = norm(x, p["mlp_norm"])
        gu = h @ p["gate_up"].T
        x = x + (F.silu(gu[:, :s.intermediate]) * gu[:, s.intermediate:]) @ p["down"].T
    return norm(x[-1:], f32(model.final_norm)) @ f32(model.embed).T


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dense_prefill_matches_float32_cpu(cuda, dtype):
    model = RandomDecoder(SHAPE, device=cuda, seed=3, dtype=dtype)
    tokens = torch.randint(0, SHAPE.vocab, (1024,), generator=torch.Generator().manual_seed(4))
    runner = ChunkedPrefillRunner(model, 1024, attention="dense", min_tokens=1)
    got = runner.prefill(tokens.to(cuda), 256).cpu()
    ref = _cpu_forward(model, tokens)[0]
    rel = float((got - ref).abs().max() / ref.abs().max())
    assert rel < 3e-2, rel


def test_fpv2_alpha_zero_equals_dense(cuda):
    model = RandomDecoder(SHAPE, device=cuda, seed=5)
    tokens = torch.randint(0, SHAPE.vocab, (1024,), generator=torch.Generator().manual_seed(6)).to(cuda)
    dense = ChunkedPrefillRunner(model, 1024, attention="dense", min_tokens=1).prefill(tokens, 256)
    fpv2 = ChunkedPrefillRunner(model, 1024, attention="fpv2", config=FPV2Config(alpha=0.0),
                                min_tokens=1).prefill(tokens, 256)
    torch.cuda.synchronize()
    assert torch.equal(dense, fpv2)


def test_runner_rejects_bad_arguments(cuda):
    model = RandomDecoder(SHAPE, device=cuda, seed=7)
    with pytest.raises(ValueError, match="attention"):
        ChunkedPrefillRunner(model, 256, attention="sparse")
    runner = ChunkedPrefillRunner(model, 256)
    with pytest.raises(ValueError, match="capacity"):
        runner.prefill(torch.zeros(512, dtype=torch.long, device=cuda), 256)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stock_sdpa_prefill_matches_float32_cpu(cuda, dtype):
    """The stock comparison path (torch's flash SDPA op, chunk queries aligned
    to the last keys of the prefix) is exact causal attention too."""
    model = RandomDecoder(SHAPE, device=cuda, seed=3, dtype=dtype)
    tokens = torch.randint(0, SHAPE.vocab, (1024,), generator=torch.Generator().manual_seed(4))
    runner = ChunkedPrefillRunner(model, 1024, attention="sdpa")
    got = runner.prefill(tokens.to(cuda), 256).cpu()
    ref = _cpu_forward(model, tokens)[0]
    rel = float((got - ref).abs().max() / ref.abs().max())
    assert rel < 3e-2, rel


def test_stock_attention_aligns_chunk_queries_to_the_last_keys(cuda):
    from fpv2.prefill_harness import _StockAttention
    hq, hk, d = 8, 2, 128
    g = torch.Generator().manual_seed(11)
    q = torch.randn((hq, 768, d), generator=g).bfloat16()
    k = torch.randn((hk, 768, d), generator=g).bfloat16()
    v = torch.randn((hk, 768, d), generator=g).bfloat16()
    layer = _StockAttention(hq, hk, d, 768, dtype=torch.bfloat16, device=cuda)
    out = torch.empty((hq, 256, d), dtype=torch.bfloat16, device=cuda)
    for start, end in ((0, 512), (512, 768)):
        o = torch.empty((hq, end - start, d), dtype=torch.bfloat16, device=cuda)
        layer.step(q[:, start:end].to(cuda), k[:, start:end].to(cuda), v[:, start:end].to(cuda),
                   scale=d ** -0.5, out=o)
    out = o.cpu().float()
    # float32 reference of the second chunk: query i sits at position 512 + i
    kf = k.float().repeat_interleave(hq // hk, dim=0)
    vf = v.float().repeat_interleave(hq // hk, dim=0)
    s = q[:, 512:].float() @ kf.transpose(1, 2) * d ** -0.5
    pos = torch.arange(512, 768)[:, None]
    s = s.masked_fill(torch.arange(768)[None, :] > pos, float("-inf"))
    ref = torch.softmax(s, dim=-1) @ vf
    assert float((out - ref).abs().max()) < 2e-2
