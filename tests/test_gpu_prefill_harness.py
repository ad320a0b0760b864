"""End-to-end prefill harness (fpv2.prefill_harness) on a tiny decoder.

The chunked GPU prefill (bf16, ChunkedPrefill per layer, strided Q/K/V views,
RoPE per chunk) is compared with a one-shot float32 CPU forward of the same
weights using full causal attention: dense and FPV2 (alpha 0.1) modes must
match it to bf16 accuracy, and FPV2 equals dense exactly when it selects every
block.  The request boundary (dense tail) follows the prompt length.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from fpv2 import FPV2Config
from fpv2.patch import _fpv2_sdpa
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


def _float32_forward_gpu(model: RandomDecoder, tokens: torch.Tensor, chunk: int) -> torch.Tensor:
    """Chunked float32 forward on the GPU with exact causal attention (plain
    torch float32 matmuls, one KV head at a time), last position's logits."""
    s, dev = model.shape, model.device
    L = tokens.numel()
    g = s.query_heads // s.kv_heads
    qd, kd, hd = s.query_heads * s.head_dim, s.kv_heads * s.head_dim, s.head_dim

    def norm(x, w):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + s.rms_eps) * w

    embed = model.embed.float()
    layers = [{k: v.float() for k, v in p.items()} for p in model.layers]
    kc = [torch.empty((s.kv_heads, L, hd), device=dev) for _ in layers]
    vc = [torch.empty((s.kv_heads, L, hd), device=dev) for _ in layers]
    x = None
    for start in range(0, L, chunk):
        end = min(start + chunk, L)
        n = end - start
        cos, sin = rope_tables(s, torch.arange(start, end, device=dev))

        def rope(t):  # [n, H, D]
            rot = torch.cat([-t[..., hd // 2:], t[..., :hd // 2]], dim=-1)
            return t * cos[:, None] + rot * sin[:, None]

        x = embed[tokens[start:end]]
        causal = torch.arange(end, device=dev)[None, :] > (start + torch.arange(n, device=dev))[:, None]
        for li, p in enumerate(layers):
            h = norm(x, p["attn_norm"])
            qkv = h @ p["qkv"].T
            q = rope(norm(qkv[:, :qd].view(n, s.query_heads, hd), p["q_norm"]))
            kc[li][:, start:end] = rope(norm(qkv[:, qd:qd + kd].view(n, s.kv_heads, hd),
                                             p["k_norm"])).transpose(0, 1)
            vc[li][:, start:end] = qkv[:, qd + kd:].view(n, s.kv_heads, hd).transpose(0, 1)
            att = torch.empty((n, s.query_heads, hd), device=dev)
            for kh in range(s.kv_heads):
                qh = q[:, kh * g:(kh + 1) * g].transpose(0, 1).reshape(g * n, hd)
                sc = (qh @ kc[li][kh, :end].T.contiguous()) * hd ** -0.5
                sc = sc.view(g, n, end).masked_fill_(causal[None], float("-inf"))
                pr = torch.softmax(sc, dim=-1).view(g * n, end)
                att[:, kh * g:(kh + 1) * g] = (pr @ vc[li][kh, :end]).view(g, n, hd).transpose(0, 1)
                del sc, pr
            x = x + att.reshape(n, qd) @ p["o"].T
            h = norm(x, p["mlp_norm"])
            gu = h @ p["gate_up"].T
            x = x + (torch.nn.functional.silu(gu[:, :s.intermediate]) * gu[:, s.intermediate:]) @ p["down"].T
    return (norm(x[-1:], model.final_norm.float()) @ embed.T)[0]


@pytest.mark.parametrize(("attention", "dtype"), [
    ("dense", torch.bfloat16), ("dense", torch.float16), ("fpv2", torch.bfloat16)])
def test_prefill_matches_float32_cpu(cuda, attention, dtype):
    """Chunked GPU prefill against the one-shot float32 CPU forward.  FPV2
    runs at alpha 0.1 (the configuration of the end-to-end bench); when every
    block is selected (random weights give near-uniform attention) its logits
    equal the dense runner's bit for bit."""
    model = RandomDecoder(SHAPE, device=cuda, seed=3, dtype=dtype)
    tokens = torch.randint(0, SHAPE.vocab, (1024,), generator=torch.Generator().manual_seed(4))
    runner = ChunkedPrefillRunner(model, 1024, attention=attention, min_tokens=1,
                                  config=FPV2Config(alpha=0.1, sink_tokens=128),
                                  collect_stats=True)
    got = runner.prefill(tokens.to(cuda), 256)
    ref = _cpu_forward(model, tokens)[0]
    rel = float((got.cpu() - ref).abs().max() / ref.abs().max())
    assert rel < 3e-2, rel
    if attention == "fpv2":
        dense = ChunkedPrefillRunner(model, 1024, attention="dense", min_tokens=1)
        want = dense.prefill(tokens.to(cuda), 256)
        torch.cuda.synchronize()
        if runner.block_sparsity() == 0.0:
            assert torch.equal(got, want)
        else:
            assert float((got - want).abs().max() / want.abs().max()) < 3e-2


def test_prompt_shorter_than_capacity_gets_the_dense_tail(cuda):
    """The request boundary is the prompt's length (``generate.py:101`` passes
    ``total_tokens=prompt_tokens``), not the cache capacity: a 768-token
    prompt in a 1024-token runner applies the dense tail on its last chunk,
    and that chunk's lists and output equal the hook on the same prefix."""
    model = RandomDecoder(SHAPE, device=cuda, seed=8)
    tokens = torch.randint(0, SHAPE.vocab, (768,), generator=torch.Generator().manual_seed(9))
    # alpha 2 selects no block on energy: only sink, window and dense tail
    config = FPV2Config(alpha=2.0, sink_tokens=128, window_tokens=128)
    runner = ChunkedPrefillRunner(model, 1024, attention="fpv2", config=config, min_tokens=1,
                                  collect_stats=True)
    runner.capture_layer = 1
    runner.prefill(tokens.to(cuda), 256)
    cap = runner.captured
    cache, keep = cap["cache"], cap["keep"]
    assert keep["config"].last_n_blocks == 2 and keep["offset"] == 512
    assert runner.block_sparsity() > 0  # pruned outside the forced blocks
    ids, counts, _, _ = keep["lists"]
    tq = keep["config"].tile_q
    nt = counts.shape[1]
    for t in (nt - 2, nt - 1):  # dense tail: every visible block selected
        visible = -(-(512 + (t + 1) * tq) // 128)
        assert bool((counts[:, t] == visible).all())
    q = cap["q"]
    k, v = cache.k[None, :, :768], cache.v[None, :, :768]
    hook = {}
    ref = _fpv2_sdpa(q[None], k, v, scale=SHAPE.head_dim ** -0.5, config=cache.config,
                     keep=hook)
    torch.cuda.synchronize()
    for a, b in zip(keep["lists"], hook["lists"]):
        assert torch.equal(a, b)
    assert torch.equal(cap["out"], ref[0])


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


def test_config5_full_qwen3_4b_prefill_65536(cuda):
    """BASELINE config 5 at full size: the random-init Qwen3-4B architecture
    (36 layers, hidden 2560, 32/8 heads, D 128, SwiGLU 9728, vocab 151936),
    65536 uniform-random token ids in 2048-token chunks, FPV2 (alpha 0.1, one
    sink block) in every layer, against dense (same kernels, every block) and
    the stock flash SDPA op.
      * FPV2 logits equal dense bit for bit when every block is selected,
        else within 0.1 of the largest logit;
      * against a float32 forward of the same weights on the GPU, FPV2's
        relative L2 and max-abs errors are at most 1.25x the stock op's (plus
        a small margin), and its top-1 is the float32 top-1 up to the stock
        op's max-abs error;
      * one layer (18) of the last chunk against the oracle on its full
        65536-key prefix: block lists outside the 1e-4 band and sampled
        attention rows within 2e-2 / 2e-3."""
    import numpy as np

    from conftest import attention_errors, to_np
    from oracle import fpv2_oracle as orc
    from fpv2.prefill_harness import QWEN3_4B

    tokens, chunk = 65536, 2048
    model = RandomDecoder(QWEN3_4B, device=cuda, seed=0)
    prompt = torch.randint(0, QWEN3_4B.vocab, (tokens,), device=cuda,
                           generator=torch.Generator(device=cuda).manual_seed(1))
    fpv2 = ChunkedPrefillRunner(model, tokens, attention="fpv2",
                                config=FPV2Config(alpha=0.1, sink_tokens=128),
                                collect_stats=True)
    fpv2.capture_layer = 18
    lf = fpv2.prefill(prompt, chunk)
    sparsity = fpv2.block_sparsity()
    cap = fpv2.captured
    keep, cache = cap["keep"], cap["cache"]
    cfg = keep["config"]
    assert cfg.last_n_blocks == 2 and keep["offset"] == tokens - chunk
    q = to_np(cap["q"])
    out = to_np(cap["out"])
    kn, vn = to_np(cache.k), to_np(cache.v)
    ids, counts, _, _ = keep["lists"]
    nb = ids.shape[-1]
    pooled_k, pooled_v = to_np(keep["pooled_k"]), to_np(keep["pooled_v"])
    lists = (to_np(ids), to_np(counts))
    del fpv2, cap
    torch.cuda.empty_cache()
    ld = ChunkedPrefillRunner(model, tokens, attention="dense").prefill(prompt, chunk)
    torch.cuda.empty_cache()
    ls = ChunkedPrefillRunner(model, tokens, attention="sdpa").prefill(prompt, chunk)
    torch.cuda.synchronize()
    if sparsity == 0.0:
        assert torch.equal(lf, ld)
    else:
        assert float((lf - ld).abs().max()) <= 0.1 * float(ld.abs().max())
    # Both bf16 paths against a float32 forward of the same weights: FPV2's
    # error must not exceed the stock op's by more than a small margin, and
    # its top-1 must be the float32 top-1 up to the stock path's error.
    l32 = _float32_forward_gpu(model, prompt, chunk)
    rel = lambda a: float((a - l32).norm() / l32.norm())  # noqa: E731
    stats = {"sparsity": sparsity, "rel_l2_fpv2": rel(lf), "rel_l2_stock": rel(ls),
             "max_abs_fpv2": float((lf - l32).abs().max()),
             "max_abs_stock": float((ls - l32).abs().max()),
             "top1_gap_fpv2": float(l32.max() - l32[int(lf.argmax())]),
             "top1_gap_stock": float(l32.max() - l32[int(ls.argmax())])}
    print(f"config 5 logits against float32: {stats}", flush=True)
    assert stats["rel_l2_fpv2"] <= 1.25 * stats["rel_l2_stock"] + 5e-3, stats
    assert stats["max_abs_fpv2"] <= 1.25 * stats["max_abs_stock"] + 0.05, stats
    assert stats["top1_gap_fpv2"] <= max(stats["max_abs_stock"], 0.05), stats

    ocfg = orc.OracleConfig(**{f: getattr(cfg, f) for f in orc.OracleConfig.__dataclass_fields__})
    tq, off = cfg.tile_q, tokens - chunk
    nt = chunk // tq
    for t0, n in ((0, 2), (nt // 2, 2), (nt - 3, 3)):
        sub = ocfg if t0 + n == nt else orc._replace(ocfg, last_n_blocks=0)
        rows0 = t0 * tq
        qs = q[:, rows0:rows0 + n * tq]
        dev_sel = np.zeros((ids.shape[0], n, nb), dtype=bool)
        for h in range(ids.shape[0]):
            for t in range(n):
                dev_sel[h, t, lists[0][h, t0 + t, :lists[1][h, t0 + t]]] = True
        sel, _, ratio = orc.block_scores_and_select(
            qs, pooled_k, scale=128 ** -0.5, config=orc._replace(sub, score_chunk_tiles=1),
            offset=off + rows0, query_length=n * tq, return_ratio=True)
        decided = np.abs(ratio - cfg.alpha) > 1e-4
        assert np.array_equal(sel[decided], dev_sel[decided]), t0
        ref = orc.fpv2_attention_blockwise(
            qs, kn, vn, scale=128 ** -0.5, selected=dev_sel, pooled_k=pooled_k,
            pooled_v=pooled_v, config=sub, offset=off + rows0, row_block=tq)
        err = attention_errors(out[:, rows0:rows0 + n * tq], ref)
        assert err["max_abs"] <= 2e-2 and err["mean_abs"] <= 2e-3, (t0, err)
