"""End-to-end chunked prefill of a random-init Qwen3-architecture decoder.

Measurement harness for the reference's end-to-end prefill comparison
(``README.md:30-46``, driven by ``fpv2/generate.py:49-130`` through mlx-lm):
the same decoder architecture with random weights (there is no network for
checkpoints), a prompt of uniform-random token ids fed in fixed-size chunks,
and attention either through FPV2 (``ChunkedPrefill`` per layer: incremental
pooling, selection, block-sparse attention), dense or stock.  Dense runs the
same kernels with every visible block selected (``alpha = 0``), which is exact
causal attention.  Stock (``"sdpa"``) is the platform's own fused attention:
PyTorch-ROCm's flash SDPA op, called directly so that torch's unfused batched
bf16 math path is never taken.

Architecture (Qwen3 as mlx-lm implements it): RMSNorm before attention and
MLP, per-head RMSNorm of Q and K, rotary embedding (rotate-half, theta 1e6),
grouped-query attention, SwiGLU MLP, final RMSNorm, tied LM head.  Linear
layers are plain 2-D GEMMs (``torch.nn.functional.linear``); the residual add
+ RMSNorm, the per-head Q/K RMSNorm + RoPE and the SwiGLU gate are fused HIP
kernels of the same library (``include/fpv2_decoder.h``), computing in float32
and storing bf16.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from fpv2 import _lib
from fpv2.chunked import ChunkedPrefill
from fpv2.selection import FPV2Config


@dataclass(frozen=True)
class DecoderShape:
    layers: int = 36
    hidden: int = 2560
    query_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    vocab: int = 151936
    rope_theta: float = 1e6
    rms_eps: float = 1e-6


QWEN3_4B = DecoderShape()


def _rows(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    """The decoder kernels take 2-D row-major operands (any row stride)."""
    if t.ndim != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with contiguous rows")
    if t.dtype != dtype:
        raise ValueError(f"{name} must have dtype {dtype}")


def _vector(t: torch.Tensor, name: str, n: int, dtype: torch.dtype) -> None:
    if t.ndim != 1 or t.numel() != n or not t.is_contiguous() or t.dtype != dtype:
        raise ValueError(f"{name} must be a contiguous [{n}] vector of dtype {dtype}")


def _add_rms_norm(x: torch.Tensor, delta: torch.Tensor | None, weight: torch.Tensor,
                  eps: float) -> torch.Tensor:
    """``x += delta`` in place (when given), then RMSNorm of ``x``'s rows
    (``fpv2_add_rms_norm``)."""
    lib = _lib.load()
    _rows(x, "x", x.dtype)
    _vector(weight, "weight", x.shape[1], x.dtype)
    if delta is not None:
        _rows(delta, "delta", x.dtype)
        if delta.shape != x.shape:
            raise ValueError("delta must have x's shape")
    _lib.require_device(x, weight, *(() if delta is None else (delta,)))
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.check(lib.fpv2_add_rms_norm(
        x.data_ptr(), _lib.ptr(delta), weight.data_ptr(), y.data_ptr(), _lib.dtype_code(x.dtype),
        x.shape[0], x.shape[1], x.stride(0), delta.stride(0) if delta is not None else 0,
        y.stride(0), eps, _lib.stream_ptr(x.device)), "fpv2_add_rms_norm")
    return y


def _qk_norm_rope(qkv: torch.Tensor, q_weight, k_weight, cos, sin, shape, *,
                  k_out: torch.Tensor | None = None,
                  v_out: torch.Tensor | None = None) -> tuple:
    """Per-head RMSNorm + RoPE of the q and k heads of fused projection rows
    (``fpv2_qk_norm_rope``).  Returns ``q`` ``[Hq, L, D]`` (a view of an
    ``[L, Hq, D]`` buffer) and ``k`` ``[Hkv, L, D]``, written into ``k_out``
    when given (any head/row stride, e.g. rows of a KV cache).  ``v_out``
    (``[Hkv, L, D]``), when given, receives a copy of the value heads."""
    lib = _lib.load()
    L, s = qkv.shape[0], shape
    _rows(qkv, "qkv", qkv.dtype)
    heads = s.query_heads + s.kv_heads * (2 if v_out is not None else 1)
    if qkv.shape[1] < heads * s.head_dim:
        raise ValueError("qkv rows are shorter than the heads read")
    _vector(q_weight, "q_weight", s.head_dim, qkv.dtype)
    _vector(k_weight, "k_weight", s.head_dim, qkv.dtype)
    for name, table in (("cos", cos), ("sin", sin)):
        if table.shape != (L, s.head_dim) or not table.is_contiguous() or table.dtype != torch.float32:
            raise ValueError(f"{name} must be a contiguous float32 [{L}, {s.head_dim}] table")
    if k_out is None:
        k_out = torch.empty((L, s.kv_heads, s.head_dim), dtype=qkv.dtype,
                            device=qkv.device).transpose(0, 1)
    for name, t in (("k_out", k_out), ("v_out", v_out)):
        if t is not None and (t.shape != (s.kv_heads, L, s.head_dim) or t.stride(-1) != 1
                              or t.dtype != qkv.dtype):
            raise ValueError(f"{name} must be [{s.kv_heads}, {L}, {s.head_dim}] of qkv's dtype "
                             "with a contiguous last dimension")
    if v_out is not None and v_out.stride()[:2] != k_out.stride()[:2]:
        raise ValueError("k_out and v_out must share strides")
    _lib.require_device(qkv, q_weight, k_weight, cos, sin, k_out,
                        *(() if v_out is None else (v_out,)))
    q = torch.empty((L, s.query_heads, s.head_dim), dtype=qkv.dtype, device=qkv.device)
    _lib.check(lib.fpv2_qk_norm_rope(
        qkv.data_ptr(), q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        q.data_ptr(), k_out.data_ptr(), _lib.ptr(v_out), _lib.dtype_code(qkv.dtype), L,
        s.query_heads, s.kv_heads, s.head_dim, qkv.stride(0), q.stride(1), q.stride(0),
        k_out.stride(0), k_out.stride(1), s.rms_eps, _lib.stream_ptr(qkv.device)),
        "fpv2_qk_norm_rope")
    return q.transpose(0, 1), k_out


def _silu_mul(gate_up: torch.Tensor, cols: int) -> torch.Tensor:
    """``silu(gate) * up`` of ``gate_up = [gate | up]`` rows (``fpv2_silu_mul``)."""
    lib = _lib.load()
    _rows(gate_up, "gate_up", gate_up.dtype)
    if gate_up.shape[1] < 2 * cols:
        raise ValueError("gate_up rows must hold 2 * cols elements")
    _lib.require_device(gate_up)
    out = torch.empty((gate_up.shape[0], cols), dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(lib.fpv2_silu_mul(
        gate_up.data_ptr(), out.data_ptr(), _lib.dtype_code(gate_up.dtype), gate_up.shape[0],
        cols, gate_up.stride(0), out.stride(0), _lib.stream_ptr(gate_up.device)),
        "fpv2_silu_mul")
    return out


def rope_tables(shape: DecoderShape, positions: torch.Tensor):
    """cos/sin ``[L, D]`` of rotate-half RoPE for integer positions."""
    half = shape.head_dim // 2
    inv = shape.rope_theta ** (-torch.arange(half, device=positions.device, dtype=torch.float64) / half)
    ang = positions.to(torch.float64)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().float(), ang.sin().float()


class RandomDecoder:
    """Random-init decoder weights (normal, std 0.02; norms at 1)."""

    def __init__(self, shape: DecoderShape, *, device, dtype=torch.bfloat16, seed: int = 0):
        self.shape, self.device, self.dtype = shape, torch.device(device), dtype
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def w(*dims):
            return (torch.randn(dims, generator=gen, device=self.device, dtype=torch.float32)
                    * 0.02).to(dtype)

        s = shape
        qd, kd = s.query_heads * s.head_dim, s.kv_heads * s.head_dim
        self.embed = w(s.vocab, s.hidden)
        self.layers = []
        for _ in range(s.layers):
            self.layers.append({
                "attn_norm": torch.ones(s.hidden, device=self.device, dtype=dtype),
                "qkv": w(qd + 2 * kd, s.hidden),  # fused q/k/v projection
                "q_norm": torch.ones(s.head_dim, device=self.device, dtype=dtype),
                "k_norm": torch.ones(s.head_dim, device=self.device, dtype=dtype),
                "o": w(s.hidden, qd),
                "mlp_norm": torch.ones(s.hidden, device=self.device, dtype=dtype),
                "gate_up": w(2 * s.intermediate, s.hidden),
                "down": w(s.hidden, s.intermediate),
            })
        self.final_norm = torch.ones(s.hidden, device=self.device, dtype=dtype)

    def parameters(self) -> int:
        n = self.embed.numel() + self.final_norm.numel()
        for layer in self.layers:
            n += sum(t.numel() for t in layer.values())
        return n


class _StockAttention:
    """One layer's KV cache attended by torch's fused SDPA kernel (the flash
    kernel of the PyTorch-ROCm build): the stock dense path that FPV2 replaces.

    The flash op's causal mask is aligned to the last key when there are fewer
    queries than keys (each chunk's queries are the last positions of the
    prefix).  It takes as many K/V heads as query heads, so the cache stores
    every KV head once per query head of its group (each chunk is expanded
    once, when appended).  Only that op is called: torch's generic SDPA front
    end could fall back to its unfused math path."""

    def __init__(self, query_heads: int, kv_heads: int, head_dim: int, capacity: int, *,
                 dtype, device):
        self.query_heads, self.kv_heads = query_heads, kv_heads
        self.k = torch.empty((query_heads, capacity, head_dim), dtype=dtype, device=device)
        self.v = torch.empty_like(self.k)
        self.capacity, self.length = capacity, 0

    def reset(self) -> None:
        self.length = 0

    def step(self, q, k, v, *, scale: float, out: torch.Tensor) -> None:
        """q ``[Hq, L, D]``, k/v ``[Hkv, L, D]``; writes ``out`` ``[Hq, L, D]``."""
        n, d = k.shape[1], k.shape[2]
        if self.length + n > self.capacity:
            raise ValueError("the KV cache capacity is exceeded")
        g, hk = self.query_heads // self.kv_heads, self.kv_heads
        a, b = self.length, self.length + n
        self.k[:, a:b].view(hk, g, n, d).copy_(k[:, None].expand(hk, g, n, d))
        self.v[:, a:b].view(hk, g, n, d).copy_(v[:, None].expand(hk, g, n, d))
        self.length = b
        o = torch.ops.aten._scaled_dot_product_flash_attention(
            q.contiguous()[None], self.k[None, :, :b], self.v[None, :, :b], 0.0, is_causal=True,
            return_debug_mask=False, scale=scale)[0]
        out.copy_(o[0])


class ChunkedPrefillRunner:
    """Chunked prefill of one prompt through a ``RandomDecoder``.

    ``attention``: ``"fpv2"`` (FPV2 with ``config``), ``"dense"`` (same
    kernels, every visible block) or ``"sdpa"`` (torch's fused flash SDPA
    kernel, the stock dense path).  ``min_tokens`` is the hook's gate: calls
    with fewer keys attend densely in both modes.  ``collect_stats`` counts
    selected and visible blocks in every layer (``block_sparsity``).
    Setting ``capture_layer`` to a layer index keeps that layer's last
    attention call in ``captured``: its queries, output, cache and block
    lists (for checking one layer of a full prefill against the oracle).
    """

    def __init__(self, model: RandomDecoder, capacity: int, *, attention: str = "fpv2",
                 config: FPV2Config | None = None, min_tokens: int = 4_096,
                 collect_stats: bool = False):
        if attention not in ("fpv2", "dense", "sdpa"):
            raise ValueError("attention must be 'fpv2', 'dense' or 'sdpa'")
        s = model.shape
        base = config if config is not None else FPV2Config()
        if attention == "dense":
            base = FPV2Config(alpha=0.0, block_k=base.block_k, tile_q=base.tile_q,
                              sink_tokens=base.sink_tokens, window_tokens=base.window_tokens,
                              last_n_blocks=base.last_n_blocks,
                              mean_correction=base.mean_correction)
        self.model, self.capacity, self.attention = model, capacity, attention
        self.capture_layer: int | None = None
        self.captured: dict | None = None
        if attention == "sdpa":
            self.caches = [_StockAttention(s.query_heads, s.kv_heads, s.head_dim, capacity,
                                           dtype=model.dtype, device=model.device)
                           for _ in range(s.layers)]
            return
        self.caches = [ChunkedPrefill(s.query_heads, s.kv_heads, s.head_dim, capacity,
                                      dtype=model.dtype, device=model.device, config=base,
                                      total_tokens=capacity, min_tokens=min_tokens,
                                      collect_stats=collect_stats)
                       for _ in range(s.layers)]

    def reset(self) -> None:
        for cache in self.caches:
            cache.reset()

    def block_sparsity(self) -> float:
        """Fraction of visible causal blocks skipped over all layers since
        the last ``reset`` (needs ``collect_stats``; 0 for ``"sdpa"``)."""
        if self.attention == "sdpa":
            return 0.0
        visible = sum(c._visible for c in self.caches)
        if not visible:
            return 0.0
        totals = [t for t in (c._selected.device_total() for c in self.caches) if t is not None]
        selected = int(torch.stack(totals).sum().item()) if totals else 0  # one synchronisation
        return 1.0 - selected / visible

    def _layer(self, li: int, x: torch.Tensor, delta: torch.Tensor | None, cos, sin):
        """One decoder layer.  The residual stream is ``x + delta``: the add is
        fused into the next RMSNorm.  Returns the new ``(x, delta)``."""
        s, p = self.model.shape, self.model.layers[li]
        L = x.shape[0]
        qd, kd = s.query_heads * s.head_dim, s.kv_heads * s.head_dim
        h = _add_rms_norm(x, delta, p["attn_norm"], s.rms_eps)
        qkv = F.linear(h, p["qkv"])
        cache = self.caches[li]
        # the attention output lands as [L, Hq * D], the layout the output
        # projection reads (the kernels write any head/row stride)
        attn = torch.empty((L, qd), dtype=x.dtype, device=x.device)
        attn_heads = attn.view(L, s.query_heads, s.head_dim).transpose(0, 1)
        if self.attention == "sdpa":
            q, k = _qk_norm_rope(qkv, p["q_norm"], p["k_norm"], cos, sin, s)
            v = qkv[:, qd + kd:].view(L, s.kv_heads, s.head_dim).transpose(0, 1)
            cache.step(q, k, v, scale=s.head_dim ** -0.5, out=attn_heads)
        else:
            # K (normalised, rotated) and V go straight into the layer's cache
            k_rows, v_rows = cache.reserve(L)
            q, _ = _qk_norm_rope(qkv, p["q_norm"], p["k_norm"], cos, sin, s,
                                 k_out=k_rows, v_out=v_rows)
            keep = {} if li == self.capture_layer else None
            cache.attend(q, scale=s.head_dim ** -0.5, out=attn_heads, keep=keep)
            if keep is not None:
                self.captured = {"q": q, "out": attn_heads, "cache": cache, "keep": keep}
        h = _add_rms_norm(x, F.linear(attn, p["o"]), p["mlp_norm"], s.rms_eps)
        act = _silu_mul(F.linear(h, p["gate_up"]), s.intermediate)
        return x, F.linear(act, p["down"])

    def prefill(self, tokens: torch.Tensor, chunk: int) -> torch.Tensor:
        """Run the prompt in ``chunk``-token pieces; returns the logits of the
        last position (float32 ``[vocab]``)."""
        m = self.model
        n = tokens.numel()
        if n > self.capacity:
            raise ValueError("prompt longer than the KV cache capacity")
        if self.attention != "sdpa":
            # the request boundary is this prompt's length, not the cache
            # capacity (generate.py:101 passes total_tokens=prompt_tokens):
            # the dense tail applies on the chunk that reaches it
            for cache in self.caches:
                cache.total_tokens = n
        x = delta = None
        for start in range(0, n, chunk):
            end = min(start + chunk, n)
            pos = torch.arange(start, end, device=m.device)
            cos, sin = rope_tables(m.shape, pos)
            x, delta = m.embed[tokens[start:end]], None
            for li in range(m.shape.layers):
                x, delta = self._layer(li, x, delta, cos, sin)
        last = _add_rms_norm(x[-1:], delta[-1:], m.final_norm, m.shape.rms_eps)
        return F.linear(last, m.embed).float()[0]


def measure(shape: DecoderShape, *, tokens: int, chunk: int, alpha: float, device,
            seed: int = 0, modes=("fpv2", "dense", "sdpa"), reps: int = 1) -> dict:
    """Prefill tok/s and time to first token (prefill + first logits) per mode."""
    model = RandomDecoder(shape, device=device, seed=seed)
    gen = torch.Generator(device=model.device).manual_seed(seed + 1)
    prompt = torch.randint(0, shape.vocab, (tokens,), generator=gen, device=model.device)
    res = {"parameters": model.parameters(), "tokens": tokens, "chunk": chunk, "alpha": alpha}
    logits = {}
    for mode in modes:
        runner = ChunkedPrefillRunner(model, tokens, attention=mode,
                                      config=FPV2Config(alpha=alpha, sink_tokens=128),
                                      collect_stats=mode == "fpv2")
        runner.prefill(prompt[:min(tokens, 2 * chunk)], chunk)  # warm-up
        best = math.inf
        for _ in range(reps):
            runner.reset()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = runner.prefill(prompt, chunk)
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        logits[mode] = out
        res[mode] = {"ttft_s": best, "prefill_tok_per_s": tokens / best}
        if mode == "fpv2":  # over every layer and chunk of the timed prefills
            res[mode]["block_sparsity"] = runner.block_sparsity()
        del runner
        torch.cuda.empty_cache()
    if "fpv2" in logits and "dense" in logits:
        a, b = logits["fpv2"], logits["dense"]
        res["logits_max_abs_diff"] = float((a - b).abs().max())
        res["top1_agree"] = bool(int(a.argmax()) == int(b.argmax()))
        res["speedup"] = res["dense"]["ttft_s"] / res["fpv2"]["ttft_s"]
    if "fpv2" in logits and "sdpa" in logits:
        a, b = logits["fpv2"], logits["sdpa"]
        res["sdpa_logits_max_abs_diff"] = float((a - b).abs().max())
        res["sdpa_top1_agree"] = bool(int(a.argmax()) == int(b.argmax()))
        res["speedup_vs_sdpa"] = res["sdpa"]["ttft_s"] / res["fpv2"]["ttft_s"]
    return res
