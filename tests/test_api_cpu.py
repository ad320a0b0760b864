"""Host-side behaviour of the product package (no GPU needed).

Validation messages follow the reference's tests (``tests/test_selection.py``,
``tests/test_kernel.py``, ``tests/test_patch.py``); the hook must pass every
ineligible call (here: CPU tensors, array masks, decode shapes) to torch's
original SDPA unchanged; the C-ABI library must load and export every symbol
``include/fpv2.h`` declares; and compute entry points must refuse non-GPU
tensors instead of falling back.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import fpv2
from fpv2 import FPV2Config, block_sparsity, disable, enable, pool_blocks
from fpv2 import _lib
from fpv2.kernel import (TileConfig, compact_block_indices, default_tile, sparse_attention,
                         _tile_for_config)
from fpv2.patch import _ORIGINAL_SDPA, _effective_config, _request_config
from fpv2.selection import block_scores_and_select, density

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(autouse=True)
def restore_sdpa():
    disable()
    yield
    disable()


# ---- FPV2Config (selection.py:30-65) -------------------------------------

@pytest.mark.parametrize("value", [0, -1, 1.5, True])
def test_score_chunk_tiles_must_be_a_positive_integer(value):
    with pytest.raises(ValueError, match="score_chunk_tiles"):
        FPV2Config(score_chunk_tiles=value)


def test_pack_gqa_must_be_boolean():
    with pytest.raises(ValueError, match="pack_gqa"):
        FPV2Config(pack_gqa=1)


@pytest.mark.parametrize("value", [-1, 1.5, True])
def test_last_n_blocks_must_be_a_non_negative_integer(value):
    with pytest.raises(ValueError, match="last_n_blocks"):
        FPV2Config(last_n_blocks=value)


def test_config_defaults_and_other_rules():
    c = FPV2Config()
    assert (c.block_k, c.tile_q, c.alpha, c.sink_tokens, c.window_tokens, c.last_n_blocks,
            c.mean_correction, c.score_chunk_tiles, c.pack_gqa) == (
        128, 128, 0.1, 256, 384, 2, True, None, False)
    with pytest.raises(ValueError, match="positive"):
        FPV2Config(block_k=0)
    with pytest.raises(ValueError, match="alpha"):
        FPV2Config(alpha=-0.1)
    with pytest.raises(ValueError, match="non-negative"):
        FPV2Config(window_tokens=-1)


# ---- validation before any device work ----------------------------------

def test_pool_blocks_rejects_unaligned_length():
    with pytest.raises(ValueError, match="divisible"):
        pool_blocks(torch.zeros((2, 7, 4)), 4)


def test_compaction_rejects_non_boolean_mask():
    with pytest.raises(ValueError, match="boolean"):
        compact_block_indices(torch.ones((1, 1, 1), dtype=torch.int32))


def test_selection_input_validation():
    cfg = FPV2Config(block_k=16, tile_q=16)
    with pytest.raises(ValueError, match="divisible by KV heads"):
        block_scores_and_select(torch.zeros(3, 16, 8), torch.zeros(2, 1, 8), scale=1.0, config=cfg)
    with pytest.raises(ValueError, match="padded to a multiple of tile_q"):
        block_scores_and_select(torch.zeros(2, 15, 8), torch.zeros(2, 1, 8), scale=1.0, config=cfg)
    with pytest.raises(ValueError, match="beyond the represented key sequence"):
        block_scores_and_select(torch.zeros(2, 32, 8), torch.zeros(2, 1, 8), scale=1.0, config=cfg)


def test_sparse_attention_validation():
    cfg = FPV2Config(block_k=16, tile_q=16)
    q = torch.zeros(4, 32, 64, dtype=torch.bfloat16)
    k = torch.zeros(2, 32, 64, dtype=torch.bfloat16)
    ids = torch.zeros(2, 2, 2, dtype=torch.int32)
    cnt = torch.zeros(2, 2, dtype=torch.int32)
    pk = torch.zeros(2, 2, 64)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        sparse_attention(q.float(), k.float(), k.float(), pk, pk, ids, cnt, ids, cnt,
                         scale=1.0, config=cfg)
    with pytest.raises(ValueError, match="head dimension"):
        sparse_attention(q[..., :48], k[..., :48], k[..., :48], pk, pk, ids, cnt, ids, cnt,
                         scale=1.0, config=cfg)
    with pytest.raises(ValueError, match="int32"):
        sparse_attention(q, k, k, pk, pk, ids.long(), cnt, ids, cnt, scale=1.0, config=cfg)
    with pytest.raises(ValueError, match="block lists must have shape"):
        sparse_attention(q, k, k, pk, pk, ids[:, :1], cnt, ids, cnt, scale=1.0, config=cfg)
    q6 = torch.zeros(6, 32, 64, dtype=torch.bfloat16)  # G = 3 does not divide bq = 16
    with pytest.raises(ValueError, match="PackGQA"):
        sparse_attention(q6, k, k, pk, pk, ids, cnt, ids, cnt, scale=1.0, config=cfg,
                         pack_gqa=True)


def test_compute_entry_points_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match="ROCm"):
        pool_blocks(torch.zeros(2, 8, 4), 4)
    with pytest.raises(RuntimeError, match="ROCm"):
        compact_block_indices(torch.zeros(1, 1, 2, dtype=torch.bool),
                              config=FPV2Config(block_k=16, tile_q=16))


def test_density_on_host_mask():
    cfg = FPV2Config(block_k=4, tile_q=4)
    sel = torch.zeros(2, 4, 4, dtype=torch.bool)
    sel[:, torch.arange(4), torch.arange(4)] = True
    assert density(sel, config=cfg).item() == pytest.approx(0.4)


# ---- tiles (kernel.py:30-88) ----------------------------------------------

def test_default_tile_dispatch():
    assert default_tile(64) == TileConfig(32, 32, 4)
    assert default_tile(96) == TileConfig(32, 32, 4)
    assert default_tile(128) == TileConfig(64, 32, 8)
    assert default_tile(256) == TileConfig(32, 16, 4)
    with pytest.raises(ValueError, match="head dimension"):
        default_tile(80)


def test_tile_fallback_for_hook_tile():
    # The hook's 32-position tile falls back to (32, 16, 4) (kernel.py:76-88).
    assert _tile_for_config(128, FPV2Config(tile_q=32)) == TileConfig(32, 16, 4)
    # tiles of fewer than 8 positions (GQA groups of 32) resolve too: the
    # gfx950 kernel takes any tile_q
    assert _tile_for_config(128, FPV2Config(tile_q=4)) == TileConfig(4, 16, 1)
    assert _tile_for_config(64, FPV2Config(tile_q=12, block_k=20)) == TileConfig(12, 16, 1)


def test_tile_check_is_well_formedness_only():
    """A tile changes neither the gfx950 launch nor the output: only positive
    integer dimensions and a supported head dimension are required (the
    reference's Apple threadgroup-memory rule is not applied)."""
    TileConfig(64, 64, 8).check(256, block_k=128, tile_q=128)
    TileConfig(64, 32, 4).check(128, block_k=128, tile_q=32)
    for bad in (TileConfig(0, 32, 4), TileConfig(32, -1, 4), TileConfig(32, 32, True),
                TileConfig(32, 32.0, 4)):
        with pytest.raises(ValueError, match="positive"):
            bad.check(128)
    with pytest.raises(ValueError, match="head dimension"):
        TileConfig(32, 32, 4).check(80)


# ---- hook helpers (patch.py:41-63) -----------------------------------------

def test_default_tile_uses_128_packed_gqa_rows():
    effective = _effective_config(FPV2Config(), query_heads=32, kv_heads=8)
    assert effective is not None and effective.tile_q == 32
    custom = FPV2Config(tile_q=64)
    assert _effective_config(custom, query_heads=32, kv_heads=8) is custom


def test_dense_tail_is_applied_only_at_known_request_end():
    config = FPV2Config(last_n_blocks=2)
    assert _request_config(config, 2_048, 8_192).last_n_blocks == 0
    assert _request_config(config, 8_192, 8_192) is config
    assert _request_config(config, 8_192, None).last_n_blocks == 0


@pytest.mark.parametrize("value", [0, -1, 1.5, True])
def test_total_tokens_must_be_a_positive_integer(value):
    with pytest.raises(ValueError, match="total_tokens"):
        enable(total_tokens=value)


def test_enable_disable_swap_torch_sdpa():
    assert F.scaled_dot_product_attention is _ORIGINAL_SDPA
    enable(min_tokens=1)
    assert fpv2.is_enabled() and F.scaled_dot_product_attention is not _ORIGINAL_SDPA
    disable()
    assert not fpv2.is_enabled() and F.scaled_dot_product_attention is _ORIGINAL_SDPA


def _inputs(length, query_length=None, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(7)
    query_length = length if query_length is None else query_length
    q = torch.randn((1, 4, query_length, 64), generator=g).to(dtype)
    k = torch.randn((1, 2, length, 64), generator=g).to(dtype)
    v = torch.randn((1, 2, length, 64), generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize(("length", "query_length", "causal"),
                         [(64, 64, True), (128, 1, True), (128, 32, True), (128, 128, False),
                          (256, 256, True)])
def test_ineligible_cpu_calls_are_bit_identical(length, query_length, causal):
    q, k, v = _inputs(length, query_length)
    expected = _ORIGINAL_SDPA(q, k, v, is_causal=causal, enable_gqa=True)
    enable(min_tokens=128, collect_stats=True)
    actual = F.scaled_dot_product_attention(q, k, v, is_causal=causal, enable_gqa=True)
    assert torch.equal(actual, expected)


def test_array_mask_falls_through_and_disable_restores_original():
    q, k, v = _inputs(128)
    mask = torch.zeros((128, 128), dtype=torch.bfloat16)
    expected = _ORIGINAL_SDPA(q, k, v, attn_mask=mask, enable_gqa=True)
    enable(min_tokens=1)
    actual = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
    assert torch.equal(actual, expected)
    disable()
    assert F.scaled_dot_product_attention is _ORIGINAL_SDPA


def test_block_sparsity_starts_at_zero():
    enable(min_tokens=1, collect_stats=True)
    assert block_sparsity() == 0.0


# ---- C ABI -----------------------------------------------------------------

def _declared_symbols() -> set[str]:
    text = "\n".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(fpv2_\w+)\s*\(", text, re.M))


def test_header_declares_the_bound_symbols():
    assert _declared_symbols() == set(_lib.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfpv2_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    loaded = _lib.load()
    assert loaded.fpv2_abi_version() == _lib.ABI_VERSION


def test_abi_struct_layouts_match_header(tmp_path):
    """ctypes mirrors of fpv2_select_params / fpv2_attn_params match the C
    header field by field (offsets and sizes, as compiled by gcc)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    include = Path(__file__).resolve().parents[1] / "include"
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "fpv2.h"', "int main(void) {"]
    for cname, cls in (("fpv2_select_params", _lib.SelectParams),
                       ("fpv2_attn_params", _lib.AttnParams)):
        lines.append(f'  printf("{cls.__name__} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cls.__name__} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-I", str(include), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    for line in out.splitlines():
        cls_name, field, value = line.split()
        cls = getattr(_lib, cls_name)
        expected = ctypes.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert int(value) == expected, line


def test_library_rejects_bad_arguments_without_a_gpu():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfpv2_hip.so not built")
    lib = _lib.load()
    status = lib.fpv2_pool_blocks(None, None, _lib.BF16, 1, 8, 1, 8, 8, 64, 8, 64, None)
    assert status == _lib.FPV2_ERR_ARGUMENT
    assert b"null" in lib.fpv2_last_error()
    params = _lib.AttnParams(query_heads=3, kv_heads=2)
    status = lib.fpv2_sparse_attention(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, _lib.BF16, params, None)
    assert status == _lib.FPV2_ERR_ARGUMENT


def test_chunked_prefill_validation_without_a_gpu():
    from fpv2 import ChunkedPrefill
    with pytest.raises(ValueError, match="divisible"):
        ChunkedPrefill(8, 3, 128, 64, device="cpu")
    with pytest.raises(ValueError, match="head dimension"):
        ChunkedPrefill(8, 2, 100, 64, device="cpu")
    with pytest.raises(ValueError, match="capacity"):
        ChunkedPrefill(8, 2, 128, 0, device="cpu")
    with pytest.raises(ValueError, match="total_tokens"):
        ChunkedPrefill(8, 2, 128, 64, total_tokens=0, device="cpu")
    with pytest.raises(RuntimeError, match="ROCm"):
        ChunkedPrefill(8, 2, 128, 64, device="cpu")


def test_decoder_ops_validate_operands_without_a_gpu():
    """The harness's decoder-kernel wrappers check shapes, dtypes and layouts
    before any launch (the C ABI cannot see a non-contiguous last dimension)."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfpv2_hip.so not built")
    from fpv2.prefill_harness import DecoderShape, _add_rms_norm, _qk_norm_rope, _silu_mul
    bf = torch.bfloat16
    with pytest.raises(ValueError, match="contiguous rows"):
        _add_rms_norm(torch.zeros(16, 8, dtype=bf).t(), None, torch.ones(8, dtype=bf), 1e-6)
    with pytest.raises(ValueError, match="weight"):
        _add_rms_norm(torch.zeros(4, 16, dtype=bf), None, torch.ones(8, dtype=bf), 1e-6)
    with pytest.raises(ValueError, match="delta"):
        _add_rms_norm(torch.zeros(4, 16, dtype=bf), torch.zeros(4, 16), torch.ones(16, dtype=bf),
                      1e-6)
    shape = DecoderShape(query_heads=2, kv_heads=1, head_dim=64)
    w = torch.ones(64, dtype=bf)
    with pytest.raises(ValueError, match="cos"):
        _qk_norm_rope(torch.zeros(4, 256, dtype=bf), w, w, torch.zeros(4, 64, dtype=bf),
                      torch.zeros(4, 64), shape)
    with pytest.raises(ValueError, match="2 \\* cols"):
        _silu_mul(torch.zeros(4, 16, dtype=bf), 16)
    with pytest.raises(RuntimeError, match="ROCm"):
        _silu_mul(torch.zeros(4, 32, dtype=bf), 16)
    lib = _lib.load()
    x = 4096  # any non-null address: the aliasing check precedes every launch
    assert lib.fpv2_add_rms_norm(x, None, 8192, x, _lib.BF16, 1, 8, 8, 0, 8, 1e-6,
                                 None) == _lib.FPV2_ERR_ARGUMENT
    assert b"alias" in lib.fpv2_last_error()


def test_score_select_rejects_more_than_the_maximum_block_count():
    """More than FPV2_MAX_BLOCKS key blocks is refused before any launch."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfpv2_hip.so not built")
    lib = _lib.load()
    nb = _lib.MAX_BLOCKS + 1
    params = _lib.SelectParams(query_heads=8, kv_heads=2, head_dim=128, padded_query_length=32,
                               query_length=32, num_blocks=nb, key_length=nb * 128,
                               offset=nb * 128 - 32, block_k=128, tile_q=32, sink_tokens=128,
                               window_tokens=384, last_n_blocks=2, scale=0.088, alpha=0.1,
                               q_head_stride=32 * 128, q_row_stride=128,
                               pooled_head_stride=nb * 128)
    status = lib.fpv2_score_select(4096, 4096, _lib.BF16, params, None, None, None, None, None,
                                   None, None)
    assert status == _lib.FPV2_ERR_UNSUPPORTED
    assert b"exceeds 8192" in lib.fpv2_last_error()


def test_block_count_and_the_selection_limit():
    """Key blocks of a hook call, ``ceil(max(Lk, offset + Lq_pad) / block_k)``
    (``patch.py:123-131``), and the hook's routing rule: eligible calls with
    more blocks than the selection kernel holds go to the original SDPA."""
    from fpv2.patch import _num_blocks, _within_block_limit
    cfg = FPV2Config(tile_q=32, block_k=128)
    assert _num_blocks(32, 128, cfg) == 1
    assert _num_blocks(33, 129, cfg) == 1 + 1  # Lq_pad 64 -> 96 + 64 = 160 keys
    assert _num_blocks(1, 100, cfg) == 2       # offset 99 + Lq_pad 32 = 131 keys
    top = _lib.MAX_BLOCKS * 128
    assert _num_blocks(32, top, cfg) == _lib.MAX_BLOCKS
    assert _within_block_limit(32, top, cfg)
    assert not _within_block_limit(32, top + 1, cfg)
    # the query padding alone can cross the limit
    assert not _within_block_limit(20, top - 10, cfg)
    assert _within_block_limit(20, top - 12, cfg)


def test_hook_passes_calls_past_the_block_limit_to_the_original(monkeypatch):
    """An otherwise eligible call past the block limit reaches the original
    SDPA and is counted as dense (as a call below ``min_tokens``)."""
    import fpv2.patch as patch
    seen = {}

    def fake_original(q, k, v, **kwargs):
        seen["original"] = True
        return q

    def fake_fpv2(*args, **kwargs):
        raise AssertionError("FPV2 path taken past the block limit")

    monkeypatch.setattr(patch, "_ORIGINAL_SDPA", fake_original)
    monkeypatch.setattr(patch, "fpv2_sdpa", fake_fpv2)
    monkeypatch.setattr(patch, "_eligible", lambda *a, **k: True)  # device rules aside
    monkeypatch.setattr(_lib, "MAX_BLOCKS", 4)
    patch.enable(min_tokens=1, collect_stats=True)
    q = torch.zeros((1, 4, 32, 64), dtype=torch.bfloat16)
    kv = torch.zeros((1, 1, 5 * 128, 64), dtype=torch.bfloat16)
    F.scaled_dot_product_attention(q, kv, kv, is_causal=True, enable_gqa=True)
    assert seen == {"original": True}
    assert patch._visible_blocks == patch._selected_dense_blocks == 5
    assert patch.block_sparsity() == 0.0
    kv4 = kv[:, :, :4 * 128]
    with pytest.raises(AssertionError, match="FPV2 path"):
        F.scaled_dot_product_attention(q, kv4, kv4, is_causal=True, enable_gqa=True)


@pytest.mark.parametrize(("lq", "lk", "variant"), [(8, 40, "lower_right"), (24, 24, "lower_right"),
                                                   (8, 40, "upper_left")])
def test_passed_through_causal_bias_calls_equal_the_original(lq, lk, variant):
    """torch dispatches a CausalBias mask only while F.scaled_dot_product_attention
    is the original function; a call the hook passes through (here: CPU
    tensors, with GQA) still returns the original's result bit for bit, and
    the bias's inner calls are not counted twice."""
    from torch.nn.attention.bias import causal_lower_right, causal_upper_left
    import fpv2.patch as patch
    g = torch.Generator().manual_seed(lq + lk)
    q = torch.randn((1, 4, lq, 16), generator=g)
    k = torch.randn((1, 2, lk, 16), generator=g)
    v = torch.randn((1, 2, lk, 16), generator=g)
    bias = (causal_lower_right if variant == "lower_right" else causal_upper_left)(lq, lk)
    expected = _ORIGINAL_SDPA(q, k, v, attn_mask=bias, enable_gqa=True)
    enable(min_tokens=1, collect_stats=True)
    actual = F.scaled_dot_product_attention(q, k, v, attn_mask=bias, enable_gqa=True)
    assert torch.equal(actual, expected)
    assert patch._visible_blocks == 0  # CPU tensors are not eligible at all
    assert not patch._forwarding


def test_kernel_ready_realigns_a_contiguous_view_off_a_16_byte_boundary():
    """A contiguous view whose first element is not 16-byte aligned reaches
    the C ABI as an aligned copy (``contiguous()`` alone returns the view)."""
    from fpv2.kernel import _kernel_ready
    base = torch.arange(2 * 64 * 128 + 8, dtype=torch.bfloat16)
    view = base[4:4 + 2 * 64 * 128].view(2, 64, 128)  # 8 bytes into the storage
    assert view.is_contiguous() and view.data_ptr() % 16 == 8
    ready = _kernel_ready(view)
    assert ready.data_ptr() % 16 == 0
    assert ready.stride() == (64 * 128, 128, 1)
    assert torch.equal(ready, view)
    aligned = base[8:8 + 2 * 64 * 128].view(2, 64, 128)
    assert _kernel_ready(aligned).data_ptr() == aligned.data_ptr()  # no copy when aligned


def test_chunked_request_config_follows_the_hook_gates():
    """Below ``min_tokens`` keys or below one tile of queries the hook calls
    the original attention (``patch.py:177-205``); the chunked layer runs
    exact attention there (alpha 0), and the dense tail only at
    ``total_tokens`` (``patch.py:55-63``)."""
    from fpv2 import ChunkedPrefill
    cp = ChunkedPrefill.__new__(ChunkedPrefill)  # request rules only: no device state
    cp.config = FPV2Config(tile_q=32)
    cp.total_tokens, cp.min_tokens, cp.length = 8192, 4096, 8192
    assert cp.request_config().alpha == 0.1
    assert cp.request_config(32).alpha == 0.1
    assert cp.request_config(31).alpha == 0.0
    assert cp.request_config(2048).last_n_blocks == 2
    cp.length = 4095
    assert cp.request_config(2048).alpha == 0.0
    cp.length = 6000
    assert cp.request_config(2048).last_n_blocks == 0


def test_selected_block_counter_folds_in_batches():
    """Selected counts are kept and summed in batches; the total is exact
    across batches, partial batches and a reset."""
    from fpv2.patch import SelectedBlockCounter
    counter = SelectedBlockCounter(fold_every=4)
    g = torch.Generator().manual_seed(3)
    tensors = [torch.randint(0, 1000, (2, 1 + i % 5), generator=g, dtype=torch.int32) for i in range(11)]
    for t in tensors:
        counter.add(t)
    assert len(counter._pending) == 11 % 4  # two folds happened
    assert counter.value() == sum(int(t.sum()) for t in tensors)
    assert not counter._pending
    counter.add(torch.full((3,), 2**30, dtype=torch.int32))  # int64 accumulation
    assert counter.value() == sum(int(t.sum()) for t in tensors) + 3 * 2**30
    counter.reset()
    assert counter.value() == 0
