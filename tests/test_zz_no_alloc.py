"""The allocation-free split entry point (``fpv2_sparse_attention_split_static``).

It runs the same kernels as ``fpv2_sparse_attention_split`` with the
partials in the library's static device scratch instead of a caller's
workspace, so on the same inputs the outputs are bit-identical.  Two calls
in a row (the second smaller, so the scratch holds the first call's
partials beyond the second's), and a split that needs more scratch than the
array holds is refused before any launch.
"""

from __future__ import annotations

import pytest
import torch

from fpv2 import FPV2Config, _lib, pool_blocks
from fpv2.kernel import compact_block_indices
from fpv2.selection import block_scores_and_select
from fpv2.synthetic import structured_qkv

pytestmark = pytest.mark.gpu


def _case(cuda, length, hq, hkv, d, seed):
    q, k, v = structured_qkv(length=length, query_heads=hq, kv_heads=hkv, head_dim=d, seed=seed,
                             dtype=torch.bfloat16, device=cuda)
    config = FPV2Config(alpha=0.2, sink_tokens=128, window_tokens=256, tile_q=128 // (hq // hkv))
    pk, pv = pool_blocks(k, 128), pool_blocks(v, 128)
    sel, _ = block_scores_and_select(q, pk, scale=d ** -0.5, config=config)
    lists = compact_block_indices(sel, config=config, query_length=length, key_length=length)
    params = _lib.AttnParams(
        query_heads=hq, kv_heads=hkv, head_dim=d, padded_query_length=length,
        query_length=length, out_rows=length, key_length=length, num_blocks=length // 128,
        offset=0, block_k=128, tile_q=config.tile_q, mean_correction=1, scale=d ** -0.5,
        q_head_stride=q.stride(0), q_row_stride=q.stride(1), k_head_stride=k.stride(0),
        k_row_stride=k.stride(1), v_head_stride=v.stride(0), v_row_stride=v.stride(1),
        o_head_stride=q.stride(0), o_row_stride=q.stride(1), pooled_head_stride=pk.stride(0))
    return (q, k, v, pk, pv, lists), params


def _ptrs(tensors, lists, out):
    q, k, v, pk, pv = tensors
    return [q.data_ptr(), k.data_ptr(), v.data_ptr(), pk.data_ptr(), pv.data_ptr(),
            *(x.data_ptr() for x in lists), out.data_ptr()]


def _run_both(cuda, length, hq, hkv, d, seed, split_tiles, seg_steps):
    lib = _lib.load()
    (q, k, v, pk, pv, lists), params = _case(cuda, length, hq, hkv, d, seed)
    stream = _lib.stream_ptr(cuda)
    need = lib.fpv2_sparse_attention_split_workspace_bytes(params, split_tiles, seg_steps)
    assert 0 < need <= _lib.SPLIT_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    out_ws = torch.empty_like(q)
    out_static = torch.empty_like(q)
    args = _ptrs((q, k, v, pk, pv), lists, out_ws)
    assert lib.fpv2_sparse_attention_split(*args, _lib.BF16, params, split_tiles, seg_steps,
                                           ws.data_ptr(), need, stream) == 0
    args = _ptrs((q, k, v, pk, pv), lists, out_static)
    assert lib.fpv2_sparse_attention_split_static(*args, _lib.BF16, params, split_tiles,
                                                  seg_steps, stream) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(out_ws.float()).all()
    assert torch.equal(out_static, out_ws)
    return need


def test_static_scratch_split_equals_workspace_split_twice(cuda):
    big = _run_both(cuda, 8192, 8, 2, 128, 1, split_tiles=4, seg_steps=8)
    small = _run_both(cuda, 2048, 4, 1, 64, 2, split_tiles=2, seg_steps=4)
    assert small < big  # the second call leaves part of the first one's partials in place


def test_static_scratch_refuses_a_split_larger_than_the_array(cuda):
    lib = _lib.load()
    (q, k, v, pk, pv, lists), params = _case(cuda, 8192, 8, 2, 128, 3)
    need = lib.fpv2_sparse_attention_split_workspace_bytes(params, 256, 1)
    assert need > _lib.SPLIT_SCRATCH_BYTES
    out = torch.full_like(q, 7.0)
    status = lib.fpv2_sparse_attention_split_static(
        *_ptrs((q, k, v, pk, pv), lists, out), _lib.BF16, params, 256, 1, _lib.stream_ptr(cuda))
    torch.cuda.synchronize()
    assert status == _lib.FPV2_ERR_UNSUPPORTED
    assert b"scratch" in lib.fpv2_last_error()
    assert bool((out == 7.0).all())  # nothing was launched
