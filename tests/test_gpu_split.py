"""Split dense-tail tiles (``fpv2_sparse_attention_split``).

The last query tiles of a call can run as key-range segments in separate
workgroups whose partials (O, row sum, scale) a second kernel merges.  On
the same inputs and block lists the result must equal the unsplit kernel's
up to float32 summation order, and the split rows must match the oracle on
the device's selection: across head dimensions and dtypes, with correction
steps inside the split tiles, with a segment that takes the online walk,
with several 128-row chunks per tile, and through the SDPA hook (which
splits its dense tail when the walk is long).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import attention_errors, to_np
from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config, pool_blocks
from fpv2.kernel import _launch_attention, compact_block_indices
from fpv2.selection import block_scores_and_select
from fpv2.synthetic import baseline_qkv, structured_qkv

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3


def _cfg(c):
    return orc.OracleConfig(**{f: getattr(c, f) for f in orc.OracleConfig.__dataclass_fields__})


def _attend(q, k, v, pk, pv, lists, config, *, split_tiles=0, seg_steps=16):
    out = torch.empty_like(q)
    _launch_attention(q, k, v, pk, pv, *lists, out, device=q.device, scale=q.shape[-1] ** -0.5,
                      config=config, offset=k.shape[1] - q.shape[1], query_length=q.shape[1],
                      key_length=k.shape[1], num_blocks=pk.shape[1],
                      padded_query_length=q.shape[1], out_rows=q.shape[1],
                      split_tiles=split_tiles, seg_steps=seg_steps)
    torch.cuda.synchronize()
    return out


def _select(q, k, v, config):
    pk, pv = pool_blocks(k, config.block_k), pool_blocks(v, config.block_k)
    off = k.shape[1] - q.shape[1]
    sel, _ = block_scores_and_select(q, pk, scale=q.shape[-1] ** -0.5, config=config, offset=off)
    lists = compact_block_indices(sel, config=config, offset=off, query_length=q.shape[1],
                                  key_length=k.shape[1])
    return pk, pv, sel, lists


def _check(q, k, v, pk, pv, sel, lists, config, split_tiles, seg_steps, *, rows=None):
    whole = _attend(q, k, v, pk, pv, lists, config)
    split = _attend(q, k, v, pk, pv, lists, config, split_tiles=split_tiles, seg_steps=seg_steps)
    # the tiles that are not split are the same kernel work: bit for bit
    tq = config.tile_q
    r0 = q.shape[1] - split_tiles * tq
    assert torch.equal(whole[:, :r0], split[:, :r0])
    diff = (whole.float() - split.float()).abs()
    assert float(diff.max()) <= 1e-2, float(diff.max())
    qn, kn, vn = (to_np(x) for x in (q, k, v))
    ref = orc.fpv2_attention_blockwise(qn, kn, vn, scale=q.shape[-1] ** -0.5, selected=to_np(sel),
                                       pooled_k=to_np(pk), pooled_v=to_np(pv), config=_cfg(config),
                                       offset=k.shape[1] - q.shape[1],
                                       tiles=range(q.shape[1] // tq - split_tiles, q.shape[1] // tq))
    err = attention_errors(to_np(split)[:, r0:], ref[:, r0:])
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err
    return split


@pytest.mark.parametrize(("d", "dtype", "heads"), [
    (128, torch.bfloat16, (8, 2)), (128, torch.float16, (8, 2)), (64, torch.bfloat16, (16, 2)),
    (96, torch.bfloat16, (6, 3)), (256, torch.bfloat16, (4, 1)), (256, torch.float16, (4, 1)),
])
@pytest.mark.parametrize("corr", [True, False])
def test_split_dense_tail_equals_whole_tiles(cuda, d, dtype, heads, corr):
    """The hook's data flow with the dense tail (last 2 tiles) split into
    segments of 16 sub-tiles (4096 keys: 128 steps, 8 segments)."""
    hq, hkv = heads
    q, k, v = structured_qkv(length=4096, query_heads=hq, kv_heads=hkv, head_dim=d, seed=d + hq,
                             dtype=dtype, device=cuda)
    config = FPV2Config(alpha=0.2, sink_tokens=128, window_tokens=256, tile_q=128 // (hq // hkv),
                        mean_correction=corr)
    pk, pv, sel, lists = _select(q, k, v, config)
    assert bool((lists[3] > 0).any()) or not corr  # the other tiles prune
    _check(q, k, v, pk, pv, sel, lists, config, split_tiles=2, seg_steps=16)


def test_split_tiles_with_correction_steps(cuda):
    """Split tiles whose lists prune blocks (so their walks end in
    correction steps): every segment of such a tile rescales its exact part,
    so the merged partials share one scale.  Segments of 5 sub-tiles, so
    segment boundaries fall inside blocks and at the exact/correction
    boundary."""
    q, k, v = structured_qkv(length=2048, query_heads=8, kv_heads=2, head_dim=128, seed=3,
                             dtype=torch.bfloat16, device=cuda)
    config = FPV2Config(alpha=0.3, sink_tokens=128, window_tokens=128, last_n_blocks=0,
                        tile_q=32)
    pk, pv, sel, lists = _select(q, k, v, config)
    assert bool((lists[3][:, -4:] > 0).all())  # the split tiles prune blocks
    _check(q, k, v, pk, pv, sel, lists, config, split_tiles=4, seg_steps=5)


def test_split_segment_with_online_walk(cuda):
    """A key whose logits lie ~200 log2 units above the rest of its rows sits
    in one segment: that segment overflows and walks again with the online
    reference, the others do not; the merge rescales by the segments'
    references."""
    g = torch.Generator().manual_seed(31)
    L, d = 2048, 128
    q = torch.randn((8, L, d), generator=g)
    k = torch.randn((2, L, d), generator=g)
    v = torch.randn((2, L, d), generator=g)
    u = torch.randn((2, d), generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    j = 1000
    k[:, j] = 40.0 * u
    q[:, j:] += 40.0 * u.repeat_interleave(4, dim=0)[:, None, :]
    q, k, v = (x.bfloat16().to(cuda) for x in (q, k, v))
    config = FPV2Config(alpha=0.0, sink_tokens=0, window_tokens=0, last_n_blocks=0, tile_q=32,
                        mean_correction=False)
    pk, pv, sel, lists = _select(q, k, v, config)
    _check(q, k, v, pk, pv, sel, lists, config, split_tiles=3, seg_steps=8)


def test_split_tiles_of_several_row_chunks(cuda):
    """tile_q 64 at G = 4: 256 packed rows, two 128-row chunks per tile, each
    split into segments."""
    q, k, v = structured_qkv(length=3072, query_heads=8, kv_heads=2, head_dim=128, seed=5,
                             dtype=torch.bfloat16, device=cuda)
    config = FPV2Config(alpha=0.15, sink_tokens=128, window_tokens=256, tile_q=64)
    pk, pv, sel, lists = _select(q, k, v, config)
    _check(q, k, v, pk, pv, sel, lists, config, split_tiles=2, seg_steps=12)


def test_hook_splits_a_long_dense_tail(cuda):
    """The hook splits its dense tail once the walk exceeds two segments of
    128 sub-tiles: at 16384 keys with the contrast generator, the last two
    tiles run as 4 segments each; outputs equal the unsplit run up to
    float32 summation order, and the tail rows match the oracle."""
    from fpv2.patch import _fpv2_sdpa
    seq = 16384
    q, k, v = baseline_qkv(seq, planted=3.0 * 128 ** 0.5, heavy_fraction=0.06, seed=4,
                           device=cuda)
    config = FPV2Config(alpha=0.1, sink_tokens=128)
    keep, keep0 = {}, {}
    out = _fpv2_sdpa(q[None], k[None], v[None], scale=128 ** -0.5, config=config, keep=keep)
    out0 = _fpv2_sdpa(q[None], k[None], v[None], scale=128 ** -0.5, config=config, keep=keep0,
                      split=0)
    torch.cuda.synchronize()
    assert keep["split_tiles"] == 2 and keep0["split_tiles"] == 0
    tq = keep["config"].tile_q
    assert torch.equal(out[0, :, :seq - 2 * tq], out0[0, :, :seq - 2 * tq])
    assert float((out.float() - out0.float()).abs().max()) <= 1e-2
    ids, counts, _, _ = keep["lists"]
    nt, nb = ids.shape[1], ids.shape[2]
    dev_sel = np.zeros((ids.shape[0], 2, nb), dtype=bool)
    idn, cn = to_np(ids[:, nt - 2:]), to_np(counts[:, nt - 2:])
    for h in range(idn.shape[0]):
        for t in range(2):
            dev_sel[h, t, idn[h, t, :cn[h, t]]] = True
    assert dev_sel.all()  # the dense tail
    ref = orc.fpv2_attention_blockwise(
        to_np(q[:, seq - 2 * tq:]), to_np(k), to_np(v), scale=128 ** -0.5, selected=dev_sel,
        pooled_k=to_np(keep["pooled_k"]), pooled_v=to_np(keep["pooled_v"]),
        config=_cfg(keep["config"]), offset=seq - 2 * tq)
    err = attention_errors(to_np(out[0, :, seq - 2 * tq:]), ref)
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err


def test_split_workspace_is_checked(cuda):
    """A workspace smaller than fpv2_sparse_attention_split_workspace_bytes
    is refused before any launch."""
    from fpv2 import _lib
    lib = _lib.load()
    q, k, v = structured_qkv(length=1024, query_heads=4, kv_heads=1, head_dim=64, seed=1,
                             dtype=torch.bfloat16, device=cuda)
    config = FPV2Config(alpha=0.1, tile_q=32)
    pk, pv, sel, lists = _select(q, k, v, config)
    params = _lib.AttnParams(
        query_heads=4, kv_heads=1, head_dim=64, padded_query_length=1024, query_length=1024,
        out_rows=1024, key_length=1024, num_blocks=8, offset=0, block_k=128, tile_q=32,
        mean_correction=1, scale=0.125, q_head_stride=1024 * 64, q_row_stride=64,
        k_head_stride=1024 * 64, k_row_stride=64, v_head_stride=1024 * 64, v_row_stride=64,
        o_head_stride=1024 * 64, o_row_stride=64, pooled_head_stride=8 * 64)
    need = lib.fpv2_sparse_attention_split_workspace_bytes(params, 2, 4)
    assert need == 1 * 2 * 1 * -(-(8 * 4 + 1) // 4) * 128 * (64 + 2) * 4
    out = torch.empty_like(q)
    ws = torch.empty(need - 16, dtype=torch.uint8, device=cuda)
    ids, counts, pids, pcounts = lists
    status = lib.fpv2_sparse_attention_split(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), pk.data_ptr(), pv.data_ptr(), ids.data_ptr(),
        counts.data_ptr(), pids.data_ptr(), pcounts.data_ptr(), out.data_ptr(), _lib.BF16, params,
        2, 4, ws.data_ptr(), need - 16, _lib.stream_ptr(cuda))
    assert status == _lib.FPV2_ERR_ARGUMENT
    assert b"workspace" in lib.fpv2_last_error()
