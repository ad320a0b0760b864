"""GPU parity over seeded random combinations of the operator's parameters.

Each case draws head_dim, dtype, query/KV head counts, block_k, tile_q,
alpha, sink/window/tail settings, mean correction, a chunk offset, an
unaligned query length and the sign of the scale, then runs the public
operators in sequence (``pool_blocks`` -> ``block_scores_and_select`` ->
``compact_block_indices`` -> ``sparse_attention``, the hook's data flow in
``fpv2/patch.py:109-174``) and checks every stage against the oracle:

  * pooled K/V bit-exact (``selection.py:68-80``);
  * block decisions equal outside the 1e-4 band around alpha
    (``selection.py:174-195``);
  * block lists and counts equal to the oracle's compaction of the device
    mask, bit for bit (``kernel.py:141-184``);
  * outputs of the valid query rows against the oracle's blockwise float32
    evaluation with the device's selection and pooled values
    (``reference.py:55-90``): max-abs <= 2e-2, mean-abs <= 2e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import attention_errors, to_np
from oracle import fpv2_oracle as orc
from fpv2 import FPV2Config, pool_blocks
from fpv2.kernel import compact_block_indices, sparse_attention
from fpv2.selection import block_scores_and_select
from fpv2.synthetic import structured_qkv

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS, BAND = 2e-2, 2e-3, 1e-4
_DT = {torch.bfloat16: "bf16", torch.float16: "f16"}


def _draw_cases(n: int, seed: int = 20261202) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        d = int(rng.choice([64, 96, 128, 256]))
        bk = int(rng.choice([16, 32, 64, 128]))
        hkv = int(rng.choice([1, 2]))
        g = int(rng.choice([1, 2, 4, 8]))
        cases.append(dict(
            case=i, head_dim=d, dtype=[torch.bfloat16, torch.float16][int(rng.integers(2))],
            kv_heads=hkv, query_heads=hkv * g, block_k=bk, tile_q=int(rng.choice([16, 32, 64])),
            alpha=float(rng.choice([0.0, 0.05, 0.15, 0.5])),
            sink=int(rng.choice([0, 1, 2])) * bk, window=int(rng.choice([0, 1, 3])) * bk,
            last_n=int(rng.integers(0, 3)), corr=bool(rng.integers(2)),
            offset=int(rng.choice([0, int(rng.integers(1, 600))])),
            qlen=int(rng.integers(100, 700)), sign=float(rng.choice([1.0, 1.0, 1.0, -1.0])),
            seed=int(rng.integers(1 << 30))))
    return cases


CASES = _draw_cases(48)


def _id(c: dict) -> str:
    return (f"c{c['case']}-d{c['head_dim']}-{_DT[c['dtype']]}-g{c['query_heads'] // c['kv_heads']}"
            f"-bk{c['block_k']}-tq{c['tile_q']}-a{c['alpha']}-corr{int(c['corr'])}"
            f"-off{c['offset']}-L{c['qlen']}{'-neg' if c['sign'] < 0 else ''}")


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_configuration_matches_oracle(cuda, c):
    _check_operators(cuda, c)


# Block sizes that are not a power of two or exceed the 32-key sub-tile
# (the last sub-tile of every block is partial for 48 and 96).
ODD_BLOCKS = [
    dict(case=100 + i, head_dim=d, dtype=torch.bfloat16, kv_heads=2, query_heads=8, block_k=bk,
         tile_q=tq, alpha=0.15, sink=bk, window=2 * bk, last_n=1, corr=True, offset=off,
         qlen=ql, sign=1.0, seed=7 + i)
    for i, (d, bk, tq, off, ql) in enumerate([(128, 48, 16, 0, 600), (64, 96, 32, 130, 500),
                                              (128, 256, 64, 0, 1100), (256, 48, 32, 77, 420),
                                              (96, 256, 16, 300, 700)])]


@pytest.mark.parametrize("c", ODD_BLOCKS, ids=[_id(c) for c in ODD_BLOCKS])
def test_block_sizes_off_the_sub_tile_grid_match_oracle(cuda, c):
    _check_operators(cuda, c)


def _check_operators(cuda, c):
    d, dtype, bk, tq = c["head_dim"], c["dtype"], c["block_k"], c["tile_q"]
    hq, hkv, offset, qlen = c["query_heads"], c["kv_heads"], c["offset"], c["qlen"]
    config = FPV2Config(block_k=bk, tile_q=tq, alpha=c["alpha"], sink_tokens=c["sink"],
                        window_tokens=c["window"], last_n_blocks=c["last_n"],
                        mean_correction=c["corr"])
    ocfg = orc.OracleConfig(**{f: getattr(config, f) for f in orc.OracleConfig.__dataclass_fields__})
    scale = c["sign"] * d ** -0.5
    lk = offset + qlen  # the queries are the last qlen keys (lower-right causal)
    q, k, v = structured_qkv(length=lk, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=bk,
                             seed=c["seed"], dtype=dtype)
    # tile-padded queries and block-padded keys, zero past the valid lengths
    lq_pad = -(-qlen // tq) * tq
    nb = -(-(offset + lq_pad) // bk)
    qp = torch.zeros((hq, lq_pad, d), dtype=dtype)
    qp[:, :qlen] = q[:, offset:]
    kp = torch.zeros((hkv, nb * bk, d), dtype=dtype)
    vp = torch.zeros((hkv, nb * bk, d), dtype=dtype)
    kp[:, :lk] = k
    vp[:, :lk] = v
    qd, kd, vd = qp.to(cuda), kp.to(cuda), vp.to(cuda)

    pk, pv = pool_blocks(kd, bk), pool_blocks(vd, bk)
    qn, kn, vn = to_np(qp), to_np(kp), to_np(vp)
    assert np.array_equal(to_np(pk), orc.pool_blocks(kn, bk, out_dtype=_DT[dtype]))
    assert np.array_equal(to_np(pv), orc.pool_blocks(vn, bk, out_dtype=_DT[dtype]))

    sel, _ = block_scores_and_select(qd, pk, scale=scale, config=config, offset=offset,
                                     query_length=qlen)
    sel_o, _, ratio = orc.block_scores_and_select(qn, to_np(pk), scale=scale, config=ocfg,
                                                  offset=offset, query_length=qlen,
                                                  return_ratio=True)
    sel_d = to_np(sel)
    differ = (sel_d != sel_o) & ~(np.abs(ratio - config.alpha) <= BAND)
    assert not differ.any(), f"{int(differ.sum())} block decisions differ outside the band"

    lists = compact_block_indices(sel, config=config, offset=offset, query_length=qlen,
                                  key_length=lk)
    want_lists = orc.compact_block_indices(sel_d, config=ocfg, offset=offset,
                                           query_length=qlen, key_length=lk)
    for got_l, want_l in zip(lists, want_lists):
        assert np.array_equal(to_np(got_l), want_l)

    out = sparse_attention(qd, kd, vd, pk, pv, *lists, scale=scale, config=config,
                           offset=offset, query_length=qlen, key_length=lk)
    torch.cuda.synchronize()
    want = orc.fpv2_attention_blockwise(qn, kn, vn, scale=scale, selected=sel_d,
                                        pooled_k=to_np(pk), pooled_v=to_np(pv), config=ocfg,
                                        offset=offset, query_length=qlen, key_length=lk)
    got = to_np(out)[:, :qlen]
    assert np.isfinite(got).all()
    err = attention_errors(got, want[:, :qlen])
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err


# ---------------------------------------------------------------------------
# The SDPA hook (fpv2/patch.py:177-285 restated in fpv2/patch.py): random
# eligible calls through torch.nn.functional.scaled_dot_product_attention.
# ---------------------------------------------------------------------------

def _draw_hook_cases(n: int, seed: int = 1202) -> list[dict]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        d = int(rng.choice([64, 96, 128, 256]))
        g = int(rng.choice([1, 2, 4, 8]))
        hkv = int(rng.choice([1, 2])) if d * g * 2 > 1024 else int(rng.choice([1, 2, 4]))
        hkv = max(1, min(hkv, 2048 // (d * g)))  # bounded oracle work
        tile_q = int(rng.choice([128, 128, 64, 32]))
        lk = int(rng.integers(200, 1400))
        lq = lk if rng.random() < 0.5 else int(rng.integers(128, lk + 1))
        cases.append(dict(
            case=i, head_dim=d, dtype=[torch.bfloat16, torch.float16][int(rng.integers(2))],
            kv_heads=hkv, query_heads=hkv * g, tile_q=tile_q,
            block_k=int(rng.choice([32, 64, 128])), alpha=float(rng.choice([0.05, 0.1, 0.3])),
            sink=int(rng.choice([0, 128])), window=int(rng.choice([0, 128, 384])),
            last_n=int(rng.choice([0, 2])), corr=bool(rng.integers(2)), lk=lk, lq=lq,
            total=bool(rng.integers(2)), scale=float(rng.choice([1.0, 0.7])) * d ** -0.5,
            seed=int(rng.integers(1 << 30))))
    return cases


HOOK_CASES = _draw_hook_cases(24)


def _hook_id(c: dict) -> str:
    return (f"h{c['case']}-d{c['head_dim']}-{_DT[c['dtype']]}-g{c['query_heads'] // c['kv_heads']}"
            f"-tq{c['tile_q']}-bk{c['block_k']}-a{c['alpha']}-corr{int(c['corr'])}"
            f"-Lq{c['lq']}-Lk{c['lk']}{'-tail' if c['total'] else ''}")


@pytest.mark.parametrize("c", HOOK_CASES, ids=[_hook_id(c) for c in HOOK_CASES])
def test_random_hook_call_matches_oracle(cuda, c):
    import torch.nn.functional as F
    from torch.nn.attention.bias import causal_lower_right
    import fpv2.patch as patch
    from fpv2 import block_sparsity, disable, enable

    d, dtype, lq, lk = c["head_dim"], c["dtype"], c["lq"], c["lk"]
    hq, hkv = c["query_heads"], c["kv_heads"]
    config = FPV2Config(block_k=c["block_k"], tile_q=c["tile_q"], alpha=c["alpha"],
                        sink_tokens=c["sink"], window_tokens=c["window"],
                        last_n_blocks=c["last_n"], mean_correction=c["corr"])
    total = lk if c["total"] else None
    q, k, v = structured_qkv(length=lk, query_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=c["block_k"], seed=c["seed"], dtype=dtype)
    q = q[:, lk - lq:]
    enable(config, min_tokens=1, collect_stats=True, total_tokens=total)
    try:
        qd, kd, vd = (x[None].to(cuda) for x in (q, k, v))
        if lq == lk:
            out = F.scaled_dot_product_attention(qd, kd, vd, is_causal=True, scale=c["scale"],
                                                 enable_gqa=True)
        else:
            out = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=causal_lower_right(lq, lk),
                                                 scale=c["scale"], enable_gqa=True)
        torch.cuda.synchronize()
        # the FPV2 path ran (an ineligible call would be counted as dense)
        assert patch._selected_dense_blocks == 0 and patch._visible_blocks > 0
        sparsity = block_sparsity()
    finally:
        disable()

    ocfg = orc.OracleConfig(**{f: getattr(config, f) for f in orc.OracleConfig.__dataclass_fields__})
    ocfg = orc.request_config(ocfg, lk, total)
    want, plan = orc.fpv2_sdpa_oracle(to_np(q), to_np(k), to_np(v), scale=c["scale"], config=ocfg,
                                      dtype=_DT[dtype], return_plan=True)
    got = to_np(out[0])
    assert got.shape == want.shape and np.isfinite(got).all()
    # rows of tiles where some block sits within the band around alpha may
    # select differently on the device (float32 energies); compare the rest
    tq = plan["config"].tile_q
    near = (np.abs(plan["ratio"] - ocfg.alpha) <= BAND).any(axis=(0, 2))
    rows = np.ones(lq, dtype=bool)
    for t in np.nonzero(near)[0]:
        rows[t * tq:(t + 1) * tq] = False
    assert rows.mean() > 0.5
    err = attention_errors(got[:, rows], want[:, rows])
    assert err["max_abs"] <= MAX_ABS and err["mean_abs"] <= MEAN_ABS, err
    if not near.any():
        # accounting: the device's selected count equals the oracle's
        visible = orc.causal_block_count(hkv, lq, plan["offset"], plan["config"])
        assert sparsity == 1.0 - int(plan["lists"][1].sum()) / visible


# ---------------------------------------------------------------------------
# The fused selection path (``fpv2_score_select`` with lists requested and no
# score output, positive scale: the hook's call, ``fpv2/patch.py``
# ``_select_attend``).  It runs the persistent streaming kernel for D <= 128
# and the owner kernel for D = 256; the cases above reach the mask-only
# kernels.  Large GQA groups (short tiles), block sizes off the 32-key grid,
# several 128-row passes per tile and Q views whose row stride is not a
# whole number of rows (the unswizzled Q fill) are covered here.
# ---------------------------------------------------------------------------

STREAM_CASES = [
    dict(case=200 + i, head_dim=d, dtype=dt, kv_heads=hkv, query_heads=hkv * g, block_k=bk,
         tile_q=tq, alpha=a, sink=bk, window=2 * bk, last_n=ln, corr=True, offset=off, qlen=ql,
         sign=1.0, seed=31 + i, pad=pad)
    for i, (d, dt, hkv, g, bk, tq, a, ln, off, ql, pad) in enumerate([
        (128, torch.bfloat16, 1, 16, 128, 8, 0.1, 1, 0, 600, 0),
        (128, torch.bfloat16, 1, 32, 64, 4, 0.15, 0, 130, 500, 0),
        (64, torch.bfloat16, 2, 16, 48, 8, 0.1, 1, 0, 700, 8),
        (128, torch.float16, 2, 8, 96, 16, 0.05, 2, 77, 650, 8),
        (64, torch.bfloat16, 1, 32, 256, 4, 0.1, 1, 0, 1100, 0),
        (128, torch.bfloat16, 2, 4, 16, 32, 0.2, 0, 300, 400, 24),
        (96, torch.bfloat16, 1, 8, 32, 16, 0.1, 1, 0, 500, 0),
        (128, torch.bfloat16, 1, 8, 128, 64, 0.1, 1, 64, 900, 8),
        (256, torch.bfloat16, 1, 16, 48, 8, 0.1, 1, 0, 600, 8),
    ])]


@pytest.mark.parametrize("c", STREAM_CASES, ids=[_id(c) + f"-pad{c['pad']}" for c in STREAM_CASES])
def test_fused_selection_lists_match_oracle(cuda, c):
    from fpv2 import _lib
    from fpv2.selection import _select_params

    d, dtype, bk, tq = c["head_dim"], c["dtype"], c["block_k"], c["tile_q"]
    hq, hkv, offset, qlen = c["query_heads"], c["kv_heads"], c["offset"], c["qlen"]
    config = FPV2Config(block_k=bk, tile_q=tq, alpha=c["alpha"], sink_tokens=c["sink"],
                        window_tokens=c["window"], last_n_blocks=c["last_n"],
                        mean_correction=c["corr"])
    ocfg = orc.OracleConfig(**{f: getattr(config, f) for f in orc.OracleConfig.__dataclass_fields__})
    scale = d ** -0.5
    lk = offset + qlen
    q, k, _ = structured_qkv(length=lk, query_heads=hq, kv_heads=hkv, head_dim=d, block_size=bk,
                             seed=c["seed"], dtype=dtype)
    lq_pad = -(-qlen // tq) * tq
    nb = -(-(offset + lq_pad) // bk)
    # queries in a buffer whose rows carry `pad` extra elements: a strided view
    qbuf = torch.zeros((hq, lq_pad, d + c["pad"]), dtype=dtype)
    qbuf[:, :qlen, :d] = q[:, offset:]
    kp = torch.zeros((hkv, nb * bk, d), dtype=dtype)
    kp[:, :lk] = k
    qd = qbuf.to(cuda)[..., :d]
    assert qd.stride(1) == d + c["pad"]
    pk = pool_blocks(kp.to(cuda), bk)

    ids = torch.empty((hkv, lq_pad // tq, nb), dtype=torch.int32, device=cuda)
    pids = torch.empty_like(ids)
    counts = torch.empty((hkv, lq_pad // tq), dtype=torch.int32, device=cuda)
    pcounts = torch.empty_like(counts)
    lib = _lib.load()
    params = _select_params(qd, nb, kv_heads=hkv, scale=scale, config=config, offset=offset,
                            query_length=qlen, padded_length=lq_pad, key_length=lk)
    with torch.cuda.device(cuda):
        status = lib.fpv2_score_select(qd.data_ptr(), pk.data_ptr(), _lib.dtype_code(dtype),
                                       params, None, None, ids.data_ptr(), counts.data_ptr(),
                                       pids.data_ptr(), pcounts.data_ptr(), _lib.stream_ptr(cuda))
    _lib.check(status, "score_select")
    torch.cuda.synchronize()
    ids_n, counts_n, pids_n, pcounts_n = (to_np(x) for x in (ids, counts, pids, pcounts))

    qn = to_np(qbuf)[..., :d]
    sel_o, _, ratio = orc.block_scores_and_select(qn, to_np(pk), scale=scale, config=ocfg,
                                                  offset=offset, query_length=qlen,
                                                  return_ratio=True)
    dev_sel = np.zeros(sel_o.shape, dtype=bool)
    for h in range(hkv):
        for t in range(ids_n.shape[1]):
            dev_sel[h, t, ids_n[h, t, :counts_n[h, t]]] = True
    differ = (dev_sel != sel_o) & ~(np.abs(ratio - config.alpha) <= BAND)
    assert not differ.any(), f"{int(differ.sum())} block decisions differ outside the band"
    # the lists are the oracle's compaction of the device's decisions, bit for bit
    o_ids, o_counts, o_pids, o_pcounts = orc.compact_block_indices(
        dev_sel, config=ocfg, offset=offset, query_length=qlen, key_length=lk)
    assert np.array_equal(ids_n, o_ids) and np.array_equal(counts_n, o_counts)
    assert np.array_equal(pcounts_n, o_pcounts)
    head = np.arange(nb)[None, None, :] < o_pcounts[..., None]
    assert np.array_equal(np.where(head, pids_n, -1), np.where(head, o_pids, -1))
    # and the mask-only kernel decides the same blocks outside the band
    sel_m, _ = block_scores_and_select(qd, pk, scale=scale, config=config, offset=offset,
                                       query_length=qlen)
    differ_m = (to_np(sel_m) != dev_sel) & ~(np.abs(ratio - config.alpha) <= BAND)
    assert not differ_m.any()
