"""A layer call too large for one launch's grid.

The one-launch layer is a one-dimensional grid of 256-thread workgroups, and
a dispatch counts its work-items in 32 bits, so it holds at most 16,777,215
workgroups.  4,096 sequences of 16 heads with 2,047 of 2,048 pages selected
need 4,096 x 16 x 256 decode workgroups (2^24) on top of the scoring ones:
the call asks for AOAKV_FLAG_SINGLE_LAUNCH and must run as the two launches
(three-dimensional grids) instead.  Its workspace (18.8 GB) also holds more
than 2^32 words, which aoakv_workspace_init clears.

Every sequence shares one page table (the same physical pages), with a query
of its own.  Three sequences are checked bit for bit against the same
sequence alone in a batch of one, run by the one-launch layer kernel (the
one- and two-launch paths give the same bits, and each sequence's result
does not depend on the batch; both paths are held to the oracle by the
other decode tests).
"""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
B, H, D, S = 4096, 16, 128, 16
P = 2048                    # pages per sequence
L = P * S
BUDGET = (P - 1) * S        # k = 2047 of 2048 pages: the top-k runs
K = BUDGET // S


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def cache():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    from aoakv import ops
    g = torch.Generator(device=DEV).manual_seed(41)
    Pm = P // S
    kv = torch.empty((P, 2, H, S, D), dtype=torch.float16, device=DEV)
    meta = torch.empty((Pm, 2, H, S, D), dtype=torch.float16, device=DEV)
    lvn = torch.empty((P, H), dtype=torch.float16, device=DEV)
    vmean = torch.empty((P, H, D), dtype=torch.float16, device=DEV)
    idx = torch.randperm(P, generator=torch.Generator().manual_seed(42)).to(DEV, torch.int32)
    midx = torch.arange(Pm, dtype=torch.int32, device=DEV)
    k = torch.randn((L, H, D), generator=g, device=DEV).half()
    v = torch.randn((L, H, D), generator=g, device=DEV).half()
    ops.append_kv_cache_prefill(k, v, kv, idx, P, S, meta, midx, lvn, vmean, ops.HND)
    q = torch.randn((B, H, D), generator=g, device=DEV).half()
    torch.cuda.synchronize()
    return dict(kv=kv, meta=meta, lvn=lvn, idx=idx, midx=midx, q=q)


def _layer(c, q, batch, ws, scores, sel, o):
    from aoakv import ops
    Pm = P // S
    ar = torch.arange(batch + 1, dtype=torch.int32, device=DEV)
    ops.sparse_decode_layer(q, o, c["kv"], ar * P, c["idx"].repeat(batch),
                            torch.full((batch,), S, dtype=torch.int32, device=DEV), c["meta"],
                            ar * Pm, c["midx"].repeat(batch), c["lvn"], scores, sel, BUDGET, ws,
                            P, ops.HND,
                            ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED | ops.FLAG_SINGLE_LAUNCH)


def _all_zero(ws, chunk=1 << 30):
    return all(not bool(torch.any(ws[i:i + chunk] != 0)) for i in range(0, ws.numel(), chunk))


def test_layer_past_one_launch_grid_runs_as_two_launches(cache):
    from aoakv import ops
    from aoakv._lib import load
    lib = load()
    n_ws = lib.aoakv_layer_workspace_size(B, H, H, D, K, P)
    assert n_ws // 4 > 2**32  # the workspace clear covers more words than one dispatch's count
    _say(f"[large-grid] batch {B} x {H} heads, {K} of {P} pages, workspace {n_ws / 1e9:.1f} GB")
    ws = ops.decode_workspace(B, H, H, K, DEV, max_pages=P)
    torch.cuda.synchronize()
    assert _all_zero(ws)
    scores = torch.zeros((B, H, P), dtype=torch.float32, device=DEV)
    sel = torch.full((B, H, K), -1, dtype=torch.int32, device=DEV)
    o = torch.full((B, H, D), float("nan"), dtype=torch.float16, device=DEV)
    _say("[large-grid] the batch")
    _layer(cache, cache["q"], B, ws, scores, sel, o)
    torch.cuda.synchronize()
    assert ops.workspace_error(ws) == 0
    assert _all_zero(ws), "workspace left non-zero"
    del ws
    torch.cuda.empty_cache()
    for b in (0, 1234, B - 1):
        _say(f"[large-grid] sequence {b} alone")
        ws1 = ops.decode_workspace(1, H, H, K, DEV, max_pages=P)
        s1 = torch.zeros((1, H, P), dtype=torch.float32, device=DEV)
        sel1 = torch.full((1, H, K), -1, dtype=torch.int32, device=DEV)
        o1 = torch.full((1, H, D), float("nan"), dtype=torch.float16, device=DEV)
        _layer(cache, cache["q"][b:b + 1].contiguous(), 1, ws1, s1, sel1, o1)
        torch.cuda.synchronize()
        assert ops.workspace_error(ws1) == 0
        assert torch.equal(sel[b], sel1[0]), f"sequence {b}: selection"
        assert torch.equal(scores[b].view(torch.int32), s1[0].view(torch.int32)), f"sequence {b}: scores"
        assert torch.equal(o[b].view(torch.int16), o1[0].view(torch.int16)), f"sequence {b}: output"
        assert not torch.isnan(o[b]).any()
