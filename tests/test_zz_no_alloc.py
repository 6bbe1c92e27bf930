"""aoakv_sparse_decode_layer_noalloc (the entry point that allocates nothing)
against aoakv_sparse_decode_layer with a caller workspace: the same bits
(output, selection, scores) on two calls in a row, the second on a smaller
input, through the C ABI.  The scratch array keeps the last call's
contents, so the second call also checks that the first left it usable."""
import sys

import numpy as np
import pytest
import torch

from helpers import HND, NHD, outlier_keys, randn16

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
D, S = 128, 16


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _layer_inputs(H, L, budget, layout, seed):
    from aoakv.utils import InferenceController, append_kv
    K = outlier_keys(randn16(seed, (L, H, D)), seed + 3)
    V = randn16(seed + 1, (L, H, D))
    q = randn16(seed + 2, (1, H, D))
    c = InferenceController(1, H, D, S, budget // S, L + S, torch.float16, DEV, layout=layout,
                            shuffle_seed=seed)
    c.prepare_metadata(L)
    c.begin_forward(L)
    append_kv(torch.from_numpy(K).to(DEV), torch.from_numpy(V).to(DEV), c, 0)
    c.end_forward()
    return c, torch.from_numpy(q).to(DEV)


def test_noalloc_layer_equals_workspace_layer_on_two_calls():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    from aoakv import ops
    F = ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED
    # the second call is smaller: fewer heads, pages and selected pages
    for H, L, budget, layout, seed in ((32, 4096 + 9, 1024, HND, 11), (8, 1500, 256, NHD, 12)):
        _say(f"[no-alloc] H={H} L={L} budget={budget} layout={layout}")
        c, q = _layer_inputs(H, L, budget, layout, seed)
        P = len(c.kv_cache.indicies)
        k = min(max(3, min(L, budget) // S), P)
        ws = ops.decode_workspace(1, H, H, k, DEV)
        outs = []
        for use_ws in (True, False):
            o = torch.full_like(q, float("nan"))
            scores = torch.zeros((1, H, P), dtype=torch.float32, device=DEV)
            sel = torch.full((1, H, k), -1, dtype=torch.int32, device=DEV)
            args = (q, o, c.kv_cache.buf_layer(0), c.kv_indptr_for_append,
                    c.kv_indices_with_last, c.kv_last_page_len_t, c.metadata_cache.buf_layer(0),
                    c.metadata_indptr_for_append, c.metadata_indices, c.v_log_norm_layer(0),
                    scores, sel, budget)
            if use_ws:
                ops.sparse_decode_layer(*args, ws, P, layout, F)
            else:
                ops.sparse_decode_layer_noalloc(*args, P, layout, F)
            torch.cuda.synchronize()
            outs.append((o.cpu().numpy(), sel.cpu().numpy(), scores.cpu().numpy()))
        (o1, s1, c1), (o2, s2, c2) = outs
        assert np.isfinite(o2.astype(np.float32)).all()
        assert np.array_equal(o1.view(np.uint16), o2.view(np.uint16))
        assert np.array_equal(s1, s2)
        assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))


def test_noalloc_layer_rejects_single_launch_and_oversized_calls():
    import aoakv  # noqa: F401
    from aoakv import AoakvError, ops
    c, q = _layer_inputs(8, 1500, 256, HND, 13)
    P = len(c.kv_cache.indicies)
    o = torch.empty_like(q)
    scores = torch.zeros((1, 8, P), dtype=torch.float32, device=DEV)
    sel = torch.zeros((1, 8, 16), dtype=torch.int32, device=DEV)
    args = (q, o, c.kv_cache.buf_layer(0), c.kv_indptr_for_append, c.kv_indices_with_last,
            c.kv_last_page_len_t, c.metadata_cache.buf_layer(0), c.metadata_indptr_for_append,
            c.metadata_indices, c.v_log_norm_layer(0), scores, sel, 256)
    with pytest.raises(AoakvError, match="two-launch"):
        ops.sparse_decode_layer_noalloc(*args, P, HND,
                                        ops.FLAG_VALUE_AWARE | ops.FLAG_SINGLE_LAUNCH)
    # 32 query heads x 8192 selected pages (a budget of 131072 tokens fills
    # the 8192-wide selection rows): a decode workspace of ~35 MB
    q32 = torch.zeros((1, 32, D), dtype=torch.float16, device=DEV)
    big_sel = torch.zeros((1, 8, 8192), dtype=torch.int32, device=DEV)
    big_scores = torch.zeros((1, 8, 16384), dtype=torch.float32, device=DEV)
    big = (q32, torch.empty_like(q32)) + args[2:10] + (big_scores, big_sel, 131072)
    with pytest.raises(AoakvError, match="scratch"):
        ops.sparse_decode_layer_noalloc(*big, 16384, HND, ops.FLAG_VALUE_AWARE)


def test_noalloc_error_word_and_graph_capture():
    """The scratch error word: a device page table of 300 pages passed with
    max_pages = 200 sets AOAKV_WS_ERR_TRUNCATED, which aoakv_noalloc_error
    reads and clears.  Then the entry point captured into a HIP graph (after
    aoakv_noalloc_init, outside capture) and replayed three times, with
    eager calls of the workspace path between the replays: every replay
    gives the workspace path's bits."""
    import aoakv  # noqa: F401
    from aoakv import ops
    F = ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED
    H, L, budget, Pmax = 8, 300 * S - 5, 1024, 200
    _say("[no-alloc] error word: 300-page table, max_pages 200")
    ops.noalloc_init()
    ops.noalloc_error(clear=True)          # whatever earlier calls left
    c, q = _layer_inputs(H, L, budget, HND, 14)
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=DEV)
    k = min(max(3, budget // S), Pmax)

    def bufs():
        return (torch.full_like(q, float("nan")),
                torch.zeros((1, H, Pmax), dtype=torch.float32, device=DEV),
                torch.full((1, H, k), -1, dtype=torch.int32, device=DEV))

    def args(o, scores, sel, P_table):
        return (q, o, c.kv_cache.buf_layer(0), t([0, P_table]), c.kv_indices_with_last,
                c.kv_last_page_len_t, c.metadata_cache.buf_layer(0), t([0, -(-P_table // S)]),
                c.metadata_indices, c.v_log_norm_layer(0), scores, sel, budget)

    outs = []
    for P_table in (Pmax, 300):
        o, scores, sel = bufs()
        ops.sparse_decode_layer_noalloc(*args(o, scores, sel, P_table), Pmax, HND, F)
        outs.append((o, scores, sel, ops.noalloc_error()))
    assert outs[0][3] == 0 and outs[1][3] == ops.WS_ERR_TRUNCATED
    for a, b in zip(outs[0][:3], outs[1][:3]):
        assert torch.equal(a, b)            # cut to the first 200 pages
    assert ops.noalloc_error(clear=True) == ops.WS_ERR_TRUNCATED
    assert ops.noalloc_error() == 0

    _say("[no-alloc] graph capture, three replays")
    ws = ops.decode_workspace(1, H, H, k, DEV)
    o_ref, sc_ref, sel_ref = bufs()
    ops.sparse_decode_layer(*args(o_ref, sc_ref, sel_ref, Pmax), ws, Pmax, HND, F)
    torch.cuda.synchronize()
    o, scores, sel = bufs()
    a = args(o, scores, sel, Pmax)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.sparse_decode_layer_noalloc(*a, Pmax, HND, F)
    for rep in range(3):
        o.fill_(float("nan"))
        scores.zero_()
        sel.fill_(-1)
        o2, sc2, sel2 = bufs()               # eager work between replays
        ops.sparse_decode_layer(*args(o2, sc2, sel2, Pmax), ws, Pmax, HND, F)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(sel, sel_ref), rep
        assert torch.equal(scores.view(torch.int32), sc_ref.view(torch.int32)), rep
        assert torch.equal(o2, o_ref), rep
    assert ops.noalloc_error() == 0
    del g
