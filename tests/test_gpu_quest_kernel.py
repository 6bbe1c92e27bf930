"""GPU parity of the reference KERNEL's selection convention
(AOAKV_FLAG_QUEST_KERNEL / ``InferenceController(semantics="quest_kernel")``)
against the oracle's ``quest_kernel_pages``.

The case grid and call sequence are the reference's own test of that path,
quest/tests/test_approx_attention.py:113-199: 32 heads, prefill kv_len - 1
tokens, append one decode token, then estimate -> top-k -> sparse decode,
or the dense path when the sequence has no more pages than the budget.  The
reference forces its own torch top-k indices into the decode
(:178-196); that call is repeated here with the oracle's indices.

Bars: page scores within fp32 sum-order noise; selections equal up to
near-ties (1e-3 relative); o within 2e-3 max-abs of the oracle; the fused
layer entry points (two launches, one launch) bit-identical to the three
calls.
"""
import sys

import numpy as np
import pytest
import torch

from helpers import HND, NHD, bits, randn16
from oracle import sim

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D, S = 128, 16
H = 32

GRID = [(L, pb) for L in (27, 61, 113, 482, 577, 1011, 1541) for pb in (4, 7, 15, 31, 55, 71)]


@pytest.fixture(scope="module", autouse=True)
def _aoakv():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    assert torch.cuda.is_available()
    yield


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _ctrl(L, pb, layout, value_aware, shuffle):
    from aoakv.utils import InferenceController
    return InferenceController(1, H, D, S, pb, L + S, torch.float16, DEV, layout=layout,
                               value_aware=value_aware, shuffle_seed=shuffle,
                               semantics="quest_kernel")


def _to_dev(x):
    """numpy (1, H, n, D) -> torch [n, H, D]."""
    return torch.from_numpy(np.ascontiguousarray(x[0].transpose(1, 0, 2))).to(DEV)


@pytest.mark.parametrize("value_aware", [False, True])
@pytest.mark.parametrize("L,pb", GRID + [(32768, 128)])  # + config 2's length and budget
def test_quest_kernel_decode_matches_oracle(L, pb, value_aware):
    from aoakv.utils import (append_kv, decode_estimate, decode_layer, decode_sparse_attn,
                             decode_topk)
    layout = HND if (L + pb) % 2 else NHD
    _say(f"[quest-kernel] L={L} page_budget={pb} va={value_aware} layout={layout}")
    q = randn16(1000 + L, (1, H, 1, D))
    K = randn16(2000 + L + pb, (1, H, L, D))
    V = randn16(3000 + L + pb, (1, H, L, D))
    ctrl = _ctrl(L, pb, layout, value_aware, shuffle=L)
    ctrl.prepare_metadata(L - 1)
    ctrl.begin_forward(L - 1)
    append_kv(_to_dev(K[:, :, :-1]), _to_dev(V[:, :, :-1]), ctrl, 0)
    ctrl.end_forward()
    ctrl.prepare_metadata(1)
    ctrl.begin_forward(1)
    append_kv(_to_dev(K[:, :, -1:]), _to_dev(V[:, :, -1:]), ctrl, 0)

    st = sim.SimLayerState(K[:, :, :-1], V[:, :, :-1])
    o_ref, scores_ref, pages_ref = sim.decode_step(
        st, q, K[:, :, -1:], V[:, :, -1:], pb * S, fixed=False, value_aware=value_aware,
        semantics="quest_kernel")
    P = (L + S - 1) // S
    k = min(pb, P)
    assert pages_ref.shape[-1] == k and ctrl.num_selected_pages() == k
    phys = np.asarray(ctrl.kv_cache.indicies)
    inv = {int(p): i for i, p in enumerate(phys)}
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    ref = o_ref[0, :, 0].astype(np.float32)

    if not ctrl.need_estimate():
        assert k == P
        o = decode_sparse_attn(qd, ctrl, 0, ctrl.kv_indices_without_last).cpu().numpy()[0]
        assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3
        return

    scores = decode_estimate(qd, ctrl, 0).cpu().numpy()
    assert scores.shape == (H, P - 1)                    # the last page is not scored
    np.testing.assert_allclose(scores, scores_ref[0, :, 0, :P - 1], rtol=2e-6, atol=2e-5)
    sel = decode_topk(scores, ctrl).cpu().numpy()
    assert sel.shape == (H, k - 1)
    sel_logical = np.vectorize(inv.get)(sel) if k > 1 else sel
    n_exact = 0
    for h in range(H):
        got = np.append(sel_logical[h], P - 1)
        ok, why = sim.selection_matches(got, pages_ref[0, h, 0], scores_ref[0, h, 0],
                                        forced={P - 1})
        assert ok, (h, why)
        assert P - 1 not in set(sel_logical[h].tolist())
        n_exact += why == "exact"
    o = decode_sparse_attn(qd, ctrl, 0, ctrl.topk_dindices_buffer).cpu().numpy()[0]
    if n_exact == H:
        assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3
    else:  # a near-tie chosen differently: the oracle's attention over the GPU's pages
        pages = np.concatenate([sel_logical, np.full((H, 1), P - 1)], axis=1)
        mask = sim.pages_to_token_mask(pages[None, :, None], S, L)
        ref2 = sim.masked_decode_attention(q, st.K, st.V, mask)[0, :, 0].astype(np.float32)
        assert np.abs(o.astype(np.float32) - ref2).max() <= 2e-3

    # the reference test's call: its own indices [H, page_budget - 1]
    # (physical ids, the last page excluded) forced into the decode
    forced = torch.from_numpy(phys[pages_ref[0, :, 0, :-1]].astype(np.int32)).to(DEV)
    o_forced = decode_sparse_attn(qd, ctrl, 0, forced).cpu().numpy()[0]
    assert np.abs(o_forced.astype(np.float32) - ref).max() <= 2e-3

    # fused entry points: the same bits and selection as the three calls
    o2 = decode_layer(qd, ctrl, 0).cpu().numpy()[0]
    assert np.array_equal(bits(o2), bits(o))
    assert np.array_equal(ctrl.topk_dindices_buffer.cpu().numpy()[0], sel)
    for rep in range(2):
        ctrl.topk_dindices_buffer.fill_(-1)
        o3 = decode_layer(qd, ctrl, 0, single_launch=True).cpu().numpy()[0]
        assert np.array_equal(bits(o3), bits(o)), rep
        assert np.array_equal(ctrl.topk_dindices_buffer.cpu().numpy()[0], sel)
        assert int(ctrl.workspace[8:12].view(torch.int32).item()) == 0, "spin-wait error flag"


def test_quest_kernel_one_page_budget_attends_the_last_page_only():
    """page_budget 1: nothing selected, the decode attends the last page."""
    from aoakv.utils import append_kv, decode_layer, decode_sparse_attn, decode_topk
    L = 100
    q = randn16(41, (1, H, 1, D))
    K = randn16(42, (1, H, L, D))
    V = randn16(43, (1, H, L, D))
    ctrl = _ctrl(L, 1, HND, True, shuffle=None)
    ctrl.prepare_metadata(L - 1)
    ctrl.begin_forward(L - 1)
    append_kv(_to_dev(K[:, :, :-1]), _to_dev(V[:, :, :-1]), ctrl, 0)
    ctrl.end_forward()
    ctrl.prepare_metadata(1)
    ctrl.begin_forward(1)
    append_kv(_to_dev(K[:, :, -1:]), _to_dev(V[:, :, -1:]), ctrl, 0)
    st = sim.SimLayerState(K[:, :, :-1], V[:, :, :-1])
    o_ref, _, pages_ref = sim.decode_step(st, q, K[:, :, -1:], V[:, :, -1:], S,
                                          fixed=False, semantics="quest_kernel")
    P = (L + S - 1) // S
    assert pages_ref.shape[-1] == 1 and int(pages_ref[0, 0, 0, 0]) == P - 1
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    assert decode_topk(None, ctrl).shape == (H, 0)
    o = decode_sparse_attn(qd, ctrl, 0, ctrl.topk_dindices_buffer).cpu().numpy()[0]
    ref = o_ref[0, :, 0].astype(np.float32)
    assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3
    o1 = decode_layer(qd, ctrl, 0, single_launch=True).cpu().numpy()[0]
    assert np.array_equal(bits(o1), bits(o))
