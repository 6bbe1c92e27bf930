"""BASELINE config 5 at its stated size against the oracle: a ragged batch of
16 sequences (L ~ U[8192, 65536], seeded), 32 heads x 128, per-sequence
budget min(2048, L/8) (k = 128 pages for every sequence here), keys with 4
channels x8, values of 10% of the pages x4 -- the very batch ``bench.py``
times (``bench.ragged_batch_inputs``).

One launch covers the whole batch.  Its 8,192 decode workgroups exceed what
the GPU holds at once, so the one-launch layer runs with its separate top-k
workgroups; rows of up to 4,096 pages take the 16-keys-per-thread top-k.
Both fused paths (one launch, two launches) must give the same bits, and
each sequence must match the oracle (filter_util.py:269-407,
quest_attention.py:265-356): scores within rtol 2e-6, selections equal up
to near-ties, outputs within 2e-3, and the value term must change at least
one selection against plain Quest in each group of sequences checked.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import sim

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
H, D, S = 32, 128, 16


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def batch():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    from aoakv import ops
    import bench
    _say("[config5] building the batch (16 sequences, 8k-64k tokens, 32 heads)")
    R = bench.ragged_batch_inputs(DEV, ops.HND, keep_kv=True)
    Ls, Ps, ks = R["Ls"], R["Ps"], R["ks"]
    Bn, maxP, kmax = len(Ls), max(Ps), max(ks)
    assert maxP > 2048 and kmax == 128  # rows past 2048 pages: the 16-keys-per-thread top-k
    outs = {}
    for name, extra in (("two", 0), ("one", ops.FLAG_SINGLE_LAUNCH)):
        o = torch.full_like(R["q"], float("nan"))
        scores = torch.zeros((Bn, H, maxP), dtype=torch.float32, device=DEV)
        sel = torch.full((Bn, H, kmax), -1, dtype=torch.int32, device=DEV)
        ws = ops.decode_workspace(Bn, H, H, kmax, DEV, max_pages=maxP)
        _say(f"[config5] {name}-launch layer")
        for _ in range(2):  # the second call runs on the workspace the first left
            ops.sparse_decode_layer(R["q"], o, R["kv"], R["kv_indptr"], R["kv_indices"], R["lpl"],
                                    R["meta"], R["m_indptr"], R["m_indices"], R["lvn"], scores,
                                    sel, 0, ws, maxP, ops.HND,
                                    ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED | extra,
                                    token_budgets=R["tb"])
        torch.cuda.synchronize()
        assert ops.workspace_error(ws) == 0
        assert int(ws.count_nonzero().item()) == 0, "workspace left non-zero"
        outs[name] = (o.cpu().numpy(), sel.cpu().numpy(), scores.cpu().numpy())
    R["out"] = outs
    R["kv_indices_np"] = R["kv_indices"].cpu().numpy()
    R["indptr_np"] = R["kv_indptr"].cpu().numpy()
    R["q_np"] = R["q"].cpu().numpy()
    return R


def test_config5_one_launch_equals_two_launches(batch):
    o1, s1, c1 = batch["out"]["one"]
    o2, s2, c2 = batch["out"]["two"]
    assert np.array_equal(o1.view(np.uint16), o2.view(np.uint16))
    assert np.array_equal(s1, s2)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))


@pytest.mark.parametrize("group", [0, 1, 2, 3])
def test_config5_sequences_match_oracle(batch, group):
    o, sel, scores = batch["out"]["one"]
    Ls, Ps, budgets = batch["Ls"], batch["Ps"], batch["budgets"]
    kvi, ip = batch["kv_indices_np"], batch["indptr_np"]
    differs_from_quest = 0
    for b in range(4 * group, 4 * group + 4):
        L, P = Ls[b], Ps[b]
        _say(f"[config5] sequence {b}: L={L}, oracle")
        Kt, Vt = batch["kept"][b]
        K, V = Kt.numpy()[None], Vt.numpy()[None]          # (1, H, L, D)
        q = batch["q_np"][b][:, None, :][None]              # (1, H, 1, D)
        st = sim.SimLayerState(K, V)
        sc, pg = sim.select_pages(st, q, budgets[b])
        np.testing.assert_allclose(scores[b, :, :P], sc[0, :, 0], rtol=2e-6, atol=2e-5)
        inv = np.empty(int(kvi.max()) + 1, np.int64)
        inv[kvi[ip[b]:ip[b + 1]]] = np.arange(P)             # physical -> logical
        k = pg.shape[-1]
        assert k == batch["ks"][b]
        sl = inv[sel[b, :, :k]]
        for h in range(H):
            ok, why = sim.selection_matches(sl[h], pg[0, h, 0], sc[0, h, 0], True)
            assert ok, (b, h, why)
        ref = sim.sparse_decode_attention(q, K, V, sl[None, :, None, :], S, L)[0, :, 0]
        err = float(np.abs(o[b].astype(np.float32) - ref.astype(np.float32)).max())
        assert err <= 2e-3, (b, err)
        _, pq = sim.select_pages(st, q, budgets[b], True, False)
        differs_from_quest += int(any(set(pq[0, h, 0]) != set(pg[0, h, 0]) for h in range(H)))
        del st, K, V
    assert differs_from_quest >= 1, "value term never changed a selection"
