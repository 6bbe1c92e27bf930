"""GPU parity of the decode hot path (libaoakv.so through its C ABI) against
the oracle (oracle/sim.py), on seeded inputs.

Bars: bit-exact for K/V storage, Kmax/Kmin, V̄ and log‖V̄‖; selected page
sets equal up to near-ties (|score - boundary| <= 1e-3 relative); attention
outputs within 2e-3 max-abs (fp16) of the simulation.
"""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import HND, NHD, bits, num_pages, outlier_keys, randn16, read_filters, read_kv
from oracle import sim

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D, S = 128, 16


@pytest.fixture(scope="module", autouse=True)
def _aoakv():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    assert torch.cuda.is_available()
    yield


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def make_ctrl(H, max_len, layout, budget_tokens=1024, shuffle=None, num_layers=1,
              fixed=True, value_aware=True):
    from aoakv.utils import InferenceController
    return InferenceController(num_layers, H, D, S, budget_tokens // S, max_len, torch.float16,
                               DEV, layout=layout, fixed=fixed, value_aware=value_aware,
                               shuffle_seed=shuffle)


def prefill(ctrl, K, V, layer=0):
    """K, V numpy (1, H, L, D) -> append through the library."""
    from aoakv.utils import append_kv
    L = K.shape[2]
    ctrl.prepare_metadata(L)
    ctrl.begin_forward(L)
    k = torch.from_numpy(np.ascontiguousarray(K[0].transpose(1, 0, 2))).to(DEV)
    v = torch.from_numpy(np.ascontiguousarray(V[0].transpose(1, 0, 2))).to(DEV)
    append_kv(k, v, ctrl, layer)
    ctrl.end_forward()


def decode_append(ctrl, kn, vn, layer=0):
    """kn, vn numpy (1, H, 1, D)."""
    from aoakv.utils import append_kv
    ctrl.prepare_metadata(1)
    ctrl.begin_forward(1)
    append_kv(torch.from_numpy(kn[0, :, 0][None].copy()).to(DEV),
              torch.from_numpy(vn[0, :, 0][None].copy()).to(DEV), ctrl, layer)


def check_metadata(ctrl, st: sim.SimLayerState, layer=0):
    L = st.kv_len
    P = num_pages(L)
    pages = ctrl.kv_cache.indicies
    torch.cuda.synchronize()
    K, V = read_kv(ctrl.kv_cache.buf_layer(layer), ctrl.layout, pages, L)
    assert np.array_equal(bits(K), bits(st.K)), "K storage"
    assert np.array_equal(bits(V), bits(st.V)), "V storage"
    pf = read_filters(ctrl.metadata_cache.buf_layer(layer), ctrl.layout,
                      ctrl.metadata_cache.indicies, P)
    assert np.array_equal(bits(pf), bits(st.page_filters)), "Kmax/Kmin"
    vm = ctrl.v_mean_layer(layer).cpu().numpy()[pages][None].transpose(0, 2, 1, 3)
    assert np.array_equal(bits(vm), bits(st.v_mean)), "page mean of V"
    lvn = ctrl.v_log_norm_layer(layer).cpu().numpy()[pages].T[None]
    ref = sim.log_v_norm(st.v_mean)
    bad = np.nonzero(bits(lvn) != bits(ref))
    assert bad[0].size == 0, f"log-norm mismatches at {list(zip(*bad))[:5]}"


# ------------------------------------------------------------------ metadata

@pytest.mark.parametrize("layout", [NHD, HND])
@pytest.mark.parametrize("L", [17, 31, 256, 4103])
def test_prefill_append_metadata_bit_exact(layout, L):
    _say(f"[prefill-append] layout={layout} L={L}")
    H = 8
    K = randn16(100 + L, (1, H, L, D))
    V = randn16(200 + L, (1, H, L, D))
    ctrl = make_ctrl(H, L + 64, layout, shuffle=L)
    prefill(ctrl, K, V)
    check_metadata(ctrl, sim.SimLayerState(K, V))


@pytest.mark.parametrize("layout", [NHD, HND])
def test_decode_append_trace_bit_exact(layout):
    """Prefill 4096+7 tokens, then 40 single-token appends crossing pages;
    metadata checked after every append (running fp16 mean, F5)."""
    _say(f"[decode-append] layout={layout}")
    H, L0, steps = 8, 4096 + 7, 40
    K = randn16(1, (1, H, L0, D))
    V = randn16(2, (1, H, L0, D))
    kn = randn16(3, (steps, 1, H, 1, D))
    vn = randn16(4, (steps, 1, H, 1, D))
    ctrl = make_ctrl(H, L0 + steps + 16, layout, shuffle=7)
    prefill(ctrl, K, V)
    st = sim.SimLayerState(K, V)
    for s in range(steps):
        decode_append(ctrl, kn[s], vn[s])
        st.append(kn[s], vn[s])
        if s % 8 == 7 or s == steps - 1:
            check_metadata(ctrl, st)


def test_prefill_append_config3a_full_size_bit_exact():
    """BASELINE config 3a at its full size: the bulk metadata build of a
    32768-token sequence over 32 heads (the bench's layout, HND).  K/V
    storage, Kmax/Kmin, page means and log-norms all bit-exact."""
    _say("[prefill-append] config 3a, 32 heads x 32768 tokens")
    H, L = 32, 32768
    K = randn16(300, (1, H, L, D))
    V = randn16(301, (1, H, L, D))
    ctrl = make_ctrl(H, L + 64, HND, shuffle=3)
    prefill(ctrl, K, V)
    check_metadata(ctrl, sim.SimLayerState(K, V))


def test_decode_append_config3b_full_trace_bit_exact():
    """BASELINE config 3b at its full size: 4096+7 tokens, then 512
    single-token appends over 32 heads (32 page boundaries crossed, partial
    pages updated by the running mean); metadata checked every 128 appends."""
    _say("[decode-append] config 3b, 32 heads, 512 appends")
    H, L0, steps = 32, 4096 + 7, 512
    K = randn16(11, (1, H, L0, D))
    V = randn16(12, (1, H, L0, D))
    kn = randn16(13, (steps, 1, H, 1, D))
    vn = randn16(14, (steps, 1, H, 1, D))
    ctrl = make_ctrl(H, L0 + steps + 16, HND, shuffle=11)
    prefill(ctrl, K, V)
    st = sim.SimLayerState(K, V)
    for s in range(steps):
        decode_append(ctrl, kn[s], vn[s])
        st.append(kn[s], vn[s])
        if s % 128 == 127:
            check_metadata(ctrl, st)


@pytest.mark.parametrize("layout", [NHD, HND])
def test_chunked_prefill_append(layout):
    """A second bulk append: the page already holding tokens continues the
    running mean token by token (update_mean_filter); every page the chunk
    opens gets the prefill page mean (compute_page_v_mean), as a prefill of
    those tokens would."""
    _say(f"[chunked-append] layout={layout}")
    H, L0, N = 4, 21, 30
    K = randn16(5, (1, H, L0 + N, D))
    V = randn16(6, (1, H, L0 + N, D))
    ctrl = make_ctrl(H, 128, layout, shuffle=2)
    prefill(ctrl, K[:, :, :L0], V[:, :, :L0])
    prefill(ctrl, K[:, :, L0:], V[:, :, L0:])
    st = sim.SimLayerState(K[:, :, :L0], V[:, :, :L0])
    cont = S - L0 % S                    # tokens that complete the partial page
    for t in range(L0, L0 + cont):
        st.append(K[:, :, t:t + 1], V[:, :, t:t + 1])
    fresh = sim.SimLayerState(K[:, :, L0 + cont:], V[:, :, L0 + cont:])
    st.page_filters = np.concatenate([st.page_filters, fresh.page_filters], axis=2)
    st.v_mean = np.concatenate([st.v_mean, fresh.v_mean], axis=2)
    st.K, st.V, st.kv_len = K, V, L0 + N
    check_metadata(ctrl, st)


def test_log_norm_whole_fp16_domain():
    """Pages whose V rows are [x, 0, ..., 0] have V̄ = x exactly and
    ‖V̄‖ = |x|: covers log() on every positive finite fp16 value."""
    _say("[log-domain]")
    xs = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16)  # 31743 values
    H = 32
    P = math.ceil(xs.size / H)
    vals = np.zeros(P * H, np.float16)
    vals[:xs.size] = xs
    V = np.zeros((1, H, P * S, D), np.float16)
    V[0, :, :, 0] = np.repeat(vals.reshape(P, H).T, S, axis=1)
    K = randn16(9, (1, H, P * S, D))
    ctrl = make_ctrl(H, P * S, HND)
    prefill(ctrl, K, V)
    torch.cuda.synchronize()
    lvn = ctrl.v_log_norm_layer(0).cpu().numpy()[ctrl.kv_cache.indicies].reshape(-1)
    with np.errstate(divide="ignore"):
        ref = torch.log(torch.from_numpy(vals.copy())).numpy()
    got = lvn.reshape(P, H).reshape(-1)
    bad = np.nonzero(bits(got)[:xs.size] != bits(ref)[:xs.size])[0]
    assert bad.size == 0, f"{bad.size} fp16 inputs differ, e.g. {vals[bad[:5]]}"


# ------------------------------------------------------------------ scores / top-k

def _sim_state(seed, H, L, outlier=False):
    K = randn16(seed, (1, H, L, D))
    V = randn16(seed + 1, (1, H, L, D))
    q = randn16(seed + 2, (1, H, 1, D))
    if outlier:
        K = outlier_keys(K, seed + 3)
    return q, K, V


def _selection_ok(sel_gpu, pages_ref, scores_ref, fixed):
    n_exact = 0
    for h in range(pages_ref.shape[1]):
        ok, why = sim.selection_matches(sel_gpu[h], pages_ref[0, h, 0], scores_ref[0, h, 0], fixed)
        assert ok, (h, why)
        n_exact += why == "exact"
    return n_exact


@pytest.mark.parametrize("layout", [NHD, HND])
@pytest.mark.parametrize("fixed,value_aware", [(True, True), (False, True), (True, False)])
def test_estimate_and_topk_match_simulation(layout, fixed, value_aware):
    from aoakv.utils import decode_estimate, decode_topk
    _say(f"[estimate+topk] layout={layout} fixed={fixed} va={value_aware}")
    H, L, budget = 32, 4096, 1024                      # config 1
    q, K, V = _sim_state(0, H, L)
    ctrl = make_ctrl(H, L + 16, layout, budget, shuffle=3, fixed=fixed, value_aware=value_aware)
    prefill(ctrl, K[:, :, :-1], V[:, :, :-1])
    decode_append(ctrl, K[:, :, -1:], V[:, :, -1:])
    st = sim.SimLayerState(K[:, :, :-1], V[:, :, :-1])
    st.append(K[:, :, -1:], V[:, :, -1:])
    scores_ref, pages_ref = sim.select_pages(st, q, budget, fixed, value_aware)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    scores = decode_estimate(qd, ctrl, 0).cpu().numpy()
    np.testing.assert_allclose(scores, scores_ref[0, :, 0], rtol=2e-6, atol=2e-5)
    sel = decode_topk(None, ctrl).cpu().numpy()                   # physical ids
    inv = {p: i for i, p in enumerate(ctrl.kv_cache.indicies)}
    sel_logical = np.vectorize(inv.get)(sel)
    assert np.all(np.diff(sel_logical, axis=-1) > 0), "not ascending"
    n = _selection_ok(sel_logical, pages_ref, scores_ref, fixed)
    _say(f"   exact heads {n}/{H}")
    # top-k on the GPU's own scores must equal the oracle's top-k of them
    k = pages_ref.shape[-1]
    ref_on_gpu_scores = sim.topk_pages(scores, k, fixed)
    assert np.array_equal(sel_logical, ref_on_gpu_scores)


def test_topk_ties_break_to_lower_index():
    """Duplicated pages give bit-identical scores; the lower pages win."""
    from aoakv import ops
    _say("[topk-ties]")
    P, k = 300, 40
    g = np.random.default_rng(4)
    s = g.standard_normal((1, 3, P)).astype(np.float32)
    s[0, 0, 100:200] = 5.0          # 100 equal top scores, k-2 taken
    s[0, 1, :] = 1.0                # all equal
    s[0, 2, 50] = -np.inf
    scores = torch.from_numpy(s).to(DEV)
    L = P * S
    indptr = torch.tensor([0, P], dtype=torch.int32, device=DEV)
    idx = torch.arange(P, dtype=torch.int32, device=DEV)
    lpl = torch.tensor([S], dtype=torch.int32, device=DEV)
    sel = torch.full((1, 3, k), -1, dtype=torch.int32, device=DEV)
    for fixed in (True, False):
        ops.topk_filtering(scores, indptr, idx, lpl, k * S, sel, S,
                           ops.FLAG_FIXED if fixed else 0)
        got = sel.cpu().numpy()[0]
        ref = sim.topk_pages(s[0], k, fixed)
        assert np.array_equal(got, ref), (fixed, got, ref)
    assert L == P * S


@pytest.mark.parametrize("P", [1000, 1500, 2048, 3000, 4096, 5000, 16384])
def test_topk_row_lengths(P):
    """Standalone top-k over rows that take each keys-per-thread variant
    (4 / 8 / 16 staged in LDS, 64 read directly); rows: plain normal scores,
    scores rounded to create ties at the boundary, one huge outlier (the
    first radix digit then holds almost every key), and mixed-sign scores
    spanning the full key range."""
    from aoakv import ops
    _say(f"[topk] P={P}")
    k = max(3, P // 16)
    g = np.random.default_rng(P)
    s = g.standard_normal((1, 4, P)).astype(np.float32)
    s[0, 1] = np.round(s[0, 1] * 4) / 4
    s[0, 2, g.integers(P)] = 1e30
    s[0, 3] = (s[0, 3] * 1e20).astype(np.float32)
    scores = torch.from_numpy(s).to(DEV)
    indptr = torch.tensor([0, P], dtype=torch.int32, device=DEV)
    perm = g.permutation(P).astype(np.int32)             # physical page ids
    idx = torch.from_numpy(perm).to(DEV)
    lpl = torch.tensor([S], dtype=torch.int32, device=DEV)
    sel = torch.full((1, 4, k), -1, dtype=torch.int32, device=DEV)
    for fixed in (True, False):
        ops.topk_filtering(scores, indptr, idx, lpl, k * S, sel, S,
                           ops.FLAG_FIXED if fixed else 0)
        got = sel.cpu().numpy()[0]
        ref = perm[sim.topk_pages(s[0], k, fixed)]
        assert np.array_equal(got, ref), (P, fixed, np.nonzero(got != ref))


@pytest.mark.parametrize("L", [32768, 3000 * S])
def test_fused_estimate_topk_long_rows(L):
    """The fused scoring + top-k kernel at config-2 length (2048 pages: 8 keys
    per thread) and at 3000 pages (16 keys per thread) against the oracle."""
    from aoakv import ops
    _say(f"[estimate_topk fused] L={L}")
    H, budget = 4, 2048
    q, K, V = _sim_state(11, H, L)
    ctrl = make_ctrl(H, L + 16, HND, budget, shuffle=5)
    prefill(ctrl, K[:, :, :-1], V[:, :, :-1])
    decode_append(ctrl, K[:, :, -1:], V[:, :, -1:])
    st = sim.SimLayerState(K[:, :, :-1], V[:, :, :-1])
    st.append(K[:, :, -1:], V[:, :, -1:])
    scores_ref, pages_ref = sim.select_pages(st, q, budget, True, True)
    P = len(ctrl.kv_cache.indicies)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    c = ctrl
    ops.estimate_topk(qd, c.metadata_cache.buf_layer(0), c.metadata_indptr_for_append,
                      c.metadata_indices, c.kv_indptr_for_append, c.kv_indices_with_last,
                      c.kv_last_page_len_t, c.v_log_norm_layer(0), c.scores, c._sel,
                      c.token_budget, c.workspace, P, HND, c.flags)
    torch.cuda.synchronize()
    scores = c.scores[0, :, :P].cpu().numpy()
    np.testing.assert_allclose(scores, scores_ref[0, :, 0], rtol=2e-6, atol=2e-5)
    sel = c.topk_dindices_buffer[0].cpu().numpy()
    inv = {p: i for i, p in enumerate(c.kv_cache.indicies)}
    sel_logical = np.vectorize(inv.get)(sel)
    _selection_ok(sel_logical, pages_ref, scores_ref, True)
    assert np.array_equal(sel_logical, sim.topk_pages(scores, pages_ref.shape[-1], True))


# ------------------------------------------------------------------ attention

@pytest.mark.parametrize("layout", [NHD, HND])
@pytest.mark.parametrize("L,budget,outlier", [(4096, 1024, False), (4096 + 9, 1024, False),
                                              (1000, 1024, False), (32768, 2048, True),
                                              (32768, 4096, True)])
def test_full_decode_step_matches_simulation(layout, L, budget, outlier):
    """Config-1 shape, and config 2 at its full size (32768 tokens, budget
    2048, 4 key channels x8): prefill L-1 tokens, append one, then estimate /
    top-k / sparse decode; o within 2e-3 of the simulation's masked
    attention; the two fused layer paths give the same bits.  Budget 4096
    (256 pages, 32 decode chunks per head) takes the split-K merge through
    two groups of 16 chunks, in both layer paths."""
    from aoakv.utils import decode_estimate, decode_sparse_attn, decode_topk, decode_layer
    _say(f"[decode-step] layout={layout} L={L} budget={budget} outlier={outlier}")
    H = 32
    q, K, V = _sim_state(11, H, L, outlier)
    ctrl = make_ctrl(H, L + 16, layout, budget, shuffle=5)
    prefill(ctrl, K[:, :, :-1], V[:, :, :-1])
    decode_append(ctrl, K[:, :, -1:], V[:, :, -1:])
    st = sim.SimLayerState(K[:, :, :-1], V[:, :, :-1])
    o_ref, scores_ref, pages_ref = sim.decode_step(st, q, K[:, :, -1:], V[:, :, -1:], budget)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    s = decode_estimate(qd, ctrl, 0)
    sel = decode_topk(s, ctrl)
    o = decode_sparse_attn(qd, ctrl, 0, ctrl.topk_dindices_buffer).cpu().numpy()[0]
    inv = {p: i for i, p in enumerate(ctrl.kv_cache.indicies)}
    sel_logical = np.vectorize(inv.get)(sel.cpu().numpy())
    exact = _selection_ok(sel_logical, pages_ref, scores_ref, True)
    ref = o_ref[0, :, 0].astype(np.float32)
    if exact == H:
        err = np.abs(o.astype(np.float32) - ref).max()
        _say(f"   max|o - sim| = {err:.2e}")
        assert err <= 2e-3
    else:  # a near-tie picked differently: compare against the GPU's own selection
        mask = sim.pages_to_token_mask(sel_logical[None, :, None], S, L)
        ref2 = sim.masked_decode_attention(q, st.K, st.V, mask)[0, :, 0].astype(np.float32)
        assert np.abs(o.astype(np.float32) - ref2).max() <= 2e-3
    # the fused layer entry points (two launches, and one launch) give the
    # same bits as the three calls
    o2 = decode_layer(qd, ctrl, 0).cpu().numpy()[0]
    assert np.array_equal(bits(o2), bits(o))
    assert np.array_equal(ctrl.topk_dindices_buffer.cpu().numpy()[0], sel.cpu().numpy())
    for rep in range(3):  # the ready flags must be clear again for every launch
        ctrl.topk_dindices_buffer.fill_(-1)
        o3 = decode_layer(qd, ctrl, 0, single_launch=True).cpu().numpy()[0]
        assert np.array_equal(bits(o3), bits(o)), rep
        assert np.array_equal(ctrl.topk_dindices_buffer.cpu().numpy()[0], sel.cpu().numpy())
        assert int(ctrl.workspace[8:12].view(torch.int32).item()) == 0, "spin-wait error flag set"


@pytest.mark.parametrize("layout", [NHD, HND])
def test_dense_decode_matches_dense_attention(layout):
    from aoakv.utils import decode_sparse_attn
    _say(f"[dense-decode] layout={layout}")
    H, L = 16, 777
    q, K, V = _sim_state(21, H, L)
    ctrl = make_ctrl(H, L + 16, layout, 4096)
    prefill(ctrl, K, V)
    ctrl.begin_forward(1)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    o = decode_sparse_attn(qd, ctrl, 0, None).cpu().numpy()[0].astype(np.float32)
    ref = sim.masked_decode_attention(q, K, V, None)[0, :, 0].astype(np.float32)
    assert np.abs(o - ref).max() <= 2e-3


def _single_launch_matches(args, kwargs, o_ref, sel_ref, ws, reps=3):
    """The one-launch layer (FLAG_SINGLE_LAUNCH) repeats the two-launch result
    bit for bit, launch after launch, without its spin-wait error flag."""
    from aoakv import ops
    o, sel, scores = args[1], args[11], args[10]
    # the caller's workspace (scores handed over through an arrival counter)
    # and one with room for the score handoff words
    wsw = ops.decode_workspace(o.shape[0], o.shape[1], scores.shape[1], sel.shape[-1],
                               max_pages=args[14])
    for wsx in (ws, wsw):
        argx = args[:13] + (wsx,) + args[14:]
        for rep in range(reps):
            o.fill_(0)
            sel.fill_(-1)
            ops.sparse_decode_layer(*argx, **kwargs,
                                    flags=ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED | ops.FLAG_SINGLE_LAUNCH)
            torch.cuda.synchronize()
            assert np.array_equal(bits(o.cpu().numpy()), bits(o_ref)), rep
            assert np.array_equal(sel.cpu().numpy(), sel_ref), rep
            assert int(wsx[8:12].view(torch.int32).item()) == 0, "spin-wait error flag set"
        # every launch leaves the whole workspace zeroed
        assert int(wsx.count_nonzero().item()) == 0


def test_batched_ragged_decode_matches_simulation():
    """Config-5 style at reduced size: a batch of ragged sequences with
    per-sequence budgets min(2048, L/8), outlier keys and x4 value pages."""
    from aoakv import ops
    _say("[batched-ragged]")
    H, B = 8, 5
    g = np.random.default_rng(31)
    Ls = [int(x) for x in g.integers(900, 5000, size=B)]
    budgets = [min(2048, L // 8) for L in Ls]
    Ps = [num_pages(L) for L in Ls]
    pool = g.permutation(sum(Ps) + 10).astype(np.int32)
    kv_indices = pool[:sum(Ps)]
    indptr = np.concatenate([[0], np.cumsum(Ps)]).astype(np.int32)
    maxP = max(Ps)
    # metadata pages: one block of ceil(P/16) per sequence
    mP = [math.ceil(P / S) for P in Ps]
    m_indices = g.permutation(sum(mP) + 3).astype(np.int32)[:sum(mP)]
    m_indptr = np.concatenate([[0], np.cumsum(mP)]).astype(np.int32)
    cap = int(pool.max()) + 1
    kv = torch.zeros((cap, 2, H, S, D), dtype=torch.float16, device=DEV)
    meta = torch.zeros((int(m_indices.max()) + 1, 2, H, S, D), dtype=torch.float16, device=DEV)
    lvn = torch.zeros((cap, H), dtype=torch.float16, device=DEV)
    vmean = torch.zeros((cap, H, D), dtype=torch.float16, device=DEV)
    qs, refs, states = [], [], []
    for b, L in enumerate(Ls):
        q, K, V = _sim_state(100 + b, H, L, outlier=True)
        vpages = np.random.default_rng(200 + b).random(Ps[b]) < 0.1
        for p in np.nonzero(vpages)[0]:
            V[:, :, p * S:(p + 1) * S] = (V[:, :, p * S:(p + 1) * S].astype(np.float32) * 4).astype(np.float16)
        idx_b = torch.from_numpy(kv_indices[indptr[b]:indptr[b + 1]].copy()).to(DEV)
        midx_b = torch.from_numpy(m_indices[m_indptr[b]:m_indptr[b + 1]].copy()).to(DEV)
        kk = torch.from_numpy(np.ascontiguousarray(K[0].transpose(1, 0, 2))).to(DEV)
        vv = torch.from_numpy(np.ascontiguousarray(V[0].transpose(1, 0, 2))).to(DEV)
        ops.append_kv_cache_prefill(kk, vv, kv, idx_b, Ps[b], (L - 1) % S + 1, meta, midx_b,
                                    lvn, vmean, HND)
        st = sim.SimLayerState(K, V)
        sc, pg = sim.select_pages(st, q, budgets[b])
        qs.append(q[0, :, 0])
        states.append((st, q, sc, pg))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    lpl = t(np.array([(L - 1) % S + 1 for L in Ls], np.int32))
    kmax = max(sim.num_selected_pages(min(L, bb), S, P) for L, bb, P in zip(Ls, budgets, Ps))
    scores = torch.zeros((B, H, maxP), dtype=torch.float32, device=DEV)
    sel = torch.full((B, H, kmax), -1, dtype=torch.int32, device=DEV)
    ws = ops.decode_workspace(B, H, H, kmax)
    qd = t(np.stack(qs))
    o = torch.empty_like(qd)
    args = (qd, o, kv, t(indptr), t(kv_indices), lpl, meta, t(m_indptr), t(m_indices), lvn,
            scores, sel, 0, ws, maxP, HND)
    kwargs = dict(token_budgets=t(np.array(budgets, np.int32)))
    ops.sparse_decode_layer(*args, **kwargs)
    o_dev, sel_dev = o, sel
    o = o.cpu().numpy()
    sel = sel.cpu().numpy()
    _single_launch_matches(args, kwargs, o, sel, ws)
    o_dev.copy_(torch.from_numpy(o))
    scores = scores.cpu().numpy()
    differs_from_quest = 0
    for b, (st, q, sc, pg) in enumerate(states):
        np.testing.assert_allclose(scores[b, :, :Ps[b]], sc[0, :, 0], rtol=2e-6, atol=2e-5)
        inv = {int(p): i for i, p in enumerate(kv_indices[indptr[b]:indptr[b + 1]])}
        k = pg.shape[-1]
        sl = np.vectorize(inv.get)(sel[b, :, :k])
        _selection_ok(sl, pg, sc, True)
        mask = sim.pages_to_token_mask(sl[None, :, None], S, Ls[b])
        ref = sim.masked_decode_attention(q, st.K, st.V, mask)[0, :, 0].astype(np.float32)
        assert np.abs(o[b].astype(np.float32) - ref).max() <= 2e-3, b
        _, pq = sim.select_pages(st, q, budgets[b], True, False)
        differs_from_quest += int(any(set(pq[0, h, 0]) != set(pg[0, h, 0]) for h in range(H)))
    assert differs_from_quest >= 1, "value term never changed a selection"


@pytest.mark.parametrize("Hq,Hkv,L,budget", [(8, 4, 1500, 256), (32, 8, 32768, 2048)])
def test_gqa_selection_and_decode(Hq, Hkv, L, budget):
    """GQA: group-consistent logsumexp selection (filter_util.py:351-368)
    and decode over the shared pages; 2 query heads per kv head at 1500
    tokens, and 4 per kv head at the config-2 length and budget."""
    from aoakv import ops
    _say(f"[gqa] Hq={Hq} Hkv={Hkv} L={L} budget={budget}")
    K = randn16(13, (1, Hkv, L, D))
    V = randn16(14, (1, Hkv, L, D))
    q = randn16(15, (1, Hq, 1, D))
    P = num_pages(L)
    st = sim.SimLayerState(K, V)
    scores_ref, pages_ref = sim.select_pages(st, q, budget, True, True, Hq // Hkv)
    kv = torch.zeros((P, 2, Hkv, S, D), dtype=torch.float16, device=DEV)
    meta = torch.zeros((math.ceil(P / S), 2, Hkv, S, D), dtype=torch.float16, device=DEV)
    lvn = torch.zeros((P, Hkv), dtype=torch.float16, device=DEV)
    vmean = torch.zeros((P, Hkv, D), dtype=torch.float16, device=DEV)
    idx = torch.arange(P, dtype=torch.int32, device=DEV)
    midx = torch.arange(meta.shape[0], dtype=torch.int32, device=DEV)
    ops.append_kv_cache_prefill(torch.from_numpy(np.ascontiguousarray(K[0].transpose(1, 0, 2))).to(DEV),
                                torch.from_numpy(np.ascontiguousarray(V[0].transpose(1, 0, 2))).to(DEV),
                                kv, idx, P, (L - 1) % S + 1, meta, midx, lvn, vmean, HND)
    indptr = torch.tensor([0, P], dtype=torch.int32, device=DEV)
    mindptr = torch.tensor([0, meta.shape[0]], dtype=torch.int32, device=DEV)
    lpl = torch.tensor([(L - 1) % S + 1], dtype=torch.int32, device=DEV)
    k = pages_ref.shape[-1]
    scores = torch.zeros((1, Hkv, P), dtype=torch.float32, device=DEV)
    sel = torch.zeros((1, Hkv, k), dtype=torch.int32, device=DEV)
    ws = ops.decode_workspace(1, Hq, Hkv, k)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    o = torch.empty_like(qd)
    args = (qd, o, kv, indptr, idx, lpl, meta, mindptr, midx, lvn, scores, sel, budget, ws, P, HND)
    ops.sparse_decode_layer(*args)
    _single_launch_matches(args, {}, o.cpu().numpy(), sel.cpu().numpy(), ws)
    # a workspace with the score words once per kv head, not once per query
    # head: the one-launch layer then runs one top-k workgroup per kv head on
    # the words (no self-selecting copies), with the same bits
    from aoakv import _lib
    lib = _lib.load()
    n1 = -(-lib.aoakv_decode_workspace_size(1, Hq, Hkv, D, k) // 256) * 256 + Hkv * P * 4
    assert n1 < lib.aoakv_layer_workspace_size(1, Hq, Hkv, D, k, P)
    ws1 = torch.zeros(n1, dtype=torch.uint8, device=DEV)
    o_two, sel_two = o.cpu().numpy(), sel.cpu().numpy()
    for rep in range(2):
        o.fill_(0)
        sel.fill_(-1)
        ops.sparse_decode_layer(*args[:13], ws1, *args[14:],
                                flags=ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED | ops.FLAG_SINGLE_LAUNCH)
        torch.cuda.synchronize()
        assert np.array_equal(bits(o.cpu().numpy()), bits(o_two)), rep
        assert np.array_equal(sel.cpu().numpy(), sel_two), rep
        assert ops.workspace_error(ws1) == 0
        assert int(ws1.count_nonzero().item()) == 0, "workspace left non-zero"
    sc = scores.cpu().numpy()[0]
    np.testing.assert_allclose(sc, scores_ref[0, :, 0], rtol=1e-5, atol=1e-4)
    sl = sel.cpu().numpy()[0]
    _selection_ok(sl, pages_ref, scores_ref, True)
    grp = Hq // Hkv
    mask = np.repeat(sim.pages_to_token_mask(sl[None, :, None], S, L), grp, axis=1)
    ref = sim.masked_decode_attention(q, np.repeat(K, grp, 1), np.repeat(V, grp, 1), mask)
    assert np.abs(o.cpu().numpy()[0].astype(np.float32) - ref[0, :, 0].astype(np.float32)).max() <= 2e-3
    # one decode workgroup per kv head serving its group (FLAG_GROUPED_DECODE):
    # the same arithmetic per query head, so the same bits, in both fused
    # paths and in the standalone decode over the selection just made
    o_ref, sel_ref = o.cpu().numpy(), sel.cpu().numpy()
    base = ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED | ops.FLAG_GROUPED_DECODE
    wsw = ops.decode_workspace(1, Hq, Hkv, k, max_pages=P)
    for fl in (base, base | ops.FLAG_SINGLE_LAUNCH):
        for wsx in (ws, wsw):
            o.fill_(0)
            sel.fill_(-1)
            ops.sparse_decode_layer(*args[:13], wsx, *args[14:], flags=fl)
            torch.cuda.synchronize()
            assert np.array_equal(bits(o.cpu().numpy()), bits(o_ref)), hex(fl)
            assert np.array_equal(sel.cpu().numpy(), sel_ref), hex(fl)
            assert ops.workspace_error(wsx) == 0
            assert int(wsx.count_nonzero().item()) == 0, "workspace left non-zero"
    o2 = torch.empty_like(qd)
    ops.decode_sparse_attn(qd, o2, kv, indptr, idx, lpl, sel, budget, ws, P, Hkv, HND,
                           flags=ops.FLAG_GROUPED_DECODE)
    torch.cuda.synchronize()
    assert np.array_equal(bits(o2.cpu().numpy()), bits(o_ref))


def test_errors_are_reported_not_crashed():
    """Bad arguments come back as AoakvError before any launch."""
    from aoakv import AoakvError, ops
    kv = torch.zeros((4, 2, 8, 16, 96), dtype=torch.float16, device=DEV)   # head_dim 96
    with pytest.raises(AoakvError, match="head_dim"):
        ops.append_kv_cache_prefill(torch.zeros((3, 8, 96), dtype=torch.float16, device=DEV),
                                    torch.zeros((3, 8, 96), dtype=torch.float16, device=DEV),
                                    kv, torch.zeros(4, dtype=torch.int32, device=DEV), 1, 3,
                                    kv, torch.zeros(1, dtype=torch.int32, device=DEV),
                                    torch.zeros((4, 8), dtype=torch.float16, device=DEV),
                                    torch.zeros((4, 8, 96), dtype=torch.float16, device=DEV),
                                    HND)


@pytest.mark.parametrize("single", [False, True])
def test_page_table_longer_than_max_pages_is_flagged(single):
    """A device page table of 300 pages passed with max_pages = 200 (buffers
    sized for 200): no fault, AOAKV_WS_ERR_TRUNCATED (and nothing else) in
    the workspace error word, and the bits of the same call on the page
    table cut to 200 pages -- scores, selection and output.  Also the dense
    decode entry point.  Nothing reads or writes past the sized buffers."""
    from aoakv import ops
    _say(f"[truncation] single_launch={single}")
    H, budget, Pdev, Pmax = 8, 1024, 300, 200
    L = Pdev * S - 5
    q, K, V = _sim_state(77, H, L)
    c = make_ctrl(H, L + 16, HND, budget, shuffle=5)
    prefill(c, K, V)
    c.begin_forward(1)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    idx = c.kv_indices_with_last
    midx = c.metadata_indices
    lpl = c.kv_last_page_len_t
    t = lambda a: torch.tensor(a, dtype=torch.int32, device=DEV)
    k = min(max(3, budget // S), Pmax)
    F = ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED | (ops.FLAG_SINGLE_LAUNCH if single else 0)

    def call(P_table):
        o = torch.full_like(qd, float("nan"))
        scores = torch.zeros((1, H, Pmax), dtype=torch.float32, device=DEV)
        sel = torch.full((1, H, k), -1, dtype=torch.int32, device=DEV)
        ws = ops.decode_workspace(1, H, H, k, DEV, max_pages=Pmax)
        ops.sparse_decode_layer(qd, o, c.kv_cache.buf_layer(0), t([0, P_table]), idx, lpl,
                                c.metadata_cache.buf_layer(0), t([0, -(-P_table // S)]), midx,
                                c.v_log_norm_layer(0), scores, sel, budget, ws, Pmax, HND, F)
        torch.cuda.synchronize()
        return o, sel, scores, ops.workspace_error(ws)

    o_ref, sel_ref, sc_ref, e_ref = call(Pmax)
    o_tr, sel_tr, sc_tr, e_tr = call(Pdev)
    assert e_ref == 0
    assert e_tr == ops.WS_ERR_TRUNCATED
    assert torch.equal(o_tr, o_ref) and torch.equal(sel_tr, sel_ref)
    assert torch.equal(sc_tr, sc_ref)
    assert not torch.isnan(o_tr).any()
    # dense decode: the 300-page table with max_pages = 200 attends the
    # first 200 pages, as the 200-page table does
    outs = []
    for P_table in (Pmax, Pdev):
        ws = ops.decode_workspace(1, H, H, Pmax, DEV)
        o = torch.full_like(qd, float("nan"))
        ops.decode_sparse_attn(qd, o, c.kv_cache.buf_layer(0), t([0, P_table]), idx, lpl, None,
                               budget, ws, Pmax, H, HND)
        torch.cuda.synchronize()
        outs.append((o, ops.workspace_error(ws)))
    assert outs[0][1] == 0 and outs[1][1] == ops.WS_ERR_TRUNCATED
    assert torch.equal(outs[0][0], outs[1][0])
    # standalone top-k over the 200-entry score rows: the 300-page table is
    # cut to the row (the 200-page table's selection) and, given a
    # workspace, flagged in its error word
    if not single:
        sels = []
        for P_table in (Pmax, Pdev):
            ws = ops.decode_workspace(1, H, H, k, DEV)
            sel = torch.full((1, H, k), -1, dtype=torch.int32, device=DEV)
            ops.topk_filtering(sc_ref, t([0, P_table]), idx, lpl, budget, sel, S, ops.FLAG_FIXED,
                               workspace=ws)
            torch.cuda.synchronize()
            sels.append((sel, ops.workspace_error(ws)))
        assert sels[0][1] == 0 and sels[1][1] == ops.WS_ERR_TRUNCATED
        assert torch.equal(sels[0][0], sel_ref) and torch.equal(sels[1][0], sel_ref)


def test_one_launch_refuses_a_workspace_whose_wait_flag_is_set():
    """The wait flag set from the host (as a wait that gave up would leave
    it): the next one-launch call consumes no handoff word -- its selection,
    partial and counter regions stay untouched (scoring items may still
    write their score words, which nothing reads) -- and writes NaN outputs;
    after workspace_init the call runs normally again.  No wait is made to
    time out: the flag is planted on the host."""
    from aoakv import ops
    _say("[wait flag planted]")
    H, L, budget = 8, 4096 + 9, 1024
    q, K, V = _sim_state(78, H, L)
    c = make_ctrl(H, L + 16, HND, budget, shuffle=6)
    prefill(c, K, V)
    c.begin_forward(1)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    P = len(c.kv_cache.indicies)
    k = min(max(3, budget // S), P)
    ws = ops.decode_workspace(1, H, H, k, DEV, max_pages=P)

    def call():
        o = torch.zeros_like(qd)
        sel = torch.zeros((1, H, k), dtype=torch.int32, device=DEV)
        ops.sparse_decode_layer(qd, o, c.kv_cache.buf_layer(0), c.kv_indptr_for_append,
                                c.kv_indices_with_last, c.kv_last_page_len_t,
                                c.metadata_cache.buf_layer(0), c.metadata_indptr_for_append,
                                c.metadata_indices, c.v_log_norm_layer(0), c.scores, sel, budget,
                                ws, P, HND, ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED |
                                ops.FLAG_SINGLE_LAUNCH)
        torch.cuda.synchronize()
        return o, sel

    o_ok, sel_ok = call()
    assert ops.workspace_error(ws) == 0 and not torch.isnan(o_ok).any()
    ws[8:12].view(torch.int32).fill_(ops.WS_ERR_WAIT)     # planted by the host
    before = ws.clone()
    o_bad, _ = call()
    assert torch.isnan(o_bad).all(), "outputs must be NaN while the wait flag is set"
    from aoakv import _lib
    dec_bytes = _lib.load().aoakv_decode_workspace_size(1, H, H, 128, k)
    assert torch.equal(ws[:dec_bytes], before[:dec_bytes]), "decode regions must be untouched"
    with pytest.raises(RuntimeError, match="gave up"):
        c.workspace = ws
        c.check_errors()        # reports and re-initializes
    assert ops.workspace_error(ws) == 0
    o2, sel2 = call()
    assert torch.equal(o2, o_ok) and torch.equal(sel2, sel_ok)


@pytest.mark.parametrize("layout", [NHD, HND])
def test_decode_ignores_unwritten_slots_of_the_last_page(layout):
    """Regression: the last page's slots past the sequence are never written
    and may hold NaN.  Their probability is 0, but 0 * NaN is NaN: the decode
    must not let them in.  The cache is filled with NaN before the append,
    so every unwritten slot is NaN; sparse (two launches, one launch) and
    dense decode must match the oracle."""
    from aoakv import ops
    from aoakv.utils import decode_layer, decode_sparse_attn
    _say(f"[decode NaN slots] layout={layout}")
    H, L, budget = 8, 4096 + 9, 1024
    q, K, V = _sim_state(79, H, L)
    c = make_ctrl(H, L + 2 * S, layout, budget, shuffle=9)
    c.kv_cache.buf_layer(0).fill_(float("nan"))
    prefill(c, K, V)
    c.begin_forward(1)
    st = sim.SimLayerState(K, V)
    sc, pg = sim.select_pages(st, q, budget)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    for single in (False, True):
        o = decode_layer(qd, c, 0, single_launch=single).cpu().numpy()[0]
        assert np.isfinite(o.astype(np.float32)).all(), single
        inv = {int(p): i for i, p in enumerate(c.kv_cache.indicies)}
        sel = np.vectorize(inv.get)(c.topk_dindices_buffer.cpu().numpy()[0])
        _selection_ok(sel, pg, sc, True)
        mask = sim.pages_to_token_mask(sel[None, :, None], S, L)
        ref = sim.masked_decode_attention(q, K, V, mask)[0, :, 0].astype(np.float32)
        assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3, single
    od = decode_sparse_attn(qd, c, 0, None).cpu().numpy()[0]
    assert np.isfinite(od.astype(np.float32)).all()
    ref = sim.masked_decode_attention(q, K, V, None)[0, :, 0].astype(np.float32)
    assert np.abs(od.astype(np.float32) - ref).max() <= 2e-3
    assert ops.workspace_error(c.workspace) == 0


def test_workspace_shared_across_shrinking_selection_sizes():
    """Regression: one workspace used by calls of different selection sizes.
    Region offsets depend on the call's selection size, so a call with a
    smaller one places its handoff words where an earlier call's split-K
    partials were; every call must leave the whole workspace zero (a stale
    partial read as a page id sent a one-launch decode to a wild address)."""
    from aoakv import ops
    _say("[workspace reuse]")
    H, budget = 8, 512
    ctrls, data = [], []
    for L, seed in ((9600, 31), (4800, 32)):   # 600 and 300 pages
        q, K, V = _sim_state(seed, H, L)
        c = make_ctrl(H, L + 16, HND, budget, shuffle=seed)
        prefill(c, K, V)
        c.begin_forward(1)
        ctrls.append(c)
        data.append(torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None])
    big, small = ctrls
    ws = ops.decode_workspace(1, H, H, 600)

    def layer(c, qd, flags):
        o = torch.empty_like(qd)
        sel = torch.zeros((1, H, 300), dtype=torch.int32, device=DEV)
        P = len(c.kv_cache.indicies)
        ops.sparse_decode_layer(qd, o, c.kv_cache.buf_layer(0), c.kv_indptr_for_append,
                                c.kv_indices_with_last, c.kv_last_page_len_t,
                                c.metadata_cache.buf_layer(0), c.metadata_indptr_for_append,
                                c.metadata_indices, c.v_log_norm_layer(0), c.scores, sel, budget,
                                ws, P, HND, flags)
        return o, sel

    F = ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED
    o_ref, sel_ref = layer(small, data[1], F)              # two launches
    for rep in range(3):
        # dense decode of the 600-page sequence: partials for 75 chunks
        o_d = torch.empty_like(data[0])
        ops.decode_sparse_attn(data[0], o_d, big.kv_cache.buf_layer(0), big.kv_indptr_for_append,
                               big.kv_indices_with_last, big.kv_last_page_len_t, None, budget, ws,
                               600, H, HND)
        # one launch on the 300-page sequence: its handoff rows now lie in
        # that partial region
        o1, sel1 = layer(small, data[1], F | ops.FLAG_SINGLE_LAUNCH)
        torch.cuda.synchronize()
        assert torch.equal(o1, o_ref) and torch.equal(sel1, sel_ref), rep
        assert int(ws[8:12].view(torch.int32).item()) == 0, "spin-wait error flag set"
    assert not torch.any(ws[256:].view(torch.int32) != 0), "workspace not left zero"


@pytest.mark.parametrize("case", ["all_selected", "quest_one_page", "plain"])
def test_one_launch_score_words_every_selection_shape(case):
    """The one-launch layer with a workspace sized by
    aoakv_layer_workspace_size hands its scores to the top-k as handoff
    words.  The top-k must consume (wait for and clear) them whatever it
    selects: nothing (the quest_kernel convention with a budget of one page),
    everything (budget at or above the context), or a proper subset.
    Outputs match the two-launch path bit for bit, no wait gives up, and the
    whole workspace is zero again after every call."""
    from aoakv import ops
    _say(f"[score words] {case}")
    # k = min(max(3, min(L, budget) // 16), P) reaches P only for L a multiple of 16
    H, L = 8, (2016 if case == "all_selected" else 2000 + 7)
    budget = {"all_selected": 4096, "quest_one_page": 16, "plain": 512}[case]
    F = ops.FLAG_VALUE_AWARE | (ops.FLAG_QUEST_KERNEL if case == "quest_one_page" else ops.FLAG_FIXED)
    q, K, V = _sim_state(77, H, L)
    c = make_ctrl(H, L + 16, HND, budget, shuffle=77)
    prefill(c, K, V)
    c.begin_forward(1)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    P = len(c.kv_cache.indicies)
    kcols = P
    ws_words = ops.decode_workspace(1, H, H, kcols, max_pages=P)
    ws_plain = ops.decode_workspace(1, H, H, kcols)

    def layer(ws, flags):
        o = torch.empty_like(qd)
        sel = torch.full((1, H, kcols), -1, dtype=torch.int32, device=DEV)
        ops.sparse_decode_layer(qd, o, c.kv_cache.buf_layer(0), c.kv_indptr_for_append,
                                c.kv_indices_with_last, c.kv_last_page_len_t,
                                c.metadata_cache.buf_layer(0), c.metadata_indptr_for_append,
                                c.metadata_indices, c.v_log_norm_layer(0), c.scores, sel, budget,
                                ws, P, HND, flags)
        torch.cuda.synchronize()
        return o, sel

    o_ref, sel_ref = layer(ws_plain, F)  # two launches
    for rep in range(3):
        o1, sel1 = layer(ws_words, F | ops.FLAG_SINGLE_LAUNCH)
        assert torch.equal(o1, o_ref) and torch.equal(sel1, sel_ref), rep
        assert int(ws_words[8:12].view(torch.int32).item()) == 0, "spin-wait error flag set"
        assert int(ws_words.count_nonzero().item()) == 0, "workspace not left zero"


def _repeated_batch_one_launch(H, L, budget, lpls, seed):
    """One sequence's cache read by len(lpls) sequences of a batch (the same
    pages, last-page lengths lpls).  Runs the one-launch layer with score
    words three times and checks it against the two-launch path: outputs
    and selections of the well-formed sequences bit for bit, no wait given
    up, and the whole workspace zero after every call."""
    from aoakv import ops
    B = len(lpls)
    q, K, V = _sim_state(seed, H, L)
    c = make_ctrl(H, L + 16, HND, budget, shuffle=seed)
    prefill(c, K, V)
    c.begin_forward(1)
    P = len(c.kv_cache.indicies)
    mP = int(c.metadata_indices.numel())
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None].repeat(B, 1, 1)
    indptr = torch.arange(0, (B + 1) * P, P, dtype=torch.int32, device=DEV)
    idx = c.kv_indices_with_last[:P].repeat(B)
    lpl = torch.tensor(lpls, dtype=torch.int32, device=DEV)
    mindptr = torch.arange(0, (B + 1) * mP, mP, dtype=torch.int32, device=DEV)
    midx = c.metadata_indices.repeat(B)
    scores = torch.zeros((B, H, P), dtype=torch.float32, device=DEV)
    kcols = sim.num_selected_pages(min(L, budget), S, P)
    ws_words = ops.decode_workspace(B, H, H, kcols, max_pages=P)
    ws_plain = ops.decode_workspace(B, H, H, kcols)

    def layer(ws, flags):
        o = torch.zeros_like(qd)
        sel = torch.full((B, H, kcols), -1, dtype=torch.int32, device=DEV)
        ops.sparse_decode_layer(qd, o, c.kv_cache.buf_layer(0), indptr, idx, lpl,
                                c.metadata_cache.buf_layer(0), mindptr, midx,
                                c.v_log_norm_layer(0), scores, sel, budget, ws, P, HND, flags)
        torch.cuda.synchronize()
        return o, sel

    F = ops.FLAG_VALUE_AWARE | ops.FLAG_FIXED
    good = [b for b, x in enumerate(lpls) if 1 <= x <= S]
    o_ref, sel_ref = layer(ws_plain, F)  # two launches
    for rep in range(3):
        o1, sel1 = layer(ws_words, F | ops.FLAG_SINGLE_LAUNCH)
        assert torch.equal(o1[good], o_ref[good]) and torch.equal(sel1[good], sel_ref[good]), rep
        assert int(ws_words[8:12].view(torch.int32).item()) == 0, "spin-wait error flag set"
        assert int(ws_words.count_nonzero().item()) == 0, "workspace not left zero"


def test_one_launch_malformed_sequence_still_clears_score_words():
    """A batch whose second sequence has a last-page length of 0 (malformed:
    no decode item attends it).  The one-launch layer still scores its pages
    and hands the scores over as words; its first decode item must wait for
    and clear them, so the whole workspace is zero again after every call."""
    _say("[malformed sequence, score words]")
    L = 2007
    _repeated_batch_one_launch(8, L, 512, [(L - 1) % S + 1, 0], 91)


def test_one_launch_more_workgroups_than_resident():
    """8 sequences x 32 heads x 8 decode chunks: more workgroups than the GPU
    holds at once, so the one-launch layer keeps its top-k workgroups and the
    selection handoff (the decode items do not select for themselves)."""
    _say("[one launch, 2048 decode items]")
    L = 2007
    _repeated_batch_one_launch(32, L, 1024, [(L - 1) % S + 1] * 8, 93)
