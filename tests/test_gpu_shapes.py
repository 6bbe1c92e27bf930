"""GPU parity of the head dims and page sizes beyond (128, 16) against the
oracle, through the same C ABI: head_dim 64 / 128 / 256 (the reference's
SWITCH_HEAD_DIM, decode_page.cuh:718-760, decode_attn.cuh:1159) and page
sizes 1..32 (its page tests sweep 1, 3, 7, 16, 31, test_page.cu:600-683; its
prefill takes 1, 8, 16, 32, prefill.cuh:1032-1036).  These shapes run the
kernels of csrc/generic.hip.

Bars as for the tuned shape: K/V storage, Kmax/Kmin, V̄ and log-norm
bit-exact after a prefill and decode appends that cross pages; page scores
within rtol 2e-6; selections equal up to near-ties; decode outputs within
2e-3 of the simulation over the same pages; the three-call decode, the
fused layer call and its one-launch flag give the same bits; prefill within
2e-3 of fp64 causal attention; RoPE within one fp16 rounding of the exactly
rounded rotation, and fused RoPE + append equal to RoPE then append.
"""
import math
import sys

import numpy as np
import pytest
import torch

from helpers import HND, NHD, bits, randn16, read_filters, read_kv
from oracle import sim

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (head_dim, page_size, layout)
SHAPES = [(64, 16, HND), (256, 16, NHD), (128, 8, HND), (128, 32, NHD), (128, 1, HND),
          (128, 7, NHD), (128, 31, HND), (64, 3, NHD), (256, 32, HND)]


@pytest.fixture(scope="module", autouse=True)
def _aoakv():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    yield


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _ctrl(H, D, S, max_len, layout, budget, hkv=None, value_aware=True, shuffle=1):
    from aoakv.utils import InferenceController
    return InferenceController(1, H, D, S, budget // S, max_len, torch.float16, DEV,
                               layout=layout, num_kv_heads=hkv, fixed=True,
                               value_aware=value_aware, shuffle_seed=shuffle)


def _prefill(c, K, V):
    from aoakv.utils import append_kv
    L = K.shape[2]
    c.prepare_metadata(L)
    c.begin_forward(L)
    append_kv(torch.from_numpy(np.ascontiguousarray(K[0].transpose(1, 0, 2))).to(DEV),
              torch.from_numpy(np.ascontiguousarray(V[0].transpose(1, 0, 2))).to(DEV), c, 0)


def _append(c, kn, vn):
    from aoakv.utils import append_kv
    c.prepare_metadata(1)
    c.begin_forward(1)
    append_kv(torch.from_numpy(kn[0, :, 0][None].copy()).to(DEV),
              torch.from_numpy(vn[0, :, 0][None].copy()).to(DEV), c, 0)


def _check_metadata(c, st):
    L, S = st.kv_len, st.chunk_size
    P = math.ceil(L / S)
    pages = c.kv_cache.indicies
    torch.cuda.synchronize()
    K, V = read_kv(c.kv_cache.buf_layer(0), c.layout, pages, L)
    assert np.array_equal(bits(K), bits(st.K)) and np.array_equal(bits(V), bits(st.V)), "K/V"
    pf = read_filters(c.metadata_cache.buf_layer(0), c.layout, c.metadata_cache.indicies, P)
    assert np.array_equal(bits(pf), bits(st.page_filters)), "Kmax/Kmin"
    vm = c.v_mean_layer(0).cpu().numpy()[pages][None].transpose(0, 2, 1, 3)
    assert np.array_equal(bits(vm), bits(st.v_mean)), "page mean of V"
    lvn = c.v_log_norm_layer(0).cpu().numpy()[pages].T[None]
    assert np.array_equal(bits(lvn), bits(sim.log_v_norm(st.v_mean))), "log-norm"


@pytest.mark.parametrize("D,S,layout", SHAPES)
def test_metadata_bit_exact(D, S, layout):
    _say(f"[shapes] metadata D={D} S={S} layout={layout}")
    H, L0, steps = 4, 37 * S + 5 if S > 1 else 300, 2 * S + 3
    K, V = randn16(D + S, (1, H, L0, D)), randn16(D + S + 1, (1, H, L0, D))
    kn, vn = randn16(7, (steps, 1, H, 1, D)), randn16(8, (steps, 1, H, 1, D))
    c = _ctrl(H, D, S, L0 + steps + S, layout, 64 * S, shuffle=S)
    _prefill(c, K, V)
    st = sim.SimLayerState(K, V, S)
    _check_metadata(c, st)
    for s in range(steps):
        _append(c, kn[s], vn[s])
        st.append(kn[s], vn[s])
    _check_metadata(c, st)


@pytest.mark.parametrize("D,S,layout,group,value_aware", [
    (64, 16, HND, 1, True), (256, 16, NHD, 1, True), (128, 8, HND, 2, True),
    (128, 32, NHD, 1, False), (128, 7, HND, 1, True), (256, 32, HND, 4, True),
    (64, 3, NHD, 1, True), (128, 1, HND, 1, True)])
def test_decode_matches_simulation(D, S, layout, group, value_aware):
    """Scores, selection and sparse attention of one decode step after a
    prefill and a few appends; the three calls, the fused layer call (with
    and without the one-launch flag, which these shapes run as two
    launches) and the dense decode."""
    from aoakv import ops
    from aoakv.utils import decode_estimate, decode_layer, decode_sparse_attn, decode_topk
    _say(f"[shapes] decode D={D} S={S} layout={layout} group={group} va={value_aware}")
    Hkv = 4
    Hq = Hkv * group
    L0 = 600 * S // 16 + 11 if S >= 8 else 400
    budget = max(24 * S, 3 * S)
    K = randn16(D * 3 + S, (1, Hkv, L0, D))
    V = randn16(D * 3 + S + 1, (1, Hkv, L0, D))
    c = _ctrl(Hq, D, S, L0 + 4 * S, layout, budget, hkv=Hkv, value_aware=value_aware, shuffle=2)
    _prefill(c, K, V)
    st = sim.SimLayerState(K, V, S)
    kn, vn = randn16(31, (3, 1, Hkv, 1, D)), randn16(32, (3, 1, Hkv, 1, D))
    for s in range(3):
        _append(c, kn[s], vn[s])
        st.append(kn[s], vn[s])
    q = randn16(33, (1, Hq, 1, D))
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    c.begin_forward(1)
    assert c.need_estimate()
    L, P = st.kv_len, math.ceil(st.kv_len / S)
    scores = decode_estimate(qd, c, 0).cpu().numpy()
    sc_ref, pg_ref = sim.select_pages(st, q, budget, True, value_aware, group)
    np.testing.assert_allclose(scores, sc_ref[0, :, 0], rtol=2e-6, atol=2e-5)
    decode_topk(c.scores[0, :, :P], c)
    sel = c.topk_dindices_buffer[0].cpu().numpy()
    inv = {p: i for i, p in enumerate(c.kv_cache.indicies)}
    mine = np.array([[inv[int(x)] for x in row] for row in sel])
    for h in range(Hkv):
        ok, why = sim.selection_matches(mine[h], pg_ref[0, h, 0], sc_ref[0, h, 0], True)
        assert ok, (h, why)
    o3 = decode_sparse_attn(qd, c, 0, c.topk_dindices_buffer).cpu().numpy()[0]
    ref = sim.sparse_decode_attention(q, np.repeat(st.K, group, 1), np.repeat(st.V, group, 1),
                                      np.repeat(mine[None, :, None, :], group, 1), S, L)
    assert np.abs(o3.astype(np.float32) - ref[0, :, 0].astype(np.float32)).max() <= 2e-3
    for single in (False, True):
        o1 = decode_layer(qd, c, 0, single_launch=single).cpu().numpy()[0]
        assert np.array_equal(bits(o1), bits(o3)), single
    assert ops.workspace_error(c.workspace) == 0
    od = decode_sparse_attn(qd, c, 0, None).cpu().numpy()[0]
    dref = sim.masked_decode_attention(q, np.repeat(st.K, group, 1), np.repeat(st.V, group, 1),
                                       None)
    assert np.abs(od.astype(np.float32) - dref[0, :, 0].astype(np.float32)).max() <= 2e-3


@pytest.mark.parametrize("D,S,layout,group,value_aware", [
    (64, 16, HND, 1, True), (256, 32, NHD, 1, False), (128, 8, HND, 2, True),
    (128, 1, NHD, 1, True), (64, 7, HND, 4, True)])
def test_quest_kernel_convention_matches_oracle(D, S, layout, group, value_aware):
    """AOAKV_FLAG_QUEST_KERNEL through the generic kernels: P - 1 pages
    scored (the last one is not), the k - 1 best of them selected, the last
    page attended after them; against the oracle's quest_kernel_pages, as
    test_gpu_quest_kernel.py does for (128, 16).  The three calls, the fused
    layer call and its one-launch flag give the same bits."""
    from aoakv.utils import (InferenceController, decode_estimate, decode_layer,
                             decode_sparse_attn, decode_topk)
    _say(f"[shapes] quest_kernel D={D} S={S} layout={layout} group={group} va={value_aware}")
    Hkv, pb = 4, 23
    Hq = Hkv * group
    L = 40 * S + 5 if S > 1 else 300
    K = randn16(D * 5 + S, (1, Hkv, L, D))
    V = randn16(D * 5 + S + 1, (1, Hkv, L, D))
    q = randn16(D * 5 + S + 2, (1, Hq, 1, D))
    c = InferenceController(1, Hq, D, S, pb, L + S, torch.float16, DEV, layout=layout,
                            num_kv_heads=Hkv, value_aware=value_aware, shuffle_seed=S + 9,
                            semantics="quest_kernel")
    _prefill(c, K[:, :, :-1], V[:, :, :-1])
    c.end_forward()
    _append(c, K[:, :, -1:], V[:, :, -1:])
    st = sim.SimLayerState(K[:, :, :-1], V[:, :, :-1], S)
    o_ref, sc_ref, pg_ref = sim.decode_step(st, q, K[:, :, -1:], V[:, :, -1:], pb * S,
                                            fixed=False, value_aware=value_aware,
                                            num_key_value_groups=group, semantics="quest_kernel")
    P = math.ceil(L / S)
    k = min(pb, P)
    assert c.need_estimate() and c.num_selected_pages() == k < P
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    scores = decode_estimate(qd, c, 0).cpu().numpy()
    assert scores.shape == (Hkv, P - 1)                  # the last page is not scored
    np.testing.assert_allclose(scores, sc_ref[0, :, 0, :P - 1], rtol=2e-6, atol=2e-5)
    sel = decode_topk(c.scores[0, :, :P - 1], c).cpu().numpy()
    assert sel.shape == (Hkv, k - 1)
    inv = {p: i for i, p in enumerate(c.kv_cache.indicies)}
    mine = np.array([[inv[int(x)] for x in row] for row in sel])
    exact = True
    for h in range(Hkv):
        got = np.append(mine[h], P - 1)
        ok, why = sim.selection_matches(got, pg_ref[0, h, 0], sc_ref[0, h, 0], forced={P - 1})
        assert ok, (h, why)
        assert P - 1 not in set(mine[h].tolist())
        exact &= why == "exact"
    o = decode_sparse_attn(qd, c, 0, c.topk_dindices_buffer).cpu().numpy()[0]
    pages = np.concatenate([mine, np.full((Hkv, 1), P - 1)], axis=1)
    mask = np.repeat(sim.pages_to_token_mask(pages[None, :, None], S, L), group, 1)
    ref = sim.masked_decode_attention(q, np.repeat(st.K, group, 1), np.repeat(st.V, group, 1),
                                      mask)[0, :, 0]
    assert np.abs(o.astype(np.float32) - ref.astype(np.float32)).max() <= 2e-3
    if exact:
        assert np.abs(o.astype(np.float32) - o_ref[0, :, 0].astype(np.float32)).max() <= 2e-3
    for single in (False, True):
        c.topk_dindices_buffer.fill_(-1)
        o1 = decode_layer(qd, c, 0, single_launch=single).cpu().numpy()[0]
        assert np.array_equal(bits(o1), bits(o)), single
        assert np.array_equal(c.topk_dindices_buffer.cpu().numpy()[0], sel), single
    from aoakv import ops
    assert ops.workspace_error(c.workspace) == 0


@pytest.mark.parametrize("D,S,layout", [(128, 1, HND), (64, 4, NHD)])
def test_decode_beyond_the_split_k_limit(D, S, layout):
    """10000 pages per head, 9000 of them selected: more than the 8192 pages
    per head (1024 chunks) the tuned kernels' split-K merge holds.  The
    generic kernels' merge (chunk order, one workgroup) takes the 1125
    chunks; sparse and dense decode against the oracle."""
    from aoakv import ops
    from aoakv.utils import decode_estimate, decode_layer, decode_sparse_attn, decode_topk
    _say(f"[shapes] beyond split-K D={D} S={S} layout={layout}")
    H, P, k = 2, 10000, 9000
    L = (P - 1) * S + 1
    K = randn16(D + 71, (1, H, L, D))
    V = randn16(D + 72, (1, H, L, D))
    q = randn16(D + 73, (1, H, 1, D))
    c = _ctrl(H, D, S, L + S, layout, k * S, shuffle=S + 3)
    _prefill(c, K, V)
    c.begin_forward(1)
    st = sim.SimLayerState(K, V, S)
    qd = torch.from_numpy(q[0, :, 0].copy()).to(DEV)[None]
    assert c.need_estimate() and c.num_selected_pages() == k
    scores = decode_estimate(qd, c, 0).cpu().numpy()
    sc_ref, pg_ref = sim.select_pages(st, q, k * S, True, True, 1)
    np.testing.assert_allclose(scores, sc_ref[0, :, 0], rtol=2e-6, atol=2e-5)
    decode_topk(c.scores[0, :, :P], c)
    sel = c.topk_dindices_buffer[0].cpu().numpy()
    inv = {p: i for i, p in enumerate(c.kv_cache.indicies)}
    mine = np.array([[inv[int(x)] for x in row] for row in sel])
    for h in range(H):
        ok, why = sim.selection_matches(mine[h], pg_ref[0, h, 0], sc_ref[0, h, 0], True)
        assert ok, (h, why)
    o = decode_sparse_attn(qd, c, 0, c.topk_dindices_buffer).cpu().numpy()[0]
    ref = sim.sparse_decode_attention(q, st.K, st.V, mine[None, :, None, :], S, L)
    assert np.abs(o.astype(np.float32) - ref[0, :, 0].astype(np.float32)).max() <= 2e-3
    o1 = decode_layer(qd, c, 0).cpu().numpy()[0]
    assert np.array_equal(bits(o1), bits(o))
    od = decode_sparse_attn(qd, c, 0, None).cpu().numpy()[0]
    dref = sim.masked_decode_attention(q, st.K, st.V, None)
    assert np.abs(od.astype(np.float32) - dref[0, :, 0].astype(np.float32)).max() <= 2e-3
    assert ops.workspace_error(c.workspace) == 0


@pytest.mark.parametrize("D,S,layout", [(64, 16, HND), (256, 16, NHD), (128, 8, NHD),
                                        (128, 32, HND), (128, 8, HND), (128, 32, NHD),
                                        (64, 8, NHD), (64, 32, HND), (64, 16, NHD),
                                        (128, 1, HND), (256, 7, HND), (64, 1, NHD),
                                        (128, 2, NHD), (64, 4, HND), (128, 4, NHD),
                                        (256, 1, HND), (256, 32, HND), (256, 8, NHD)])
@pytest.mark.parametrize("L,Lq,group", [(300, 300, 1), (333, 70, 2), (1100, 1100, 1),
                                        (777, 300, 4)])
def test_prefill_matches_causal_attention(D, S, layout, L, Lq, group):
    from aoakv import ops
    _say(f"[shapes] prefill D={D} S={S} layout={layout} L={L} Lq={Lq} group={group}")
    if L > 1000 and not (D in (64, 128, 256) and S in (1, 2, 4, 8, 16, 32)):
        pytest.skip("the long case is for the MFMA kernel's page sizes (several query tiles)")
    Hkv = 2
    Hq = Hkv * group
    q = randn16(L + D, (Lq, Hq, D), 0.5)
    k = randn16(L + D + 1, (L, Hkv, D), 0.5)
    v = randn16(L + D + 2, (L, Hkv, D), 0.5)
    c = _ctrl(Hq, D, S, L + S, layout, 64 * S, hkv=Hkv, shuffle=5)
    c.prepare_metadata(L)
    c.begin_forward(L)
    from aoakv.utils import append_kv
    append_kv(torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV), c, 0)
    o = ops.prefill_with_paged_kv_cache(torch.from_numpy(q).to(DEV), c.kv_cache.buf_layer(0),
                                        c.kv_indices_with_last, len(c.kv_cache.indicies),
                                        c.kv_cache.last_page_len, layout).cpu().numpy()
    ref = sim.causal_prefill_rows(q, np.repeat(k, group, 1), np.repeat(v, group, 1))
    assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3


def _rope_err(got, x, ref):
    """|got - ref| over one fp16 rounding plus fp32 evaluation of the terms."""
    a = np.abs(ref).astype(np.float16)
    ulp = np.maximum(np.spacing(a).astype(np.float64), 2.0 ** -24)
    xf = np.abs(x.astype(np.float64))
    half = x.shape[-1] // 2
    terms = xf + np.concatenate([xf[..., half:], xf[..., :half]], -1)
    return np.abs(got.astype(np.float64) - ref) / (ulp + 2.0 ** -21 * terms)


@pytest.mark.parametrize("D", [64, 256])
def test_rope_and_fused_rope_append(D):
    """apply_rope_in_place at head_dim 64 / 256 against the oracle's exactly
    rounded rotation (frequencies rcp_scale * rcp_theta^(2i/D)), and the fused
    RoPE + append equal to RoPE then append."""
    from aoakv import ops
    _say(f"[shapes] rope D={D}")
    N, Hq, Hkv, past = 37, 4, 2, 1000
    q = randn16(D, (N, Hq, D))
    k = randn16(D + 1, (N, Hkv, D))
    qd, kd = torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV)
    ops.apply_rope_in_place(qd, kd, past, rope_scale=4.0, rope_theta=5e5)
    pos = past + np.arange(N)
    for got, x in ((qd, q), (kd, k)):
        ref = sim.apply_rope(x, pos, 4.0, 5e5)
        assert _rope_err(got.cpu().numpy(), x, ref).max() <= 1.0
    # fused: one decode token per step on a prefilled cache
    S, L0 = 16, 77
    K, V = randn16(5, (1, Hkv, L0, D)), randn16(6, (1, Hkv, L0, D))
    outs = []
    for fused in (False, True):
        c = _ctrl(Hq, D, S, L0 + 40, HND, 256, hkv=Hkv, shuffle=9)
        _prefill(c, K, V)
        qs, ks, vs = randn16(40, (5, 1, Hq, D)), randn16(41, (5, 1, Hkv, D)), randn16(42, (5, 1, Hkv, D))
        for t in range(5):
            c.prepare_metadata(1)
            c.begin_forward(1)
            qt, kt = torch.from_numpy(qs[t]).to(DEV), torch.from_numpy(ks[t]).to(DEV)
            vt = torch.from_numpy(vs[t]).to(DEV)
            if fused:
                ops.rope_append_kv_cache_decode(
                    qt, kt, vt, c.kv_cache.buf_layer(0), c.kv_indptr_for_append,
                    c.kv_indices_with_last, c.kv_last_page_len_t, c.metadata_cache.buf_layer(0),
                    c.metadata_indptr_for_append, c.metadata_indices, c.v_log_norm[0],
                    c.v_mean[0], HND)
            else:
                ops.apply_rope_in_place(qt, kt, L0 + t)
                ops.append_kv_cache_decode(
                    kt, vt, c.kv_cache.buf_layer(0), c.kv_indptr_for_append,
                    c.kv_indices_with_last, c.kv_last_page_len_t, c.metadata_cache.buf_layer(0),
                    c.metadata_indptr_for_append, c.metadata_indices, c.v_log_norm[0],
                    c.v_mean[0], HND)
            outs.append((qt.cpu().numpy(), kt.cpu().numpy()))
        torch.cuda.synchronize()
        # the sequence's pages only (the pools' other pages are never written)
        pages, L = c.kv_cache.indicies, c.kv_cache.seqlen
        Kc, Vc = read_kv(c.kv_cache.buf_layer(0), HND, pages, L)
        pf = read_filters(c.metadata_cache.buf_layer(0), HND, c.metadata_cache.indicies,
                          len(pages))
        outs.append((Kc, Vc, pf, c.v_mean[0].cpu().numpy()[pages],
                     c.v_log_norm[0].cpu().numpy()[pages]))
    half = len(outs) // 2
    for a, b in zip(outs[:half], outs[half:]):
        for x, y in zip(a, b):
            assert np.array_equal(bits(x), bits(y))


def test_unsupported_shapes_are_refused():
    """head_dim outside 64 / 128 / 256 and page sizes outside 1..32 are
    refused by the entry points, not run."""
    from aoakv.utils import InferenceController
    from aoakv import _lib
    for D, S in ((96, 16), (128, 33), (128, 64)):
        c = InferenceController(1, 2, D, S, 4, 200, torch.float16, DEV, layout=HND)
        c.prepare_metadata(50)
        c.begin_forward(50)
        from aoakv.utils import append_kv
        k = torch.zeros((50, 2, D), dtype=torch.float16, device=DEV)
        with pytest.raises(RuntimeError, match="unsupported"):
            append_kv(k, k, c, 0)
    assert _lib.load() is not None
