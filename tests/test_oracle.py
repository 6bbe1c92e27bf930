"""Pin the numpy oracle (oracle/sim.py) before trusting it.

Three kinds of checks, chosen so a plausible mistake (dropped term, wrong
rounding point, wrong index, transposed operand) fails at least one:

1. golden fixtures written from the reference's own ``filter_util.py``
   (tests/golden/make_golden.py);
2. torch's library routines the reference calls, on the whole fp16 domain
   where it is small (log) and on stress inputs (mean / norm);
3. closed forms and invariants (brute force on tiny inputs).
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import sim

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_sim.npz"))


def randn16(seed, shape, scale=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


# ---------------------------------------------------------------- fixtures

@pytest.mark.parametrize("L", [17, 31, 256, 4103])
def test_metadata_matches_reference_fixture(L):
    nh = 4 if L < 4096 else 2
    K = randn16(100 + L, (1, nh, L, 128))
    V = randn16(200 + L, (1, nh, L, 128))
    pf = sim.get_max_min_filters(K, 16)
    vm = sim.compute_page_v_mean(L, 16, V)
    lvn = sim.log_v_norm(vm)
    assert np.array_equal(bits(pf), bits(GOLD[f"meta_L{L}_filters"]))
    assert np.array_equal(bits(vm), bits(GOLD[f"meta_L{L}_vmean"]))
    assert np.array_equal(bits(lvn), bits(GOLD[f"meta_L{L}_lvn"]))


def test_decode_trace_matches_reference_fixture():
    nh, d, L0, steps = 4, 128, 21, 40
    K = randn16(300, (1, nh, L0, d))
    V = randn16(301, (1, nh, L0, d))
    kn = randn16(302, (steps, 1, nh, 1, d))
    vn = randn16(303, (steps, 1, nh, 1, d))
    st = sim.SimLayerState(K, V)
    for s in range(steps):
        st.append(kn[s], vn[s])
        assert np.array_equal(bits(st.v_mean[:, :, -1]),
                              bits(GOLD["trace_vmean_last_page_per_step"][s])), s
        assert np.array_equal(bits(st.page_filters[:, :, -1]),
                              bits(GOLD["trace_filters_last_page_per_step"][s])), s
    assert np.array_equal(bits(st.page_filters), bits(GOLD["trace_final_filters"]))
    assert np.array_equal(bits(st.v_mean), bits(GOLD["trace_final_vmean"]))


def _selection_inputs(tag):
    seed, nh, nkvh, L, budget, fixed, va, outlier = [int(x) for x in GOLD[f"sel_{tag}_params"]]
    d = 128
    K = randn16(seed, (1, nkvh, L, d))
    V = randn16(seed + 1, (1, nkvh, L, d))
    q = randn16(seed + 2, (1, nh, 1, d))
    if outlier:
        ch = np.random.default_rng(seed + 3).permutation(d)[:4]
        K[..., ch] = (K[..., ch].astype(np.float32) * 8).astype(np.float16)
    if tag == "ties":
        for dst in range(9, 21):
            K[:, :, dst * 16:(dst + 1) * 16] = K[:, :, 5 * 16:6 * 16]
            V[:, :, dst * 16:(dst + 1) * 16] = V[:, :, 5 * 16:6 * 16]
    return q, K, V, nh, nkvh, L, budget, bool(fixed), bool(va)


SEL_TAGS = ["c1_fixed", "c1_free", "c1_quest", "ragged_outlier", "tiny", "gqa", "gqa_quest", "ties"]


@pytest.mark.parametrize("tag", SEL_TAGS)
def test_selection_matches_reference_fixture(tag):
    q, K, V, nh, nkvh, L, budget, fixed, va = _selection_inputs(tag)
    st = sim.SimLayerState(K, V)
    scores, pages = sim.select_pages(st, q, budget, fixed, va, nh // nkvh)
    # the page bound agrees with the reference's to fp32 summation-order noise
    pb = sim.page_bound(q, st.page_filters, nh // nkvh)[0]
    ref_pb = GOLD[f"sel_{tag}_page_bound"]
    np.testing.assert_allclose(pb, ref_pb, rtol=2e-6, atol=2e-5)
    ref_sel = GOLD[f"sel_{tag}_pages"]
    exact = 0
    for hh in range(ref_sel.shape[0]):
        kvh = hh // (nh // nkvh)
        ok, why = sim.selection_matches(pages[0, kvh, 0], ref_sel[hh], scores[0, kvh, 0], fixed)
        assert ok, (tag, hh, why)
        exact += why == "exact"
    if tag != "ties":
        assert exact == ref_sel.shape[0], f"{tag}: only {exact} heads exact"


def test_planted_mistakes_fail_the_fixture():
    """Mistakes planted in the oracle (on the CPU) must be caught."""
    q, K, V, nh, nkvh, L, budget, fixed, va = _selection_inputs("c1_fixed")
    st = sim.SimLayerState(K, V)
    ref_sel = GOLD["sel_c1_fixed_pages"]
    scores, _ = sim.select_pages(st, q, budget, fixed, True)
    k = ref_sel.shape[1]

    def n_fail(pages):
        return sum(not sim.selection_matches(pages[hh], ref_sel[hh], scores[0, hh, 0], fixed)[0]
                   for hh in range(nh))

    # dropped value term
    chunk = sim.page_bound(q, st.page_filters)[:, :, None, :]
    no_v = sim.topk_pages((2 * (chunk / np.float32(math.sqrt(128))))[:, :, 0], k, fixed)[0]
    assert n_fail(no_v) > nh // 2
    # value term with the wrong sign
    lvn = sim.log_v_norm(st.v_mean)
    wrong = sim.value_aware_page_scores(chunk, (-lvn.astype(np.float32)).astype(np.float16), 1, 128)
    assert n_fail(sim.topk_pages(wrong[:, :, 0], k, fixed)[0]) > nh // 2
    # value term of page p read at p // 16 (the index slip of the kernel tree)
    slip = sim.value_aware_page_scores(chunk, lvn[:, :, np.arange(lvn.shape[-1]) // 16], 1, 128)
    assert n_fail(sim.topk_pages(slip[:, :, 0], k, fixed)[0]) > nh // 2
    # bound from Kmax only (the min/max choice by sign of q dropped)
    only_max = np.concatenate([st.page_filters[:, :, :, :1]] * 2, axis=3)
    om = sim.value_aware_page_scores(sim.page_bound(q, only_max)[:, :, None, :], lvn, 1, 128)
    assert n_fail(sim.topk_pages(om[:, :, 0], k, fixed)[0]) > nh // 2
    # 1/sqrt(d) scaling dropped
    nsc = sim.value_aware_page_scores(chunk * np.float32(math.sqrt(128)), lvn, 1, 128)
    assert n_fail(sim.topk_pages(nsc[:, :, 0], k, fixed)[0]) > nh // 2


def test_decode_attention_matches_torch_fixture():
    nh, d, L = 4, 128, 300
    q = randn16(400, (1, nh, 1, d))
    K = randn16(401, (1, nh, L, d))
    V = randn16(402, (1, nh, L, d))
    mask = GOLD["attn_mask"]
    o = sim.masked_decode_attention(q, K, V, mask)
    ref = GOLD["attn_out"]
    err = np.abs(o.astype(np.float32) - ref.astype(np.float32)).max()
    assert err <= 2e-3
    assert (bits(o) == bits(ref)).mean() > 0.95


# ---------------------------------------------------------------- library routines

def test_log_fp16_whole_domain_matches_torch():
    allh = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)
    ref = torch.log(torch.from_numpy(allh.copy())).numpy()
    assert np.array_equal(bits(sim.log_fp16(allh)), bits(ref))


def test_mean_and_norm_match_torch_on_stress_inputs():
    g = torch.Generator().manual_seed(5)
    e = torch.randint(-14, 10, (1, 4, 64 * 16, 128), generator=g).float()
    v = (torch.randn(1, 4, 64 * 16, 128, generator=g) * torch.exp2(e)).clamp(-6e4, 6e4).half()
    ref = v.reshape(1, 4, 64, 16, 128).mean(dim=3).numpy()
    assert np.array_equal(bits(sim.compute_page_v_mean(64 * 16, 16, v.numpy())), bits(ref))
    part = v[:, :, :13]
    refp = part.mean(dim=2, keepdim=True).numpy()
    assert np.array_equal(bits(sim.compute_page_v_mean(13, 16, part.numpy())), bits(refp))
    nref = v.norm(p=2, dim=-1).numpy()
    assert np.array_equal(bits(sim.norm_fp16(v.numpy())), bits(nref))


def test_running_mean_matches_torch_ops():
    g = torch.Generator().manual_seed(6)
    m = torch.randn(8, 128, generator=g).half()
    x = torch.randn(8, 128, generator=g).half()
    for n in range(1, 16):
        ref = ((m * n + x) / (n + 1)).numpy()
        assert np.array_equal(bits(sim.update_mean_filter(m.numpy(), x.numpy(), n)), bits(ref))


# ---------------------------------------------------------------- closed forms / invariants

def test_filters_bound_every_key_and_are_attained():
    K = randn16(1, (1, 3, 53, 128))
    pf = sim.get_max_min_filters(K, 16)
    for p in range(pf.shape[2]):
        blk = K[:, :, p * 16:(p + 1) * 16].astype(np.float32)
        assert np.array_equal(pf[:, :, p, 0].astype(np.float32), blk.max(axis=2))
        assert np.array_equal(pf[:, :, p, 1].astype(np.float32), blk.min(axis=2))


def test_page_bound_is_an_upper_bound_and_tight_for_single_token_pages():
    q = randn16(2, (1, 2, 1, 128))
    K = randn16(3, (1, 2, 64, 128))
    pf = sim.get_max_min_filters(K, 16)
    pb = sim.page_bound(q, pf)
    qk = np.einsum("bhd,bhld->bhl", q[:, :, 0].astype(np.float64), K.astype(np.float64))
    pmax = qk.reshape(1, 2, 4, 16).max(-1)
    assert np.all(pb >= pmax - 1e-4)
    # one-token pages: bound == q.k exactly (up to fp32 rounding)
    pf1 = sim.get_max_min_filters(K, 1)
    np.testing.assert_allclose(sim.page_bound(q, pf1), qk, rtol=1e-5, atol=1e-4)


def test_k_rule_and_fixed_forcing():
    assert sim.num_selected_pages(2048, 16, 2048) == 128
    assert sim.num_selected_pages(1024, 16, 256) == 64
    assert sim.num_selected_pages(20, 16, 100) == 3
    assert sim.num_selected_pages(4096, 16, 10) == 10
    s = np.array([[0.0, 5, 4, 3, -1.0]], np.float32)
    assert list(sim.topk_pages(s, 3, True)[0]) == [0, 1, 4]
    assert list(sim.topk_pages(s, 3, False)[0]) == [1, 2, 3]
    # ties: lowest index first
    s = np.array([[1.0, 2, 2, 2, 0]], np.float32)
    assert list(sim.topk_pages(s, 2, False)[0]) == [1, 2]


def test_full_budget_reduces_to_dense_attention():
    q = randn16(4, (1, 2, 1, 128))
    # L = 112 = 7 full pages.  (For L not a page multiple the reference's
    # k = min(L, budget) // 16 leaves one page out even at a huge budget.)
    K = randn16(5, (1, 2, 112, 128))
    V = randn16(6, (1, 2, 112, 128))
    st = sim.SimLayerState(K[:, :, :111], V[:, :, :111])
    o, _, pages = sim.decode_step(st, q, K[:, :, 111:], V[:, :, 111:], 4096)
    assert pages.shape[-1] == 7
    s = np.einsum("hd,hld->hl", q[0, :, 0].astype(np.float64), K[0].astype(np.float64)) / math.sqrt(128)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    dense = np.einsum("hl,hld->hd", p, V[0].astype(np.float64))
    assert np.abs(o[0, :, 0].astype(np.float64) - dense).max() < 2e-3


def test_causal_prefill_rows_small_bruteforce():
    q = randn16(7, (5, 2, 8))
    k = randn16(8, (9, 2, 8))
    v = randn16(9, (9, 2, 8))
    out = sim.causal_prefill_rows(q, k, v)
    for i in range(5):
        last = 9 - 5 + i
        for hh in range(2):
            s = np.array([q[i, hh].astype(np.float64) @ k[j, hh].astype(np.float64) for j in range(last + 1)])
            s /= math.sqrt(8)
            p = np.exp(s - s.max())
            p /= p.sum()
            ref = sum(p[j] * v[j, hh].astype(np.float64) for j in range(last + 1))
            np.testing.assert_allclose(out[i, hh], ref, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------
# quest_kernel convention: restated from the reference's own test of the
# kernel path (quest/tests/test_approx_attention.py:17-110), which builds the
# expected selection from raw keys with the sign trick, not from the page
# metadata the oracle uses.
# --------------------------------------------------------------------------

def _reference_kernel_convention(q, K, V, page_size, page_budget):
    """test_approx_attention.py:38-110 in numpy: plain-Quest page bound from
    sign(q)*k page maxima (padding with fp16 min), the last page removed,
    top (page_budget - 1), the last page appended; dense when the sequence
    has no more pages than the budget.  q (h, d), K/V (h, L, d) fp16.
    Returns (selected page sets per head or None, o (h, d) float64, the
    page bounds of the first P - 1 pages (h, P - 1) or None)."""
    h, L, d = K.shape
    qf = q.astype(np.float64)
    s = np.einsum("hd,hld->hl", qf, K.astype(np.float64))
    s = s.astype(np.float16).astype(np.float64) / math.sqrt(d)   # fp16 matmul, fp16 / sqrt(d)
    s = s.astype(np.float16).astype(np.float64)
    P = (L + page_size - 1) // page_size
    sets = None
    if P > page_budget:
        sign = np.where(q > 0, 1.0, -1.0)
        mk = K.astype(np.float64) * sign[:, None, :]
        pad = page_size - ((L - 1) % page_size + 1)
        mk = np.concatenate([mk, np.full((h, pad, d), -65504.0)], axis=1)
        pmax = mk.reshape(h, P, page_size, d).max(axis=2)
        approx = np.einsum("hd,hpd->hp", np.abs(qf), pmax)[:, :P - 1]
        sets = []
        mask = np.zeros((h, L), bool)
        for i in range(h):
            top = np.argsort(-approx[i], kind="stable")[:page_budget - 1]
            chosen = set(int(x) for x in top) | {P - 1}
            sets.append(chosen)
            for p in chosen:
                mask[i, p * page_size:min(L, (p + 1) * page_size)] = True
        s = np.where(mask, s, -65504.0)
    e = np.exp(s - s.max(-1, keepdims=True))
    p = (e / e.sum(-1, keepdims=True)).astype(np.float16).astype(np.float64)
    return sets, np.einsum("hl,hld->hd", p, V.astype(np.float64)), approx if sets else None


QK_GRID = [(L, pb) for L in (27, 61, 113, 482, 577, 1011, 1541) for pb in (4, 7, 15, 31, 55, 71)]


@pytest.mark.parametrize("L,pb", QK_GRID)
def test_quest_kernel_convention_matches_reference_test_construction(L, pb):
    H = 4
    q = randn16(100 + L, (1, H, 1, 128))
    K = randn16(200 + L + pb, (1, H, L, 128))
    V = randn16(300 + L + pb, (1, H, L, 128))
    st = sim.SimLayerState(K[:, :, :L - 1], V[:, :, :L - 1])
    o, scores, pages = sim.decode_step(st, q, K[:, :, L - 1:], V[:, :, L - 1:], pb * 16,
                                       fixed=False, value_aware=False, semantics="quest_kernel")
    ref_sets, ref_o, approx = _reference_kernel_convention(q[0, :, 0], K[0], V[0], 16, pb)
    P = (L + 15) // 16
    assert pages.shape[-1] == min(pb, P)
    for i in range(H):
        got = pages[0, i, 0]
        assert got[-1] == P - 1  # the last page is always attended
        if ref_sets is None:
            assert list(got) == list(range(P))
        else:
            # the reference ranks by its own float64 bound: allow near-ties
            ok, why = sim.selection_matches(got, np.array(sorted(ref_sets[i])),
                                            np.append(approx[i], np.inf), forced={P - 1})
            assert ok, (i, why)
    # the reference test's tolerance (assert_close, fp16: rtol = atol = 5e-3)
    np.testing.assert_allclose(o[0, :, 0].astype(np.float64), ref_o, rtol=5e-3, atol=5e-3)


def test_quest_kernel_convention_is_not_the_simulation_rule():
    """The construction above tells the two conventions apart: the
    simulation's rule (k = max(3, budget/16), first and last page forced)
    selects other pages on some grid case."""
    differs = 0
    for L, pb in QK_GRID:
        P = (L + 15) // 16
        if P <= pb:
            continue
        q = randn16(100 + L, (1, 4, 1, 128))
        K = randn16(200 + L + pb, (1, 4, L, 128))
        V = randn16(300 + L + pb, (1, 4, L, 128))
        st = sim.SimLayerState(K, V)
        _, sim_pages = sim.select_pages(st, q, pb * 16, fixed=True, value_aware=False)
        _, qk_pages = sim.select_pages(st, q, pb * 16, value_aware=False,
                                       semantics="quest_kernel")
        differs += int(any(set(sim_pages[0, i, 0]) != set(qk_pages[0, i, 0]) for i in range(4)))
    assert differs > 0


def test_quest_kernel_pages_edge_cases():
    s = np.array([[3.0, 9, 1, 9, 100.0]], np.float32)  # entry P-1 is never ranked
    assert list(sim.quest_kernel_pages(s, 1)[0]) == [4]
    assert list(sim.quest_kernel_pages(s, 0)[0]) == [4]
    assert list(sim.quest_kernel_pages(s, 2)[0]) == [1, 4]       # tie 9/9: lower index
    assert list(sim.quest_kernel_pages(s, 3)[0]) == [1, 3, 4]
    assert list(sim.quest_kernel_pages(s, 99)[0]) == [0, 1, 2, 3, 4]
    assert list(sim.quest_kernel_pages(np.zeros((1, 1), np.float32), 5)[0]) == [0]


# --------------------------------------------------------------------------
# RoPE (apply_rope_in_place): pinned against the library routine the
# reference's test compares with (HF apply_rotary_pos_emb,
# quest/tests/test_rope.py:17-30), against the complex-rotation form, and
# by invariants.
# --------------------------------------------------------------------------

def _rope_angles(positions, D, rope_scale=1.0, rope_theta=1e4):
    """fp32 angles pos * f_i with f_i = (1/scale) * (1/theta)^(2i/D), the
    reciprocals in fp32 as the reference kernel forms them
    (decode_page.cuh:855-856), the power in fp64, rounded to fp32 once.
    (HF's inv_freq = 1 / theta^(2i/D) differs from this in the last fp32
    bits; the GPU test compares with HF's fp16 result at the reference
    test's tolerance.)"""
    i = np.arange(D // 2)
    freq = (np.float64(np.float32(1.0) / np.float32(rope_scale)) *
            np.power(np.float64(np.float32(1.0) / np.float32(rope_theta)), (2 * i) / D)
            ).astype(np.float32)
    return (np.asarray(positions, np.float32)[:, None] * freq[None, :]).astype(np.float64)


@pytest.mark.parametrize("past,n,scale,theta", [(0, 5, 1.0, 1e4), (1110, 7, 1.0, 1e4),
                                                (311, 19, 2.0, 5e5)])
def test_rope_matches_hf_apply_rotary_pos_emb(past, n, scale, theta):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    q = randn16(70 + n, (n, 4, 128))
    k = randn16(71 + n, (n, 2, 128))
    pos = past + np.arange(n)
    ang = _rope_angles(pos, 128, scale, theta)
    emb = np.concatenate([ang, ang], axis=-1)                      # HF: cat(freqs, freqs)
    cos = torch.from_numpy(np.cos(emb))[None]
    sin = torch.from_numpy(np.sin(emb))[None]
    qt = torch.from_numpy(q.astype(np.float64)).transpose(0, 1)[None]   # [1, H, N, D]
    kt = torch.from_numpy(k.astype(np.float64)).transpose(0, 1)[None]
    qr, kr = apply_rotary_pos_emb(qt, kt, cos, sin)
    np.testing.assert_allclose(sim.apply_rope(q, pos, scale, theta),
                               qr[0].transpose(0, 1).numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(sim.apply_rope(k, pos, scale, theta),
                               kr[0].transpose(0, 1).numpy(), rtol=0, atol=1e-12)


def test_rope_is_the_complex_rotation_of_dim_pairs():
    x = randn16(80, (6, 3, 128))
    pos = np.array([0, 1, 17, 250, 4096, 65535])
    ang = _rope_angles(pos, 128)
    z = (x[..., :64].astype(np.float64) + 1j * x[..., 64:].astype(np.float64)) * \
        np.exp(1j * ang)[:, None, :]
    out = sim.apply_rope(x, pos)
    np.testing.assert_allclose(out[..., :64], z.real, atol=1e-12)
    np.testing.assert_allclose(out[..., 64:], z.imag, atol=1e-12)
    # position 0 is the identity; each (i, i + 64) pair keeps its length
    np.testing.assert_array_equal(out[0], x[0].astype(np.float64))
    r_in = np.hypot(x[..., :64].astype(np.float64), x[..., 64:].astype(np.float64))
    np.testing.assert_allclose(np.hypot(out[..., :64], out[..., 64:]), r_in, rtol=1e-12)


def test_rope_scores_depend_on_relative_position_only():
    q = randn16(90, (1, 1, 128))
    k = randn16(91, (1, 1, 128))
    def score(m, n):
        return float(np.sum(sim.apply_rope(q, [m])[0, 0] * sim.apply_rope(k, [n])[0, 0]))
    for m, n, t in ((10, 3, 5), (40, 40, 7), (100, 1, 64)):
        assert abs(score(m, n) - score(m + t, n + t)) < 1e-3


def test_rope_planted_mistakes_fail_the_hf_check():
    """A wrong partner sign, an unwrapped frequency index, theta instead of
    1/theta: each moves the result far beyond fp16 noise."""
    x = randn16(95, (3, 2, 128))
    pos = np.array([5, 77, 300])
    good = sim.apply_rope(x, pos)
    xf = x.astype(np.float64)
    ang = _rope_angles(pos, 128)[:, None, :]
    c, s = np.cos(ang), np.sin(ang)
    wrong_sign = np.concatenate([xf[..., :64] * c + xf[..., 64:] * s,
                                 xf[..., 64:] * c - xf[..., :64] * s], -1)
    i = np.arange(128)
    f_unwrapped = np.power(np.float32(1e-4), (2 * i).astype(np.float32) / np.float32(128))
    a2 = (pos[:, None].astype(np.float32) * f_unwrapped[None]).astype(np.float64)[:, None, :]
    rot = np.concatenate([-xf[..., 64:], xf[..., :64]], -1)
    unwrapped = xf * np.cos(a2) + rot * np.sin(a2)
    for bad in (wrong_sign, unwrapped, sim.apply_rope(x, pos, 1.0, 1e-4)):
        assert np.abs(bad - good).max() > 0.05


def _fma32(a, b, c):
    """fp32 fused multiply-add: a*b is exact in float64 for fp32 a, b, and
    for the operands below the float64 sum rounds as the fused result does."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def test_logit_division_by_sqrt_head_dim_is_exact_for_every_fp16():
    """The decode kernel divides each fp16 logit by sqrt(128) with a
    reciprocal product and one Newton step (device.hpp,
    div_sqrt_head_dim_f16).  Over every finite fp16 value that equals the
    IEEE fp32 quotient, and so fp16(fp16(q.k)/sqrt(d)) of the simulation
    (quest_attention.py:265-268), once the sign of a zero is restored."""
    x = np.arange(65536, dtype=np.uint16).view(np.float16)
    x = x[np.isfinite(x)].astype(np.float32)
    c = np.float32(math.sqrt(128.0))
    assert c == np.float32(11.313708498984761)
    r = np.float32(1.0) / c
    q0 = (x * r).astype(np.float32)
    q1 = _fma32(_fma32(-q0, np.full_like(x, c), x), np.full_like(x, r), q0)
    q1 = np.copysign(q1, x)
    ref = (x / c).astype(np.float32)
    assert np.array_equal(q1.view(np.uint32), ref.view(np.uint32))
    # a plain reciprocal product is not enough (the step matters)
    assert not np.array_equal(q0.astype(np.float16).view(np.uint16), ref.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("L,k,seed", [(100, 3, 0), (4096 + 9, 64, 1), (777, 49, 2)])
def test_sparse_decode_attention_equals_masked_form(L, k, seed):
    """sim.sparse_decode_attention (selected tokens only) against the
    simulation's masked form over every token (quest_attention.py:347-356):
    the same fp16 result up to one ulp of the final product's summation
    order, on random selections including the partial last page."""
    H, D = 4, 128
    g = np.random.default_rng(seed)
    q = (g.standard_normal((1, H, 1, D)).astype(np.float32)).astype(np.float16)
    K = (g.standard_normal((1, H, L, D)).astype(np.float32)).astype(np.float16)
    V = (g.standard_normal((1, H, L, D)).astype(np.float32)).astype(np.float16)
    P = sim.num_pages(L) if hasattr(sim, "num_pages") else -(-L // 16)
    pages = np.stack([np.sort(g.choice(P, size=k, replace=False)) for _ in range(H)])
    pages[:, -1] = P - 1  # the partial last page takes part
    pages = pages[None, :, None, :]
    ref = sim.masked_decode_attention(q, K, V, sim.pages_to_token_mask(pages, 16, L))
    got = sim.sparse_decode_attention(q, K, V, pages, 16, L)
    diff = np.abs(ref.astype(np.float32) - got.astype(np.float32))
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
    assert np.all(diff <= ulp), float(diff.max())
    # a planted mistake: dropping the last selected page must show
    bad = sim.sparse_decode_attention(q, K, V, pages[..., :-1], 16, L)
    assert np.abs(bad.astype(np.float32) - ref.astype(np.float32)).max() > 1e-3
