"""GPU parity of the MFMA causal paged prefill (aoakv_prefill_with_paged_kv_cache)
against the oracle's fp64 textbook causal attention (oracle.sim.causal_prefill_rows,
after quest/tests/test_prefill_attention.py:17-44 and cpu_reference.h:56-159).

Bar: max |o - ref| <= 2e-3 (fp16 output, fp32 accumulation).  Inputs
q, K, V ~ N(0, 0.5^2) as in BASELINE config 4.  At config 4's sizes (8k and
16k tokens, 32 heads) every row is held to a plain PyTorch fp32 causal
attention on the GPU, which is itself held to the fp64 oracle on sampled rows.
"""
import sys

import numpy as np
import pytest
import torch

from helpers import HND, NHD, randn16
from oracle import sim

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
D, S = 128, 16


@pytest.fixture(scope="module", autouse=True)
def _aoakv():
    import aoakv  # noqa: F401
    yield


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _run(L, Lq, H, layout, seed, causal=True, shuffle=None, via_utils=False):
    from aoakv import ops
    from aoakv.utils import InferenceController, append_kv, prefill_forward
    q = randn16(seed, (Lq, H, D), 0.5)
    k = randn16(seed + 1, (L, H, D), 0.5)
    v = randn16(seed + 2, (L, H, D), 0.5)
    c = InferenceController(1, H, D, S, 64, L + S, torch.float16, DEV, layout=layout,
                            shuffle_seed=shuffle)
    c.prepare_metadata(L)
    c.begin_forward(L)
    append_kv(torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV), c, 0)
    qd = torch.from_numpy(q).to(DEV)
    if via_utils:
        assert Lq == L and causal
        o = prefill_forward(qd, c, 0)
    else:
        o = ops.prefill_with_paged_kv_cache(qd, c.kv_cache.buf_layer(0), c.kv_indices_with_last,
                                            len(c.kv_cache.indicies), c.kv_cache.last_page_len,
                                            layout, causal=causal)
    torch.cuda.synchronize()
    return q, k, v, o.cpu().numpy()


def _ref_rows(q, k, v, rows, causal):
    if causal:
        return sim.causal_prefill_rows(q, k, v, rows)
    res = []  # non-causal: every query sees every key
    for r in rows:
        s = np.einsum("hd,lhd->hl", q[r].astype(np.float64), k.astype(np.float64)) / np.sqrt(D)
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        res.append(np.einsum("hl,lhd->hd", p, v.astype(np.float64)))
    return np.stack(res).astype(np.float32)


@pytest.mark.parametrize("layout", [NHD, HND])
@pytest.mark.parametrize("L,Lq", [(1, 1), (15, 15), (16, 16), (17, 17), (100, 100), (300, 300),
                                  (300, 40), (777, 129), (1000, 1000)])
def test_prefill_matches_causal_attention(layout, L, Lq):
    _say(f"[prefill] layout={layout} L={L} Lq={Lq}")
    H = 4
    q, k, v, o = _run(L, Lq, H, layout, seed=L + Lq, shuffle=L)
    ref = _ref_rows(q, k, v, np.arange(Lq), True)
    err = np.abs(o.astype(np.float32) - ref).max()
    assert err <= 2e-3, err


def test_prefill_non_causal():
    _say("[prefill] non-causal")
    q, k, v, o = _run(200, 64, 2, HND, seed=5, causal=False)
    ref = _ref_rows(q, k, v, np.arange(64), False)
    assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3


def test_prefill_forward_via_controller():
    _say("[prefill] utils.prefill_forward")
    q, k, v, o = _run(333, 333, 8, HND, seed=9, shuffle=2, via_utils=True)
    ref = _ref_rows(q, k, v, np.arange(333), True)
    assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3


def _torch_causal_fp32(q, k, v, chunk=512):
    """Plain PyTorch fp32 causal attention on the GPU, in query chunks:
    (L, H, D) fp16 arrays in, (L, H, D) float32 out."""
    torch.backends.cuda.matmul.allow_tf32 = False
    qf = torch.from_numpy(q).to(DEV).float().transpose(0, 1).contiguous()   # H, L, D
    kt = torch.from_numpy(k).to(DEV).float().permute(1, 2, 0).contiguous()  # H, D, L
    vf = torch.from_numpy(v).to(DEV).float().transpose(0, 1).contiguous()   # H, L, D
    L = qf.shape[1]
    out = torch.empty_like(qf)
    for r0 in range(0, L, chunk):
        r1 = min(L, r0 + chunk)
        s = torch.matmul(qf[:, r0:r1], kt[:, :, :r1].contiguous()) / np.sqrt(D)
        dead = torch.arange(r1, device=DEV)[None, :] > torch.arange(r0, r1, device=DEV)[:, None]
        s.masked_fill_(dead, float("-inf"))
        out[:, r0:r1] = torch.matmul(torch.softmax(s, -1), vf[:, :r1].contiguous())
    return out.transpose(0, 1).cpu().numpy()


@pytest.mark.parametrize("layout,L", [(NHD, 8192), (HND, 8192), (HND, 16384)])
def test_prefill_config4_every_row(layout, L):
    """BASELINE config 4 shapes (32 heads, 8192 and 16384 tokens), every
    query row of every head against a plain PyTorch fp32 causal attention;
    that reference is itself held to the fp64 oracle on rows sampled across
    the causal range, including tile and page boundaries."""
    _say(f"[prefill] config-4 L={L} layout={layout}")
    q, k, v, o = _run(L, L, 32, layout, seed=0, shuffle=4)
    rows = np.array([0, 1, 15, 16, 63, 64, 127, 128, 129, 1000, 4095, 4096, 6000,
                     L - 66, L - 2, L - 1])
    ref_rows = _ref_rows(q, k, v, rows, True)
    err = np.abs(o[rows].astype(np.float32) - ref_rows).max()
    _say(f"   sampled rows vs fp64 oracle: max err {err:.2e}")
    assert err <= 2e-3
    ref = _torch_causal_fp32(q, k, v)
    assert np.abs(ref[rows] - ref_rows).max() <= 1e-5  # the fp32 reference holds to fp64
    err_all = np.abs(o.astype(np.float32) - ref).max(axis=(1, 2))
    _say(f"   every row vs torch fp32: max err {err_all.max():.2e} (row {int(err_all.argmax())})")
    assert err_all.max() <= 2e-3
    assert np.isfinite(o.astype(np.float32)).all()


@pytest.mark.parametrize("layout", [NHD, HND])
@pytest.mark.parametrize("group", [2, 4])
def test_prefill_gqa(layout, group):
    """num_qo_heads = group * num_kv_heads: query head h attends kv head
    h // group (the reference's prefill kernel takes both head counts,
    prefill.cuh:688-870)."""
    from aoakv import ops
    from aoakv.utils import InferenceController, append_kv
    _say(f"[prefill] gqa group={group} layout={layout}")
    L, Lq, Hkv = 500, 300, 2
    Hq = Hkv * group
    q = randn16(40 + group, (Lq, Hq, D), 0.5)
    k = randn16(41 + group, (L, Hkv, D), 0.5)
    v = randn16(42 + group, (L, Hkv, D), 0.5)
    c = InferenceController(1, Hq, D, S, 64, L + S, torch.float16, DEV, layout=layout,
                            num_kv_heads=Hkv, shuffle_seed=3)
    c.prepare_metadata(L)
    c.begin_forward(L)
    append_kv(torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV), c, 0)
    o = ops.prefill_with_paged_kv_cache(torch.from_numpy(q).to(DEV), c.kv_cache.buf_layer(0),
                                        c.kv_indices_with_last, len(c.kv_cache.indicies),
                                        c.kv_cache.last_page_len, layout).cpu().numpy()
    ref = sim.causal_prefill_rows(q, np.repeat(k, group, axis=1), np.repeat(v, group, axis=1))
    assert np.abs(o.astype(np.float32) - ref).max() <= 2e-3


@pytest.mark.parametrize("L", [100, 777, 4096 + 9])
def test_prefill_ignores_unwritten_slots_past_the_sequence(L):
    """Regression: the cache's slots past the last token are never written
    and may hold NaN.  Their probability is 0, but 0 * NaN is NaN in the
    MFMA: the tile holding the sequence's end must not let them in.  The
    cache is filled with NaN before the append, so every unwritten slot is
    NaN here."""
    from aoakv import ops
    from aoakv.utils import InferenceController, append_kv
    _say(f"[prefill NaN slots] L={L}")
    H = 8
    q = randn16(90 + L, (L, H, D), 0.5)
    k = randn16(91 + L, (L, H, D), 0.5)
    v = randn16(92 + L, (L, H, D), 0.5)
    c = InferenceController(1, H, D, S, 64, L + 2 * S, torch.float16, DEV, layout=HND,
                            shuffle_seed=3)
    c.kv_cache.buf_layer(0).fill_(float("nan"))
    c.prepare_metadata(L)
    c.begin_forward(L)
    append_kv(torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV), c, 0)
    o = ops.prefill_with_paged_kv_cache(torch.from_numpy(q).to(DEV), c.kv_cache.buf_layer(0),
                                        c.kv_indices_with_last, len(c.kv_cache.indicies),
                                        c.kv_cache.last_page_len, HND).cpu().numpy()
    assert np.isfinite(o.astype(np.float32)).all()
    rows = np.unique(np.linspace(0, L - 1, 24).astype(np.int64))
    ref = sim.causal_prefill_rows(q, k, v, rows)
    assert np.abs(o[rows].astype(np.float32) - ref).max() <= 2e-3
