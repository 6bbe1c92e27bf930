"""GPU parity of RoPE (aoakv_apply_rope_in_place) and of the fused decode
step RoPE + append (aoakv_rope_append_kv_cache_decode), through the C ABI.

Grid: the reference's own test, quest/tests/test_rope.py:32-50 (32 heads x
128, fp16, past_kv_len x seq_len).  Bars: within one fp16 ulp (plus fp32
evaluation noise of the two rotated terms, 2^-21 of their magnitudes) of the
oracle's exactly rounded value (sim.apply_rope); within the reference
test's tolerance (rtol = atol = 5e-3) of the HF fp16 computation it
compares with; the fused decode step bit-identical to RoPE followed by the
plain decode append, and its metadata bit-exact against the simulation fed
the rotated keys.
"""
import sys

import numpy as np
import pytest
import torch

from helpers import HND, NHD, bits, num_pages, randn16, read_filters, read_kv
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


def _ulp16(x):
    """fp16 spacing at |x| (subnormal spacing near zero)."""
    a = np.abs(x).astype(np.float16)
    return np.maximum(np.spacing(a).astype(np.float64), 2.0 ** -24)


def _rope_err(got, x, ref):
    """|got - ref| in units of the bound one fp16 rounding plus fp32
    evaluation allows: an fp16 ulp of the result plus 2^-21 of the two terms'
    magnitudes (x_d cos a and x_partner sin a can cancel to a result far below
    them, where fp32 noise is no longer small against the fp16 spacing)."""
    xf = np.abs(x.astype(np.float64))
    half = x.shape[-1] // 2
    terms = xf + np.concatenate([xf[..., half:], xf[..., :half]], -1)
    return np.abs(got.astype(np.float64) - ref) / (_ulp16(ref) + 2.0 ** -21 * terms)


def _hf_fp16(x, pos, scale=1.0, theta=1e4):
    """HF LlamaRotaryEmbedding + apply_rotary_pos_emb on fp16 tensors, as the
    reference test computes its expectation: cos / sin rounded to fp16, then
    fp16 elementwise ops."""
    N, H, Dd = x.shape
    i = np.arange(Dd // 2)
    inv = (np.float32(1.0 / scale) / np.power(np.float32(theta),
                                               (2 * i).astype(np.float32) / np.float32(Dd),
                                               dtype=np.float32)).astype(np.float32)
    ang = (np.asarray(pos, np.float32)[:, None] * inv[None]).astype(np.float32)
    emb = np.concatenate([ang, ang], -1)
    c = np.cos(emb).astype(np.float16)[:, None, :]
    s = np.sin(emb).astype(np.float16)[:, None, :]
    rot = np.concatenate([-x[..., Dd // 2:], x[..., :Dd // 2]], -1)
    return ((x * c).astype(np.float16) + (rot * s).astype(np.float16)).astype(np.float16)


GRID = [(p, n) for p in (13, 24, 51, 77, 244, 311, 502, 1110)
        for n in (2, 5, 7, 19, 31, 69, 111, 251)]


@pytest.mark.parametrize("past,n", GRID)
def test_rope_matches_oracle_and_reference_tolerance(past, n):
    from aoakv import ops
    Hq, Hkv = (32, 8) if (past + n) % 3 == 0 else (32, 32)
    q = randn16(1000 + past + n, (n, Hq, D))
    k = randn16(2000 + past + n, (n, Hkv, D))
    qd = torch.from_numpy(q).to(DEV)
    kd = torch.from_numpy(k).to(DEV)
    ops.apply_rope_in_place(qd, kd, past)
    qg, kg = qd.cpu().numpy(), kd.cpu().numpy()
    pos = past + np.arange(n)
    for got, x in ((qg, q), (kg, k)):
        ref = sim.apply_rope(x, pos)
        err = _rope_err(got, x, ref)
        assert err.max() <= 1.0, f"max error {err.max():.2f} of the bound"
        hf = _hf_fp16(x, pos).astype(np.float64)
        assert np.all(np.abs(got.astype(np.float64) - hf) <= 5e-3 + 5e-3 * np.abs(hf))


@pytest.mark.parametrize("scale,theta,past", [(2.0, 5e5, 0), (1.0, 1e6, 40000), (0.5, 1e4, 7)])
def test_rope_scale_theta_and_long_positions(scale, theta, past):
    from aoakv import ops
    n = 33
    q = randn16(3000 + past, (n, 16, D))
    k = randn16(3001 + past, (n, 16, D))
    qd, kd = torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV)
    ops.apply_rope_in_place(qd, kd, past, scale, theta)
    pos = past + np.arange(n)
    for got, x in ((qd.cpu().numpy(), q), (kd.cpu().numpy(), k)):
        ref = sim.apply_rope(x, pos, scale, theta)
        assert _rope_err(got, x, ref).max() <= 1.0


@pytest.mark.parametrize("layout", [NHD, HND])
@pytest.mark.parametrize("L0", [100, 16 * 20])
def test_fused_rope_append_equals_rope_then_append(layout, L0):
    """Decode steps through aoakv_rope_append_kv_cache_decode vs
    aoakv_apply_rope_in_place + aoakv_append_kv_cache_decode on a twin cache:
    q, k, cache, Kmax/Kmin, V mean and log-norm bit-identical after every
    step (crossing a page boundary); metadata equal to the simulation's for
    the rotated keys."""
    from aoakv.utils import InferenceController, append_kv, apply_rope_in_place, rope_append_kv
    _say(f"[rope-append] layout={layout} L0={L0}")
    H, Hq, steps = 8, 16, 20
    K0 = randn16(50, (1, H, L0, D))
    V0 = randn16(51, (1, H, L0, D))
    ctrls = [InferenceController(1, Hq, D, S, 8, L0 + steps + S, torch.float16, DEV,
                                 layout=layout, num_kv_heads=H, shuffle_seed=9) for _ in range(2)]
    for c in ctrls:
        c.prepare_metadata(L0)
        c.begin_forward(L0)
        append_kv(torch.from_numpy(np.ascontiguousarray(K0[0].transpose(1, 0, 2))).to(DEV),
                  torch.from_numpy(np.ascontiguousarray(V0[0].transpose(1, 0, 2))).to(DEV), c, 0)
        c.end_forward()
    st = sim.SimLayerState(K0, V0)
    for t in range(steps):
        qn = randn16(60 + t, (1, Hq, D))
        kn = randn16(70 + t, (1, H, D))
        vn = randn16(80 + t, (1, H, D))
        pos = L0 + t
        outs = []
        for i, c in enumerate(ctrls):
            c.prepare_metadata(1)
            c.begin_forward(1)
            qd, kd, vd = (torch.from_numpy(x.copy()).to(DEV) for x in (qn, kn, vn))
            if i == 0:
                rope_append_kv(qd, kd, vd, c, 0)
            else:
                apply_rope_in_place(qd, kd, c.kv_cache.seqlen - 1)
                append_kv(kd, vd, c, 0)
            outs.append((qd.cpu().numpy(), kd.cpu().numpy()))
        assert np.array_equal(bits(outs[0][0]), bits(outs[1][0])), t
        assert np.array_equal(bits(outs[0][1]), bits(outs[1][1])), t
        ref_k = sim.apply_rope(kn, [pos])
        assert _rope_err(outs[0][1], kn, ref_k).max() <= 1.0
        st.append(outs[0][1][0][None, :, None, :], vn[0][None, :, None, :])
    torch.cuda.synchronize()
    L = L0 + steps
    # the written part of each cache (same page tables: same shuffle seed)
    state = []
    for c in ctrls:
        pages = c.kv_cache.indicies
        Kc, Vc = read_kv(c.kv_cache.buf_layer(0), layout, pages, L)
        pf = read_filters(c.metadata_cache.buf_layer(0), layout, c.metadata_cache.indicies,
                          num_pages(L))
        vm = c.v_mean_layer(0).cpu().numpy()[pages][None].transpose(0, 2, 1, 3)
        lvn = c.v_log_norm_layer(0).cpu().numpy()[pages]
        state.append((Kc, Vc, pf, vm, lvn))
    for name, x, y in zip(("K", "V", "Kmax/Kmin", "V mean", "log-norm"), *state):
        assert np.array_equal(bits(x), bits(y)), name
    Kc, Vc, pf, vm, lvn = state[0]
    assert np.array_equal(bits(Kc), bits(st.K)) and np.array_equal(bits(Vc), bits(st.V))
    assert np.array_equal(bits(pf), bits(st.page_filters))
    assert np.array_equal(bits(vm), bits(st.v_mean))
    assert np.array_equal(bits(lvn.T[None]), bits(sim.log_v_norm(st.v_mean)))
