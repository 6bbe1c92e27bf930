"""End-to-end checks of the Llama shim (aoakv.shim, the QuestAttention /
LlamaModel integration of quest/models/QuestAttention.py:56-181 and
llama.py:424-486) on the GPU, small random models.

* With a budget that covers the sequence every layer attends densely: the
  hidden states after prefill and after each decode step match a plain torch
  fp32 Llama forward (RoPE, causal attention, RMSNorm, SiLU MLP) of the same
  weights within fp16 noise.
* With a sparse budget, the one-launch decode layer and the reference's three
  calls give identical hidden states at every step, and the selection changes
  the result (the sparse layers are really sparse).
"""
import math
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _aoakv():
    import aoakv  # noqa: F401  (fails loudly if libaoakv.so is missing)
    assert torch.cuda.is_available()
    yield


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _make(cfg, single_launch=True, budget=4096, semantics="sim", value_aware=True, max_len=512):
    from aoakv.shim import QuestLlamaModel
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(DEV):
            m = QuestLlamaModel(cfg, single_launch=single_launch).random_init(3, std=0.05)
    finally:
        torch.set_default_dtype(torch.float32)
    m.quest_init(page_size=16, max_seq_len=max_len, token_budget=budget, device=DEV,
                 value_aware=value_aware, semantics=semantics)
    return m


def _rope_t(x, pos, scale, theta):
    """fp32 torch RoPE, rotate-half form; x [N, H, D]."""
    D = x.shape[-1]
    i = torch.arange(D // 2, device=x.device, dtype=torch.float64)
    f = ((1.0 / scale) * (1.0 / theta) ** (2 * i / D)).float()
    a = pos.float()[:, None] * f[None]
    c = torch.cat([a.cos(), a.cos()], -1)[:, None]
    s = torch.cat([a.sin(), a.sin()], -1)[:, None]
    rot = torch.cat([-x[..., D // 2:], x[..., :D // 2]], -1)
    return x * c + rot * s


class _RefLlama:
    """Plain fp32 forward of the shim's weights with a growing KV list."""

    def __init__(self, m):
        self.m, self.cfg = m, m.cfg
        self.K = [None] * len(m.layers)
        self.V = [None] * len(m.layers)
        self.L = 0

    def _norm(self, n, x):
        return n.weight.float() * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + n.eps))

    def forward(self, x):
        cfg = self.cfg
        Hq, Hkv = cfg.num_attention_heads, cfg.num_key_value_heads
        D = cfg.hidden_size // Hq
        n = x.shape[1]
        pos = torch.arange(self.L, self.L + n, device=x.device)
        h = x[0].float()
        for li, layer in enumerate(self.m.layers):
            a = layer.self_attn
            t = self._norm(layer.input_layernorm, h)
            q = (t @ a.q_proj.weight.float().T).view(n, Hq, D)
            k = (t @ a.k_proj.weight.float().T).view(n, Hkv, D)
            v = (t @ a.v_proj.weight.float().T).view(n, Hkv, D)
            q = _rope_t(q, pos, cfg.rope_scale, cfg.rope_theta)
            k = _rope_t(k, pos, cfg.rope_scale, cfg.rope_theta)
            self.K[li] = k if self.K[li] is None else torch.cat([self.K[li], k])
            self.V[li] = v if self.V[li] is None else torch.cat([self.V[li], v])
            Kf = self.K[li].repeat_interleave(Hq // Hkv, dim=1)
            Vf = self.V[li].repeat_interleave(Hq // Hkv, dim=1)
            s = torch.einsum("nhd,lhd->hnl", q, Kf) / math.sqrt(D)
            Ltot = Kf.shape[0]
            mask = torch.arange(Ltot, device=x.device)[None] <= (pos[:, None])
            s = s.masked_fill(~mask[None], float("-inf"))
            o = torch.einsum("hnl,lhd->nhd", s.softmax(-1), Vf).reshape(n, Hq * D)
            h = h + o @ a.o_proj.weight.float().T
            t = self._norm(layer.post_attention_layernorm, h)
            mlp = layer.mlp
            g = torch.nn.functional.silu(t @ mlp.gate_proj.weight.float().T)
            h = h + (g * (t @ mlp.up_proj.weight.float().T)) @ mlp.down_proj.weight.float().T
        self.L += n
        return self._norm(self.m.norm, h)


def _cfg(hidden, heads, kv_heads, layers=3, scale=1.0):
    from aoakv.shim import LlamaShape
    return LlamaShape(hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=kv_heads,
                      num_hidden_layers=layers, intermediate_size=2 * hidden, rope_scale=scale)


@pytest.mark.parametrize("heads,kv_heads,scale", [(2, 2, 1.0), (4, 2, 8.0)])
def test_dense_budget_matches_fp32_llama(heads, kv_heads, scale):
    _say(f"[shim-dense] heads={heads} kv={kv_heads} scale={scale}")
    cfg = _cfg(128 * heads, heads, kv_heads, scale=scale)
    m = _make(cfg, budget=1 << 16)
    ref = _RefLlama(m)
    g = torch.Generator(device=DEV).manual_seed(5)
    for step, n in enumerate([200] + [1] * 30):
        x = torch.randn(1, n, cfg.hidden_size, generator=g, device=DEV).half()
        with torch.inference_mode():
            out = m(x)[0].float()
            want = ref.forward(x.float())
        rel = ((out - want).norm() / want.norm()).item()
        assert rel < 5e-3, (step, rel)


def test_sparse_one_launch_equals_three_calls():
    cfg = _cfg(256, 2, 2, layers=4)
    ms = [_make(cfg, single_launch=s, budget=64) for s in (True, False)]
    dense = _make(cfg, budget=1 << 16)
    g = torch.Generator(device=DEV).manual_seed(6)
    differs = 0
    for step, n in enumerate([400] + [1] * 40):
        x = torch.randn(1, n, cfg.hidden_size, generator=g, device=DEV).half()
        with torch.inference_mode():
            a, b, d = (mm(x) for mm in (*ms, dense))
        assert torch.equal(a, b), step
        assert torch.isfinite(a).all()
        if n == 1:
            differs += int(not torch.equal(a, d))
    assert differs > 0, "the sparse layers never changed the output"
    err = [int(mm.iController.workspace[8:12].view(torch.int32).item()) for mm in ms]
    assert err == [0, 0]


def test_quest_kernel_semantics_and_plain_quest_run():
    cfg = _cfg(256, 2, 2, layers=3)
    g = torch.Generator(device=DEV).manual_seed(7)
    xs = [torch.randn(1, n, cfg.hidden_size, generator=g, device=DEV).half()
          for n in [300] + [1] * 10]
    outs = []
    for sem, va in (("sim", True), ("quest_kernel", True), ("sim", False)):
        m = _make(cfg, budget=64, semantics=sem, value_aware=va)
        with torch.inference_mode():
            o = [m(x) for x in xs]
        assert all(torch.isfinite(t).all() for t in o)
        outs.append(torch.cat([t[:, -1] for t in o[1:]]))
    # different selection rules attend different pages
    assert not torch.equal(outs[0], outs[1]) and not torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("heads,kv_heads,single_launch", [(2, 2, True), (4, 2, True), (2, 2, False)])
def test_graphed_decode_equals_forward(heads, kv_heads, single_launch):
    """decode_graphed (the layers replayed from a HIP graph, the grids sized
    for the cache's capacity, captured again when the sparse layers start
    selecting) gives the bits of the eager forward at every step: a prefill
    below the budget, then decode steps that cross five page boundaries and
    the budget, then a second conversation after quest_clear.  Every replay
    is checked, with the planner's eager work and the other model's launches
    between replays."""
    _say(f"[shim-graph] heads={heads} kv={kv_heads} single_launch={single_launch}")
    cfg = _cfg(128 * heads, heads, kv_heads, layers=4)
    eager, graphed = (_make(cfg, single_launch=single_launch, budget=64) for _ in range(2))
    g = torch.Generator(device=DEV).manual_seed(8)
    for conv, (n0, steps) in enumerate([(40, 70), (150, 20)]):
        for step, n in enumerate([n0] + [1] * steps):
            x = torch.randn(1, n, cfg.hidden_size, generator=g, device=DEV).half()
            with torch.inference_mode():
                want = eager(x)
                got = graphed(x) if n > 1 else graphed.decode_graphed(x)
            assert torch.equal(got, want), (conv, step)
        for mm in (eager, graphed):
            assert int(mm.iController.workspace[8:12].view(torch.int32).item()) == 0
            mm.quest_clear()
