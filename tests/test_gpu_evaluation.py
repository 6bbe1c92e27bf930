"""GPU parity of the evaluation-side stand-in (aoakv.evaluation) against the
oracle: an HF LlamaAttention patched by ``enable_quest_attention_eval``, driven
the way the reference's tuple-cache decoder layer calls it
(evaluation/llama.py:507-536): a prefill, a block of question tokens, then
single-token decode steps, the cache going back in as ``past_key_value``.

Per call the output (``o_proj`` replaced by the identity) is held to the
oracle's restatement of the reference forward (quest_attention.py:196-382):
the prefill to fp64 causal attention; every decode token -- each token of
the question block as well as the single-token steps -- to ``sim.decode_step``
(append, scores, group-consistent top-k, masked attention) with the
selection compared tie-aware and the output within 2e-3 of the oracle's
attention over the stand-in's own pages.  Layers 0-1 attend every page.  A
short context (fewer tokens than the budget, a partial last page) checks
that quest layers select on every step, as the reference does (k = P - 1
there: the lowest page is dropped).  The question tokens are decoded one at a
time here (the reference's block form is documented in aoakv/evaluation.py).
"""
import sys
import types

import numpy as np
import pytest
import torch
from torch import nn

from oracle import sim

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
S = 16


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _setup(hq, hkv, layer_id, value_aware, budget, seed):
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaAttention, LlamaRotaryEmbedding
    from aoakv import evaluation as ev
    d = 128
    cfg = LlamaConfig(hidden_size=hq * d, num_attention_heads=hq, num_key_value_heads=hkv,
                      num_hidden_layers=layer_id + 1, intermediate_size=256,
                      max_position_embeddings=8192)
    torch.manual_seed(seed)
    model = nn.Module()
    model.config = cfg
    model.layers = nn.ModuleList(nn.ModuleDict({"self_attn": LlamaAttention(cfg, layer_idx=i)})
                                 for i in range(layer_id + 1))
    attn = model.layers[layer_id]["self_attn"]
    for lin in (attn.q_proj, attn.k_proj, attn.v_proj):
        nn.init.normal_(lin.weight, std=1.0 / np.sqrt(cfg.hidden_size))
    attn.o_proj = nn.Identity()
    attn.rotary_emb = LlamaRotaryEmbedding(cfg)  # the 4.45 module attribute
    model.to(DEV, torch.float16)
    args = types.SimpleNamespace(quest=True, value_aware=value_aware, token_budget=budget,
                                 chunk_size=S, fixed=True, max_gen=64)
    ev.enable_quest_attention_eval(model, args, classes=(LlamaAttention,))
    assert attn.layer_id == layer_id
    return attn


def _qkv(attn, x, pos):
    """q, k (rotated) and v of hidden states x (1, n, hidden) as (n, H, D) fp16 numpy."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    hq, hkv = attn.config.num_attention_heads, attn.config.num_key_value_heads
    n = x.shape[1]
    q = attn.q_proj(x).view(1, n, hq, 128).transpose(1, 2)
    k = attn.k_proj(x).view(1, n, hkv, 128).transpose(1, 2)
    v = attn.v_proj(x).view(1, n, hkv, 128).transpose(1, 2)
    cos, sin = attn.rotary_emb(v, pos)
    q, k = apply_rotary_pos_emb(q, k, cos, sin)
    f = lambda t: t[0].transpose(0, 1).to(torch.float16).cpu().numpy()
    return f(q), f(k), f(v)


@pytest.mark.parametrize("hq,hkv,layer_id,value_aware,L0", [
    (4, 4, 3, True, 1500), (8, 2, 3, True, 1500), (4, 4, 3, False, 1500), (4, 4, 1, True, 1500),
    (4, 4, 3, True, 203), (8, 2, 3, False, 203)])
def test_stand_in_matches_oracle(hq, hkv, layer_id, value_aware, L0):
    _say(f"[eval] hq={hq} hkv={hkv} layer={layer_id} value_aware={value_aware} L0={L0}")
    from aoakv import evaluation as ev
    group = hq // hkv
    budget, n_question, n_decode = 256, 5, 12
    attn = _setup(hq, hkv, layer_id, value_aware, budget, seed=hq + layer_id)
    g = torch.Generator(device=DEV).manual_seed(3)
    hid = attn.config.hidden_size
    xs = torch.randn((1, L0 + n_question + n_decode, hid), generator=g, device=DEV).half()
    with torch.no_grad():
        # prefill
        pos = torch.arange(L0, device=DEV)[None]
        out, w, past = attn(hidden_states=xs[:, :L0], attention_mask=None, position_ids=pos,
                            past_key_value=None, output_attentions=False, use_cache=True,
                            padding_mask=None)
        assert w is None and len(past) == 3 and past[-1] == L0
        assert isinstance(past[0], ev.LayerCache)
        past[0].keep_selections = True
        q, k, v = _qkv(attn, xs[:, :L0], pos)
        ref = sim.causal_prefill_rows(q, np.repeat(k, group, 1), np.repeat(v, group, 1))
        o = out[0].view(L0, hq, 128).float().cpu().numpy()
        assert np.abs(o - ref).max() <= 2e-3
        state = sim.SimLayerState(k.transpose(1, 0, 2)[None], v.transpose(1, 0, 2)[None], S)
        # question block (several tokens), then decode steps
        t = L0
        dropped = 0  # quest-layer steps that attended fewer pages than the sequence has
        for n in [n_question] + [1] * n_decode:
            pos = torch.arange(t, t + n, device=DEV)[None]
            out, _, past = attn(hidden_states=xs[:, t:t + n], attention_mask=None,
                                position_ids=pos, past_key_value=past, output_attentions=False,
                                use_cache=True, padding_mask=None)
            assert past[-1] == t + n
            o = out[0].view(n, hq, 128).float().cpu().numpy()
            q, k, v = _qkv(attn, xs[:, t:t + n], pos)
            c = past[0].ctrl
            # the stand-in's selection of each token of this call
            sels = past[0].selections[-n:] if layer_id >= 2 else []
            assert layer_id < 2 or len(past[0].selections) == t + n - L0
            for i in range(n):
                qi = q[i][None, :, None, :]
                st_k, st_v = k[i][None, :, None, :], v[i][None, :, None, :]
                if layer_id >= 2:
                    o_ref, scores, pages = sim.decode_step(state, qi, st_k, st_v, budget, True,
                                                           value_aware, group)
                    # the stand-in's selection of this token: as many pages as
                    # the oracle's k, the same set up to near-ties
                    inv = {p: j for j, p in enumerate(c.kv_cache.indicies)}
                    mine = np.array([[inv[int(x)] for x in row] for row in sels[i].cpu().numpy()])
                    assert mine.shape[-1] == pages.shape[-1], (t + i, mine.shape, pages.shape)
                    dropped += int(mine.shape[-1] < len(c.kv_cache.indicies))
                    for hh in range(hkv):
                        ok, why = sim.selection_matches(mine[hh], pages[0, hh, 0],
                                                        scores[0, hh, 0], True)
                        assert ok, (t + i, hh, why)
                    o_ref = sim.sparse_decode_attention(
                        qi, np.repeat(state.K, group, 1), np.repeat(state.V, group, 1),
                        np.repeat(mine[None, :, None, :], group, 1), S, state.kv_len)
                else:
                    state.append(st_k, st_v)
                    o_ref = sim.masked_decode_attention(qi, np.repeat(state.K, group, 1),
                                                        np.repeat(state.V, group, 1), None)
                err = float(np.abs(o[i] - o_ref[0, :, 0].astype(np.float32)).max())
                assert err <= 2e-3, (t + i, err)
            t += n
        if layer_id >= 2:  # every step selects, also below the budget
            assert dropped >= 1, "no quest step dropped a page"



def test_cache_capacity_is_enforced():
    """A generation past the prefill plus decode_headroom raises instead of
    writing past the paged cache."""
    attn = _setup(4, 4, 3, True, 256, seed=1)
    attn.decode_headroom = 2
    x = torch.randn((1, 40, attn.config.hidden_size), device=DEV).half()
    with torch.no_grad():
        _, _, past = attn(hidden_states=x[:, :37], position_ids=torch.arange(37, device=DEV)[None],
                          past_key_value=None, use_cache=True)
        for t in (37, 38):
            _, _, past = attn(hidden_states=x[:, t:t + 1],
                              position_ids=torch.tensor([[t]], device=DEV),
                              past_key_value=past, use_cache=True)
        with pytest.raises(RuntimeError, match="outgrew"):
            attn(hidden_states=x[:, 39:40], position_ids=torch.tensor([[39]], device=DEV),
                 past_key_value=past, use_cache=True)
