"""The evaluation-side tree switch on the CPU: ``aoakv.evaluation``'s
``enable_quest_attention_eval`` numbers and patches an HF model's attention
modules as the reference's installer does (evaluation/quest_attention.py:
541-613): layer ids from the last layer down, the per-module settings, and
the value-aware or plain forward by ``args``; the forwards keep the
reference's signatures (quest_attention.py:38-47,196-206)."""
import inspect
import types

import pytest
import torch
from torch import nn

from aoakv import evaluation as ev

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig  # noqa: E402
from transformers.models.llama.modeling_llama import LlamaAttention  # noqa: E402


def _model(n_layers=4):
    cfg = LlamaConfig(hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
                      num_hidden_layers=n_layers, intermediate_size=512)
    m = nn.Module()
    m.config = cfg
    m.layers = nn.ModuleList()
    for i in range(n_layers):
        blk = nn.Module()
        blk.self_attn = LlamaAttention(cfg, layer_idx=i)
        blk.mlp = nn.Linear(4, 4)
        m.layers.append(blk)
    return m


def _args(**kw):
    base = dict(quest=True, value_aware=True, token_budget=1024, chunk_size=16, fixed=True,
                task="narrativeqa")
    base.update(kw)
    return types.SimpleNamespace(**base)


def test_layer_ids_settings_and_value_aware_forward():
    m = _model()
    assert ev.enable_quest_attention_eval(m, _args(max_gen=128)) == 4
    for i, blk in enumerate(m.layers):
        a = blk.self_attn
        assert a.layer_id == i
        assert (a.quest, a.token_budget, a.chunk_size, a.fixed) == (True, 1024, 16, True)
        assert a.decode_headroom == 128
        assert a.forward.__func__ is ev.forward_quest_value_aware_group_consistent_sum


def test_plain_quest_and_naive():
    m = _model()
    ev.enable_quest_attention_eval(m, _args(value_aware=False))
    assert all(b.self_attn.forward.__func__ is ev.forward_quest_group_consistent_sum
               for b in m.layers)
    m = _model()
    own = [b.self_attn.forward for b in m.layers]
    ev.enable_quest_attention_eval(m, _args(quest=False))
    assert [b.self_attn.forward for b in m.layers] == own  # naive: untouched


def test_unsupported_mode_is_refused():
    with pytest.raises(NotImplementedError):
        ev.enable_quest_attention_eval(_model(), _args(va_mode="avg_v_l2norm"))


def test_forward_signatures_match_the_reference():
    want = ["self", "hidden_states", "attention_mask", "position_ids", "past_key_value",
            "output_attentions", "use_cache", "input_ids", "kwargs"]
    for fn in (ev.forward_quest_value_aware_group_consistent_sum,
               ev.forward_quest_group_consistent_sum):
        assert list(inspect.signature(fn).parameters) == want
    assert "LlamaAttention" in [c.__name__ for c in ev.attention_classes()]
