"""Kernel-backed attention forwards for the reference's evaluation driver.

The reference's LongBench driver (evaluation/LongBench/pred.py:18,277-290)
patches every attention module of an HF model with
``enable_quest_attention_eval(model, args)`` (evaluation/quest_attention.py:
541-613), which installs one of its torch forwards:

* ``forward_quest_value_aware_group_consistent_sum`` (quest_attention.py:
  196-382) with ``args.quest and args.value_aware``;
* ``forward_quest_group_consistent_sum`` (quest_attention.py:38-194) with
  ``args.quest`` alone.

This module has the same three names, the same call convention (the
4.45-era attention call of the reference's tuple-cache decoder layer,
evaluation/llama.py:507-536: ``hidden_states, attention_mask, position_ids,
past_key_value, output_attentions, use_cache, **kwargs`` -> ``(attn_output,
None, past_key_value)``), and computes the attention on libaoakv.so: a
driver switches trees by importing ``enable_quest_attention_eval`` from
``aoakv.evaluation`` instead of ``evaluation.quest_attention``.

What the forwards do, per layer and sequence (batch 1, as the reference's
driver):

* projections and RoPE as the module defines them (its ``q/k/v/o_proj`` and
  ``rotary_emb``, or the ``position_embeddings`` a newer decoder layer
  passes), then q, k, v in fp16 (the kernels' type; the reference casts its
  prefill to fp16 the same way, quest_attention.py:223-227);
* prefill (no past): the paged append with the page filters, page means of V
  and their log-norms (``get_max_min_filters`` / ``compute_page_v_mean``,
  quest_attention.py:238-245) and the causal prefill kernel;
* decode (one new token): the decode append (``update_page_filters``,
  ``update_mean_page_filters``) and, from layer 2 on, the value-aware (or
  plain) page scores, the group-consistent top-k of
  ``k = min(max(3, min(kv_seq_len, token_budget) // chunk_size), P)`` pages
  and the sparse attention over them (quest_attention.py:249-356,
  filter_util.py:373) -- on every step, as the reference selects on every
  step: with ``kv_seq_len <= token_budget`` and a partial last page, k is
  P - 1 and the lowest-scored page is dropped.  Two launches (estimate +
  top-k, then decode), which have no bounded waits.  Layers 0 and 1 attend
  every page;
* several new tokens after a prefill (the driver's question stage,
  pred.py:144-215): decoded one token after another, each as a decode step.
  The reference's torch forward instead scores that block's rows against
  filters that already hold the whole block's keys and masks the result
  causally (quest_attention.py:296-330); one token at a time is what
  generation does, and it is what the kernels compute.

The cache that comes back in ``past_key_value`` is ``(LayerCache, layer_id,
kv_seq_len)``: the paged cache object, and the sequence length last, which is
where the reference's model forward reads it (evaluation/llama.py:411-415).
Its capacity is the prefill length plus ``decode_headroom`` tokens
(``args.max_gen`` if the driver has it, else 4096); a longer generation
raises.
"""
from __future__ import annotations

import types
from typing import Optional

import torch

from . import utils as qutils
from .utils import InferenceController, TensorLayout

DEFAULT_HEADROOM = 4096


def _heads(mod):
    """(query heads, kv heads, head dim, hidden size) of an attention module
    (4.45 attributes, or the config of newer transformers)."""
    cfg = getattr(mod, "config", None)
    hq = getattr(mod, "num_heads", None) or cfg.num_attention_heads
    hkv = getattr(mod, "num_key_value_heads", None) or cfg.num_key_value_heads
    d = getattr(mod, "head_dim", None) or (cfg.hidden_size // cfg.num_attention_heads)
    return hq, hkv, d, hq * d


class LayerCache:
    """One attention layer's paged cache for one sequence: a one-layer
    ``InferenceController`` (HND pages of ``chunk_size`` tokens) with the
    layer's page filters, page means of V and their log-norms."""

    def __init__(self, mod, capacity: int, device, value_aware: bool):
        hq, hkv, d, _ = _heads(mod)
        self.chunk_size = int(getattr(mod, "chunk_size", 16))
        budget = int(getattr(mod, "token_budget", 0))
        self.ctrl = InferenceController(
            1, hq, d, self.chunk_size, max(budget // self.chunk_size, 0), capacity,
            torch.float16, device, layout=TensorLayout.HND, num_kv_heads=hkv,
            fixed=bool(getattr(mod, "fixed", False)), value_aware=value_aware)
        self.capacity = capacity
        # with keep_selections set, every decode token's selection (physical
        # page ids [Hkv, k], a copy) is appended to `selections` (for checks)
        self.keep_selections = False
        self.selections = []

    @property
    def seq_len(self) -> int:
        return self.ctrl.kv_cache.seqlen

    def append(self, k: torch.Tensor, v: torch.Tensor):
        """k, v: (n, Hkv, D) fp16, already rotated."""
        n = k.shape[0]
        if self.seq_len + n > self.capacity:
            raise RuntimeError(f"aoakv.evaluation: the sequence outgrew its cache ({self.capacity} "
                               "tokens); raise decode_headroom (args.max_gen)")
        c = self.ctrl
        c.prepare_metadata(n)
        c.begin_forward(n)
        qutils.append_kv(k, v, c, 0)


def _rope(mod, q, k, v, position_ids, kwargs):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    pe = kwargs.get("position_embeddings")
    if pe is not None:
        cos, sin = pe
    else:
        cos, sin = mod.rotary_emb(v, position_ids.to(v.device))
    return apply_rotary_pos_emb(q, k, cos, sin)


def _decode_one(mod, cache: LayerCache, q: torch.Tensor, quest: bool) -> torch.Tensor:
    """Attention of one query (Hq, D) fp16 over the cache (its token already
    appended): the budget's selection from layer 2 on (every step, as
    quest_attention.py:324-331), every page before."""
    c = cache.ctrl
    budget_tokens = int(getattr(mod, "token_budget", 0))
    c.set_page_budget(budget_tokens // cache.chunk_size if quest else c.max_kv_pages)
    c.begin_forward(1, updateTensor=False)
    q3 = q.view(1, c.num_heads, c.head_dim)
    if quest and budget_tokens > 0:
        o = qutils.decode_layer(q3, c, 0, single_launch=False)
        if cache.keep_selections:
            cache.selections.append(c._sel[0, :, :c.num_selected_pages()].clone())
        return o
    return qutils.decode_sparse_attn(q3, c, 0, None)


def _forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_value=None,
             output_attentions=False, use_cache=False, input_ids=None, value_aware=True,
             **kwargs):
    bsz, q_len, _ = hidden_states.size()
    if bsz != 1:
        raise ValueError("aoakv.evaluation: batch size 1 (as the reference's evaluation driver)")
    hq, hkv, d, hidden = _heads(self)
    dtype = hidden_states.dtype
    q = self.q_proj(hidden_states).view(bsz, q_len, hq, d).transpose(1, 2)
    k = self.k_proj(hidden_states).view(bsz, q_len, hkv, d).transpose(1, 2)
    v = self.v_proj(hidden_states).view(bsz, q_len, hkv, d).transpose(1, 2)
    past_len = 0 if past_key_value is None else int(past_key_value[-1])
    if position_ids is None:
        position_ids = torch.arange(past_len, past_len + q_len, device=hidden_states.device)[None]
    q, k = _rope(self, q, k, v, position_ids, kwargs)
    # (tokens, heads, dim) fp16 for the kernels
    q16 = q[0].transpose(0, 1).to(torch.float16).contiguous()
    k16 = k[0].transpose(0, 1).to(torch.float16).contiguous()
    v16 = v[0].transpose(0, 1).to(torch.float16).contiguous()
    quest = bool(getattr(self, "quest", True)) and getattr(self, "layer_id", 0) >= 2
    if past_key_value is None:  # prefill
        headroom = int(getattr(self, "decode_headroom", DEFAULT_HEADROOM))
        cache = LayerCache(self, q_len + headroom, hidden_states.device, value_aware)
        cache.append(k16, v16)
        o = qutils.prefill_forward(q16, cache.ctrl, 0)
    else:
        cache = past_key_value[0]
        if not isinstance(cache, LayerCache):
            raise TypeError("aoakv.evaluation: past_key_value was not made by this forward")
        rows = []
        for i in range(q_len):  # one decode step per new token
            cache.append(k16[i:i + 1], v16[i:i + 1])
            rows.append(_decode_one(self, cache, q16[i], quest).view(1, hq, d))
        o = torch.cat(rows, 0)
    attn_output = self.o_proj(o.to(dtype).reshape(bsz, q_len, hidden))
    kv_seq_len = past_len + q_len
    past = (cache, getattr(self, "layer_id", None), kv_seq_len) if use_cache else None
    return attn_output, None, past


def forward_quest_value_aware_group_consistent_sum(
        self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
        position_ids: Optional[torch.LongTensor] = None, past_key_value=None,
        output_attentions: bool = False, use_cache: bool = False,
        input_ids: Optional[torch.LongTensor] = None, **kwargs):
    """quest_attention.py:196-382 on libaoakv.so: value-aware page scores
    (2 (bound / sqrt(d)) + 2 log ||mean V||), group-consistent over the query
    heads of a kv head."""
    return _forward(self, hidden_states, attention_mask, position_ids, past_key_value,
                    output_attentions, use_cache, input_ids, value_aware=True, **kwargs)


def forward_quest_group_consistent_sum(
        self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
        position_ids: Optional[torch.LongTensor] = None, past_key_value=None,
        output_attentions: bool = False, use_cache: bool = False,
        input_ids: Optional[torch.LongTensor] = None, **kwargs):
    """quest_attention.py:38-194 on libaoakv.so: plain Quest page bounds,
    summed over the query heads of a kv head."""
    return _forward(self, hidden_states, attention_mask, position_ids, past_key_value,
                    output_attentions, use_cache, input_ids, value_aware=False, **kwargs)


def attention_classes() -> tuple:
    """The attention module classes the reference's installer patches
    (LlamaAttention, MistralAttention, Qwen2Attention and, where the installed
    transformers has them, Qwen2's flash / SDPA variants)."""
    out = []
    for mod, names in (("transformers.models.llama.modeling_llama", ("LlamaAttention",)),
                       ("transformers.models.mistral.modeling_mistral", ("MistralAttention",)),
                       ("transformers.models.qwen2.modeling_qwen2",
                        ("Qwen2Attention", "Qwen2FlashAttention2", "Qwen2SdpaAttention"))):
        try:
            m = __import__(mod, fromlist=list(names))
        except Exception:  # noqa: BLE001  (an absent model family)
            continue
        out += [getattr(m, n) for n in names if hasattr(m, n)]
    return tuple(out)


def enable_quest_attention_eval(model, args, classes: Optional[tuple] = None) -> int:
    """quest_attention.py:541-613: numbers the attention modules from the
    last layer down (layer_id, as the reference's walk over reversed
    children), sets ``quest``, ``token_budget``, ``chunk_size``, ``fixed`` (and
    ``decode_headroom`` from ``args.max_gen``) on each, and installs the
    value-aware forward (``args.quest and args.value_aware``) or the plain
    one (``args.quest``); without ``args.quest`` the modules keep their own
    forward.  ``classes`` overrides the module classes to patch.  Returns the
    number of modules numbered.  The reference keeps its layer counter in a
    module global across calls; here each call numbers its own model."""
    classes = attention_classes() if classes is None else classes
    n_layers = getattr(getattr(model, "config", None), "num_hidden_layers", None)
    if getattr(args, "va_mode", "default") == "avg_v_l2norm":
        raise NotImplementedError("va_mode avg_v_l2norm (quest_attention.py:385-539) has no "
                                  "kernel here; the value-aware mode is the default one")
    found = []

    def walk(m):
        for name, child in reversed(list(m._modules.items())):
            if child is None:
                continue
            if len(list(child.children())) > 0:
                walk(child)
            if isinstance(child, classes):
                found.append(child)

    walk(model)
    total = n_layers if n_layers is not None else len(found)
    for i, mod in enumerate(found):  # found from the last layer down
        mod.layer_id = total - 1 - i
        mod.flash_forward = mod.forward
        mod.quest = bool(getattr(args, "quest", False))
        mod.token_budget = int(getattr(args, "token_budget", 0))
        mod.chunk_size = int(getattr(args, "chunk_size", 16))
        mod.fixed = bool(getattr(args, "fixed", False))
        mod.decode_headroom = int(getattr(args, "max_gen", None) or DEFAULT_HEADROOM)
        if mod.quest and getattr(args, "value_aware", False):
            mod.forward = types.MethodType(forward_quest_value_aware_group_consistent_sum, mod)
        elif mod.quest:
            mod.forward = types.MethodType(forward_quest_group_consistent_sum, mod)
    return len(found)
