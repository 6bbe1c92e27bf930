"""A Llama decoder stack whose attention is QuestAttention over libaoakv.so.

Mirrors the reference's model integration: ``QuestAttention.forward``
(quest/models/QuestAttention.py:56-181) and the controller calls of
``LlamaModel.forward`` / ``LlamaForCausalLM.quest_init`` (quest/models/
llama.py:424-486, 520-560), including the two leading layers that attend
densely (``_quest_skip_layer = 2``).  There is no checkpoint here: weights
are random (seeded), which is what a latency measurement needs; the shapes
are the model's.  Projections and the MLP are plain torch (hipBLASLt GEMMs);
RMSNorm, RoPE, the paged append, prefill and the decode layer are the
library's kernels.  Batch size 1, as the reference's QuestAttention.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch
from torch import nn

from . import tracing as tr
from . import utils as qutils
from .utils import InferenceController, TensorLayout


@dataclasses.dataclass
class LlamaShape:
    """Model shape (HF LlamaConfig fields the attention path reads)."""
    hidden_size: int = 4096
    num_attention_heads: int = 32
    num_key_value_heads: int = 32
    num_hidden_layers: int = 32
    intermediate_size: int = 11008
    rms_norm_eps: float = 1e-6
    rope_scale: float = 1.0  # linear RoPE scaling factor (longchat-v1.5: 8)
    rope_theta: float = 1e4


# The reference's latency models (latency/bench_latency.py:37-41), by shape.
MODEL_SHAPES = {
    "longchat-7b-v1.5-32k": LlamaShape(rope_scale=8.0),
    "llama2-7b": LlamaShape(rms_norm_eps=1e-5),
    "vicuna-7b-v1.5-16k": LlamaShape(rms_norm_eps=1e-5, rope_scale=4.0),
}


class RMSNorm(nn.Module):
    """The reference model's LlamaRMSNorm (quest/models/llama.py:62-72): one
    launch of the library's rms_norm kernel (utils.rms_norm_forward)."""

    def __init__(self, n: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return qutils.rms_norm_forward(x, self.weight, self.eps)


class QuestAttention(nn.Module):
    """QuestAttention.forward (QuestAttention.py:56-181) over aoakv.utils:
    projections, RoPE + append (one launch for a decode step), then prefill
    attention, dense decode (budget covers the sequence) or the sparse
    decode layer (one launch with ``single_launch``, else the reference's
    three calls estimate / top-k / sparse attention)."""

    def __init__(self, cfg: LlamaShape, layer_idx: int, single_launch: bool = True):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_heads = cfg.num_attention_heads
        self.num_key_value_heads = cfg.num_key_value_heads
        self.head_dim = cfg.hidden_size // cfg.num_attention_heads
        self.hidden_size = cfg.hidden_size
        self.rope_scale = cfg.rope_scale
        self.rope_theta = cfg.rope_theta
        self.single_launch = single_launch
        self.q_proj = nn.Linear(self.hidden_size, self.num_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim,
                                bias=False)
        self.v_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim,
                                bias=False)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, self.hidden_size, bias=False)

    def forward(self, hidden_states: torch.Tensor, iController: InferenceController):
        bsz, q_len, _ = hidden_states.shape
        assert bsz == 1, "QuestAttention only supports batch size 1."
        c = iController
        # roctx ranges named as the reference's nvtx ranges (QuestAttention.py:87-176);
        # RoPE and the append are one launch here
        with tr.range("qkv_proj"):
            q = self.q_proj(hidden_states).view(q_len, self.num_heads, self.head_dim)
            k = self.k_proj(hidden_states).view(q_len, self.num_key_value_heads, self.head_dim)
            v = self.v_proj(hidden_states).view(q_len, self.num_key_value_heads, self.head_dim)
        with tr.range("RoPE+append_kv"):
            qutils.rope_append_kv(q, k, v, c, self.layer_idx, rope_scale=self.rope_scale,
                                  rope_theta=self.rope_theta)
        if q_len > 1:
            with tr.range("prefill_attn"):
                o = qutils.prefill_forward(q, c, self.layer_idx)
        elif not c.need_estimate():
            with tr.range("full_attn"):
                o = qutils.decode_sparse_attn(q, c, self.layer_idx, c.kv_indices_without_last)
        elif self.single_launch:
            with tr.range("estimate+topk+approx_attn"):
                o = qutils.decode_layer(q, c, self.layer_idx, single_launch=True)
        else:
            with tr.range("estimate"):
                s = qutils.decode_estimate(q, c, self.layer_idx)
            with tr.range("topk"):
                qutils.decode_topk(s, c)
            with tr.range("approx_attn"):
                o = qutils.decode_sparse_attn(q, c, self.layer_idx, c.topk_dindices_buffer)
        with tr.range("o_proj"):
            return self.o_proj(o.reshape(1, q_len, self.hidden_size))


class LlamaMLP(nn.Module):
    def __init__(self, cfg: LlamaShape):
        super().__init__()
        self.gate_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.up_proj = nn.Linear(cfg.hidden_size, cfg.intermediate_size, bias=False)
        self.down_proj = nn.Linear(cfg.intermediate_size, cfg.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(nn.functional.silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, cfg: LlamaShape, layer_idx: int, single_launch: bool = True):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.self_attn = QuestAttention(cfg, layer_idx, single_launch)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.mlp = LlamaMLP(cfg)

    def forward(self, h, iController):
        # ranges as the reference's decoder layer (llama.py:138-164)
        with tr.range("input_norm"):
            x = self.input_layernorm(h)
        with tr.range("LlamaAttention"):
            h = h + self.self_attn(x, iController)
        with tr.range("norm"):
            x = self.post_attention_layernorm(h)
        with tr.range("mlp"):
            return h + self.mlp(x)


class QuestLlamaModel(nn.Module):
    """LlamaModel with the Quest controller (llama.py:424-486): the first
    ``skip_layers`` layers attend densely, the rest under the page budget."""

    def __init__(self, cfg: LlamaShape, single_launch: bool = True, skip_layers: int = 2):
        super().__init__()
        self.cfg = cfg
        self.layers = nn.ModuleList(DecoderLayer(cfg, i, single_launch)
                                    for i in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.iController: Optional[InferenceController] = None
        self._skip = skip_layers
        self._page_budget = 0
        self._max_page_limit = 1024 * 1024  # "arbitrary large" (llama.py:529)

    @torch.no_grad()
    def random_init(self, seed: int = 0, std: float = 0.02):
        g = torch.Generator(device=next(self.parameters()).device).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("layernorm.weight") or name == "norm.weight":
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=g)
        return self

    def quest_init(self, page_size: int, max_seq_len: int, token_budget: int = 512,
                   dtype=torch.float16, device="cuda:0", value_aware: bool = True,
                   semantics: str = "sim", layout: int = TensorLayout.HND):
        """Allocates the paged caches for max_seq_len tokens (llama.py:520-552)."""
        assert self.iController is None, "Can't init Quest Controller twice."
        cfg = self.cfg
        self._page_budget = token_budget // page_size
        self.iController = InferenceController(
            cfg.num_hidden_layers, cfg.num_attention_heads,
            cfg.hidden_size // cfg.num_attention_heads, page_size, self._page_budget,
            max_seq_len, dtype, device, layout=layout, num_kv_heads=cfg.num_key_value_heads,
            value_aware=value_aware, semantics=semantics)

    def quest_clear(self):
        """Frees the sequence's pages for a new conversation (llama.py:554-560)."""
        assert self.iController is not None, "Must be called after init."
        self.iController.clean_states()
        self.drop_graph()

    @torch.no_grad()
    def forward(self, inputs_embeds: torch.Tensor) -> torch.Tensor:
        c = self.iController
        assert c is not None, "Please init Quest Controller first."
        seq_len = inputs_embeds.shape[1]
        c.prepare_metadata(seq_len)
        if self._skip > 0:
            c.set_page_budget(self._max_page_limit)
            c.begin_forward(seq_len)
        return self._layers(inputs_embeds, seq_len, tables_written=self._skip > 0)

    def _layers(self, h: torch.Tensor, seq_len: int, tables_written: bool) -> torch.Tensor:
        """The decoder layers and the final norm, switching to the page budget
        after the dense layers (llama.py:465-475).  Past the first
        begin_forward (which writes the device page tables) the controller
        calls here change host state only."""
        c = self.iController
        for idx, layer in enumerate(self.layers):
            if idx == self._skip:
                c.end_forward()
                c.set_page_budget(self._page_budget)
                c.begin_forward(seq_len, updateTensor=(idx == 0 and not tables_written))
            with tr.range(f"layer={idx}"):  # llama.py:465-475
                h = layer(h, c)
        c.end_forward()
        return self.norm(h)

    @torch.no_grad()
    def decode_graphed(self, inputs_embeds: torch.Tensor) -> torch.Tensor:
        """One decode step (inputs_embeds [1, 1, hidden]) with the layers
        replayed from a HIP graph: the host planner runs first (it writes the
        device page tables: new page ids, page counts, the last page's length),
        then one replay launches every kernel of the step, instead of the
        dozens of host dispatches per layer of ``forward``.  The kernels take
        the token's position, page table and page count from those device
        tables; inside the graph the host passes them the cache's capacity as
        the page bound (``static_page_bound``), so the only argument that
        changes over a generation is whether the sparse layers select at all
        (the sequence outgrew the page budget), and the graph is captured
        again when it does.  The returned tensor is the graph's output
        buffer, overwritten by the next step.  Same results as ``forward``
        (the page bound sizes grids only)."""
        c = self.iController
        assert c is not None, "Please init Quest Controller first."
        assert tuple(inputs_embeds.shape[:2]) == (1, 1), "one token per decode step"
        assert not c.debug_checks, "debug_checks synchronize; not inside a graph"
        if not getattr(self, "_graph_warm", False):
            # the first single-token step runs eagerly: the GEMM libraries set
            # up their single-row paths on first use, which a capture cannot do
            self._graph_warm = True
            return self.forward(inputs_embeds)
        c.prepare_metadata(1)
        c.set_page_budget(self._max_page_limit if self._skip > 0 else self._page_budget)
        c.begin_forward(1)
        key = len(c.kv_cache.indicies) > self._page_budget  # the sparse layers select
        if getattr(self, "_graph_key", None) != key:
            # the previous graph and its memory pool go first (each capture
            # has a pool of its own)
            self._graph, self._graph_out = None, None
            if getattr(self, "_graph_in", None) is None:
                self._graph_in = torch.empty_like(inputs_embeds)
            self._graph_in.copy_(inputs_embeds)
            g = torch.cuda.CUDAGraph()
            c.static_page_bound = True
            try:
                with torch.cuda.graph(g):
                    self._graph_out = self._layers(self._graph_in, 1, tables_written=True)
            finally:
                c.static_page_bound = False
            self._graph, self._graph_key = g, key
        else:
            self._graph_in.copy_(inputs_embeds)
            # the host state forward leaves behind (page budget, selection view)
            c.end_forward()
            c.set_page_budget(self._page_budget)
            c.begin_forward(1, updateTensor=False)
        self._graph.replay()
        return self._graph_out

    def drop_graph(self):
        """Forget the captured decode step (quest_clear does, for a new
        conversation)."""
        self._graph, self._graph_out, self._graph_key = None, None, None
