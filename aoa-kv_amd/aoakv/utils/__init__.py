"""Mirror of the reference's ``quest.utils`` op wrappers
(kernels/aoa_kv/quest/utils/__init__.py:69-285), backed by libaoakv.so.

Same names, same argument meaning, same call order as QuestAttention.forward
(QuestAttention.py:99-157)::

    append_kv(k, v, ctrl, layer)                  # [N, H, D] new tokens
    o = prefill_forward(q, ctrl, layer)           # N > 1
    s = decode_estimate(q, ctrl, layer)           # [Hkv, P] fp32 page scores
    decode_topk(s, ctrl)                          # -> ctrl.topk_dindices_buffer
    o = decode_sparse_attn(q, ctrl, layer, ctrl.topk_dindices_buffer)

``decode_sparse_attn(q, ctrl, layer, ctrl.kv_indices_without_last)`` (or
``None``) attends every page, as the reference's dense-layer path does.  Any
other ``topk_indices`` tensor of physical page ids, ``[Hkv, n]``, is attended
as given (with the quest_kernel convention the last page is added, as the
reference's ``decode_sparse_attn`` does with ``kv_last_page_idx``).
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import ops
from .controller import InferenceController
from .kv_cache import KvCache, KvPool
from .utils import TensorLayout

__all__ = [
    "TensorLayout",
    "KvCache",
    "KvPool",
    "InferenceController",
    "apply_rope_in_place",
    "rms_norm_forward",
    "append_kv",
    "rope_append_kv",
    "prefill_forward",
    "decode_estimate",
    "decode_topk",
    "decode_sparse_attn",
    "decode_layer",
]


def apply_rope_in_place(q: torch.Tensor, k: torch.Tensor, past_kv_len: int,
                        rope_scale: Optional[float] = None, rope_theta: Optional[float] = None):
    """RoPE of q [N, Hq, D] and k [N, Hkv, D] in place, token n at position
    past_kv_len + n (reference __init__.py:25-52; defaults scale 1, theta 1e4)."""
    ops.apply_rope_in_place(q, k, past_kv_len, 1.0 if rope_scale is None else rope_scale,
                            1e4 if rope_theta is None else rope_theta)


def rms_norm_forward(input: torch.Tensor, weight: torch.Tensor, epsilon: float) -> torch.Tensor:
    """RMSNorm of the last dim (reference __init__.py:54-67): libaoakv's
    rms_norm kernel (aoakv_rms_norm_forward), r = 1/sqrt(sum(x^2)/n + eps) in
    fp32 over the fp32 values of x, then (x * r) * weight in fp32, rounded
    once to fp16.  A new output tensor, as the reference returns."""
    o = torch.empty_like(input)
    ops.rms_norm_forward(input.contiguous(), weight.contiguous(), o, epsilon)
    return o


def rope_append_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   iController: InferenceController, layer_idx: int,
                   rope_scale: Optional[float] = None, rope_theta: Optional[float] = None):
    """apply_rope_in_place(q, k, seqlen - N) then append_kv(k, v) -- the
    reference's two calls at QuestAttention.py:98-111 -- with the decode step
    (N == 1) in one launch.  q and k are left rotated, as the reference leaves
    them.  Call after begin_forward, like append_kv."""
    c = iController
    scale = 1.0 if rope_scale is None else rope_scale
    theta = 1e4 if rope_theta is None else rope_theta
    if k.size(0) > 1:
        ops.apply_rope_in_place(q, k, c.kv_cache.seqlen - k.size(0), scale, theta)
        append_kv(k, v, c, layer_idx)
        return
    ops.rope_append_kv_cache_decode(
        q.view(1, -1, c.head_dim), k, v, c.kv_cache.buf_layer(layer_idx),
        c.kv_indptr_for_append, c.kv_indices_with_last, c.kv_last_page_len_t,
        c.metadata_cache.buf_layer(layer_idx), c.metadata_indptr_for_append, c.metadata_indices,
        c.v_log_norm_layer(layer_idx), c.v_mean_layer(layer_idx), c.layout, scale, theta)


def append_kv(k: torch.Tensor, v: torch.Tensor, iController: InferenceController,
              layer_idx: int):
    """Append new k/v [N, H, D] to the layer's cache and metadata
    (reference __init__.py:69-131).  N > 1: bulk append; N == 1: decode append."""
    c = iController
    if k.size(0) > 1:
        ops.append_kv_cache_prefill(
            k, v, c.kv_cache.buf_layer(layer_idx), c.kv_indices_with_last,
            len(c.kv_cache.indicies), c.kv_cache.last_page_len,
            c.metadata_cache.buf_layer(layer_idx), c.metadata_indices,
            c.v_log_norm_layer(layer_idx), c.v_mean_layer(layer_idx), c.layout)
    else:
        ops.append_kv_cache_decode(
            k, v, c.kv_cache.buf_layer(layer_idx), c.kv_indptr_for_append,
            c.kv_indices_with_last, c.kv_last_page_len_t,
            c.metadata_cache.buf_layer(layer_idx), c.metadata_indptr_for_append,
            c.metadata_indices, c.v_log_norm_layer(layer_idx), c.v_mean_layer(layer_idx),
            c.layout)


def prefill_forward(q: torch.Tensor, iController: InferenceController, layer_idx: int,
                    rope_scale: Optional[float] = None, rope_theta: Optional[float] = None
                    ) -> torch.Tensor:
    """Causal attention of the new tokens over the cache (reference
    __init__.py:133-175).  RoPE is applied by the caller (rope_* unused)."""
    c = iController
    return ops.prefill_with_paged_kv_cache(
        q, c.kv_cache.buf_layer(layer_idx), c.kv_indices_with_last, len(c.kv_cache.indicies),
        c.kv_cache.last_page_len, c.layout, causal=True)


def decode_estimate(q: torch.Tensor, iController: InferenceController, layer_idx: int
                    ) -> torch.Tensor:
    """Page scores of every page, [Hkv, P] fp32 (reference __init__.py:177-214);
    [Hkv, P - 1] with the quest_kernel convention (the last page unscored)."""
    c = iController
    P = len(c.kv_cache.indicies)
    ops.estimate_attn_score(
        q.view(1, c.num_heads, c.head_dim), c.scores, c.metadata_cache.buf_layer(layer_idx),
        c.metadata_indptr_for_append, c.metadata_indices, c.kv_indptr_for_append,
        c.kv_indices_with_last, c.kv_last_page_len_t, c.v_log_norm_layer(layer_idx),
        c.decode_max_pages, c.layout, c.flags)
    return c.scores[0, :, :P - 1 if c.quest_kernel else P]


def decode_topk(estimated_attn_score: torch.Tensor, iController: InferenceController):
    """Top-k pages per kv head into ``topk_dindices_buffer`` [Hkv, k] (physical
    page ids, ascending) (reference __init__.py:216-246); [Hkv, k - 1], the
    pages besides the last, with the quest_kernel convention."""
    c = iController
    ops.topk_filtering(c.scores, c.kv_indptr_for_append, c.kv_indices_with_last,
                       c.kv_last_page_len_t, c.token_budget, c._sel, c.page_size, c.flags,
                       workspace=c.workspace)
    return c.topk_dindices_buffer[0]


def decode_sparse_attn(q: torch.Tensor, iController: InferenceController, layer_idx: int,
                       topk_indices: Optional[torch.Tensor],
                       rope_scale: Optional[float] = None,
                       rope_theta: Optional[float] = None) -> torch.Tensor:
    """Attention of q [1, H, D] over the selected pages (reference
    __init__.py:248-285); dense over all pages when topk_indices is None or
    ``iController.kv_indices_without_last``."""
    c = iController
    dense = topk_indices is None or topk_indices is c.kv_indices_without_last
    if dense:
        sel = None
    elif (topk_indices.dtype == torch.int32 and topk_indices.is_cuda and
          topk_indices.untyped_storage().data_ptr() == c._sel.untyped_storage().data_ptr()):
        sel = c._sel  # this controller's own top-k output (row stride max_kv_pages)
    else:
        if topk_indices.dim() == 3:
            topk_indices = topk_indices[0]
        if topk_indices.dim() != 2 or topk_indices.shape[0] != c.num_kv_heads:
            raise ValueError(f"topk_indices must be [{c.num_kv_heads}, n] physical page ids, "
                             f"got {tuple(topk_indices.shape)}")
        sel = topk_indices.to(device=c.device, dtype=torch.int32).contiguous().unsqueeze(0)
        if sel.shape[-1] == 0:  # quest_kernel with a one-page budget: the last page only
            sel = torch.zeros((1, c.num_kv_heads, 1), dtype=torch.int32, device=c.device)
    q3 = q.view(1, c.num_heads, c.head_dim)
    o = torch.empty_like(q3)
    ops.decode_sparse_attn(
        q3, o, c.kv_cache.buf_layer(layer_idx), c.kv_indptr_for_append, c.kv_indices_with_last,
        c.kv_last_page_len_t, sel, c.token_budget, c.workspace, c.decode_max_pages,
        c.num_kv_heads, c.layout, flags=c.flags & ops.FLAG_QUEST_KERNEL)
    return o.view_as(q)


def decode_layer(q: torch.Tensor, iController: InferenceController, layer_idx: int,
                 single_launch: bool = False) -> torch.Tensor:
    """estimate + top-k + sparse decode in two launches (or one, with
    ``single_launch``).  A one-launch call whose wait gave up leaves NaN
    outputs from then on until the workspace is re-initialized;
    ``iController.check_errors()`` reports it (and re-initializes), and with
    ``iController.debug_checks`` it runs after every call."""
    c = iController
    q3 = q.view(1, c.num_heads, c.head_dim)
    o = torch.empty_like(q3)
    ops.sparse_decode_layer(
        q3, o, c.kv_cache.buf_layer(layer_idx), c.kv_indptr_for_append, c.kv_indices_with_last,
        c.kv_last_page_len_t, c.metadata_cache.buf_layer(layer_idx),
        c.metadata_indptr_for_append, c.metadata_indices, c.v_log_norm_layer(layer_idx),
        c.scores, c._sel, c.token_budget, c.workspace, c.decode_max_pages, c.layout,
        c.flags | (ops.FLAG_SINGLE_LAUNCH if single_launch else 0))
    if c.debug_checks:
        c.check_errors()
    return o.view_as(q)
