"""torch-tensor wrappers of the libaoakv.so entry points.

Each function checks dtypes, devices and shapes, then calls the C ABI with
raw device pointers on torch's current HIP stream.  Tensors are never
copied or converted here: a wrong dtype / layout is an error, not a cast.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from ._lib import (FLAG_FIXED, FLAG_GROUPED_DECODE, FLAG_QUEST_KERNEL,  # noqa: F401
                   FLAG_SINGLE_LAUNCH, FLAG_VALUE_AWARE)  # (re-exported)

NHD = 0
HND = 1


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def cache_dims(kv_data: torch.Tensor, layout: int):
    """(max_pages, page_size, num_heads, head_dim) of a paged cache tensor
    [max_pages, 2, S, H, D] (NHD) or [max_pages, 2, H, S, D] (HND)."""
    if kv_data.dim() != 5 or kv_data.shape[1] != 2:
        raise ValueError(f"paged cache must be 5-d [pages, 2, ., ., D], got {tuple(kv_data.shape)}")
    if layout == NHD:
        P, _, S, H, D = kv_data.shape
    elif layout == HND:
        P, _, H, S, D = kv_data.shape
    else:
        raise ValueError(f"unknown layout {layout}")
    return P, S, H, D


def append_kv_cache_prefill(k, v, kv_data, kv_indices, num_kv_pages: int, kv_last_page_len: int,
                            metadata_data, metadata_indices, v_log_norm, v_mean, layout: int):
    """Reference: quest/ops/csrc/page.cu:107-222 (append_kv_cache_prefill)."""
    for t, n in ((k, "k"), (v, "v"), (kv_data, "kv_data"), (metadata_data, "metadata_data"),
                 (v_log_norm, "v_log_norm"), (v_mean, "v_mean")):
        _need(t, n, torch.float16)
    _need(kv_indices, "kv_indices", torch.int32)
    _need(metadata_indices, "metadata_indices", torch.int32)
    _, S, H, D = cache_dims(kv_data, layout)
    if k.shape != v.shape or k.dim() != 3 or k.shape[1] != H or k.shape[2] != D:
        raise ValueError(f"k/v must be [N, {H}, {D}], got {tuple(k.shape)} / {tuple(v.shape)}")
    if kv_indices.numel() < num_kv_pages:
        raise ValueError("kv_indices shorter than num_kv_pages")
    _lib.call("aoakv_append_kv_cache_prefill", k.data_ptr(), v.data_ptr(), k.shape[0],
              kv_data.data_ptr(), kv_indices.data_ptr(), num_kv_pages, kv_last_page_len,
              metadata_data.data_ptr(), metadata_indices.data_ptr(), v_log_norm.data_ptr(),
              v_mean.data_ptr(), H, D, S, layout, _stream())


def append_kv_cache_decode(k, v, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                           metadata_data, metadata_indptr, metadata_indices, v_log_norm, v_mean,
                           layout: int):
    """Reference: quest/ops/csrc/page.cu:6-105 (append_kv_cache_decode); k, v
    are [B, H, D], one new token per sequence."""
    for t, n in ((k, "k"), (v, "v"), (kv_data, "kv_data"), (metadata_data, "metadata_data"),
                 (v_log_norm, "v_log_norm"), (v_mean, "v_mean")):
        _need(t, n, torch.float16)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                 (kv_last_page_len, "kv_last_page_len"), (metadata_indptr, "metadata_indptr"),
                 (metadata_indices, "metadata_indices")):
        _need(t, n, torch.int32)
    _, S, H, D = cache_dims(kv_data, layout)
    B = k.shape[0]
    if k.shape != (B, H, D) or v.shape != (B, H, D):
        raise ValueError(f"k/v must be [B, {H}, {D}]")
    if kv_indptr.numel() != B + 1 or kv_last_page_len.numel() != B or metadata_indptr.numel() != B + 1:
        raise ValueError("indptr / last_page_len sizes do not match the batch")
    _lib.call("aoakv_append_kv_cache_decode", k.data_ptr(), v.data_ptr(), B, kv_data.data_ptr(),
              kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
              metadata_data.data_ptr(), metadata_indptr.data_ptr(), metadata_indices.data_ptr(),
              v_log_norm.data_ptr(), v_mean.data_ptr(), H, D, S, layout, _stream())


def apply_rope_in_place(q, k, past_kv_len: int, rope_scale: float = 1.0,
                        rope_theta: float = 1e4):
    """Reference: quest/ops/csrc/page.cu:224-265.  q [N, Hq, D], k [N, Hkv, D]
    fp16, rotated in place; token n at position past_kv_len + n."""
    _need(q, "q", torch.float16)
    _need(k, "k", torch.float16)
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError(f"q / k must be [N, H, D] with the same N and D, got "
                         f"{tuple(q.shape)} / {tuple(k.shape)}")
    _lib.call("aoakv_apply_rope_in_place", q.data_ptr(), k.data_ptr(), q.shape[0], past_kv_len,
              q.shape[1], k.shape[1], q.shape[2], float(rope_scale), float(rope_theta),
              _stream())


def rms_norm_forward(input, weight, output, epsilon: float):
    """Reference: quest/ops/csrc/rms_norm.cu:185-213 (bsk_ops.h:29): RMSNorm of
    input [..., n] fp16 (rows over the leading dims) with weight [n] into
    output (input's shape; may be input itself)."""
    _need(input, "input", torch.float16)
    _need(weight, "weight", torch.float16)
    _need(output, "output", torch.float16)
    n = input.shape[-1]
    if weight.shape != (n,) or output.shape != input.shape:
        raise ValueError(f"weight must be [{n}] and output {tuple(input.shape)}, got "
                         f"{tuple(weight.shape)} / {tuple(output.shape)}")
    _lib.call("aoakv_rms_norm_forward", input.data_ptr(), weight.data_ptr(), output.data_ptr(),
              input.numel() // n, n, float(epsilon), _stream())


def rope_append_kv_cache_decode(q, k, v, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                                metadata_data, metadata_indptr, metadata_indices, v_log_norm,
                                v_mean, layout: int, rope_scale: float = 1.0,
                                rope_theta: float = 1e4):
    """apply_rope_in_place + append_kv_cache_decode in one launch: q [B, Hq, D]
    and k [B, H, D] rotated in place at each sequence's new position, then k, v
    appended with metadata (reference calls QuestAttention.py:98-111)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (kv_data, "kv_data"),
                 (metadata_data, "metadata_data"), (v_log_norm, "v_log_norm"), (v_mean, "v_mean")):
        _need(t, n, torch.float16)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                 (kv_last_page_len, "kv_last_page_len"), (metadata_indptr, "metadata_indptr"),
                 (metadata_indices, "metadata_indices")):
        _need(t, n, torch.int32)
    _, S, H, D = cache_dims(kv_data, layout)
    B = k.shape[0]
    if k.shape != (B, H, D) or v.shape != (B, H, D) or q.dim() != 3 or q.shape[0] != B \
            or q.shape[2] != D:
        raise ValueError(f"q must be [B, Hq, {D}], k/v [B, {H}, {D}]")
    if kv_indptr.numel() != B + 1 or kv_last_page_len.numel() != B or metadata_indptr.numel() != B + 1:
        raise ValueError("indptr / last_page_len sizes do not match the batch")
    _lib.call("aoakv_rope_append_kv_cache_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), B,
              q.shape[1], kv_data.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
              kv_last_page_len.data_ptr(), metadata_data.data_ptr(), metadata_indptr.data_ptr(),
              metadata_indices.data_ptr(), v_log_norm.data_ptr(), v_mean.data_ptr(), H, D, S,
              layout, float(rope_scale), float(rope_theta), _stream())


def estimate_attn_score(q, scores, metadata_data, metadata_indptr, metadata_indices, kv_indptr,
                        kv_indices, kv_last_page_len, v_log_norm, max_pages: int, layout: int,
                        flags: int = FLAG_VALUE_AWARE):
    """Reference: quest/ops/csrc/estimate.cu:6-90.  q [B, Hq, D] fp16 ->
    scores [B, Hkv, stride] fp32 (stride = scores.shape[-1])."""
    _need(q, "q", torch.float16)
    _need(scores, "scores", torch.float32)
    _need(metadata_data, "metadata_data", torch.float16)
    for t, n in ((metadata_indptr, "metadata_indptr"), (metadata_indices, "metadata_indices"),
                 (kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                 (kv_last_page_len, "kv_last_page_len")):
        _need(t, n, torch.int32)
    if flags & FLAG_VALUE_AWARE:
        _need(v_log_norm, "v_log_norm", torch.float16)
    _, S, Hkv, D = cache_dims(metadata_data, layout)
    B, Hq, Dq = q.shape
    if Dq != D or scores.dim() != 3 or scores.shape[0] != B or scores.shape[1] != Hkv:
        raise ValueError(f"scores must be [B, {Hkv}, >= max_pages]")
    _lib.call("aoakv_estimate_attn_score", q.data_ptr(), scores.data_ptr(), scores.shape[2],
              metadata_data.data_ptr(), metadata_indptr.data_ptr(), metadata_indices.data_ptr(),
              kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
              _ptr(v_log_norm), B, max_pages, Hq, Hkv, D, S, layout, flags, _stream())


def topk_filtering(scores, kv_indptr, kv_indices, kv_last_page_len, token_budget: int, sel_pages,
                   page_size: int = 16, flags: int = FLAG_FIXED, token_budgets=None,
                   workspace=None):
    """Reference: quest/ops/csrc/topk.cu:7-46.  Writes sel_pages [B, Hkv, k_max]
    (physical page ids, ascending logical order).  ``workspace``: a decode
    workspace whose error word receives WS_ERR_TRUNCATED when a page table
    holds more pages than a score row (None: not reported)."""
    _need(scores, "scores", torch.float32)
    _need(sel_pages, "sel_pages", torch.int32)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                 (kv_last_page_len, "kv_last_page_len")):
        _need(t, n, torch.int32)
    if token_budgets is not None:
        _need(token_budgets, "token_budgets", torch.int32)
    B, Hkv, stride = scores.shape
    if sel_pages.dim() != 3 or sel_pages.shape[:2] != (B, Hkv):
        raise ValueError("sel_pages must be [B, Hkv, k_max]")
    err = None
    if workspace is not None:
        _need(workspace, "workspace", torch.uint8)
        if workspace.numel() < 12:
            raise ValueError("workspace too small to hold the error word")
        err = workspace.data_ptr() + 4 * WS_ERR_WORD
    _lib.call("aoakv_topk_filtering", scores.data_ptr(), stride, kv_indptr.data_ptr(),
              kv_indices.data_ptr(), kv_last_page_len.data_ptr(), token_budget,
              _ptr(token_budgets), sel_pages.data_ptr(), sel_pages.shape[2], B, Hkv, page_size,
              flags, err, _stream())


def decode_workspace(batch: int, num_qo_heads: int, num_kv_heads: int, max_sel_pages: int,
                     device="cuda", max_pages: int = 0, head_dim: int = 128) -> torch.Tensor:
    """Caller-owned decode workspace (replaces BatchDecodeHandler's buffers,
    decode_handler.cuh:73-136), zeroed.  With max_pages it also holds the
    one-launch layer's score handoff words (aoakv_layer_workspace_size).
    Its split-K partials hold head_dim + 4 floats per chunk."""
    lib = _lib.load()
    if max_pages:
        n = lib.aoakv_layer_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim,
                                           max_sel_pages, max_pages)
    else:
        n = lib.aoakv_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim,
                                            max_sel_pages)
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    _lib.call("aoakv_workspace_init", ws.data_ptr(), n, _stream())
    return ws


# bytes of a workspace's control words (aoakv.h AOAKV_WORKSPACE_CTL_BYTES)
WORKSPACE_CTL_BYTES = 256
# the workspace error word (aoakv.h AOAKV_WS_ERR_WORD) and its bits
WS_ERR_WORD = 2
WS_ERR_WAIT = 1
WS_ERR_TRUNCATED = 2


def workspace_error(workspace: torch.Tensor) -> int:
    """The workspace's error bits (32-bit word 2, aoakv.h AOAKV_WS_ERR_WORD):
    WS_ERR_WAIT when a one-launch layer call had a bounded wait give up (its
    output is invalid; later one-launch calls write NaN until
    ``workspace_init``), WS_ERR_TRUNCATED when a device page table held more
    pages than a call was sized for.  Reads the word back, so it
    synchronizes with the stream."""
    w = 4 * WS_ERR_WORD
    return int(workspace[w:w + 4].view(torch.int32).item())


def workspace_wait_failed(workspace: torch.Tensor) -> bool:
    """True when a one-launch layer call on this workspace had a bounded wait
    give up (WS_ERR_WAIT; reads the word back, so it synchronizes).  The
    workspace must be re-initialized (``workspace_init``) before it is used
    again."""
    return bool(workspace_error(workspace) & WS_ERR_WAIT)


def workspace_init(workspace: torch.Tensor) -> None:
    """Zero a decode workspace (aoakv_workspace_init) on the current stream."""
    _lib.call("aoakv_workspace_init", workspace.data_ptr(), workspace.numel(), _stream())


def decode_sparse_attn(q, o, kv_data, kv_indptr, kv_indices, kv_last_page_len, sel_pages,
                       token_budget: int, workspace, max_pages: int, num_kv_heads: int,
                       layout: int, token_budgets=None, flags: int = 0):
    """Reference: quest/ops/csrc/approx_attn.cu:68-151.  sel_pages None = dense.
    ``flags`` = FLAG_QUEST_KERNEL: sel_pages rows hold the pages chosen
    besides the last page, which is attended as well."""
    _need(q, "q", torch.float16)
    _need(o, "o", torch.float16)
    _need(kv_data, "kv_data", torch.float16)
    _need(workspace, "workspace", torch.uint8)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                 (kv_last_page_len, "kv_last_page_len")):
        _need(t, n, torch.int32)
    if sel_pages is not None:
        _need(sel_pages, "sel_pages", torch.int32)
    if token_budgets is not None:
        _need(token_budgets, "token_budgets", torch.int32)
    _, S, Hkv, D = cache_dims(kv_data, layout)
    if Hkv != num_kv_heads:
        raise ValueError("num_kv_heads does not match kv_data")
    B, Hq, _ = q.shape
    if o.shape != q.shape:
        raise ValueError("o must have q's shape")
    _lib.call("aoakv_decode_sparse_attn", q.data_ptr(), o.data_ptr(), kv_data.data_ptr(),
              kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
              _ptr(sel_pages), 0 if sel_pages is None else sel_pages.shape[-1], token_budget,
              _ptr(token_budgets), workspace.data_ptr(), workspace.numel(), B, max_pages, Hq,
              Hkv, D, S, layout, flags, _stream())


def sparse_decode_layer(q, o, kv_data, kv_indptr, kv_indices, kv_last_page_len, metadata_data,
                        metadata_indptr, metadata_indices, v_log_norm, scores, sel_pages,
                        token_budget: int, workspace, max_pages: int, layout: int,
                        flags: int = FLAG_VALUE_AWARE | FLAG_FIXED, token_budgets=None):
    """Fused estimate + top-k + sparse decode for one layer (reference call
    sequence QuestAttention.py:135-157)."""
    _need(q, "q", torch.float16)
    _need(o, "o", torch.float16)
    _need(kv_data, "kv_data", torch.float16)
    _need(metadata_data, "metadata_data", torch.float16)
    _need(scores, "scores", torch.float32)
    _need(sel_pages, "sel_pages", torch.int32)
    _need(workspace, "workspace", torch.uint8)
    if flags & FLAG_VALUE_AWARE:
        _need(v_log_norm, "v_log_norm", torch.float16)
    if token_budgets is not None:
        _need(token_budgets, "token_budgets", torch.int32)
    _, S, Hkv, D = cache_dims(kv_data, layout)
    B, Hq, _ = q.shape
    _lib.call("aoakv_sparse_decode_layer", q.data_ptr(), o.data_ptr(), kv_data.data_ptr(),
              kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
              metadata_data.data_ptr(), metadata_indptr.data_ptr(), metadata_indices.data_ptr(),
              _ptr(v_log_norm), scores.data_ptr(), scores.shape[-1], sel_pages.data_ptr(),
              sel_pages.shape[-1], token_budget, _ptr(token_budgets), workspace.data_ptr(),
              workspace.numel(), B, max_pages, Hq, Hkv, D, S, layout, flags, _stream())


def sparse_decode_layer_noalloc(q, o, kv_data, kv_indptr, kv_indices, kv_last_page_len,
                                metadata_data, metadata_indptr, metadata_indices, v_log_norm,
                                scores, sel_pages, token_budget: int, max_pages: int, layout: int,
                                flags: int = FLAG_VALUE_AWARE | FLAG_FIXED, token_budgets=None):
    """sparse_decode_layer without a workspace (aoakv_sparse_decode_layer_noalloc):
    the library's own per-GPU scratch array, two launches, nothing allocated.
    For callers that cannot allocate; calls that overlap on one GPU race."""
    _need(q, "q", torch.float16)
    _need(o, "o", torch.float16)
    _need(kv_data, "kv_data", torch.float16)
    _need(metadata_data, "metadata_data", torch.float16)
    _need(scores, "scores", torch.float32)
    _need(sel_pages, "sel_pages", torch.int32)
    if flags & FLAG_VALUE_AWARE:
        _need(v_log_norm, "v_log_norm", torch.float16)
    if token_budgets is not None:
        _need(token_budgets, "token_budgets", torch.int32)
    _, S, Hkv, D = cache_dims(kv_data, layout)
    B, Hq, _ = q.shape
    _lib.call("aoakv_sparse_decode_layer_noalloc", q.data_ptr(), o.data_ptr(),
              kv_data.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
              kv_last_page_len.data_ptr(), metadata_data.data_ptr(), metadata_indptr.data_ptr(),
              metadata_indices.data_ptr(), _ptr(v_log_norm), scores.data_ptr(), scores.shape[-1],
              sel_pages.data_ptr(), sel_pages.shape[-1], token_budget, _ptr(token_budgets), B,
              max_pages, Hq, Hkv, D, S, layout, flags, _stream())


def noalloc_init() -> None:
    """Look up the library's scratch array on the current device
    (aoakv_noalloc_init): call before capturing sparse_decode_layer_noalloc
    into a graph."""
    _lib.call("aoakv_noalloc_init")


def noalloc_error(clear: bool = False) -> int:
    """The current device's scratch error bits (WS_ERR_*) set by
    sparse_decode_layer_noalloc calls (aoakv_noalloc_error); synchronizes the
    current stream.  ``clear`` zeroes a non-zero word afterwards."""
    bits = ctypes.c_uint32(0)
    _lib.call("aoakv_noalloc_error", ctypes.byref(bits), 1 if clear else 0, _stream())
    return int(bits.value)


def estimate_topk(q, metadata_data, metadata_indptr, metadata_indices, kv_indptr, kv_indices,
                  kv_last_page_len, v_log_norm, scores, sel_pages, token_budget: int, workspace,
                  max_pages: int, layout: int, flags: int = FLAG_VALUE_AWARE | FLAG_FIXED,
                  token_budgets=None):
    """Page scores + top-k in one launch (the first half of sparse_decode_layer)."""
    _need(q, "q", torch.float16)
    _need(metadata_data, "metadata_data", torch.float16)
    _need(scores, "scores", torch.float32)
    _need(sel_pages, "sel_pages", torch.int32)
    _need(workspace, "workspace", torch.uint8)
    if token_budgets is not None:
        _need(token_budgets, "token_budgets", torch.int32)
    _, S, Hkv, D = cache_dims(metadata_data, layout)
    B, Hq, _ = q.shape
    _lib.call("aoakv_estimate_topk", q.data_ptr(), metadata_data.data_ptr(),
              metadata_indptr.data_ptr(), metadata_indices.data_ptr(), kv_indptr.data_ptr(),
              kv_indices.data_ptr(), kv_last_page_len.data_ptr(), _ptr(v_log_norm),
              scores.data_ptr(), scores.shape[-1], sel_pages.data_ptr(), sel_pages.shape[-1],
              token_budget, _ptr(token_budgets), workspace.data_ptr(), workspace.numel(), B,
              max_pages, Hq, Hkv, D, S, layout, flags, _stream())


def prefill_with_paged_kv_cache(q, kv_data, kv_indices, num_kv_pages: int, kv_last_page_len: int,
                                layout: int, causal: bool = True, o=None):
    """Reference: quest/ops/csrc/batch_prefill.cu:27-117.  q [L, Hq, D] -> o;
    the cache holds Hkv heads, Hq a multiple of Hkv (GQA)."""
    _need(q, "q", torch.float16)
    _need(kv_data, "kv_data", torch.float16)
    _need(kv_indices, "kv_indices", torch.int32)
    _, S, H, D = cache_dims(kv_data, layout)
    if q.dim() != 3 or q.shape[2] != D:
        raise ValueError(f"q must be [L, Hq, {D}], got {tuple(q.shape)}")
    if o is None:
        o = torch.empty_like(q)
    _lib.call("aoakv_prefill_with_paged_kv_cache", q.data_ptr(), o.data_ptr(), kv_data.data_ptr(),
              kv_indices.data_ptr(), num_kv_pages, kv_last_page_len, q.shape[0], int(causal),
              q.shape[1], H, D, S, layout, _stream())
    return o
