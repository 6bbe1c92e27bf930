"""CPU restatement of AOA-KV's PyTorch simulation (the parity oracle).

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` use it, and only as the checker / CPU baseline.

Every function restates one function of the reference simulation with numpy,
with the fp16 rounding points made explicit:

* ``filtering/filter_util.py`` (page metadata, value statistic, page scores,
  top-k mask) and
* ``evaluation/quest_attention.py:196-382`` (the value-aware decode step) and
  ``:38-193`` (the plain Quest arm).

Arrays use the reference's simulation layout ``(b, h, tokens, d)``; fp16
tensors are ``np.float16`` arrays.  The reference runs these ops in torch on
fp16 tensors; the rounding model below was fixed by measuring torch's CPU
kernels (see the pinning tests under ``tests/``):

* fp16 elementwise op with a Python scalar or another fp16 tensor: computed in
  fp32, rounded once to fp16 (round-to-nearest-even).
* fp16 ``mean`` over pages (``filter_util.py:825,829``): fp32 accumulation in
  token order, one fp32 division by the count, one rounding to fp16.
* fp16 ``norm(p=2)`` over ``d`` (``filter_util.py:325``): fp32 sum of squares in
  index order, ``sqrtf``, one rounding to fp16.
* fp16 ``log`` (``filter_util.py:325``): fp16(RN32(ln x)), i.e. the correctly
  rounded fp32 logarithm rounded again to fp16.
* fp32 tensor divided by a Python float (``filter_util.py:329``): a true fp32
  division by ``float32(sqrt(d))``.
* fp16 ``matmul`` (``quest_attention.py:265-268,353-356``): fp32 accumulation,
  one rounding to fp16.

Parity status per function is in the module docstrings below and in the
tests; no function here is "parity unpinned" except where stated.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

FP16_MAX = np.float32(65504.0)          # torch.finfo(torch.float16).max
FP16_MIN = np.float32(-65504.0)         # torch.finfo(torch.float16).min
FP32_MAX = np.float32(np.finfo(np.float32).max)
FP32_MIN = np.float32(np.finfo(np.float32).min)


def h(x) -> np.ndarray:
    """Round an fp32/fp64 array to fp16 (round-to-nearest-even)."""
    return np.asarray(x).astype(np.float16)


def f(x) -> np.ndarray:
    """Widen to fp32 (exact).  Large fp16 arrays are widened by torch's CPU
    conversion, which gives the same values about ten times faster than
    numpy's."""
    x = np.asarray(x)
    if x.dtype == np.float16 and x.size >= (1 << 20):
        import torch
        return torch.from_numpy(np.ascontiguousarray(x)).float().numpy()
    return x.astype(np.float32)


# --------------------------------------------------------------------------
# Page metadata: Kmax / Kmin
# --------------------------------------------------------------------------

def get_max_min_filters(key_states: np.ndarray, page_size: int) -> np.ndarray:
    """Per-page elementwise key max / min.

    Follows ``filtering/filter_util.py:555-638``: pad the sequence to a page
    multiple with fp16 ``finfo.min`` (for the max) and ``finfo.max`` (for the
    min), then ``amax`` / ``amin`` over the tokens of each page.

    key_states: (b, h, L, d) fp16  ->  (b, h, P, 2, d) fp16, [...,0,:]=max,
    [...,1,:]=min.  Exact (min/max need no rounding).
    """
    b, nh, L, d = key_states.shape
    P = math.ceil(L / page_size)
    nfull = L // page_size
    # full pages reduce in place; the padded last page (fp16 finfo.min /
    # finfo.max padding never wins a max / min against a real key) separately
    # (reduced in fp32: the fp16 values widen exactly, and the extremes
    # narrow back exactly)
    full = f(key_states[:, :, :nfull * page_size]).reshape(b, nh, nfull, page_size, d)
    kmax = [h(full.max(axis=3, keepdims=True))]
    kmin = [h(full.min(axis=3, keepdims=True))]
    if nfull < P:
        pad = P * page_size - L
        last = key_states[:, :, nfull * page_size:]
        kmax.append(np.concatenate([last, np.full((b, nh, pad, d), FP16_MIN, np.float16)],
                                   axis=2).max(axis=2, keepdims=True)[:, :, :, None])
        kmin.append(np.concatenate([last, np.full((b, nh, pad, d), FP16_MAX, np.float16)],
                                   axis=2).min(axis=2, keepdims=True)[:, :, :, None])
    kmax = np.concatenate(kmax, axis=2)
    kmin = np.concatenate(kmin, axis=2)
    return np.concatenate([kmax, kmin], axis=3)


def update_filter(last_filter: np.ndarray, key_states: np.ndarray) -> np.ndarray:
    """``filter_util.py:524-553``: fold one key into a page's (max, min).

    last_filter: (b, h, 2, d) fp16, key_states: (b, h, 1, d) fp16.
    """
    mx = np.maximum(last_filter[:, :, 0:1, :], key_states)
    mn = np.minimum(last_filter[:, :, 1:2, :], key_states)
    return np.concatenate([mx, mn], axis=2)


def update_page_filters(page_filters: np.ndarray, cur_key_states: np.ndarray,
                        past_seq_len: int, chunk_size: int) -> np.ndarray:
    """``filter_util.py:758-795``: decode-time metadata append.

    A token that starts a new page (``past_seq_len % chunk_size == 0``) opens
    a page whose max and min both equal the key; otherwise the last page's
    (max, min) absorbs the key.
    """
    if past_seq_len % chunk_size != 0:
        last = update_filter(page_filters[:, :, -1], cur_key_states)
        return np.concatenate([page_filters[:, :, :-1], last[:, :, None]], axis=2)
    new = np.concatenate([cur_key_states[:, :, None], cur_key_states[:, :, None]], axis=3)
    return np.concatenate([page_filters, new], axis=2)


def repeat_filter(page_filters: np.ndarray, n_rep: int) -> np.ndarray:
    """``filter_util.py:515-522``: GQA expansion of page filters."""
    if n_rep == 1:
        return page_filters
    return np.repeat(page_filters, n_rep, axis=1)


# --------------------------------------------------------------------------
# Value statistic: page mean of V and its log-norm
# --------------------------------------------------------------------------

def _mean_tokens_fp16(x: np.ndarray, axis: int) -> np.ndarray:
    """torch CPU fp16 ``mean``: fp32 accumulation in token order, one fp32
    division, one rounding to fp16."""
    n = x.shape[axis]
    xs = np.moveaxis(f(x), axis, 0)
    acc = np.zeros(xs.shape[1:], np.float32)
    for t in range(n):          # token order, one fp32 rounding per add
        acc += xs[t]
    return h((acc / np.float32(n)).astype(np.float32))


def compute_page_v_mean(kv_seq_len: int, chunk_size: int,
                        value_states: np.ndarray) -> np.ndarray:
    """``filter_util.py:797-834``: per-page mean of V (full pages, then the
    mean of the partial last page).  (b, h, L, d) fp16 -> (b, h, P, d) fp16."""
    b, nh, L, d = value_states.shape
    nfull = kv_seq_len // chunk_size
    full = value_states[:, :, :nfull * chunk_size].reshape(b, nh, nfull, chunk_size, d)
    means = [_mean_tokens_fp16(full, axis=3)]
    if kv_seq_len % chunk_size != 0:
        left = value_states[:, :, nfull * chunk_size:kv_seq_len]
        means.append(_mean_tokens_fp16(left, axis=2)[:, :, None])
    return np.concatenate(means, axis=2)


def update_mean_filter(prev_mean: np.ndarray, new_token: np.ndarray,
                       n_prev: int) -> np.ndarray:
    """``filter_util.py:669-679``: ``(prev*n + new)/(n+1)`` with each of the
    three fp16 ops rounded to fp16 (fp16 tensor with Python ints)."""
    t = h(f(prev_mean) * np.float32(n_prev))
    t = h(f(t) + f(new_token))
    return h(f(t) / np.float32(n_prev + 1))


def update_mean_page_filters(page_filters: np.ndarray, cur_states: np.ndarray,
                             past_seq_len: int, chunk_size: int) -> np.ndarray:
    """``filter_util.py:681-716``: decode-time running page mean.

    page_filters: (b, h, P, 1, d) fp16, cur_states (b, h, 1, d) fp16.
    """
    if past_seq_len % chunk_size != 0:
        n = past_seq_len % chunk_size
        last = update_mean_filter(page_filters[:, :, -1], cur_states, n)
        return np.concatenate([page_filters[:, :, :-1], last[:, :, None]], axis=2)
    return np.concatenate([page_filters, cur_states[:, :, None]], axis=2)


def norm_fp16(x: np.ndarray) -> np.ndarray:
    """torch CPU fp16 ``norm(p=2, dim=-1)``: fp32 sum of squares in index
    order, ``sqrtf``, rounding to fp16."""
    xf = f(x)
    acc = np.zeros(xf.shape[:-1], np.float32)
    for i in range(xf.shape[-1]):
        acc = (acc + (xf[..., i] * xf[..., i]).astype(np.float32)).astype(np.float32)
    return h(np.sqrt(acc).astype(np.float32))


def log_fp16(x: np.ndarray) -> np.ndarray:
    """torch CPU fp16 ``log``: fp16(RN32(ln x)).  ln(0) = -inf."""
    with np.errstate(divide="ignore"):
        return h(np.log(np.asarray(x).astype(np.float64)).astype(np.float32))


def log_v_norm(value_states_page_mean: np.ndarray) -> np.ndarray:
    """``filter_util.py:325``: ``log(norm(V̄) + 1e-8)`` with fp16 rounding after
    each op.  The ``+1e-8`` is an fp16 op and leaves every fp16 value
    unchanged (1e-8 is below half the smallest fp16 subnormal)."""
    nrm = norm_fp16(value_states_page_mean)
    nrm = h(f(nrm) + np.float32(1e-8))
    return log_fp16(nrm)


# --------------------------------------------------------------------------
# Page scores and selection
# --------------------------------------------------------------------------

def page_bound(query_states: np.ndarray, page_filters: np.ndarray,
               num_key_value_groups: int = 1) -> np.ndarray:
    """Per-page Quest bound ``sum_d |q_d| * max(s_d Kmax_d, s_d Kmin_d)``
    (``filter_util.py:986-1016``) computed once per page in fp32.

    The reference computes the same value for every token of the page (each
    page's row is repeated ``chunk_size`` times before the fp32 matmul) and
    then takes the page ``amax`` (``:314-321``), so one value per page is the
    same quantity.  Products are exact in fp32; the summation order of the
    128-term dot is the BLAS's and is not reproducible bit for bit.
    q: (b, nh, 1, d) fp16, page_filters (b, nkvh, P, 2, d) fp16 -> (b, nh, P) fp32.
    """
    sign = np.where(query_states > 0, np.float16(1), np.float16(-1))      # :984
    pos_q = f(query_states * sign)                                         # :985
    pf = repeat_filter(page_filters, num_key_value_groups)
    mk = (pf * sign[:, :, :, None, :]).max(axis=3)                         # :987-996
    return np.matmul(pos_q, np.swapaxes(f(mk), 2, 3))[:, :, 0, :].astype(np.float32)


def compute_attn_weights_for_selection(query_states, page_filters, num_key_value_groups,
                                       chunk_size, seq_length, num_pages):
    """``filter_util.py:968-1018``: token-level Quest bound, (b, nh, 1, L) fp32.
    Every token of page p carries page p's bound."""
    pb = page_bound(query_states, page_filters, num_key_value_groups)
    tok = np.repeat(pb, chunk_size, axis=-1)[:, :, :seq_length]
    return tok[:, :, None, :]


def _pad_and_page_max(attn_weights: np.ndarray, chunk_size: int) -> np.ndarray:
    """``filter_util.py:289-321``: pad with fp32 min to a page multiple and take
    the per-page max.  (b, nh, q, L) -> (b, nh, q, P)."""
    b, nh, q, L = attn_weights.shape
    pad = chunk_size - ((L - 1) % chunk_size + 1)
    a = np.concatenate([attn_weights, np.full((b, nh, q, pad), FP32_MIN, np.float32)], axis=-1)
    return a.reshape(b, nh, q, -1, chunk_size).max(axis=-1)


def num_selected_pages(token_budget: int, chunk_size: int, num_pages: int) -> int:
    """``filter_util.py:373``: k = min(max(3, budget // page), P)."""
    return min(max(3, token_budget // chunk_size), num_pages)


def value_aware_page_scores(chunk_max: np.ndarray, log_vn: np.ndarray,
                            num_key_value_groups: int, head_dim: int) -> np.ndarray:
    """``filter_util.py:329,361,367``: ``2*(x/sqrt(d))`` (fp32, true division),
    logsumexp over the query heads of a KV group when GQA, then
    ``+ 2*log_v_norm`` (fp16 doubling, fp32 add).

    chunk_max: (b, nh, q, P) fp32 page bound; log_vn: (b, nkvh, P) fp16.
    Returns (b, nkvh, q, P) fp32.
    """
    b, nh, q, P = chunk_max.shape
    nkvh = nh // num_key_value_groups
    x = chunk_max.reshape(b, nkvh, num_key_value_groups, q, P)
    x = (np.float32(2) * (x / np.float32(math.sqrt(head_dim))).astype(np.float32)).astype(np.float32)
    if num_key_value_groups > 1:
        m = x.max(axis=2, keepdims=True)
        x = (m + np.log(np.exp(x - m).sum(axis=2, keepdims=True))).astype(np.float32)
    two_lvn = h(f(log_vn) * np.float32(2))                                # fp16 2*x (exact)
    x = (x + f(two_lvn)[:, :, None, None, :]).astype(np.float32)
    return x[:, :, 0]


def topk_pages(scores: np.ndarray, k: int, fixed_selection: bool) -> np.ndarray:
    """``filter_util.py:375-380``: force pages 0 and P-1 to fp32 max when
    ``fixed``, then top-k.  Ties are broken towards the lower page index
    (torch leaves tie order unspecified).  Returns indices sorted ascending.
    scores: (..., P) fp32 -> (..., k) int64."""
    s = scores.copy()
    if fixed_selection:
        s[..., 0] = FP32_MAX
        s[..., -1] = FP32_MAX
    order = np.argsort(-s.astype(np.float64), axis=-1, kind="stable")[..., :k]
    return np.sort(order, axis=-1)


def quest_kernel_pages(scores: np.ndarray, page_budget: int) -> np.ndarray:
    """The reference KERNEL's selection convention (``controller.py:113-124``,
    ``quest/utils/__init__.py:196-246``, ``decode_attn.cuh:297-306``; the
    reference's own test of it is ``quest/tests/test_approx_attention.py:38-93``):
    the last page is not scored and is always attended; with
    ``k = min(max(1, page_budget), P)`` the k - 1 best of the other pages are
    selected (ties towards the lower page index) and the last page added.

    scores (..., P) fp32, entry P-1 ignored -> (..., k) int64, ascending."""
    P = scores.shape[-1]
    k = min(max(1, page_budget), P)
    head = scores[..., :P - 1].astype(np.float64)
    order = np.argsort(-head, axis=-1, kind="stable")[..., :k - 1]
    last = np.full(order.shape[:-1] + (1,), P - 1, dtype=order.dtype)
    return np.sort(np.concatenate([order, last], axis=-1), axis=-1)


def local_heavy_hitter_mask_value_aware_group_consistent_sum(
        attn_weights, token_budget, chunk_size, value_states_page_mean,
        num_key_value_groups, head_dim, fixed_selection=False,
        return_pages: bool = False):
    """``filter_util.py:269-407``: AOA-KV value-aware page selection.

    attn_weights (b, nh, q, L) fp32; value_states_page_mean (b, nkvh, P, d)
    fp16.  Returns the token mask (b, nh, q, L) bool; with ``return_pages``
    also the page scores (b, nkvh, q, P) fp32 (before fixed forcing) and the
    selected pages (b, nkvh, q, k) int64 (ascending).
    """
    b, nh, q, L = attn_weights.shape
    chunk_max = _pad_and_page_max(attn_weights, chunk_size)
    lvn = log_v_norm(value_states_page_mean)
    scores = value_aware_page_scores(chunk_max, lvn, num_key_value_groups, head_dim)
    P = scores.shape[-1]
    k = num_selected_pages(token_budget, chunk_size, P)
    pages = topk_pages(scores, k, fixed_selection)
    mask = pages_to_token_mask(pages, chunk_size, L)
    mask = np.repeat(mask, num_key_value_groups, axis=1)
    if return_pages:
        return mask, scores, pages
    return mask


def local_heavy_hitter_mask_group_consistent_sum(
        attn_weights, token_budget, chunk_size, num_key_value_groups,
        fixed_selection=False, return_pages: bool = False):
    """``filter_util.py:165-266``: plain Quest selection (page max of the
    bound, SUM over a GQA group, fixed forcing, top-k)."""
    b, nh, q, L = attn_weights.shape
    chunk_max = _pad_and_page_max(attn_weights, chunk_size)
    nkvh = nh // num_key_value_groups
    s = chunk_max.reshape(b, nkvh, num_key_value_groups, q, -1)
    if num_key_value_groups > 1:
        s = s.sum(axis=2, keepdims=True, dtype=np.float32)
    s = s[:, :, 0]
    P = s.shape[-1]
    k = num_selected_pages(token_budget, chunk_size, P)
    pages = topk_pages(s, k, fixed_selection)
    mask = np.repeat(pages_to_token_mask(pages, chunk_size, L), num_key_value_groups, axis=1)
    if return_pages:
        return mask, s, pages
    return mask


def pages_to_token_mask(pages: np.ndarray, chunk_size: int, L: int) -> np.ndarray:
    """``filter_util.py:384-401``: expand selected pages to a token mask and
    drop the padding.  pages (b, nkvh, q, k) -> (b, nkvh, q, L) bool."""
    b, nkvh, q, k = pages.shape
    P = math.ceil(L / chunk_size)
    pm = np.zeros((b, nkvh, q, P), bool)
    np.put_along_axis(pm, pages, True, axis=-1)
    return np.repeat(pm, chunk_size, axis=-1)[..., :L]


# --------------------------------------------------------------------------
# Decode attention (quest_attention.py value-aware arm)
# --------------------------------------------------------------------------

def masked_decode_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray,
                            mask: Optional[np.ndarray]) -> np.ndarray:
    """``evaluation/quest_attention.py:265-268,347-356``.

    logits = fp16(q @ K^T) then fp16(logits / sqrt(d)); non-selected tokens
    set to fp16 min; softmax in fp32, probabilities rounded to fp16; output
    fp16(p @ V).  q (b, nh, 1, d), K/V (b, nh, L, d) fp16 (already repeated
    for GQA), mask (b, nh, 1, L) bool or None.  Returns (b, nh, 1, d) fp16.
    """
    d = q.shape[-1]
    w = h(np.matmul(f(q), np.swapaxes(f(K), 2, 3)))
    w = h(f(w) / np.float32(math.sqrt(d)))
    w = f(w)
    if mask is not None:
        w = np.where(mask, w, FP16_MIN)
    m = w.max(axis=-1, keepdims=True)
    e = np.exp((w - m).astype(np.float32)).astype(np.float32)
    p = h(e / e.sum(axis=-1, keepdims=True, dtype=np.float32))
    return h(np.matmul(f(p), f(V)))


def sparse_decode_attention(q: np.ndarray, K: np.ndarray, V: np.ndarray, pages: np.ndarray,
                            chunk_size: int, L: int) -> np.ndarray:
    """``masked_decode_attention`` with the page mask ``pages`` (b, h, 1, k),
    evaluated on the selected tokens only.

    The masked form fills the logits of unselected tokens with fp16
    ``finfo.min``; with a selected logit m >= -65400 their fp32 probability
    exp(-65504 - m) is exactly 0, so every rounded intermediate of the
    selected tokens is unchanged and the result is the same up to the
    summation order of the final fp32 product (tests/test_oracle.py pins it
    against ``masked_decode_attention``).  q (b, h, 1, d), K/V (b, h, L, d),
    pages per head (logical page ids); returns (b, h, 1, d) fp16."""
    b, nh, _, d = q.shape
    out = np.empty((b, nh, 1, d), np.float16)
    for bi in range(b):
        for hi in range(nh):
            pg = np.unique(np.asarray(pages[bi, hi]).ravel())
            tok = (pg[:, None] * chunk_size + np.arange(chunk_size)[None, :]).ravel()
            tok = tok[tok < L]
            w = h(np.matmul(f(q[bi, hi]), f(K[bi, hi, tok]).T))
            w = f(h(f(w) / np.float32(math.sqrt(d))))
            m = w.max(axis=-1, keepdims=True)
            assert float(m.min()) >= -65400.0, "masked tokens would not vanish"
            e = np.exp((w - m).astype(np.float32)).astype(np.float32)
            p = h(e / e.sum(axis=-1, keepdims=True, dtype=np.float32))
            out[bi, hi] = h(np.matmul(f(p), f(V[bi, hi, tok])))
    return out


class SimLayerState:
    """Per-layer cache of the value-aware simulation for one sequence
    (``quest_attention.py:237-245,366-373``): K, V, V̄ per page, (Kmax, Kmin)
    per page and the sequence length.  Arrays are (1, h, ., d) fp16."""

    def __init__(self, K: np.ndarray, V: np.ndarray, chunk_size: int = 16):
        self.chunk_size = chunk_size
        self.K = K
        self.V = V
        self.kv_len = K.shape[2]
        self.page_filters = get_max_min_filters(K, chunk_size)           # :238
        self.v_mean = compute_page_v_mean(self.kv_len, chunk_size, V)    # :239

    def append(self, k_new: np.ndarray, v_new: np.ndarray) -> None:
        """Decode-time metadata and cache update (``quest_attention.py:254-263,
        287-293``)."""
        past = self.kv_len
        self.v_mean = update_mean_page_filters(self.v_mean[:, :, :, None], v_new, past,
                                               self.chunk_size)[:, :, :, 0]
        self.page_filters = update_page_filters(self.page_filters, k_new, past, self.chunk_size)
        self.K = np.concatenate([self.K, k_new], axis=2)
        self.V = np.concatenate([self.V, v_new], axis=2)
        self.kv_len += 1


def select_pages(state: SimLayerState, q: np.ndarray, token_budget: int,
                 fixed: bool = True, value_aware: bool = True,
                 num_key_value_groups: int = 1, semantics: str = "sim"):
    """Scoring and selection of one decode step (``quest_attention.py:296-332``).

    ``semantics="quest_kernel"`` keeps the same page scores but selects by
    the reference kernel's convention (``quest_kernel_pages`` with a page
    budget of ``token_budget // page_size``; ``fixed`` does not apply).
    Returns (scores (1, nkvh, 1, P) fp32, pages (1, nkvh, 1, k) int64)."""
    if semantics not in ("sim", "quest_kernel"):
        raise ValueError(f"unknown semantics {semantics!r}")
    L = state.kv_len
    P = math.ceil(L / state.chunk_size)
    w = compute_attn_weights_for_selection(q, state.page_filters, num_key_value_groups,
                                           state.chunk_size, L, P)
    tb = min(L, token_budget)                                              # :326
    if value_aware:
        _, scores, pages = local_heavy_hitter_mask_value_aware_group_consistent_sum(
            w, tb, state.chunk_size, state.v_mean, num_key_value_groups,
            q.shape[-1], fixed, return_pages=True)
    else:
        _, scores, pages = local_heavy_hitter_mask_group_consistent_sum(
            w, tb, state.chunk_size, num_key_value_groups, fixed, return_pages=True)
    if semantics == "quest_kernel":
        pages = quest_kernel_pages(scores, token_budget // state.chunk_size)
    return scores, pages


def decode_step(state: SimLayerState, q: np.ndarray, k_new: np.ndarray, v_new: np.ndarray,
                token_budget: int, fixed: bool = True, value_aware: bool = True,
                num_key_value_groups: int = 1, semantics: str = "sim"):
    """One value-aware decode step of one layer (``quest_attention.py:249-356``):
    metadata append, page scores, top-k mask, masked attention.
    Returns (o (1, nh, 1, d) fp16, scores, pages)."""
    state.append(k_new, v_new)
    scores, pages = select_pages(state, q, token_budget, fixed, value_aware,
                                 num_key_value_groups, semantics)
    mask = pages_to_token_mask(pages, state.chunk_size, state.kv_len)
    mask = np.repeat(mask, num_key_value_groups, axis=1)
    K = np.repeat(state.K, num_key_value_groups, axis=1)
    V = np.repeat(state.V, num_key_value_groups, axis=1)
    o = masked_decode_attention(q, K, V, mask)
    return o, scores, pages


# --------------------------------------------------------------------------
# Rotary position embedding (apply_rope_in_place)
# --------------------------------------------------------------------------

def apply_rope(x: np.ndarray, positions: np.ndarray, rope_scale: float = 1.0,
               rope_theta: float = 1e4) -> np.ndarray:
    """Llama RoPE, rotate-half form, as the reference kernel computes it
    (``QKApplyRotaryInPlaceKernel``, decode_page.cuh:785-840: frequency
    ``rcp_scale * rcp_theta^(2i/D)`` in fp32, angle = fp32(position) * freq,
    fp32 arithmetic, one rounding to fp16) and as its test checks it
    (quest/tests/test_rope.py:17-30, HF ``apply_rotary_pos_emb``).  The fp32
    frequency is the correctly rounded one.

    x (N, H, D) fp16, positions (N,) ints.  The angle is formed in fp32 as
    the kernel does; cos / sin and the rotation are evaluated in float64, so
    the result is the exactly rounded value the fp32 kernel approximates.
    Returns float64 (N, H, D) (round with ``h()`` for the fp16 result)."""
    N, H, D = x.shape
    half = D // 2
    i = np.arange(D) % half
    rcp_scale = np.float64(np.float32(1.0) / np.float32(rope_scale))
    rcp_theta = np.float64(np.float32(1.0) / np.float32(rope_theta))
    # the correctly rounded fp32 frequency (fp64 evaluation, one rounding)
    freq = (rcp_scale * np.power(rcp_theta, (2 * i) / D)).astype(np.float32)
    ang = (np.asarray(positions, np.float32)[:, None] * freq[None, :]).astype(np.float64)
    c, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    xf = x.astype(np.float64)
    rot = np.concatenate([-xf[..., half:], xf[..., :half]], axis=-1)   # rotate_half
    return xf * c + rot * sn


# --------------------------------------------------------------------------
# RMSNorm (the model's norm, outside the decode layer)
# --------------------------------------------------------------------------

def rms_norm_forward(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The reference's rms_norm_forward kernel (quest/ops/csrc/rms_norm.cu:
    76-159, ``rmsnorm_twoPassAlgo_e8``): per row, s = sum of the fp32 squares
    (fp32), r = 1/sqrt(s / n + eps), out = fp16((x * r) * w) with each
    product in fp32.  The kernel sums in a thread/warp tree; here the row is
    summed in float64 and rounded to fp32 once (the two differ by a few fp32
    ulps of s, far below one fp16 ulp of the output), and r is the correctly
    rounded fp32 reciprocal square root.

    x (..., n) fp16, w (n,) fp16; returns fp16 of x's shape."""
    xf = x.astype(np.float32)
    s = (xf.astype(np.float64) ** 2).sum(axis=-1, keepdims=True).astype(np.float32)
    u = (s / np.float32(x.shape[-1])).astype(np.float32) + np.float32(eps)   # fp32 ops
    r = (1.0 / np.sqrt(u.astype(np.float64))).astype(np.float32)
    return ((xf * r).astype(np.float32) * w.astype(np.float32)).astype(np.float16)


# --------------------------------------------------------------------------
# Dense causal prefill (textbook; quest/tests/test_prefill_attention.py:17-44,
# kernels/src/include/cpu_reference.h:56-159)
# --------------------------------------------------------------------------

def causal_prefill_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                        rows: Optional[np.ndarray] = None) -> np.ndarray:
    """Causal softmax(q k^T / sqrt(d)) v in fp64 for the given query rows.

    q (Lq, h, d), k/v (Lk, h, d) NHD fp16 with the queries aligned to the end
    of the keys (query i sees keys ``<= Lk - Lq + i``).  Returns
    (len(rows), h, d) fp32.
    """
    Lq, nh, d = q.shape
    Lk = k.shape[0]
    if rows is None:
        rows = np.arange(Lq)
    out = np.empty((len(rows), nh, d), np.float32)
    kf = k.astype(np.float64)
    vf = v.astype(np.float64)
    scale = 1.0 / math.sqrt(d)
    for j, i in enumerate(rows):
        last = Lk - Lq + int(i)
        s = np.einsum("hd,lhd->hl", q[i].astype(np.float64), kf[:last + 1]) * scale
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[j] = np.einsum("hl,lhd->hd", p, vf[:last + 1]).astype(np.float32)
    return out


def selection_matches(sel: np.ndarray, sel_ref: np.ndarray, scores: np.ndarray,
                      fixed: bool = False, rel_tol: float = 1e-3,
                      forced: Optional[set] = None) -> Tuple[bool, str]:
    """Tie-aware comparison of a selected page set with the reference's, for
    one head.

    They agree when equal, or when every page in their symmetric difference
    has a reference score within ``rel_tol`` (relative) of the boundary score
    (the smallest score the reference selected, forced pages excluded): the
    sets then differ only among near-ties at the selection boundary.
    ``scores`` are the reference page scores before fixed forcing.
    ``forced`` names the always-selected pages explicitly (default: pages 0
    and P-1 when ``fixed``; ``{P-1}`` for the quest_kernel convention)."""
    a = set(int(x) for x in np.ravel(sel))
    b = set(int(x) for x in np.ravel(sel_ref))
    if len(a) != len(b):
        return False, f"size {len(a)} != {len(b)}"
    if a == b:
        return True, "exact"
    P = scores.shape[-1]
    if forced is None:
        forced = {0, P - 1} if fixed else set()
    if not forced <= a:
        return False, f"forced pages {sorted(forced - a)} missing"
    free = [float(scores[i]) for i in b - forced]
    boundary = min(free)
    for i in a ^ b:
        s = float(scores[i])
        if not abs(s - boundary) <= rel_tol * max(abs(boundary), 1e-30):
            return False, f"page {i} score {s} not within {rel_tol} of boundary {boundary}"
    return True, f"near-ties: {sorted(a ^ b)}"
