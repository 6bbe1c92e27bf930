"""InferenceController: host planner of the paged cache for one sequence.

Mirrors the reference's InferenceController (kernels/aoa_kv/quest/utils/
controller.py:7-164): the same attributes and call order
(prepare_metadata -> begin_forward -> ops -> end_forward), so a driver can
switch trees.  Differences, by design:

* selection follows the simulation (every page scored, fixed forcing of the
  first and last page, k = min(max(3, min(L, budget)/page), P));
* the decode workspace is allocated once, not per begin_forward, and no op
  synchronises with the host;
* the device page tables live in buffers allocated once: begin_forward
  writes only what changed since the last call (the new page ids, the page
  counts, the last page's length) with fills that carry the value as a
  kernel argument, so a decode step makes no host-to-device copy and no
  allocation; ``kv_indices_without_last`` is a broadcast view, not the
  reference's per-head copy (controller.py:130-131);
* scores are fp32 and the per-page value statistic is written for every
  page, with the page mean of V kept in ``v_mean`` for the running mean.

``semantics="quest_kernel"`` switches to the reference kernel's convention
instead (controller.py:113-124, quest/utils/__init__.py:196-246): the last
page is never scored and always attended, ``inference_page_budget - 1``
pages are selected from the others, and ``topk_dindices_buffer`` is the
reference's ``[H, inference_page_budget - 1]`` top-k output.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import ops
from .kv_cache import KvCache
from .utils import TensorLayout


class InferenceController:
    def __init__(self, num_layers, num_heads, head_dim, page_size, page_budget, max_seq_len,
                 dtype, device, layout: int = TensorLayout.HND,
                 num_kv_heads: Optional[int] = None, fixed: bool = True,
                 value_aware: bool = True, shuffle_seed: Optional[int] = None,
                 semantics: str = "sim"):
        if dtype != torch.float16:
            raise TypeError("only float16 caches are supported")
        if semantics not in ("sim", "quest_kernel"):
            raise ValueError(f"semantics must be 'sim' or 'quest_kernel', got {semantics!r}")
        self.semantics = semantics
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads or num_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.layout = layout
        self.device = torch.device(device)
        self.dtype = dtype
        self.fixed = fixed
        self.value_aware = value_aware

        max_kv_pages = (max_seq_len + page_size - 1) // page_size
        self.max_kv_pages = max_kv_pages
        self.kv_cache = KvCache(num_layers, self.num_kv_heads, head_dim, max_seq_len, page_size,
                                dtype, device, layout, shuffle_seed)
        self.metadata_cache = KvCache(num_layers, self.num_kv_heads, head_dim, max_kv_pages,
                                      page_size, dtype, device, layout,
                                      None if shuffle_seed is None else shuffle_seed + 1)
        # log-norm of the page mean of V per (layer, physical page, kv head)
        # (reference controller.py:43-47) and the page means themselves
        self.v_log_norm = torch.zeros((num_layers, max_kv_pages, self.num_kv_heads), dtype=dtype,
                                      device=device)
        self.v_mean = torch.zeros((num_layers, max_kv_pages, self.num_kv_heads, head_dim),
                                  dtype=dtype, device=device)

        self._page_budget = page_budget
        self.inference_page_budget = None

        self.kv_indices_with_last = None
        self.metadata_indices = None
        self.kv_last_page_idx = None
        self.metadata_last_page_idx = None
        self.kv_indptr_for_append = None
        self.metadata_indptr_for_append = None
        self.kv_last_page_len_t = None
        self._kv_without_last = None

        # device page tables, written incrementally by begin_forward: page
        # ids [0, n) of kv / metadata are on the device (n_up), as are the
        # page counts and last page length last written
        max_md_pages = (max_kv_pages + page_size - 1) // page_size
        i32 = dict(dtype=torch.int32, device=device)
        self._kv_ids = torch.zeros(max_kv_pages, **i32)
        self._md_ids = torch.zeros(max_md_pages, **i32)
        self._kv_indptr = torch.zeros(2, **i32)
        self._md_indptr = torch.zeros(2, **i32)
        self._lpl = torch.zeros(1, **i32)
        self._up = {"kv": 0, "md": 0, "P": 0, "Pm": 0, "lpl": 0}

        # fixed-size decode buffers (one layer at a time)
        self.scores = torch.empty((1, self.num_kv_heads, max_kv_pages), dtype=torch.float32,
                                  device=device)
        self.topk_dindices_buffer = None
        self._sel = torch.empty((1, self.num_kv_heads, max_kv_pages), dtype=torch.int32,
                                device=device)
        self.workspace = ops.decode_workspace(1, num_heads, self.num_kv_heads, max_kv_pages,
                                              device, max_pages=max_kv_pages,
                                              head_dim=head_dim)
        # check the workspace error word after every fused decode layer call
        # (synchronizes: for debugging; check_errors() once per token is cheap)
        self.debug_checks = False
        # decode calls size their grids for the cache's capacity instead of
        # the current page count (a graph replayed over many steps; the
        # kernels read the page count from the device tables either way)
        self.static_page_bound = False

    # ------------------------------------------------------------ budget
    @property
    def token_budget(self) -> int:
        return self._page_budget * self.page_size

    def set_page_budget(self, page_budget: int):
        self._page_budget = page_budget

    @property
    def quest_kernel(self) -> bool:
        return self.semantics == "quest_kernel"

    @property
    def flags(self) -> int:
        """Selection flags of the scoring / top-k / decode calls (``fixed``
        applies to the simulation's convention only)."""
        if self.quest_kernel:
            return ops.FLAG_QUEST_KERNEL | (ops.FLAG_VALUE_AWARE if self.value_aware else 0)
        return ((ops.FLAG_VALUE_AWARE if self.value_aware else 0) |
                (ops.FLAG_FIXED if self.fixed else 0))

    # ------------------------------------------------------------ planning
    def prepare_metadata(self, seq_len: int):
        """Reserve cache slots for seq_len new tokens (controller.py:84-88)."""
        new_pages = self.kv_cache.append_seq(seq_len)
        self.metadata_cache.append_seq(new_pages)

    @staticmethod
    def _sync_ids(buf: torch.Tensor, ids, done: int) -> int:
        """Writes ids[done:] into buf (ids [0, done) are there already);
        returns len(ids).  One new page (a decode step every page_size
        tokens) is a fill; more (a prefill) one copy."""
        n = len(ids)
        if n - done == 1:
            buf[n - 1].fill_(ids[n - 1])
        elif n > done:
            buf[done:n].copy_(torch.tensor(ids[done:], dtype=torch.int32))
        return n

    def begin_forward(self, seq_len: int, updateTensor: bool = True):
        """Update the device page tables for the coming ops (controller.py:92-141):
        only what changed since the last call is written."""
        kv = self.kv_cache.indicies
        md = self.metadata_cache.indicies
        if updateTensor:
            up = self._up
            P, Pm, lpl = len(kv), len(md), self.kv_cache.last_page_len
            if P < up["kv"] or Pm < up["md"]:  # pages were released
                up.update(kv=0, md=0)
            up["kv"] = self._sync_ids(self._kv_ids, kv, up["kv"])
            up["md"] = self._sync_ids(self._md_ids, md, up["md"])
            for key, val, t in (("P", P, self._kv_indptr[1]), ("Pm", Pm, self._md_indptr[1]),
                                ("lpl", lpl, self._lpl[0])):
                if up[key] != val:
                    t.fill_(val)
                    up[key] = val
            self.kv_indices_with_last = self._kv_ids[:P]
            self.metadata_indices = self._md_ids[:Pm]
            self.kv_indptr_for_append = self._kv_indptr
            self.metadata_indptr_for_append = self._md_indptr
            self.kv_last_page_len_t = self._lpl
            self.kv_last_page_idx = kv[-1]
            self.metadata_last_page_idx = md[-1]
            self._kv_without_last = None
        if seq_len == 1:
            P = len(kv)
            self.inference_page_budget = min(self._page_budget, P)
            k = self.num_selected_pages()
            # quest_kernel: the rows hold the pages chosen besides the last
            self.topk_dindices_buffer = self._sel[:, :, :k - 1 if self.quest_kernel else k]

    def end_forward(self):
        pass

    @property
    def kv_indices_without_last(self) -> Optional[torch.Tensor]:
        """[num_heads, P - 1]: every page but the last, per head (the dense
        decode's page list, controller.py:130-131); a broadcast view of the
        page table, the same object until the next begin_forward."""
        if self.kv_indices_with_last is None:
            return None
        if self._kv_without_last is None:
            P = self.kv_indices_with_last.numel()
            self._kv_without_last = self._kv_ids[:max(P - 1, 0)].unsqueeze(0).expand(
                self.num_heads, max(P - 1, 0))
        return self._kv_without_last

    @property
    def decode_max_pages(self) -> int:
        """The page-count bound the decode calls pass by value: the current
        page count, or the capacity with ``static_page_bound``."""
        return self.max_kv_pages if self.static_page_bound else len(self.kv_cache.indicies)

    def need_estimate(self) -> bool:
        """True when the sequence has more pages than the page budget."""
        if self.inference_page_budget is None:
            return False
        return len(self.kv_cache.indicies) > self.inference_page_budget

    def num_selected_pages(self) -> int:
        """Pages attended per kv head: the simulation's k (filter_util.py:373)
        or, with the quest_kernel convention, min(page_budget, P) including
        the last page (controller.py:118)."""
        L = self.kv_cache.seqlen
        P = len(self.kv_cache.indicies)
        if self.quest_kernel:
            return min(max(1, self._page_budget), P)
        return min(max(3, min(L, self.token_budget) // self.page_size), P)

    def check_errors(self):
        """Raise if a decode call on this controller's workspace flagged an
        error: a one-launch layer's wait gave up (the workspace is
        re-initialized, so the next call runs normally again) or a page
        table exceeded what a call was sized for.  Reads the workspace error
        word back, so it synchronizes: call it once per generated token, not
        per layer."""
        err = ops.workspace_error(self.workspace)
        if err:
            ops.workspace_init(self.workspace)
            what = []
            if err & ops.WS_ERR_WAIT:
                what.append("a one-launch decode layer's wait gave up (its outputs are invalid)")
            if err & ops.WS_ERR_TRUNCATED:
                what.append("a page table held more pages than the call was sized for")
            raise RuntimeError("aoakv decode workspace error: " + "; ".join(what))

    def clean_states(self):
        self.kv_cache.release()
        self.metadata_cache.release()
        self._up.update(kv=0, md=0)

    def v_log_norm_layer(self, layer_idx: int):
        return self.v_log_norm[layer_idx]

    def v_mean_layer(self, layer_idx: int):
        return self.v_mean[layer_idx]
