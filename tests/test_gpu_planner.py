"""The host planner's device page tables (InferenceController.begin_forward),
written incrementally: after every step they equal what the reference's
controller uploads in full (controller.py:92-141) -- the page ids, the
append indptrs, the last page's length and the per-head page list without
the last page -- across a prefill, decode steps that open new pages, a
step with updateTensor=False, and a release (clean_states) followed by a
new sequence."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_incremental_tables_equal_full_uploads():
    from aoakv.utils import InferenceController
    c = InferenceController(1, 4, 128, 16, 8, 2000, torch.float16, DEV, shuffle_seed=3)

    def check(tag):
        torch.cuda.synchronize()
        kv, md = c.kv_cache.indicies, c.metadata_cache.indicies
        assert c.kv_indices_with_last.tolist() == kv, tag
        assert c.metadata_indices.tolist() == md, tag
        assert c.kv_indptr_for_append.tolist() == [0, len(kv)], tag
        assert c.metadata_indptr_for_append.tolist() == [0, len(md)], tag
        assert c.kv_last_page_len_t.tolist() == [c.kv_cache.last_page_len], tag
        w = c.kv_indices_without_last
        assert w is c.kv_indices_without_last, tag  # one object per step
        assert w.shape == (4, len(kv) - 1) and w.tolist() == [kv[:-1]] * 4, tag

    for i, n in enumerate([37, 1, 1, 10, 1, 1, 300] + [1] * 40):
        print(f"[planner] step {i}: {n} tokens", file=sys.stderr, flush=True)
        c.prepare_metadata(n)
        c.begin_forward(n)
        check(i)
        c.begin_forward(n, updateTensor=False)
        check(i)
    c.clean_states()
    for n in (5, 1, 1, 20):
        c.prepare_metadata(n)
        c.begin_forward(n)
        check(("after release", n))
