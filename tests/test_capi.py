"""CPU checks of the C ABI and the host logic (no GPU needed).

* libaoakv.so loads and exports every entry point include/aoakv.h declares;
* argument validation returns error codes before any launch;
* workspace sizing and the page-pool / controller bookkeeping on the host.
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aoakv.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"(?:int|size_t|char\*)\s+(aoakv_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from aoakv import _lib
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), f"{n} declared in aoakv.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_ctypes_signatures_match_header_arity():
    """Each ctypes argtypes list has as many entries as the C prototype."""
    from aoakv import _lib
    text = open(HEADER).read()
    for name, argtypes in _lib.SIGNATURES.items():
        m = re.search(r"(?:int|size_t|char\*)\s+%s\s*\(([^)]*)\)" % name, text)
        assert m, name
        params = [p for p in m.group(1).replace("\n", " ").split(",") if p.strip() not in ("", "void")]
        assert len(params) == len(argtypes), (name, len(params), len(argtypes))


def test_version():
    import aoakv
    assert "gfx950" in aoakv.version()


def test_validation_errors_without_gpu():
    from aoakv import _lib
    lib = _lib.load()
    nul = None
    # unsupported head_dim (not 64 / 128 / 256) and page sizes (not 1..32) are
    # rejected before anything touches the device
    rc = lib.aoakv_append_kv_cache_prefill(1, 1, 4, 1, 1, 1, 4, 1, 1, 1, 1, 32, 96, 16, 1, nul)
    assert rc == _lib.AOAKV_ERR_UNSUPPORTED
    assert b"head_dim" in lib.aoakv_last_error()
    for page_size in (0, 33, 64):
        rc = lib.aoakv_append_kv_cache_prefill(1, 1, 4, 1, 1, 1, 4, 1, 1, 1, 1, 32, 128,
                                               page_size, 1, nul)
        assert rc == _lib.AOAKV_ERR_UNSUPPORTED and b"page_size" in lib.aoakv_last_error()
    rc = lib.aoakv_append_kv_cache_prefill(1, 1, 4, 1, 1, 1, 4, 1, 1, 1, 1, 32, 128, 16, 7, nul)
    assert rc == _lib.AOAKV_ERR_UNSUPPORTED and b"layout" in lib.aoakv_last_error()
    # null pointers
    rc = lib.aoakv_append_kv_cache_prefill(nul, 1, 4, 1, 1, 1, 4, 1, 1, 1, 1, 32, 128, 16, 1, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"null" in lib.aoakv_last_error()
    # more new tokens than the reserved cache holds
    rc = lib.aoakv_append_kv_cache_prefill(1, 1, 40, 1, 1, 2, 4, 1, 1, 1, 1, 32, 128, 16, 1, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"new tokens" in lib.aoakv_last_error()
    # last_page_len out of range
    rc = lib.aoakv_append_kv_cache_prefill(1, 1, 4, 1, 1, 2, 17, 1, 1, 1, 1, 32, 128, 16, 1, nul)
    assert rc == _lib.AOAKV_ERR_INVALID
    # GQA group of 3 unsupported
    rc = lib.aoakv_estimate_attn_score(1, 1, 64, 1, 1, 1, 1, 1, 1, 1, 1, 64, 12, 4, 128, 16, 1,
                                       1, nul)
    assert rc == _lib.AOAKV_ERR_UNSUPPORTED and b"group" in lib.aoakv_last_error()
    # score stride smaller than max_pages
    rc = lib.aoakv_estimate_attn_score(1, 1, 10, 1, 1, 1, 1, 1, 1, 1, 1, 64, 32, 32, 128, 16, 1,
                                       1, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"score_stride" in lib.aoakv_last_error()
    # value-aware scoring without v_log_norm
    rc = lib.aoakv_estimate_attn_score(1, 1, 64, 1, 1, 1, 1, 1, 1, nul, 1, 64, 32, 32, 128, 16, 1,
                                       1, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"v_log_norm" in lib.aoakv_last_error()
    # workspace too small
    rc = lib.aoakv_decode_sparse_attn(1, 1, 1, 1, 1, 1, 1, 128, 2048, nul, 1, 16, 1, 2048, 32,
                                      32, 128, 16, 1, 0, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"workspace" in lib.aoakv_last_error()
    # the quest_kernel convention forces no page: FIXED with it is an error
    qk = _lib.FLAG_QUEST_KERNEL
    rc = lib.aoakv_estimate_attn_score(1, 1, 64, 1, 1, 1, 1, 1, 1, 1, 1, 64, 32, 32, 128, 16, 1,
                                       qk | _lib.FLAG_FIXED, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"QUEST_KERNEL" in lib.aoakv_last_error()
    rc = lib.aoakv_topk_filtering(1, 64, 1, 1, 1, 1024, nul, 1, 64, 1, 32, 16,
                                  qk | _lib.FLAG_FIXED, nul, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"QUEST_KERNEL" in lib.aoakv_last_error()
    # unknown flag bits
    rc = lib.aoakv_topk_filtering(1, 64, 1, 1, 1, 1024, nul, 1, 64, 1, 32, 16, 16, nul, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"unknown flags" in lib.aoakv_last_error()
    rc = lib.aoakv_decode_sparse_attn(1, 1, 1, 1, 1, 1, 1, 128, 2048, nul, 1, 1 << 30, 1, 2048,
                                      32, 32, 128, 16, 1, 2, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"unknown flags" in lib.aoakv_last_error()
    # quest_kernel score rows hold P - 1 entries: stride 63 for 64 pages is
    # accepted up to the next check (missing v_log_norm), stride 62 is not
    rc = lib.aoakv_estimate_attn_score(1, 1, 63, 1, 1, 1, 1, 1, 1, nul, 1, 64, 32, 32, 128, 16,
                                       1, qk | _lib.FLAG_VALUE_AWARE, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"v_log_norm" in lib.aoakv_last_error()
    rc = lib.aoakv_estimate_attn_score(1, 1, 62, 1, 1, 1, 1, 1, 1, 1, 1, 64, 32, 32, 128, 16, 1,
                                       qk | _lib.FLAG_VALUE_AWARE, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"score_stride" in lib.aoakv_last_error()
    # prefill attention reports its own status
    rc = lib.aoakv_topk_filtering(nul, 64, 1, 1, 1, 1024, nul, 1, 64, 1, 32, 16, 2, nul, nul)
    assert rc == _lib.AOAKV_ERR_INVALID


def test_workspace_size_grows_with_selection():
    from aoakv import _lib
    lib = _lib.load()
    a = lib.aoakv_decode_workspace_size(1, 32, 32, 128, 128)
    b = lib.aoakv_decode_workspace_size(1, 32, 32, 128, 2048)
    c = lib.aoakv_decode_workspace_size(16, 32, 32, 128, 128)
    assert 0 < a < b and a < c
    # per (head, chunk of 8 pages): 132 floats of partial state
    assert a >= 32 * 16 * 132 * 4


def test_kv_cache_page_bookkeeping_on_host():
    from aoakv.utils import KvCache
    c = KvCache(1, 2, 128, 100, 16, torch.float16, "cpu")
    assert c.append_seq(17) == 2 and c.seqlen == 17 and c.last_page_len == 1
    assert c.append_seq(15) == 0 and c.last_page_len == 16
    assert c.append_seq(1) == 1 and len(c.indicies) == 3
    assert c.indicies == [0, 1, 2]
    c.release()
    assert c.seqlen == 0 and c.pool.num_free_blocks == 7
    s = KvCache(1, 2, 128, 100, 16, torch.float16, "cpu", shuffle_seed=3)
    s.append_seq(100)
    assert sorted(s.indicies) == list(range(7)) and s.indicies != list(range(7))
    with pytest.raises(RuntimeError):
        s.append_seq(100)


def test_rope_validation_without_gpu():
    from aoakv import _lib
    lib = _lib.load()
    nul = None
    rc = lib.aoakv_apply_rope_in_place(1, 1, 4, 0, 32, 32, 96, 1.0, 1e4, nul)
    assert rc == _lib.AOAKV_ERR_UNSUPPORTED and b"head_dim" in lib.aoakv_last_error()
    rc = lib.aoakv_apply_rope_in_place(1, 1, 4, 0, 32, 32, 128, 0.0, 1e4, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"rope_scale" in lib.aoakv_last_error()
    rc = lib.aoakv_apply_rope_in_place(1, 1, 4, 1 << 24, 32, 32, 128, 1.0, 1e4, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"2^24" in lib.aoakv_last_error()
    rc = lib.aoakv_rope_append_kv_cache_decode(nul, 1, 1, 1, 32, 1, 1, 1, 1, 1, 1, 1, 1, 1, 32,
                                               128, 16, 1, 1.0, 1e4, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"null" in lib.aoakv_last_error()
    rc = lib.aoakv_rope_append_kv_cache_decode(1, 1, 1, 1, 32, 1, 1, 1, 1, 1, 1, 1, 1, 1, 32,
                                               128, 16, 1, 1.0, -1.0, nul)
    assert rc == _lib.AOAKV_ERR_INVALID and b"rope_theta" in lib.aoakv_last_error()


def test_workspace_wait_flag_reads_word_2():
    """ops.workspace_wait_failed reads 32-bit word 2 of a workspace (host
    tensor here: no GPU needed)."""
    import torch
    from aoakv import ops
    ws = torch.zeros(64, dtype=torch.uint8)
    assert not ops.workspace_wait_failed(ws)
    ws[8:12].view(torch.int32).fill_(1)
    assert ops.workspace_wait_failed(ws)
    ws[8:12].view(torch.int32).fill_(0)
    ws[12:16].view(torch.int32).fill_(7)   # other words do not count
    assert not ops.workspace_wait_failed(ws)


def test_noalloc_entry_point_rejects_without_gpu():
    """aoakv_sparse_decode_layer_noalloc checks its flags and its scratch
    need on the host before touching the device."""
    from aoakv import _lib
    lib = _lib.load()
    p = 1  # never dereferenced: the calls are rejected first
    # a budget of 131072 tokens selects 8192 pages per head (the selection
    # row's width): 32 heads x 8192 pages need more than the scratch array
    args = [p] * 11 + [16384, p, 8192, 131072, None, 1, 16384, 32, 8, 128, 16, 1]
    rc = lib.aoakv_sparse_decode_layer_noalloc(*args, _lib.FLAG_SINGLE_LAUNCH, None)
    assert rc == _lib.AOAKV_ERR_INVALID and b"two-launch" in lib.aoakv_last_error()
    rc = lib.aoakv_sparse_decode_layer_noalloc(*args, _lib.FLAG_VALUE_AWARE, None)
    assert rc == _lib.AOAKV_ERR_INVALID and b"scratch" in lib.aoakv_last_error()
    # the error-word reader needs somewhere to put the bits
    rc = lib.aoakv_noalloc_error(None, 1, None)
    assert rc == _lib.AOAKV_ERR_INVALID and b"error_bits" in lib.aoakv_last_error()
