"""Write the golden fixtures for the oracle from the reference simulation.

Run in the build container only (``/root/reference`` must exist):

    python tests/golden/make_golden.py

It imports ``filtering/filter_util.py`` from the reference (plain torch code,
CPU) and records, for seeded inputs, the outputs of the functions whose fp16
rounding or tie behaviour no closed form fixes:

* ``get_max_min_filters`` / ``compute_page_v_mean`` for ragged lengths,
* a 40-step decode trace through ``update_page_filters`` /
  ``update_mean_page_filters`` crossing page boundaries,
* ``compute_attn_weights_for_selection`` +
  ``local_heavy_hitter_mask_value_aware_group_consistent_sum`` (and the plain
  Quest variant) at the config-1 shape, fixed in {True, False},
* a tie case with duplicated pages,
* GQA (2 query heads per KV head) selection.

``evaluation/quest_attention.py`` cannot be imported here (its module imports
``Qwen2FlashAttention2``, absent from this transformers), so the small
decode-attention outputs are produced by torch ops following its lines
265-268 and 347-356 (fp16 matmul, fp16 scale, fp16-min masking, fp32
softmax, fp16 probabilities, fp16 PV).

Inputs are drawn with numpy's PCG64 (``np.random.default_rng(seed)``) so the
tests can regenerate them; large inputs are not stored, only seeds, outputs
and sha256 digests of large outputs.
"""
import hashlib
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("AOAKV_REFERENCE", "/root/reference")
sys.path.insert(0, REF)
from filtering import filter_util as fu  # noqa: E402


def randn16(seed, shape, scale=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def metadata_cases(out):
    """Prefill metadata for ragged lengths (b=1, h=4, d=128)."""
    for L in (17, 31, 256, 4103):
        nh = 4 if L < 4096 else 2
        K = randn16(100 + L, (1, nh, L, 128))
        V = randn16(200 + L, (1, nh, L, 128))
        pf = fu.get_max_min_filters(t(K), 16).numpy()
        vm = fu.compute_page_v_mean(L, 16, t(V)).numpy()
        out[f"meta_L{L}_filters"] = pf
        out[f"meta_L{L}_vmean"] = vm
        lvn = torch.log(t(vm).norm(p=2, dim=-1) + 1e-8).numpy()
        out[f"meta_L{L}_lvn"] = lvn


def decode_trace(out):
    """Prefill 21 tokens then 40 decode appends (crosses pages 2->4)."""
    nh, d, L0, steps = 4, 128, 21, 40
    K = randn16(300, (1, nh, L0, d))
    V = randn16(301, (1, nh, L0, d))
    kn = randn16(302, (steps, 1, nh, 1, d))
    vn = randn16(303, (steps, 1, nh, 1, d))
    pf = fu.get_max_min_filters(t(K), 16)
    vm = fu.compute_page_v_mean(L0, 16, t(V))
    L = L0
    pfs, vms = [], []
    for s in range(steps):
        vm = fu.update_mean_page_filters(vm.unsqueeze(-2), t(vn[s]), L, 16).squeeze(-2)
        pf = fu.update_page_filters(pf, t(kn[s]), L, 16)
        L += 1
        pfs.append(pf.numpy().copy())
        vms.append(vm.numpy().copy())
    out["trace_final_filters"] = pfs[-1]
    out["trace_final_vmean"] = vms[-1]
    out["trace_vmean_last_page_per_step"] = np.stack([v[:, :, -1] for v in vms])
    out["trace_filters_last_page_per_step"] = np.stack([p[:, :, -1] for p in pfs])


def selection_case(out, tag, seed, nh, nkvh, L, budget, fixed, value_aware,
                   outlier=False, dup_pages=None):
    d = 128
    groups = nh // nkvh
    K = randn16(seed, (1, nkvh, L, d))
    V = randn16(seed + 1, (1, nkvh, L, d))
    q = randn16(seed + 2, (1, nh, 1, d))
    if outlier:
        ch = np.random.default_rng(seed + 3).permutation(d)[:4]
        K[..., ch] = (K[..., ch].astype(np.float32) * 8).astype(np.float16)
    if dup_pages is not None:
        src, dsts = dup_pages
        for dst in dsts:
            K[:, :, dst * 16:(dst + 1) * 16] = K[:, :, src * 16:(src + 1) * 16]
            V[:, :, dst * 16:(dst + 1) * 16] = V[:, :, src * 16:(src + 1) * 16]
    P = math.ceil(L / 16)
    pf = fu.get_max_min_filters(t(K), 16)
    vm = fu.compute_page_v_mean(L, 16, t(V))
    w = fu.compute_attn_weights_for_selection(t(q), pf, groups, 16, L, P)
    tb = min(L, budget)
    if value_aware:
        mask = fu.local_heavy_hitter_mask_value_aware_group_consistent_sum(
            w, tb, 16, vm, groups, d, fixed)
    else:
        mask, _ = fu.local_heavy_hitter_mask_group_consistent_sum(w, tb, 16, groups, fixed)
    mask = mask.numpy()[0, :, 0]                        # (nh, L)
    pad = P * 16 - L
    pm = np.concatenate([mask, np.zeros((nh, pad), bool)], axis=1).reshape(nh, P, 16).any(-1)
    k = min(max(3, tb // 16), P)
    sel = np.stack([np.nonzero(pm[i])[0] for i in range(nh)])
    assert sel.shape[1] == k, (sel.shape, k)
    out[f"sel_{tag}_pages"] = sel.astype(np.int32)
    out[f"sel_{tag}_weights_sha"] = np.array(sha(w.numpy()))
    out[f"sel_{tag}_params"] = np.array([seed, nh, nkvh, L, budget, int(fixed),
                                         int(value_aware), int(outlier)], np.int64)
    # per-page bound as the reference computed it (page max of the token weights)
    wp = np.concatenate([w.numpy()[0, :, 0], np.full((nh, pad), -np.inf, np.float32)],
                        axis=1).reshape(nh, P, 16).max(-1)
    out[f"sel_{tag}_page_bound"] = wp.astype(np.float32)


def decode_attention_case(out):
    """Masked decode attention at a small shape, torch ops of
    quest_attention.py:265-268,347-356."""
    nh, d, L = 4, 128, 300
    q = randn16(400, (1, nh, 1, d))
    K = randn16(401, (1, nh, L, d))
    V = randn16(402, (1, nh, L, d))
    g = np.random.default_rng(403)
    mask = g.random((1, nh, 1, L)) < 0.4
    mask[..., -1] = True
    aw = torch.matmul(t(q), t(K).transpose(2, 3)) / math.sqrt(d)
    aw[~t(mask)] = torch.tensor(torch.finfo(aw.dtype).min)
    p = torch.nn.functional.softmax(aw, dim=-1, dtype=torch.float32).to(torch.float16)
    o = torch.matmul(p, t(V))
    out["attn_mask"] = mask
    out["attn_out"] = o.numpy()
    out["attn_logits"] = aw.numpy()


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    out = {}
    metadata_cases(out)
    decode_trace(out)
    # config-1 shape: 32 heads, 4096 tokens, budget 1024 -> 64 pages
    selection_case(out, "c1_fixed", 0, 32, 32, 4096, 1024, True, True)
    selection_case(out, "c1_free", 0, 32, 32, 4096, 1024, False, True)
    selection_case(out, "c1_quest", 0, 32, 32, 4096, 1024, True, False)
    selection_case(out, "ragged_outlier", 7, 8, 8, 2000 + 9, 512, True, True, outlier=True)
    selection_case(out, "tiny", 11, 4, 4, 40, 16, True, True)       # P=3 -> k=3
    selection_case(out, "gqa", 13, 8, 2, 1500, 256, True, True)
    selection_case(out, "gqa_quest", 13, 8, 2, 1500, 256, True, False)
    # tie case: page 5 duplicated into pages 9..20 -> equal scores
    selection_case(out, "ties", 17, 4, 4, 512, 128, False, True, dup_pages=(5, list(range(9, 21))))
    decode_attention_case(out)
    out["versions"] = np.array(f"torch {torch.__version__}; numpy {np.__version__}")
    path = os.path.join(HERE, "golden_sim.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes", len(out), "arrays")


if __name__ == "__main__":
    main()
