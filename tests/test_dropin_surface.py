"""The names a reference driver takes from ``quest`` / ``quest.utils`` exist in
``aoakv.utils`` with call signatures that accept the reference's calls, so a
driver switches trees by changing its imports only.

The reference signatures below are restated from
kernels/aoa_kv/quest/utils/__init__.py (apply_rope_in_place :25-31,
rms_norm_forward :54-58, append_kv :69-74, prefill_forward :133-139,
decode_estimate :177-181, decode_topk :216-219, decode_sparse_attn :248-255)
and controller.py (InferenceController :8-18, set_page_budget :79,
prepare_metadata :84, begin_forward :92, end_forward :146, need_estimate
:149, clean_states :156, v_log_norm_layer :161).  The call sites they serve:
QuestAttention.py:99-157, llama.py:20-22,72,425-486,520-560 and
latency/bench_latency.py:125-168.  CPU only: nothing here launches a kernel.
"""
import inspect

import pytest
import torch

torch = pytest.importorskip("torch")
import aoakv  # noqa: E402
from aoakv import utils as qutils  # noqa: E402
from aoakv.utils import controller as qcontroller  # noqa: E402

# function -> (positional parameter names, keyword parameters with defaults)
REF_FUNCTIONS = {
    "apply_rope_in_place": (["q", "k", "past_kv_len"], ["rope_scale", "rope_theta"]),
    "rms_norm_forward": (["input", "weight", "epsilon"], []),
    "append_kv": (["k", "v", "iController", "layer_idx"], []),
    "prefill_forward": (["q", "iController", "layer_idx"], ["rope_scale", "rope_theta"]),
    "decode_estimate": (["q", "iController", "layer_idx"], []),
    "decode_topk": (["estimated_attn_score", "iController"], []),
    "decode_sparse_attn": (["q", "iController", "layer_idx", "topk_indices"],
                           ["rope_scale", "rope_theta"]),
}

# controller method -> positional parameter names after self (+ keywords used)
REF_METHODS = {
    "set_page_budget": (["page_budget"], []),
    "prepare_metadata": (["seq_len"], []),
    "begin_forward": (["seq_len"], ["updateTensor"]),
    "end_forward": ([], []),
    "need_estimate": ([], []),
    "clean_states": ([], []),
    "v_log_norm_layer": (["layer_idx"], []),
}

# attributes the reference drivers read off a controller after begin_forward
REF_ATTRIBUTES = ["kv_cache", "metadata_cache", "kv_indices_with_last", "kv_indices_without_last",
                  "metadata_indices", "kv_indptr_for_append", "metadata_indptr_for_append",
                  "kv_last_page_idx", "metadata_last_page_idx",
                  "inference_page_budget", "topk_dindices_buffer"]


def _accepts(fn, positional, keywords):
    sig = inspect.signature(fn)
    # the reference call: every positional by position, every keyword by name
    args = [object()] * len(positional)
    kwargs = {k: None for k in keywords}
    sig.bind(*args, **kwargs)
    # and by name, as call sites such as QuestAttention.py:99 pass some of them
    sig.bind(**{n: object() for n in positional}, **kwargs)


@pytest.mark.parametrize("name", sorted(REF_FUNCTIONS))
def test_quest_utils_function_resolves_with_reference_signature(name):
    fn = getattr(qutils, name)
    pos, kw = REF_FUNCTIONS[name]
    _accepts(fn, pos, kw)


@pytest.mark.parametrize("name", sorted(REF_METHODS))
def test_controller_method_resolves_with_reference_signature(name):
    fn = getattr(qcontroller.InferenceController, name)
    pos, kw = REF_METHODS[name]
    sig = inspect.signature(fn)
    sig.bind(object(), *[object()] * len(pos), **{k: True for k in kw})


def test_controller_constructor_takes_the_reference_arguments():
    # llama.py:540-549 passes all eight by keyword; controller.py:8-18 order
    sig = inspect.signature(qcontroller.InferenceController.__init__)
    names = ["num_layers", "num_heads", "head_dim", "page_size", "page_budget", "max_seq_len",
             "dtype", "device"]
    sig.bind(object(), **{n: object() for n in names})
    sig.bind(object(), *[object()] * len(names))
    assert qutils.InferenceController is qcontroller.InferenceController


def test_controller_exposes_the_reference_attributes():
    # an attribute the constructor or begin_forward sets, or a property
    cls = qcontroller.InferenceController
    src = inspect.getsource(cls)
    for attr in REF_ATTRIBUTES:
        assert f"self.{attr}" in src or isinstance(getattr(cls, attr, None), property), attr


def test_rms_norm_oracle_is_pinned_by_the_formula():
    """The oracle's rms_norm_forward (the reference kernel rms_norm.cu:76-159:
    fp32 sum of squares, 1/sqrt(mean + eps), (x * r) * w in fp32, one fp16
    rounding) against the float64 formula, and by its invariances: a dropped
    eps, a sum for the mean or a missing weight fails these."""
    import numpy as np
    from oracle import sim
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 4096)).astype(np.float16)
    w = (rng.random(4096) + 0.5).astype(np.float16)
    out = sim.rms_norm_forward(x, w, 1e-5)
    assert out.dtype == np.float16 and out.shape == x.shape
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-5) * w.astype(np.float64)
    # one fp16 rounding of a value computed in fp32
    np.testing.assert_allclose(out.astype(np.float64), ref, rtol=2e-3, atol=1e-3)
    # a row scaled by 2 normalises to the same output (eps 0), eps matters
    # where the mean square is small
    assert np.array_equal(sim.rms_norm_forward((x.astype(np.float32) * 2).astype(np.float16),
                                               w, 0.0), sim.rms_norm_forward(x, w, 0.0))
    tiny = (x.astype(np.float32) * 1e-3).astype(np.float16)
    assert not np.allclose(sim.rms_norm_forward(tiny, w, 1e-2).astype(np.float32),
                           sim.rms_norm_forward(tiny, w, 0.0).astype(np.float32), rtol=0.1)


def test_rms_norm_forward_refuses_host_tensors():
    """The drop-in rms_norm_forward runs the library kernel: host tensors are
    refused, not computed on the CPU."""
    x = torch.zeros(2, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="device tensor"):
        qutils.rms_norm_forward(x, torch.ones(64, dtype=torch.float16), 1e-6)