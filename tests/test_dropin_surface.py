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


def test_rms_norm_forward_matches_fp32_formula_on_cpu():
    # reference rms_norm.cu: fp32 sum of squares, rsqrt(mean + eps), x * s * w
    # in fp32, one rounding to the input dtype
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 4096, generator=g).half()
    w = (torch.rand(4096, generator=g) + 0.5).half()
    out = qutils.rms_norm_forward(x, w, 1e-5)
    assert out.dtype == torch.float16 and out.shape == x.shape
    xd = x.double()
    ref = xd / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-5) * w.double()
    # one fp16 rounding of a value computed in fp32
    assert torch.allclose(out.double(), ref, rtol=2e-3, atol=1e-3)
    # a row scaled by c normalises to the same output (scale invariance)
    out2 = qutils.rms_norm_forward((x.float() * 2.0).half(), w, 0.0)
    assert torch.equal(out2, qutils.rms_norm_forward(x, w, 0.0))
