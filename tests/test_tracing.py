"""roctx ranges of the model shim (aoakv.tracing), on the CPU: the ranges
open and close without a GPU, nest, survive an exception in their body, and
cost nothing when disabled.  The names follow the reference's nvtx ranges
(quest/models/QuestAttention.py:87-176, quest/models/llama.py:138-164,465-475);
that they reach a trace is shown by rocprofv3 --marker-trace on the GPU box."""
import pytest

from aoakv import tracing


@pytest.fixture
def on():
    was = tracing.enabled()
    tracing.enable()
    yield
    tracing.enable(was)


def test_backend_is_roctx_or_torch():
    assert "roctx" in tracing.backend() or tracing.backend() == "torch.cuda.nvtx"


def test_ranges_nest_and_close(on):
    with tracing.range("layer=0"):
        with tracing.range("LlamaAttention"):
            with tracing.range("qkv_proj"):
                pass
    with pytest.raises(ValueError):
        with tracing.range("estimate"):
            raise ValueError("the range still closes")


def test_disabled_ranges_call_nothing(monkeypatch):
    tracing.enable(False)
    calls = []
    monkeypatch.setattr(tracing, "_impl", (lambda s: calls.append(s), lambda: calls.append(0), "x"))
    with tracing.range("topk"):
        pass
    assert calls == []
    tracing.enable()
    try:
        with tracing.range("topk"):
            pass
    finally:
        tracing.enable(False)
    assert calls == ["topk", 0]
