"""The E2E latency driver's command line (aoakv.latency, mirroring
latency/bench_latency.py:27-64): tree selection and the graph switch.  CPU
only: arguments are parsed, nothing is launched."""
import pytest


def test_kernel_flag_picks_the_tree():
    from aoakv import latency
    assert latency.parse_args(["--kernel", "aoa_kv"]).method == "AOA_KV"
    assert latency.parse_args(["--kernel", "quest_orig"]).method == "QUEST"
    assert latency.parse_args([]).method == "AOA_KV"
    with pytest.raises(SystemExit):
        latency.parse_args(["--kernel", "aoa_kv", "--method", "QUEST"])


def test_graph_flag():
    from aoakv import latency
    assert latency.parse_args(["--graph"]).graph
    assert not latency.parse_args([]).graph
    # the per-step error check synchronizes, which a graph replay cannot hold
    with pytest.raises(SystemExit):
        latency.parse_args(["--graph", "--debug_checks"])
