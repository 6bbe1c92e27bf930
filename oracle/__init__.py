"""Parity oracle: a CPU restatement of AOA-KV's PyTorch simulation.

TEST INFRASTRUCTURE ONLY -- imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, never by the shipped library.
"""
