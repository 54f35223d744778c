"""Test infrastructure: the strict-FP32 oracle for the Transformer forward.

Importable only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``.  Nothing in the shipped package imports it.
"""
