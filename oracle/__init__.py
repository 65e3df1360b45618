"""CPU oracle for the MoE hot path -- test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``; the product path never uses it.
"""
