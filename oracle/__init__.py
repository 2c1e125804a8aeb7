"""CPU oracle for the gated-delta path: test infrastructure only.

Import rule: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import anything here, and only as the
checker or the timed CPU comparator, never as a product code path.
"""
