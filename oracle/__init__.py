"""CPU oracle of the decode hot path -- test infrastructure only.

Importable by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker; the product never imports it.
"""
