"""CPU oracle for the packed binary low-rank linear — TEST INFRASTRUCTURE ONLY.

Importable only from tests/, ``__graft_entry__.smoke()`` and the CPU-baseline
leg of ``bench.py``. The product package never imports it.
"""
