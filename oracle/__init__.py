"""CPU oracle for the Lighthouse layer (test infrastructure only).

Importable only from ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py``; the product package never imports it.
"""
