"""Parity oracle for the bloom retrieval path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package.  The product (``silvertorch_amd``) never
does: it fails loudly when its HIP library is missing instead of falling back.
"""
