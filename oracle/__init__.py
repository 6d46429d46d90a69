"""TEST INFRASTRUCTURE ONLY: the CPU parity oracle for the lossless IVF query path.

Imported by tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg as the
checker; never by the product package ``trident_amd``.
"""
