"""CPU oracle for the gated delta-rule core — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference results are
checked against (or as the timed CPU baseline). The product path (``vagus_amd``) never imports it and has no
CPU fallback: when the HIP library is missing it raises.
"""
