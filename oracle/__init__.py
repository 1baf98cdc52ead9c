"""CPU oracle for the MoE feed-forward block: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the timed
CPU baseline). The product path (``pluggy_amd``) never imports it and has no
CPU fallback.
"""
