"""CPU oracle of the paged KV-cache path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the
timed CPU baseline).  The product (``gpu_offloading_amd``) never imports it and
has no CPU fallback.
"""
