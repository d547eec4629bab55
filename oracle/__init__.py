"""CPU oracle of the triangle-attention block -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The product package ``fireprot_amd`` never imports it.
"""
