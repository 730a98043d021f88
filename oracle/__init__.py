"""CPU oracle for the lightning-indexer-with-fetch path. TEST INFRASTRUCTURE ONLY.

This package restates, in numpy and plain Python, the algorithms of the KVIP
reference (paths below are relative to the reference tree) so that the HIP kernels of
``kvip_amd`` can be checked against them. Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
or as the timed CPU baseline. The product path (``kvip_amd``) never imports it and
has no CPU fallback.

Modules:
  indexer  - fp8/bf16 decoding, LI score, bf16 CAST_ROUND, sortable keys, TopK-2048,
             Fetch gather, identity KV payload.
  cache    - update_abc CPU golden, SlotLRU linked-list LRU, hot-slot bitmap selector.

Every function cites the reference file:line it follows; how each one is pinned
(golden vectors, known answers, closed forms, brute force) is listed in its
docstring and exercised by tests/test_oracle_*.py.
"""
