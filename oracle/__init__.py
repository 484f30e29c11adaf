"""CPU oracle for the Maba v2 hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithms on the CPU (numpy float64 and a
small C/OpenMP library) so that the HIP kernels can be checked against them.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import, call, link or execute anything in this directory, and
only as the checker or the timed CPU baseline.  The product package
(``maba-v2-architecture_amd/maba_sparse``) never imports it.

Modules and the reference code they follow (paths relative to the reference
checkout):

* ``oracle.dgda``        -- token-sequential DGDA prefill/step
  (``maba_sparse/kernels/common.py:229-309``) in float64, and the chunked
  WY/UT algorithm of ``maba_sparse/kernels/cpu_dgda.py:33-197``.
* ``oracle.indexer``     -- centroid pooling (``common.py:329-350``), causal
  prefill scoring + top-k (``cpu_indexer.py:53-112``), decode scoring + top-k
  (``layers/indexer.py:101-112``) and the decode centroid cache
  (``layers/indexer.py:62-82``).
* ``oracle.sparse_attn`` -- the three MABA-SA decode streams
  (``layers/sparse_attention.py:79-219``) and the gate superposition
  (``common.py:406-438``, ``cpu_indexer.py:115-150``).
* ``oracle/dgda_chunked.c`` -- C/OpenMP restatement of the chunked CPU DGDA
  algorithm, streamed chunk by chunk (the CPU baseline); built by
  ``oracle/Makefile`` into ``oracle/_build/liboracle_dgda.so``.

Pinning status of every function is listed in each module's docstring; the
tests under ``tests/test_oracle_*.py`` hold the checks.
"""
