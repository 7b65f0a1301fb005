"""CPU oracle for the paged-attention hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the shipped package imports this
directory: only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may use it, and only to check results (or, for the CPU
baseline, as the timed torch-native restatement). The product path raises when
its HIP library is missing; it never falls back to anything here.

Modules
-------
``attention``     float64 numpy restatement of decode / extend / verify over the
                  ``req_to_token`` + token-pool layout (the closed form that the
                  reference's GPU tests check its kernels against).
``torch_native``  the torch-native SDPA form of the same three modes (per-sequence
                  gather, fp32 ``scaled_dot_product_attention``), which is what the
                  reference's own GPU tests call and what ``bench.py`` times as the
                  CPU baseline.
``fp8``           bit-level decoding of OCP e4m3fn / e5m2 bytes.
``metadata``      page-table / query-start / verify-row metadata construction.
``kv_write``      the token pool's write with quantisation on write (divide in the
                  source dtype, round to nearest even onto the fp8 grid).

The seeded generators of the five benchmark workloads are not part of the oracle:
they live in ``sglang_restomod_amd/workloads.py``.

How each function is pinned (so that a plausible mistake fails a test) is
listed in its docstring and exercised in ``tests/test_oracle_*.py``.
"""
