"""Oracle of the DSALT hot path - TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference algorithm that the HIP library is checked against:

* ``select_oracle.c`` / ``select.py``: landmark selection (hybrid score, z statistics,
  exclusion, top-k, block-causal prefix selection) with the canonical arithmetic the GPU
  kernels follow bit for bit;
* ``attention.py``: float64 forward/backward of the kernel semantics, dense brute force,
  and the reference's literal CPU-fallback mask;
* ``sdpa_cpu.py``: the reference's masked-SDPA CPU path (torch CPU), timed as the CPU
  baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import anything under ``oracle/``.  The product package ``dsalt_amd`` never does, and
has no CPU fallback.

Parity status of each function (how it is pinned) is listed in ``tests/test_oracle.py``.
"""
