"""Parity oracle for the fast-matmul Linear path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline. The product (``rdna3-fastmm_amd/``) never imports it.

Every function is pinned by tests/test_oracle.py; none is "parity unpinned".
"""
