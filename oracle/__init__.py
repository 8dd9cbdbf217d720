"""CPU oracle for the SMAQ quantized-KV hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``smaq_amd`` imports this package.  The
only permitted callers are ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and they use it as the *checker* (or the
timed CPU baseline), never as the thing that is measured or shipped.

``smaq_ref`` is an op-for-op torch-CPU restatement of the reference algorithm
(gauravsaini/smaq, pure Python over torch).  Every function cites the
reference file:line it follows.  How each function is pinned (golden vectors,
closed forms, brute force, invariants) is listed in ``PINNING`` inside
``smaq_ref`` and exercised by ``tests/test_oracle_*.py``.
"""

from oracle import smaq_ref  # noqa: F401
