"""TEST INFRASTRUCTURE -- CPU oracle for the SSSD Cayley-scan path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this package, and only as the checker.  The product (``verace-v1_amd/``)
never imports, links or calls anything here.

Contents (each function cites the reference lines it restates):

* ``sssd_eager``  -- fp32 torch restatement of the reference's eager SSSD path,
  op for op (``verace_v1/modules/sssd_attention.py:21-217``): the parity target.
* ``sssd_closed`` -- fp64 token-sequential closed form (numpy, and the C library
  built from ``sssd_oracle.c``): the ground truth used to adjudicate fp32 drift.
* ``cham_ns``     -- restatement of the CHAM Newton-Schulz retraction
  (``verace_v1/modules/cham_memory.py:21-51``, ``:296-315``).

How each function is pinned (checked against something other than itself) is
listed in ``tests/test_oracle_pins.py``; no function here is left unpinned.
"""
