"""CPU oracle for the WKV time-mixing recurrence.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
directory: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker (or
as the CPU baseline that is timed beside the GPU), never as the thing that is
measured or shipped.

Modules:

* :mod:`oracle.wkv4` -- RWKV-4 / SpikeGPT WKV: the sequential loop, the
  closed-form span, the associative-monoid form, the reference kernel's
  explicit backward, the op contracts and the single-token decode step.
* :mod:`oracle.wkv7` -- RWKV-7 DPLR recurrence (``S <- S (diag(w) + a b^T) +
  v k^T``), sequential fp64 loop.  The reference no longer contains an RWKV-7
  implementation, so this one is pinned only by the mathematics (special cases
  that reduce to causal linear attention, autograd, finite differences).

Every function cites the reference file:line it restates.  How each one is
pinned (closed forms, invariants, finite differences, special cases) is
listed in each module's docstring and exercised by ``tests/test_oracle_*.py``.
"""
