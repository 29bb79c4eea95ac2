"""CPU oracle for the linear-recurrent mixer ops — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU in float64 (or float32 when timed as the CPU
baseline), the arithmetic of the reference's mixer ops:

- ``oracle.gdn``  gated delta rule: gating, L2 norm, per-token recurrence,
  chunked WY form, varlen packing and slot-indexed decode.
- ``oracle.gka``  Gated KalmaNet: Chebyshev ridge solve + beta^2 gated linear
  attention, decode step and per-token prefill.
- ``oracle.ssd``  Mamba2 SSD: per-token recurrence, chunked form, one-step
  state update.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker / the timed CPU baseline. The
product path (``hmx``) never imports it and has no CPU fallback.

Every function cites the reference ``file:line`` it follows (paths relative to
the reference repository root).  Each function is pinned by tests in
``tests/test_oracle_*.py`` against closed forms, special cases, brute force and
cross-form equivalences; the reference ships no golden vectors for these ops.
"""
