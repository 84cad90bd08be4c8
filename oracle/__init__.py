"""TEST INFRASTRUCTURE ONLY: the oracle of the xnn_amd hot path.

CPU restatements of the reference's (molssi-ai/xnn) algorithms for this path, each
citing the reference file:line it follows. Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it, and there only as the checker or
the timed CPU baseline; the product package ``xnn_amd`` never imports it.

* ``oracle/neighbor.c`` + :mod:`oracle.nl` -- brute-force radius graph
  (neighborlist.py:462-506), with margin statistics around the cutoff
* :mod:`oracle.reference` -- edge vectors, radial bases, envelopes, spherical harmonics
  (from the reference's own Legendre-recurrence real harmonics), edge -> atom sums,
  float64 structure sums and autograd forces / stress, in PyTorch on the CPU
* :mod:`oracle.d4` -- D4 coordination numbers and BJ two-body energy
"""
