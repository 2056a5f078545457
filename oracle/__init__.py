"""CPU oracle for the sphops hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path
"spatial-grid binning + SPH neighbour perception forward/backward"
(TheDevilWillBeBee/NPA, ``sphops/``).  It exists to *check* the HIP path and to
time a CPU baseline.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``npa_amd``) never does and has no CPU fallback.

Modules
-------
binning      numpy restatement of cell assignment, hashing, stable counting sort,
             ``bin_offsets`` and the grid-mode block table
             (``sphops/utils.cuh:303-524``, ``sphops/sph_cuda.cu:32-206,1926-1992``).
neighbors    candidate enumeration over the 3^D cell stencil exactly as the
             reference traverses it, with the in-radius test emulated in fp32
             (``sphops/sph_cuda.cu:1561-1640``, ``utils.cuh:321-362``).
sph          float64 SPH operators (forward and explicit gather-form backward)
             restated from ``sphops/torch_sph.py:96-471`` and
             ``sphops/sph_cuda.cu:414-721,1160-1375``.
bruteforce   dense all-pairs float64/float32 torch restatement of
             ``sphops/torch_sph.py`` with autograd backward; pins ``sph`` and is
             the timed CPU baseline ("port").
perceive     torch restatement of NPA.perceive's feature assembly (scaling,
             log-normalisation, concatenation; ``models/npa.py:83-137``) and of
             step_euler's update (``models/npa.py:125-133, 154-204``).

Pinning status (what checks each function; see tests/test_oracle_*.py)
---------------------------------------------------------------------
* binning: closed forms (floor/clamp/mod, row-major and Morton hashes checked
  against brute-force coordinate enumeration, bincount/cumsum offsets,
  stable argsort) and the FTZ special case.
* neighbors: equality with an all-pairs scan restricted to the stencil.
* sph forward: kernel normalisation integrals (poly6 and spiky integrate to 1),
  constant-field and linear-field exactness, translation invariance,
  permutation equivariance, pair symmetry, two-particle closed forms.
* sph backward: equality with torch.autograd of ``bruteforce`` in float64 and
  ``torch.autograd.gradcheck``.
* safe inverse: product with the input is the identity; identity below tol.
* perceive: the log-normalisation's closed form (length log(1 + |v|), direction
  of v, zero at zero), torch.autograd.gradcheck in float64, and an independent
  closed-form Jacobian (tests/test_perceive_glue.py).
* euler_update: closed forms (|dx| = alpha eps u / (1 + u), direction of a,
  masked particles unchanged, zero padding lane unchanged), gradcheck in
  float64, and the kernel's closed-form gradient (tests/test_perceive_glue.py).
No function is left "parity unpinned".  The reference holds no golden vectors
for this path (it draws random data at run time, ``sphops/test.py:107-154``).
"""
