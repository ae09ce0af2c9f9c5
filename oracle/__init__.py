"""CPU oracle for the thundersync_amd hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain PyTorch/Python, the reference
algorithms the HIP kernels replace (seilk/thundersync; each function cites the
reference file:line it follows).  It is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it.  Nothing in ``thundersync_amd`` imports it, and no product
path falls back to it.

How each function is pinned (checked against something other than itself)
is stated in its module docstring; see tests/test_oracle_*.py.
"""
