"""CPU oracle for the fused-contraction path (test infrastructure only).

``cpu_ref`` restates the reference's CPU torch path; ``brute`` holds the
independent float64 formulas that pin it. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import this
package; the product package ``trntensor_amd`` never does.
"""
