"""CPU oracle of the verify round — TEST INFRASTRUCTURE ONLY.

Restatements of the reference's algorithms (each function cites the
reference file:line it follows), used as the checker by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg.  Nothing in
naivllm_amd imports this package.
"""
