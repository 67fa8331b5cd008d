"""CPU oracle of the SNNtome wave hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg may use
this package.  The product (snntome_amd/) never imports it.
"""
