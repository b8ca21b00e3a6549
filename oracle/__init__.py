"""TEST INFRASTRUCTURE ONLY -- the CPU checker for the HIP kernels.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package; the product (churten_amd) never does.
"""
