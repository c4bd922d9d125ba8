"""CPU oracle for the decode-step sampler: test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package; the product package promptboot_amd never does.
"""
