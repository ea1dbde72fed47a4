"""CPU oracle for the paged-attention path (test infrastructure, not product).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or as the timed CPU baseline.
"""
