"""CPU oracle for the fused logprob/entropy path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or, for bench.py, as the timed
CPU baseline).  The product never imports it.
"""
