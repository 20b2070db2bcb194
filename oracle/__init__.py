"""CPU oracle for the minicompiler HIP backend - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline;
the product never imports, links or calls it. See oracle/oracle.h for what
each function restates (reference file:line) and what is pinned how.
"""
