"""CPU oracle for the sparse flash attention path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, to compare the HIP kernels' results against it; the
product path never does.
"""
