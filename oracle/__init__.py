"""CPU oracle for the paged-decode attention (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker or the timed CPU baseline.  The product
(xllms_amd, libxllm_hip_backend.so) never imports or links it.
"""
