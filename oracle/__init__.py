"""TEST INFRASTRUCTURE ONLY: the CPU restatement of TensorFlow's CPU kernels
for the hot path (parity checker and CPU baseline).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it; the
product never does."""
