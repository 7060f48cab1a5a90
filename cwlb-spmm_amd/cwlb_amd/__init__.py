"""Python access to the MI355X CWLB-SpMM library (libcwlb.so) for tests and
benchmarks.  The library itself is C++17/HIP behind a C ABI (include/cwlb.h);
this package only binds it with ctypes and holds the synthetic workloads.
"""
from . import paths  # noqa: F401
