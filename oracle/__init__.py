"""CPU oracle for the MetalNN hot path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference layers' arithmetic (zkeown/MetalAudio, Sources/MetalNN),
each function citing the reference lines it follows. It is the checker: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and never as the
measured or shipped path. The product runs on libmnn.so's HIP kernels.

Every function computes in the dtype of its inputs' `dtype` argument (float64 by default) so
that parity can be judged against an fp64 result. How each function is pinned (reference
golden vectors, closed forms, library routines, invariants) is listed in tests/test_oracle.py.
"""
from .layers import *  # noqa: F401,F403
