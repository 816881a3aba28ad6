"""CPU oracle of the MOD-DiT sparse-attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (MoD/mod/*.py, *.cu under the MOD-DiT
source tree; every function cites the lines it follows) in numpy so that the HIP
kernels can be checked against it. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker or the timed CPU baseline —
never as a product code path.

Pinning (what checks each function against something other than itself) is listed in
each docstring; the tests under tests/test_oracle*.py carry the checks.
"""
from .moddit_ref import *  # noqa: F401,F403
