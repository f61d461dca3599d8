"""CPU oracle for the batch-invariant operator path -- TEST INFRASTRUCTURE ONLY.

A restatement, with stock PyTorch CPU ops in float64, of what each reference operator of
yiannisha/robotics-batch-invariant-ops computes (batch_invariant_ops/batch_invariant_ops.py and
batch_invariant_ops/moe.py; each function cites the lines it follows), including the points
where the reference rounds to the working dtype.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s CPU-baseline leg may import it, and only as the checker; the product
(``batch_invariant_ops``) never does.

Every function here is pinned by tests/test_oracle.py against closed forms, exact
integer-valued cases and mathematical invariants (see that file).
"""

from .reference_ops import *  # noqa: F401,F403
from .reference_ops import __all__  # noqa: F401
