"""CPU oracle for the atlas-rnn memory-layer recurrence.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (`atlas_rnn_amd`) imports this
package. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may use it, and only as the checker (or as the timed CPU baseline), never as a code path of
the product.

Every function restates the reference algorithm from its source text and names the
reference `file:line` it follows (paths are relative to the engineerA314/atlas-rnn tree).
How each function is pinned (golden vectors, closed forms, cross-checks) is listed in the
module docstring of `oracle.recurrence`.
"""

from .recurrence import (  # noqa: F401
    scalar_assoc_scan,
    scalar_assoc_scan_sequential,
    sliding_sum_along_time,
    poly_feature_map,
    lag_weights,
    memory_recurrence_loop,
    memory_recurrence_vectorised,
    affine_associative_scan,
    affine_scan_sequential,
)
