"""CPU oracle for the DenseGPA hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference's ``backend="torch"`` algorithm on the CPU
(`oracle.reference`; the counted core and its moment recurrences in
`oracle.paper`, the config-5 LM in `oracle.lm`).  Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only as the checker or as
the timed CPU baseline; the `gpa_amd` product never imports it and has no CPU
fallback.

Pinning (how the restatement itself is checked):
  * golden vectors written by importing the reference in the build container
    (`tests/golden/make_golden.py`, fixtures `tests/golden/*.npz`): default
    initialisation, token and chunk forward, carried state, 1-token
    continuation and gradients (tests/test_oracle_golden.py);
  * the published optimiser KAT of examples/smoke.py (initial MSE 0.9177752,
    docs/VALIDATION.md:61-63) (tests/test_oracle_math.py);
  * the counted core's fixtures (`tests/golden/make_paper_golden.py`,
    `tests/golden/paper_*.npz`, `moment_*.npz`) and the closed forms of its
    decayed moment and count recurrences (tests/test_oracle_paper.py);
  * mathematics: the GDN scan against its closed-form special cases (pure
    decay at beta=0, exact recall of orthonormal keys, the unrolled matrix
    form), partition invariance of cached calls, Q-independence of storage,
    and gradcheck (tests/test_oracle_math.py).
"""
from .reference import (  # noqa: F401
    OracleRun, additive_scan, forward, gdn_read, gdn_scan, gdn_step, initial_state, rope, two_stage, unit,
)
