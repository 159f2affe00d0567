"""`GPAConfig`: the validated, frozen model description of a DenseGPA core.

Field names, defaults and the `ValueError` contract mirror the reference
`GPAConfig` (src/gpa/attention.py:17-75) so that configurations and
checkpoints move between the two packages unchanged.  Every default equals the
reference's except one, on purpose: `backend` defaults to and only accepts
``"hip"``.  The ``torch``/``fla`` backends belong to the reference package;
this package is the gfx950 backend that drops in beside them.  As in the
reference, ``chunk_size`` defaults to 1, which selects the tokenwise model
(attention.py:264-297); ``chunk_size > 1`` selects the block-lagged chunk
model.

`execution` is accepted for API compatibility and ignored: every reference
schedule (reference/packed/triton/staged) computes the same function
(reference tests/test_packed.py, tests/test_staged.py), and the HIP backend
always runs its own level-major schedule.
"""
from __future__ import annotations

from dataclasses import dataclass

_SLOT_FEATURES = ("linear", "softmax", "tanh")
_POSITIONAL = ("gated", "moments", "none")
_EXECUTIONS = ("reference", "packed", "triton", "staged")


@dataclass(frozen=True)
class GPAConfig:
    heads: int = 4
    key_dim: int = 32
    value_dim: int = 32
    slots: tuple[int, ...] = (16, 16, 16, 16)
    positional_mode: str = "gated"
    query_scale: float = 1 / 16
    beta_init: float = .1
    beta_max: float = .9
    decay_init: float = .001
    relation_beta_init: float = .6
    relation_decay_init: float = .0001
    chunk_size: int = 1
    backend: str = "hip"
    execution: str = "reference"
    read_scale: float = 1.
    shared_query_center: bool = False
    rsa_update: bool = False
    paper_product_read: bool = False
    control_dim: int = 0
    slot_feature: str = "linear"
    slot_scale: float = 4.
    balanced_bridge: bool = False
    relation_marginal: bool = False
    quadratic_features: bool = False
    learn_read_scale: bool = False

    def __post_init__(self):
        object.__setattr__(self, "slots", tuple(int(m) for m in self.slots))
        checks = (
            (min(self.heads, self.key_dim, self.value_dim, self.chunk_size) > 0,
             "dimensions and chunk_size must be positive"),
            (self.control_dim >= 0, "control_dim must be nonnegative"),
            (self.slot_feature in _SLOT_FEATURES and self.slot_scale > 0,
             "slot_feature must be linear/softmax/tanh, slot_scale positive"),
            (self.paper_product_read or not self.relation_marginal,
             "relation marginal correction needs product reading"),
            (len(self.slots) > 0 and min(self.slots) > 0,
             "slots must contain positive capacities"),
            (self.positional_mode in _POSITIONAL, "unknown positional_mode"),
            (self.positional_mode != "moments" or self.key_dim % 2 == 0,
             "positional moments require even key_dim"),
            (0 < self.beta_init < self.beta_max <= 1,
             "require 0 < beta_init < beta_max <= 1"),
            (0 < self.relation_beta_init < 1, "relation_beta_init must be in (0,1)"),
            (self.decay_init > 0 and self.relation_decay_init > 0,
             "initial decays must be positive"),
            (self.backend == "hip",
             "gpa_amd implements backend='hip'; the torch/fla backends live in the "
             "reference gpa package"),
            (self.execution in _EXECUTIONS,
             "execution must be reference, packed, triton, or staged"),
            (self.read_scale > 0, "read_scale must be positive"),
            (not self.shared_query_center or self.query_scale > 0,
             "shared query-center parameterization needs query_scale > 0"),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)

    @property
    def levels(self) -> int:
        return len(self.slots)

    @property
    def edges(self) -> tuple[tuple[int, int], ...]:
        """Ordered (source, target) pairs, source-major (attention.py:122)."""
        n = self.levels
        return tuple((i, j) for i in range(n) for j in range(n) if i != j)
