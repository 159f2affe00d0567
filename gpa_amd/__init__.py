"""gpa_amd: the MI355X (gfx950) HIP backend of the DenseGPA attention core.

Drop-in for the reference `gpa` package's DenseGPA/GPAConfig/GPAState API
and its counted core PaperDenseGPA/PaperConfig/PaperState (src/gpa/__init__.py:1-9)
with ``backend="hip"``.  The compute path is the
hand-written HIP library `libgpa_hip.so` (C ABI declared in include/gpa_hip.h)
driven from PyTorch-ROCm; there is no CPU or eager fallback.
"""
from .config import GPAConfig
from .graph import DecodeGraph, GradientGraph
from .module import DenseGPA, QuadraticFeatures
from .ops import TwoStageState, two_stage_gdn
from .paper_dense import PaperConfig, PaperDenseGPA, PaperState
from .state import GPAState, LevelState, RelationState, ResidualSnapshot

__all__ = ["DenseGPA", "GPAConfig", "GPAState", "LevelState", "RelationState", "ResidualSnapshot",
           "TwoStageState", "two_stage_gdn", "GradientGraph", "DecodeGraph", "QuadraticFeatures",
           "PaperConfig", "PaperDenseGPA", "PaperState"]
__version__ = "0.1.0"
