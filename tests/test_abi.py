"""The C ABI library builds, loads on a CPU-only host and exports every symbol
that include/gpa_hip.h declares (no compute call is made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gpa_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(gpa_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = _declared()
    for expected in ("gpa_hip_abi_version", "gpa_hip_last_error", "gpa_gdn_nchunks", "gpa_gdn_path",
                     "gpa_gdn_forward", "gpa_gdn_backward", "gpa_gdn_read", "gpa_gdn_read_backward",
                     "gpa_decode_step", "gpa_route_forward", "gpa_count_logits_forward",
                     "gpa_count_logits_backward", "gpa_slot_gates_forward", "gpa_slot_gates_backward",
                     "gpa_route_backward", "gpa_route_weight_grads", "gpa_level_forward", "gpa_level_backward"):
        assert expected in names


def test_library_loads_and_exports_every_declared_symbol():
    from gpa_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libgpa_hip.so not built (python -m gpa_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    typed = _lib.load()
    assert typed.gpa_hip_abi_version() == _lib.ABI_VERSION
    assert set(_lib.EXPORTS) <= set(_declared())
    # Pure host helpers.
    assert typed.gpa_gdn_nchunks(130, 0, 64) == 3
    assert typed.gpa_gdn_nchunks(1, 63, 64) == 1
    assert typed.gpa_gdn_nchunks(2, 63, 64) == 2
    assert typed.gpa_gdn_nchunks(5, 4, 4) == 0  # offset must be < chunk
    prob = _lib.Problem()
    prob.dtype, prob.kdim = 1, 128
    assert typed.gpa_gdn_path(prob) == 1      # bf16, K % 16 == 0: MFMA recurrences
    prob.kdim = 40
    assert typed.gpa_gdn_path(prob) == 0
    prob.dtype, prob.kdim = 0, 128
    assert typed.gpa_gdn_path(prob) == 0      # fp32: FMA recurrences


def test_ctypes_structs_match_c_layout():
    from gpa_amd import _lib
    assert ctypes.sizeof(_lib.Operand) == 32
    # 8 int32, 5 operands, pointer + 2 int64
    assert ctypes.sizeof(_lib.Problem) == 32 + 5 * 32 + 24
    assert ctypes.sizeof(_lib.Saved) == 15 * 8
    assert ctypes.sizeof(_lib.Grads) == 32 + 7 * 8 + 5 * 32 + 8
    assert ctypes.sizeof(_lib.Timing) == (_lib.MAX_TIMED + 1) * 8 + 8 and _lib.MAX_TIMED == 40
    assert ctypes.sizeof(_lib.DecodeState) == 16
    # slots (+pad), 7 parameter pointers, 5 states, 3 output pointers
    assert ctypes.sizeof(_lib.DecodeLevel) == 8 + 7 * 8 + 5 * 16 + 3 * 8
    # 7 int32 + 3 float, 4 operands, 8 pointers, 4 levels, 12 states, 12 pointers
    assert _lib.DecodeProblem.level.offset == 40 + 4 * 32 + 8 * 8
    assert ctypes.sizeof(_lib.DecodeProblem) == 232 + 4 * 168 + 12 * 16 + 12 * 8
    # 7 int32 + float, 5 operands, 11 pointers, 2 operands, 3 pointers
    assert ctypes.sizeof(_lib.RouteProblem) == 32 + 5 * 32 + 11 * 8 + 2 * 32 + 3 * 8 + 8 + 3 * 8
    # 7 operands, 4 pointers
    assert ctypes.sizeof(_lib.RouteGrads) == 7 * 32 + 5 * 8 + 2 * 32 + 8
    # 9 int32 (+pad), 2 operands, 4 pointers, 2 int64, 1 pointer, 3 operands, 3 pointers
    assert ctypes.sizeof(_lib.LevelProblem) == 40 + 2 * 32 + 4 * 8 + 2 * 8 + 8 + 3 * 32 + 3 * 8 + 8
    assert ctypes.sizeof(_lib.LevelGrads) == 4 * 32 + 5 * 8 + 32
    # 5 int32 (+pad), 2 operands, count0 + its stride, 5 pointers
    assert ctypes.sizeof(_lib.CountProblem) == 24 + 2 * 32 + 2 * 8 + 5 * 8
    assert ctypes.sizeof(_lib.CountGrads) == 2 * 8 + 2 * 32 + 3 * 8
    # 6 int32, key operand, 3 pointers, 2 operands; 3 operands, 2 pointers
    assert ctypes.sizeof(_lib.SlotProblem) == 24 + 32 + 3 * 8 + 2 * 32
    assert ctypes.sizeof(_lib.TokenSlot) == 2 * 8 + ctypes.sizeof(_lib.GateProblem) + 32
    assert ctypes.sizeof(_lib.SlotGrads) == 3 * 32 + 2 * 8
    # 7 int32 (+pad), base, 3 messages, 3 norms, counts, 3 pointers; pointer, 3 operands, 5 pointers
    assert ctypes.sizeof(_lib.ProductProblem) == 32 + 32 + 3 * 32 + 3 * 32 + 32 + 3 * 8
    assert ctypes.sizeof(_lib.ProductGrads) == 8 + 3 * 32 + 3 * 8 + 2 * 8
    # gpa_moment_problem: ten int32, five operands, s0 and its two strides, final
    assert ctypes.sizeof(_lib.MomentProblem) == 40 + 5 * 32 + 3 * 8 + 8
    assert ctypes.sizeof(_lib.QuadProblem) == 16 + 8 + 8 + 3 * 8 + 8
    assert ctypes.sizeof(_lib.QuadGrads) == 5 * 8


def test_backend_refuses_cpu_tensors():
    import torch
    from gpa_amd import _lib
    from gpa_amd.ops import gdn_scan_hip
    x = torch.zeros(1, 2, 1, 4)
    with pytest.raises(_lib.HipBackendError):
        gdn_scan_hip(x, x, x, torch.zeros(1, 2, 1), torch.zeros(1, 2, 1), None, chunk=2)
