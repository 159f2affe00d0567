"""ctypes binding of libgpa_hip.so (C ABI in include/gpa_hip.h).

The library is loaded from the package directory only.  If it is missing, or
no gfx950 device is present, every entry point raises: there is no fallback.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgpa_hip.so")
ABI_VERSION = 31
DECODE_MAX_LEVELS = 4
DECODE_MAX_EDGES = 12
DECODE_MAX_WIDTH = 256
MAX_TIMED = 40
CHUNK_ROWS = 64
MAX_KDIM = 256
MAX_VDIM = 1024
DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1}

c_i32, c_i64, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
c_fp = ctypes.POINTER(ctypes.c_float)


class Operand(ctypes.Structure):
    _fields_ = [("ptr", c_vp), ("sb", c_i64), ("st", c_i64), ("sh", c_i64)]


class Problem(ctypes.Structure):
    _fields_ = [("batch", c_i32), ("heads", c_i32), ("tokens", c_i32), ("offset", c_i32),
                ("chunk", c_i32), ("kdim", c_i32), ("vdim", c_i32), ("dtype", c_i32),
                ("q", Operand), ("k", Operand), ("v", Operand), ("g", Operand), ("beta", Operand),
                ("s0", c_vp), ("s0_sb", c_i64), ("s0_sh", c_i64)]


class Saved(ctypes.Structure):
    _fields_ = [(n, c_vp) for n in ("kn", "qn", "w", "u", "delta", "tri", "gam", "beta", "states", "final",
                                    "wrow", "wcol", "krow", "kcol", "qcol")]


class Grads(ctypes.Structure):
    _fields_ = [("dout", Operand), ("dstates", c_vp), ("dfinal", c_vp),
                ("dd0", c_vp), ("o", c_vp), ("ddelta", c_vp), ("dhend", c_vp), ("dw", c_vp),
                ("dq", Operand), ("dk", Operand), ("dv", Operand), ("dg", Operand), ("dbeta", Operand),
                ("ds0", c_vp)]


class Timing(ctypes.Structure):
    _fields_ = [("events", c_vp * (MAX_TIMED + 1)), ("launched", c_i32)]


class DecodeState(ctypes.Structure):
    _fields_ = [("ptr", c_vp), ("sb", c_i64)]


class DecodeLevel(ctypes.Structure):
    _fields_ = [("slots", c_i32)] + [(n, c_vp) for n in ("center", "gate_weight", "gate_bias", "route_weight",
                                                           "query_weight", "route_up", "route_down")] + \
               [(n, DecodeState) for n in ("inner", "outer", "count", "snap_inner", "snap_outer")] + \
               [(n, c_vp) for n in ("inner_out", "outer_out", "count_out")]


class DecodeProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "heads", "key_dim", "value_dim", "levels", "dtype",
                                     "positional_none")] + \
               [(n, ctypes.c_float) for n in ("read_scale", "query_scale", "beta_max")] + \
               [(n, Operand) for n in ("q", "k", "v", "out")] + \
               [(n, c_vp) for n in ("residual_raw", "count_gain_raw", "route_mlp_gain", "output_logits",
                                    "relation_gain", "edge_logits", "relation_decay_raw", "relation_beta_raw")] + \
               [("level", DecodeLevel * DECODE_MAX_LEVELS), ("relation", DecodeState * DECODE_MAX_EDGES),
                ("relation_out", c_vp * DECODE_MAX_EDGES)]


ROUTE_MAX_WIDTH = 256
ROUTE_MAX_INCOMING = 3
ROUTE_ROWS = 32
ROUTE_MAX_PACK = 4
TOKEN_MAX_PACK = 12
GDN_MAX_PACK = 12


class RouteProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "slots", "key_dim", "incoming", "dtype")] + \
               [("query_scale", ctypes.c_float), ("base", Operand), ("msg", Operand * ROUTE_MAX_INCOMING),
                ("q", Operand)] + \
               [(n, c_vp) for n in ("edge_weight", "gain", "mlp_gain", "up_t", "down_t", "rs_t", "qs_t",
                                    "up", "down", "rs", "qs")] + \
               [("qo", Operand), ("route", Operand)] + [(n, c_vp) for n in ("r0", "h1", "hd")] + \
               [("rsa", c_i32), ("balanced", c_i32), ("mix", c_vp), ("qr", c_vp), ("qdir", c_vp)]


class RouteGrads(ctypes.Structure):
    _fields_ = [(n, Operand) for n in ("dqo", "droute", "dbase")] + \
               [("dmsg", Operand * ROUTE_MAX_INCOMING), ("dq", Operand)] + \
               [(n, c_vp) for n in ("dh1", "dhd", "dqs", "hg", "partials")] + \
               [("dqr", Operand), ("ddir", Operand), ("mix_partials", c_vp)]


PRODUCT_ROWS = 4


class ProductProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "slots", "incoming", "dtype", "marginal")] + \
               [("base", Operand), ("msg", Operand * ROUTE_MAX_INCOMING), ("norm", Operand * ROUTE_MAX_INCOMING),
                ("counts", Operand)] + [(n, c_vp) for n in ("edge_weight", "gexp", "out")]


class ProductGrads(ctypes.Structure):
    _fields_ = [("dout", c_vp), ("dmsg", Operand * ROUTE_MAX_INCOMING), ("dnorm", c_vp * ROUTE_MAX_INCOMING)] + \
               [(n, c_vp) for n in ("dcounts", "partials")]


LEVEL_MAX_WIDTH = 256


class LevelProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "key_dim", "value_dim", "slots", "chunk",
                                     "offset", "dtype")] + \
               [("key", Operand), ("value", Operand)] + \
               [(n, c_vp) for n in ("a_states", "b_states", "a_first", "b_first")] + \
               [("a_first_sb", c_i64), ("b_first_sb", c_i64), ("eta", c_vp)] + \
               [(n, Operand) for n in ("write", "key_out", "value_out")] + [("rk", c_vp), ("rv", c_vp),
                                                                             ("stats", c_vp)] + \
               [("given_write", c_i32)]


class LevelGrads(ctypes.Structure):
    _fields_ = [(n, Operand) for n in ("dwrite", "dkey_out", "dvalue_out", "dkey")] + \
               [(n, c_vp) for n in ("da_states", "db_states", "da_first", "db_first", "deta")] + \
               [("dwrite_given", Operand)]


class CountProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "slots", "dtype")] + \
               [("raw", Operand), ("write", Operand), ("count0", c_vp), ("count0_sb", c_i64)] + \
               [(n, c_vp) for n in ("gain", "scale", "logits", "final_count", "prefix")]


class CountGrads(ctypes.Structure):
    _fields_ = [("dlogits", c_vp), ("dfinal", c_vp), ("draw", Operand), ("dwrite", Operand)] + \
               [(n, c_vp) for n in ("dcount0", "partials", "tsum")]


class SlotProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "key_dim", "slots", "dtype")] + \
               [("key", Operand), ("center", c_vp), ("center_t", c_vp), ("gate_w", c_vp), ("slot", Operand),
                ("raw", Operand)]


class SlotGrads(ctypes.Structure):
    _fields_ = [(n, Operand) for n in ("dslot", "draw", "dkey")] + [(n, c_vp) for n in ("dcenter", "dgate_w")]


class GateProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "dtype")] + \
               [("raw", Operand), ("bias", c_vp), ("beta_max", ctypes.c_float), ("decay_scale", ctypes.c_float)] + \
               [(n, c_vp) for n in ("g_in", "b_in", "g_out", "b_out")]


GATE_MAX_HEADS = 256


class GateGrads(ctypes.Structure):
    _fields_ = [("dg_in", c_vp), ("db_in", c_vp), ("dg_out", c_vp), ("db_out", c_vp), ("draw", Operand),
                ("dbias", c_vp)]


class TokenSlot(ctypes.Structure):
    _fields_ = [("center", c_vp), ("gate_w", c_vp), ("gates", GateProblem), ("slot", Operand)]


TOKEN_LOGITS_MAX_SLOTS = 256
TOKEN_LOGITS_MAX_PACK = 8


class TokenLogitsProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "heads", "slots", "dtype")] + \
               [("raw", Operand), ("write", Operand), ("count0", c_vp), ("count0_sb", c_i64)] + \
               [(n, c_vp) for n in ("gain", "scale", "logits", "count", "local")]


class MixProblem(ctypes.Structure):
    _fields_ = [(n, c_i32) for n in ("batch", "tokens", "heads", "value_dim", "levels", "dtype")] + \
               [("read", Operand * DECODE_MAX_LEVELS), ("weights", c_vp), ("out", Operand)]


MIX_MAX_HEADS = 256


class MixGrads(ctypes.Structure):
    _fields_ = [("dout", Operand), ("dread", Operand * DECODE_MAX_LEVELS), ("dweights", c_vp)]


GATE_NONE, GATE_TOKEN, GATE_KEY, GATE_VALUE = 0, 1, 2, 3
MOMENT_MAX_KDIM = 256
MOMENT_MAX_PACK = 4


class MomentProblem(ctypes.Structure):
    _fields_ = [("batch", c_i32), ("heads", c_i32), ("tokens", c_i32), ("kdim", c_i32), ("vdim", c_i32),
                ("dtype", c_i32), ("gate", c_i32), ("reverse", c_i32), ("y_f32", c_i32), ("pad_", c_i32),
                ("q", Operand), ("k", Operand), ("v", Operand), ("g", Operand), ("y", Operand),
                ("s0", c_vp), ("s0_sb", c_i64), ("s0_sh", c_i64), ("final", c_vp)]

QUAD_MAX_DIM = 256
SUM_MAX = 8


class QuadProblem(ctypes.Structure):
    _fields_ = [("rows", c_i32), ("heads", c_i32), ("dim", c_i32), ("dtype", c_i32), ("x", c_vp),
                ("row_stride", c_i64), ("wt", c_vp), ("w", c_vp), ("gain", c_vp), ("out", c_vp)]


class QuadGrads(ctypes.Structure):
    _fields_ = [("dout", c_vp), ("dx", c_vp), ("u", c_vp), ("dab", c_vp), ("dgain", c_vp)]

EXPORTS = {
    "gpa_hip_abi_version": ([], ctypes.c_int),
    "gpa_hip_last_error": ([], ctypes.c_char_p),
    "gpa_gdn_nchunks": ([c_i32, c_i32, c_i32], c_i32),
    "gpa_gdn_path": ([ctypes.POINTER(Problem)], c_i32),
    "gpa_gdn_forward": ([ctypes.POINTER(Problem), ctypes.POINTER(Saved), Operand, ctypes.POINTER(Timing), c_vp],
                        ctypes.c_int),
    "gpa_gdn_backward": ([ctypes.POINTER(Problem), ctypes.POINTER(Saved), ctypes.POINTER(Grads),
                          ctypes.POINTER(Timing), c_vp], ctypes.c_int),
    "gpa_gdn_read": ([ctypes.POINTER(Problem), ctypes.POINTER(Saved), Operand, c_vp], ctypes.c_int),
    "gpa_gdn_scan_noalloc": ([ctypes.POINTER(Problem), Operand, c_vp, c_vp], ctypes.c_int),
    "gpa_gdn_read_backward": ([ctypes.POINTER(Problem), ctypes.POINTER(Saved), Operand, Operand, c_vp],
                              ctypes.c_int),
    "gpa_level_token_forward": ([ctypes.POINTER(LevelProblem), c_vp], ctypes.c_int),
    "gpa_token_level_forward": ([ctypes.POINTER(Problem), c_vp, Operand, ctypes.POINTER(LevelProblem), c_vp],
                                ctypes.c_int),
    "gpa_token_slot_step": ([ctypes.POINTER(Problem), ctypes.POINTER(TokenSlot), c_vp, Operand,
                             ctypes.POINTER(LevelProblem), c_vp], ctypes.c_int),
    "gpa_gdn_forward_many": ([ctypes.POINTER(Problem), ctypes.POINTER(Saved), ctypes.POINTER(Operand), c_i32,
                              ctypes.POINTER(Timing), c_vp], ctypes.c_int),
    "gpa_gdn_backward_many": ([ctypes.POINTER(Problem), ctypes.POINTER(Saved), ctypes.POINTER(Grads), c_i32,
                               ctypes.POINTER(Timing), c_vp], ctypes.c_int),
    "gpa_gdn_token_step": ([ctypes.POINTER(Problem), c_vp, Operand, c_vp], ctypes.c_int),
    "gpa_gdn_token_step_many": ([ctypes.POINTER(Problem), ctypes.POINTER(c_vp), ctypes.POINTER(Operand), c_i32,
                                 c_vp], ctypes.c_int),
    "gpa_decode_step": ([ctypes.POINTER(DecodeProblem), c_vp], ctypes.c_int),
    "gpa_route_forward": ([ctypes.POINTER(RouteProblem), c_vp], ctypes.c_int),
    "gpa_route_forward_many": ([ctypes.POINTER(RouteProblem), c_i32, c_vp], ctypes.c_int),
    "gpa_route_backward": ([ctypes.POINTER(RouteProblem), ctypes.POINTER(RouteGrads), c_vp], ctypes.c_int),
    "gpa_route_weight_grads": ([ctypes.POINTER(RouteProblem), ctypes.POINTER(RouteGrads), c_vp, c_vp, c_vp,
                                c_vp, c_vp], ctypes.c_int),
    "gpa_level_forward": ([ctypes.POINTER(LevelProblem), c_vp], ctypes.c_int),
    "gpa_level_backward": ([ctypes.POINTER(LevelProblem), ctypes.POINTER(LevelGrads), c_vp], ctypes.c_int),
    "gpa_count_logits_forward": ([ctypes.POINTER(CountProblem), c_vp], ctypes.c_int),
    "gpa_count_logits_backward": ([ctypes.POINTER(CountProblem), ctypes.POINTER(CountGrads), c_vp],
                                  ctypes.c_int),
    "gpa_slot_gates_forward": ([ctypes.POINTER(SlotProblem), c_vp], ctypes.c_int),
    "gpa_slot_gates_backward": ([ctypes.POINTER(SlotProblem), ctypes.POINTER(SlotGrads), c_vp], ctypes.c_int),
    "gpa_gate_act_forward": ([ctypes.POINTER(GateProblem), c_vp], ctypes.c_int),
    "gpa_gate_act_backward": ([ctypes.POINTER(GateProblem), ctypes.POINTER(GateGrads), c_vp], ctypes.c_int),
    "gpa_slot_gates_act_forward": ([ctypes.POINTER(SlotProblem), ctypes.POINTER(GateProblem), c_vp], ctypes.c_int),
    "gpa_token_logits_many": ([ctypes.POINTER(TokenLogitsProblem), ctypes.c_int32, c_vp], ctypes.c_int),
    "gpa_product_read_forward": ([ctypes.POINTER(ProductProblem), c_vp], ctypes.c_int),
    "gpa_product_read_backward": ([ctypes.POINTER(ProductProblem), ctypes.POINTER(ProductGrads), c_vp], ctypes.c_int),
    "gpa_token_logits_forward": ([ctypes.POINTER(TokenLogitsProblem), c_vp], ctypes.c_int),
    "gpa_output_mix_forward": ([ctypes.POINTER(MixProblem), c_vp], ctypes.c_int),
    "gpa_output_mix_backward": ([ctypes.POINTER(MixProblem), ctypes.POINTER(MixGrads), c_vp], ctypes.c_int),
    "gpa_row_softmax_forward": ([c_vp, c_vp, c_i64, c_i32, c_i32, c_vp], ctypes.c_int),
    "gpa_row_softmax_backward": ([c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp], ctypes.c_int),
    "gpa_copy_many": ([ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), ctypes.POINTER(ctypes.c_int64), c_i32, c_vp],
                      ctypes.c_int),
    "gpa_moment_scan_many": ([ctypes.POINTER(MomentProblem), c_i32, c_vp], ctypes.c_int),
    "gpa_quad_features_forward": ([ctypes.POINTER(QuadProblem), c_vp], ctypes.c_int),
    "gpa_quad_features_backward": ([ctypes.POINTER(QuadProblem), ctypes.POINTER(QuadGrads), c_vp], ctypes.c_int),
    "gpa_sum_many": ([c_vp, ctypes.POINTER(c_vp), c_i32, c_i64, c_i32, c_vp], ctypes.c_int),
}

_lib = None


class HipBackendError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load and type the library (no device needed); raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipBackendError(f"{LIB_PATH} is not built: run `python -m gpa_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in EXPORTS.items():
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res
    if lib.gpa_hip_abi_version() != ABI_VERSION:
        raise HipBackendError("libgpa_hip.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def require_device(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise HipBackendError("backend='hip' needs tensors on a ROCm GPU (no CPU fallback)")
    arch = getattr(torch.cuda.get_device_properties(t.device), "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise HipBackendError(f"backend='hip' is built for gfx950, found {arch!r}")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise HipBackendError(f"{what} failed ({rc}): {load().gpa_hip_last_error().decode()}")


def operand(t: torch.Tensor | None, heads_dim: int = 2) -> Operand:
    """Operand for a [B,T,H,...] tensor (or [B,T,H] scalars); last dim contiguous."""
    if t is None:
        return Operand(None, 0, 0, 0)
    if t.ndim == 4 and t.stride(3) != 1:
        raise ValueError("operand needs a contiguous last dimension")
    return Operand(t.data_ptr(), t.stride(0), t.stride(1), t.stride(heads_dim))


def stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
