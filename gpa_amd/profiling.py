"""Per-kernel launch timing with HIP events, for roofline accounting.

Inside `kernel_timer()`, every library entry point gets a `gpa_timing` of
fresh HIP events; the library records them on its launch stream between the
kernels it enqueues.  On exit the elapsed times are read and aggregated per
kernel name (template instantiation, the grouping rocprofv3 --stats uses),
together with each launch's algorithmic FLOP count:

  gdn_prep       (4CK + 2CV + C^2/3)      per token: K K^T, W, U, triangular solve
  gdn_state_fwd  4KV                      W S, K^T D
  gdn_out_fwd    2KV + 2CK + 2CV          Q S, Q K^T, P D
  gdn_dd0        2CK + 2CV                Q K^T, P^T dO
  gdn_state_bwd  4KV (+2KV with a read)   K dS, W^T dD (+ Q^T dO)
  gdn_chunk_bwd  4KV + 4CV + 4CK + 2C^2   D dS^T, Y S^T, dD D^T, T^T dD, K K^T, T^T X,
                 (+2KV + 2CV + 6CK)       dKK K (+ dO S^T, dO D^T, Q K^T, dQK K, dQK^T Q)
with C the chunk length, K/V the scan widths, per real token of every stream.
Outside the context manager nothing is recorded and no event exists.
"""
from __future__ import annotations

import contextlib
import ctypes

from . import _lib

_active: "_Timer | None" = None
_hip = None


def _hip_runtime():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
    return _hip


def _kmax(k: int) -> int:
    return 64 if k <= 64 else (128 if k <= 128 else 256)


def _mfma(k: int, dtype) -> bool:
    """Mirror of the library's choice of the MFMA state recurrences."""
    return _tag(dtype) == "bf16" and k % 16 == 0


def _tag(dtype) -> str:
    return "bf16" if str(dtype).endswith("bfloat16") else "f32"


class _Timer:
    def __init__(self):
        self.pending: list[tuple[_lib.Timing, list[tuple[str, float]]]] = []
        self.events: list[int] = []
        self.stats: dict[str, list[float]] = {}  # name -> [launches, total_ms, flop]

    def timing(self, kernels: list[tuple[str, float]]) -> _lib.Timing:
        hip = _hip_runtime()
        t = _lib.Timing()
        for i in range(len(kernels) + 1):
            ev = ctypes.c_void_p()
            if hip.hipEventCreate(ctypes.byref(ev)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.events.append(ev.value)
            t.events[i] = ev.value
        self.pending.append((t, kernels))
        return t

    def collect(self):
        hip = _hip_runtime()
        for t, kernels in self.pending:
            if t.launched != len(kernels) + 1:
                continue
            hip.hipEventSynchronize(t.events[t.launched - 1])
            for i, (name, flop) in enumerate(kernels):
                ms = ctypes.c_float()
                hip.hipEventElapsedTime(ctypes.byref(ms), t.events[i], t.events[i + 1])
                row = self.stats.setdefault(name, [0, 0.0, 0.0])
                row[0] += 1
                row[1] += ms.value
                row[2] += flop
        for ev in self.events:
            hip.hipEventDestroy(ev)
        self.pending, self.events = [], []

    def table(self) -> list[dict]:
        rows = [{"name": n, "launches": int(c), "total_ms": ms, "avg_us": ms / c * 1e3,
                 "tflops": (fl / (ms * 1e-3) / 1e12) if ms > 0 else 0.0}
                for n, (c, ms, fl) in self.stats.items()]
        return sorted(rows, key=lambda r: -r["total_ms"])

    def dominant(self) -> dict | None:
        rows = self.table()
        return rows[0] if rows else None


@contextlib.contextmanager
def kernel_timer():
    """Time every library kernel launched inside the block (see module doc)."""
    global _active
    timer = _Timer()
    _active = timer
    try:
        yield timer
    finally:
        _active = None
        timer.collect()


def forward_timing(k: int, v: int, c: int, tokens: int, dtype, read: bool):
    if _active is None:
        return None
    e, km = _tag(dtype), _kmax(k)
    state = f"gdn_state_fwd_mfma<{km}>" if _mfma(k, dtype) else f"gdn_state_fwd<{km}>"
    kernels = [(f"gdn_prep_mfma<{e},{km},{'true' if _mfma(k, dtype) else 'false'}>",
                (4 * c * k + 2 * c * v + c * c / 3) * tokens),
               (state, 4 * k * v * tokens)]
    if read:
        kernels.append((f"gdn_out_fwd<{e},{km}>", (2 * k * v + 2 * c * k + 2 * c * v) * tokens))
    return _active.timing(kernels)


def backward_timing(k: int, v: int, c: int, tokens: int, dtype, read: bool):
    if _active is None:
        return None
    e, km = _tag(dtype), _kmax(k)
    kernels = []
    if read:
        kernels.append((f"gdn_dd0<{e},{km}>", (2 * c * k + 2 * c * v) * tokens))
    state = f"gdn_state_bwd_mfma<{km}>" if _mfma(k, dtype) else f"gdn_state_bwd<{e},{km}>"
    kernels.append((state, (6 if read else 4) * k * v * tokens))
    chunk = 4 * k * v + 4 * c * v + 4 * c * k + 2 * c * c
    if read:
        chunk += 2 * k * v + 2 * c * v + 6 * c * k
    mfma_chunk = k % 4 == 0 and not (km == 256 and e == "f32")
    name = "gdn_chunk_bwd_mfma" if mfma_chunk else "gdn_chunk_bwd"
    kernels.append((f"{name}<{e},{km}>", chunk * tokens))
    return _active.timing(kernels)
