"""Per-kernel launch timing with HIP events, for roofline accounting.

Inside `kernel_timer()`, every library entry point gets a `gpa_timing` of
fresh HIP events; the library records them on its launch stream between the
kernels it enqueues.  On exit the elapsed times are read and aggregated per
kernel name (template instantiation, the grouping rocprofv3 --stats uses),
together with each launch's algorithmic FLOP count:

  gdn_prep       (4CK + 2CV + C^2/3)      per token: K K^T, W, U, triangular solve
  gdn_state_fwd  4KV                      W S, K^T D
  gdn_out_*      2KV + 2CK + 2CV          Q S, Q K^T, P D
  gdn_dd0*       2CK + 2CV                Q K^T, P^T dO
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


def _prep(k, v, c, tokens, dtype):
    e, km = _tag(dtype), _kmax(k)
    return (f"gdn_prep_mfma<{e},{km},{'true' if _mfma(k, dtype) else 'false'}>",
            (4 * c * k + 2 * c * v + c * c / 3) * tokens)


def _on_strips(k, dtype) -> bool:
    """Mirror of the library's choice of the strip state kernels (packable)."""
    return _mfma(k, dtype) and k <= 128


def _state_fwd_name(k, dtype) -> str:
    km = _kmax(k)
    if _mfma(k, dtype):
        return f"gdn_state_fwd_strip<{km}>" if km <= 128 else f"gdn_state_fwd_mfma<{km}>"
    return f"gdn_state_fwd<{km}>"


def _state_bwd_name(k, dtype) -> str:
    km = _kmax(k)
    if _mfma(k, dtype):
        return f"gdn_state_bwd_strip<{km}>" if km <= 128 else f"gdn_state_bwd_mfma<{km}>"
    return f"gdn_state_bwd<{_tag(dtype)},{km}>"


def _out(k, v, c, tokens, dtype):
    e, km = _tag(dtype), _kmax(k)
    name = f"gdn_out_mfma<{km}>" if _mfma(k, dtype) and v <= 256 else f"gdn_out_fwd<{e},{km}>"
    return name, (2 * k * v + 2 * c * k + 2 * c * v) * tokens


def _dd0(k, v, c, tokens, dtype):
    e, km = _tag(dtype), _kmax(k)
    name = f"gdn_dd0_mfma<{km}>" if _mfma(k, dtype) and v <= 256 else f"gdn_dd0<{e},{km}>"
    return name, (2 * c * k + 2 * c * v) * tokens


def _chunk_bwd(k, v, c, tokens, dtype, read):
    e, km = _tag(dtype), _kmax(k)
    flop = 4 * k * v + 4 * c * v + 4 * c * k + 2 * c * c
    if read:
        flop += 2 * k * v + 2 * c * v + 6 * c * k
    mfma_chunk = k % 4 == 0 and not (km == 256 and e == "f32")
    return f"{'gdn_chunk_bwd_mfma' if mfma_chunk else 'gdn_chunk_bwd'}<{e},{km}>", flop * tokens


def forward_timing(k: int, v: int, c: int, tokens: int, dtype, read: bool):
    return forward_timing_many([(k, v, c, tokens, dtype, read)])


def backward_timing(k: int, v: int, c: int, tokens: int, dtype, read: bool):
    return backward_timing_many([(k, v, c, tokens, dtype, read, None)])


_MFMA_MAXP = 5  # problems per packed launch of the 256-key MFMA state kernels


def _state_launches(groups, key, name, flop):
    """The state launches of a many-call in the library's order: the groups on
    the strip kernels with equal `key` share one launch, at the position of the
    first of them, and so do up to five 256-key MFMA groups; the others launch
    alone."""
    kernels, done = [], [False] * len(groups)
    for i, gi in enumerate(groups):
        if done[i]:
            continue
        strips, wide = _on_strips(gi[0], gi[4]), _mfma(gi[0], gi[4]) and gi[0] > 128
        if not (strips or wide):
            kernels.append((name(gi[0], gi[4]), flop(gi)))
            continue
        total, count = 0.0, 0
        for j in range(i, len(groups)):
            gj = groups[j]
            same = _on_strips(gj[0], gj[4]) if strips else (_mfma(gj[0], gj[4]) and gj[0] > 128)
            if done[j] or not same or key(gj) != key(gi) or (wide and count == _MFMA_MAXP):
                continue
            total += flop(gj)
            count += 1
            done[j] = True
        kernels.append((name(gi[0], gi[4]), total))
    return kernels


def forward_timing_many(groups):
    """Kernel list of gpa_gdn_forward_many over groups (k, v, c, tokens, dtype,
    read): every prep, the state launches, every read."""
    if _active is None:
        return None
    kernels = [_prep(*g[:5]) for g in groups]
    kernels += _state_launches(groups, lambda g: _kmax(g[0]), _state_fwd_name, lambda g: 4 * g[0] * g[1] * g[3])
    kernels += [_out(*g[:5]) for g in groups if g[5]]
    return _active.timing(kernels)


def backward_timing_many(groups):
    """Kernel list of gpa_gdn_backward_many over groups (k, v, c, tokens,
    dtype, read, injected): every dd0, the state launches, every chunk kernel."""
    if _active is None:
        return None
    kernels = [_dd0(*g[:5]) for g in groups if g[5]]
    kernels += _state_launches(groups, lambda g: (_kmax(g[0]), g[5], g[6]), _state_bwd_name,
                               lambda g: (6 if g[5] else 4) * g[0] * g[1] * g[3])
    kernels += [_chunk_bwd(*g[:6]) for g in groups]
    return _active.timing(kernels)


def summarize_trace(path: str, gap_ms: float = 100.0, top: int = 25) -> str:
    """Markdown summary of a rocprofv3 `--kernel-trace --output-format csv`
    kernel trace: per-kernel calls, total and average duration, busy time and
    concurrency, over the whole run and over each segment that follows an idle
    gap of at least `gap_ms` (bench.py leaves one before its timed steps and
    one before its single-stream timing step)."""
    import csv

    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    recs = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in rows)
    if not recs:
        return "(empty trace)\n"
    cuts, last_end = [], recs[0][1]
    for i, (b, e, _) in enumerate(recs[1:], 1):
        if b - last_end >= gap_ms * 1e6:
            cuts.append(i)
        last_end = max(last_end, e)

    def short(name: str) -> str:
        name = name.replace("void ", "").replace("(anonymous namespace)::", "")
        depth = 0
        for i, ch in enumerate(name):
            depth += ch == "<"
            depth -= ch == ">"
            if ch == "(" and depth == 0:
                name = name[:i]
                break
        return name if len(name) <= 90 else name[:87] + "..."

    def table(part, title):
        stats: dict = {}
        for b, e, n in part:
            c, t = stats.get(short(n), (0, 0))
            stats[short(n)] = (c + 1, t + (e - b))
        span = (max(e for _, e, _ in part) - min(b for b, _, _ in part)) / 1e6
        total = sum(t for _, t in stats.values())
        busy, cur_b, cur_e = 0, None, None  # union of the kernel intervals
        for b, e, _ in sorted(part):
            if cur_e is None or b > cur_e:
                busy += (cur_e - cur_b) if cur_e is not None else 0
                cur_b, cur_e = b, e
            else:
                cur_e = max(cur_e, e)
        busy = (busy + cur_e - cur_b) / 1e6
        lines = [f"### {title}", "",
                 f"{len(part)} dispatches, {len(stats)} kernels, {total / 1e6:.2f} ms kernel time "
                 f"in a {span:.2f} ms span; some kernel running for {busy:.2f} ms "
                 f"(mean concurrency {total / 1e6 / max(busy, 1e-9):.2f} while busy).", "",
                 "| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
        for n, (c, t) in sorted(stats.items(), key=lambda kv: -kv[1][1])[:top]:
            lines.append(f"| `{n}` | {c} | {t / 1e6:.2f} | {t / c / 1e3:.1f} | {100 * t / total:.2f} |")
        return "\n".join(lines) + "\n"

    out = table(recs, "Whole run")
    bounds = cuts + [len(recs)]
    for n, (lo, hi) in enumerate(zip(bounds[:-1], bounds[1:]), 1):
        out += "\n" + table(recs[lo:hi], f"Segment {n} after an idle gap of at least {gap_ms:g} ms")
    return out


def _kernel_name(raw: str) -> str:
    return raw.replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]


def _read_counters(path: str) -> dict:
    """{(kernel, counter): (dispatches, total)} of a rocprofv3 counter_collection.csv."""
    import csv

    stats: dict = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            key = (_kernel_name(r["Kernel_Name"]), r["Counter_Name"])
            c, t = stats.get(key, (0, 0.0))
            stats[key] = (c + 1, t + float(r["Counter_Value"]))
    return stats


def summarize_counters(path: str) -> str:
    """Markdown table of a rocprofv3 `--pmc` counter_collection.csv: per kernel
    and counter, the dispatch count and the mean value per dispatch."""
    stats = _read_counters(path)
    lines = ["| kernel | counter | dispatches | mean per dispatch |", "|---|---|---:|---:|"]
    for (n, ctr), (c, t) in sorted(stats.items(), key=lambda kv: -kv[1][1]):
        lines.append(f"| `{n[:90]}` | {ctr} | {c} | {t / c:.1f} |")
    return "\n".join(lines) + "\n"


def _ours(kernel: str) -> bool:
    """A kernel of this library's scans or route reader."""
    return "gdn_" in kernel or "route_" in kernel


def timer_name(kernel: str) -> str:
    """The name `kernel_timer` gives a kernel of a trace: the namespace and
    spaces dropped, bf16_t written bf16, and the state recurrences grouped by
    their key width alone (their other template flags select variants)."""
    n = kernel.replace("gpa::", "").replace("bf16_t", "bf16").replace(" ", "")
    if n.startswith("gdn_state_") and "<" in n:
        n = n.split(",")[0].rstrip(">") + ">"
    return n


def summarize_traffic(fetch: str, write: str, copy_fetch: str, copy_write: str, copy_bytes: int) -> str:
    """HBM bytes per dispatch of every gdn kernel from a FETCH_SIZE and a
    WRITE_SIZE pass (KiB per dispatch), each scaled by what the same counter
    reads for a plain copy of `copy_bytes` bytes."""
    f, w = _read_counters(fetch), _read_counters(write)
    cf, cw = _read_counters(copy_fetch), _read_counters(copy_write)

    def per_dispatch(stats, kernel, ctr):
        c, t = stats[(kernel, ctr)]
        return t / c

    copy = "__amd_rocclr_copyBuffer"
    kib = copy_bytes / 1024
    sf = kib / per_dispatch(cf, copy, "FETCH_SIZE")
    sw = kib / per_dispatch(cw, copy, "WRITE_SIZE")
    groups: dict = {}
    for (kernel, ctr), (c, t) in f.items():
        if ctr != "FETCH_SIZE" or not _ours(kernel) or (kernel, "WRITE_SIZE") not in w:
            continue
        wc, wt = w[(kernel, "WRITE_SIZE")]
        g = groups.setdefault(timer_name(kernel), [0, 0.0, 0.0])
        g[0] += c
        g[1] += t
        g[2] += wt * c / wc  # the write pass may count dispatches differently; weight by the fetch pass
    lines = [f"Copy calibration ({copy_bytes} bytes read and written): FETCH_SIZE x {sf:.3f}, WRITE_SIZE x {sw:.3f}.",
             "", "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM MB read | HBM MB written |",
             "|---|---:|---:|---:|---:|---:|"]
    for name, (c, ft, wt) in sorted(groups.items(), key=lambda kv: -(kv[1][1] * sf + kv[1][2] * sw) / kv[1][0]):
        fk, wk = ft / c, wt / c
        lines.append(f"| `{name}` | {c} | {fk:,.1f} | {wk:,.1f} | {fk * sf * 1.024e-3:,.1f} | {wk * sw * 1.024e-3:,.1f} |")
    return "\n".join(lines) + "\n"


def summarize_mfma(path: str, clock_mhz: float = 2400.0, xcds: int = 8, simds: int = 1024) -> str:
    """MFMA use per gdn kernel from one `--pmc` pass holding GRBM_GUI_ACTIVE,
    SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_VALU_MFMA_MOPS_BF16/_F32 (512 FLOP per
    unit), SQ_WAVE_CYCLES, SQ_WAIT_ANY and SQ_WAIT_INST_ANY: the kernel's
    duration (GRBM_GUI_ACTIVE counts every XCD), the share of all SIMD cycles
    in which an MFMA was busy, and the executed bf16 MFMA rate against the
    2.5 PFLOP/s dense peak."""
    s = _read_counters(path)
    kernels = sorted({k for k, c in s if c == "SQ_VALU_MFMA_BUSY_CYCLES" and _ours(k)})
    lines = ["| kernel | dispatches | us per dispatch | MFMA busy (% of SIMD cycles) | executed bf16 MFMA TFLOP/s "
             "| % of bf16 peak | executed fp32 MFMA TFLOP/s | waves waiting (% of wave cycles) |",
             "|---|---:|---:|---:|---:|---:|---:|---:|"]
    rows = []
    for k in kernels:
        def mean(ctr):
            c, t = s.get((k, ctr), (1, 0.0))
            return t / c
        n = s[(k, "SQ_VALU_MFMA_BUSY_CYCLES")][0]
        cycles = mean("GRBM_GUI_ACTIVE") / xcds
        us = cycles / clock_mhz
        busy = mean("SQ_VALU_MFMA_BUSY_CYCLES") / (cycles * simds)
        bf = mean("SQ_INSTS_VALU_MFMA_MOPS_BF16") * 512 / (us * 1e-6) / 1e12
        f32 = mean("SQ_INSTS_VALU_MFMA_MOPS_F32") * 512 / (us * 1e-6) / 1e12
        wait = mean("SQ_WAIT_ANY") / max(mean("SQ_WAVE_CYCLES"), 1.0)
        rows.append((n * us, f"| `{timer_name(k)}` ({k.split('<')[-1].rstrip('>')}) | {n} | {us:,.1f} | "
                             f"{100 * busy:.1f} | {bf:,.1f} | {100 * bf / 2500:.2f} | {f32:,.1f} | {100 * wait:.0f} |"))
    lines += [r for _, r in sorted(rows, key=lambda x: -x[0])]
    return "\n".join(lines) + "\n"


STALL_PASSES = (
    ("SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_ANY",
     "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_SCA"),
    ("SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_WAVES"),
)


def summarize_stalls(first: str, second: str, top: int = 24) -> str:
    """Where the waves of each kernel spend their cycles, from the two `--pmc`
    passes of STALL_PASSES: the share of wave cycles waiting at an s_waitcnt
    or barrier (WAIT_ANY), waiting for an instruction's dependency to issue
    (WAIT_INST_ANY, of which LDS: WAIT_INST_LDS), and issuing any, VALU (MFMA
    included), LDS and scalar instructions; and the share of LDS-active
    cycles lost to bank conflicts.  Kernels in order of total wave cycles."""
    a, b = _read_counters(first), _read_counters(second)
    kernels = {k for k, c in a if c == "SQ_WAVE_CYCLES"}

    def tot(stats, k, ctr):
        return stats.get((k, ctr), (0, 0.0))[1]

    order = sorted(kernels, key=lambda k: -tot(a, k, "SQ_WAVE_CYCLES"))[:top]
    cols = STALL_PASSES[0][1:]
    lines = ["| kernel | dispatches | " + " | ".join(c[3:].lower() for c in cols) + " | LDS bank conflict |",
             "|---|---:|" + "---:|" * (len(cols) + 1)]
    for k in order:
        w = tot(a, k, "SQ_WAVE_CYCLES") or 1.0
        conflict = tot(b, k, "SQ_LDS_BANK_CONFLICT") / (tot(b, k, "SQ_LDS_IDX_ACTIVE") or 1.0)
        lines.append(f"| `{timer_name(k)}` | {a[(k, 'SQ_WAVE_CYCLES')][0]} | "
                     + " | ".join(f"{100 * tot(a, k, c) / w:.0f} %" for c in cols) + f" | {100 * conflict:.0f} % |")
    return "\n".join(lines) + "\n"


def copy_kernel(nbytes: int, reps: int = 3) -> None:
    """A plain device copy of `nbytes` (reads and writes that many bytes per
    launch): the calibration kernel for FETCH_SIZE / WRITE_SIZE."""
    import torch

    x = torch.ones(nbytes // 4, device="cuda", dtype=torch.float32)
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(f"copied {nbytes} bytes x {reps}", flush=True)


if __name__ == "__main__":
    import sys

    cmd, args = sys.argv[1], sys.argv[2:]
    if cmd == "trace":
        print(summarize_trace(args[0]))
    elif cmd == "counters":
        print(summarize_counters(args[0]))
    elif cmd == "traffic":
        print(summarize_traffic(*args[:4], int(args[4])))
    elif cmd == "mfma":
        print(summarize_mfma(args[0]))
    elif cmd == "stalls":
        print(summarize_stalls(args[0], args[1]))
    elif cmd == "copy":
        copy_kernel(int(args[0]))
    else:
        raise SystemExit("usage: python -m gpa_amd.profiling trace|counters|mfma <csv> | stalls <csv> <csv> | "
                         "traffic <fetch csv> <write csv> <copy fetch csv> <copy write csv> <copy bytes> | copy <bytes>")
