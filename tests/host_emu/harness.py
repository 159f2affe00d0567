"""Host build of libgpa_hip's kernels for CPU tests (test infrastructure).

`build(dir)` compiles the named kernel sources with host clang and
AddressSanitizer against the HIP emulation in this directory (workgroups as
threads, barriers, wave shuffles, MFMA lane layouts, dynamic LDS sized per
launch).  `HostLib` stands in for the loaded library: each entry point dumps
its struct arguments and every buffer they point into (the whole storage of
each live tensor, found through the garbage collector) to a runner process,
which allocates each buffer with its exact size, runs the kernels and writes
the buffers back.  Any out-of-bounds access aborts the runner.
"""
from __future__ import annotations

import ctypes
import gc
import os
import re
import shutil
import struct
import subprocess

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CLANG = "/opt/rocm/llvm/bin/clang++"
ENTRIES = {"gpa_decode_step": 0, "gpa_route_forward": 1, "gpa_route_backward": 2, "gpa_route_weight_grads": 3,
           "gpa_level_forward": 4, "gpa_level_backward": 5, "gpa_route_forward_many": 6, "gpa_gdn_token_step": 7,
           "gpa_gdn_token_step_many": 8, "gpa_level_token_forward": 9,
           "gpa_token_level_forward": 10, "gpa_product_read_forward": 11, "gpa_product_read_backward": 12,
           "gpa_token_slot_step": 13, "gpa_slot_gates_act_forward": 14, "gpa_moment_scan_many": 15,
           "gpa_quad_features_forward": 16, "gpa_quad_features_backward": 17, "gpa_gdn_forward": 18,
           "gpa_gdn_backward": 19, "gpa_gdn_forward_many": 20, "gpa_gdn_backward_many": 21,
           "gpa_gdn_nchunks": 22, "gpa_gdn_path": 23}
SOURCES = ["gpa_decode.hip", "route_reader.hip", "level_mix.hip", "gdn_token.hip", "level_token.hip",
           "product_read.hip", "slot_gates.hip", "moment_scan.hip",
           "quad_features.hip", "gdn_scan.hip", "gdn_prep_mfma.hip", "gdn_state_mfma.hip", "gdn_out_mfma.hip",
           "gdn_chunk_bwd_mfma.hip"]
# Test-side sources of the host build: stand-ins for kernels it does not emulate.
HOST_SOURCES = ["strip_absent.cpp"]


def compiler() -> str | None:
    return CLANG if os.path.exists(CLANG) else shutil.which("clang++")


_EXTERN_SHARED = re.compile(r"extern\s+__shared__\s+(?:__align__\(\d+\)\s+)?(\w+(?:\s+\w+)*?)\s+(\w+)\[\];")


def _host_source(out_dir: str, name: str) -> str:
    """The kernel source as the host build compiles it.  `__shared__` is a
    static object here, so `extern __shared__ T x[];` (the launch's dynamic
    LDS) is spelled `HIP_DYNAMIC_SHARED(T, x)`, which points x at the
    launch's allocation; a #line directive keeps diagnostics and
    AddressSanitizer reports on the original file and lines."""
    path = os.path.join(ROOT, "gpa_amd", "csrc", name)
    text = open(path).read()
    if not _EXTERN_SHARED.search(text):
        return path
    copy = os.path.join(out_dir, name)
    with open(copy, "w") as f:
        f.write(f'#line 1 "{path}"\n' + _EXTERN_SHARED.sub(r"HIP_DYNAMIC_SHARED(\1, \2)", text))
    return copy


def build(out_dir: str, sources=None, jobs: int = 8) -> str:
    """Compile every source to an object (up to `jobs` compilers at once),
    then link the runner."""
    exe = os.path.join(out_dir, "host_runner")
    flags = [compiler(), "-std=c++20", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
             "-Wno-unused-command-line-argument", "-Wno-psabi", "-I", HERE, "-I", os.path.join(ROOT, "include"),
             "-I", os.path.join(ROOT, "gpa_amd", "csrc")]
    units = [_host_source(out_dir, s) for s in (sources or SOURCES)]
    units += [os.path.join(HERE, s) for s in HOST_SOURCES + ["runner.cpp"]]
    objs, running = [], []

    def finish(proc):
        out, err = proc.communicate()
        if proc.returncode:
            raise RuntimeError(err[-4000:])

    for i, src in enumerate(units):
        obj = os.path.join(out_dir, f"{i:02d}_{os.path.basename(src)}.o")
        objs.append(obj)
        running.append(subprocess.Popen(flags + ["-x", "c++", "-c", src, "-o", obj], stdout=subprocess.PIPE,
                                        stderr=subprocess.PIPE, text=True))
        if len(running) >= jobs:
            finish(running.pop(0))
    for proc in running:
        finish(proc)
    res = subprocess.run(flags + objs + ["-o", exe, "-lpthread"], capture_output=True, text=True)
    if res.returncode:
        raise RuntimeError(res.stderr[-4000:])
    return exe


def _pointer_fields(ctype, base=0):
    out = []
    if issubclass(ctype, ctypes.Array):  # an array of structs, pointers or scalars passed as one blob
        for i in range(ctype._length_):
            off = base + i * ctypes.sizeof(ctype._type_)
            if ctype._type_ is ctypes.c_void_p:
                out.append(off)
            elif issubclass(ctype._type_, (ctypes.Structure, ctypes.Array)):
                out += _pointer_fields(ctype._type_, off)
        return out
    for name, t in ctype._fields_:
        off = base + getattr(ctype, name).offset
        if t is ctypes.c_void_p:
            out.append(off)
        elif issubclass(t, ctypes.Structure):
            out += _pointer_fields(t, off)
        elif issubclass(t, ctypes.Array):
            for i in range(t._length_):
                o = off + i * ctypes.sizeof(t._type_)
                if t._type_ is ctypes.c_void_p:
                    out.append(o)
                elif issubclass(t._type_, ctypes.Structure):
                    out += _pointer_fields(t._type_, o)
    return out


def _storages():
    spans = {}
    for o in gc.get_objects():
        if isinstance(o, torch.Tensor) and o.device.type == "cpu":
            s = o.untyped_storage()
            if s.nbytes():
                spans[s.data_ptr()] = s.nbytes()
    return sorted(spans.items())


class HostLib:
    """Stands in for `gpa_amd._lib.load()` with the host build."""

    def __init__(self, exe: str, workdir: str):
        self.exe, self.workdir = exe, workdir

    def _locate(self, spans, p):
        hit = [(i, p - b) for i, (b, n) in enumerate(spans) if b <= p < b + n]
        if len(hit) != 1:
            raise AssertionError(f"pointer {p:#x} is not inside exactly one live tensor storage")
        return hit[0]

    def _call(self, entry: str, blobs, raw=()):
        spans = _storages()
        fin, fout = os.path.join(self.workdir, "in.bin"), os.path.join(self.workdir, "out.bin")
        with open(fin, "wb") as f:
            f.write(struct.pack("<qq", ENTRIES[entry], len(blobs)))
            for blob in blobs:
                data = ctypes.string_at(ctypes.addressof(blob), ctypes.sizeof(blob))
                f.write(struct.pack("<q", len(data)) + data)
            f.write(struct.pack("<q", len(spans)))
            for b, n in spans:
                f.write(struct.pack("<q", n) + ctypes.string_at(b, n))
            for blob in blobs:
                data = ctypes.string_at(ctypes.addressof(blob), ctypes.sizeof(blob))
                recs = []
                for off in _pointer_fields(type(blob)):
                    p = struct.unpack_from("<Q", data, off)[0]
                    if p:
                        recs.append((off, *self._locate(spans, p)))
                f.write(struct.pack("<q", len(recs)))
                for rec in recs:
                    f.write(struct.pack("<qqq", *rec))
            f.write(struct.pack("<q", len(raw)))
            for p in raw:
                f.write(struct.pack("<qq", *(self._locate(spans, p) if p else (-1, 0))))
        res = subprocess.run([self.exe, fin, fout], capture_output=True, text=True, timeout=900)
        if res.returncode:
            raise AssertionError(f"host run of {entry} failed ({res.returncode}):\n{res.stderr[-6000:]}")
        data = open(fout, "rb").read()
        pos = 0
        for b, n in spans:
            ctypes.memmove(b, data[pos:pos + n], n)
            pos += n
        return int(res.stdout.split()[-1])

    def gpa_decode_step(self, prob, stream):
        return self._call("gpa_decode_step", [prob])

    def gpa_route_forward(self, prob, stream):
        return self._call("gpa_route_forward", [prob])

    def gpa_route_forward_many(self, probs, n, stream):
        assert n == len(probs)
        return self._call("gpa_route_forward_many", [probs])

    def gpa_route_backward(self, prob, grads, stream):
        return self._call("gpa_route_backward", [prob, grads])

    def gpa_route_weight_grads(self, prob, grads, d_up, d_down, d_rs, d_qs, stream):
        return self._call("gpa_route_weight_grads", [prob, grads], [d_up, d_down, d_rs, d_qs])

    def gpa_level_forward(self, prob, stream):
        return self._call("gpa_level_forward", [prob])

    def gpa_level_backward(self, prob, grads, stream):
        return self._call("gpa_level_backward", [prob, grads])

    def gpa_gdn_token_step(self, prob, final, out, stream):
        return self._call("gpa_gdn_token_step", [prob, out], [final])

    def gpa_gdn_token_step_many(self, probs, finals, outs, n, stream):
        assert n == len(probs) == len(finals) == len(outs)
        return self._call("gpa_gdn_token_step_many", [probs, finals, outs])

    def gpa_level_token_forward(self, prob, stream):
        return self._call("gpa_level_token_forward", [prob])

    def gpa_token_level_forward(self, step, final, out, level, stream):
        return self._call("gpa_token_level_forward", [step, out, level], [final])

    def gpa_token_slot_step(self, step, slot, final, out, level, stream):
        blobs = [step, slot, out] + ([level] if level is not None else [])
        return self._call("gpa_token_slot_step", blobs, [final])

    def gpa_slot_gates_act_forward(self, prob, gates, stream):
        return self._call("gpa_slot_gates_act_forward", [prob, gates])

    def gpa_product_read_forward(self, prob, stream):
        return self._call("gpa_product_read_forward", [prob])

    def gpa_product_read_backward(self, prob, grads, stream):
        return self._call("gpa_product_read_backward", [prob, grads])

    def gpa_moment_scan_many(self, probs, n, stream):
        assert n == len(probs)
        return self._call("gpa_moment_scan_many", [probs])

    def gpa_quad_features_forward(self, prob, stream):
        return self._call("gpa_quad_features_forward", [prob])

    def gpa_quad_features_backward(self, prob, grads, stream):
        return self._call("gpa_quad_features_backward", [prob, grads])

    def gpa_gdn_forward(self, prob, saved, out, timing, stream):
        assert not timing
        return self._call("gpa_gdn_forward", [prob, saved, out])

    def gpa_gdn_backward(self, prob, saved, grads, timing, stream):
        assert not timing
        return self._call("gpa_gdn_backward", [prob, saved, grads])

    def gpa_gdn_forward_many(self, probs, saved, outs, n, timing, stream):
        assert not timing and n == len(probs) == len(saved) == len(outs)
        return self._call("gpa_gdn_forward_many", [probs, saved, outs])

    def gpa_gdn_backward_many(self, probs, saved, grads, n, timing, stream):
        assert not timing and n == len(probs) == len(saved) == len(grads)
        return self._call("gpa_gdn_backward_many", [probs, saved, grads])

    def gpa_gdn_nchunks(self, tokens, offset, chunk):
        return self._call("gpa_gdn_nchunks", [(ctypes.c_int32 * 3)(tokens, offset, chunk)])

    def gpa_gdn_path(self, prob):
        return self._call("gpa_gdn_path", [prob])

    def gpa_hip_last_error(self):
        return b""


def use_host(monkeypatch, host: HostLib) -> None:
    """Route `gpa_amd._lib` to the host build for the duration of a test."""
    from gpa_amd import _lib

    monkeypatch.setattr(_lib, "load", lambda: host)
    monkeypatch.setattr(_lib, "require_device", lambda t: None)
    monkeypatch.setattr(_lib, "stream_handle", lambda d: 0)
