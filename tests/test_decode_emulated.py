"""The fused decode kernel (gpa_amd/csrc/gpa_decode.hip) built for the host and
compared with the oracle's reference forward, on the CPU.

The kernel source is compiled with g++ against tests/host_emu/ (workgroups as
threads, barriers, wave shuffles) and AddressSanitizer.  `decode.decode_step`
builds its `gpa_decode_problem` exactly as on the GPU; the call is redirected to
a runner process that copies every buffer the problem points into (each whole
tensor storage) to an allocation of its exact size, runs the kernel, and copies
the buffers back.  Any out-of-bounds access aborts the runner.

Checked per decode step: the output and, at the end, every tensor of the cache,
against the oracle, from a prefill part-way into a block and across block
boundaries (residual snapshot refresh), and from an empty cache (broadcast
prefixes, batch stride 0).  Tolerances: 1e-5 relative in float32 and bfloat16
(both follow the reference's rounding points, so only fp32 summation order
differs).
"""
import copy
import ctypes
import os
import shutil
import struct
import subprocess

import pytest
import torch

import oracle
from gpa_amd import DenseGPA, GPAConfig, _lib
from gpa_amd import decode as dec
from gpa_amd.state import tensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EMU = os.path.join(ROOT, "tests", "host_emu")

CASES = {
    "tiny_unequal_c3": dict(cfg=dict(heads=2, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=3), b=2,
                            prefill=4, steps=3),
    "tiny_none_c4": dict(cfg=dict(heads=1, key_dim=4, value_dim=3, slots=(3, 2, 4), chunk_size=4,
                                  positional_mode="none"), b=2, prefill=0, steps=5),
    "one_level": dict(cfg=dict(heads=2, key_dim=8, value_dim=5, slots=(6,), chunk_size=4), b=1, prefill=2,
                      steps=4),
    "c2_dims": dict(cfg=dict(heads=2, key_dim=32, value_dim=48, slots=(64, 64, 64, 128), chunk_size=8), b=1,
                    prefill=15, steps=2),
    "c3_dims": dict(cfg=dict(heads=1, key_dim=128, value_dim=128, slots=(128, 128, 128, 256), chunk_size=4),
                    b=1, prefill=3, steps=2),
}


@pytest.fixture(scope="module")
def runner(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("host_emu") / "decode_runner")
    cmd = ["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address", "-static-libasan", "-fno-omit-frame-pointer",
           "-I", EMU, "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "gpa_amd", "csrc"),
           "-x", "c++", os.path.join(ROOT, "gpa_amd", "csrc", "gpa_decode.hip"),
           "-x", "none", os.path.join(EMU, "runner.cpp"), "-o", exe, "-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return exe


def _pointer_fields(ctype, base=0):
    out = []
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


class _HostLib:
    """Stands in for the loaded library: `gpa_decode_step` runs the host build."""

    def __init__(self, exe, workdir):
        self.exe, self.workdir, self.live = exe, workdir, []

    def gpa_decode_step(self, prob, stream):
        raw = ctypes.string_at(ctypes.addressof(prob), ctypes.sizeof(prob))
        storages = {}
        for t in self.live:
            s = t.untyped_storage()
            if s.nbytes():
                storages[s.data_ptr()] = s.nbytes()
        spans = sorted(storages.items())
        ptrs = []
        for off in _pointer_fields(type(prob)):
            p = struct.unpack_from("<Q", raw, off)[0]
            if not p:
                continue
            hit = [(i, p - b) for i, (b, n) in enumerate(spans) if b <= p < b + n]
            assert len(hit) == 1, f"pointer field at byte {off} is not inside exactly one known storage"
            ptrs.append((off, *hit[0]))
        fin, fout = os.path.join(self.workdir, "in.bin"), os.path.join(self.workdir, "out.bin")
        with open(fin, "wb") as f:
            f.write(struct.pack("<q", len(raw)) + raw + struct.pack("<q", len(spans)))
            for b, n in spans:
                f.write(struct.pack("<q", n) + ctypes.string_at(b, n))
            f.write(struct.pack("<q", len(ptrs)))
            for rec in ptrs:
                f.write(struct.pack("<qqq", *rec))
        res = subprocess.run([self.exe, fin, fout], capture_output=True, text=True, timeout=600)
        assert res.returncode == 0, res.stderr[-6000:]
        data = open(fout, "rb").read()
        pos = 0
        for b, n in spans:
            ctypes.memmove(b, data[pos:pos + n], n)
            pos += n
        return 0

    def gpa_hip_last_error(self):
        return b""


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return ((a - b).norm() / max(b.norm().item(), 1e-30)).item()


@pytest.mark.parametrize("name,dtype", [(n, torch.float32) for n in CASES]
                         + [(n, torch.bfloat16) for n in ("tiny_unequal_c3", "c3_dims")],
                         ids=[f"{n}-f32" for n in CASES] + ["tiny_unequal_c3-bf16", "c3_dims-bf16"])
def test_host_built_decode_kernel_matches_oracle(name, dtype, runner, tmp_path, monkeypatch):
    host = _HostLib(runner, str(tmp_path))
    monkeypatch.setattr(dec, "FUSED_DECODE", True)
    monkeypatch.setattr(_lib, "load", lambda: host)
    monkeypatch.setattr(_lib, "require_device", lambda t: None)
    monkeypatch.setattr(_lib, "stream_handle", lambda d: 0)
    real_empty = torch.empty

    def tracked_empty(*a, **k):
        t = real_empty(*a, **k)
        host.live.append(t)
        return t

    real_state_arg = dec._state_arg

    def tracked_state_arg(t):
        arg, t2 = real_state_arg(t)
        host.live.append(t2)
        return arg, t2

    monkeypatch.setattr(dec.torch, "empty", tracked_empty)
    monkeypatch.setattr(dec, "_state_arg", tracked_state_arg)

    spec = CASES[name]
    torch.manual_seed(11)
    model = DenseGPA(GPAConfig(**spec["cfg"]))
    with torch.no_grad():
        for w in model.gate_weight:
            w.normal_(0, .1)
        for p in model.relation_prefix:
            p.normal_(0, .01)
        model.edge_logits.normal_(0, .5)
    ref = oracle.OracleRun(copy.deepcopy(model))
    cfg = model.config
    gen = torch.Generator().manual_seed(5)
    b, n0, steps = spec["b"], spec["prefill"], spec["steps"]
    q = torch.randn(b, n0 + steps, cfg.heads, cfg.key_dim, generator=gen)
    k = torch.nn.functional.normalize(torch.randn(q.shape, generator=gen), dim=-1)
    v = torch.randn(b, n0 + steps, cfg.heads, cfg.value_dim, generator=gen)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    with torch.no_grad():
        if n0:
            _, ref_state = ref(q[:, :n0], k[:, :n0], v[:, :n0])
            state = copy.deepcopy(ref_state)
        else:
            ref_state, state = None, model.initial_state(b, dtype=dtype)
        for t in range(n0, n0 + steps):
            xs = [x[:, t:t + 1].contiguous() for x in (q, k, v)]
            host.live[:] = [p.data for p in model.parameters()] + xs + list(tensors(state))
            assert dec.decode_supported(model, *xs, state, None)
            y, state = dec.decode_step(model, *xs, state)
            y_ref, ref_state = ref(*xs, ref_state)
            assert y.dtype == dtype
            assert _rel(y, y_ref) < 1e-5, t
            assert state.chunk_offset == ref_state.chunk_offset and state.position == ref_state.position
            assert (state.frozen is None) == (ref_state.frozen is None)
        for n, (a, r) in enumerate(zip(tensors(state), tensors(ref_state))):
            assert a.shape == r.shape, n
            assert _rel(a, r) < 1e-5, n
