"""The quadratic Q/K feature map on the device (`gpa_quad_features_forward`,
`gpa_quad_features_backward`): reference src/gpa/features.py:17-25.

One kernel launch forward (unit(x), the two products on the MFMA, the
normalised output) and one backward (dx, plus u and d(a)|d(b) for the weight
gradients, which are one batched product each: u^T [da | db]).  The weights
are passed as two zero-padded copies in the activation type (transposed for
the forward products, row-major for the backward's); they are parameters of
a few hundred KB, rebuilt per call.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib


def _pad(d: int) -> int:
    return -(-d // 32) * 32


def _weights(left: Tensor, right: Tensor, dtype: torch.dtype):
    """wt [H][2][DP][DP] (wt[h][p][n][k] = W_p[h][k][n]) and w [H][DP][2DP]
    (w[h][k][p*DP + n] = W_p[h][k][n]), zero-padded, in `dtype`."""
    h, d, _ = left.shape
    dp = _pad(d)
    both = torch.stack((left, right), 1).to(dtype)                     # [H,2,D,D] (k, n)
    both = F.pad(both, (0, dp - d, 0, dp - d))                         # [H,2,DP,DP]
    wt = both.transpose(-1, -2).contiguous()                           # [H,2,DP(n),DP(k)]
    w = both.permute(0, 2, 1, 3).reshape(h, dp, 2 * dp).contiguous()  # [H,DP(k),2*DP]
    return wt, w


def _problem(x: Tensor, wt: Tensor, w: Tensor, gain: Tensor, out: Tensor | None) -> _lib.QuadProblem:
    rows, heads, dim = x.shape
    p = _lib.QuadProblem()
    p.rows, p.heads, p.dim, p.dtype = rows, heads, dim, _lib.DTYPE_CODES[x.dtype]
    p.x, p.row_stride = x.data_ptr(), x.stride(0)
    p.wt, p.w, p.gain = wt.data_ptr(), w.data_ptr(), gain.data_ptr()
    p.out = out.data_ptr() if out is not None else None
    return p


class _QuadFeatures(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, left, right, gain):
        lib = _lib.load()
        wt, w = _weights(left, right, x.dtype)
        gain = gain.float().contiguous()
        out = torch.empty_like(x)
        _lib.check(lib.gpa_quad_features_forward(_problem(x, wt, w, gain, out), _lib.stream_handle(x.device)),
                   "gpa_quad_features_forward")
        ctx.save_for_backward(x, left, right, gain)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        x, left, right, gain = ctx.saved_tensors
        rows, heads, dim = x.shape
        dp = _pad(dim)
        wt, w = _weights(left, right, x.dtype)
        dout = dout.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        u = torch.empty(heads, rows, dp, device=x.device, dtype=x.dtype)
        dab = torch.empty(heads, rows, 2 * dp, device=x.device, dtype=x.dtype)
        dgain = torch.empty(-(-rows // 32), heads, device=x.device, dtype=torch.float32)
        grads = _lib.QuadGrads(dout.data_ptr(), dx.data_ptr(), u.data_ptr(), dab.data_ptr(), dgain.data_ptr())
        _lib.check(lib.gpa_quad_features_backward(_problem(x, wt, w, gain, None), grads,
                                                  _lib.stream_handle(x.device)), "gpa_quad_features_backward")
        # dW_p = u^T d(u W_p): one batched product, contiguous operands, in the activation type
        dw = torch.bmm(u.transpose(1, 2).contiguous(), dab)               # [H, DP, 2DP]
        dleft = dw[:, :dim, :dim].to(left.dtype)
        dright = dw[:, :dim, dp:dp + dim].to(right.dtype)
        return dx, dleft, dright, dgain.sum(0)


def supported(x: Tensor) -> bool:
    return x.is_cuda and x.dtype in _lib.DTYPE_CODES and 1 <= x.shape[-1] <= _lib.QUAD_MAX_DIM


def quadratic_features(x: Tensor, left: Tensor, right: Tensor, gain_raw: Tensor) -> Tensor:
    """x [..., H, D] -> the feature map of x (same shape and dtype)."""
    _lib.require_device(x)
    if not supported(x):
        raise _lib.HipBackendError("quadratic features: float32/bfloat16 with dim 1..256")
    heads, dim = x.shape[-2:]
    gain = 2 * gain_raw.sigmoid() * math.sqrt(dim)
    flat = x.reshape(-1, heads, dim).contiguous()
    if flat.shape[0] == 0:
        return x.clone()
    return _QuadFeatures.apply(flat, left, right, gain).reshape(x.shape)
