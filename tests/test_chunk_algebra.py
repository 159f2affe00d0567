"""The chunked backward algebra the HIP kernels implement, checked in float64.

gdn_scan.hip computes the GDN backward per chunk from saved intermediates:
  dD    = P^T dO + diag(e^{G_C-G}) K dS_end                 (gdn_dd0, gdn_state_bwd)
  dS_n  = e^{G_C} dS_end + Q^T diag(e^G) dO - W^T dD + inj  (gdn_state_bwd)
  dQ, dK, dV, dg, dbeta from T, W, D, S_n, dS_end          (gdn_chunk_bwd, phases A-D)
Here the same steps, written with dense torch ops, must equal autograd through
the per-token oracle recurrence, for every input and the initial state, with
gradients injected at every chunk start.
"""
import torch

import oracle


def _norm_bwd(x, dxh):
    n = x.norm(dim=-1, keepdim=True)
    xh = x / n.clamp_min(1e-6)
    return torch.where(n > 1e-6, (dxh - xh * (xh * dxh).sum(-1, keepdim=True)) / n, dxh / 1e-6)


def _chunk_fwd(qn, kn, v, g, b, s):
    gam = g.cumsum(0)
    c = kn.shape[0]
    diff = gam[:, None] - gam[None, :]
    strict = torch.tril(torch.ones(c, c, dtype=torch.bool), -1)
    causal = torch.tril(torch.ones(c, c, dtype=torch.bool))
    kk = kn @ kn.T
    a = torch.where(strict, b[:, None] * diff.exp() * kk, torch.zeros(()))
    tri = torch.linalg.inv(torch.eye(c, dtype=kn.dtype) + a)
    u = tri @ (b[:, None] * v)
    w = tri @ ((b * gam.exp())[:, None] * kn)
    d = u - w @ s
    p = torch.where(causal, diff.exp() * (qn @ kn.T), torch.zeros(()))
    o = gam.exp()[:, None] * (qn @ s) + p @ d
    s_next = gam[-1].exp() * s + ((gam[-1] - gam).exp()[:, None] * kn).T @ d
    return dict(gam=gam, kk=kk, a=a, tri=tri, w=w, d=d, p=p, o=o, s_next=s_next, strict=strict, causal=causal)


def test_chunk_backward_algebra_equals_autograd():
    torch.manual_seed(0)
    t_len, c, kd, vd = 10, 4, 5, 3
    q = torch.randn(t_len, kd, dtype=torch.float64)
    k = torch.randn(t_len, kd, dtype=torch.float64)
    v = torch.randn(t_len, vd, dtype=torch.float64)
    g = -torch.rand(t_len, dtype=torch.float64) * .7
    b = torch.rand(t_len, dtype=torch.float64)
    s0 = torch.randn(kd, vd, dtype=torch.float64)
    nch = (t_len + c - 1) // c
    w_out = torch.randn(t_len, vd, dtype=torch.float64)
    w_starts = torch.randn(nch, kd, vd, dtype=torch.float64)
    w_final = torch.randn(kd, vd, dtype=torch.float64)

    # Autograd through the per-token oracle.
    leaves = [x.clone().requires_grad_() for x in (q, k, v, g, b, s0)]
    lq, lk, lv, lg, lb, ls = leaves
    state, outs, loss = ls[None, None], [], 0.
    for n in range(nch):
        lo, hi = n * c, min(t_len, (n + 1) * c)
        loss = loss + (state[0, 0] * w_starts[n]).sum()
        y, state = oracle.gdn_scan(lq[None, lo:hi, None], lk[None, lo:hi, None], lv[None, lo:hi, None],
                                   lg[None, lo:hi, None], lb[None, lo:hi, None], state)
        outs.append(y[0, :, 0])
    loss = loss + (torch.cat(outs) * w_out).sum() + (state[0, 0] * w_final).sum()
    loss.backward()

    # Kernel algebra.
    qn = q / q.norm(dim=-1, keepdim=True)
    kn = k / k.norm(dim=-1, keepdim=True)
    fw, s = [], s0
    for n in range(nch):
        lo, hi = n * c, min(t_len, (n + 1) * c)
        f = _chunk_fwd(qn[lo:hi], kn[lo:hi], v[lo:hi], g[lo:hi], b[lo:hi], s)
        f["s"] = s
        fw.append(f)
        s = f["s_next"]
    ds = w_final.clone()
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dg, db = torch.zeros_like(g), torch.zeros_like(b)
    for n in reversed(range(nch)):
        lo, hi = n * c, min(t_len, (n + 1) * c)
        f = fw[n]
        gam, tri, w, d, p, sn = f["gam"], f["tri"], f["w"], f["d"], f["p"], f["s"]
        qc, kc, vc, bc = qn[lo:hi], kn[lo:hi], v[lo:hi], b[lo:hi]
        do = w_out[lo:hi]
        eg, ek, gc = gam.exp(), (gam[-1] - gam).exp(), gam[-1]
        # gdn_dd0 + gdn_state_bwd
        dd = p.T @ do + (ek[:, None] * kc) @ ds
        ds_end = ds
        ds = gc.exp() * ds + qc.T @ (eg[:, None] * do) - w.T @ dd + w_starts[n]
        # gdn_chunk_bwd phase A
        dgam = torch.zeros_like(gam)
        dqn = eg[:, None] * (do @ sn.T)
        dw = -(dd @ sn.T)
        dkn = ek[:, None] * (d @ ds_end.T)
        rk = (dkn * kc).sum(-1)
        dgam += (dqn * qc).sum(-1) - rk
        dgam[-1] += rk.sum() + gc.exp() * (ds_end * sn).sum()
        # phase B
        dp = torch.where(f["causal"], do @ d.T, torch.zeros(()))
        gp = dp * p
        dgam += gp.sum(1) - gp.sum(0)
        dqk = dp * (gam[:, None] - gam[None, :]).exp() * f["causal"]
        dqn += dqk @ kc
        dkn += dqk.T @ qc
        # phase C
        sc = bc * eg
        dt = dd @ (bc[:, None] * vc).T + (dw @ kc.T) * sc[None, :]
        da = -(tri.T @ (dt @ tri.T)) * f["strict"]
        e = (gam[:, None] - gam[None, :]).exp() * f["strict"]
        ekk = e * f["kk"]
        db[lo:hi] += (da * ekk).sum(1)
        ga = da * bc[:, None] * ekk
        dgam += ga.sum(1) - ga.sum(0)
        dkk = da * bc[:, None] * e
        dkn += (dkk + dkk.T) @ kc
        tdw = tri.T @ dw
        dkn += sc[:, None] * tdw
        rdot = (kc * tdw).sum(-1)
        db[lo:hi] += eg * rdot
        dgam += bc * eg * rdot
        tdd = tri.T @ dd
        dv[lo:hi] = bc[:, None] * tdd
        db[lo:hi] += (vc * tdd).sum(-1)
        # phase D
        dg[lo:hi] = dgam.flip(0).cumsum(0).flip(0)
        dq[lo:hi] = _norm_bwd(q[lo:hi], dqn)
        dk[lo:hi] = _norm_bwd(k[lo:hi], dkn)
    for name, mine, ref in (("dq", dq, lq.grad), ("dk", dk, lk.grad), ("dv", dv, lv.grad), ("dg", dg, lg.grad),
                            ("dbeta", db, lb.grad), ("ds0", ds, ls.grad)):
        torch.testing.assert_close(mine, ref, rtol=1e-10, atol=1e-10, msg=name)
