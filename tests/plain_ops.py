"""The gated delta recurrence written as plain tensor ops, differentiated by torch autograd on the CPU.

This restates the reference's second test oracle, `gated_delta_ops` (reference tests/gated_delta_ref.h:100-120:
GQA by repeating key heads, then per step decay, kv_mem, delta, update, y), and the reference checks its
hand-written backward against autodiff through exactly that (reference tests/test_deltanet.cpp:103-137). Here the
same comparison pins the oracle's backward. It shares no code with the oracle.
"""
from __future__ import annotations

import numpy as np
import torch


def gated_delta_ops(q, k, v, g, beta, state):
    """q, k [B, T, Hk, Dk]; v [B, T, Hv, Dv]; g (factor), beta [B, T, Hv]; state [B, Hv, Dv, Dk]."""
    B, T, Hk, _ = q.shape
    Hv = v.shape[2]
    rep = Hv // Hk
    qr = q.repeat_interleave(rep, dim=2) if rep > 1 else q
    kr = k.repeat_interleave(rep, dim=2) if rep > 1 else k
    ys = []
    for t in range(T):
        qt, kt = qr[:, t], kr[:, t].unsqueeze(2)  # [B,H,Dk], [B,H,1,Dk]
        gt = g[:, t].reshape(B, Hv, 1, 1)
        bt = beta[:, t].unsqueeze(2)
        state = state * gt
        kv_mem = (state * kt).sum(-1)  # [B,H,Dv]
        delta = (v[:, t] - kv_mem) * bt
        state = state + kt * delta.unsqueeze(3)
        ys.append((state * qt.unsqueeze(2)).sum(-1))
    if not ys:  # an empty sequence leaves the state as it was
        return v.new_zeros(B, 0, Hv, v.shape[3]), state
    return torch.stack(ys, 1), state


def fwd_bwd(inputs: dict, cu_seqlens=None, g_is_log=True, dtype=torch.float64):
    """Forward and autograd backward of sum(y * dy) + sum(s_out * ds_out), per packed sequence when cu_seqlens
    is given. Returns numpy arrays keyed like oracle.gdn_ref.fwd_bwd (without ckpt)."""
    t = {n: (None if inputs.get(n) is None else torch.tensor(np.asarray(inputs[n]), dtype=dtype))
         for n in ("q", "k", "v", "g", "beta", "s0", "dy", "ds_out")}
    B, T, Hk, Dk = t["q"].shape
    Hv, Dv = t["v"].shape[2], t["v"].shape[3]
    leaves = {n: t[n].clone().requires_grad_(True) for n in ("q", "k", "v", "g", "beta")}
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    s0 = t["s0"] if t["s0"] is not None else torch.zeros(N, Hv, Dv, Dk, dtype=dtype)
    s0 = s0.clone().requires_grad_(True)
    gf = torch.exp(leaves["g"]) if g_is_log else leaves["g"]
    if cu_seqlens is None:
        y, s_out = gated_delta_ops(leaves["q"], leaves["k"], leaves["v"], gf, leaves["beta"], s0)
    else:
        ys, ss = [], []
        for n in range(N):
            a, b = int(cu_seqlens[n]), int(cu_seqlens[n + 1])
            sl = slice(a, b)
            yn, sn = gated_delta_ops(leaves["q"][:, sl], leaves["k"][:, sl], leaves["v"][:, sl], gf[:, sl],
                                     leaves["beta"][:, sl], s0[n:n + 1])
            ys.append(yn)
            ss.append(sn)
        y, s_out = torch.cat(ys, 1), torch.cat(ss, 0)
    loss = (y * t["dy"]).sum()
    if t["ds_out"] is not None:
        loss = loss + (s_out * t["ds_out"]).sum()
    loss.backward()
    out = {"y": y.detach().numpy(), "s_out": s_out.detach().numpy()}
    for n, name in (("q", "dq"), ("k", "dk"), ("v", "dv"), ("g", "dg"), ("beta", "dbeta")):
        out[name] = leaves[n].grad.numpy()
    out["ds0"] = s0.grad.numpy()
    return out
