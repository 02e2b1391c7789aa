"""The CPU reference of the LoRA training step: the Qwen3.5-architecture model of quotebound_amd/lora.py restated
with torch's own CPU library ops in float32 or float64, its recurrence the oracle's (gdn_ref: the C restatement of
the gated delta rule, forward and hand-written backward) inside an autograd function.

Test infrastructure only: tests/ compare the GPU step with it. It does not round to bf16 anywhere:
given the bf16 base weights' values it computes the step in the arithmetic it is called with.

Ops, each from torch's library rather than restated by hand:
  rms_norm                   F.rms_norm                              src/model.cpp:361, 364; attention q/k :75-76
  causal depthwise conv      F.conv1d(groups=C) on the left-padded sequence, then F.silu   src/deltanet.cpp:74-88
  q/k norm, beta, log-decay  F.rms_norm times 1/Dk, 1/sqrt(Dk) (float32 scalars); torch.sigmoid; -exp(A_log) *
                             F.softplus                              src/deltanet.cpp:22-33, 94-100
  recurrence                 gdn_ref.fwd / gdn_ref.bwd (log-decay)   src/deltanet.cpp:101-119
  gated RMSNorm              F.silu(z) * F.rms_norm(y, weight)       src/deltanet.cpp:35-45, 122
  attention                  F.scaled_dot_product_attention(is_causal) over key/value heads repeated per group,
                             rotate-half rope on the first rope_dims dims, output gate   src/model.cpp:59-99
  MLP                        F.silu(gate) * up                       src/model.cpp:31-39, 366
  loss                       F.cross_entropy (mean) of the tied head's logits at the trained positions
                             src/loss.cpp:10-27; src/train.cpp:247-264
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import gdn_ref


class Recurrence(torch.autograd.Function):
    """y of the gated delta rule from a zero state, g the log-decay; forward and backward by the oracle."""

    @staticmethod
    def forward(ctx, q, k, v, log_decay, beta):
        wide = torch.float64 if q.dtype == torch.float64 else torch.float32  # narrower inputs run in float32
        dt = np.float64 if wide == torch.float64 else np.float32
        host = [t.detach().to(wide).contiguous().numpy() for t in (q, k, v, log_decay, beta)]
        y, _, ckpt = gdn_ref.fwd(*host, None, g_is_log=True, dtype=dt)
        ctx.host, ctx.ckpt, ctx.dt = host, ckpt, dt
        return torch.from_numpy(np.ascontiguousarray(y)).to(q.dtype)

    @staticmethod
    def backward(ctx, dy):
        dyw = dy.detach().to(torch.float64 if ctx.dt == np.float64 else torch.float32).contiguous().numpy()
        grads = gdn_ref.bwd(*ctx.host, ctx.ckpt, dyw, None, g_is_log=True, dtype=ctx.dt)
        return tuple(torch.from_numpy(np.ascontiguousarray(g)).to(dy.dtype) for g in grads[:5])


def _lin(x, w, ad, scale):
    y = F.linear(x, w)
    if ad is not None:
        y = y + scale * F.linear(F.linear(x, ad[0]), ad[1])
    return y


def _rope(x, dims, theta):
    L = x.shape[2]
    freqs = 1.0 / theta ** (torch.arange(0, dims, 2, dtype=torch.float64) / dims)
    ang = (torch.arange(L, dtype=torch.float64)[:, None] * freqs[None, :]).to(x.dtype)
    c, s = torch.cos(ang), torch.sin(ang)
    half = dims // 2
    x1, x2, rest = x[..., :half], x[..., half:dims], x[..., dims:]
    return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c, rest], -1)


def _attention(x, w, p, ads, scale, cfg):
    B, L, _ = x.shape
    hd, H, KV = cfg.head_dim, cfg.heads, cfg.kv_heads
    a = p + "self_attn."
    qg = _lin(x, w[a + "q_proj.weight"], ads.get(a + "q_proj"), scale).view(B, L, H, 2 * hd)
    q, gate = qg[..., :hd], qg[..., hd:].reshape(B, L, H * hd)
    k = _lin(x, w[a + "k_proj.weight"], ads.get(a + "k_proj"), scale).view(B, L, KV, hd)
    v = _lin(x, w[a + "v_proj.weight"], ads.get(a + "v_proj"), scale).view(B, L, KV, hd)
    q = F.rms_norm(q, (hd,), weight=w[a + "q_norm.weight"], eps=cfg.eps).transpose(1, 2)
    k = F.rms_norm(k, (hd,), weight=w[a + "k_norm.weight"], eps=cfg.eps).transpose(1, 2)
    q, k = _rope(q, cfg.rope_dims, cfg.rope_theta), _rope(k, cfg.rope_dims, cfg.rope_theta)
    k = k.repeat_interleave(H // KV, dim=1)
    v = v.transpose(1, 2).repeat_interleave(H // KV, dim=1)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=hd ** -0.5)
    o = o.transpose(1, 2).reshape(B, L, H * hd) * torch.sigmoid(gate)
    return _lin(o, w[a + "o_proj.weight"], ads.get(a + "o_proj"), scale)


def _deltanet(x, w, p, ads, scale, cfg):
    B, S, _ = x.shape
    Hk, Hv, Dk, Dv, K = cfg.lin_k_heads, cfg.lin_v_heads, cfg.lin_k_dim, cfg.lin_v_dim, cfg.conv_kernel
    a = p + "linear_attn."
    qkv = _lin(x, w[a + "in_proj_qkv.weight"], ads.get(a + "in_proj_qkv"), scale)
    z = _lin(x, w[a + "in_proj_z.weight"], ads.get(a + "in_proj_z"), scale).view(B, S, Hv, Dv)
    b = _lin(x, w[a + "in_proj_b.weight"], ads.get(a + "in_proj_b"), scale)
    g_in = _lin(x, w[a + "in_proj_a.weight"], ads.get(a + "in_proj_a"), scale)
    C = qkv.shape[-1]
    conv = F.conv1d(F.pad(qkv.transpose(1, 2), (K - 1, 0)), w[a + "conv1d.weight"].transpose(1, 2), groups=C)
    conv = F.silu(conv.transpose(1, 2))
    kd = Hk * Dk
    q = conv[..., :kd].reshape(B, S, Hk, Dk)
    k = conv[..., kd:2 * kd].reshape(B, S, Hk, Dk)
    v = conv[..., 2 * kd:].reshape(B, S, Hv, Dv)
    inv = float(Dk) ** -0.5
    sq, sk = float(np.float32(inv * inv)), float(np.float32(inv))
    q = sq * F.rms_norm(q, (Dk,), eps=1e-6)
    k = sk * F.rms_norm(k, (Dk,), eps=1e-6)
    beta = torch.sigmoid(b)
    log_decay = -torch.exp(w[a + "A_log"]) * F.softplus(g_in + w[a + "dt_bias"])
    y = Recurrence.apply(q, k, v, log_decay, beta)
    o = F.silu(z) * F.rms_norm(y, (Dv,), weight=w[a + "norm.weight"], eps=cfg.eps)
    return _lin(o.reshape(B, S, Hv * Dv), w[a + "out_proj.weight"], ads.get(a + "out_proj"), scale)


def mean_loss(weights, adapters, tokens, positions, targets, cfg, dtype=torch.float32):
    """The mean cross-entropy at the trained positions. weights: name -> host tensor; adapters as
    quotebound_amd.lora.init_adapters makes them (their tensors used as given, in dtype)."""
    w = {n: t.to(dtype) for n, t in weights.items()}
    ads, scale = adapters["adapters"], adapters["scale"]
    h = F.embedding(tokens, w["model.embed_tokens.weight"])
    for layer in range(cfg.layers):
        p = f"model.layers.{layer}."
        x = F.rms_norm(h, (cfg.hidden,), weight=w[p + "input_layernorm.weight"], eps=cfg.eps)
        mix = _deltanet if cfg.is_linear(layer) else _attention
        r = h + mix(x, w, p, ads, scale, cfg)
        x = F.rms_norm(r, (cfg.hidden,), weight=w[p + "post_attention_layernorm.weight"], eps=cfg.eps)
        m = p + "mlp."
        gate = _lin(x, w[m + "gate_proj.weight"], ads.get(m + "gate_proj"), scale)
        up = _lin(x, w[m + "up_proj.weight"], ads.get(m + "up_proj"), scale)
        h = r + _lin(F.silu(gate) * up, w[m + "down_proj.weight"], ads.get(m + "down_proj"), scale)
    h = F.rms_norm(h, (cfg.hidden,), weight=w["model.norm.weight"], eps=cfg.eps)
    logits = F.linear(h.reshape(-1, cfg.hidden)[positions], w["model.embed_tokens.weight"])
    return F.cross_entropy(logits, targets, reduction="mean")


def loss_and_grads(weights, adapters, tokens, positions, targets, cfg, dtype=torch.float32):
    """(mean loss, gradients of the adapter list: a then b, projection by projection)."""
    names = list(adapters["adapters"])
    params = [t.detach().to(dtype).requires_grad_(True) for n in names for t in adapters["adapters"][n]]
    ads = {"scale": adapters["scale"], "adapters": {n: (params[2 * i], params[2 * i + 1]) for i, n in enumerate(names)}}
    loss = mean_loss(weights, ads, tokens, positions, targets, cfg, dtype)
    grads = torch.autograd.grad(loss, params)
    return loss.detach(), list(grads)
