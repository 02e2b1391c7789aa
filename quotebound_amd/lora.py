"""One LoRA training step of a Qwen3.5-architecture decoder whose Gated DeltaNet layers run this library's kernels.

The model follows the reference's (src/model.cpp:59-99 attention, :359-367 block, :389-407 hidden, :409-412
logits_at; src/deltanet.cpp:63-124 the DeltaNet layer), its adapters src/lora.cpp:25-49 (LoRA linear
src/model.cpp:109-115), its loss src/loss.cpp:10-27 with the mean over trained positions src/train.cpp:247-264, and
its update src/adamw.cpp:17-42. In each DeltaNet layer the prologue (q/k RMSNorm with 1/Dk and 1/sqrt(Dk), beta,
log-decay), the recurrence (chunked, fed the log-decay) and the gated RMSNorm are the library's HIP kernels through
neighbours.py and gdn.py; torch does the projections (hipBLASLt), the causal conv, attention, the MLP and the loss.

Dtypes follow the reference's: frozen base weights in bf16 except the DeltaNet's A_log and gated-norm weight
(float32, as the checkpoints store them); adapters, optimizer state and the low-rank path in float32, added back
in the activations' dtype; logits cast to float32 for the loss. Each op's output takes its inputs' promoted dtype,
as MLX's do. With float32 weights the whole model runs in float32 (the recurrence then takes its float32 design).

Config() is the tiny random-init Qwen3.5 of the LoRA workload: 8 layers repeating 3 Gated DeltaNet : 1 full
attention (every fourth layer and the last are attention, tests/tiny.h:23), hidden 1024, DeltaNet 4 key and 8 value
heads of 128, causal conv of width 4, vocabulary 32000, tied embeddings. The attention layers take tests/tiny.h's
shape scaled to hidden 1024 (4 query heads and 1 key/value head of 256, rope on the first 64 dims, output gate),
and the MLP 2x hidden, as tests/tiny.h does.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import gdn, neighbours


@dataclass(frozen=True)
class Config:
    hidden: int = 1024
    layers: int = 8
    heads: int = 4
    kv_heads: int = 1
    head_dim: int = 256
    rope_dims: int = 64
    rope_theta: float = 1e7
    intermediate: int = 2048
    vocab: int = 32000
    eps: float = 1e-6
    lin_k_heads: int = 4
    lin_v_heads: int = 8
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    conv_kernel: int = 4
    # The DeltaNet layers' prologue fused into the recurrence's kernels (gdn.gated_delta_prologue) where the
    # activations are bf16; else, and for float32 activations, the separate prologue pass then the recurrence.
    fused_prologue: bool = True

    def is_linear(self, layer: int) -> bool:
        """Gated DeltaNet (else full attention): every fourth layer and the last are attention (tests/tiny.h:23)."""
        return layer % 4 != 3 and layer != self.layers - 1


# "LoRA on q/k/v/o": attention's four projections, and the DeltaNet's input and output projections
# (the projection names of src/lora.cpp:19-23).
LORA_TARGETS = ("q_proj", "k_proj", "v_proj", "o_proj", "in_proj_qkv", "out_proj")
FLOAT32_WEIGHTS = (".linear_attn.A_log", ".linear_attn.norm.weight")  # float32 in the checkpoints


def _bf16_values(t):
    return t.to(torch.bfloat16).float()


def init_weights(cfg: Config, seed: int = 7) -> dict:
    """Random weights with the distributions of the reference's test models (tests/tiny.h:24-66), as float32 host
    tensors holding the values of the dtype each is stored in (bf16, or float32 for FLOAT32_WEIGHTS)."""
    g = torch.Generator().manual_seed(seed)

    def rnd(shape, mean, sd):
        return torch.randn(shape, generator=g) * sd + mean

    def lin(out, inp):
        return rnd((out, inp), 0.0, 1.0 / math.sqrt(inp))

    def norm(n):
        return rnd((n,), 1.0, 0.1)

    q, kv = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    kd, vd = cfg.lin_k_heads * cfg.lin_k_dim, cfg.lin_v_heads * cfg.lin_v_dim
    conv = 2 * kd + vd
    w = {"model.embed_tokens.weight": rnd((cfg.vocab, cfg.hidden), 0.0, 1.0 / math.sqrt(cfg.hidden)),
         "model.norm.weight": norm(cfg.hidden)}
    for layer in range(cfg.layers):
        p = f"model.layers.{layer}."
        w[p + "input_layernorm.weight"] = norm(cfg.hidden)
        w[p + "post_attention_layernorm.weight"] = norm(cfg.hidden)
        w[p + "mlp.gate_proj.weight"] = lin(cfg.intermediate, cfg.hidden)
        w[p + "mlp.up_proj.weight"] = lin(cfg.intermediate, cfg.hidden)
        w[p + "mlp.down_proj.weight"] = lin(cfg.hidden, cfg.intermediate)
        if cfg.is_linear(layer):
            a = p + "linear_attn."
            w[a + "in_proj_qkv.weight"] = lin(conv, cfg.hidden)
            w[a + "in_proj_z.weight"] = lin(vd, cfg.hidden)
            w[a + "in_proj_b.weight"] = lin(cfg.lin_v_heads, cfg.hidden)
            w[a + "in_proj_a.weight"] = lin(cfg.lin_v_heads, cfg.hidden)
            w[a + "conv1d.weight"] = rnd((conv, cfg.conv_kernel, 1), 0.0, 0.5)
            w[a + "dt_bias"] = rnd((cfg.lin_v_heads,), 1.0, 0.1)
            w[a + "A_log"] = torch.log(torch.rand(cfg.lin_v_heads, generator=g) * 15.0 + 1.0)
            w[a + "norm.weight"] = rnd((cfg.lin_v_dim,), 1.0, 0.1)
            w[a + "out_proj.weight"] = lin(cfg.hidden, vd)
        else:
            a = p + "self_attn."
            w[a + "q_proj.weight"] = lin(2 * q, cfg.hidden)  # [query | gate] per head
            w[a + "k_proj.weight"] = lin(kv, cfg.hidden)
            w[a + "v_proj.weight"] = lin(kv, cfg.hidden)
            w[a + "o_proj.weight"] = lin(cfg.hidden, q)
            w[a + "q_norm.weight"] = norm(cfg.head_dim)
            w[a + "k_norm.weight"] = norm(cfg.head_dim)
    return {n: (t if n.endswith(FLOAT32_WEIGHTS) else _bf16_values(t)) for n, t in w.items()}


def to_device(weights: dict, device="cuda", dtype=torch.bfloat16) -> dict:
    """The frozen weights on the device: dtype (bf16, or float32 for a float32 model), FLOAT32_WEIGHTS float32."""
    return {n: t.to(device=device, dtype=torch.float32 if n.endswith(FLOAT32_WEIGHTS) else dtype)
            for n, t in weights.items()}


def projection_names(cfg: Config, layer: int) -> list:
    """A layer's projections in the reference's fixed order (src/model.cpp:320-331), without ".weight"."""
    p = f"model.layers.{layer}."
    if cfg.is_linear(layer):
        mixer = [p + "linear_attn." + n for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj")]
    else:
        mixer = [p + "self_attn." + n for n in ("q_proj", "k_proj", "v_proj", "o_proj")]
    return mixer + [p + "mlp." + n for n in ("gate_proj", "up_proj", "down_proj")]


def init_adapters(cfg: Config, weights: dict, *, rank=16, alpha=32.0, targets=LORA_TARGETS, seed=0,
                  b_std=0.0) -> dict:
    """Adapters on every projection whose short name is a target, in model order (src/lora.cpp:25-49):
    a ~ U(-1/sqrt(in), 1/sqrt(in)) [rank, in], b = 0 [out, rank], float32 host tensors; scale = alpha / rank.
    b_std > 0 draws b ~ N(0, b_std) instead, so the low-rank path and the gradient through a are live (the
    reference's tests do this, tests/test_train.cpp:50-57)."""
    if rank < 1:
        raise ValueError("LoRA rank must be at least 1")
    g = torch.Generator().manual_seed(seed)
    out = {}
    for layer in range(cfg.layers):
        for name in projection_names(cfg, layer):
            if name.rsplit(".", 1)[1] not in targets:
                continue
            n_out, n_in = weights[name + ".weight"].shape
            bound = 1.0 / math.sqrt(n_in)
            a = (torch.rand((rank, n_in), generator=g) * 2.0 - 1.0) * bound
            b = torch.randn((n_out, rank), generator=g) * b_std if b_std > 0 else torch.zeros(n_out, rank)
            out[name] = (a, b)
    if not out:
        raise ValueError("no projection of this model is a LoRA target")
    return {"scale": alpha / rank, "adapters": out}


def adapter_list(adapters: dict) -> list:
    """a then b, projection by projection, layer by layer (src/model.cpp:339-344; src/lora.cpp:51-56)."""
    return [t for ab in adapters["adapters"].values() for t in ab]


def with_adapter_list(adapters: dict, arrays) -> dict:
    names = list(adapters["adapters"])
    if len(arrays) != 2 * len(names):
        raise ValueError("adapter list length does not match the adapters")
    return {"scale": adapters["scale"],
            "adapters": {n: (arrays[2 * i], arrays[2 * i + 1]) for i, n in enumerate(names)}}


def adapters_to(adapters: dict, device) -> dict:
    return with_adapter_list(adapters, [t.to(device=device, dtype=torch.float32) for t in adapter_list(adapters)])


# ---- the model ----------------------------------------------------------------------------------------------------


def rms_norm(x, w, eps):
    """MLX fast::rms_norm: normalise in float32 (or x's dtype when wider), cast to the promoted dtype of x and w,
    times w."""
    xf = x.to(torch.promote_types(x.dtype, torch.float32))
    n = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
    dt = torch.promote_types(x.dtype, w.dtype)
    return n.to(dt) * w.to(dt)


def linear(x, w, ad=None, scale=1.0):
    """x W^T, plus the adapter's scale (x A^T) B^T in float32 added back in x W^T's dtype (src/model.cpp:109-115)."""
    y = F.linear(x, w)
    if ad is None:
        return y
    z = F.linear(F.linear(x.float(), ad[0]), ad[1])
    return y + (z * scale).to(y.dtype)


def silu(x):
    return x * torch.sigmoid(x)  # each op rounds to x's dtype, as the reference's compiled silu


def rope(x, dims, theta):
    """Rotate-half rope on the first `dims` of each head (mx::fast::rope, traditional=false), positions from 0;
    x [B, H, L, D], computed in float32 (or x's dtype when wider) and cast back."""
    L = x.shape[2]
    ct = torch.promote_types(x.dtype, torch.float32)
    inv = theta ** (-torch.arange(0, dims, 2, dtype=ct, device=x.device) / dims)
    ang = torch.arange(L, dtype=ct, device=x.device)[:, None] * inv[None, :]
    cos, sin = torch.cos(ang), torch.sin(ang)
    xr = x[..., :dims].to(ct)
    x1, x2 = xr[..., : dims // 2], xr[..., dims // 2:]
    rot = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1).to(x.dtype)
    return torch.cat([rot, x[..., dims:]], -1)


def causal_conv(x, w):
    """Depthwise causal conv over time (src/deltanet.cpp:74-88 without a cache): out[t] = sum_j w[:, j] x[t - K + 1
    + j], zeros before the start, accumulated in float32 (or x's dtype when wider) and cast to x's dtype.
    x [B, S, C], w [C, K, 1]."""
    K, S = w.shape[1], x.shape[1]
    ct = torch.promote_types(x.dtype, torch.float32)
    xp = F.pad(x, (0, 0, K - 1, 0)).to(ct)
    wf = w[:, :, 0].to(ct)
    acc = xp[:, 0:S] * wf[:, 0]
    for j in range(1, K):
        acc = acc + xp[:, j:j + S] * wf[:, j]
    return acc.to(x.dtype)


def attention(x, w, p, ads, scale, cfg):
    """src/model.cpp:59-99 without a cache: q_proj holds [query | gate] per head; q/k RMSNorm, rope, causal
    attention (float32 inside), output gate, o_proj."""
    B, L, _ = x.shape
    hd, H, KV = cfg.head_dim, cfg.heads, cfg.kv_heads
    a = p + "self_attn."
    qg = linear(x, w[a + "q_proj.weight"], ads.get(a + "q_proj"), scale).view(B, L, H, 2 * hd)
    q, gate = qg[..., :hd], qg[..., hd:].reshape(B, L, H * hd)
    k = linear(x, w[a + "k_proj.weight"], ads.get(a + "k_proj"), scale).view(B, L, KV, hd)
    v = linear(x, w[a + "v_proj.weight"], ads.get(a + "v_proj"), scale).view(B, L, KV, hd)
    q = rope(rms_norm(q, w[a + "q_norm.weight"], cfg.eps).transpose(1, 2), cfg.rope_dims, cfg.rope_theta)
    k = rope(rms_norm(k, w[a + "k_norm.weight"], cfg.eps).transpose(1, 2), cfg.rope_dims, cfg.rope_theta)
    v = v.transpose(1, 2)
    qf = q.float()
    kf = k.float().repeat_interleave(H // KV, dim=1)
    vf = v.float().repeat_interleave(H // KV, dim=1)
    s = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * (hd ** -0.5)
    causal = torch.ones(L, L, dtype=torch.bool, device=x.device).triu(1)
    prob = torch.softmax(s.masked_fill(causal, float("-inf")), dim=-1)
    o = torch.matmul(prob, vf).to(x.dtype).transpose(1, 2).reshape(B, L, H * hd)
    o = o * torch.sigmoid(gate)
    return linear(o, w[a + "o_proj.weight"], ads.get(a + "o_proj"), scale)


def deltanet(x, w, p, ads, scale, cfg):
    """src/deltanet.cpp:63-124 without a cache, training form: projections, causal conv + SiLU, the library's
    prologue and recurrence (one fused call on bf16 activations), its gated RMSNorm, out_proj."""
    B, S, _ = x.shape
    Hk, Hv, Dk, Dv = cfg.lin_k_heads, cfg.lin_v_heads, cfg.lin_k_dim, cfg.lin_v_dim
    kd = Hk * Dk
    a = p + "linear_attn."
    qkv = linear(x, w[a + "in_proj_qkv.weight"], ads.get(a + "in_proj_qkv"), scale)
    z = linear(x, w[a + "in_proj_z.weight"], ads.get(a + "in_proj_z"), scale).view(B, S, Hv, Dv)
    b = linear(x, w[a + "in_proj_b.weight"], ads.get(a + "in_proj_b"), scale)
    g_in = linear(x, w[a + "in_proj_a.weight"], ads.get(a + "in_proj_a"), scale)
    conv = silu(causal_conv(qkv, w[a + "conv1d.weight"]))
    q_raw = conv[..., :kd].reshape(B, S, Hk, Dk)
    k_raw = conv[..., kd:2 * kd].reshape(B, S, Hk, Dk)
    v = conv[..., 2 * kd:].reshape(B, S, Hv, Dv)
    if cfg.fused_prologue and x.dtype == torch.bfloat16:
        y, _ = gdn.gated_delta_prologue(q_raw, k_raw, v, g_in, b, w[a + "A_log"], w[a + "dt_bias"], None)
    else:
        q, k, beta, log_decay = neighbours.prologue(q_raw, k_raw, g_in, b, w[a + "A_log"], w[a + "dt_bias"])
        y, _ = gdn.gated_delta_trainable(q, k, v, log_decay, beta, None, log_decay=True)
    o = neighbours.epilogue(y, z, w[a + "norm.weight"], cfg.eps)
    return linear(o.reshape(B, S, Hv * Dv), w[a + "out_proj.weight"], ads.get(a + "out_proj"), scale)


def block(h, w, layer, ads, scale, cfg):
    """src/model.cpp:359-367."""
    p = f"model.layers.{layer}."
    x = rms_norm(h, w[p + "input_layernorm.weight"], cfg.eps)
    mix = deltanet if cfg.is_linear(layer) else attention
    r = h + mix(x, w, p, ads, scale, cfg)
    x = rms_norm(r, w[p + "post_attention_layernorm.weight"], cfg.eps)
    m = p + "mlp."
    gate = linear(x, w[m + "gate_proj.weight"], ads.get(m + "gate_proj"), scale)
    up = linear(x, w[m + "up_proj.weight"], ads.get(m + "up_proj"), scale)
    return r + linear(silu(gate) * up, w[m + "down_proj.weight"], ads.get(m + "down_proj"), scale)


def hidden(w, adapters, tokens, cfg):
    """src/model.cpp:389-407 without layer checkpoints (HBM holds every activation): the final normed hidden
    states [B, L, hidden]."""
    ads, scale = adapters["adapters"], adapters["scale"]
    h = F.embedding(tokens, w["model.embed_tokens.weight"])
    for layer in range(cfg.layers):
        h = block(h, w, layer, ads, scale, cfg)
    return rms_norm(h, w["model.norm.weight"], cfg.eps)


def mean_loss(w, adapters, tokens, positions, targets, cfg):
    """The mean over trained positions of the cross-entropy of the float32 logits (tied head), src/loss.cpp:10-27
    and src/train.cpp:247-264; positions index the flattened [B, L] rows, targets the next tokens."""
    h = hidden(w, adapters, tokens, cfg)
    rows = h.reshape(-1, cfg.hidden)[positions]
    logits = F.linear(rows, w["model.embed_tokens.weight"]).float()
    picked = logits.gather(1, targets[:, None])[:, 0]
    return (torch.logsumexp(logits, -1) - picked).sum() / positions.shape[0]


def loss_and_grads(w, adapters, tokens, positions, targets, cfg):
    """(mean loss, gradients of the adapter list, their global norm), src/train.cpp:247-264."""
    params = [t.detach().requires_grad_(True) for t in adapter_list(adapters)]
    loss = mean_loss(w, with_adapter_list(adapters, params), tokens, positions, targets, cfg)
    grads = torch.autograd.grad(loss, params)
    # The global norm in float32 (src/adamw.cpp:17-21), from one multi-tensor launch of per-array norms.
    norm = torch.linalg.vector_norm(torch.stack(torch._foreach_norm(grads)))
    return loss.detach(), list(grads), norm


@dataclass
class AdamW:
    """src/adamw.h:8-12 and src/adamw.cpp:17-42: global-norm clipping, bias-corrected moments, decoupled decay."""
    lr: float = 1e-4
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.0
    clip: float = 1.0

    def init(self, params):
        return {"m": [torch.zeros_like(p) for p in params], "v": [torch.zeros_like(p) for p in params], "step": 0}

    def update(self, params, grads, norm, state):
        coef = torch.clamp(self.clip / (norm + 1e-6), max=1.0) if self.clip > 0 else None
        state["step"] += 1
        bc1 = 1.0 - self.beta1 ** state["step"]
        bc2_sqrt = math.sqrt(1.0 - self.beta2 ** state["step"])
        out = []
        for i, (p, g) in enumerate(zip(params, grads)):
            if coef is not None:
                g = g * coef
            state["m"][i] = self.beta1 * state["m"][i] + (1.0 - self.beta1) * g
            state["v"][i] = self.beta2 * state["v"][i] + (1.0 - self.beta2) * g * g
            q = p * (1.0 - self.lr * self.weight_decay)
            denom = torch.sqrt(state["v"][i]) / bc2_sqrt + self.eps
            out.append(q - (self.lr / bc1) * (state["m"][i] / denom))
        return out


def adamw_update_(opt: AdamW, params, grads, norm, m, v, count):
    """opt's update in place on device tensors, its step count a device scalar (count), so that the update can be
    captured in a graph and replayed: the bias corrections are computed on the device from the count."""
    count.add_(1.0)
    bc1 = 1.0 - torch.pow(opt.beta1, count)
    bc2_sqrt = torch.sqrt(1.0 - torch.pow(opt.beta2, count))
    g = list(grads)
    if opt.clip > 0:  # one multi-tensor launch per op over all adapter arrays instead of one per array
        g = torch._foreach_mul(g, torch.clamp(opt.clip / (norm + 1e-6), max=1.0))
    torch._foreach_mul_(m, opt.beta1)
    torch._foreach_add_(m, g, alpha=1.0 - opt.beta1)
    torch._foreach_mul_(v, opt.beta2)
    torch._foreach_addcmul_(v, g, g, value=1.0 - opt.beta2)
    torch._foreach_mul_(params, 1.0 - opt.lr * opt.weight_decay)
    denom = torch._foreach_sqrt(v)
    torch._foreach_div_(denom, bc2_sqrt)
    torch._foreach_add_(denom, opt.eps)
    step = torch._foreach_div(m, denom)
    torch._foreach_mul_(step, opt.lr / bc1)
    torch._foreach_sub_(params, step)


class GraphStep:
    """The training step (loss, adapter gradients, AdamW) on static device tensors: the adapters, the moments and
    the step count are updated in place, and each call copies its batch into static inputs. With capture=True the
    step is recorded once in a HIP graph (torch.cuda.graph) and each call replays it, so the ~1,500 launches of a
    step cost one; with capture=False each call runs the same step eagerly. example = (tokens, positions, targets)
    fixes the batch shapes."""

    def __init__(self, w, adapters, opt: AdamW, cfg: Config, example, capture=True, warmup=2):
        self.w, self.opt, self.cfg, self.scale = w, opt, cfg, adapters["scale"]
        self.names = list(adapters["adapters"])
        self.params = [t.detach().clone() for t in adapter_list(adapters)]
        self.m = [torch.zeros_like(p) for p in self.params]
        self.v = [torch.zeros_like(p) for p in self.params]
        self.count = torch.zeros((), dtype=torch.float32, device=self.params[0].device)
        self.inputs = [t.clone() for t in example]
        self.graph = None
        if not capture:
            return
        start = [t.clone() for t in self.params + self.m + self.v + [self.count]]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # the first runs set up libraries and the allocator outside the capture
            for _ in range(warmup):
                self._step()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = self._step()
        for t, s0 in zip(self.params + self.m + self.v + [self.count], start):  # undo the warm-up steps
            t.copy_(s0)

    def _step(self):
        ads = {"scale": self.scale,
               "adapters": {n: (self.params[2 * i], self.params[2 * i + 1]) for i, n in enumerate(self.names)}}
        loss, grads, norm = loss_and_grads(self.w, ads, *self.inputs, self.cfg)
        adamw_update_(self.opt, self.params, grads, norm, self.m, self.v, self.count)
        return loss, norm

    def __call__(self, tokens, positions, targets):
        """One step on this batch; returns (loss, gradient norm) as device scalars (overwritten by the next call
        when captured)."""
        for dst, src in zip(self.inputs, (tokens, positions, targets)):
            dst.copy_(src)
        if self.graph is None:
            return self._step()
        self.graph.replay()
        return self.out

    def adapters(self) -> dict:
        return {"scale": self.scale,
                "adapters": {n: (self.params[2 * i], self.params[2 * i + 1]) for i, n in enumerate(self.names)}}


def train_step(w, adapters, opt: AdamW, opt_state, tokens, positions, targets, cfg):
    """One step: loss and adapter gradients, then the AdamW update. Returns (loss, norm, new adapters)."""
    loss, grads, norm = loss_and_grads(w, adapters, tokens, positions, targets, cfg)
    new = opt.update(adapter_list(adapters), grads, norm, opt_state)
    return loss, norm, with_adapter_list(adapters, new)


def last_half_batch(batch: int, seq: int, vocab: int, seed: int = 0, device="cpu"):
    """The LoRA workload's batch: `batch` sequences of `seq` uniform-random token ids, the loss on the last half
    (targets tokens seq/2 .. seq-1, predicted from the position before each). Returns (tokens [B, L] int64,
    positions [N] into the flattened rows, targets [N])."""
    g = torch.Generator().manual_seed(seed)
    tokens = torch.randint(0, vocab, (batch, seq), generator=g)
    t = torch.arange(seq // 2 - 1, seq - 1)
    positions = (torch.arange(batch)[:, None] * seq + t[None, :]).reshape(-1)
    targets = tokens[:, seq // 2:].reshape(-1)
    return tokens.to(device), positions.to(device), targets.to(device)


def main(argv=None) -> None:
    """python -m quotebound_amd.lora [--steps K] [--warmup W] [--graph]: the LoRA workload's training step (the
    default Config, bf16 base, 4 sequences of 1024 random tokens, loss on the last half) on cuda:0, timed over K
    steps after W; prints one JSON line."""
    import argparse
    import json
    import time

    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--graph", action="store_true", help="replay the step from a captured HIP graph")
    args = ap.parse_args(argv)
    cfg = Config()
    host = init_weights(cfg, seed=31)
    w = to_device(host, "cuda", torch.bfloat16)
    ads = adapters_to(init_adapters(cfg, host, seed=32, b_std=0.05), "cuda")
    batch = tuple(t.cuda() for t in last_half_batch(4, 1024, cfg.vocab, seed=33))
    step = GraphStep(w, ads, AdamW(lr=1e-4), cfg, batch, capture=args.graph)
    for _ in range(args.warmup):
        step(*batch)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss, norm = step(*batch)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    print(json.dumps({"ms_per_step": ms, "tokens_per_s": 4 * 1024 / (ms * 1e-3), "loss": float(loss),
                      "grad_norm": float(norm), "graph": args.graph}))


if __name__ == "__main__":
    main()

