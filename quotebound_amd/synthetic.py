"""Seeded synthetic inputs for the gated delta rule, with the distributions of the benchmark workloads.

q, k ~ N(0, 1) L2-normalised per (token, head) over Dk; v ~ N(0, 1); log-decay a = -softplus(N(0, 1)) (optionally
clipped to [-8, 0]); beta = sigmoid(N(0, 1)); upstream gradient dy ~ N(0, 1); initial state zero or N(0, s0_std).
The inputs the reference's model feeds the recurrence have the same form: unit-norm keys, beta = sigmoid(b) and
g = exp(-exp(A_log) * softplus(.)) (reference src/deltanet.cpp:22-33, 90-100).

Everything is generated on the host with numpy's PCG64 so the same seed gives the same bits on every machine;
bf16 inputs are rounded to nearest-even once here, and the float32 copies of those bf16 values are what a CPU
check consumes, so both sides see identical inputs.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even. Inputs here are finite."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u >> 16) & 1) + np.uint32(0x7FFF)
    return ((u + r) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(to_bf16_bits(x))


@dataclass
class Workload:
    """Shape and input distribution of one gated-delta call."""

    name: str
    B: int
    T: int
    Hk: int
    Hv: int
    Dk: int
    Dv: int
    dtype: str = "bf16"  # dtype of q, k, v, beta, y, dy and of dq, dk, dv, dbeta ("f32" or "bf16")
    seed: int = 0
    clip_log_decay: float | None = -8.0
    s0_std: float = 0.0  # 0: zero initial state
    ds_out: bool = False  # a cotangent on the final state too
    seq_lens: list[int] | None = None  # packed sequences (B == 1, T == sum)
    chunk: int = 64

    @property
    def cu_seqlens(self) -> np.ndarray | None:
        if self.seq_lens is None:
            return None
        return np.concatenate([[0], np.cumsum(self.seq_lens)]).astype(np.int32)

    @property
    def n_states(self) -> int:
        return len(self.seq_lens) if self.seq_lens is not None else self.B

    @property
    def tokens(self) -> int:
        return self.B * self.T


@dataclass
class Inputs:
    """Host arrays. f32 holds float32 copies (bf16-rounded where the dtype is bf16); bits holds the bf16 patterns."""

    w: Workload
    f32: dict = field(default_factory=dict)
    bits: dict = field(default_factory=dict)


def _normal(rng, shape):
    return rng.standard_normal(size=shape, dtype=np.float32)


def _softplus(x):
    return np.logaddexp(x, np.float32(0)).astype(np.float32)


def make_inputs(w: Workload) -> Inputs:
    rng = np.random.default_rng(w.seed)
    B, T, Hk, Hv, Dk, Dv = w.B, w.T, w.Hk, w.Hv, w.Dk, w.Dv
    q = _normal(rng, (B, T, Hk, Dk))
    k = _normal(rng, (B, T, Hk, Dk))
    q /= np.maximum(np.linalg.norm(q, axis=-1, keepdims=True), np.float32(1e-6))
    k /= np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), np.float32(1e-6))
    v = _normal(rng, (B, T, Hv, Dv))
    a = -_softplus(_normal(rng, (B, T, Hv)))
    if w.clip_log_decay is not None:
        a = np.clip(a, np.float32(w.clip_log_decay), np.float32(0)).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-_normal(rng, (B, T, Hv))))).astype(np.float32)
    dy = _normal(rng, (B, T, Hv, Dv))
    N = w.n_states
    s0 = (_normal(rng, (N, Hv, Dv, Dk)) * np.float32(w.s0_std)) if w.s0_std > 0 else None
    ds_out = _normal(rng, (N, Hv, Dv, Dk)) if w.ds_out else None

    out = Inputs(w)
    for name, x in (("q", q), ("k", k), ("v", v), ("beta", beta), ("dy", dy)):
        if w.dtype == "bf16":
            out.bits[name] = to_bf16_bits(x)
            out.f32[name] = bf16_bits_to_f32(out.bits[name]).reshape(x.shape)
        else:
            out.f32[name] = np.ascontiguousarray(x)
    out.f32["g"] = np.ascontiguousarray(a)  # log-decay, always float32
    out.f32["s0"] = s0
    out.f32["ds_out"] = ds_out
    return out


def varlen_lengths(seed: int, n: int = 8, lo: int = 256, hi: int = 2048) -> list[int]:
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=n)]


def workload(name: str) -> Workload:
    """The named workloads: the tiny fp32 case, the Qwen3.5-4B and -9B layer shapes, the packed batch, the 4B shape
    with float32 activations, and qwen35_4b_t<T>, the 4B head shape at T tokens."""
    if name == "tiny":
        return Workload("tiny", 1, 64, 2, 2, 32, 32, dtype="f32", seed=0, clip_log_decay=None)
    if name == "qwen35_4b":
        return Workload("qwen35_4b", 1, 4096, 16, 32, 128, 128, seed=1)
    if name == "qwen35_9b":
        return Workload("qwen35_9b", 1, 4096, 16, 48, 128, 128, seed=2, s0_std=0.02)
    if name == "qwen35_4b_varlen":
        lens = varlen_lengths(3)
        return Workload("qwen35_4b_varlen", 1, sum(lens), 16, 32, 128, 128, seed=3, seq_lens=lens)
    if name == "qwen35_4b_f32":  # the 4B layer shape with float32 activations, the reference op's own dtype
        return Workload("qwen35_4b_f32", 1, 4096, 16, 32, 128, 128, dtype="f32", seed=1)
    if name.startswith("qwen35_4b_t") and name[11:].isdigit():  # the 4B head shape at T tokens (the T sweep)
        T = int(name[11:])
        return Workload(name, 1, T, 16, 32, 128, 128, seed=40 + T)
    raise KeyError(name)


WORKLOADS = ("tiny", "qwen35_4b", "qwen35_9b", "qwen35_4b_varlen", "qwen35_4b_f32")


def to_device(inp: Inputs, device="cuda"):
    """torch tensors on device: bf16 inputs from their exact bit patterns, g and states in float32."""
    import torch

    out = {}
    for name in ("q", "k", "v", "beta", "dy"):
        if name in inp.bits:
            t = torch.from_numpy(inp.bits[name].view(np.int16).reshape(inp.f32[name].shape))
            out[name] = t.view(torch.bfloat16).to(device)
        else:
            out[name] = torch.from_numpy(inp.f32[name]).to(device)
    for name in ("g", "s0", "ds_out"):
        x = inp.f32.get(name)
        out[name] = None if x is None else torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(device)
    return out
