"""On-disk formats around the LoRA step, as the reference writes them (safetensors; reference src/lora.cpp:58-145,
src/train.cpp:125-200, 341-383):

  <dir>/adapters.safetensors   every adapter array, float32, named model.layers.<l>.<projection>.lora_a / .lora_b
  <dir>/adapter_config.json    rank, alpha, seed, step, dev_loss (null when unknown), targets, model_type, layers,
                               hidden, adapters_sha256 (of adapters.safetensors), base, run
  <dir>/state.safetensors      the training state: p.<name>, m.<name>, v.<name> (adapter and AdamW moments, float32)
                               per adapter array, plus any extra int32 arrays (the trainer's batch plan); string
                               metadata step, opt_step, run and the caller's other fields
  <dir>/state.prev.safetensors the state before the last save: a state that will not read falls back to it

Each file is written under a temporary name and renamed into place, so a crash leaves the old file or the new one.
Reading checks what the reference checks: the sha256 of the adapters, the model they are for, every name present
with its shape and float32 dtype and no unexpected one, the run key of a state, and optimizer step == step.
"""
from __future__ import annotations

import hashlib
import json
import math
import os

import torch
from safetensors import SafetensorError, safe_open
from safetensors.torch import load_file, save_file

from . import lora


class Unreadable(RuntimeError):
    """A state file that cannot be read (missing, torn, or lacking a field): the caller may fall back."""


def adapter_names(adapters: dict) -> list:
    """The saved names of the adapter list, a then b per projection (src/lora.cpp:58-65)."""
    return [n + suffix for n in adapters["adapters"] for suffix in (".lora_a", ".lora_b")]


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def _commit(tmp, path):
    os.replace(tmp, path)


def _host_f32(t):
    return t.detach().to(device="cpu", dtype=torch.float32).contiguous()


def save_adapters(out_dir, cfg: lora.Config, adapters: dict, *, rank, alpha, seed=0, targets=lora.LORA_TARGETS,
                  step=0, dev_loss=float("nan"), model_type="qwen3_5", base=None, run=None) -> str:
    """Writes adapters.safetensors and adapter_config.json (src/lora.cpp:77-100); returns the adapters' sha256."""
    os.makedirs(out_dir, exist_ok=True)
    arrays = dict(zip(adapter_names(adapters), (_host_f32(t) for t in lora.adapter_list(adapters))))
    tmp = os.path.join(out_dir, "adapters.tmp.safetensors")
    save_file(arrays, tmp)
    sha = _sha256(tmp)
    _commit(tmp, os.path.join(out_dir, "adapters.safetensors"))
    config = {"rank": int(rank), "alpha": float(alpha), "seed": int(seed), "step": int(step),
              "dev_loss": None if not math.isfinite(dev_loss) else float(dev_loss), "targets": list(targets),
              "model_type": model_type, "layers": cfg.layers, "hidden": cfg.hidden, "adapters_sha256": sha,
              "base": base if base is not None else {}, "run": run if run is not None else {}}
    tmp = os.path.join(out_dir, "adapter_config.tmp.json")
    with open(tmp, "w") as f:
        json.dump(config, f, indent=1)
        f.write("\n")
    _commit(tmp, os.path.join(out_dir, "adapter_config.json"))
    return sha


def load_adapters(out_dir, cfg: lora.Config, weights: dict, *, model_type="qwen3_5", base=None):
    """Reads adapters written by save_adapters into a fresh adapter set for (cfg, weights) (src/lora.cpp:102-145).
    Returns (adapters as float32 host tensors, config dict). Raises RuntimeError naming what does not fit."""
    path = os.path.join(out_dir, "adapter_config.json")
    with open(path) as f:
        c = json.load(f)
    if c["model_type"] != model_type or c["layers"] != cfg.layers or c["hidden"] != cfg.hidden:
        raise RuntimeError(f"{path}: the adapters are for another model (model_type, layers or hidden differ)")
    if base is not None and c.get("base") != base:
        raise RuntimeError(f"{path}: the adapters were trained on another base checkpoint")
    file = os.path.join(out_dir, "adapters.safetensors")
    if _sha256(file) != c["adapters_sha256"]:
        raise RuntimeError(f"{file} is not the file {path} was written with (sha256 differs)")
    fresh = lora.init_adapters(cfg, weights, rank=c["rank"], alpha=c["alpha"], targets=tuple(c["targets"]),
                               seed=c["seed"])
    saved = load_file(file)
    arrays = []
    for name, now in zip(adapter_names(fresh), lora.adapter_list(fresh)):
        if name not in saved:
            raise RuntimeError(f"{file}: missing {name}")
        t = saved.pop(name)
        if t.shape != now.shape or t.dtype != torch.float32:
            raise RuntimeError(f"{file}: {name} has the wrong shape or dtype")
        arrays.append(t)
    if saved:
        raise RuntimeError(f"{file}: unexpected {next(iter(saved))}")
    return lora.with_adapter_list(fresh, arrays), c


def save_state(out_dir, adapters: dict, opt_state: dict, *, step: int, run: str, extra_arrays=None,
               extra_meta=None) -> None:
    """Writes state.safetensors (src/train.cpp:341-372): adapters and AdamW moments by name, extra int32 arrays,
    string metadata; the previous state becomes state.prev.safetensors."""
    os.makedirs(out_dir, exist_ok=True)
    names = adapter_names(adapters)
    params = lora.adapter_list(adapters)
    arrays = {}
    for i, n in enumerate(names):
        arrays["p." + n] = _host_f32(params[i])
        arrays["m." + n] = _host_f32(opt_state["m"][i])
        arrays["v." + n] = _host_f32(opt_state["v"][i])
    for k, a in (extra_arrays or {}).items():
        arrays[k] = torch.as_tensor(a, dtype=torch.int32).contiguous()
    meta = {"step": str(int(step)), "opt_step": str(int(opt_step_of(opt_state))), "run": str(run)}
    meta.update({k: str(v) for k, v in (extra_meta or {}).items()})
    tmp = os.path.join(out_dir, "state.tmp.safetensors")
    state = os.path.join(out_dir, "state.safetensors")
    save_file(arrays, tmp, metadata=meta)
    if os.path.exists(state):
        os.replace(state, os.path.join(out_dir, "state.prev.safetensors"))
    _commit(tmp, state)


def opt_step_of(opt_state: dict) -> int:
    return int(opt_state["step"])


def _read_state(file, adapters: dict, run: str):
    try:
        arrays = load_file(file)
        with safe_open(file, "pt") as f:
            meta = f.metadata() or {}
    except (OSError, SafetensorError, ValueError) as e:
        raise Unreadable(f"{file}: {e}") from None

    def field(k):
        if k not in meta:
            raise Unreadable(f"{file}: no {k}")
        return meta[k]

    def array(k):
        if k not in arrays:
            raise Unreadable(f"{file}: no {k}")
        return arrays[k]

    names = adapter_names(adapters)
    params = [array("p." + n) for n in names]
    m = [array("m." + n) for n in names]
    v = [array("v." + n) for n in names]
    if field("run") != run:
        raise RuntimeError(f"{file} is from a run with other arguments, data or base:\n  saved: {field('run')}\n"
                           f"  now:   {run}")
    for i, now in enumerate(lora.adapter_list(adapters)):
        for a in (params[i], m[i], v[i]):
            if a.shape != now.shape or a.dtype != torch.float32:
                raise RuntimeError(f"{file}: {names[i]} has the wrong shape or dtype")
    step, opt_step = int(field("step")), int(field("opt_step"))
    if opt_step != step:
        raise RuntimeError(f"{file}: step {step} and optimizer step {opt_step} do not fit")
    extra = {k: a for k, a in arrays.items() if not k[:2] in ("p.", "m.", "v.")}
    return (lora.with_adapter_list(adapters, params), {"m": m, "v": v, "step": opt_step}, step, dict(meta), extra)


def load_state(out_dir, adapters: dict, run: str):
    """Reads state.safetensors, or state.prev.safetensors when the former will not read (src/train.cpp:125-200,
    374-383). adapters gives the names and shapes expected. Returns (adapters, opt_state, step, metadata,
    extra arrays), float32 host tensors."""
    state = os.path.join(out_dir, "state.safetensors")
    prev = os.path.join(out_dir, "state.prev.safetensors")
    try:
        return _read_state(state, adapters, run)
    except Unreadable:
        if not os.path.exists(prev):
            raise
        return _read_state(prev, adapters, run)
