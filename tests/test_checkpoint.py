"""The on-disk formats around the LoRA step (quotebound_amd/checkpoint.py): adapters and training state in
safetensors, as the reference writes them (src/lora.cpp:58-145, src/train.cpp:125-200, 341-383).

  * adapters round-trip bit for bit, with the reference's names and config fields; a changed file, another model or
    an unexpected array is refused;
  * resume: N training steps straight equal N/2 steps, the state saved and read into fresh objects, then N/2 more:
    adapters and AdamW moments bit for bit (the reference's property, tests/test_train.cpp:434-473). With the
    newest state torn, the read falls back to state.prev and still ends bit-identical. Another run's state is
    refused. On the CPU the steps take their gradients from the CPU reference; on the GPU, from the library's step.
"""
import json
import os

import pytest
import torch
from safetensors.torch import load_file

from oracle import lora_ref
from quotebound_amd import checkpoint, lora

TINY = lora.Config(hidden=64, layers=4, heads=2, kv_heads=1, head_dim=32, rope_dims=16, rope_theta=1e4,
                   intermediate=128, vocab=97, lin_k_heads=2, lin_v_heads=4, lin_k_dim=32, lin_v_dim=32)


def _same(a, b):
    return all(torch.equal(x.cpu(), y.cpu()) for x, y in zip(a, b))


def test_adapters_round_trip(tmp_path):
    w = lora.init_weights(TINY, seed=3)
    ads = lora.init_adapters(TINY, w, rank=4, alpha=8.0, seed=1, b_std=0.05)
    d = str(tmp_path / "best")
    sha = checkpoint.save_adapters(d, TINY, ads, rank=4, alpha=8.0, seed=1, step=12, dev_loss=2.5)
    saved = load_file(os.path.join(d, "adapters.safetensors"))
    assert sorted(saved) == sorted(checkpoint.adapter_names(ads))
    assert "model.layers.0.linear_attn.in_proj_qkv.lora_a" in saved
    with open(os.path.join(d, "adapter_config.json")) as f:
        c = json.load(f)
    assert c["adapters_sha256"] == sha and c["rank"] == 4 and c["step"] == 12 and c["dev_loss"] == 2.5
    assert c["layers"] == TINY.layers and c["hidden"] == TINY.hidden and c["model_type"] == "qwen3_5"
    back, c2 = checkpoint.load_adapters(d, TINY, w)
    assert _same(lora.adapter_list(back), lora.adapter_list(ads)) and back["scale"] == ads["scale"]
    with pytest.raises(RuntimeError, match="another model"):
        checkpoint.load_adapters(d, lora.Config(hidden=64, layers=8, vocab=97), w)
    with open(os.path.join(d, "adapters.safetensors"), "r+b") as f:  # one byte of the data changed
        f.seek(-1, 2)
        last = f.read(1)
        f.seek(-1, 2)
        f.write(bytes([last[0] ^ 1]))
    with pytest.raises(RuntimeError, match="sha256 differs"):
        checkpoint.load_adapters(d, TINY, w)


def _cpu_step(w, ads, opt, state, batch):
    loss, grads = lora_ref.loss_and_grads(w, ads, *batch, TINY, torch.float32)
    norm = torch.sqrt(sum((g.double() * g.double()).sum() for g in grads)).float()
    new = opt.update(lora.adapter_list(ads), grads, norm, state)
    return lora.with_adapter_list(ads, new)


def _fresh(opt):
    w = lora.init_weights(TINY, seed=3)
    ads = lora.init_adapters(TINY, w, rank=4, alpha=8.0, seed=1)
    return w, ads, opt.init(lora.adapter_list(ads))


def test_resume_is_bit_identical(tmp_path, oracle):
    opt = lora.AdamW(lr=5e-3)
    batches = [lora.last_half_batch(2, 20, TINY.vocab, seed=s) for s in range(4)]
    w, ads, st = _fresh(opt)
    for b in batches:
        ads = _cpu_step(w, ads, opt, st, b)
    d = str(tmp_path / "run")
    w1, a1, s1 = _fresh(opt)
    for i in range(2):
        a1 = _cpu_step(w1, a1, opt, s1, batches[i])
        checkpoint.save_state(d, a1, s1, step=i + 1, run="tiny-run", extra_arrays={"plan": [3, 1, 0, 2]})
    _, template, _ = _fresh(opt)
    a2, s2, step, meta, extra = checkpoint.load_state(d, template, "tiny-run")
    assert step == 2 and meta["opt_step"] == "2" and extra["plan"].tolist() == [3, 1, 0, 2]
    for b in batches[2:]:
        a2 = _cpu_step(w1, a2, opt, s2, b)
    assert _same(lora.adapter_list(a2), lora.adapter_list(ads))
    assert _same(s2["m"], st["m"]) and _same(s2["v"], st["v"])

    # A torn state: the read falls back to state.prev (step 1) and the run still ends bit-identical.
    os.truncate(os.path.join(d, "state.safetensors"), 1024)
    a3, s3, step, _, _ = checkpoint.load_state(d, template, "tiny-run")
    assert step == 1
    for b in batches[1:]:
        a3 = _cpu_step(w1, a3, opt, s3, b)
    assert _same(lora.adapter_list(a3), lora.adapter_list(ads)) and _same(s3["v"], st["v"])

    with pytest.raises(RuntimeError, match="other arguments"):
        checkpoint.load_state(d, template, "another-run")
    os.remove(os.path.join(d, "state.prev.safetensors"))
    with pytest.raises(checkpoint.Unreadable):
        checkpoint.load_state(d, template, "tiny-run")


@pytest.mark.gpu
def test_resume_is_bit_identical_on_the_gpu(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    cfg = lora.Config(hidden=256, layers=4, heads=2, kv_heads=1, head_dim=128, rope_dims=32, intermediate=512,
                      vocab=1000, lin_k_heads=2, lin_v_heads=4, lin_k_dim=128, lin_v_dim=128)
    host = lora.init_weights(cfg, seed=51)
    w = lora.to_device(host, "cuda", torch.bfloat16)
    opt = lora.AdamW(lr=1e-3)
    batches = [tuple(t.cuda() for t in lora.last_half_batch(2, 128, cfg.vocab, seed=60 + i)) for i in range(4)]

    def fresh():
        ads = lora.adapters_to(lora.init_adapters(cfg, host, seed=52), "cuda")
        return ads, opt.init(lora.adapter_list(ads))

    ads, st = fresh()
    for b in batches:
        _, _, ads = lora.train_step(w, ads, opt, st, *b, cfg)
    a1, s1 = fresh()
    for b in batches[:2]:
        _, _, a1 = lora.train_step(w, a1, opt, s1, *b, cfg)
    d = str(tmp_path / "gpu-run")
    checkpoint.save_state(d, a1, s1, step=2, run="gpu-run")
    template, _ = fresh()
    a2, s2, step, _, _ = checkpoint.load_state(d, template, "gpu-run")
    a2 = lora.adapters_to(a2, "cuda")
    s2 = {"m": [t.cuda() for t in s2["m"]], "v": [t.cuda() for t in s2["v"]], "step": s2["step"]}
    for b in batches[2:]:
        _, _, a2 = lora.train_step(w, a2, opt, s2, *b, cfg)
    torch.cuda.synchronize()
    assert step == 2
    assert _same(lora.adapter_list(a2), lora.adapter_list(ads))
    assert _same(s2["m"], st["m"]) and _same(s2["v"], st["v"])
