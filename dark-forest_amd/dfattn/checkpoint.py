"""StaticGPT2 checkpoints in the reference engine's two formats.

* The engine's own binary checkpoint (darkforest-core/src/engine/static_gpt2.rs:1924-2114):
  every tensor as a little-endian u64 element count followed by that many little-endian f32
  values; first the weights (tok_emb, pos_emb, ln_f gamma and beta, lm_head, then per layer
  ln1 gamma/beta, Wq, bq, Wk, bk, Wv, bv, Wo, bo, ln2 gamma/beta, W1, b1, W2, b2), then the AdamW
  moments m and v of each weight in the same order, then a footer: step count (u64) and lr,
  beta1, beta2, eps, weight decay (f32 each). Loading checks every element count against the
  model and fails on a short file, as load_checkpoint does.
* GPT-2 safetensors (darkforest-core/src/engine/safetensors.rs:156-373): export under the names
  and shapes save_gpt2_safetensors writes (transformer.* plus lm_head.weight, Q/K/V packed row by
  row into c_attn [d_model, 3 d_model]); import looks each name up bare, then with the
  "transformer." and "model." prefixes, splits c_attn by its shape ([d_model, 3 d_model] row by row,
  otherwise three consecutive blocks), falls back to wte for a missing lm_head and leaves tensors
  the file lacks untouched. Weights keep the engine's [out, in] layout in both directions, as the
  reference's setters and getters copy the data unchanged.

Host-side file I/O only: weights move through host memory with one copy per tensor.
"""
from __future__ import annotations

import json
import struct

import numpy as np

_LAYER_KEYS = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1", "b1",
               "w2", "b2")


def _torch():
    import torch

    return torch


def ordered_weights(model):
    """The weights in the order static_gpt2.rs:1947-1975 writes them."""
    out = [model.tok_emb, model.pos_emb, model.ln_f_g, model.ln_f_b, model.lm_head]
    for lw in model.layers:
        out += [lw[k] for k in _LAYER_KEYS]
    return out


def _host_f32(t) -> np.ndarray:
    return np.ascontiguousarray(t.detach().to("cpu", _torch().float32).numpy().reshape(-1), dtype="<f4")


def _write_tensor(f, values: np.ndarray) -> None:
    f.write(struct.pack("<Q", values.size))
    f.write(values.tobytes())


def _read_exact(f, n: int) -> bytes:
    b = f.read(n)
    if len(b) != n:
        raise ValueError(f"load_checkpoint: file ends early (wanted {n} bytes, got {len(b)})")
    return b


def _read_tensor(f, numel: int) -> np.ndarray:
    (n,) = struct.unpack("<Q", _read_exact(f, 8))
    if n != numel:
        raise ValueError(f"load_checkpoint: tensor size mismatch: file={n} model={numel}")
    return np.frombuffer(_read_exact(f, 4 * n), dtype="<f4")


def _adam_group(model):
    groups = model.opt.param_groups
    if len(groups) != 1:
        raise ValueError("checkpoint: StaticGPT2 keeps one AdamW parameter group")
    return groups[0]


def step_count(model) -> int:
    """AdamW steps taken (0 before the first)."""
    for p in model.parameters():
        st = model.opt.state.get(p)
        if st and "step" in st:
            return int(float(st["step"]))
    return 0


def save_checkpoint(model, path) -> None:
    """static_gpt2.rs:1924-2004: weights, AdamW moments, footer."""
    weights = ordered_weights(model)
    g = _adam_group(model)
    with open(path, "wb") as f:
        for w in weights:
            _write_tensor(f, _host_f32(w))
        for w in weights:
            st = model.opt.state.get(w, {})
            for key in ("exp_avg", "exp_avg_sq"):
                m = st.get(key)
                _write_tensor(f, _host_f32(m) if m is not None else np.zeros(w.numel(), "<f4"))
        b1, b2 = g["betas"]
        f.write(struct.pack("<Q", step_count(model)))
        f.write(struct.pack("<5f", g["lr"], b1, b2, g["eps"], g["weight_decay"]))


def load_checkpoint(model, path) -> None:
    """static_gpt2.rs:2010-2114: the model must have the checkpoint's dimensions."""
    torch = _torch()
    weights = ordered_weights(model)
    with open(path, "rb") as f:
        values = [_read_tensor(f, w.numel()) for w in weights]
        moments = [(_read_tensor(f, w.numel()), _read_tensor(f, w.numel())) for w in weights]
        (steps,) = struct.unpack("<Q", _read_exact(f, 8))
        lr, b1, b2, eps, wd = struct.unpack("<5f", _read_exact(f, 20))
    with torch.no_grad():
        for w, v in zip(weights, values):
            w.copy_(torch.from_numpy(v.copy()).view_as(w))
    g = _adam_group(model)
    for w, (m, v) in zip(weights, moments):
        model.opt.state[w] = {
            # a fused or capturable AdamW keeps its step counts beside the parameters
            "step": torch.tensor(float(steps), dtype=torch.float32,
                                 device=w.device if g.get("capturable") or g.get("fused") else "cpu"),
            "exp_avg": torch.from_numpy(m.copy()).view_as(w).to(w.device),
            "exp_avg_sq": torch.from_numpy(v.copy()).view_as(w).to(w.device),
        }
    g["lr"], g["betas"], g["eps"], g["weight_decay"] = lr, (b1, b2), eps, wd
    # A recorded step has the old hyper-parameters in its AdamW launch: drop it, and StaticGPT2.replay
    # records the step again (the engine clears its graph on load too, static_gpt2.rs:2106).
    if hasattr(model, "_graph"):
        model._graph = None


# ---------------------------------------------------------------- safetensors
def _layer_names(l):
    p = f"h.{l}."
    return {"ln1_g": p + "ln_1.weight", "ln1_b": p + "ln_1.bias", "wo": p + "attn.c_proj.weight",
            "bo": p + "attn.c_proj.bias", "ln2_g": p + "ln_2.weight", "ln2_b": p + "ln_2.bias",
            "w1": p + "mlp.c_fc.weight", "b1": p + "mlp.c_fc.bias", "w2": p + "mlp.c_proj.weight",
            "b2": p + "mlp.c_proj.bias"}


def save_gpt2_safetensors(model, path) -> None:
    """safetensors.rs:246-373: F32 tensors under the GPT-2 names."""
    from safetensors.numpy import save_file

    d = model.d_model
    t = {"transformer.wte.weight": _host_f32(model.tok_emb).reshape(model.vocab_size, d),
         "transformer.wpe.weight": _host_f32(model.pos_emb).reshape(model.seq_len, d),
         "transformer.ln_f.weight": _host_f32(model.ln_f_g),
         "transformer.ln_f.bias": _host_f32(model.ln_f_b),
         "lm_head.weight": _host_f32(model.lm_head).reshape(model.vocab_size, d)}
    for l, lw in enumerate(model.layers):
        names = _layer_names(l)
        for key, name in names.items():
            t["transformer." + name] = _host_f32(lw[key]).reshape(tuple(lw[key].shape))
        # row r of c_attn = row r of Wq, Wk, Wv side by side
        t[f"transformer.h.{l}.attn.c_attn.weight"] = np.concatenate(
            [_host_f32(lw[k]).reshape(d, d) for k in ("wq", "wk", "wv")], axis=1)
        t[f"transformer.h.{l}.attn.c_attn.bias"] = np.concatenate([_host_f32(lw[k]) for k in ("bq", "bk", "bv")])
    save_file({k: np.ascontiguousarray(v, dtype=np.float32) for k, v in t.items()}, str(path))


class _SafeTensors:
    """Name lookup of safetensors.rs:135-148 (bare, "transformer.", "model.")."""

    def __init__(self, path):
        from safetensors.numpy import load_file

        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            header = json.loads(f.read(n))
        for name, meta in header.items():
            if name != "__metadata__" and meta.get("dtype") != "F32":
                raise ValueError(f"safetensors: tensor {name} is {meta.get('dtype')}; only F32 is read")
        self.tensors = load_file(str(path))

    def get(self, name):
        for key in (name, "transformer." + name, "model." + name):
            if key in self.tensors:
                return self.tensors[key]
        return None


def _set(w, data, name):
    torch = _torch()
    flat = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
    if flat.size != w.numel():
        raise ValueError(f"safetensors: {name} has {flat.size} values, the model expects {w.numel()}")
    with torch.no_grad():
        w.copy_(torch.from_numpy(flat.copy()).view_as(w))


def load_gpt2_safetensors(model, path) -> None:
    """safetensors.rs:156-244."""
    sf = _SafeTensors(path)
    d = model.d_model
    for name, w in (("wte.weight", model.tok_emb), ("wpe.weight", model.pos_emb), ("ln_f.weight", model.ln_f_g),
                    ("ln_f.bias", model.ln_f_b)):
        data = sf.get(name)
        if data is not None:
            _set(w, data, name)
    head = sf.get("lm_head.weight")
    if head is None:
        head = sf.get("wte.weight")
    if head is not None:
        _set(model.lm_head, head, "lm_head.weight")
    for l, lw in enumerate(model.layers):
        for key, name in _layer_names(l).items():
            data = sf.get(name)
            if data is not None:
                _set(lw[key], data, name)
        qkv = sf.get(f"h.{l}.attn.c_attn.weight")
        if qkv is not None:
            if qkv.size != 3 * d * d:
                raise ValueError(f"Packed QKV tensor size mismatch: expected {3 * d * d}, got {qkv.size}")
            if qkv.shape == (d, 3 * d):
                parts = (qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:])
            else:  # three consecutive [d, d] blocks
                flat = qkv.reshape(-1)
                parts = (flat[:d * d], flat[d * d:2 * d * d], flat[2 * d * d:])
            for key, part in zip(("wq", "wk", "wv"), parts):
                _set(lw[key], part, f"h.{l}.attn.c_attn.weight")
        bias = sf.get(f"h.{l}.attn.c_attn.bias")
        if bias is not None:
            if bias.size != 3 * d:
                raise ValueError(f"Packed QKV bias size mismatch: expected {3 * d}, got {bias.size}")
            for i, key in enumerate(("bq", "bk", "bv")):
                _set(lw[key], bias[i * d:(i + 1) * d], f"h.{l}.attn.c_attn.bias")
