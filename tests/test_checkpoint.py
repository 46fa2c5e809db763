"""StaticGPT2 checkpoints in the reference's binary format and as GPT-2 safetensors (CPU).

The binary layout is checked with a reader written from the format's definition (u64 LE count +
f32 LE values per tensor, weights then AdamW moments then a u64 + 5 x f32 footer; static_gpt2.rs:
1924-2004, read the same way by the reference's scripts/verify_loss_parity.py:72-107), not with the
module's own loader; the safetensors files are read back with the safetensors library.
"""
import struct

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from dfattn import checkpoint as C  # noqa: E402
from dfattn.gpt2_step import StaticGPT2  # noqa: E402

DIMS = dict(vocab_size=97, d_model=32, n_heads=4, n_layers=2, d_ff=64, seq_len=16)


def tiny(seed=0):
    return StaticGPT2(**DIMS, seed=seed, device="cpu", attention="sdpa")


def batch(seed=5):
    g = torch.Generator().manual_seed(seed)
    t = torch.randint(0, DIMS["vocab_size"], (DIMS["seq_len"] + 1,), generator=g)
    return t[:-1], t[1:]


def trained(steps=2):
    m = tiny()
    for i in range(steps):
        m.step(*batch(i))
    return m


def read_reference_layout(path, n_tensors):
    with open(path, "rb") as f:
        def tensor():
            (n,) = struct.unpack("<Q", f.read(8))
            return np.frombuffer(f.read(4 * n), dtype="<f4")
        weights = [tensor() for _ in range(n_tensors)]
        moments = [(tensor(), tensor()) for _ in range(n_tensors)]
        footer = struct.unpack("<Q5f", f.read(28))
        assert f.read() == b""
    return weights, moments, footer


def test_binary_checkpoint_layout(tmp_path):
    m = trained()
    path = tmp_path / "model.ckpt"
    C.save_checkpoint(m, path)
    names = ["tok_emb", "pos_emb", "ln_f_g", "ln_f_b", "lm_head"]
    expect = [m.tok_emb, m.pos_emb, m.ln_f_g, m.ln_f_b, m.lm_head]
    for lw in m.layers:  # static_gpt2.rs:1955-1972
        for k in ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1", "b1",
                  "w2", "b2"):
            expect.append(lw[k])
            names.append(k)
    weights, moments, footer = read_reference_layout(path, len(expect))
    for name, w, got, (mm, vv) in zip(names, expect, weights, moments):
        assert np.array_equal(got, w.detach().numpy().reshape(-1)), name
        st = m.opt.state[w]
        assert np.array_equal(mm, st["exp_avg"].numpy().reshape(-1)), name
        assert np.array_equal(vv, st["exp_avg_sq"].numpy().reshape(-1)), name
        assert np.abs(vv).max() > 0, name  # two steps taken: moments are live
    steps, lr, b1, b2, eps, wd = footer
    assert steps == 2
    assert np.float32(lr) == np.float32(3e-4) and (b1, b2) == (np.float32(0.9), np.float32(0.95))
    assert eps == np.float32(1e-8) and wd == np.float32(0.1)


def test_binary_checkpoint_resumes_training_exactly(tmp_path):
    a = trained()
    path = tmp_path / "model.ckpt"
    C.save_checkpoint(a, path)
    b = tiny(seed=123)
    C.load_checkpoint(b, path)
    assert C.step_count(b) == 2
    for wa, wb in zip(a.parameters(), b.parameters()):
        assert torch.equal(wa, wb)
    la, lb = a.step(*batch(9)), b.step(*batch(9))
    assert torch.equal(la, lb)
    for wa, wb in zip(a.parameters(), b.parameters()):
        assert torch.equal(wa, wb)


def test_fresh_model_checkpoint_has_zero_moments(tmp_path):
    path = tmp_path / "fresh.ckpt"
    C.save_checkpoint(tiny(), path)
    n = len(C.ordered_weights(tiny()))
    _, moments, footer = read_reference_layout(path, n)
    assert footer[0] == 0 and all(not mm.any() and not vv.any() for mm, vv in moments)


def test_binary_checkpoint_errors(tmp_path):
    path = tmp_path / "model.ckpt"
    C.save_checkpoint(tiny(), path)
    other = StaticGPT2(**{**DIMS, "d_ff": 48}, device="cpu", attention="sdpa")
    with pytest.raises(ValueError, match="tensor size mismatch"):
        C.load_checkpoint(other, path)
    data = path.read_bytes()
    short = tmp_path / "short.ckpt"
    short.write_bytes(data[:-3])
    with pytest.raises(ValueError, match="ends early"):
        C.load_checkpoint(tiny(), short)


def test_safetensors_export_names_shapes_and_packing(tmp_path):
    from safetensors.numpy import load_file

    m = trained(1)
    path = tmp_path / "gpt2.safetensors"
    C.save_gpt2_safetensors(m, path)
    t = load_file(str(path))
    d, v, s, f = DIMS["d_model"], DIMS["vocab_size"], DIMS["seq_len"], DIMS["d_ff"]
    want = {"transformer.wte.weight": (v, d), "transformer.wpe.weight": (s, d), "transformer.ln_f.weight": (d,),
            "transformer.ln_f.bias": (d,), "lm_head.weight": (v, d)}
    for l in range(DIMS["n_layers"]):
        p = f"transformer.h.{l}."
        want.update({p + "ln_1.weight": (d,), p + "ln_1.bias": (d,), p + "attn.c_attn.weight": (d, 3 * d),
                     p + "attn.c_attn.bias": (3 * d,), p + "attn.c_proj.weight": (d, d), p + "attn.c_proj.bias": (d,),
                     p + "ln_2.weight": (d,), p + "ln_2.bias": (d,), p + "mlp.c_fc.weight": (f, d),
                     p + "mlp.c_fc.bias": (f,), p + "mlp.c_proj.weight": (d, f), p + "mlp.c_proj.bias": (d,)})
    assert {k: tuple(a.shape) for k, a in t.items()} == want
    lw = m.layers[1]
    qkv = t["transformer.h.1.attn.c_attn.weight"]
    for r in (0, 7, d - 1):  # safetensors.rs:283-289: row r = [Wq[r], Wk[r], Wv[r]]
        assert np.array_equal(qkv[r], np.concatenate([lw[k].detach().numpy()[r] for k in ("wq", "wk", "wv")]))
    b = t["transformer.h.1.attn.c_attn.bias"]
    assert np.array_equal(b[d:2 * d], lw["bk"].detach().numpy())
    assert np.array_equal(t["transformer.h.0.mlp.c_fc.weight"], m.layers[0]["w1"].detach().numpy())


def test_safetensors_round_trip(tmp_path):
    a = trained(1)
    path = tmp_path / "gpt2.safetensors"
    C.save_gpt2_safetensors(a, path)
    b = tiny(seed=77)
    C.load_gpt2_safetensors(b, path)
    for wa, wb in zip(a.parameters(), b.parameters()):
        assert torch.equal(wa, wb)


def test_safetensors_import_bare_names_tied_head_and_block_qkv(tmp_path):
    """HF-style bare names, no lm_head (tied to wte), c_attn as three [d, d] blocks, a missing tensor."""
    from safetensors.numpy import save_file

    d = DIMS["d_model"]
    rng = np.random.default_rng(3)
    wte = rng.standard_normal((DIMS["vocab_size"], d)).astype(np.float32)
    blocks = rng.standard_normal((3 * d, d)).astype(np.float32)
    ln = rng.standard_normal(d).astype(np.float32)
    save_file({"wte.weight": wte, "h.0.attn.c_attn.weight": blocks, "model.h.1.ln_2.bias": ln}, str(tmp_path / "x"))
    m = tiny()
    before = m.pos_emb.detach().clone()
    C.load_gpt2_safetensors(m, tmp_path / "x")
    assert np.array_equal(m.tok_emb.detach().numpy(), wte) and np.array_equal(m.lm_head.detach().numpy(), wte)
    assert np.array_equal(m.layers[0]["wk"].detach().numpy(), blocks[d:2 * d])
    assert np.array_equal(m.layers[1]["ln2_b"].detach().numpy(), ln)
    assert torch.equal(m.pos_emb, before)


def test_safetensors_import_errors(tmp_path):
    from safetensors.numpy import save_file

    save_file({"h.0.attn.c_attn.bias": np.zeros(5, np.float32)}, str(tmp_path / "bad"))
    with pytest.raises(ValueError, match="Packed QKV bias size mismatch"):
        C.load_gpt2_safetensors(tiny(), tmp_path / "bad")
    save_file({"wte.weight": np.zeros((2, 2), np.float16)}, str(tmp_path / "f16"))
    with pytest.raises(ValueError, match="only F32"):
        C.load_gpt2_safetensors(tiny(), tmp_path / "f16")



def test_load_drops_the_recorded_step_and_replay_records_it_again(tmp_path, monkeypatch):
    """CPU stand-in for the graph: after load_checkpoint, replay() calls capture() on the stored
    batch with no warm-up steps (which would train the loaded weights), then replays the new graph;
    replay before any capture raises."""
    m = trained()
    with pytest.raises(RuntimeError, match="before capture"):
        m.replay()
    C.save_checkpoint(m, tmp_path / "m.ckpt")
    calls = []

    class Graph:
        def replay(self):
            calls.append("replay")

    def fake_capture(tokens, targets, warmup=3):
        calls.append(("capture", warmup, torch.equal(tokens, m._tokens)))
        m._graph, m._loss = Graph(), torch.zeros(())
        return m._loss

    m._tokens, m._targets = batch(0)
    m._graph = Graph()
    monkeypatch.setattr(m, "capture", fake_capture)
    C.load_checkpoint(m, tmp_path / "m.ckpt")
    assert m._graph is None
    m.replay()
    m.replay()
    assert calls == [("capture", 0, True), "replay", "replay"]
