"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Inputs:
  * the reference's two known-answer tests, regenerated from their closed
    forms (darkforest-cuda/src/lib.rs:2610-2617 forward, :2757-2769 backward);
  * small multi-head cases from seeded PCG64 streams (the reference has no
    multi-head test; these pin the [S, H*D] layout, attention_fused.cu:60-66).

Expected outputs come from PyTorch float64 on the CPU —
torch.nn.functional.scaled_dot_product_attention plus autograd, the library
the reference itself compares against (scripts/verify_loss_parity.py:58) —
and not from the oracle, so the fixtures are an independent check of it.
Logsumexp (which the reference does not produce) comes from torch.logsumexp
over the masked, scaled scores.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def torch_attention(q, k, v, d_out, n_heads, scale, causal):
    """float64 forward + backward of [S, H*D] tensors. Returns dict of numpy arrays."""
    seq_len, dm = q.shape
    d_head = dm // n_heads

    def heads(a):
        return torch.tensor(np.asarray(a, dtype=np.float64)).view(seq_len, n_heads, d_head).transpose(0, 1)

    tq, tk, tv = (heads(a).clone().requires_grad_(True) for a in (q, k, v))
    out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=bool(causal), scale=scale)
    scores = torch.matmul(tq.detach(), tk.detach().transpose(-1, -2)) * scale
    if causal:
        mask = torch.triu(torch.ones(seq_len, seq_len, dtype=torch.bool), 1)
        scores = scores.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    res = {"o": out, "lse": lse}
    if d_out is not None:
        out.backward(heads(d_out))
        res.update(dq=tq.grad, dk=tk.grad, dv=tv.grad)

    def flat(t):
        t = t.detach()
        return t.transpose(0, 1).reshape(seq_len, dm).numpy() if t.dim() == 3 else t.numpy()

    return {name: flat(t) for name, t in res.items()}


def kat_forward():
    # lib.rs:2608-2617: seq_len 5, d_head 4, q_i=(i-7)/11, k_i=(3-i)/13, v_i=sin(i), scale 1/sqrt(4), causal.
    seq_len, d_head = 5, 4
    n = seq_len * d_head
    q = np.array([(i - 7.0) / 11.0 for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    k = np.array([(3.0 - i) / 13.0 for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    v = np.array([math.sin(float(i)) for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d_head)))
    exp = torch_attention(q, k, v, None, 1, scale, True)
    return {"source": "darkforest-cuda/src/lib.rs:2605-2628", "seq_len": seq_len, "d_head": d_head,
            "scale": scale, "causal": True, "tolerance": 2e-4,
            "q": q.tolist(), "k": k.tolist(), "v": v.tolist(),
            "expected_o": exp["o"].tolist(), "expected_lse": exp["lse"].tolist()}


def kat_backward():
    # lib.rs:2755-2769: seq_len 4, d_head 3, q=(i-4)/9, k=(2-i)/10, v=(i+1)/8, d_out=(i-3)/7, scale 1/sqrt(3).
    seq_len, d_head = 4, 3
    n = seq_len * d_head
    q = np.array([(i - 4.0) / 9.0 for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    k = np.array([(2.0 - i) / 10.0 for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    v = np.array([(i + 1.0) / 8.0 for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    d_out = np.array([(i - 3.0) / 7.0 for i in range(n)], dtype=np.float32).reshape(seq_len, d_head)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d_head)))
    exp = torch_attention(q, k, v, d_out, 1, scale, True)
    return {"source": "darkforest-cuda/src/lib.rs:2752-2829", "seq_len": seq_len, "d_head": d_head,
            "scale": scale, "causal": True, "tolerance": 2e-4, "fd_delta": 1e-3, "fd_tolerance": 2e-3,
            "q": q.tolist(), "k": k.tolist(), "v": v.tolist(), "d_out": d_out.tolist(),
            "expected_o": exp["o"].tolist(), "expected_dq": exp["dq"].tolist(),
            "expected_dk": exp["dk"].tolist(), "expected_dv": exp["dv"].tolist()}


# (name, n_heads, seq_len, d_head, causal, seed)
MHA_CASES = [
    ("mha_h3_s7_d5_causal", 3, 7, 5, True, 101),
    ("mha_h2_s20_d64_causal", 2, 20, 64, True, 202),
    ("mha_h2_s20_d64_full", 2, 20, 64, False, 303),
    ("mha_h1_s9_d128_causal", 1, 9, 128, True, 404),
]


def mha_case(n_heads, seq_len, d_head, causal, seed):
    dm = n_heads * d_head
    arrays = {}
    for i, name in enumerate(["q", "k", "v", "do"]):
        rng = np.random.Generator(np.random.PCG64(seed + i))
        arrays[name] = rng.standard_normal((seq_len, dm), dtype=np.float32)
    scale = 1.0 / math.sqrt(d_head)
    exp = torch_attention(arrays["q"], arrays["k"], arrays["v"], arrays["do"], n_heads, scale, causal)
    out = {f"in_{k}": v for k, v in arrays.items()}
    out.update({f"exp_{k}": v for k, v in exp.items()})
    out["meta"] = np.array([n_heads, seq_len, d_head, int(causal)], dtype=np.int64)
    out["scale"] = np.array([scale], dtype=np.float64)
    return out


def main():
    with open(os.path.join(HERE, "kat_forward.json"), "w") as f:
        json.dump(kat_forward(), f, indent=1)
    with open(os.path.join(HERE, "kat_backward.json"), "w") as f:
        json.dump(kat_backward(), f, indent=1)
    for name, h, s, d, causal, seed in MHA_CASES:
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **mha_case(h, s, d, causal, seed))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
