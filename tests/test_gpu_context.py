"""GPU tests of the host-side mirror: AttentionContext (darkforest-cuda/src/lib.rs:1949-2368),
the host-slice helpers (lib.rs:2371-2479) and the autograd wrapper, against the CPU oracle.

Tolerances as in test_gpu_parity.py: the fp16-operand MFMA path is held to
max-abs <= 2e-3 * max(1, max|ref|) and rel-L2 <= 1e-3; the single-head helpers
with d_head != 64 run the exact fp32 kernels and meet the reference's 2e-4.
"""
import json
import os

import numpy as np
import pytest

import dfattn
import oracle as O
from conftest import GOLDEN, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-context] {msg}", flush=True)


def close(name, got, want, tol=2e-3, rel=1e-3):
    got = np.asarray(got, np.float64)
    bar = tol * max(1.0, float(np.max(np.abs(want))))
    ea, er = max_abs(got, want), rel_l2(got, want)
    assert np.all(np.isfinite(got)) and ea <= bar and er <= rel, f"{name}: {ea:.2e} (bar {bar:.2e}) {er:.2e}"


def dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(device)


def test_context_device_path_matches_oracle(device):
    import torch

    h, s, d = 12, 256, 64
    say("context device path H=12 S=256")
    x = O.seeded_inputs(s, h, d, 11000)
    q, k, v, g = (dev(x[n], device) for n in ("q", "k", "v", "do"))
    ctx = dfattn.AttentionContext(h, s, d)
    out = torch.empty_like(q)
    ctx.forward_device_into(q, k, v, 0.125, True, out)
    dq, dk, dv = ctx.backward_device(q, k, v, g, 0.125, True)
    torch.cuda.synchronize()
    want_o, _ = O.mha_forward(x["q"], x["k"], x["v"], h, 0.125, True, threads=8)
    want = O.backward(x["q"], x["k"], x["v"], x["do"], h, 0.125, True, threads=8)
    close("O", out.cpu().numpy(), want_o)
    for name, got, w in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        close(name, got.cpu().numpy(), w)
    ctx.close()


def test_context_backward_without_matching_forward_recomputes(device):
    """A backward on other q, k, v than the last forward must not reuse that forward's O."""
    import torch

    h, s, d = 4, 128, 64
    say("context backward recompute")
    a = O.seeded_inputs(s, h, d, 11100)
    b = O.seeded_inputs(s, h, d, 11200)
    ctx = dfattn.AttentionContext(h, s, d)
    qa, ka, va = (dev(a[n], device) for n in ("q", "k", "v"))
    qb, kb, vb, gb = (dev(b[n], device) for n in ("q", "k", "v", "do"))
    ctx.forward_device(qa, ka, va, 0.125, True)  # remembered: a
    grads = ctx.backward_device(qb, kb, vb, gb, 0.125, True)  # different tensors: recompute for b
    torch.cuda.synchronize()
    want = O.backward(b["q"], b["k"], b["v"], b["do"], h, 0.125, True, threads=8)
    for name, got, w in zip(("dq", "dk", "dv"), grads, want):
        close(name, got.cpu().numpy(), w)
    ctx.close()


def test_context_output_shape_mismatch_is_an_error(device):
    import torch

    ctx = dfattn.AttentionContext(2, 64, 64)
    q = torch.zeros((64, 128), device=device)
    bad = torch.zeros((63, 128), device=device)
    with pytest.raises(dfattn.DfattnError) as e:
        ctx.forward_device_into(q, q, q, 0.125, True, bad)
    assert e.value.status == -3 and "shape mismatch" in str(e.value)
    ctx.close()


def test_host_slice_context_and_helpers_match_reference_kats(device):
    """The reference's KATs (lib.rs:2605-2628, 2752-2829) through the host-slice API."""
    say("host-slice KATs")
    kf = json.load(open(os.path.join(GOLDEN, "kat_forward.json")))
    out = dfattn.fused_attention_forward(kf["q"], kf["k"], kf["v"], kf["seq_len"], kf["d_head"], kf["scale"], True)
    assert max_abs(out, np.array(kf["expected_o"]).reshape(-1)) <= kf["tolerance"]
    kb = json.load(open(os.path.join(GOLDEN, "kat_backward.json")))
    grads = dfattn.attention_backward_host(kb["q"], kb["k"], kb["v"], kb["d_out"], kb["seq_len"], kb["d_head"],
                                           kb["scale"], True)
    for name, got in zip(("dq", "dk", "dv"), grads):
        assert max_abs(got, np.array(kb["expected_" + name]).reshape(-1)) <= kb["tolerance"]
    ctx = dfattn.AttentionContext(1, kb["seq_len"], kb["d_head"])
    ctx.forward(kb["q"], kb["k"], kb["v"], kb["scale"], True)
    for name, got in zip(("dq", "dk", "dv"), ctx.backward(kb["d_out"], kb["scale"], True)):
        assert max_abs(got, np.array(kb["expected_" + name]).reshape(-1)) <= kb["tolerance"]
    ctx.close()


def test_host_slice_single_head_d64(device):
    say("host-slice single head S=200 D=64")
    x = O.seeded_inputs(200, 1, 64, 11300)
    ctx = dfattn.AttentionContext(1, 200, 64)
    out = ctx.forward(x["q"], x["k"], x["v"], 0.125, True)
    close("O", out.reshape(200, 64), O.mha_forward(x["q"], x["k"], x["v"], 1, 0.125, True)[0])
    grads = ctx.backward(x["do"], 0.125, True)
    for name, got, w in zip(("dq", "dk", "dv"), grads, O.backward(x["q"], x["k"], x["v"], x["do"], 1, 0.125, True)):
        close(name, got.reshape(200, 64), w)
    ctx.close()


def test_autograd_function_matches_float64_torch(device):
    """FusedCausalAttention inside torch autograd vs float64 CPU scaled_dot_product_attention."""
    import torch

    h, s, d = 4, 160, 64
    say("autograd wrapper")
    x = O.seeded_inputs(s, h, d, 11400)
    q, k, v = (dev(x[n], device).requires_grad_(True) for n in ("q", "k", "v"))
    o = dfattn.FusedCausalAttention.apply(q, k, v, h, 0.125, True)
    o.backward(dev(x["do"], device))
    ref = [torch.from_numpy(x[n]).double().view(s, h, d).transpose(0, 1).requires_grad_(True) for n in ("q", "k", "v")]
    ro = torch.nn.functional.scaled_dot_product_attention(*ref, is_causal=True, scale=0.125)
    ro.backward(torch.from_numpy(x["do"]).double().view(s, h, d).transpose(0, 1))
    close("O", o.detach().cpu().numpy(), ro.detach().transpose(0, 1).reshape(s, h * d).numpy())
    for t, r, name in zip((q, k, v), ref, ("dq", "dk", "dv")):
        close(name, t.grad.cpu().numpy(), r.grad.transpose(0, 1).reshape(s, h * d).numpy())


def test_sync_survives_errors_already_returned(device):
    """darkforest_sync does not abort for an error a status-returning entry point already returned
    (it synchronises the device and returns). Its aborting branch, for an argument error of a void
    launcher, is host-only logic and is tested on the CPU (test_abi.py)."""
    import subprocess
    import sys

    from conftest import ROOT

    pkg = os.path.join(ROOT, "dark-forest_amd")
    returned = ("import sys; sys.path.insert(0, %r); import ctypes, dfattn; lib = dfattn.lib(); "
                "h = ctypes.c_void_p(); assert lib.dfattn_context_create(12, 128, 0, ctypes.byref(h)) == -4; "
                "lib.darkforest_sync(); print('survived')") % pkg
    out = subprocess.run([sys.executable, "-c", returned], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "survived" in out.stdout, out.stderr


def test_context_backward_reads_current_q_after_in_place_change(device):
    """By default backward_device_into differentiates the current contents of q, k, v (the
    reference recomputes, lib.rs:2240-2293): q changed in place after the forward, and the
    forward's O dropped, still give the oracle's gradients of the new q."""
    import gc

    import torch

    h, s, d = 12, 192, 64
    say("context: q changed in place between forward and backward")
    x = O.seeded_inputs(s, h, d, 11500)
    q, k, v, g = (dev(x[n], device) for n in ("q", "k", "v", "do"))
    ctx = dfattn.AttentionContext(h, s, d)
    out = ctx.forward_device(q, k, v, 0.125, True)
    del out
    gc.collect()
    torch.cuda.empty_cache()
    q.mul_(0.5).add_(0.25)
    junk = torch.full((s, h * d), float("nan"), device=device)  # may take the freed O's block
    dq, dk, dv = ctx.backward_device(q, k, v, g, 0.125, True)
    torch.cuda.synchronize()
    q_new = (x["q"] * np.float32(0.5) + np.float32(0.25)).astype(np.float32)
    want = O.backward(q_new, x["k"], x["v"], x["do"], h, 0.125, True, threads=8)
    for name, got, w in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        close(name, got.cpu().numpy(), w)
    del junk
    ctx.close()


def test_context_reuse_forward_matches_recompute(device):
    """With forward reuse on (the engine's contract: q, k, v and O untouched in between) the backward
    gives the recomputing backward's gradients bit for bit, and the wrapper holds the forward's
    tensors while the context may read them."""
    import torch

    h, s, d = 12, 320, 64
    say("context: opt-in forward reuse")
    x = O.seeded_inputs(s, h, d, 11600)
    q, k, v, g = (dev(x[n], device) for n in ("q", "k", "v", "do"))
    plain = dfattn.AttentionContext(h, s, d)
    ref = plain.backward_device(q, k, v, g, 0.125, True)
    reuse = dfattn.AttentionContext(h, s, d, reuse_forward=True)
    out = reuse.forward_device(q, k, v, 0.125, True)
    assert reuse._last is not None and reuse._last[3] is out
    got = reuse.backward_device(q, k, v, g, 0.125, True)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    reuse.set_reuse_forward(False)
    assert reuse._last is None
    plain.close()
    reuse.close()
