"""GPU: the row-strided training pair and context calls (dfattn_*_strided) against the contiguous
calls on the same data.

The strided kernels differ from the contiguous ones only in the addresses they read Q, K, V from and
write dQ, dK, dV to; every arithmetic step is the same, so the bar is equality, bit for bit, of O,
lse, dQ, dK and dV. Columns of the wide tensors outside the three blocks (padding) must come back
untouched, and the wide inputs unchanged. One shape is also checked against the oracle directly.
"""
import numpy as np
import pytest

import dfattn
import oracle as O
from test_gpu_parity import compare, host, oracle_fwd_bwd, say, to_dev

pytestmark = pytest.mark.gpu

SENTINEL = 7.25
# (seq_len, n_heads, causal, input pad, gradient pad, block order): pads are extra floats per row.
SHAPES = [(4096, 12, True, 0, 0, (0, 1, 2)), (1000, 3, False, 4, 12, (2, 0, 1)),
          (2049, 5, True, 12, 0, (1, 2, 0)), (64, 1, True, 0, 4, (0, 1, 2))]


def wide(blocks, pad, order, device, shape=None):
    """One [S, 3*dm + pad] tensor holding blocks[i] in column block order[i], SENTINEL in the pad
    and where a block is None; returns it and the three column views (in the order of `blocks`)."""
    import torch

    S, dm = shape or blocks[0].shape
    w = torch.full((S, 3 * dm + pad), SENTINEL, device=device)
    views = [w[:, order[i] * dm:(order[i] + 1) * dm] for i in range(3)]
    for view, b in zip(views, blocks):
        if b is not None:
            view.copy_(b)
    return w, views


def pad_untouched(w, dm):
    return bool((w[:, 3 * dm:] == SENTINEL).all()) if w.shape[1] > 3 * dm else True


def training_pair(q, k, v, g, n_heads, scale, causal, grads, flags):
    import torch

    S, dm = g.shape
    ws = torch.full((dfattn.bwd_workspace_bytes(n_heads, S, dm // n_heads) // 4,), float("nan"), device=g.device)
    o, lse = dfattn.forward_train(q, k, v, n_heads, ws, scale, causal)
    dfattn.backward_preprocess(q, k, v, o, g, lse, ws, n_heads, scale, flags=flags)
    dfattn.backward_main(q, k, v, o, g, lse, *grads, ws, n_heads, scale, causal)
    torch.cuda.synchronize()
    return [host(t) for t in (o, lse, *grads)]


def assert_equal(tag, got, want):
    for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), got, want):
        assert a.shape == b.shape and np.array_equal(a, b), \
            f"{tag} {name}: differs from the contiguous call (max diff {np.max(np.abs(a - b)):.3e})"


@pytest.mark.parametrize("flags", [0, 1])
@pytest.mark.parametrize("seq_len,n_heads,causal,pad,gpad,order", SHAPES)
def test_strided_training_pair_is_the_contiguous_one(device, seq_len, n_heads, causal, pad, gpad, order, flags):
    """forward_train / backward_preprocess (with and without DFATTN_BWD_QKV_SAVED) / backward_main on
    Q, K, V read from one wide tensor and dQ, dK, dV written into another, and the two mixed cases
    (strided inputs with contiguous gradients and the reverse), against the contiguous calls."""
    import torch

    say(f"strided training pair S={seq_len} H={n_heads} causal={causal} pad={pad}/{gpad} order={order} "
        f"flags={flags}")
    x = O.seeded_inputs(seq_len, n_heads, 64, 9100 + seq_len)
    q, k, v, g = (to_dev(x[n], device) for n in ("q", "k", "v", "do"))
    scale = 0.125
    want = training_pair(q, k, v, g, n_heads, scale, causal, [torch.empty_like(q) for _ in range(3)], flags)
    wq, views = wide([q, k, v], pad, order, device)
    before = wq.clone()
    for tag, ins, strided_grads in (("both", views, True), ("inputs", views, False), ("grads", (q, k, v), True)):
        if strided_grads:
            wg, gviews = wide([None] * 3, gpad, order, device, q.shape)
        else:
            wg, gviews = None, [torch.full_like(q, float("nan")) for _ in range(3)]
        got = training_pair(*ins, g, n_heads, scale, causal, gviews, flags)
        assert_equal(tag, got, want)
        if wg is not None:
            assert pad_untouched(wg, q.shape[1]), f"{tag}: gradient padding overwritten"
    assert torch.equal(wq, before), "wide input modified"
    if seq_len == 1000:  # one shape straight against the oracle as well
        compare("strided vs oracle", dict(zip(("o", "lse", "dq", "dk", "dv"), got)),
                oracle_fwd_bwd(x, n_heads, scale, causal), scaled=True)
    say(f"S={seq_len}: strided == contiguous, bit for bit")


@pytest.mark.parametrize("reuse", [True, False])
@pytest.mark.parametrize("seq_len,n_heads,causal,pad,gpad,order", SHAPES[:2])
def test_strided_context_is_the_contiguous_one(device, seq_len, n_heads, causal, pad, gpad, order, reuse):
    """AttentionContext.forward_device_into / backward_device_into on column blocks of wide tensors
    (the *_strided context calls), with forward reuse on and off, against the same context calls on
    contiguous tensors; then a contiguous backward after a strided forward (the reuse key includes
    the row stride, so the context recomputes the forward rather than reuse the wrong one)."""
    import torch

    say(f"strided context S={seq_len} H={n_heads} causal={causal} reuse={reuse}")
    x = O.seeded_inputs(seq_len, n_heads, 64, 9200 + seq_len)
    q, k, v, g = (to_dev(x[n], device) for n in ("q", "k", "v", "do"))
    scale = 0.125
    ctx = dfattn.AttentionContext(n_heads, seq_len, 64, reuse_forward=reuse)
    try:
        out = ctx.forward_device(q, k, v, scale, causal)
        want_g = ctx.backward_device(q, k, v, g, scale, causal)
        torch.cuda.synchronize()
        want = [host(out), *(host(t) for t in want_g)]
        _, views = wide([q, k, v], pad, order, device)
        wg, gviews = wide([None] * 3, gpad, order, device, q.shape)
        out2 = ctx.forward_device(*views, scale, causal)
        ctx.backward_device_into(*views, g, scale, causal, *gviews)
        torch.cuda.synchronize()
        got = [host(out2), *(host(t) for t in gviews)]
        for name, a, b in zip(("o", "dq", "dk", "dv"), got, want):
            assert np.array_equal(a, b), f"context {name}: differs from the contiguous call"
        assert pad_untouched(wg, q.shape[1])
        # Strided forward, then the contiguous backward on the same values: same gradients.
        ctx.forward_device(*views, scale, causal)
        grads = ctx.backward_device(q, k, v, g, scale, causal)
        torch.cuda.synchronize()
        for name, a, b in zip(("dq", "dk", "dv"), grads, want_g):
            assert torch.equal(a, b), f"contiguous backward after a strided forward: {name} differs"
    finally:
        ctx.close()

