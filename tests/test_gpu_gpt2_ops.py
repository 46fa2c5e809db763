"""The GPT-2 step's non-attention kernels (include/dfgpt2.h) on the GPU against PyTorch fp32
operators of the same maths (float64 for AdamW), plus bitwise reproducibility of the reductions and
the reference launchers (null stream) against the stream entry points."""
import ctypes

import pytest

import dfattn
from dfattn import ops

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-gpt2-ops] {msg}", flush=True)


def P(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def close(a, b, rtol, atol, what):
    import torch

    err = (a - b).abs().max().item()
    ok = torch.allclose(a, b, rtol=rtol, atol=atol)
    say(f"{what}: max abs err {err:.3e}")
    assert ok, f"{what}: max abs err {err}"


# (rows, features): the GPT-2 width (register path), a width that is not a multiple of 4 and one
# above the register path's 1024 (generic paths), a single row
LN_SHAPES = [(1024, 768), (37, 130), (64, 2048), (1, 768)]


@pytest.mark.parametrize("rows,f", LN_SHAPES)
@pytest.mark.parametrize("affine", [True, False])
def test_layernorm_forward_and_backward_match_torch(device, rows, f, affine):
    import torch

    say(f"layernorm rows={rows} f={f} affine={affine}")
    g = torch.Generator(device="cpu").manual_seed(rows * 31 + f)
    x = (torch.randn(rows, f, generator=g) * 3 + 0.5).to(device)
    gamma = (torch.randn(f, generator=g)).to(device) if affine else None
    beta = (torch.randn(f, generator=g)).to(device) if affine else None
    dy = torch.randn(rows, f, generator=g).to(device)
    out, means, rstds = ops.layer_norm_forward(x, gamma, beta)
    xr = x.clone().requires_grad_(True)
    gr = gamma.clone().requires_grad_(True) if affine else None
    br = beta.clone().requires_grad_(True) if affine else None
    ref = torch.nn.functional.layer_norm(xr, (f,), gr, br, 1e-5)
    close(out, ref.detach(), 1e-5, 1e-5, "out")
    close(means, x.mean(1), 1e-5, 1e-5, "means")
    close(rstds, (x.var(1, unbiased=False) + 1e-5).rsqrt(), 1e-5, 1e-6, "rstds")
    ref.backward(dy)
    gx, gg, gb = ops.layer_norm_backward(dy, x, gamma, means, rstds)
    close(gx, xr.grad, 1e-4, 1e-5, "grad_x")
    if affine:
        close(gg, gr.grad, 1e-4, 1e-4 * rows ** 0.5, "grad_gamma")
        close(gb, br.grad, 1e-4, 1e-4 * rows ** 0.5, "grad_beta")


def test_layernorm_backward_accumulates_parameter_gradients(device):
    """grad_gamma / grad_beta are added to, as the reference's atomics add (layernorm.cu:140-141)."""
    import torch

    rows, f = 256, 768
    x, dy = torch.randn(rows, f, device=device), torch.randn(rows, f, device=device)
    gamma = torch.randn(f, device=device)
    _, means, rstds = ops.layer_norm_forward(x, gamma, None)
    _, gg, gb = ops.layer_norm_backward(dy, x, gamma, means, rstds)
    gx = torch.empty_like(x)
    acc_g, acc_b = torch.full((f,), 2.0, device=device), torch.full((f,), -1.0, device=device)
    dfattn._check(ops.ops_lib().dfgpt2_layernorm_backward(P(dy), P(x), P(gamma), P(means), P(rstds), P(gx),
                                                          P(acc_g), P(acc_b), rows, f, None))
    torch.cuda.synchronize()
    assert torch.equal(acc_g, gg + 2.0) and torch.equal(acc_b, gb - 1.0)


@pytest.mark.parametrize("rows,n", [(1024, 768), (1024, 3072), (1000, 50), (1, 768), (0, 64)])
def test_bias_gradient_is_the_column_sum(device, rows, n):
    import torch

    say(f"bias grad rows={rows} n={n}")
    gy = torch.randn(rows, n, device=device)
    gb = ops.bias_grad(gy)
    close(gb, gy.double().sum(0).float(), 0, 2e-5 * max(rows, 1) ** 0.5, "bias grad")
    # accumulate onto an existing gradient
    acc = torch.ones(n, device=device)
    dfattn._check(ops.ops_lib().dfgpt2_linear_grad_bias(P(gy), P(acc), rows, n, 1, None))
    torch.cuda.synchronize()
    assert torch.equal(acc, gb + 1.0)


def test_reductions_are_bitwise_reproducible(device):
    import torch

    x, dy = torch.randn(1024, 768, device=device), torch.randn(1024, 768, device=device)
    gamma = torch.randn(768, device=device)
    _, m, r = ops.layer_norm_forward(x, gamma, None)
    first = ops.layer_norm_backward(dy, x, gamma, m, r) + (ops.bias_grad(dy),)
    for _ in range(3):
        again = ops.layer_norm_backward(dy, x, gamma, m, r) + (ops.bias_grad(dy),)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


@pytest.mark.parametrize("n", [1024 * 3072, 1001, 3])
def test_gelu_forward_and_backward_match_torch(device, n):
    import torch

    x = torch.randn(n, device=device) * 3
    dy = torch.randn(n, device=device)
    xr = x.clone().requires_grad_(True)
    ref = torch.nn.functional.gelu(xr, approximate="tanh")
    close(ops.gelu_forward(x), ref.detach(), 1e-5, 1e-6, "gelu")
    ref.backward(dy)
    close(ops.gelu_backward(dy, x), xr.grad, 1e-5, 1e-5, "gelu backward")
    # misaligned (offset by one float) views take the scalar path
    if n > 8:
        close(ops.gelu_forward(x[1:]), ref.detach()[1:], 1e-5, 1e-6, "gelu, unaligned")


def _adamw_ref(p, m, v, g, lr, b1, b2, eps, wd, t):
    """matmul.cu:300-306 in float64."""
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
    return p * (1 - lr * wd) - lr * (m / bc1) / ((v / bc2).sqrt() + eps), m, v


def test_adamw_matches_the_reference_update_and_counts_steps(device):
    import torch

    n = 1_000_003
    p, g = torch.randn(n, device=device), torch.randn(n, device=device) * 1e-2
    m, v = torch.zeros(n, device=device), torch.zeros(n, device=device)
    step = torch.zeros(1, device=device)
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-8, 0.1
    pd, md, vd = p.double(), m.double(), v.double()
    for t in range(1, 4):
        gt = g * t
        dfattn._check(ops.ops_lib().dfgpt2_adamw_update(P(p), P(m), P(v), P(gt), n, lr, b1, b2, eps, wd, P(step),
                                                        None))
        pd, md, vd = _adamw_ref(pd, md, vd, gt.double(), lr, b1, b2, eps, wd, t)
        torch.cuda.synchronize()
        assert float(step) == t
        close(p.double(), pd, 0, 1e-6, f"adamw p, step {t}")
        close(m.double(), md, 1e-5, 1e-9, f"adamw m, step {t}")
        close(v.double(), vd, 1e-5, 1e-12, f"adamw v, step {t}")


def test_reference_launchers_match_the_stream_entry_points(device):
    import torch

    lib = ops.ops_lib()
    lib.dfattn_clear_error()
    rows, f = 333, 768
    x, dy = torch.randn(rows, f, device=device), torch.randn(rows, f, device=device)
    gamma, beta = torch.randn(f, device=device), torch.randn(f, device=device)
    out, m, r = torch.empty_like(x), torch.empty(rows, device=device), torch.empty(rows, device=device)
    gx, gg, gb = torch.empty_like(x), torch.zeros(f, device=device), torch.zeros(f, device=device)
    bias, ge, gge = torch.empty(f, device=device), torch.empty_like(x), torch.empty_like(x)
    lib.launch_layernorm(P(x), P(gamma), P(beta), P(out), P(m), P(r), rows, f)
    lib.launch_layernorm_backward(P(dy), P(x), P(gamma), P(m), P(r), P(gx), P(gg), P(gb), rows, f)
    lib.launch_linear_grad_bias(P(dy), P(bias), rows, f)
    lib.launch_gelu(P(x), P(ge), rows * f)
    lib.launch_gelu_backward(P(dy), P(x), P(gge), rows * f)
    lib.darkforest_sync()
    want_out, wm, wr = ops.layer_norm_forward(x, gamma, beta)
    wgx, wgg, wgb = ops.layer_norm_backward(dy, x, gamma, wm, wr)
    torch.cuda.synchronize()
    for a, b in [(out, want_out), (m, wm), (r, wr), (gx, wgx), (gg, wgg), (gb, wgb), (bias, ops.bias_grad(dy)),
                 (ge, ops.gelu_forward(x)), (gge, ops.gelu_backward(dy, x))]:
        assert torch.equal(a, b)
    # the reference AdamW takes the bias corrections from the caller
    n = 4099
    p, g = torch.randn(n, device=device), torch.randn(n, device=device)
    mm, vv = torch.zeros(n, device=device), torch.zeros(n, device=device)
    p0 = p.double()
    lib.launch_adamw_update(P(p), P(mm), P(vv), P(g), n, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1 - 0.9, 1 - 0.95)
    lib.darkforest_sync()
    want, _, _ = _adamw_ref(p0, 0, 0, g.double(), 1e-3, 0.9, 0.95, 1e-8, 0.1, 1)
    close(p.double(), want, 0, 1e-6, "launch_adamw_update")


# ---------------------------------------------------------------- cross-entropy (softmax.cu:325-413)
@pytest.mark.parametrize("rows,vocab", [(512, 50257), (7, 1000), (3, 1), (4, 512), (4, 513), (5, 4097),
                                       (3, 51200), (2, 51201)])
def test_chunked_cross_entropy_matches_torch(device, rows, vocab):
    """dfgpt2_logit_ce_chunk + dfgpt2_sum against torch's fp64 log-softmax: the gradient
    (softmax - one_hot) / total_rows per value and the mean loss, with the gradient written to its
    own buffer and in place; the reference launcher writes the softmax back and sums the loss with
    atomics. The vocabularies cover each register-resident row size (up to 1, 8, 32 and 100 values
    per thread, full and one past) and the two-read kernel for longer rows."""
    import torch

    say(f"cross-entropy rows={rows} vocab={vocab}")
    total = 4 * rows  # the chunk is a quarter of the sequence
    g = torch.Generator(device="cpu").manual_seed(rows + vocab)
    logits = (torch.randn(rows, vocab, generator=g) * 2).to(device)
    targets = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int32).to(device)
    lp = torch.log_softmax(logits.double(), dim=1)
    want_grad = (lp.exp() - torch.nn.functional.one_hot(targets.long(), vocab).double()) / total
    want_rows = -lp.gather(1, targets.long()[:, None])[:, 0] / total
    grad = torch.empty_like(logits)
    row_loss = torch.empty(rows, device=device)
    loss = torch.empty(1, device=device)
    ops.logit_ce_chunk(logits, targets, grad, row_loss, total)
    ops.sum_into(row_loss, loss)
    torch.cuda.synchronize()
    close(grad.double(), want_grad, 1e-5, 1e-9, "grad")
    close(row_loss.double(), want_rows, 1e-5, 1e-8, "row losses")
    close(loss.double(), want_rows.sum()[None], 1e-5, 1e-8, "loss")
    # in place: the gradient overwrites the logits, bit for bit the same
    inplace = logits.clone()
    ops.logit_ce_chunk(inplace, targets, inplace, row_loss, total)
    torch.cuda.synchronize()
    assert torch.equal(inplace, grad)
    # the reference's launcher: probabilities written back, loss added atomically
    probs = logits.clone()
    grad2 = torch.empty_like(logits)
    loss2 = torch.full((1,), 0.25, device=device)
    ops.ops_lib().launch_fused_chunked_logit_ce(P(probs), P(targets), P(grad2), P(loss2), rows, vocab, total)
    torch.cuda.synchronize()
    close(probs.double(), lp.exp(), 1e-5, 1e-9, "probabilities")
    assert torch.equal(grad2, grad)
    close(loss2.double(), 0.25 + want_rows.sum()[None], 1e-5, 1e-8, "atomic loss")


# ---------------------------------------------------------------- embedding (elementwise.cu:255-298)
def test_embedding_forward_and_backward_match_torch(device):
    """Gather of table rows; the gradient adds every position's row into its token's table row,
    repeated ids included (fp64 index_add as the reference), accumulating onto what the table
    gradient held, reproducibly; ids past the table are zero rows / skipped."""
    import torch

    say("embedding S=1024 d=768, vocab 50257 with repeated ids")
    g = torch.Generator(device="cpu").manual_seed(99)
    vocab, dim, seq = 50257, 768, 1024
    table = torch.randn(vocab, dim, generator=g).to(device)
    ids = torch.randint(0, 300, (seq,), generator=g, dtype=torch.int32)  # many repeats
    ids[5] = ids[900] = ids[1023] = 7
    ids = ids.to(device)
    out = torch.empty(seq, dim, device=device)
    ops.embedding_forward(ids, table, out)
    torch.cuda.synchronize()
    assert torch.equal(out, table.index_select(0, ids.long()))
    gy = torch.randn(seq, dim, generator=g).to(device)
    base = torch.randn(vocab, dim, generator=g).to(device) * 0.1
    gt = base.clone()
    ops.embedding_backward(ids, gy, gt)
    want = base.double().index_add(0, ids.long(), gy.double())
    torch.cuda.synchronize()
    close(gt.double(), want, 1e-6, 1e-5, "table gradient")
    again = base.clone()
    ops.embedding_backward(ids, gy, again)
    torch.cuda.synchronize()
    assert torch.equal(again, gt)
    # positions (unique ids, the position table's gradient)
    pos = torch.arange(seq, dtype=torch.int32, device=device)
    gp = torch.zeros(seq, dim, device=device)
    ops.embedding_backward(pos, gy, gp)
    torch.cuda.synchronize()
    assert torch.equal(gp, gy)
    # ids past the table
    bad = ids.clone()
    bad[3] = vocab + 5
    out2 = torch.empty_like(out)
    ops.embedding_forward(bad, table, out2)
    gt2 = torch.zeros(vocab, dim, device=device)
    ops.embedding_backward(bad, gy, gt2)
    torch.cuda.synchronize()
    assert torch.all(out2[3] == 0) and torch.equal(out2[4], out[4])
    keep = torch.ones(seq, dtype=torch.bool)
    keep[3] = False
    want2 = torch.zeros(vocab, dim, dtype=torch.float64).index_add(0, ids.long().cpu()[keep], gy.double().cpu()[keep])
    close(gt2.double().cpu(), want2, 1e-6, 1e-5, "table gradient, one id past the table")
    # the reference's launchers on the null stream
    out3 = torch.empty_like(out)
    gt3 = base.clone()
    ops.ops_lib().launch_embedding_forward(P(ids), P(table), P(out3), seq, dim)
    ops.ops_lib().launch_embedding_backward(P(ids), P(gy), P(gt3), seq, dim)
    dfattn.darkforest_sync()
    assert torch.equal(out3, out) and torch.equal(gt3, gt)


@pytest.mark.parametrize("rows,f", LN_SHAPES)
def test_add_layernorm_is_the_add_then_the_layernorm(device, rows, f):
    """dfgpt2_add_layernorm_forward: sum_out is x + y bit for bit and out is the LayerNorm of it
    bit for bit (the same kernel as dfgpt2_layernorm_forward); out also against torch."""
    import torch

    say(f"add+layernorm rows={rows} f={f}")
    g = torch.Generator(device="cpu").manual_seed(rows * 7 + f)
    x = (torch.randn(rows, f, generator=g) * 2).to(device)
    y = (torch.randn(rows, f, generator=g) + 0.25).to(device)
    gamma, beta = torch.randn(f, generator=g).to(device), torch.randn(f, generator=g).to(device)
    s, out = torch.empty_like(x), torch.empty_like(x)
    stats = torch.empty((2, rows), device=device)
    ops.add_layer_norm_forward_into(x, y, gamma, beta, s, out, stats)
    want_out, want_m, want_r = ops.layer_norm_forward(x + y, gamma, beta)
    torch.cuda.synchronize()
    assert torch.equal(s, x + y)
    assert torch.equal(out, want_out) and torch.equal(stats[0], want_m) and torch.equal(stats[1], want_r)
    ref = torch.nn.functional.layer_norm(x + y, (f,), gamma, beta, 1e-5)
    close(out, ref, 1e-5, 1e-5, "add+layernorm vs torch")


@pytest.mark.parametrize("rows,cols", [(1024, 2304), (7, 13), (3, 4)])
@pytest.mark.parametrize("offset", [0, 1])
def test_elementwise_launchers_are_the_torch_ops(device, rows, cols, offset):
    """dfgpt2_add_bias (out of place and in place) and the reference's launch_add_bias, launch_add,
    launch_scale and launch_fill: one fp32 operation per value, so bit for bit torch's; offset 1
    starts every tensor one float into its buffer (not 16-byte aligned: the value-by-value path)."""
    import torch

    say(f"elementwise rows={rows} cols={cols} offset={offset}")
    g = torch.Generator(device="cpu").manual_seed(rows + cols + offset)
    n = rows * cols
    buf = lambda: torch.randn(n + 1, generator=g).to(device)
    x, y, bias = buf()[offset:offset + n].view(rows, cols), buf()[offset:offset + n], buf()[offset:offset + cols]
    out = torch.full_like(x, float("nan"))
    ops.add_bias_into(x, bias, out)
    torch.cuda.synchronize()
    assert torch.equal(out, x + bias)
    inplace = x.clone()
    ops.add_bias_into(inplace, bias)
    lib = ops.ops_lib()
    ref_out = torch.full_like(x, float("nan"))
    lib.launch_add_bias(P(x), P(bias), P(ref_out), rows, cols)
    xf = x.reshape(-1)
    c = torch.full_like(y, float("nan"))
    lib.launch_add(P(xf), P(y), P(c), n)
    s = torch.full_like(y, float("nan"))
    lib.launch_scale(P(xf), 0.37, P(s), n)
    f = torch.full_like(y, float("nan"))
    lib.launch_fill(P(f), -2.5, n)
    dfattn.darkforest_sync()
    assert torch.equal(inplace, x + bias) and torch.equal(ref_out, x + bias)
    assert torch.equal(c, xf + y) and torch.equal(s, 0.37 * xf) and bool((f == -2.5).all())


@pytest.mark.parametrize("rows,f", LN_SHAPES + [(5, 100), (1030, 1024)])
@pytest.mark.parametrize("residual,bias", [(True, True), (False, True), (True, False)])
def test_fused_layernorm_backward_is_the_separate_calls(device, rows, f, residual, bias):
    """dfgpt2_layernorm_backward_fused: grad_x bit for bit the separate dfgpt2_layernorm_backward_residual's,
    the parameter gradients and grad_x's column sums (the next bias gradient) against float64 sums
    of the same products, all three written over what their buffers held, bitwise reproducible;
    the partial-sum workspace filled with NaN first (nothing in it is read before written)."""
    import torch

    say(f"fused layernorm backward rows={rows} f={f} residual={residual} bias={bias}")
    g = torch.Generator(device="cpu").manual_seed(rows * 7 + f)
    x, dy = torch.randn(rows, f, generator=g).to(device), torch.randn(rows, f, generator=g).to(device)
    res = torch.randn(rows, f, generator=g).to(device) if residual else None
    gamma, beta = torch.randn(f, generator=g).to(device), torch.randn(f, generator=g).to(device)
    _, m, r = ops.layer_norm_forward(x, gamma, beta)
    stats = torch.stack([m, r])
    gx0 = torch.empty_like(x)
    gg0, gb0 = torch.empty(f, device=device), torch.empty(f, device=device)
    ops.layer_norm_backward_residual_into(dy, x, gamma, stats, res, gx0, gg0, gb0)
    ws = torch.full((ops.layer_norm_backward_fused_workspace_bytes(rows, f) // 4,), float("nan"), device=device)
    outs = []
    for _ in range(2):
        gx = torch.full_like(x, float("nan"))
        gg, gb = torch.full((f,), 7.0, device=device), torch.full((f,), -3.0, device=device)
        gbias = torch.full((f,), 5.0, device=device) if bias else None
        ops.layer_norm_backward_fused_into(dy, x, gamma, stats, res, gx, gg, gb, gbias, ws)
        torch.cuda.synchronize()
        outs.append((gx, gg, gb, gbias))
    gx, gg, gb, gbias = outs[0]
    assert torch.equal(gx, gx0)
    xh = (x.double() - m.double()[:, None]) * r.double()[:, None]
    n = max(rows, 1) ** 0.5
    close(gg.double(), (dy.double() * xh).sum(0), 0, 2e-5 * n, "grad gamma")
    close(gb.double(), dy.double().sum(0), 0, 2e-5 * n, "grad beta")
    if bias:
        close(gbias.double(), gx0.double().sum(0), 0, 2e-5 * n * max(1.0, gx0.abs().max().item()), "grad bias")
    for a, b2 in zip(outs[0], outs[1]):
        assert a is None or torch.equal(a, b2)


@pytest.mark.parametrize("rows,f", LN_SHAPES)
def test_layernorm_backward_residual_adds_and_overwrites(device, rows, f):
    """dfgpt2_layernorm_backward_residual: grad_x is dfgpt2_layernorm_backward's plus the residual
    (one fp32 add), the parameter gradients are written over whatever their buffers held."""
    import torch

    say(f"layernorm backward + residual rows={rows} f={f}")
    g = torch.Generator(device="cpu").manual_seed(rows * 5 + f)
    x, dy = torch.randn(rows, f, generator=g).to(device), torch.randn(rows, f, generator=g).to(device)
    res = torch.randn(rows, f, generator=g).to(device)
    gamma, beta = torch.randn(f, generator=g).to(device), torch.randn(f, generator=g).to(device)
    _, m, r = ops.layer_norm_forward(x, gamma, beta)
    gx0, gg0, gb0 = ops.layer_norm_backward(dy, x, gamma, m, r)
    gx = torch.empty_like(x)
    gg, gb = torch.full((f,), 7.0, device=device), torch.full((f,), -3.0, device=device)
    stats = torch.stack([m, r])
    ops.layer_norm_backward_residual_into(dy, x, gamma, stats, res, gx, gg, gb)
    torch.cuda.synchronize()
    assert torch.equal(gx, gx0 + res)
    assert torch.equal(gg, gg0) and torch.equal(gb, gb0)
    # without a residual: grad_x alone
    ops.layer_norm_backward_residual_into(dy, x, gamma, stats, None, gx, gg, gb)
    torch.cuda.synchronize()
    assert torch.equal(gx, gx0)


@pytest.mark.parametrize("rows,cols", [(1024, 3072), (7, 13), (5, 8)])
def test_bias_gelu_is_the_bias_add_then_gelu(device, rows, cols):
    """dfgpt2_bias_gelu_forward: h becomes h + bias (per column) bit for bit, out = gelu of it bit for
    bit (dfgpt2_gelu_forward's function); also against torch's tanh GELU."""
    import torch

    say(f"bias+gelu rows={rows} cols={cols}")
    h = torch.randn(rows, cols, device=device) * 3
    b = torch.randn(cols, device=device)
    want_h = h + b
    want = ops.gelu_forward(want_h)
    out = torch.empty_like(h)
    ops.bias_gelu_forward_into(h, b, out)
    torch.cuda.synchronize()
    assert torch.equal(h, want_h) and torch.equal(out, want)
    close(out, torch.nn.functional.gelu(want_h, approximate="tanh"), 1e-5, 1e-6, "bias+gelu vs torch")



@pytest.mark.parametrize("dim", [768, 771])
def test_embedding_backward_sums_a_heavily_repeated_id_in_a_fixed_order(device, dim):
    """S = 8192 with one id (a padding token) at 6000 positions and the rest random. The table row of
    that id is, bit for bit, ((s0 + s1) + s2) + s3, where s_w is the float32 sum, in increasing
    position, of its rows in the 64-position blocks b = w (mod 4) (the owner's four waves); the
    other rows equal index_add within fp32 rounding. dim 771 takes the unaligned scalar path."""
    import numpy as np
    import torch

    say(f"embedding backward S=8192 d={dim}, id 3 at 6000 positions")
    g = torch.Generator(device="cpu").manual_seed(7)
    vocab, seq = 5000, 8192
    ids = torch.randint(0, vocab, (seq,), generator=g, dtype=torch.int32)
    pad = torch.randperm(seq, generator=g)[:6000]
    ids[pad] = 3
    gy = torch.randn(seq, dim, generator=g)
    base = (torch.randn(vocab, dim, generator=g) * 0.1)
    gt = base.to(device)
    ops.embedding_backward(ids.to(device), gy.to(device), gt)
    torch.cuda.synchronize()
    part = np.zeros((4, dim), np.float32)
    for q in np.nonzero(ids.numpy() == 3)[0]:  # increasing positions
        part[(q // 64) % 4] = part[(q // 64) % 4] + gy.numpy()[q]
    total = ((part[0] + part[1]) + part[2]) + part[3]
    got = gt.cpu().numpy()
    assert np.array_equal(got[3], base.numpy()[3] + total)
    want = base.double().index_add(0, ids.long(), gy.double())
    keep = torch.ones(vocab, dtype=torch.bool)
    keep[3] = False
    close(torch.from_numpy(got)[keep].double(), want[keep], 1e-6, 1e-5, "other rows")
