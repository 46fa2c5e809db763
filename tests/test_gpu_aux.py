"""GPU parity of the elementwise kernels beside the decode family (attention_fused.cu:1098-1231).

Through the reference's own symbols (null stream, errors at darkforest_sync), against the oracle:
  * position interpolation and both paged row copies: bit-exact (no FMA contraction on either side;
    the bf16 rounding is the same round-to-nearest-even, NaN included);
  * RoPE: pos 0 is the identity bit for bit and pair norms are kept to 1e-6; otherwise the oracle's
    fp32 result within 1e-6 * (1 + r) + r * angle * 2^-21 per value, where r is the pair's norm: powf
    on the GPU and in libm may differ by an ulp or two, and an angle of pos * theta moves by
    pos * ulp(theta), which the rotation turns into r times that much.
"""
import numpy as np
import pytest

import dfattn
import oracle as O
from test_gpu_parity import host, say, to_dev

pytestmark = pytest.mark.gpu


def dev_any(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@pytest.mark.parametrize("d_model", [1, 768, 1000])
def test_pos_embed_interpolate_bit_exact(device, d_model):
    import torch

    trained = 1024
    table = np.random.default_rng(20 + d_model).standard_normal((trained, d_model)).astype(np.float32)
    dt = to_dev(table, device)
    out = torch.empty(d_model, device=device)
    for pos, max_ctx in ((0, 1024), (5, 1024), (1023, 1024), (0, 8192), (1, 8192), (4000, 8192), (8191, 8192),
                         (9000, 8192), (3000, 1024), (777, 3001), (131071, 131072)):
        say(f"pos_embed d_model={d_model} pos={pos} max={max_ctx}")
        out.fill_(float("nan"))
        dfattn.launch_pos_embed_interpolate(dt, out, pos, trained, max_ctx, d_model)
        dfattn.darkforest_sync()
        want = O.pos_embed_interpolate(table, pos, trained, max_ctx)
        assert np.array_equal(host(out), want), f"pos {pos} max {max_ctx}"


@pytest.mark.parametrize("n_heads,d_head,base", [(12, 64, 10000.0), (1, 128, 10000.0), (5, 7, 500.0),
                                                 (40, 64, 1e6)])
def test_apply_rope(device, n_heads, d_head, base):
    x = np.random.default_rng(30 + d_head).standard_normal(n_heads * d_head).astype(np.float32)
    half = d_head // 2
    for pos in (0, 1, 17, 4095, 131071):
        say(f"rope H={n_heads} D={d_head} base={base} pos={pos}")
        qk = to_dev(x, device)
        dfattn.launch_apply_rope(qk, pos, n_heads, d_head, base)
        dfattn.darkforest_sync()
        got = host(qk)
        if pos == 0:
            assert np.array_equal(got, x)
            continue
        want = O.apply_rope(x, pos, n_heads, d_head, base)
        r = np.ones_like(x)
        xr = x.reshape(n_heads, d_head)
        rr = r.reshape(n_heads, d_head)
        pair_r = np.hypot(xr[:, 0:2 * half:2], xr[:, 1:2 * half:2])
        rr[:, 0:2 * half:2] = pair_r
        rr[:, 1:2 * half:2] = pair_r
        theta = (base ** (-2.0 * np.arange(half) / d_head)).astype(np.float64)
        ang = np.zeros((n_heads, d_head))
        ang[:, 0:2 * half:2] = pos * theta
        ang[:, 1:2 * half:2] = pos * theta
        tol = 1e-6 * (1 + r) + r * ang.reshape(-1) * 2.0 ** -21
        assert np.all(np.abs(got - want) <= tol), f"pos {pos}: max err {np.abs(got - want).max():.2e}"
        gr = got.reshape(n_heads, d_head)
        out_r = np.hypot(gr[:, 0:2 * half:2], gr[:, 1:2 * half:2])
        assert np.abs(out_r - pair_r).max() <= 1e-6 * (1 + pair_r.max())
        if d_head % 2:
            assert np.array_equal(gr[:, -1], xr[:, -1])


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("d_model", [768, 1000, 3])
def test_paged_copy_row_bit_exact(device, bf16, d_model):
    page, n_blocks = 16, 5
    rng = np.random.default_rng(40 + d_model)
    rows = rng.standard_normal((6, d_model)).astype(np.float32)
    if bf16:  # ties, overflow, subnormals, infinities and NaN in the first row
        sp = np.array([1.00390625, 1.01171875, 3.4028235e38, 1e-40, np.inf, -np.inf, np.nan, -0.0], np.float32)
        rows[0, :min(d_model, sp.size)] = sp[:min(d_model, sp.size)]
    dtype = np.uint16 if bf16 else np.float32
    sentinel = np.full((n_blocks * page, d_model), 0x5a5a if bf16 else 7.0, dtype)
    want = sentinel.copy()
    pool = dev_any(sentinel.view(np.int16) if bf16 else sentinel, device)
    for i, (blk, off) in enumerate(((3, 0), (3, 15), (0, 7), (4, 15), (1, 1), (3, 1))):
        say(f"paged copy bf16={bf16} d_model={d_model} block={blk} offset={off}")
        src = to_dev(rows[i], device)
        if bf16:
            dfattn.launch_paged_copy_row_f32_to_bf16(src, pool, blk, off, page, d_model)
        else:
            dfattn.launch_paged_copy_row(src, pool, blk, off, page, d_model)
        O.paged_copy_row(rows[i], want, blk, off, page)
    dfattn.darkforest_sync()
    got = host(pool).view(np.uint16) if bf16 else host(pool)
    assert np.array_equal(got.view(np.uint32 if not bf16 else np.uint16), want.view(np.uint32 if not bf16 else np.uint16))


def test_paged_append_then_bf16_decode(device):
    """The engine's decode step (paged_kv.rs:288-303, then attention_fused.cu:1075): rows appended one at a
    time into a bf16 pool on the GPU, then decoded from it, equal the oracle's decode of the rounded rows."""
    import torch

    H, D, S, page = 12, 64, 300, 16
    x = O.seeded_inputs(S, H, D, 50, with_grad=False)
    n_pages = (S + page - 1) // page
    table = np.random.default_rng(51).permutation(n_pages + 4)[:n_pages].astype(np.int32)
    pk = torch.zeros((n_pages + 4) * page * H * D, dtype=torch.int16, device=device)
    pv = torch.zeros_like(pk)
    dk, dv = to_dev(x["k"], device), to_dev(x["v"], device)
    say(f"append {S} rows into a bf16 pool, then decode")
    for t in range(S):
        blk, off = int(table[t // page]), t % page
        dfattn.launch_paged_copy_row_f32_to_bf16(dk[t], pk, blk, off, page, H * D)
        dfattn.launch_paged_copy_row_f32_to_bf16(dv[t], pv, blk, off, page, H * D)
    out = torch.full((H * D,), float("nan"), device=device)
    dfattn.launch_paged_mha_decode_kv_bf16(to_dev(x["q"][S - 1], device), pk, pv, dev_any(table, device), out, H, S,
                                           D, 0.125, page)
    dfattn.darkforest_sync()
    want, _ = O.decode(x["q"][S - 1], O.to_bf16_bits(x["k"]), O.to_bf16_bits(x["v"]), H, S, 0.125)
    err = np.abs(host(out) - want).max()
    assert err <= 2e-5, f"max-abs {err:.2e}"
