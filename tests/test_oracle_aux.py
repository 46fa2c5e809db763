"""Pins the oracle's elementwise restatements (attention_fused.cu:1098-1231) before they check the GPU.

Each check compares with something other than the oracle's own formula:
  * position interpolation: the trained-range copy, a table linear in the position (on which linear
    interpolation is exact up to rounding), hand-worked midpoints, and the endpoints;
  * RoPE: the textbook complex form z_i * exp(i * pos * base^(-2i/d)) in float64 numpy, pos 0 = identity,
    preserved pair norms, rotations composing (pos a then b = pos a + b);
  * bf16 rounding: torch's own float -> bfloat16 conversion (round to nearest even) on ties, overflow,
    subnormals, infinities and NaN;
  * paged copy: rows written one by one are the pool oracle.decode reads as the contiguous cache.
Planted mistakes in the C restatement (oracle.AUX_MUTATIONS) must each fail one of these checks.
"""
import numpy as np
import pytest

import oracle as O


# ---------------------------------------------------------------- checks (each returns a list of failures)
def check_interpolation():
    fails = []
    rng = np.random.default_rng(11)
    trained, d = 16, 40
    table = rng.standard_normal((trained, d)).astype(np.float32)
    for pos in (0, 5, 15):  # inside the trained range and max <= trained: the row itself
        if not np.array_equal(O.pos_embed_interpolate(table, pos, trained, trained), table[pos]):
            fails.append(f"copy pos {pos}")
    # linear table: row p = a + p * b, so interpolation at x is a + x * b
    a = rng.standard_normal(d).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    lin = (a[None, :] + np.arange(trained, dtype=np.float32)[:, None] * b[None, :]).astype(np.float32)
    for max_ctx in (31, 64, 1000):
        for pos in (0, 1, 7, max_ctx // 2, max_ctx - 2, max_ctx - 1):
            x = pos * (trained - 1) / (max_ctx - 1)
            want = a.astype(np.float64) + x * b.astype(np.float64)
            got = O.pos_embed_interpolate(lin, pos, trained, max_ctx)
            if np.abs(got - want).max() > 1e-4 * (1 + np.abs(want).max()):
                fails.append(f"linear max {max_ctx} pos {pos}")
    # hand-worked: trained 3, max 5 -> positions 0, .5, 1, 1.5, 2
    t3 = np.array([[0.0, 10.0], [2.0, 30.0], [4.0, 70.0]], np.float32)
    for pos, want in ((0, [0, 10]), (1, [1, 20]), (2, [2, 30]), (3, [3, 50]), (4, [4, 70])):
        if not np.allclose(O.pos_embed_interpolate(t3, pos, 3, 5), want, atol=1e-6):
            fails.append(f"hand-worked pos {pos}")
    # past the last row: the last row
    if not np.array_equal(O.pos_embed_interpolate(t3, 9, 3, 5), t3[2]):
        fails.append("past the table")
    if not np.array_equal(O.pos_embed_interpolate(t3, 7, 3, 3), t3[2]):
        fails.append("pos >= trained with max == trained")
    return fails


def rope_complex(x, pos, n_heads, d_head, base):
    """Textbook RoPE: pairs as complex numbers times exp(i * pos * base^(-2i/d)), float64."""
    x = np.asarray(x, np.float64).reshape(n_heads, d_head)
    half = d_head // 2
    z = x[:, 0:2 * half:2] + 1j * x[:, 1:2 * half:2]
    theta = base ** (-2.0 * np.arange(half) / d_head)
    z = z * np.exp(1j * pos * theta)[None, :]
    out = x.copy()
    out[:, 0:2 * half:2], out[:, 1:2 * half:2] = z.real, z.imag
    return out.reshape(-1)


def check_rope():
    fails = []
    rng = np.random.default_rng(12)
    for n_heads, d_head, base in ((12, 64, 10000.0), (3, 7, 500.0), (2, 128, 1e6)):
        x = rng.standard_normal(n_heads * d_head).astype(np.float32)
        if not np.array_equal(O.apply_rope(x, 0, n_heads, d_head, base), x):
            fails.append(f"pos 0 H{n_heads} D{d_head}")
        for pos in (1, 3, 100, 4095):
            want = rope_complex(x, pos, n_heads, d_head, base)
            got64 = O.apply_rope(x, pos, n_heads, d_head, base, dtype=np.float64)
            got32 = O.apply_rope(x, pos, n_heads, d_head, base)
            if np.abs(got64 - want).max() > 1e-9:
                fails.append(f"f64 vs complex pos {pos} D{d_head}")
            # fp32: the angle pos * theta carries about pos * 2^-24 of error
            if np.abs(got32 - want).max() > 1e-5 + 3 * pos * 2.0 ** -24 * np.abs(x).max():
                fails.append(f"f32 vs complex pos {pos} D{d_head}")
            half = d_head // 2
            r_in = np.hypot(x[0:2 * half:2], x[1:2 * half:2])
            r_out = np.hypot(got32[0:2 * half:2], got32[1:2 * half:2])
            if np.abs(r_out - r_in).max() > 1e-5:
                fails.append(f"norm pos {pos}")
        # rotations compose
        ab = O.apply_rope(O.apply_rope(x, 20, n_heads, d_head, base, np.float64), 30, n_heads, d_head, base,
                          np.float64)
        if np.abs(ab - O.apply_rope(x, 50, n_heads, d_head, base, np.float64)).max() > 1e-9:
            fails.append("composition")
    return fails


BF16_SPECIALS = np.array([
    0.0, -0.0, 1.0, -1.0, 1.00390625, 1.01171875,            # exact ties: to even (down), to even (up)
    1.0 + 2 ** -8 + 2 ** -20, 1.0 + 2 ** -9, 3.4028235e38,  # above a tie; below; FLT_MAX overflows to inf
    3.3895314e38, 1e-40, -1e-40, 1.1754944e-38, 9.2e-41,    # bf16 max; subnormals; FLT_MIN
    np.inf, -np.inf, 65504.0, 3.14159265, -2.71828182, 1e-30], np.float32)


def check_bf16():
    torch = pytest.importorskip("torch")
    fails = []
    rng = np.random.default_rng(13)
    vals = np.concatenate([BF16_SPECIALS, rng.standard_normal(5000).astype(np.float32),
                           (rng.standard_normal(3000) * 1e30).astype(np.float32),
                           rng.integers(0, 2 ** 32, 3000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    finite = vals[~np.isnan(vals)]
    want = torch.from_numpy(finite.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16(finite)
    if not np.array_equal(got, want):
        bad = np.nonzero(got != want)[0][:3]
        fails.append(f"bf16 rounding differs from torch at {finite[bad]}")
    nans = np.array([0x7fc00000, 0xffc00001, 0x7f800001, 0x7fbfffff], np.uint32).view(np.float32)
    gn = O.f32_to_bf16(nans)
    if not np.all(np.isnan(O.from_bf16_bits(gn))):
        fails.append("NaN not kept")
    if not np.array_equal(gn >> 15, (nans.view(np.uint32) >> 31).astype(np.uint16)):
        fails.append("NaN sign")
    return fails


def check_paged_copy():
    fails = []
    H, D, S, page = 2, 32, 45, 8
    x = O.seeded_inputs(S, H, D, 14, with_grad=False)
    n_pages = (S + page - 1) // page
    table = np.random.default_rng(15).permutation(n_pages + 2)[:n_pages].astype(np.int32)
    for bf16 in (False, True):
        dtype = np.uint16 if bf16 else np.float32
        pk = np.zeros(((n_pages + 2) * page, H * D), dtype)
        pv = np.zeros_like(pk)
        for t in range(S):  # paged_kv.rs:206-209 and 288-303: one row per decoded position
            O.paged_copy_row(x["k"][t], pk, table[t // page], t % page, page)
            O.paged_copy_row(x["v"][t], pv, table[t // page], t % page, page)
        kc = O.to_bf16_bits(x["k"]) if bf16 else x["k"]
        vc = O.to_bf16_bits(x["v"]) if bf16 else x["v"]
        want = O.decode(x["q"][S - 1], kc, vc, H, S, 0.125)
        got = O.decode(x["q"][S - 1], pk, pv, H, S, 0.125, block_table=table, page_size=page)
        if not (np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])):
            fails.append(f"paged copy then decode, bf16={bf16}")
        used = np.zeros(pk.shape[0], bool)
        for t in range(S):
            used[table[t // page] * page + t % page] = True
        if np.any(pk[~used] != 0):
            fails.append(f"rows outside the written ones changed, bf16={bf16}")
    return fails


AUX_CHECKS = [check_interpolation, check_rope, check_bf16, check_paged_copy]


@pytest.mark.parametrize("check", AUX_CHECKS, ids=lambda f: f.__name__)
def test_aux_oracle_pinned(check):
    O.set_mutation("none")
    assert check() == []


@pytest.mark.parametrize("mutation", O.AUX_MUTATIONS)
def test_aux_planted_mistake_is_caught(mutation):
    O.set_mutation(mutation)
    try:
        fails = [f for check in AUX_CHECKS for f in check()]
    finally:
        O.set_mutation("none")
    assert fails, f"mutation {mutation} passed every check"


def test_numpy_bf16_helper_agrees_on_finite_values():
    """tests use oracle.to_bf16_bits (vectorised) for finite data; it must equal the C rounding there."""
    x = np.concatenate([BF16_SPECIALS[np.isfinite(BF16_SPECIALS)],
                        np.random.default_rng(16).standard_normal(2000).astype(np.float32)])
    x = x[np.abs(x) < 3.3e38]
    assert np.array_equal(O.to_bf16_bits(x), O.f32_to_bf16(x))
