"""Pins the CPU oracle (oracle/attention_oracle.c) before it is trusted as the parity checker.

Checks, each against something other than the oracle's own formula:
  * the reference's known-answer tests (darkforest-cuda/src/lib.rs:2605-2628,
    :2752-2829) with expected values from PyTorch float64 (tests/golden/);
  * the reference's finite-difference check of the backward (lib.rs:2786-2828);
  * multi-head golden cases (PyTorch float64) for the [S, H*D] layout;
  * closed forms and invariants the mathematics fixes;
  * an independent vectorised float64 numpy implementation;
  * planted mistakes in the oracle, each of which must fail at least one check.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O
from conftest import GOLDEN, max_abs

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def load_json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def load_case(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


MHA_CASES = ["mha_h3_s7_d5_causal", "mha_h2_s20_d64_causal", "mha_h2_s20_d64_full", "mha_h1_s9_d128_causal"]


# ---------------------------------------------------------------- independent numpy fp64 implementation
def numpy_attention(q, k, v, d_out, n_heads, scale, causal):
    """Vectorised float64 attention forward/backward (matrix form, no loops over rows)."""
    seq_len, dm = q.shape
    d = dm // n_heads
    f = lambda a: np.asarray(a, np.float64).reshape(seq_len, n_heads, d).transpose(1, 0, 2)
    Q, K, V = f(q), f(k), f(v)
    s = scale * Q @ K.transpose(0, 2, 1)
    if causal:
        s = np.where(np.triu(np.ones((seq_len, seq_len), bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    lse = (m + np.log(e.sum(-1, keepdims=True)))[..., 0]
    p = e / e.sum(-1, keepdims=True)
    o = p @ V
    back = lambda t: t.transpose(1, 0, 2).reshape(seq_len, dm)
    res = {"o": back(o), "lse": lse}
    if d_out is not None:
        G = f(d_out)
        dp = G @ V.transpose(0, 2, 1)
        ds = p * (dp - (p * dp).sum(-1, keepdims=True))
        res["dq"] = back(scale * ds @ K)
        res["dk"] = back(scale * ds.transpose(0, 2, 1) @ Q)
        res["dv"] = back(p.transpose(0, 2, 1) @ G)
    return res


# ---------------------------------------------------------------- the pinning checks, as functions
def check_kat_forward(tol=1e-5):
    kat = load_json("kat_forward.json")
    q, k, v = (np.array(kat[n], np.float32) for n in ("q", "k", "v"))
    out = O.reference_attention(q, k, v, kat["scale"], True)
    o_mha, lse = O.mha_forward(q, k, v, 1, kat["scale"], True)
    exp_o = np.array(kat["expected_o"])
    exp_lse = np.array(kat["expected_lse"])[0]
    errs = [max_abs(out, exp_o), max_abs(o_mha, exp_o), max_abs(lse[0], exp_lse)]
    return [f"kat_forward err {e:.2e}" for e in errs if not e <= tol]


def check_kat_backward(tol=1e-5):
    kat = load_json("kat_backward.json")
    q, k, v, g = (np.array(kat[n], np.float32) for n in ("q", "k", "v", "d_out"))
    dq, dk, dv = O.backward(q, k, v, g, 1, kat["scale"], True)
    fails = []
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        e = max_abs(got, np.array(kat["expected_" + name]))
        if not e <= tol:
            fails.append(f"kat_backward {name} err {e:.2e}")
    return fails


def check_finite_difference(delta=1e-3, tol=2e-3):
    """The reference's check (lib.rs:2786-2828): objective = sum(O * dO)."""
    kat = load_json("kat_backward.json")
    q, k, v, g = (np.array(kat[n], np.float32) for n in ("q", "k", "v", "d_out"))
    sc = kat["scale"]
    grads = O.backward(q, k, v, g, 1, sc, True)

    def objective(qq, kk, vv):
        o, _ = O.mha_forward(qq, kk, vv, 1, sc, True)
        return float(np.sum(o.astype(np.float64) * g))

    fails = []
    for which, analytical in zip(range(3), grads):
        base = [q, k, v]
        for idx in range(q.size):
            plus = [a.copy() for a in base]
            minus = [a.copy() for a in base]
            plus[which].flat[idx] += np.float32(delta)
            minus[which].flat[idx] -= np.float32(delta)
            numerical = (objective(*plus) - objective(*minus)) / (2 * delta)
            if not abs(analytical.flat[idx] - numerical) <= tol:
                fails.append(f"fd input {which} idx {idx}: {analytical.flat[idx]} vs {numerical}")
    return fails


def check_mha_golden(tol=2e-5):
    fails = []
    for name in MHA_CASES:
        c = load_case(name)
        h, s, d, causal = (int(x) for x in c["meta"])
        sc = float(c["scale"][0])
        o, lse = O.mha_forward(c["in_q"], c["in_k"], c["in_v"], h, sc, causal)
        dq, dk, dv = O.backward(c["in_q"], c["in_k"], c["in_v"], c["in_do"], h, sc, causal)
        for key, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            e = max_abs(got, c["exp_" + key])
            if not e <= tol:
                fails.append(f"{name} {key} err {e:.2e}")
    return fails


def check_closed_forms():
    fails = []
    x = O.seeded_inputs(40, 3, 16, 11)
    h, sc = 3, 0.25
    o, lse = O.mha_forward(x["q"], x["k"], x["v"], h, sc, True)
    dq, dk, dv = O.backward(x["q"], x["k"], x["v"], x["do"], h, sc, True)
    # Row 0 sees only key 0: O_0 = V_0, lse_0 = scale q_0.k_0, dQ_0 = 0.
    if max_abs(o[0], x["v"][0]) > 1e-6:
        fails.append("O_0 != V_0")
    for hd in range(h):
        sl = slice(hd * 16, hd * 16 + 16)
        want = sc * float(np.dot(x["q"][0, sl].astype(np.float64), x["k"][0, sl]))
        if abs(lse[hd, 0] - want) > 1e-5:
            fails.append("lse_0 != scale q0.k0")
    if max_abs(dq[0], 0.0) > 1e-6:
        fails.append("dQ_0 != 0")
    # sum_j dK_j = 0 (rows of dS sum to zero); sum_j dV_j = sum_i dO_i (rows of P sum to one).
    if max_abs(dk.astype(np.float64).sum(0), 0.0) > 1e-4:
        fails.append("sum_j dK_j != 0")
    if max_abs(dv.astype(np.float64).sum(0), x["do"].astype(np.float64).sum(0)) > 1e-4:
        fails.append("sum_j dV_j != sum_i dO_i")
    # q = 0: uniform weights, O_i = mean_{j<=i} V_j and lse_i = ln(i+1).
    z = np.zeros_like(x["q"])
    o0, lse0 = O.mha_forward(z, x["k"], x["v"], h, sc, True)
    means = np.cumsum(x["v"].astype(np.float64), 0) / np.arange(1, 41)[:, None]
    if max_abs(o0, means) > 1e-5:
        fails.append("q=0: O != running mean of V")
    if max_abs(lse0, np.log(np.arange(1, 41))[None, :].repeat(h, 0)) > 1e-5:
        fails.append("q=0: lse != ln(i+1)")
    # Constant V gives constant O.
    cv = np.full_like(x["v"], 0.75)
    oc, _ = O.mha_forward(x["q"], x["k"], cv, h, sc, True)
    if max_abs(oc, 0.75) > 1e-6:
        fails.append("V const: O != const")
    return fails


def check_numpy_reference(tol32=2e-5):
    fails = []
    for causal in (True, False):
        x = O.seeded_inputs(65, 2, 64, 5 + int(causal))
        sc = 0.125
        ref = numpy_attention(x["q"], x["k"], x["v"], x["do"], 2, sc, causal)
        o32, lse32 = O.mha_forward(x["q"], x["k"], x["v"], 2, sc, causal)
        g32 = O.backward(x["q"], x["k"], x["v"], x["do"], 2, sc, causal)
        o64, lse64 = O.mha_forward(x["q"], x["k"], x["v"], 2, sc, causal, dtype=np.float64)
        g64 = O.backward(x["q"], x["k"], x["v"], x["do"], 2, sc, causal, dtype=np.float64)
        pairs = [("o", o32, o64), ("lse", lse32, lse64)] + [
            (n, a, b) for n, a, b in zip(("dq", "dk", "dv"), g32, g64)]
        for name, a32, a64 in pairs:
            e32, e64 = max_abs(a32, ref[name]), max_abs(a64, ref[name])
            if not e32 <= tol32:
                fails.append(f"numpy {name} fp32 err {e32:.2e}")
            if not e64 <= 1e-11:
                fails.append(f"numpy {name} fp64 err {e64:.2e}")
    return fails


ALL_CHECKS = [check_kat_forward, check_kat_backward, check_mha_golden, check_closed_forms,
              check_numpy_reference, check_finite_difference]


# ---------------------------------------------------------------- tests
@pytest.mark.parametrize("check", ALL_CHECKS, ids=lambda f: f.__name__)
def test_oracle_pinned(check):
    O.set_mutation("none")
    assert check() == []


def test_kat_reference_tolerance():
    """The reference's own bars: 2e-4 forward and backward, FD 2e-3."""
    assert check_kat_forward(tol=load_json("kat_forward.json")["tolerance"]) == []
    assert check_kat_backward(tol=load_json("kat_backward.json")["tolerance"]) == []


@pytest.mark.parametrize("mutation", [m for m in O.MUTATIONS if m != "none" and m not in O.AUX_MUTATIONS])
def test_planted_mistake_is_caught(mutation):
    """Every planted mistake must fail at least one pinning check."""
    O.set_mutation(mutation)
    try:
        fails = []
        for check in ALL_CHECKS[:-1]:  # the FD check is slow; the others catch everything
            fails += check()
    finally:
        O.set_mutation("none")
    assert fails, f"mutation {mutation} passed every check"


def test_threads_do_not_change_bits():
    x = O.seeded_inputs(130, 4, 64, 9)
    a = O.mha_forward(x["q"], x["k"], x["v"], 4, 0.125, True, threads=1)
    b = O.mha_forward(x["q"], x["k"], x["v"], 4, 0.125, True, threads=4)
    ga = O.backward(x["q"], x["k"], x["v"], x["do"], 4, 0.125, True, threads=1)
    gb = O.backward(x["q"], x["k"], x["v"], x["do"], 4, 0.125, True, threads=4)
    for u, w in zip(a + ga, b + gb):
        assert np.array_equal(u, w)


def test_heads_are_independent_single_head_runs():
    """H-head result == H single-head runs on the de-interleaved columns, bit for bit."""
    h, d = 3, 8
    x = O.seeded_inputs(33, h, d, 21)
    o, lse = O.mha_forward(x["q"], x["k"], x["v"], h, 0.3, True)
    g = O.backward(x["q"], x["k"], x["v"], x["do"], h, 0.3, True)
    for hd in range(h):
        sl = slice(hd * d, (hd + 1) * d)
        oh, lh = O.mha_forward(x["q"][:, sl], x["k"][:, sl], x["v"][:, sl], 1, 0.3, True)
        gh = O.backward(x["q"][:, sl], x["k"][:, sl], x["v"][:, sl], x["do"][:, sl], 1, 0.3, True)
        assert np.array_equal(o[:, sl], oh) and np.array_equal(lse[hd], lh[0])
        for full, part in zip(g, gh):
            assert np.array_equal(full[:, sl], part)


def test_row_sampled_forward_matches_full():
    x = O.seeded_inputs(300, 2, 64, 31, with_grad=False)
    o, lse = O.mha_forward(x["q"], x["k"], x["v"], 2, 0.125, True)
    rows = np.array([0, 1, 63, 64, 150, 299])
    orows, lrows = O.mha_forward_rows(x["q"], x["k"], x["v"], rows, 2, 0.125, True, threads=2)
    assert np.array_equal(orows, o[rows])
    assert np.array_equal(lrows, lse[:, rows].T)


def test_fp32_oracle_error_vs_fp64_is_tiny():
    """The fp32 restatement is ~1e-6 from exact, far inside the 2e-3 / 1e-3 parity bar."""
    x = O.seeded_inputs(256, 2, 64, 77)
    o32, l32 = O.mha_forward(x["q"], x["k"], x["v"], 2, 0.125, True)
    o64, l64 = O.mha_forward(x["q"], x["k"], x["v"], 2, 0.125, True, dtype=np.float64)
    assert max_abs(o32, o64) < 1e-5 and max_abs(l32, l64) < 1e-5
    g32 = O.backward(x["q"], x["k"], x["v"], x["do"], 2, 0.125, True)
    g64 = O.backward(x["q"], x["k"], x["v"], x["do"], 2, 0.125, True, dtype=np.float64)
    for a, b in zip(g32, g64):
        assert max_abs(a, b) < 1e-4


def test_seeded_inputs_are_reproducible():
    a = O.seeded_inputs(8, 2, 4, 3)
    b = O.seeded_inputs(8, 2, 4, 3)
    assert all(np.array_equal(a[n], b[n]) for n in a)
    assert not np.array_equal(a["q"], a["k"])
    assert math.isclose(float(O.seeded_inputs(4096, 1, 64, 1, with_grad=False)["q"].std()), 1.0, rel_tol=0.02)


# ---------------------------------------------------------------- decode (attention_fused.cu:551-1033)
def _paged_pool(rows, page_size, seed):
    """Scatter `rows` into a pool of pages in a random physical order; returns (pool, block_table)."""
    n = rows.shape[0]
    n_pages = (n + page_size - 1) // page_size
    perm = np.random.default_rng(seed).permutation(n_pages + 3)[:n_pages].astype(np.int32)
    pool = np.random.default_rng(seed + 1).standard_normal(((n_pages + 3) * page_size, rows.shape[1])).astype(
        rows.dtype) if rows.dtype != np.uint16 else np.zeros(((n_pages + 3) * page_size, rows.shape[1]), np.uint16)
    for lp in range(n_pages):
        m = min(page_size, n - lp * page_size)
        pool[perm[lp] * page_size: perm[lp] * page_size + m] = rows[lp * page_size: lp * page_size + m]
    return pool, perm


@pytest.mark.parametrize("cur_len", [1, 2, 63, 64, 65, 300])
def test_decode_is_the_causal_forward_of_the_last_row(cur_len):
    """Decode of query i over keys 0..i is row i of the (separately pinned) causal forward."""
    H, D = 4, 64
    x = O.seeded_inputs(cur_len, H, D, 7100 + cur_len, with_grad=False)
    o, lse = O.mha_forward(x["q"], x["k"], x["v"], H, 0.125, True, dtype=np.float64)
    i = cur_len - 1
    d64, l64 = O.decode(x["q"][i], x["k"], x["v"], H, cur_len, 0.125, dtype=np.float64)
    assert np.abs(d64 - o[i]).max() < 1e-12 and np.abs(l64 - lse[:, i]).max() < 1e-12
    d32, l32 = O.decode(x["q"][i], x["k"], x["v"], H, cur_len, 0.125)
    assert np.abs(d32 - o[i]).max() < 2e-6 and np.abs(l32 - lse[:, i]).max() < 2e-6


def test_decode_matches_torch_float64_sdpa():
    torch = pytest.importorskip("torch")
    H, D, S = 3, 32, 77
    x = O.seeded_inputs(S, H, D, 7200, with_grad=False)
    q = torch.from_numpy(x["q"][S - 1].astype(np.float64)).view(1, H, 1, D)
    k = torch.from_numpy(x["k"].astype(np.float64)).view(S, H, D).permute(1, 0, 2).unsqueeze(0)
    v = torch.from_numpy(x["v"].astype(np.float64)).view(S, H, D).permute(1, 0, 2).unsqueeze(0)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.2).reshape(-1).numpy()
    got, _ = O.decode(x["q"][S - 1], x["k"], x["v"], H, S, 0.2, dtype=np.float64)
    assert np.abs(got - want).max() < 1e-12


@pytest.mark.parametrize("page_size", [1, 7, 16])
def test_decode_paged_equals_contiguous(page_size):
    H, D, S = 2, 64, 100
    x = O.seeded_inputs(S, H, D, 7300, with_grad=False)
    pk, table = _paged_pool(x["k"], page_size, 1)
    pv, table_v = _paged_pool(x["v"], page_size, 1)
    assert np.array_equal(table, table_v)
    want = O.decode(x["q"][5], x["k"], x["v"], H, S, 0.125)
    got = O.decode(x["q"][5], pk, pv, H, S, 0.125, block_table=table, page_size=page_size)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_decode_bf16_pool_is_the_widened_values():
    H, D, S = 2, 64, 90
    x = O.seeded_inputs(S, H, D, 7400, with_grad=False)
    kb, vb = O.to_bf16_bits(x["k"]), O.to_bf16_bits(x["v"])
    # bf16 conversion round trip is exact for values already representable, and rounds to nearest
    assert np.array_equal(O.to_bf16_bits(O.from_bf16_bits(kb)), kb)
    assert np.abs(O.from_bf16_bits(kb) - x["k"]).max() <= np.abs(x["k"]).max() * 2.0 ** -8
    got = O.decode(x["q"][0], kb, vb, H, S, 0.125)
    want = O.decode(x["q"][0], O.from_bf16_bits(kb), O.from_bf16_bits(vb), H, S, 0.125)
    assert np.array_equal(got[0], want[0])


def test_decode_closed_forms():
    H, D, S = 2, 16, 40
    x = O.seeded_inputs(S, H, D, 7500, with_grad=False)
    out, lse = O.decode(x["q"][0], x["k"], x["v"], H, 1, 0.5)
    assert np.array_equal(out, x["v"][0])  # one key: P = 1
    qk = (x["q"][0].reshape(H, D).astype(np.float64) * x["k"][0].reshape(H, D)).sum(1) * 0.5
    assert np.abs(lse - qk).max() < 1e-5
    out, lse = O.decode(np.zeros(H * D, np.float32), x["k"], x["v"], H, S, 0.5)  # q = 0: the mean of V
    assert np.abs(out - x["v"].mean(0)).max() < 1e-5 and np.abs(lse - math.log(S)).max() < 1e-5
    assert O.decode(x["q"][0], x["k"], x["v"], H, 0, 0.5) == (None, None)  # nothing computed
