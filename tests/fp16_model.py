"""A float64 model of the roundings the d_head = 64 MFMA path applies (test infrastructure).

The HIP kernels (dark-forest_amd/csrc/attn_fwd_d64.hip, attn_bwd_d64.hip) round their matrix
operands to fp16 and accumulate in fp32. This module recomputes causal (or full) attention and its
gradients in float64, rounding to fp16 (numpy's round-to-nearest-even) at exactly the points
where the kernels round, and nowhere else:

* forward: c2*Q with c2 = fp32(scale * log2(e)), rounded to fp32 and then to fp16 (the kernels'
  round_scaled4); K and V to fp16; P = exp2(S - m) rounded to fp16 both for O's product and for
  the row sum l (the forward adds the same fp16 P); O = sum(P V) / l, lse = (m + log2 l) ln 2.
  m is taken as the row maximum: the kernel's reference point may sit up to 8 below it, and a
  power-of-two shift commutes with fp16 rounding of normal numbers;
* backward: each 64-row block of dO times its power-of-two scale sigma_b (the kernels'
  block_scale) rounded to fp16; Delta from exactly those rounded values and the forward's O;
  P = exp2(S - lse log2 e) and dS = P (dP - Delta) from the same S; fp16(P) and fp16(dS) into
  dV, dK and dQ. Under causal masking rows 0-63 also add their rounding residues
  lo = fp16(x - fp16(x)) of sigma_b*dO, c2*Q and dS to dV and dK (the kernels' kLoRows:
  dV += P^T dO_lo, dK += dS^T (c2 Q)_lo + dS_lo^T (c2 Q)), and rows 0-127 those of K and dS
  over keys 0-63 to dQ (dQ += dS K_lo + dS_lo K); `lo_rows=0` leaves them out.

With `rounding=False` every rounding is the identity and the model is exact attention in float64
(tests/test_fp16_model.py checks it against the oracle's float64 twin). The model exists to pin
what fp16 operands cost against the fp32 oracle: it reproduces the GPU's errors (the fixture
tests/golden/parity_margin_c1_c2.json holds both for 16 seeds at C1 and C2) and predicts them for
seeds and shapes no GPU run has covered. It is never imported by the product path.
"""
from __future__ import annotations

import numpy as np

LOG2E_F32 = float(np.float32(1.4426950408889634))
LN2 = float(np.log(2.0))


def _f16(a, rounding=True):
    return a.astype(np.float16).astype(np.float64) if rounding else a


def block_scale(amax: float) -> float:
    """The dO scale of one 64-row block (attn_bwd_d64.hip block_scale): 2^e with e = 1 (mod 4) and
    max|2^e x| in [2, 32); 1 for a zero or non-finite maximum."""
    if not (amax > 0.0) or not np.isfinite(amax):
        return 1.0
    e_fine = 3 - int(np.frexp(np.float32(amax))[1] - 1)  # ilogb
    e = e_fine - 2 + (((3 - e_fine) % 4) + 4) % 4
    return float(np.ldexp(1.0, max(-123, min(125, e))))


def attention(q, k, v, d_out, n_heads, scale, causal=True, rounding=True, backward=True, lo_rows=64):
    """O [S, H*D], lse [H, S] and, with backward=True, dQ, dK, dV [S, H*D] (float64) of the model."""
    q, k, v = (np.asarray(t, np.float32) for t in (q, k, v))
    S, HD = q.shape
    D = HD // n_heads
    c2 = np.float32(np.float32(scale) * np.float32(LOG2E_F32))
    out = {name: np.zeros((S, HD)) for name in (("o", "dq", "dk", "dv") if backward else ("o",))}
    out["lse"] = np.zeros((n_heads, S))
    mask = np.tril(np.ones((S, S), bool)) if causal else None
    for h in range(n_heads):
        cols = slice(h * D, (h + 1) * D)
        if rounding:
            q16 = (q[:, cols] * c2).astype(np.float32).astype(np.float16).astype(np.float64)
        else:
            q16 = q[:, cols].astype(np.float64) * float(scale) * np.log2(np.e)
        k16, v16 = _f16(k[:, cols].astype(np.float64), rounding), _f16(v[:, cols].astype(np.float64), rounding)
        s = q16 @ k16.T  # log2 domain
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        p16 = _f16(np.exp2(s - m), rounding)
        l = p16.sum(axis=1, keepdims=True)
        o = (p16 @ v16) / l
        lse = (m[:, 0] + np.log2(l[:, 0])) * LN2
        out["o"][:, cols] = o
        out["lse"][h] = lse
        if not backward:
            continue
        g = np.asarray(d_out, np.float32)[:, cols]
        sig = np.ones(S)
        if rounding:
            for b0 in range(0, S, 64):
                sig[b0:b0 + 64] = block_scale(float(np.max(np.abs(g[b0:b0 + 64]))))
            g16 = (g * sig[:, None].astype(np.float32)).astype(np.float32).astype(np.float16).astype(np.float64)
        else:
            g16 = g.astype(np.float64)
        o32 = o.astype(np.float32).astype(np.float64) if rounding else o
        delta = (g16 * o32).sum(axis=1)
        lse2 = (lse.astype(np.float32) * np.float32(LOG2E_F32)).astype(np.float64) if rounding else lse / LN2
        p = np.exp2(s - lse2[:, None])
        dp = g16 @ v16.T
        ds = p * (dp - delta[:, None])
        p16b, ds16 = _f16(p, rounding), _f16(ds, rounding)
        # The residues of rows 0 .. R-1 (causal only).
        R = min(lo_rows, S) if (rounding and causal) else 0
        glo, qlo, dslo = np.zeros((R, D)), np.zeros((R, D)), np.zeros((R, S))
        if R:
            gx = (g[:R] * sig[:R, None].astype(np.float32)).astype(np.float64)
            glo = _f16(gx - g16[:R])
            qx = (q[:R, cols] * c2).astype(np.float32).astype(np.float64)
            qlo = _f16(qx - q16[:R])
            dslo = _f16(ds[:R] - ds16[:R])
        # dV = P^T dO / sigma, dK = scale dS^T Q (= ln2 dS^T (c2 Q)), dQ = scale dS K / sigma (per row).
        # Every 64-row block of N(0,1)-like dO has the same sigma, so the dK/dV sums divide once.
        if rounding and not np.all(sig == sig[0]):
            inv = (1.0 / sig)[:, None]
            out["dv"][:, cols] = p16b.T @ (g16 * inv) + p16b[:R].T @ (glo * inv[:R])
            out["dk"][:, cols] = LN2 * ((ds16 * inv).T @ q16 + (dslo * inv[:R]).T @ q16[:R]
                                        + (ds16[:R] * inv[:R]).T @ qlo)
        else:
            out["dv"][:, cols] = (p16b.T @ g16 + p16b[:R].T @ glo) / sig[0]
            out["dk"][:, cols] = LN2 * (ds16.T @ q16 + dslo.T @ q16[:R] + ds16[:R].T @ qlo) / sig[0]
        dq = ds16 @ k16
        if R:
            rq = min(2 * lo_rows, S)
            klo = _f16(k[:R, cols].astype(np.float64) - k16[:R])
            dq[:rq] += _f16(ds[:rq, :R] - ds16[:rq, :R]) @ k16[:R] + ds16[:rq, :R] @ klo
        out["dq"][:, cols] = float(scale) * dq / sig[:, None]
        del s, p, dp, ds, p16b, ds16, p16
    return out
