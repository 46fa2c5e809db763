"""One GPU's share of sequence (context) parallel attention, built from the C ABI.

A sequence of 2*B rows is split into two shards of B rows, as G = 2 GPUs would
hold it. Under causal masking the three non-empty (query shard, key shard)
blocks are: the two diagonal blocks (causal) and the off-diagonal block of
shard 1's queries against shard 0's keys (no mask). Each block is one call of
the ordinary entry points with seq_len = B:

* forward: every block yields (O_b, lse_b); a query shard's blocks merge with
  the logsumexp identity lse = log(sum_b exp(lse_b)),
  O = sum_b exp(lse_b - lse) O_b (the same algebra as the reference's split-K
  decode reduce, attention_fused.cu:714-760);
* backward: every block runs dfattn_bwd with the *merged* O and lse of its
  query rows (so P and Delta are the global ones), and a shard's dQ, dK, dV
  are the sums of its blocks' contributions.

The merged results must match the oracle's single causal attention over the
whole 2*B sequence to the north star's bar.
"""
import numpy as np
import pytest

import dfattn
import oracle as O
from conftest import oracle_threads
from test_gpu_parity import MAX_ABS, REL_L2, assert_close, host, say, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("block", [512, 1000])
def test_two_shard_causal_attention_matches_the_whole_sequence(device, block):
    import torch

    H, D, scale = 12, 64, 0.125
    B = block
    say(f"context-parallel shards: 2 x {B} rows, H={H}")
    x = O.seeded_inputs(2 * B, H, D, 9000 + B)
    shard = lambda a, i: np.ascontiguousarray(a[i * B:(i + 1) * B])  # noqa: E731
    q = [to_dev(shard(x["q"], i), device) for i in range(2)]
    k = [to_dev(shard(x["k"], i), device) for i in range(2)]
    v = [to_dev(shard(x["v"], i), device) for i in range(2)]
    g = [to_dev(shard(x["do"], i), device) for i in range(2)]
    # (query shard, key shard, causal) of the non-empty blocks
    blocks = [(0, 0, True), (1, 0, False), (1, 1, True)]

    fwd = {(i, j): dfattn.attention_forward(q[i], k[j], v[j], H, scale, causal) for i, j, causal in blocks}
    o_glob, lse_glob = [], []
    for i in range(2):
        parts = [(fwd[(ii, j)]) for ii, j, _ in blocks if ii == i]
        lse_stack = torch.stack([lse for _, lse in parts])        # [blocks, H, B]
        lse = torch.logsumexp(lse_stack, dim=0)                    # [H, B]
        w = torch.exp(lse_stack - lse)                             # [blocks, H, B]
        o = sum(part_o.view(B, H, D) * wb.t().unsqueeze(-1) for (part_o, _), wb in zip(parts, w))
        o_glob.append(o.reshape(B, H * D).contiguous())
        lse_glob.append(lse.contiguous())

    dq = [torch.zeros_like(q[0]) for _ in range(2)]
    dk = [torch.zeros_like(k[0]) for _ in range(2)]
    dv = [torch.zeros_like(v[0]) for _ in range(2)]
    for i, j, causal in blocks:
        bq, bk, bv = dfattn.attention_backward(q[i], k[j], v[j], o_glob[i], g[i], lse_glob[i], H, scale, causal)
        dq[i] += bq
        dk[j] += bk
        dv[j] += bv
    torch.cuda.synchronize()

    got = {"o": np.concatenate([host(t) for t in o_glob]),
           "lse": np.concatenate([host(t) for t in lse_glob], axis=1),
           "dq": np.concatenate([host(t) for t in dq]),
           "dk": np.concatenate([host(t) for t in dk]),
           "dv": np.concatenate([host(t) for t in dv])}
    t = oracle_threads()
    o_ref, lse_ref = O.mha_forward(x["q"], x["k"], x["v"], H, scale, True, threads=t)
    dq_ref, dk_ref, dv_ref = O.backward(x["q"], x["k"], x["v"], x["do"], H, scale, True, threads=t)
    want = {"o": o_ref, "lse": lse_ref, "dq": dq_ref, "dk": dk_ref, "dv": dv_ref}
    report = {n: assert_close(f"2x{B} {n}", got[n], want[n], MAX_ABS, REL_L2) for n in want}
    say(f"2x{B}: " + ", ".join(f"{n} {a:.1e}/{r:.1e}" for n, (a, r) in report.items()))
