"""Child process of tests/test_zz_no_alloc.py (GPU): the process's first dfattn_bwd_noalloc call
is made under torch.cuda.graph capture.

That first call looks up the static array's address, which makes the runtime place the array.
The capture must succeed, and each replay must give dfattn_bwd's gradients bit for bit, on
inputs changed between the replays. It prints one line per step and exits 0 on success.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("dark-forest_amd", "oracle"):
    sys.path.insert(0, os.path.join(ROOT, sub))

import torch  # noqa: E402

import dfattn  # noqa: E402
import oracle as O  # noqa: E402


def say(msg):
    print(f"[no-alloc capture] {msg}", flush=True)


def main():
    H, D, S = 12, 64, 1024
    device = torch.device("cuda:0")
    x = O.seeded_inputs(S, H, D, 12300)
    q, k, v, g = (torch.from_numpy(x[n]).to(device) for n in ("q", "k", "v", "do"))
    o, lse = dfattn.attention_forward(q, k, v, H, 0.125, True)
    got = [torch.full_like(q, float("nan")) for _ in range(3)]
    torch.cuda.synchronize()
    say(f"H={H} S={S}: first dfattn_bwd_noalloc call of the process, under capture")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dfattn.attention_backward_noalloc(q, k, v, o, g, lse, H, 0.125, True, *got)
    say("captured")
    for rep in range(3):
        y = O.seeded_inputs(S, H, D, 12400 + rep)
        for dst, name in zip((q, k, v, g), ("q", "k", "v", "do")):
            dst.copy_(torch.from_numpy(y[name]).to(device))
        o2, l2 = dfattn.attention_forward(q, k, v, H, 0.125, True)
        o.copy_(o2)
        lse.copy_(l2)
        graph.replay()
        torch.cuda.synchronize()
        want = dfattn.attention_backward(q, k, v, o, g, lse, H, 0.125, True)
        torch.cuda.synchronize()
        for name, a, b in zip(("dQ", "dK", "dV"), got, want):
            if not torch.equal(a, b):
                say(f"replay {rep}: {name} differs from dfattn_bwd")
                return 1
        say(f"replay {rep}: dQ, dK, dV equal to dfattn_bwd")
    return 0


if __name__ == "__main__":
    sys.exit(main())
