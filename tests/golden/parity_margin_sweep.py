"""Parity margin at the BASELINE training shapes: max-abs / rel-L2 errors of O, lse, dQ, dK, dV
against the fp32 oracle for 16 seeds each of C1 (H=12, S=1024) and C2 (H=12, S=4096).

  python tests/golden/parity_margin_sweep.py --model   # the fp16 rounding model (CPU, tests/fp16_model.py)
  python tests/golden/parity_margin_sweep.py --gpu     # the HIP training pair (dfattn_fwd_train,
                                                       # dfattn_bwd_preprocess, dfattn_bwd_main)

Each run merges its rows into tests/golden/parity_margin_c1_c2.json (keyed by source, shape and
seed), which tests/test_fp16_model.py reads. Seeds: 2000 + 50 k (C1) and 3000 + 100 k (C2),
k = 0..15 (C2's first 1024 rows of seed s are C1's inputs of seed s, so the two ranges do not
overlap); 2000, 2500, 3000 and 3500 are the seeds tests/test_gpu_parity.py runs.
"""
import argparse
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for sub in ("tests", "oracle", "dark-forest_amd"):
    sys.path.insert(0, os.path.join(ROOT, sub))
OUT = os.path.join(HERE, "parity_margin_c1_c2.json")
SHAPES = {"C1": (1024, 2000, 50), "C2": (4096, 3000, 100)}
H, D, SCALE = 12, 64, 0.125
NAMES = ("o", "lse", "dq", "dk", "dv")


def errors(got, want):
    res = {}
    for n in NAMES:
        g, w = np.asarray(got[n], np.float64), np.asarray(want[n], np.float64)
        res[n] = [float(np.max(np.abs(g - w))), float(np.linalg.norm(g - w) / np.linalg.norm(w))]
    return res


def oracle_ref(x, threads):
    import oracle as O

    o, lse = O.mha_forward(x["q"], x["k"], x["v"], H, SCALE, True, threads=threads)
    dq, dk, dv = O.backward(x["q"], x["k"], x["v"], x["do"], H, SCALE, True, threads=threads)
    return {"o": o, "lse": lse, "dq": dq, "dk": dk, "dv": dv}


def model_row(args):
    import oracle as O
    import fp16_model

    shape, seed, threads = args
    S = SHAPES[shape][0]
    x = O.seeded_inputs(S, H, D, seed)
    got = fp16_model.attention(x["q"], x["k"], x["v"], x["do"], H, SCALE, True)
    return f"model/{shape}/{seed}", errors(got, oracle_ref(x, threads))


def gpu_rows(seeds):
    import oracle as O
    import torch

    import dfattn

    dev = torch.device("cuda:0")
    rows = {}
    for shape, seed in seeds:
        S = SHAPES[shape][0]
        x = O.seeded_inputs(S, H, D, seed)
        q, k, v, g = (torch.from_numpy(x[n]).to(dev) for n in ("q", "k", "v", "do"))
        ws = torch.full((dfattn.bwd_workspace_bytes(H, S, D) // 4,), float("nan"), device=dev)
        o, lse = dfattn.forward_train(q, k, v, H, ws, SCALE, True)
        grads = [torch.empty_like(q) for _ in range(3)]
        dfattn.backward_preprocess(q, k, v, o, g, lse, ws, H, SCALE, flags=dfattn.BWD_QKV_SAVED)
        dfattn.backward_main(q, k, v, o, g, lse, *grads, ws, H, SCALE, True)
        torch.cuda.synchronize()
        got = {"o": o.cpu().numpy(), "lse": lse.cpu().numpy(), "dq": grads[0].cpu().numpy(),
               "dk": grads[1].cpu().numpy(), "dv": grads[2].cpu().numpy()}
        rows[f"gpu/{shape}/{seed}"] = errors(got, oracle_ref(x, 16))
        print(f"gpu {shape} seed {seed}: dv {rows[f'gpu/{shape}/{seed}']['dv'][0]:.3e}", flush=True)
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", action="store_true")
    ap.add_argument("--gpu", action="store_true")
    ap.add_argument("--seeds", type=int, default=16)
    ap.add_argument("--workers", type=int, default=4)
    ap.add_argument("--out", default=OUT, help="the JSON file to merge the rows into")
    args = ap.parse_args()
    seeds = [(shape, base + step * i) for shape, (_, base, step) in SHAPES.items() for i in range(args.seeds)]
    table = json.load(open(args.out)) if os.path.exists(args.out) else {}
    if args.model:
        from multiprocessing import Pool

        os.environ.setdefault("OMP_NUM_THREADS", "2")
        with Pool(args.workers) as pool:
            for key, row in pool.imap_unordered(model_row, [(s, sd, 2) for s, sd in seeds]):
                table[key] = row
                print(f"{key}: dv {row['dv'][0]:.3e} dk {row['dk'][0]:.3e}", flush=True)
    if args.gpu:
        table.update(gpu_rows(seeds))
    with open(args.out, "w") as f:
        json.dump(dict(sorted(table.items())), f, indent=0)
        f.write("\n")


if __name__ == "__main__":
    main()
