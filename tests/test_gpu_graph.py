"""The attention entry points recorded into a HIP graph and replayed.

The bench's step (dfattn_fwd_train, dfattn_bwd_preprocess with DFATTN_BWD_QKV_SAVED,
dfattn_bwd_main) and the no-allocation backward (dfattn_bwd_noalloc) are captured once on
static buffers. Each replay follows new inputs copied into those buffers and unrelated eager work
with a synchronisation, and every replay's outputs must equal, bit for bit, the same calls made
eagerly on the same inputs into separate outputs. The launches record no memset, and the
backward's schedule rides in the kernel arguments, so a replay has nothing stale to reuse.
"""
import pytest

import dfattn

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-graph] {msg}", flush=True)


def _inputs(S, d_model, seed, device):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    return [torch.randn(S, d_model, generator=g).to(device) for _ in range(4)]


@pytest.mark.parametrize("S", [1024, 4096])
def test_training_step_graph_replays_match_eager_calls(device, S):
    import torch

    H, D = 12, 64
    say(f"training fwd + phase 1 + main in a graph, H={H} S={S}")
    q, k, v, do = _inputs(S, H * D, 100, device)
    ws = torch.empty(dfattn.bwd_workspace_bytes(H, S, D) // 4, dtype=torch.float32, device=device)
    out, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
    lse = torch.empty(H, S, dtype=torch.float32, device=device)

    def step():
        dfattn.forward_train(q, k, v, H, ws, out=out, lse=lse)
        dfattn.backward_preprocess(q, k, v, out, do, lse, ws, H, flags=dfattn.BWD_QKV_SAVED)
        dfattn.backward_main(q, k, v, out, do, lse, dq, dk, dv, ws, H)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()

    ws2 = torch.empty_like(ws)
    for rep in range(3):
        for dst, src in zip((q, k, v, do), _inputs(S, H * D, 200 + rep, device)):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (out, lse, dq, dk, dv)]
        o2, l2 = dfattn.forward_train(q, k, v, H, ws2)
        dfattn.backward_preprocess(q, k, v, o2, do, l2, ws2, H, flags=dfattn.BWD_QKV_SAVED)
        want = [o2, l2] + [torch.empty_like(q) for _ in range(3)]
        dfattn.backward_main(q, k, v, o2, do, l2, want[2], want[3], want[4], ws2, H)
        _ = torch.ones(1 << 20, device=device).sum().item()  # unrelated eager work between replays
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "lse", "dQ", "dK", "dV"), got, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager calls"
        say(f"replay {rep}: O, lse, dQ, dK, dV equal to the eager calls")


def test_noalloc_backward_graph_replays_match_eager_calls(device):
    import torch

    H, D, S = 12, 64, 2048
    say(f"dfattn_bwd_noalloc in a graph, H={H} S={S}")
    q, k, v, do = _inputs(S, H * D, 300, device)
    out, lse = dfattn.attention_forward(q, k, v, H)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))

    def bwd():
        dfattn.attention_backward_noalloc(q, k, v, out, do, lse, H, d_q=dq, d_k=dk, d_v=dv)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        bwd()  # the first call on the device also finds the static array's address
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        bwd()

    for rep in range(3):
        q2, k2, v2, do2 = _inputs(S, H * D, 400 + rep, device)
        for dst, src in zip((q, k, v, do), (q2, k2, v2, do2)):
            dst.copy_(src)
        o2, l2 = dfattn.attention_forward(q, k, v, H)
        out.copy_(o2)
        lse.copy_(l2)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (dq, dk, dv)]
        want = dfattn.attention_backward_noalloc(q, k, v, out, do, lse, H)
        torch.cuda.synchronize()
        for name, a, b in zip(("dQ", "dK", "dV"), got, want):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
        say(f"replay {rep}: dQ, dK, dV equal to the eager call")
