"""GPT-2 training step around the fused attention: the harness that reports "GPT-2 step ms".

Mirrors the reference's static engine step (darkforest-core/src/engine/static_gpt2.rs):

* model (static_gpt2.rs:276-567): learned token and position embeddings, L
  pre-LayerNorm blocks (LN eps 1e-5, darkforest-cuda/kernels/layernorm.cu:14),
  Q/K/V/O projections with biases, tanh-GELU MLP (elementwise.cu:181-192),
  final LayerNorm and an untied lm_head [vocab, d_model];
* initialisation (static_gpt2.rs:285-319): weights N(0, 0.02), the residual
  projections Wo and W2 N(0, 0.02 / sqrt(2 L)), LayerNorm gamma 1 / beta 0,
  biases 0 — drawn from a seeded generator (the reference's thread_rng is
  unseeded, static_gpt2.rs:264-271);
* step (static_gpt2.rs:1375-1696): forward, mean cross-entropy over the S
  positions, backward, AdamW with beta (0.9, 0.95), eps 1e-8 and weight decay
  0.1 on every parameter (static_gpt2.rs:518-521; update rule lib.rs:1755-1788);
* attention: per layer the fused causal kernel with scale (d_model/H)^-0.5
  (static_gpt2.rs:1291, 1329-1336, 1500-1510) — here dfattn's fast path through
  FusedCausalAttention, which keeps the forward's O and logsumexp for the
  backward.

On the GPU the step's other kernels are this library's too (dfattn.ops, include/dfgpt2.h):
LayerNorm forward and backward, tanh GELU, the linear layers' bias gradients and AdamW over one
arena holding every weight, gradient and moment (the engine's single allocation), all fp32; the
GEMMs are hipBLASLt fp32. On the CPU (the checkpoint tests' twin) the same model runs on PyTorch's
operators and optimizer. `attention="sdpa"`
swaps in torch's scaled_dot_product_attention (the reference's own parity
comparator, scripts/verify_loss_parity.py:58) for loss-parity checks.
"""
from __future__ import annotations

import math
import struct
import time

from . import FusedCausalAttention
from . import ops as _ops


def _torch():
    import torch

    return torch


class StaticGPT2:
    """GPT-2 with the reference engine's architecture, init and optimizer."""

    def __init__(self, vocab_size=50257, d_model=768, n_heads=12, n_layers=12, d_ff=3072, seq_len=1024, lr=3e-4,
                 seed=0, device="cuda", attention="dfattn", capturable=False):
        torch = _torch()
        if d_model % n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        if d_model // n_heads > 128:
            raise ValueError(f"StaticGPT2 head dimension must be <= 128, got {d_model // n_heads}")
        if attention not in ("dfattn", "sdpa"):
            raise ValueError("attention must be 'dfattn' or 'sdpa'")
        self.vocab_size, self.d_model, self.n_heads = vocab_size, d_model, n_heads
        self.n_layers, self.d_ff, self.seq_len = n_layers, d_ff, seq_len
        self.attention = attention
        self.device = torch.device(device)
        gen = torch.Generator(device="cpu").manual_seed(seed)
        std, std_res = 0.02, 0.02 / math.sqrt(2.0 * n_layers)

        def randn(*shape, s=std):
            return (torch.randn(*shape, generator=gen) * s).to(self.device).requires_grad_(True)

        def const(v, *shape):
            return torch.full(shape, float(v), device=self.device).requires_grad_(True)

        self.tok_emb = randn(vocab_size, d_model)
        self.pos_emb = randn(seq_len, d_model)
        self.layers = []
        for _ in range(n_layers):
            self.layers.append({
                "ln1_g": const(1, d_model), "ln1_b": const(0, d_model),
                "wq": randn(d_model, d_model), "bq": const(0, d_model),
                "wk": randn(d_model, d_model), "bk": const(0, d_model),
                "wv": randn(d_model, d_model), "bv": const(0, d_model),
                "wo": randn(d_model, d_model, s=std_res), "bo": const(0, d_model),
                "ln2_g": const(1, d_model), "ln2_b": const(0, d_model),
                "w1": randn(d_ff, d_model), "b1": const(0, d_ff),
                "w2": randn(d_model, d_ff, s=std_res), "b2": const(0, d_model),
            })
        self.ln_f_g = const(1, d_model)
        self.ln_f_b = const(0, d_model)
        self.lm_head = randn(vocab_size, d_model)
        # The engine keeps its hyper-parameters as f32 (static_gpt2.rs:518-521), which its checkpoint
        # footer stores; holding the same f32 values makes a resumed run continue bit for bit.
        f32 = lambda x: struct.unpack("<f", struct.pack("<f", x))[0]  # noqa: E731
        # On the GPU: one arena for weights, gradients and moments, the AdamW update in one launch
        # (the engine's update is one kernel per tensor, lib.rs:1755-1788), the step count on the
        # device, so a step can always be recorded into a graph. On the CPU: torch's AdamW.
        self.native = self.device.type == "cuda"
        hp = dict(lr=f32(lr), betas=(f32(0.9), f32(0.95)), eps=f32(1e-8), weight_decay=f32(0.1))
        if self.native:
            arena = _ops.ParamArena(self.parameters(), self.device)
            self._rebind(arena.adopt(self.parameters()))
            self.opt = _ops.ArenaAdamW(arena, self.parameters(), **hp)
        else:
            self.opt = torch.optim.AdamW(self.parameters(), **hp, capturable=capturable)
        self._graph = None

    def parameters(self):
        ps = [self.tok_emb, self.pos_emb]
        for lw in self.layers:
            ps += list(lw.values())
        return ps + [self.ln_f_g, self.ln_f_b, self.lm_head]

    def _rebind(self, tensors):
        """Replace the parameters (in parameters() order) with `tensors`."""
        it = iter(tensors)
        self.tok_emb, self.pos_emb = next(it), next(it)
        for lw in self.layers:
            for key in lw:
                lw[key] = next(it)
        self.ln_f_g, self.ln_f_b, self.lm_head = next(it), next(it), next(it)

    def load_state(self, other: "StaticGPT2"):
        """Copy another instance's weights (the parity harness loads identical weights into both)."""
        torch = _torch()
        with torch.no_grad():
            for a, b in zip(self.parameters(), other.parameters()):
                a.copy_(b)

    def _attention(self, q, k, v):
        torch = _torch()
        scale = (self.d_model / self.n_heads) ** -0.5
        if self.attention == "dfattn":
            return FusedCausalAttention.apply(q, k, v, self.n_heads, scale, True)
        s, h, d = q.shape[0], self.n_heads, self.d_model // self.n_heads
        qh, kh, vh = (t.view(s, h, d).transpose(0, 1).contiguous() for t in (q, k, v))
        o = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
        return o.transpose(0, 1).reshape(s, h * d)

    def loss(self, tokens, targets):
        """Mean cross-entropy of one sequence (static_gpt2.rs:1386-1418)."""
        F = _torch().nn.functional
        if self.native:
            # the parameter gradients go straight into the arena (ops: direct accumulation)
            ln = lambda t, g, b: _ops.layer_norm(t, g, b, direct=True)  # noqa: E731
            lin = lambda t, w, b=None: _ops.linear(t, w, b, direct=True)  # noqa: E731
            gelu = _ops.gelu
            x = _ops.embedding(self.tok_emb, tokens, direct=True)
        else:
            d = self.d_model
            ln = lambda t, g, b: F.layer_norm(t, (d,), g, b, 1e-5)  # noqa: E731
            lin, gelu = F.linear, lambda t: F.gelu(t, approximate="tanh")  # noqa: E731
            x = self.tok_emb[tokens]
        x = x + self.pos_emb[:tokens.shape[0]]
        for lw in self.layers:
            h = ln(x, lw["ln1_g"], lw["ln1_b"])
            q = lin(h, lw["wq"], lw["bq"])
            k = lin(h, lw["wk"], lw["bk"])
            v = lin(h, lw["wv"], lw["bv"])
            x = x + lin(self._attention(q, k, v), lw["wo"], lw["bo"])
            h = ln(x, lw["ln2_g"], lw["ln2_b"])
            x = x + lin(gelu(lin(h, lw["w1"], lw["b1"])), lw["w2"], lw["b2"])
        h = ln(x, self.ln_f_g, self.ln_f_b)
        return F.cross_entropy(lin(h, self.lm_head), targets)

    def step(self, tokens, targets):
        """One training step: forward, loss, backward, AdamW. Returns the loss tensor (not synchronised)."""
        self.opt.zero_grad(set_to_none=False)
        loss = self.loss(tokens, targets)
        loss.backward()
        self.opt.step()
        return loss.detach()


    def capture(self, tokens, targets, warmup=3):
        """Record one whole training step into a HIP graph (the engine replays a captured step too,
        static_gpt2.rs graph_exec) after `warmup` eager steps on a side stream, which allocate the
        optimizer state and the autograd buffers. Returns the static loss tensor every replay() updates.
        On the CPU it needs capturable=True (the GPU optimizer always keeps its step count on the
        device). The batch is copied into static buffers; set_batch() changes it."""
        torch = _torch()
        if not self.opt.param_groups[0]["capturable"]:
            raise ValueError("StaticGPT2.capture needs capturable=True")
        self._tokens, self._targets = tokens.clone(), targets.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.step(self._tokens, self._targets)
        torch.cuda.current_stream().wait_stream(side)
        self._graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph):
            self._loss = self.step(self._tokens, self._targets)
        return self._loss

    def set_batch(self, tokens, targets):
        self._tokens.copy_(tokens)
        self._targets.copy_(targets)

    def replay(self):
        """One captured training step on the current batch; returns the static loss tensor."""
        if self._graph is None:
            raise RuntimeError("StaticGPT2.replay before capture")
        self._graph.replay()
        return self._loss


def synthetic_batch(vocab_size, seq_len, seed, device):
    """Token ids and next-token targets uniform in [0, vocab) from a seeded generator."""
    torch = _torch()
    gen = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(0, vocab_size, (seq_len + 1,), generator=gen)
    return ids[:-1].to(device), ids[1:].to(device)


def time_steps(model, steps=10, warmup=3, seed=1, graph=False):
    """Median and all per-step wall times (ms) of full training steps, device-synchronised per step.

    The methodology of the reference's step benchmark (benchmark/bench_darkforest_e2e.py:116-133:
    warmup, then timed steps each ending in a device sync), with seeded tokens. graph=True records
    one step into a HIP graph after the warmup steps (StaticGPT2.capture) and times its replays: the
    same kernels without the Python dispatch between them, like the engine's host-side loop.
    """
    torch = _torch()
    tokens, targets = synthetic_batch(model.vocab_size, model.seq_len, seed, model.device)
    losses = []
    if graph:
        static_loss = model.capture(tokens, targets, warmup=warmup)
        run = model.replay
    else:
        for _ in range(warmup):
            losses.append(float(model.step(tokens, targets)))
        run = lambda: model.step(tokens, targets)  # noqa: E731
    torch.cuda.synchronize()
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        loss = run()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
        losses.append(float(static_loss if graph else loss))
    ordered = sorted(times)
    return {"median_ms": ordered[len(ordered) // 2], "min_ms": ordered[0], "times_ms": times, "losses": losses,
            "peak_mem_mb": torch.cuda.max_memory_allocated() / 2 ** 20}
