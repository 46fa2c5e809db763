"""GPT-2 training step around the fused attention: the harness that reports "GPT-2 step ms".

Mirrors the reference's static engine (darkforest-core/src/engine/static_gpt2.rs):

* model (static_gpt2.rs:276-567): learned token and position embeddings, L
  pre-LayerNorm blocks (LN eps 1e-5, darkforest-cuda/kernels/layernorm.cu:14),
  Q/K/V/O projections with biases, tanh-GELU MLP (elementwise.cu:181-192),
  final LayerNorm and an untied lm_head [vocab, d_model];
* initialisation (static_gpt2.rs:285-319): weights N(0, 0.02), the residual
  projections Wo and W2 N(0, 0.02 / sqrt(2 L)), LayerNorm gamma 1 / beta 0,
  biases 0 — drawn from a seeded generator (the reference's thread_rng is
  unseeded, static_gpt2.rs:264-271);
* step (static_gpt2.rs:1375-1696): forward, mean cross-entropy over the S
  positions in chunks of at most 512 rows, backward, AdamW with beta (0.9, 0.95),
  eps 1e-8 and weight decay 0.1 on every parameter (static_gpt2.rs:518-521;
  update rule lib.rs:1755-1788);
* attention: per layer one dfattn AttentionContext (static_gpt2.rs:401-406) whose
  forward_device_into / backward_device_into the step calls with the layer's
  retained q, k, v (static_gpt2.rs:1329-1336, 1500-1510) and scale (d_model/H)^-0.5
  (static_gpt2.rs:1291, 1439).

On the GPU (attention="dfattn") the step is the engine's own explicit forward and backward, with no
autograd: every activation and backward scratch buffer is a view of one allocation sized at
construction (`_NativeEngine`), the weights, gradients and AdamW moments are one more
(`ops.ParamArena`), and every kernel but the GEMMs is this library's (include/dfgpt2.h and the
attention contexts): embedding gather and gradient, LayerNorm, tanh GELU, the bias gradients, the
chunked fused cross-entropy and one AdamW launch over the whole arena, all fp32; the GEMMs are
hipBLASLt / rocBLAS fp32, with per-shape solutions TunableOp measured (GEMM_SOLUTIONS).
attention="sdpa", and any model on the CPU, is the reference's own parity comparator
instead (scripts/verify_loss_parity.py:58): the same model in plain PyTorch operators with torch's
scaled_dot_product_attention and torch's AdamW, differentiated by autograd.
"""
from __future__ import annotations

import math
import os
import struct
import time

from . import AttentionContext
from . import ops as _ops


def _torch():
    import torch

    return torch


def _f32(x):
    """The float32 value of x (the engine keeps its hyper-parameters as f32, static_gpt2.rs:518-521)."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


# GEMM solutions PyTorch's TunableOp measured fastest for the engine's GEMM shapes (GPT-2 small, S =
# 1024) on MI355X with this image's PyTorch, HIP, hipBLASLt and rocBLAS (written by tune_gemms). Each
# call keeps its math mode: the fast fp32 call sites choose among hipBLASLt's fast fp32 solutions,
# the exact ones among exact fp32 solutions (rocBLAS or hipBLASLt). The file's validators make
# TunableOp ignore it under other library versions or GPUs, shapes it does not list keep the
# library's default solution, and no tuning runs inside a step.
GEMM_SOLUTIONS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_solutions_gpt2_mi355x.csv")
_solutions_loaded = False


def _load_gemm_solutions():
    global _solutions_loaded
    if _solutions_loaded:
        return
    _solutions_loaded = True
    tun = _torch().cuda.tunable
    if not tun.is_enabled():
        # TunableOp writes its table to its file at exit once enabled: not into the caller's cwd.
        tun.set_filename(os.devnull)
    if os.path.exists(GEMM_SOLUTIONS):
        tun.read_file(GEMM_SOLUTIONS)


def tune_gemms(path=GEMM_SOLUTIONS, seq_len=1024, steps=2, seed=0):
    """Measure the engine's GEMM shapes with TunableOp (GPT-2 small at seq_len) and write the
    fastest solution per shape, with the library versions as validators, to `path` (the format
    TunableOp reads). Takes a few seconds on the GPU."""
    torch = _torch()
    tun = torch.cuda.tunable
    model = StaticGPT2(seq_len=seq_len, seed=seed, tuned_gemms=False)
    tokens, targets = synthetic_batch(model.vocab_size, seq_len, 1, model.device)
    prev = tun.is_enabled(), tun.tuning_is_enabled()
    tun.set_filename(os.devnull)  # TunableOp's own write at exit; the file is written below
    tun.enable(True)
    tun.tuning_enable(True)
    try:
        for _ in range(steps):
            model._engine.step(tokens, targets, tuned=False)
        torch.cuda.synchronize()
        validators = tun.get_validators()
        results = tun.get_results()
    finally:
        tun.tuning_enable(prev[1])
        tun.enable(prev[0])
    with open(path, "w") as f:
        for key, value in validators:
            f.write(f"Validator,{key},{value}\n")
        for op_sig, param_sig, solution, ms in results:
            f.write(f"{op_sig},{param_sig},{solution},{ms}\n")
    return len(results)


# A layer's parameters in parameters() (and arena) order.
_PARAM_ORDER = ("ln1_g", "ln1_b", "wq", "wk", "wv", "bq", "bk", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1", "b1", "w2",
                "b2")


class StaticGPT2:
    """GPT-2 with the reference engine's architecture, init and optimizer."""

    def __init__(self, vocab_size=50257, d_model=768, n_heads=12, n_layers=12, d_ff=3072, seq_len=1024, lr=3e-4,
                 seed=0, device="cuda", attention="dfattn", capturable=False, fast_gemm=True, tuned_gemms=True):
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
            lw = {
                "ln1_g": const(1, d_model), "ln1_b": const(0, d_model),
                "wq": randn(d_model, d_model), "bq": const(0, d_model),
                "wk": randn(d_model, d_model), "bk": const(0, d_model),
                "wv": randn(d_model, d_model), "bv": const(0, d_model),
                "wo": randn(d_model, d_model, s=std_res), "bo": const(0, d_model),
                "ln2_g": const(1, d_model), "ln2_b": const(0, d_model),
                "w1": randn(d_ff, d_model), "b1": const(0, d_ff),
                "w2": randn(d_model, d_ff, s=std_res), "b2": const(0, d_model),
            }
            # Parameter (and arena) order keeps Q, K, V's weights, and their biases, adjacent, so
            # the engine runs the three projections as one [3 d_model, d_model] linear layer.
            self.layers.append({k: lw[k] for k in _PARAM_ORDER})
        self.ln_f_g = const(1, d_model)
        self.ln_f_b = const(0, d_model)
        self.lm_head = randn(vocab_size, d_model)
        # Holding the same f32 hyper-parameters as the engine's checkpoint footer makes a resumed
        # run continue bit for bit.
        hp = dict(lr=_f32(lr), betas=(_f32(0.9), _f32(0.95)), eps=_f32(1e-8), weight_decay=_f32(0.1))
        self.native = self.device.type == "cuda" and attention == "dfattn"
        # The engine's GEMMs take hipBLASLt's fast fp32 path (torch's allow_tf32 on ROCm): relative
        # error ~5e-6 on these shapes against 1e-6 for the exact path, far inside the TF32 the
        # reference's cuBLAS GEMMs use (lib.rs:45-48), and up to 2.3x faster on the lm_head GEMM.
        self.fast_gemm = fast_gemm
        # tuned_gemms: the engine's GEMMs take the solutions in GEMM_SOLUTIONS (TunableOp, no tuning
        # at run time); the comparator's are untouched.
        self.tuned_gemms = tuned_gemms
        if self.native:
            arena = _ops.ParamArena(self.parameters(), self.device)
            self._rebind(arena.adopt(self.parameters()))
            self.opt = _ops.ArenaAdamW(arena, self.parameters(), **hp)
            self._engine = _NativeEngine(self)
        else:
            self.opt = torch.optim.AdamW(self.parameters(), **hp, capturable=capturable)
            self._engine = None
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

    # ------------------------------------------------------------ the PyTorch comparator
    def _torch_loss(self, tokens, targets):
        """Mean cross-entropy of one sequence in plain PyTorch operators (autograd-differentiable)."""
        torch = _torch()
        F = torch.nn.functional
        d, h = self.d_model, self.n_heads
        scale = (d / h) ** -0.5
        s = tokens.shape[0]
        x = self.tok_emb[tokens] + self.pos_emb[:s]
        for lw in self.layers:
            y = F.layer_norm(x, (d,), lw["ln1_g"], lw["ln1_b"], 1e-5)
            q, k, v = (F.linear(y, lw[w], lw[b]) for w, b in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")))
            qh, kh, vh = (t.view(s, h, d // h).transpose(0, 1).contiguous() for t in (q, k, v))
            o = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
            x = x + F.linear(o.transpose(0, 1).reshape(s, d), lw["wo"], lw["bo"])
            y = F.layer_norm(x, (d,), lw["ln2_g"], lw["ln2_b"], 1e-5)
            x = x + F.linear(F.gelu(F.linear(y, lw["w1"], lw["b1"]), approximate="tanh"), lw["w2"], lw["b2"])
        y = F.layer_norm(x, (d,), self.ln_f_g, self.ln_f_b, 1e-5)
        return F.cross_entropy(F.linear(y, self.lm_head), targets)

    # ------------------------------------------------------------ public step API
    def loss(self, tokens, targets):
        """Mean cross-entropy of one sequence, without an optimizer step (static_gpt2.rs:1386-1418)."""
        if self.native:
            return self._engine.forward_loss(tokens, targets).clone()
        return self._torch_loss(tokens, targets)

    def step(self, tokens, targets):
        """One training step: forward, loss, backward, AdamW. Returns the loss tensor (not synchronised)."""
        if self.native:
            return self._engine.step(tokens, targets)
        self.opt.zero_grad(set_to_none=False)
        loss = self._torch_loss(tokens, targets)
        loss.backward()
        self.opt.step()
        return loss.detach()

    def capture(self, tokens, targets, warmup=3):
        """Record one whole training step into a HIP graph (the engine replays a captured step too,
        static_gpt2.rs graph_exec) after `warmup` eager steps on a side stream. Returns the static
        loss tensor every replay() updates. The comparator needs capturable=True. The batch is copied
        into static buffers; set_batch() changes it."""
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
        """One captured training step on the current batch; returns the static loss tensor.

        After load_checkpoint dropped the recorded step (its AdamW launch holds the old
        hyper-parameters) the step is recorded again here, on the current batch and without eager
        warm-up steps, which would train the loaded weights (the engine re-captures on its next step,
        static_gpt2.rs:619-629). The returned tensor is then a new one."""
        if self._graph is None:
            if getattr(self, "_tokens", None) is None:
                raise RuntimeError("StaticGPT2.replay before capture")
            self.capture(self._tokens, self._targets, warmup=0)
        self._graph.replay()
        return self._loss

    def activation_bytes(self):
        """Bytes of the native engine's single activation allocation (0 for the comparator)."""
        return self._engine.arena_bytes if self.native else 0


class _NativeEngine:
    """The step of static_gpt2.rs:1286-1696 on preallocated buffers.

    Every activation the backward needs and every backward scratch tensor is a view of one flat
    float32 allocation made here (the engine's arena, static_gpt2.rs:401-567), each view starting
    on a 256-byte boundary; token ids, targets and positions are one int32 allocation. Per layer the
    step keeps x_in, the LayerNorm outputs and statistics, q, k, v, the attention output, x_mid and
    both MLP activations, as the reference's LayerActs do (static_gpt2.rs:45-60); the backward
    scratch (static_gpt2.rs:61-74) is shared by all layers. Each layer's AttentionContext reuses
    its forward in the backward (the q, k, v and output views are not touched in between).
    """

    def __init__(self, m: StaticGPT2):
        torch = _torch()
        self.m = m
        self.exact_sites = dict(self.EXACT_SITES)
        S, d, F, V, L, H = m.seq_len, m.d_model, m.d_ff, m.vocab_size, m.n_layers, m.n_heads
        self.chunk = min(S, 512)  # static_gpt2.rs:423
        dev = m.device
        plan = []  # (name, shape)

        def buf(name, *shape):
            plan.append((name, shape))

        # The strided attention calls (Q, K, V read from the fused projection's output in place)
        # take d_head 64; other head sizes get contiguous copies.
        self.packed = d // H != 64
        for l in range(L + 1):
            buf(f"x{l}", S, d)
        for l in range(L):
            for n in ("ln1", "att", "xmid", "ln2"):
                buf(f"{n}{l}", S, d)
            buf(f"qkv{l}", S, 3 * d)  # the fused projection's output: q | k | v by row
            if self.packed:
                buf(f"qkvc{l}", 3, S, d)
            buf(f"st1{l}", 2, S)
            buf(f"st2{l}", 2, S)
            buf(f"h{l}", S, F)
            buf(f"a{l}", S, F)
        buf("lnf", S, d)
        buf("stf", 2, S)
        buf("tmp", S, d)
        buf("logits", self.chunk, V)
        # lm_head's input gradient d(lnf) = dlogits lm_head has K = vocab: it runs as a batched
        # product over `ksplit` slices of the vocabulary into these partial sums, then one sum.
        self.ksplit = max(1, min(32, V // 256))
        buf("dx_part", self.ksplit, self.chunk, d)
        buf("row_loss", S)
        buf("loss", 1)
        for n in ("g0", "g1", "dlnf", "dln", "datt"):
            buf(n, S, d)
        buf("wide", S, 3 * d)  # [S, 3 d_model]: dq | dk | dv by row, the fused projection's gradient
        if self.packed:
            buf("dqkv", 3, S, d)
        buf("dh", S, F)
        # partial column sums of the fused LayerNorm backward
        buf("ln_ws", (_ops.layer_norm_backward_fused_workspace_bytes(S, d) + 3) // 4)
        buf("da", S, F)
        offsets, n = {}, 0
        for name, shape in plan:
            size = 1
            for s in shape:
                size *= s
            offsets[name] = (n, shape, size)
            n += (size + 63) // 64 * 64
        self.arena = torch.empty(n, dtype=torch.float32, device=dev)
        self.arena_bytes = n * 4
        self.b = {name: self.arena[o:o + size].view(shape) for name, (o, shape, size) in offsets.items()}
        ints = torch.empty(3 * ((S + 63) // 64 * 64), dtype=torch.int32, device=dev)
        w = (S + 63) // 64 * 64
        self.ids, self.tgt, self.pos = ints[:S], ints[w:w + S], ints[2 * w:2 * w + S]
        self.pos.copy_(torch.arange(S, dtype=torch.int32, device=dev))
        self.ctx = [AttentionContext(H, S, d // H, reuse_forward=True) for _ in range(L)]
        # In a captured step the backward's weight-gradient GEMMs run on this stream, beside the
        # input-gradient ones (eager dispatch of the cross-stream waits costs more than it gains).
        self.side = torch.cuda.Stream(device=dev) if torch.device(dev).type == "cuda" else None
        self._overlap = False
        self.scale = (d / H) ** -0.5
        # Views of each layer's Q, K, V weights (and biases, and their gradients) as one [3d, d]
        # ([3d]) tensor: they are adjacent in the parameter arena.
        self.wqkv, self.bqkv = [], []
        for lw in m.layers:
            self.wqkv.append(self._adjacent([lw["wq"], lw["wk"], lw["wv"]]))
            self.bqkv.append(self._adjacent([lw["bq"], lw["bk"], lw["bv"]]))

    def _qkv(self, l):
        """Layer l's q, k, v: the column blocks of its projection output, or their copies."""
        if self.packed:
            return self.b[f"qkvc{l}"].unbind(0)
        return self.b[f"qkv{l}"].split(self.m.d_model, dim=1)

    @staticmethod
    def _adjacent(ts):
        """The parameters ts, consecutive in memory, as one tensor stacked on dim 0 (its .grad the
        same view of their gradients)."""
        torch = _torch()
        first = ts[0]
        n = first.numel()
        for i, t in enumerate(ts):
            if t.data_ptr() != first.data_ptr() + i * n * 4 or t.grad.data_ptr() != first.grad.data_ptr() + i * n * 4:
                raise RuntimeError("Q, K, V parameters are not adjacent in the arena")
        shape = (len(ts) * first.shape[0],) + tuple(first.shape[1:])
        w = torch.as_strided(first.detach(), shape, first.stride())
        w.grad = torch.as_strided(first.grad, shape, first.grad.stride())
        return w

    # Per GEMM call site: the exact fp32 path (True) or the fast one, whichever measured faster at
    # that site with the tuned solutions (whole replayed steps: qkv_fwd exact is 0.12 ms slower,
    # qkv_dw and wo_dx exact no faster). *_fwd: the forward product (o and fc2 with the bias in the
    # GEMM's epilogue); *_dx / *_dw: the input and weight gradients.
    EXACT_SITES = {"qkv_fwd": False, "o_fwd": True, "fc1_fwd": False, "fc2_fwd": True,
                   "fc2_dx": False, "fc2_dw": False, "fc1_dx": True, "fc1_dw": False,
                   "wo_dx": False, "wo_dw": True, "qkv_dx": True, "qkv_dw": False}

    # ---------------------------------------------------------------- pieces
    @staticmethod
    def _exact(flag=True):
        """Switch the GEMMs that follow to hipBLASLt's exact fp32 path (flag) or back to the step's
        setting (measured per call site: the fast path wins on the wide or deep products, the exact
        one on the square 768 x 768 ones and on the products whose bias it fuses)."""
        torch = _torch()
        torch.backends.cuda.matmul.allow_tf32 = (not flag) and _NativeEngine._fast

    def _linear(self, x, w, b, out, exact=True):
        """out = x W^T + b (static_gpt2.rs linear_into; hipBLASLt). exact: one GEMM with the bias in
        its epilogue on the exact fp32 path; otherwise the fast-path GEMM, then the bias added in
        place (dfgpt2_add_bias)."""
        torch = _torch()
        if exact:
            self._exact(True)
            torch.addmm(b, x, w.t(), out=out)
            self._exact(False)
        else:
            torch.mm(x, w.t(), out=out)
            _ops.add_bias_into(out, b)

    def _linear_backward(self, x, w, dy, dx, exact_dx=False, exact_dw=False, bias=None):
        """dx = dy W and W's gradient dy^T x, into the arena gradient view (static_gpt2.rs
        linear_backward_into); exact_dx / exact_dw: that product on the exact fp32 GEMM path;
        bias: its gradient too (the column sums of dy), beside W's."""
        torch = _torch()
        if self._overlap:
            # The previous weight gradient has finished before this one starts (and before the main
            # stream goes on to overwrite what that one read); this one starts after dy is written.
            main = torch.cuda.current_stream()
            main.wait_stream(self.side)
            self.side.wait_stream(main)
        self._exact(exact_dx)
        torch.mm(dy, w, out=dx)
        self._exact(exact_dw)
        if self._overlap:
            with torch.cuda.stream(self.side):
                torch.mm(dy.t(), x, out=w.grad)
                if bias is not None:
                    self._bias_grad(dy, bias)
        else:
            torch.mm(dy.t(), x, out=w.grad)
            if bias is not None:
                self._bias_grad(dy, bias)
        self._exact(False)

    @staticmethod
    def _bias_grad(dy, b):
        rows, n = dy.shape
        _ops._check(_ops.ops_lib().dfgpt2_linear_grad_bias(_ops._dev_ptr(dy), _ops._dev_ptr(b.grad), rows, n, 0,
                                                           _ops._stream_ptr()))

    @staticmethod
    def _ln(x, g, b, out, stats):
        rows, f = x.shape
        _ops._check(_ops.ops_lib().dfgpt2_layernorm_forward(
            _ops._dev_ptr(x), _ops._dev_ptr(g), _ops._dev_ptr(b), _ops._dev_ptr(out), _ops._dev_ptr(stats[0]),
            _ops._dev_ptr(stats[1]), rows, f, _ops._stream_ptr()))

    def _ln_backward(self, dy, x, g, b, stats, dx, residual=None, bias=None):
        """dx = LayerNorm's input gradient (+ residual, a residual connection's gradient); gamma's
        and beta's gradients written into their arena views, and with `bias`, the gradient of the
        linear layer's bias whose output gradient dx is (its column sums), from the same read."""
        _ops.layer_norm_backward_fused_into(dy, x, g, stats, residual, dx, g.grad, b.grad,
                                            bias.grad if bias is not None else None, self.b["ln_ws"])

    def _set_batch(self, tokens, targets):
        if tokens.shape[0] != self.m.seq_len or targets.shape[0] != self.m.seq_len:
            raise ValueError(f"the engine runs sequences of exactly seq_len = {self.m.seq_len} tokens")
        self.ids.copy_(tokens)
        self.tgt.copy_(targets)

    # ---------------------------------------------------------------- forward (static_gpt2.rs:1286-1373)
    def _forward(self):
        """Each residual add runs inside the LayerNorm that follows it (x_mid and LayerNorm 2, then
        x_in[l+1] and the next layer's LayerNorm 1 or the final one), and the first MLP bias inside
        GELU; the values are those of the separate operations."""
        torch = _torch()
        m, b, ex = self.m, self.b, self.exact_sites
        S, L = m.seq_len, m.n_layers
        x0 = b["x0"]
        _ops.embedding_forward(self.ids, m.tok_emb, x0)
        torch.add(x0, m.pos_emb[:S], out=x0)  # positions 0..S-1 of the position table
        self._ln(x0, m.layers[0]["ln1_g"], m.layers[0]["ln1_b"], b["ln10"], b["st10"])
        for l, lw in enumerate(m.layers):
            x, ln1, ln2 = b[f"x{l}"], b[f"ln1{l}"], b[f"ln2{l}"]
            qkv, att, xmid = b[f"qkv{l}"], b[f"att{l}"], b[f"xmid{l}"]
            # Q, K, V in one GEMM ([S, 3d]); attention reads its three column blocks in place
            # (the strided context call).
            self._linear(ln1, self.wqkv[l], self.bqkv[l], qkv, ex["qkv_fwd"])
            if self.packed:
                b[f"qkvc{l}"].copy_(qkv.view(S, 3, -1).transpose(0, 1))
            self.ctx[l].forward_device_into(*self._qkv(l), self.scale, True, att)
            self._linear(att, lw["wo"], lw["bo"], b["tmp"], ex["o_fwd"])
            _ops.add_layer_norm_forward_into(x, b["tmp"], lw["ln2_g"], lw["ln2_b"], xmid, ln2, b[f"st2{l}"])
            # h = ln2 W1^T; the bias goes into h as GELU reads it
            self._exact(ex["fc1_fwd"])
            torch.mm(ln2, lw["w1"].t(), out=b[f"h{l}"])
            self._exact(False)
            _ops.bias_gelu_forward_into(b[f"h{l}"], lw["b1"], b[f"a{l}"])
            self._linear(b[f"a{l}"], lw["w2"], lw["b2"], b["tmp"], ex["fc2_fwd"])
            if l + 1 < L:
                nxt = m.layers[l + 1]
                _ops.add_layer_norm_forward_into(xmid, b["tmp"], nxt["ln1_g"], nxt["ln1_b"], b[f"x{l + 1}"],
                                                 b[f"ln1{l + 1}"], b[f"st1{l + 1}"])
            else:
                _ops.add_layer_norm_forward_into(xmid, b["tmp"], m.ln_f_g, m.ln_f_b, b[f"x{L}"], b["lnf"], b["stf"])

    # ---------------------------------------------------------------- loss (static_gpt2.rs:1386-1418)
    def _loss_and_head_backward(self):
        """Chunks of at most 512 rows: logits = lnf lm_head^T, the fused cross-entropy (the gradient
        overwrites the logits in place), then the chunk's share of d(lnf) and of lm_head's
        gradient; finally the rows' losses summed in order."""
        torch = _torch()
        m, b = self.m, self.b
        S = m.seq_len
        for start in range(0, S, self.chunk):
            c = min(self.chunk, S - start)
            lg = b["logits"][:c]
            x = b["lnf"][start:start + c]
            torch.mm(x, m.lm_head.t(), out=lg)
            _ops.logit_ce_chunk(lg, self.tgt[start:start + c], lg, b["row_loss"][start:start + c], S)
            self._head_dx(lg, b["dlnf"][start:start + c])
            if start == 0:
                torch.mm(lg.t(), x, out=m.lm_head.grad)
            else:
                m.lm_head.grad.addmm_(lg.t(), x)
        _ops.sum_into(b["row_loss"], b["loss"])

    def _head_dx(self, lg, out):
        """out = lg lm_head with K = vocab split into `ksplit` slices: one strided batched GEMM
        (slice j of every row of lg against rows j*Kc .. of lm_head, no copies) into the partial
        sums, their sum over the slices, and the vocabulary's remainder rows added last. hipBLASLt's
        single GEMM over K = 50257 keeps few workgroups busy (0.57 ms per 512 rows against 0.15)."""
        torch = _torch()
        m = self.m
        rows, V = lg.shape
        B = self.ksplit
        kc = V // B
        part = self.b["dx_part"][:, :rows]
        torch.bmm(lg[:, :B * kc].view(rows, B, kc).permute(1, 0, 2), m.lm_head[:B * kc].view(B, kc, -1), out=part)
        torch.sum(part, dim=0, out=out)
        if B * kc < V:
            out.addmm_(lg[:, B * kc:], m.lm_head[B * kc:])

    # ---------------------------------------------------------------- backward (static_gpt2.rs:1424-1575)
    def _backward(self):
        m, b, ex = self.m, self.b, self.exact_sites
        self._overlap = self.side is not None and _torch().cuda.is_current_stream_capturing()
        if self._overlap:
            self.side.wait_stream(_torch().cuda.current_stream())
        L = m.n_layers
        g, other = b["g0"], b["g1"]  # gradient of the residual stream, and the next layer's
        # Each LayerNorm backward also writes the bias gradient of the linear layer below it in the
        # backward order (b2, or bo), the column sums of the residual-stream gradient it produces.
        self._ln_backward(b["dlnf"], b[f"x{L}"], m.ln_f_g, m.ln_f_b, b["stf"], g,
                          bias=m.layers[L - 1]["b2"] if L else None)
        for l in reversed(range(L)):
            lw = m.layers[l]
            # MLP: g is d(x_in[l+1]) = d(mlp out) = d(x_mid) through the residual
            self._linear_backward(b[f"a{l}"], lw["w2"], g, b["da"], ex["fc2_dx"], ex["fc2_dw"])
            _ops._check(_ops.ops_lib().dfgpt2_gelu_backward(_ops._dev_ptr(b["da"]), _ops._dev_ptr(b[f"h{l}"]),
                                                            _ops._dev_ptr(b["dh"]), b["dh"].numel(),
                                                            _ops._stream_ptr()))
            self._linear_backward(b[f"ln2{l}"], lw["w1"], b["dh"], b["dln"], ex["fc1_dx"], ex["fc1_dw"], lw["b1"])
            # d(x_mid) = g + LayerNorm 2's gradient
            self._ln_backward(b["dln"], b[f"xmid{l}"], lw["ln2_g"], lw["ln2_b"], b[f"st2{l}"], other, residual=g,
                              bias=lw["bo"])
            g, other = other, g
            # attention: output projection, the fused attention backward, the Q/K/V projections
            self._linear_backward(b[f"att{l}"], lw["wo"], g, b["datt"], ex["wo_dx"], ex["wo_dw"])
            # dq | dk | dv side by side ([S, 3d]) for the fused projection's backward
            wide = b["wide"]
            grads = b["dqkv"].unbind(0) if self.packed else wide.split(m.d_model, dim=1)
            self.ctx[l].backward_device_into(*self._qkv(l), b["datt"], self.scale, True, *grads)
            if self.packed:
                wide.view(m.seq_len, 3, -1).copy_(b["dqkv"].transpose(0, 1))
            self._linear_backward(b[f"ln1{l}"], self.wqkv[l], wide, b["dln"], ex["qkv_dx"], ex["qkv_dw"],
                                  self.bqkv[l])
            # d(x_in[l]) = d(x_mid) + LayerNorm 1's gradient
            self._ln_backward(b["dln"], b[f"x{l}"], lw["ln1_g"], lw["ln1_b"], b[f"st1{l}"], other, residual=g,
                              bias=m.layers[l - 1]["b2"] if l else None)
            g, other = other, g
        # embeddings (static_gpt2.rs:1559-1574): the token rows, and positions 0..S-1
        _ops.embedding_backward(self.ids, g, m.tok_emb.grad)
        _ops.embedding_backward(self.pos, g, m.pos_emb.grad)
        if self._overlap:
            _torch().cuda.current_stream().wait_stream(self.side)  # the last weight gradient

    def _zero_accumulated_grads(self):
        """Only the embedding gradients are accumulated (the embedding backward adds into them);
        every other gradient of the arena is written whole by the step."""
        self.m.tok_emb.grad.zero_()
        self.m.pos_emb.grad.zero_()

    # ---------------------------------------------------------------- public
    # (The parameters are autograd leaves for the comparator-facing API; the engine differentiates
    # by hand, so its torch calls run under no_grad. The GEMM precision setting is scoped to the
    # engine's own calls and restored afterwards.)
    _fast = True  # the fast GEMM path is allowed in the running step (StaticGPT2.fast_gemm)

    def _run(self, fn, tuned=True):
        torch = _torch()
        tun = torch.cuda.tunable
        prev = torch.backends.cuda.matmul.allow_tf32
        prev_tun = tun.is_enabled(), tun.tuning_is_enabled()
        _NativeEngine._fast = bool(self.m.fast_gemm)
        torch.backends.cuda.matmul.allow_tf32 = _NativeEngine._fast
        if tuned and self.m.tuned_gemms:
            _load_gemm_solutions()
            tun.enable(True)
            tun.tuning_enable(False)
        try:
            with torch.no_grad():
                fn()
        finally:
            if tuned and self.m.tuned_gemms:
                tun.tuning_enable(prev_tun[1])
                tun.enable(prev_tun[0])
            torch.backends.cuda.matmul.allow_tf32 = prev

    def forward_loss(self, tokens, targets):
        def run():
            self._set_batch(tokens, targets)
            self._forward()
            self._loss_and_head_backward()
        self._run(run)
        return self.b["loss"][0]

    def step(self, tokens, targets, tuned=True):
        """static_gpt2.rs:1375-1696: forward, chunked loss, backward, AdamW over the whole parameter
        arena in one launch; returns the device loss. tuned=False: TunableOp's state is left as
        the caller set it (tune_gemms measures through it)."""
        def run():
            self._zero_accumulated_grads()
            self._set_batch(tokens, targets)
            self._forward()
            self._loss_and_head_backward()
            self._backward()
            self.m.opt.step()
        self._run(run, tuned=tuned)
        return self.b["loss"][0]


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
