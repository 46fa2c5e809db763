"""The GPT-2 step's non-attention kernels of libdfattn.so (include/dfgpt2.h) for PyTorch tensors.

* `layer_norm`, `linear`, `gelu`, `embedding`: autograd functions on the HIP kernels — LayerNorm
  forward and backward (darkforest-cuda/kernels/layernorm.cu:97, 187), the linear layer's bias
  gradient (matmul.cu:240; the two products of a linear layer stay hipBLASLt GEMMs) and tanh GELU
  (elementwise.cu:195, 217); with direct=True the parameter gradients are added straight into the
  arena's gradient buffers;
* `ParamArena` / `ArenaAdamW`: the engine's single allocation for its weights, gradients and AdamW
  moments (static_gpt2.rs:401-567) and its AdamW update (matmul.cu:341, lib.rs:1755-1788) as one
  launch over the whole arena, with the step count on the device.

Every reduction adds in a fixed order, so a step is reproducible bit for bit.
"""
from __future__ import annotations

import ctypes

from . import _check, _dev_ptr, _stream_ptr, _torch, lib

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_I = ctypes.c_int

# ctypes signatures of include/dfgpt2.h
SYMBOLS = {
    "launch_layernorm": (None, [_P] * 6 + [_U32, _U32]),
    "launch_layernorm_backward": (None, [_P] * 8 + [_U32, _U32]),
    "launch_gelu": (None, [_P, _P, _U32]),
    "launch_gelu_backward": (None, [_P, _P, _P, _U32]),
    "launch_linear_grad_bias": (None, [_P, _P, _U32, _U32]),
    "launch_adamw_update": (None, [_P] * 4 + [_U32] + [_F] * 7),
    "dfgpt2_layernorm_forward": (_I, [_P] * 6 + [_U32, _U32, _P]),
    "dfgpt2_layernorm_backward": (_I, [_P] * 8 + [_U32, _U32, _P]),
    "dfgpt2_gelu_forward": (_I, [_P, _P, _SZ, _P]),
    "dfgpt2_gelu_backward": (_I, [_P, _P, _P, _SZ, _P]),
    "dfgpt2_linear_grad_bias": (_I, [_P, _P, _U32, _U32, _I, _P]),
    "dfgpt2_adamw_update": (_I, [_P] * 4 + [_SZ] + [_F] * 5 + [_P, _P]),
}

_typed = None


def ops_lib():
    """libdfattn.so with the dfgpt2.h symbols typed (raises DfattnNotBuilt if it is missing)."""
    global _typed
    handle = lib()
    if _typed is not handle:
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _typed = handle
    return handle


def _rows_cols(t):
    if t.dim() != 2:
        raise ValueError("expected a 2-D [rows, features] tensor")
    return t.shape[0], t.shape[1]


def layer_norm_forward(x, gamma, beta):
    """(out, means, rstds) of LayerNorm over the last dim of a [rows, F] tensor, eps 1e-5."""
    torch = _torch()
    rows, f = _rows_cols(x)
    out = torch.empty_like(x)
    stats = torch.empty((2, rows), dtype=torch.float32, device=x.device)
    _check(ops_lib().dfgpt2_layernorm_forward(_dev_ptr(x), _dev_ptr(gamma), _dev_ptr(beta), _dev_ptr(out),
                                              _dev_ptr(stats[0]), _dev_ptr(stats[1]), rows, f, _stream_ptr()))
    return out, stats[0], stats[1]


def layer_norm_backward(grad_out, x, gamma, means, rstds):
    """(grad_x, grad_gamma, grad_beta); the parameter gradients are column sums over the rows."""
    torch = _torch()
    rows, f = _rows_cols(x)
    grad_x = torch.empty_like(x)
    pg = torch.zeros((2, f), dtype=torch.float32, device=x.device)  # the kernel adds into them
    _check(ops_lib().dfgpt2_layernorm_backward(_dev_ptr(grad_out), _dev_ptr(x), _dev_ptr(gamma), _dev_ptr(means),
                                               _dev_ptr(rstds), _dev_ptr(grad_x), _dev_ptr(pg[0]), _dev_ptr(pg[1]),
                                               rows, f, _stream_ptr()))
    return grad_x, pg[0], pg[1]


def bias_grad(grad_out):
    """Column sums of a [rows, N] gradient: the bias gradient of a linear layer."""
    torch = _torch()
    rows, n = _rows_cols(grad_out)
    out = torch.empty(n, dtype=torch.float32, device=grad_out.device)
    _check(ops_lib().dfgpt2_linear_grad_bias(_dev_ptr(grad_out), _dev_ptr(out), rows, n, 0, _stream_ptr()))
    return out


def gelu_forward(x):
    torch = _torch()
    out = torch.empty_like(x)
    _check(ops_lib().dfgpt2_gelu_forward(_dev_ptr(x), _dev_ptr(out), x.numel(), _stream_ptr()))
    return out


def gelu_backward(grad_out, x):
    torch = _torch()
    grad_x = torch.empty_like(x)
    _check(ops_lib().dfgpt2_gelu_backward(_dev_ptr(grad_out), _dev_ptr(x), _dev_ptr(grad_x), x.numel(),
                                          _stream_ptr()))
    return grad_x


def _grad_of(t, direct):
    """The arena gradient buffer of parameter t when the caller asked for direct accumulation."""
    return t.grad if (direct and t is not None and t.grad is not None) else None


def _autograd_functions():
    torch = _torch()

    # direct=True (parameters that are ParamArena views): the backward adds the parameter gradients
    # straight into their .grad buffers in the arena and returns None for them, instead of returning
    # fresh tensors that autograd would then add into .grad (one more read-modify-write of every
    # gradient per step). Each parameter is used once per forward, so the sums are the same.

    class LayerNormFn(torch.autograd.Function):
        """LayerNorm (eps 1e-5) of [rows, F]: static_gpt2.rs layernorm_into / layernorm_backward_into."""

        @staticmethod
        def forward(ctx, x, gamma, beta, direct):
            out, means, rstds = layer_norm_forward(x, gamma, beta)
            ctx.save_for_backward(x, gamma, means, rstds)
            ctx.gg, ctx.gb = _grad_of(gamma, direct), _grad_of(beta, direct)
            return out

        @staticmethod
        def backward(ctx, grad_out):
            x, gamma, means, rstds = ctx.saved_tensors
            grad_out = grad_out.contiguous()
            if ctx.gg is not None and ctx.gb is not None:
                rows, f = _rows_cols(x)
                grad_x = torch.empty_like(x)
                _check(ops_lib().dfgpt2_layernorm_backward(
                    _dev_ptr(grad_out), _dev_ptr(x), _dev_ptr(gamma), _dev_ptr(means), _dev_ptr(rstds),
                    _dev_ptr(grad_x), _dev_ptr(ctx.gg), _dev_ptr(ctx.gb), rows, f, _stream_ptr()))
                return grad_x, None, None, None
            return layer_norm_backward(grad_out, x, gamma, means, rstds) + (None,)

    class LinearFn(torch.autograd.Function):
        """y = x W^T (+ b): GEMMs on hipBLASLt, the bias gradient on dfgpt2_linear_grad_bias."""

        @staticmethod
        def forward(ctx, x, w, b, direct):
            ctx.save_for_backward(x, w)
            ctx.has_bias = b is not None
            ctx.gw, ctx.gb = _grad_of(w, direct), _grad_of(b, direct)
            return torch.addmm(b, x, w.t()) if b is not None else x.mm(w.t())

        @staticmethod
        def backward(ctx, grad_out):
            x, w = ctx.saved_tensors
            grad_out = grad_out.contiguous()
            gx = grad_out.mm(w) if ctx.needs_input_grad[0] else None
            gw = gb = None
            if ctx.gw is not None:
                ctx.gw.addmm_(grad_out.t(), x)
            elif ctx.needs_input_grad[1]:
                gw = grad_out.t().mm(x)
            if ctx.has_bias:
                if ctx.gb is not None:
                    rows, n = _rows_cols(grad_out)
                    _check(ops_lib().dfgpt2_linear_grad_bias(_dev_ptr(grad_out), _dev_ptr(ctx.gb), rows, n, 1,
                                                             _stream_ptr()))
                elif ctx.needs_input_grad[2]:
                    gb = bias_grad(grad_out)
            return gx, gw, gb, None

    class GeluFn(torch.autograd.Function):
        """tanh GELU (elementwise.cu:181-240)."""

        @staticmethod
        def forward(ctx, x):
            ctx.save_for_backward(x)
            return gelu_forward(x)

        @staticmethod
        def backward(ctx, grad_out):
            (x,) = ctx.saved_tensors
            return gelu_backward(grad_out.contiguous(), x)

    class EmbeddingFn(torch.autograd.Function):
        """Rows of a table by token id; the backward adds each row's gradient into the table gradient
        with the sort-based (deterministic) accumulating index_put."""

        @staticmethod
        def forward(ctx, w, ids, direct):
            ctx.save_for_backward(ids)
            ctx.gw, ctx.shape = _grad_of(w, direct), w.shape
            return w.index_select(0, ids)

        @staticmethod
        def backward(ctx, grad_out):
            (ids,) = ctx.saved_tensors
            grad_out = grad_out.contiguous()
            if ctx.gw is not None:
                ctx.gw.index_put_((ids,), grad_out, accumulate=True)
                return None, None, None
            g = torch.zeros(ctx.shape, dtype=grad_out.dtype, device=grad_out.device)
            g.index_put_((ids,), grad_out, accumulate=True)
            return g, None, None

    return LayerNormFn, LinearFn, GeluFn, EmbeddingFn


_fns = None


def _functions():
    global _fns
    if _fns is None:
        _fns = _autograd_functions()
    return _fns


def layer_norm(x, gamma, beta, direct=False):
    return _functions()[0].apply(x, gamma, beta, direct)


def linear(x, w, b=None, direct=False):
    return _functions()[1].apply(x, w, b, direct)


def gelu(x):
    return _functions()[2].apply(x)


def embedding(w, ids, direct=False):
    return _functions()[3].apply(w, ids, direct)


class ParamArena:
    """One flat float32 allocation each for the weights, their gradients and the two AdamW moments
    (each tensor starts at a multiple of 4 floats, so the arena updates as float4). `adopt` turns
    existing tensors into leaf views of the weight arena whose .grad are views of the gradient
    arena; autograd then accumulates into the arena in place."""

    def __init__(self, tensors, device):
        torch = _torch()
        self.shapes = [tuple(t.shape) for t in tensors]
        self.offsets, n = [], 0
        for t in tensors:
            self.offsets.append(n)
            n += (t.numel() + 3) // 4 * 4
        self.numel = n
        self.p = torch.zeros(n, dtype=torch.float32, device=device)
        self.g = torch.zeros(n, dtype=torch.float32, device=device)
        self.m = torch.zeros(n, dtype=torch.float32, device=device)
        self.v = torch.zeros(n, dtype=torch.float32, device=device)
        self.step = torch.zeros(1, dtype=torch.float32, device=device)

    def view(self, flat, i):
        off, shape = self.offsets[i], self.shapes[i]
        size = 1
        for s in shape:
            size *= s
        return flat[off:off + size].view(shape)

    def adopt(self, tensors):
        torch = _torch()
        out = []
        with torch.no_grad():
            for i, t in enumerate(tensors):
                pv = self.view(self.p, i)
                pv.copy_(t)
                pv.requires_grad_(True)
                pv.grad = self.view(self.g, i)
                out.append(pv)
        return out


class _ArenaState:
    """optimizer.state for the arena: state[p] gives views of p's moments and the shared step count;
    assigning a dict copies moments and step into the arena (the checkpoint loader does that)."""

    def __init__(self, arena, params):
        self._arena = arena
        self._index = {id(p): i for i, p in enumerate(params)}

    def get(self, p, default=None):
        i = self._index.get(id(p))
        if i is None:
            return default
        a = self._arena
        return {"step": a.step[0], "exp_avg": a.view(a.m, i), "exp_avg_sq": a.view(a.v, i)}

    def __getitem__(self, p):
        st = self.get(p)
        if st is None:
            raise KeyError("not an arena parameter")
        return st

    def __setitem__(self, p, st):
        torch = _torch()
        i = self._index[id(p)]
        a = self._arena
        with torch.no_grad():
            a.view(a.m, i).copy_(st["exp_avg"])
            a.view(a.v, i).copy_(st["exp_avg_sq"])
            a.step.fill_(float(st["step"]))


class ArenaAdamW:
    """AdamW over a ParamArena in one launch (dfgpt2_adamw_update): decoupled weight decay on every
    parameter, bias corrections from the device step count. Mirrors the torch optimizer surface the
    harness and the checkpoint code use (param_groups, state, zero_grad, step)."""

    def __init__(self, arena, params, lr, betas, eps, weight_decay):
        self.arena = arena
        self.param_groups = [{"params": list(params), "lr": lr, "betas": tuple(betas), "eps": eps,
                              "weight_decay": weight_decay, "capturable": True, "fused": True}]
        self.state = _ArenaState(arena, params)

    def zero_grad(self, set_to_none=False):
        self.arena.g.zero_()

    def step(self):
        g, a = self.param_groups[0], self.arena
        b1, b2 = g["betas"]
        _check(ops_lib().dfgpt2_adamw_update(_dev_ptr(a.p), _dev_ptr(a.m), _dev_ptr(a.v), _dev_ptr(a.g), a.numel,
                                             g["lr"], b1, b2, g["eps"], g["weight_decay"], _dev_ptr(a.step),
                                             _stream_ptr()))
