"""The GPT-2 step's non-attention kernels of libdfattn.so (include/dfgpt2.h) for PyTorch tensors.

* `layer_norm_forward` / `layer_norm_backward`, `gelu_forward` / `gelu_backward`, `bias_grad`: the
  LayerNorm, tanh GELU and bias-gradient kernels (darkforest-cuda/kernels/layernorm.cu:97, 187;
  elementwise.cu:195, 217; matmul.cu:240) on fresh output tensors;
* `logit_ce_chunk` / `sum_into`, `embedding_forward` / `embedding_backward`: the chunked fused
  cross-entropy (softmax.cu:396) and the token embedding and its gradient (elementwise.cu:268, 291);
* `ParamArena` / `ArenaAdamW`: the engine's single allocation for its weights, gradients and AdamW
  moments (static_gpt2.rs:401-567) and its AdamW update (matmul.cu:341, lib.rs:1755-1788) as one
  launch over the whole arena, with the step count on the device.

Every reduction adds in a fixed order, so a step is reproducible bit for bit. The GPT-2 engine
(gpt2_step._NativeEngine) calls these and the C ABI directly.
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
    "launch_fused_chunked_logit_ce": (None, [_P] * 4 + [_U32, _U32, _U32]),
    "launch_embedding_forward": (None, [_P] * 3 + [_U32, _U32]),
    "launch_embedding_backward": (None, [_P] * 3 + [_U32, _U32]),
    "dfgpt2_logit_ce_chunk": (_I, [_P] * 4 + [_U32, _U32, _U32, _P]),
    "dfgpt2_sum": (_I, [_P, _U32, _P, _I, _P]),
    "dfgpt2_embedding_forward": (_I, [_P] * 3 + [_U32, _U32, _U32, _P]),
    "dfgpt2_embedding_backward": (_I, [_P] * 3 + [_U32, _U32, _U32, _P]),
    "dfgpt2_add_layernorm_forward": (_I, [_P] * 8 + [_U32, _U32, _P]),
    "dfgpt2_layernorm_backward_residual": (_I, [_P] * 9 + [_U32, _U32, _P]),
    "dfgpt2_bias_gelu_forward": (_I, [_P] * 3 + [_U32, _U32, _P]),
    "dfgpt2_layernorm_backward_fused_workspace_bytes": (_SZ, [_U32, _U32]),
    "launch_add_bias": (None, [_P] * 3 + [_U32, _U32]),
    "launch_fill": (None, [_P, _F, _U32]),
    "launch_add": (None, [_P] * 3 + [_U32]),
    "launch_scale": (None, [_P, _F, _P, _U32]),
    "dfgpt2_add_bias": (_I, [_P] * 3 + [_U32, _U32, _P]),
    "dfgpt2_layernorm_backward_fused": (_I, [_P] * 11 + [_SZ, _U32, _U32, _P]),
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


def add_layer_norm_forward_into(x, y, gamma, beta, sum_out, out, stats):
    """dfgpt2_add_layernorm_forward: sum_out = x + y, out = LayerNorm(sum_out) with eps 1e-5;
    stats[0], stats[1] receive the rows' means and reciprocal standard deviations."""
    rows, f = _rows_cols(x)
    _check(ops_lib().dfgpt2_add_layernorm_forward(_dev_ptr(x), _dev_ptr(y), _dev_ptr(gamma), _dev_ptr(beta),
                                                  _dev_ptr(sum_out), _dev_ptr(out), _dev_ptr(stats[0]),
                                                  _dev_ptr(stats[1]), rows, f, _stream_ptr()))


def layer_norm_backward_residual_into(grad_out, x, gamma, stats, residual, grad_x, grad_gamma, grad_beta):
    """dfgpt2_layernorm_backward_residual: grad_x = LayerNorm backward (+ residual unless None);
    grad_gamma and grad_beta are overwritten."""
    rows, f = _rows_cols(x)
    res = _dev_ptr(residual) if residual is not None else None
    _check(ops_lib().dfgpt2_layernorm_backward_residual(
        _dev_ptr(grad_out), _dev_ptr(x), _dev_ptr(gamma), _dev_ptr(stats[0]), _dev_ptr(stats[1]), res,
        _dev_ptr(grad_x), _dev_ptr(grad_gamma), _dev_ptr(grad_beta), rows, f, _stream_ptr()))


def layer_norm_backward_fused_workspace_bytes(rows, features):
    return int(ops_lib().dfgpt2_layernorm_backward_fused_workspace_bytes(rows, features))


def layer_norm_backward_fused_into(grad_out, x, gamma, stats, residual, grad_x, grad_gamma, grad_beta, grad_bias,
                                   workspace):
    """dfgpt2_layernorm_backward_fused: layer_norm_backward_residual_into, plus grad_bias (unless None)
    = the column sums of grad_x, with the rows read once; workspace: a float32 device tensor of at
    least layer_norm_backward_fused_workspace_bytes(rows, features) bytes."""
    rows, f = _rows_cols(x)
    opt = lambda t: _dev_ptr(t) if t is not None else None
    _check(ops_lib().dfgpt2_layernorm_backward_fused(
        _dev_ptr(grad_out), _dev_ptr(x), opt(gamma), _dev_ptr(stats[0]), _dev_ptr(stats[1]), opt(residual),
        _dev_ptr(grad_x), opt(grad_gamma), opt(grad_beta), opt(grad_bias), _dev_ptr(workspace),
        workspace.numel() * workspace.element_size(), rows, f, _stream_ptr()))


def add_bias_into(x, bias, out=None):
    """dfgpt2_add_bias: out = x + bias per row (out=None: in place)."""
    rows, cols = _rows_cols(x)
    out = x if out is None else out
    _check(ops_lib().dfgpt2_add_bias(_dev_ptr(x), _dev_ptr(bias), _dev_ptr(out), rows, cols, _stream_ptr()))
    return out


def bias_gelu_forward_into(h, bias, out):
    """dfgpt2_bias_gelu_forward: h += bias (per column, in place), out = gelu(h)."""
    rows, cols = _rows_cols(h)
    _check(ops_lib().dfgpt2_bias_gelu_forward(_dev_ptr(h), _dev_ptr(bias), _dev_ptr(out), rows, cols, _stream_ptr()))


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


def _ids_ptr(t):
    """Token ids: a contiguous int32 device tensor, passed as the kernels' uint32 ids."""
    torch = _torch()
    if not t.is_cuda or t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError("token ids must be a contiguous int32 device tensor")
    return ctypes.c_void_p(t.data_ptr())


def logit_ce_chunk(logits, targets, grad, row_loss, total_rows):
    """dfgpt2_logit_ce_chunk over logits [rows, V] (int32 targets [rows]); grad may be logits itself.
    Each row's loss goes to row_loss[row]."""
    rows, v = _rows_cols(logits)
    _check(ops_lib().dfgpt2_logit_ce_chunk(_dev_ptr(logits), _ids_ptr(targets), _dev_ptr(grad), _dev_ptr(row_loss),
                                           rows, v, total_rows, _stream_ptr()))


def sum_into(values, out, accumulate=False):
    """dfgpt2_sum: out (a 1-element tensor) = (out if accumulate) + sum(values), fixed order."""
    _check(ops_lib().dfgpt2_sum(_dev_ptr(values), values.numel(), _dev_ptr(out), int(bool(accumulate)),
                                _stream_ptr()))


def embedding_forward(ids, table, out):
    """dfgpt2_embedding_forward: out[p] = table[ids[p]] (ids past the table give zero rows)."""
    rows_in_table, dim = _rows_cols(table)
    _check(ops_lib().dfgpt2_embedding_forward(_ids_ptr(ids), _dev_ptr(table), _dev_ptr(out), ids.numel(), dim,
                                              rows_in_table, _stream_ptr()))


def embedding_backward(ids, grad_out, grad_table):
    """dfgpt2_embedding_backward: grad_table[ids[p]] += grad_out[p], rows of one id summed in order."""
    rows_in_table, dim = _rows_cols(grad_table)
    _check(ops_lib().dfgpt2_embedding_backward(_ids_ptr(ids), _dev_ptr(grad_out), _dev_ptr(grad_table), ids.numel(),
                                               dim, rows_in_table, _stream_ptr()))


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

