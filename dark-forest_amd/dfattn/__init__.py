"""dfattn — Python binding of libdfattn.so, the gfx950 fused causal attention library.

The library's C ABI is include/dfattn.h. This module loads the in-tree build
(dark-forest_amd/lib/libdfattn.so) with ctypes and offers:

* ``lib()``: the raw ctypes handle with every exported symbol typed;
* torch-tensor wrappers over the fast path (``attention_forward``,
  ``attention_backward``) and over the reference's launcher symbols
  (``launch_fused_mha_forward`` ...), taking device tensors and passing their
  pointers and torch's current HIP stream;
* ``AttentionContext``, the mirror of the reference's per-layer context
  (darkforest-cuda/src/lib.rs:1949-2368), and the host-slice helpers
  ``fused_attention_forward`` / ``attention_backward_host`` (lib.rs:2371, 2421);
* ``FusedCausalAttention``, a torch.autograd.Function over the fast path.

There is no CPU fallback: if the library is missing every call raises
``DfattnNotBuilt``.
"""
from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_PKG_DIR), "lib", "libdfattn.so")

DFATTN_OK = 0
STATUS_NAMES = {
    0: "DFATTN_OK",
    -1: "DFATTN_ERR_NULL_POINTER",
    -2: "DFATTN_ERR_MISALIGNED",
    -3: "DFATTN_ERR_SHAPE",
    -4: "DFATTN_ERR_HEAD_DIM",
    -5: "DFATTN_ERR_OVERFLOW",
    -6: "DFATTN_ERR_WORKSPACE",
    -7: "DFATTN_ERR_HIP",
}

# Every symbol include/dfattn.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_F = ctypes.c_float
SYMBOLS = {
    "launch_fused_attention": (None, [_P, _P, _P, _P, _U32, _U32, _F, _U32]),
    "launch_fused_mha_forward": (None, [_P, _P, _P, _P, _U32, _U32, _U32, _F, _U32]),
    "launch_attention_backward": (None, [_P] * 8 + [_U32, _U32, _F, _U32]),
    "launch_fused_mha_backward": (None, [_P] * 8 + [_U32, _U32, _U32, _F, _U32]),
    "darkforest_sync": (None, []),
    "dfattn_fwd": (ctypes.c_int, [_P] * 5 + [_U32, _U32, _U32, _F, _U32, _P]),
    "dfattn_bwd_workspace_bytes": (ctypes.c_size_t, [_U32, _U32, _U32]),
    "dfattn_bwd": (ctypes.c_int, [_P] * 10 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _P]),
    "dfattn_fwd_train": (ctypes.c_int, [_P] * 6 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _P]),
    "dfattn_bwd_preprocess": (ctypes.c_int, [_P] * 7 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _P]),
    "dfattn_bwd_main": (ctypes.c_int, [_P] * 10 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _P]),
    "dfattn_fwd_train_strided": (ctypes.c_int, [_P] * 6 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _U32, _P]),
    "dfattn_bwd_preprocess_strided": (ctypes.c_int, [_P] * 7 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _U32,
                                                                 _P]),
    "dfattn_bwd_main_strided": (ctypes.c_int, [_P] * 5 + [ctypes.c_size_t, _U32, _U32, _U32, _F, _U32, _U32, _P]),
    "dfattn_bwd_noalloc": (ctypes.c_int, [_P] * 9 + [_U32, _U32, _U32, _F, _U32, _P]),
    "launch_fused_mha_decode_kv": (None, [_P] * 4 + [_U32, _U32, _U32, _F]),
    "launch_fused_mha_decode_kv_splitk": (None, [_P] * 7 + [_U32, _U32, _U32, _F, _U32]),
    "launch_paged_mha_decode_kv": (None, [_P] * 5 + [_U32, _U32, _U32, _F, _U32]),
    "launch_paged_mha_decode_kv_splitk": (None, [_P] * 8 + [_U32, _U32, _U32, _F, _U32, _U32]),
    "launch_paged_mha_decode_kv_bf16": (None, [_P] * 5 + [_U32, _U32, _U32, _F, _U32]),
    "launch_pos_embed_interpolate": (None, [_P, _P, _U32, _U32, _U32, _U32]),
    "launch_apply_rope": (None, [_P, _U32, _U32, _U32, _F]),
    "launch_paged_copy_row": (None, [_P, _P, ctypes.c_int32, _U32, _U32, _U32]),
    "launch_paged_copy_row_f32_to_bf16": (None, [_P, _P, ctypes.c_int32, _U32, _U32, _U32]),
    "dfattn_decode_workspace_bytes": (ctypes.c_size_t, [_U32, _U32, _U32]),
    "dfattn_decode": (ctypes.c_int, [_P] * 4 + [_U32, _U32, _P, _P, _U32, _U32, _U32, _F, _P, ctypes.c_size_t, _P]),
    "dfattn_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "dfattn_last_error": (ctypes.c_int, []),
    "dfattn_last_error_message": (ctypes.c_char_p, []),
    "dfattn_clear_error": (None, []),
    "dfattn_version": (ctypes.c_char_p, []),
    "dfattn_context_create": (ctypes.c_int, [_U32, _U32, _U32, ctypes.POINTER(ctypes.c_void_p)]),
    "dfattn_context_destroy": (None, [_P]),
    "dfattn_context_dims": (ctypes.c_int, [_P] + [ctypes.POINTER(_U32)] * 4),
    "dfattn_context_lse": (_P, [_P]),
    "dfattn_context_set_reuse_forward": (ctypes.c_int, [_P, _U32]),
    "dfattn_context_forward_device_into": (ctypes.c_int, [_P] * 4 + [_F, _U32, _P, ctypes.c_size_t, _P]),
    "dfattn_context_backward_device_into": (ctypes.c_int,
                                            [_P] * 5 + [_F, _U32, _P, _P, _P, ctypes.c_size_t, _P]),
    "dfattn_context_forward_device_into_strided": (ctypes.c_int,
                                                   [_P] * 4 + [_F, _U32, _P, ctypes.c_size_t, _U32, _P]),
    "dfattn_context_backward_device_into_strided": (ctypes.c_int, [_P] * 5 + [_F, _U32, _P, _P, _P, ctypes.c_size_t,
                                                                              _U32, _U32, _P]),
    "dfattn_context_forward": (ctypes.c_int, [_P] * 4 + [ctypes.c_size_t, _F, _U32, _P]),
    "dfattn_context_backward": (ctypes.c_int, [_P, _P, ctypes.c_size_t, _F, _U32, _P, _P, _P]),
    "dfattn_fused_attention_forward": (ctypes.c_int, [_P] * 3 + [ctypes.c_size_t, _U32, _U32, _F, _U32, _P]),
    "dfattn_attention_backward": (ctypes.c_int,
                                  [_P] * 4 + [ctypes.c_size_t, _U32, _U32, _F, _U32, _P, _P, _P]),
}


class DfattnNotBuilt(RuntimeError):
    """libdfattn.so is missing: run __graft_entry__.build() (or make -C dark-forest_amd/csrc)."""


class DfattnError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_lib = None


def lib():
    """The loaded library with typed symbols. Raises DfattnNotBuilt if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DfattnNotBuilt(f"{LIB_PATH} not found; build it with __graft_entry__.build()")
    # The library and torch must share one HIP runtime: the wrappers pass torch's streams and device
    # pointers to it. torch bundles its own libamdhip64 under the same soname, so loading torch first
    # makes the dynamic linker bind the library to that copy; loaded the other way round the process
    # would hold two runtimes, and the one the library uses may not see the GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SYMBOLS.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return handle


def version() -> str:
    return lib().dfattn_version().decode()


def _check(status: int) -> None:
    if status != DFATTN_OK:
        msg = lib().dfattn_last_error_message().decode()
        raise DfattnError(status, msg)


# ---------------------------------------------------------------- torch layer
def _torch():
    import torch

    return torch


def _stream_ptr(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dev_ptr(t):
    if t is None:
        return None
    torch = _torch()
    if not t.is_cuda:
        raise ValueError("dfattn works on device tensors; got a CPU tensor")
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError("dfattn tensors must be contiguous float32")
    return ctypes.c_void_p(t.data_ptr())


def _row_stride(t):
    """Row stride in floats of a 2-D float32 tensor whose rows are contiguous, such as a column
    block of a wider tensor; None when the tensor is contiguous. Raises for any other layout."""
    torch = _torch()
    if t.dtype != torch.float32:
        raise ValueError("dfattn tensors must be float32")
    if t.is_contiguous():
        return None
    if t.dim() != 2 or t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        raise ValueError("dfattn tensors must be contiguous or 2-D with contiguous rows")
    return t.stride(0)


def _rows_ptr(t):
    """(device pointer, row stride or None) of a tensor _row_stride accepts."""
    stride = _row_stride(t)
    if not t.is_cuda:
        raise ValueError("dfattn works on device tensors; got a CPU tensor")
    return ctypes.c_void_p(t.data_ptr()), stride


def _same_stride(name, *tensors):
    """The device pointers and the one row stride of `tensors` (None: all contiguous); raises when
    they differ."""
    ptrs, strides = zip(*(_rows_ptr(t) for t in tensors))
    if len(set(strides)) != 1:
        raise ValueError(f"{name} must share one row stride")
    return ptrs, strides[0]


def _dims(q, n_heads):
    seq_len, dm = q.shape
    if dm % n_heads:
        raise ValueError("q.shape[1] must be n_heads * d_head")
    return seq_len, dm // n_heads


def attention_forward(q, k, v, n_heads, scale=None, causal=True, out=None, lse=None, stream=None):
    """Fast-path forward. q, k, v: [S, H*D] float32 on the GPU. Returns (O, lse[H, S])."""
    torch = _torch()
    seq_len, d_head = _dims(q, n_heads)
    if scale is None:
        scale = d_head ** -0.5
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty((n_heads, seq_len), dtype=torch.float32, device=q.device)
    _check(lib().dfattn_fwd(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(out), _dev_ptr(lse),
                            n_heads, seq_len, d_head, scale, int(bool(causal)), _stream_ptr(stream)))
    return out, lse


def forward_train(q, k, v, n_heads, workspace, scale=None, causal=True, out=None, lse=None, stream=None):
    """attention_forward that also leaves the backward's fp16 copies of Q, K, V in `workspace`
    (dfattn_fwd_train); follow with backward_preprocess(..., flags=BWD_QKV_SAVED)."""
    torch = _torch()
    seq_len, d_head = _dims(q, n_heads)
    if scale is None:
        scale = d_head ** -0.5
    if out is None:  # contiguous even when q is a column block of a wider tensor
        out = torch.empty((seq_len, n_heads * d_head), dtype=torch.float32, device=q.device)
    if lse is None:
        lse = torch.empty((n_heads, seq_len), dtype=torch.float32, device=q.device)
    (pq, pk, pv), stride = _same_stride("q, k and v", q, k, v)
    ws = (_dev_ptr(workspace), workspace.numel() * workspace.element_size())
    if stride is None:
        _check(lib().dfattn_fwd_train(pq, pk, pv, _dev_ptr(out), _dev_ptr(lse), *ws, n_heads, seq_len, d_head,
                                      scale, int(bool(causal)), _stream_ptr(stream)))
    else:  # q, k, v are column blocks of a wider tensor (dfattn_fwd_train_strided)
        _check(lib().dfattn_fwd_train_strided(pq, pk, pv, _dev_ptr(out), _dev_ptr(lse), *ws, n_heads, seq_len, d_head,
                                              scale, int(bool(causal)), stride, _stream_ptr(stream)))
    return out, lse


def bwd_workspace_bytes(n_heads, seq_len, d_head) -> int:
    return int(lib().dfattn_bwd_workspace_bytes(n_heads, seq_len, d_head))


def attention_backward(q, k, v, o, d_o, lse, n_heads, scale=None, causal=True, d_q=None, d_k=None,
                       d_v=None, workspace=None, stream=None):
    """Fast-path backward from the forward's O and lse. Returns (dQ, dK, dV)."""
    torch = _torch()
    seq_len, d_head = _dims(q, n_heads)
    if scale is None:
        scale = d_head ** -0.5
    d_q = torch.empty_like(q) if d_q is None else d_q
    d_k = torch.empty_like(q) if d_k is None else d_k
    d_v = torch.empty_like(q) if d_v is None else d_v
    need = bwd_workspace_bytes(n_heads, seq_len, d_head)
    if workspace is None:
        workspace = torch.empty(max(need, 4) // 4, dtype=torch.float32, device=q.device)
    _check(lib().dfattn_bwd(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(o), _dev_ptr(d_o), _dev_ptr(lse),
                            _dev_ptr(d_q), _dev_ptr(d_k), _dev_ptr(d_v), _dev_ptr(workspace),
                            workspace.numel() * workspace.element_size(), n_heads, seq_len, d_head, scale,
                            int(bool(causal)), _stream_ptr(stream)))
    return d_q, d_k, d_v


NOALLOC_SCRATCH_BYTES = 32 << 20  # DFATTN_NOALLOC_SCRATCH_BYTES


def attention_backward_noalloc(q, k, v, o, d_o, lse, n_heads, scale=None, causal=True, d_q=None, d_k=None,
                               d_v=None, stream=None):
    """dfattn_bwd_noalloc: attention_backward with the workspace in the library's static device array
    (nothing is allocated by the library; pass d_q, d_k, d_v to allocate nothing here either).
    Calls that overlap on one GPU race on that array."""
    torch = _torch()
    seq_len, d_head = _dims(q, n_heads)
    if scale is None:
        scale = d_head ** -0.5
    d_q = torch.empty_like(q) if d_q is None else d_q
    d_k = torch.empty_like(q) if d_k is None else d_k
    d_v = torch.empty_like(q) if d_v is None else d_v
    _check(lib().dfattn_bwd_noalloc(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(o), _dev_ptr(d_o), _dev_ptr(lse),
                                    _dev_ptr(d_q), _dev_ptr(d_k), _dev_ptr(d_v), n_heads, seq_len, d_head, scale,
                                    int(bool(causal)), _stream_ptr(stream)))
    return d_q, d_k, d_v


BWD_QKV_SAVED = 1  # DFATTN_BWD_QKV_SAVED


def backward_preprocess(q, k, v, o, d_o, lse, workspace, n_heads, scale=None, flags=0, stream=None):
    """First phase of attention_backward (row statistics, the dO range and the fp16 operand
    copies, all in the workspace); flags=BWD_QKV_SAVED after forward_train."""
    seq_len, d_head = _dims(q, n_heads)
    if scale is None:
        scale = d_head ** -0.5
    (pq, pk, pv), stride = _same_stride("q, k and v", q, k, v)
    rest = (_dev_ptr(o), _dev_ptr(d_o), _dev_ptr(lse), _dev_ptr(workspace), workspace.numel() * workspace.element_size(),
            n_heads, seq_len, d_head, scale, int(flags))
    if stride is None:
        _check(lib().dfattn_bwd_preprocess(pq, pk, pv, *rest, _stream_ptr(stream)))
    else:
        _check(lib().dfattn_bwd_preprocess_strided(pq, pk, pv, *rest, stride, _stream_ptr(stream)))


def backward_main(q, k, v, o, d_o, lse, d_q, d_k, d_v, workspace, n_heads, scale=None, causal=True, stream=None):
    """Second phase of attention_backward (the fused dQ/dK/dV kernel); same q, k, v, o, d_o,
    lse, workspace and scale as backward_preprocess. q, k, v, and d_q, d_k, d_v, may each be
    column blocks of one wider tensor; the strided kernel then reads only the workspace."""
    seq_len, d_head = _dims(q, n_heads)
    if scale is None:
        scale = d_head ** -0.5
    (pdq, pdk, pdv), stride = _same_stride("d_q, d_k and d_v", d_q, d_k, d_v)
    (pq, pk, pv), qkv_stride = _same_stride("q, k and v", q, k, v)
    ws = (_dev_ptr(workspace), workspace.numel() * workspace.element_size())
    if stride is None and qkv_stride is not None:
        stride = n_heads * d_head  # contiguous gradients, but the unstrided call would take q, k, v as packed
    if stride is None:
        _check(lib().dfattn_bwd_main(pq, pk, pv, _dev_ptr(o), _dev_ptr(d_o), _dev_ptr(lse), pdq, pdk, pdv, *ws,
                                     n_heads, seq_len, d_head, scale, int(bool(causal)), _stream_ptr(stream)))
    else:  # gradients into column blocks of a wider tensor (dfattn_bwd_main_strided)
        _check(lib().dfattn_bwd_main_strided(_dev_ptr(lse), pdq, pdk, pdv, *ws, n_heads, seq_len, d_head, scale,
                                             int(bool(causal)), stride, _stream_ptr(stream)))


def launch_fused_mha_forward(q, k, v, out, n_heads, seq_len, d_head, scale, causal):
    """The reference's launcher symbol (attention_fused.cu:233), null stream."""
    lib().launch_fused_mha_forward(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(out), n_heads, seq_len,
                                   d_head, scale, int(bool(causal)))


def launch_fused_attention(q, k, v, out, seq_len, d_head, scale, causal):
    """attention_fused.cu:223, null stream."""
    lib().launch_fused_attention(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(out), seq_len, d_head, scale,
                                 int(bool(causal)))


def launch_fused_mha_backward(q, k, v, d_out, d_q, d_k, d_v, probabilities, n_heads, seq_len, d_head, scale,
                              causal):
    """attention_fused.cu:518, null stream."""
    lib().launch_fused_mha_backward(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(d_out), _dev_ptr(d_q),
                                    _dev_ptr(d_k), _dev_ptr(d_v), _dev_ptr(probabilities), n_heads, seq_len,
                                    d_head, scale, int(bool(causal)))


def launch_attention_backward(q, k, v, d_out, d_q, d_k, d_v, probabilities, seq_len, d_head, scale, causal):
    """attention_fused.cu:361, null stream."""
    lib().launch_attention_backward(_dev_ptr(q), _dev_ptr(k), _dev_ptr(v), _dev_ptr(d_out), _dev_ptr(d_q),
                                    _dev_ptr(d_k), _dev_ptr(d_v), _dev_ptr(probabilities), seq_len, d_head,
                                    scale, int(bool(causal)))


def darkforest_sync():
    """matmul.cu:21: device synchronize; aborts the process on error."""
    lib().darkforest_sync()


# ---------------------------------------------------------------- decode (attention_fused.cu:551-1090)
KV_F32, KV_BF16 = 0, 1  # DFATTN_KV_F32, DFATTN_KV_BF16


def _dev_any(t):
    """Device pointer of a contiguous CUDA tensor of any dtype (the cache pools: float32 or bf16 bits)."""
    if t is None:
        return None
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("dfattn decode takes contiguous device tensors")
    return ctypes.c_void_p(t.data_ptr())


def decode_workspace_bytes(n_heads, cur_seq_len, d_head) -> int:
    return int(lib().dfattn_decode_workspace_bytes(n_heads, cur_seq_len, d_head))


def decode(q, k_cache, v_cache, n_heads, cur_seq_len, scale=None, block_table=None, page_size=1, out=None,
           lse=None, workspace="auto", stream=None):
    """One query q [H*D] against the first cur_seq_len cached keys. k_cache, v_cache: float32, or bfloat16 /
    int16 / uint16 (bf16 bit patterns) [rows, H*D]; block_table: int32 pages (None: contiguous).
    workspace: "auto" allocates dfattn_decode_workspace_bytes, None walks the keys with one workgroup per head.
    Returns (out [H*D], lse [H])."""
    torch = _torch()
    d_head = q.numel() // n_heads
    if scale is None:
        scale = d_head ** -0.5
    kv_dtype = KV_F32 if k_cache.dtype == torch.float32 else KV_BF16
    if out is None:
        out = torch.empty(n_heads * d_head, dtype=torch.float32, device=q.device)
    if lse is None:
        lse = torch.empty(n_heads, dtype=torch.float32, device=q.device)
    if isinstance(workspace, str):
        nbytes = decode_workspace_bytes(n_heads, cur_seq_len, d_head)
        workspace = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=q.device) if nbytes else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(lib().dfattn_decode(_dev_ptr(q), _dev_any(k_cache), _dev_any(v_cache), _dev_any(block_table),
                               int(page_size), kv_dtype, _dev_ptr(out), _dev_ptr(lse), n_heads, int(cur_seq_len),
                               d_head, scale, _dev_any(workspace), ws_bytes, _stream_ptr(stream)))
    return out, lse


def launch_fused_mha_decode_kv(q, k_cache, v_cache, out, n_heads, cur_seq_len, d_head, scale):
    """attention_fused.cu:617, null stream."""
    lib().launch_fused_mha_decode_kv(_dev_ptr(q), _dev_ptr(k_cache), _dev_ptr(v_cache), _dev_ptr(out), n_heads,
                                     cur_seq_len, d_head, scale)


def launch_fused_mha_decode_kv_splitk(q, k_cache, v_cache, partial_m, partial_l, partial_o, out, n_heads,
                                      cur_seq_len, d_head, scale, chunk_size):
    """attention_fused.cu:762, null stream."""
    lib().launch_fused_mha_decode_kv_splitk(_dev_ptr(q), _dev_ptr(k_cache), _dev_ptr(v_cache), _dev_ptr(partial_m),
                                            _dev_ptr(partial_l), _dev_ptr(partial_o), _dev_ptr(out), n_heads,
                                            cur_seq_len, d_head, scale, chunk_size)


def launch_paged_mha_decode_kv(q, k_pool, v_pool, block_table, out, n_heads, cur_seq_len, d_head, scale, page_size):
    """attention_fused.cu:1028, null stream."""
    lib().launch_paged_mha_decode_kv(_dev_ptr(q), _dev_ptr(k_pool), _dev_ptr(v_pool), _dev_any(block_table),
                                     _dev_ptr(out), n_heads, cur_seq_len, d_head, scale, page_size)


def launch_paged_mha_decode_kv_splitk(q, k_pool, v_pool, block_table, partial_m, partial_l, partial_o, out,
                                      n_heads, cur_seq_len, d_head, scale, page_size, chunk_size):
    """attention_fused.cu:1045, null stream."""
    lib().launch_paged_mha_decode_kv_splitk(_dev_ptr(q), _dev_ptr(k_pool), _dev_ptr(v_pool), _dev_any(block_table),
                                            _dev_ptr(partial_m), _dev_ptr(partial_l), _dev_ptr(partial_o),
                                            _dev_ptr(out), n_heads, cur_seq_len, d_head, scale, page_size,
                                            chunk_size)


def launch_paged_mha_decode_kv_bf16(q, k_pool, v_pool, block_table, out, n_heads, cur_seq_len, d_head, scale,
                                    page_size):
    """attention_fused.cu:1075 (bf16 pools as bit patterns), null stream."""
    lib().launch_paged_mha_decode_kv_bf16(_dev_ptr(q), _dev_any(k_pool), _dev_any(v_pool), _dev_any(block_table),
                                          _dev_ptr(out), n_heads, cur_seq_len, d_head, scale, page_size)


# ---------------------------------------------------------------- elementwise companions (attention_fused.cu:1098-1231)
def launch_pos_embed_interpolate(pos_table, out, pos, trained_ctx_len, max_ctx_len, d_model):
    """attention_fused.cu:1123, null stream: out [d_model] := row pos of pos_table, or its linear
    interpolation at pos * (trained - 1) / (max - 1) outside the trained range."""
    lib().launch_pos_embed_interpolate(_dev_ptr(pos_table), _dev_ptr(out), pos, trained_ctx_len, max_ctx_len, d_model)


def launch_apply_rope(qk, pos, n_heads, d_head, base_freq):
    """attention_fused.cu:1164, null stream: rotary embedding of qk [n_heads * d_head] in place."""
    lib().launch_apply_rope(_dev_ptr(qk), pos, n_heads, d_head, base_freq)


def launch_paged_copy_row(src, pool, phys_block, page_offset, page_size, d_model):
    """attention_fused.cu:1192, null stream: pool row phys_block * page_size + page_offset := src."""
    lib().launch_paged_copy_row(_dev_ptr(src), _dev_ptr(pool), phys_block, page_offset, page_size, d_model)


def launch_paged_copy_row_f32_to_bf16(src, pool, phys_block, page_offset, page_size, d_model):
    """attention_fused.cu:1219, null stream: the same into a bf16 pool (int16 / uint16 / bfloat16 bits),
    rounded to nearest even."""
    lib().launch_paged_copy_row_f32_to_bf16(_dev_ptr(src), _dev_any(pool), phys_block, page_offset, page_size,
                                            d_model)



# ---------------------------------------------------------------- the reference's context
def _host_f32(a, name, n):
    import numpy as np

    arr = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    if arr.size != n:
        raise DfattnError(-3, f"{name} must have {n} elements, got {arr.size}")
    return arr


class AttentionContext:
    """Mirror of the reference's per-layer AttentionContext (darkforest-cuda/src/lib.rs:1949-2368).

    ``AttentionContext(n_heads, seq_len, d_head)`` validates like ``new_shared``
    (lib.rs:1975-1989) and allocates its logsumexp and backward workspace up
    front. Device-path methods take torch device tensors of shape
    [seq_len, n_heads * d_head]; host-slice methods take array-likes of
    seq_len * d_head floats and run one head, as the reference's do.
    """

    def __init__(self, n_heads, seq_len, d_head, reuse_forward=False):
        handle = ctypes.c_void_p()
        _check(lib().dfattn_context_create(n_heads, seq_len, d_head, ctypes.byref(handle)))
        self._h = handle
        self.n_heads, self.seq_len, self.d_head = n_heads, seq_len, d_head
        self.d_model = n_heads * d_head
        self._last = None  # q, k, v, out of the last device forward (kept alive while reuse is on)
        self.reuse_forward = False
        if reuse_forward:
            self.set_reuse_forward(True)

    def set_reuse_forward(self, enable):
        """dfattn_context_set_reuse_forward: let backward_device_into reuse the last
        forward_device_into on the same q, k, v (the caller promises not to modify q, k, v or that
        forward's out in between). This wrapper keeps those four tensors referenced, so they
        cannot be freed and reused by torch's allocator while the context may still read them."""
        _check(lib().dfattn_context_set_reuse_forward(self._h, int(bool(enable))))
        self.reuse_forward = bool(enable)
        if not enable:
            self._last = None

    def close(self):
        if getattr(self, "_h", None):
            lib().dfattn_context_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _elems(self, t):
        if tuple(t.shape) != (self.seq_len, self.d_model):
            return -1
        return t.numel()

    def forward_device_into(self, q, k, v, scale, causal, out, stream=None):
        """lib.rs:2042: O into `out`; also the context's logsumexp. q, k, v may be column blocks of
        one wider tensor (rows contiguous, one row stride: the strided context call)."""
        (pq, pk, pv), stride = _same_stride("q, k and v", q, k, v)
        n = self._elems(out) & ((1 << 64) - 1)
        if stride is None:
            _check(lib().dfattn_context_forward_device_into(self._h, pq, pk, pv, scale, int(bool(causal)),
                                                            _dev_ptr(out), n, _stream_ptr(stream)))
        else:
            _check(lib().dfattn_context_forward_device_into_strided(self._h, pq, pk, pv, scale, int(bool(causal)),
                                                                    _dev_ptr(out), n, stride, _stream_ptr(stream)))
        if self.reuse_forward:
            self._last = (q, k, v, out)

    def forward_device(self, q, k, v, scale, causal, stream=None):
        """lib.rs:2029: allocate O and run forward_device_into."""
        out = _torch().empty((self.seq_len, self.d_model), dtype=q.dtype, device=q.device)
        self.forward_device_into(q, k, v, scale, causal, out, stream)
        return out

    def backward_device_into(self, q, k, v, d_out, scale, causal, d_q, d_k, d_v, stream=None):
        """lib.rs:2240: dQ, dK, dV into the given tensors. q, k, v, and d_q, d_k, d_v, may each be
        column blocks of one wider tensor (the strided context call)."""
        n = min(self._elems(d_q), self._elems(d_k), self._elems(d_v)) & ((1 << 64) - 1)
        (pq, pk, pv), qs = _same_stride("q, k and v", q, k, v)
        (pdq, pdk, pdv), gs = _same_stride("d_q, d_k and d_v", d_q, d_k, d_v)
        if qs is None and gs is None:
            _check(lib().dfattn_context_backward_device_into(self._h, pq, pk, pv, _dev_ptr(d_out), scale,
                                                             int(bool(causal)), pdq, pdk, pdv, n, _stream_ptr(stream)))
        else:
            dm = self.d_model
            _check(lib().dfattn_context_backward_device_into_strided(
                self._h, pq, pk, pv, _dev_ptr(d_out), scale, int(bool(causal)), pdq, pdk, pdv, n,
                qs or dm, gs or dm, _stream_ptr(stream)))

    def backward_device(self, q, k, v, d_out, scale, causal, stream=None):
        """lib.rs:2226: allocate dQ, dK, dV and run backward_device_into."""
        torch = _torch()
        grads = [torch.empty((self.seq_len, self.d_model), dtype=q.dtype, device=q.device) for _ in range(3)]
        self.backward_device_into(q, k, v, d_out, scale, causal, *grads, stream=stream)
        return tuple(grads)

    def forward(self, q, k, v, scale, causal):
        """lib.rs:2295: host slices [seq_len * d_head] in, host O out."""
        import numpy as np

        n = self.seq_len * self.d_head
        arrs = [_host_f32(a, name, n) for a, name in ((q, "q"), (k, "k"), (v, "v"))]
        out = np.empty(n, dtype=np.float32)
        _check(lib().dfattn_context_forward(self._h, *(a.ctypes.data for a in arrs), n, scale, int(bool(causal)),
                                            out.ctypes.data))
        return out

    def backward(self, d_out, scale, causal):
        """lib.rs:2328: host dO in, host (dQ, dK, dV) out, for the last host forward's q, k, v."""
        import numpy as np

        n = self.seq_len * self.d_head
        g = _host_f32(d_out, "d_out", n)
        outs = [np.empty(n, dtype=np.float32) for _ in range(3)]
        _check(lib().dfattn_context_backward(self._h, g.ctypes.data, n, scale, int(bool(causal)),
                                             *(o.ctypes.data for o in outs)))
        return tuple(outs)


def fused_attention_forward(q, k, v, seq_len, d_head, scale, causal):
    """lib.rs:2371: one head from host slices; returns host O [seq_len * d_head]."""
    import numpy as np

    n = seq_len * d_head
    arrs = [_host_f32(a, name, n) for a, name in ((q, "q"), (k, "k"), (v, "v"))]
    out = np.empty(n, dtype=np.float32)
    _check(lib().dfattn_fused_attention_forward(*(a.ctypes.data for a in arrs), n, seq_len, d_head, scale,
                                                int(bool(causal)), out.ctypes.data))
    return out


def attention_backward_host(q, k, v, d_out, seq_len, d_head, scale, causal):
    """lib.rs:2421 attention_backward: one head from host slices; returns host (dQ, dK, dV)."""
    import numpy as np

    n = seq_len * d_head
    arrs = [_host_f32(a, name, n) for a, name in ((q, "q"), (k, "k"), (v, "v"), (d_out, "d_out"))]
    outs = [np.empty(n, dtype=np.float32) for _ in range(3)]
    _check(lib().dfattn_attention_backward(*(a.ctypes.data for a in arrs), n, seq_len, d_head, scale,
                                           int(bool(causal)), *(o.ctypes.data for o in outs)))
    return tuple(outs)


class FusedCausalAttention:
    """torch.autograd.Function over the fast path (the role of the reference's
    CudaAttentionGradFn, darkforest-core/src/autograd/grad_fn.rs:23-57).

    ``FusedCausalAttention.apply(q, k, v, n_heads, scale, causal)`` with q, k, v
    [S, H*D] float32 device tensors; the backward reuses the forward's O and
    logsumexp.
    """

    _fn = None

    @classmethod
    def apply(cls, q, k, v, n_heads, scale=None, causal=True):
        if cls._fn is None:
            torch = _torch()

            class _Fn(torch.autograd.Function):
                @staticmethod
                def forward(ctx, q, k, v, n_heads, scale, causal):
                    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
                    o, lse = attention_forward(q, k, v, n_heads, scale, causal)
                    ctx.save_for_backward(q, k, v, o, lse)
                    ctx.n_heads, ctx.scale, ctx.causal = n_heads, scale, causal
                    return o

                @staticmethod
                def backward(ctx, d_o):
                    q, k, v, o, lse = ctx.saved_tensors
                    dq, dk, dv = attention_backward(q, k, v, o, d_o.contiguous(), lse, ctx.n_heads, ctx.scale,
                                                    ctx.causal)
                    return dq, dk, dv, None, None, None

            cls._fn = _Fn
        d_head = q.shape[1] // n_heads
        return cls._fn.apply(q, k, v, n_heads, d_head ** -0.5 if scale is None else scale, causal)
