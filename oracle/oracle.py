"""numpy front end of the CPU attention oracle (oracle/attention_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker, and by bench.py's cpu_baseline leg. The product path
(dark-forest_amd/dfattn and libdfattn.so) never imports this module.

Every function takes and returns contiguous numpy arrays in the reference's
layout: [S, H*D] for Q, K, V, O, dO, dQ, dK, dV and [H, S] for logsumexp.
The restated reference functions are named in attention_oracle.c's header:
static_gpt2.rs:2766-2798 (multi-head forward), lib.rs:2493-2527
(reference_attention) and lib.rs:2529-2586 (reference_backward).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

MUTATIONS = {
    "none": 0,
    "causal_off_by_one": 1,
    "drop_scale": 2,
    "k_from_v": 3,
    "drop_correction": 4,
    "dk_sign": 5,
    "head_index": 6,
    "lse_log2": 7,
    "dv_from_ds": 8,
    "transpose_dq": 9,
    "rope_sin_sign": 10,
    "rope_freq": 11,
    "interp_same_row": 12,
    "bf16_truncate": 13,
    "page_offset": 14,
}
# Mistakes planted in the elementwise restatements (RoPE, interpolation, paged copy, bf16).
AUX_MUTATIONS = ("rope_sin_sign", "rope_freq", "interp_same_row", "bf16_truncate", "page_offset")


def build() -> str:
    """Compile liboracle.so with oracle/Makefile (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    f32p = ctypes.POINTER(ctypes.c_float)
    f64p = ctypes.POINTER(ctypes.c_double)
    i64p = ctypes.POINTER(ctypes.c_int64)
    c_int, c_float, c_double = ctypes.c_int, ctypes.c_float, ctypes.c_double
    lib.oracle_mha_forward_f32.argtypes = [f32p, f32p, f32p, f32p, f32p, c_int, c_int, c_int, c_float, c_int, c_int]
    lib.oracle_mha_forward_f64.argtypes = [f64p, f64p, f64p, f64p, f64p, c_int, c_int, c_int, c_double, c_int, c_int]
    lib.oracle_mha_forward_rows_f32.argtypes = [f32p, f32p, f32p, i64p, c_int, f32p, f32p, c_int, c_int, c_int, c_float, c_int, c_int]
    lib.oracle_reference_attention_f32.argtypes = [f32p, f32p, f32p, f32p, c_int, c_int, c_float, c_int]
    lib.oracle_reference_backward_f32.argtypes = [f32p] * 7 + [c_int, c_int, c_int, c_float, c_int, c_int]
    lib.oracle_backward_f64.argtypes = [f64p] * 7 + [c_int, c_int, c_int, c_double, c_int, c_int]
    vp, i32p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32)
    lib.oracle_decode_f32.argtypes = [f32p, vp, vp, i32p, c_int, c_int, f32p, f32p, c_int, c_int, c_int, c_float]
    lib.oracle_decode_f64.argtypes = [f64p, vp, vp, i32p, c_int, c_int, f64p, f64p, c_int, c_int, c_int, c_double]
    lib.oracle_decode_f32.restype = lib.oracle_decode_f64.restype = None
    u32 = ctypes.c_uint32
    lib.oracle_pos_embed_interpolate_f32.argtypes = [f32p, f32p, u32, u32, u32, u32]
    lib.oracle_apply_rope_f32.argtypes = [f32p, u32, u32, u32, c_float]
    lib.oracle_apply_rope_f64.argtypes = [f64p, u32, u32, u32, c_double]
    lib.oracle_paged_copy_row.argtypes = [f32p, vp, c_int, ctypes.c_int32, u32, u32, u32]
    lib.oracle_f32_to_bf16.argtypes = [c_float]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    for fn in (lib.oracle_pos_embed_interpolate_f32, lib.oracle_apply_rope_f32, lib.oracle_apply_rope_f64,
               lib.oracle_paged_copy_row):
        fn.restype = None
    lib.oracle_set_mutation.argtypes = [c_int]
    lib.oracle_get_mutation.restype = c_int
    lib.oracle_max_threads.restype = c_int
    for fn in (lib.oracle_mha_forward_f32, lib.oracle_mha_forward_f64, lib.oracle_mha_forward_rows_f32,
               lib.oracle_reference_attention_f32, lib.oracle_reference_backward_f32, lib.oracle_backward_f64,
               lib.oracle_set_mutation):
        fn.restype = None
    _lib = lib
    return lib


def _ptr(a, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _as(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def default_threads() -> int:
    return int(_load().oracle_max_threads())


def set_mutation(name: str) -> None:
    """Plant a known mistake in the oracle (tests of the pinning checks only)."""
    _load().oracle_set_mutation(MUTATIONS[name])


def mha_forward(q, k, v, n_heads, scale, causal=True, threads=1, dtype=np.float32):
    """Multi-head forward (static_gpt2.rs:2766-2798). Returns (O, lse)."""
    lib = _load()
    ct = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    q, k, v = _as(q, dtype), _as(k, dtype), _as(v, dtype)
    seq_len, dm = q.shape
    d_head = dm // n_heads
    out = np.empty_like(q)
    lse = np.empty((n_heads, seq_len), dtype=dtype)
    fn = lib.oracle_mha_forward_f32 if dtype == np.float32 else lib.oracle_mha_forward_f64
    fn(_ptr(q, ct), _ptr(k, ct), _ptr(v, ct), _ptr(out, ct), _ptr(lse, ct),
       n_heads, seq_len, d_head, ct(scale), int(bool(causal)), int(threads))
    return out, lse


def mha_forward_rows(q, k, v, rows, n_heads, scale, causal=True, threads=1):
    """Forward for selected query rows only. Returns (O_rows [n, H*D], lse_rows [n, H])."""
    lib = _load()
    q, k, v = _as(q, np.float32), _as(k, np.float32), _as(v, np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    seq_len, dm = q.shape
    d_head = dm // n_heads
    out = np.empty((rows.size, dm), dtype=np.float32)
    lse = np.empty((rows.size, n_heads), dtype=np.float32)
    lib.oracle_mha_forward_rows_f32(_ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float),
                                    _ptr(rows, ctypes.c_int64), int(rows.size), _ptr(out, ctypes.c_float),
                                    _ptr(lse, ctypes.c_float), n_heads, seq_len, d_head, ctypes.c_float(scale),
                                    int(bool(causal)), int(threads))
    return out, lse


def reference_attention(q, k, v, scale, causal=True):
    """Single-head forward (lib.rs:2493-2527), tensors [S, D]."""
    lib = _load()
    q, k, v = _as(q, np.float32), _as(k, np.float32), _as(v, np.float32)
    seq_len, d_head = q.shape
    out = np.empty_like(q)
    lib.oracle_reference_attention_f32(_ptr(q, ctypes.c_float), _ptr(k, ctypes.c_float), _ptr(v, ctypes.c_float),
                                       _ptr(out, ctypes.c_float), seq_len, d_head, ctypes.c_float(scale),
                                       int(bool(causal)))
    return out


def backward(q, k, v, d_out, n_heads, scale, causal=True, threads=1, dtype=np.float32):
    """Backward (lib.rs:2529-2586 per head). Returns (dQ, dK, dV)."""
    lib = _load()
    ct = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    q, k, v, d_out = (_as(a, dtype) for a in (q, k, v, d_out))
    seq_len, dm = q.shape
    d_head = dm // n_heads
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    fn = lib.oracle_reference_backward_f32 if dtype == np.float32 else lib.oracle_backward_f64
    fn(_ptr(q, ct), _ptr(k, ct), _ptr(v, ct), _ptr(d_out, ct), _ptr(dq, ct), _ptr(dk, ct), _ptr(dv, ct),
       n_heads, seq_len, d_head, ct(scale), int(bool(causal)), int(threads))
    return dq, dk, dv


def decode(q, k_cache, v_cache, n_heads, cur_len, scale, block_table=None, page_size=1, dtype=np.float32):
    """Single-query KV-cache decode (attention_fused.cu:551-615; paged 800-866; bf16 968-1033).

    q: [H*D]. k_cache, v_cache: [rows, H*D] float (fp32, or fp64 with dtype) or uint16 bf16 bit
    patterns. block_table: int32 logical page -> physical block (None: contiguous cache).
    Returns (out [H*D], lse [H]); cur_len = 0 returns (None, None) as nothing is computed.
    """
    lib = _load()
    ct = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    q = _as(q, dtype).reshape(-1)
    bf16 = np.asarray(k_cache).dtype == np.uint16
    if bf16:
        k_cache, v_cache = (np.ascontiguousarray(a, dtype=np.uint16) for a in (k_cache, v_cache))
    else:
        k_cache, v_cache = _as(k_cache, dtype), _as(v_cache, dtype)
    d_head = q.size // n_heads
    out = np.full(q.size, np.nan, dtype=dtype)
    lse = np.full(n_heads, np.nan, dtype=dtype)
    if block_table is not None:
        block_table = np.ascontiguousarray(block_table, dtype=np.int32)
        bt = block_table.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    else:
        bt = None
    fn = lib.oracle_decode_f32 if dtype == np.float32 else lib.oracle_decode_f64
    fn(_ptr(q, ct), k_cache.ctypes.data_as(ctypes.c_void_p), v_cache.ctypes.data_as(ctypes.c_void_p), bt,
       int(page_size), int(bf16), _ptr(out, ct), _ptr(lse, ct), n_heads, int(cur_len), d_head, ct(scale))
    if cur_len <= 0:
        return None, None
    return out, lse


def pos_embed_interpolate(table, pos, trained_ctx_len, max_ctx_len):
    """attention_fused.cu:1098-1121 on table [trained, d_model]; returns out [d_model]."""
    lib = _load()
    table = _as(table, np.float32)
    d_model = table.shape[-1]
    out = np.full(d_model, np.nan, dtype=np.float32)
    lib.oracle_pos_embed_interpolate_f32(_ptr(table, ctypes.c_float), _ptr(out, ctypes.c_float), int(pos),
                                         int(trained_ctx_len), int(max_ctx_len), d_model)
    return out


def apply_rope(qk, pos, n_heads, d_head, base_freq, dtype=np.float32):
    """attention_fused.cu:1139-1162 on a copy of qk [n_heads * d_head]; returns the rotated row."""
    lib = _load()
    ct = ctypes.c_float if dtype == np.float32 else ctypes.c_double
    x = _as(qk, dtype).reshape(-1).copy()
    fn = lib.oracle_apply_rope_f32 if dtype == np.float32 else lib.oracle_apply_rope_f64
    fn(_ptr(x, ct), int(pos), int(n_heads), int(d_head), ct(base_freq))
    return x


def paged_copy_row(src, pool, phys_block, page_offset, page_size):
    """attention_fused.cu:1178-1217: writes src into row phys_block * page_size + page_offset of pool
    (float32, or uint16 bf16 bit patterns) in place."""
    lib = _load()
    src = _as(src, np.float32).reshape(-1)
    assert pool.flags["C_CONTIGUOUS"] and pool.dtype in (np.float32, np.uint16)
    lib.oracle_paged_copy_row(_ptr(src, ctypes.c_float), pool.ctypes.data_as(ctypes.c_void_p),
                              int(pool.dtype == np.uint16), int(phys_block), int(page_offset), int(page_size),
                              src.size)
    return pool


def f32_to_bf16(a):
    """fp32 -> bf16 bit patterns through the oracle's scalar rounding (NaN-aware), as uint16."""
    lib = _load()
    flat = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    return np.array([lib.oracle_f32_to_bf16(float(x)) for x in flat], dtype=np.uint16).reshape(np.shape(a))


def to_bf16_bits(a):
    """fp32 -> bf16 bit patterns (round to nearest even), as uint16."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def from_bf16_bits(b):
    """bf16 bit patterns (uint16) -> fp32, exactly."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def seeded_inputs(seq_len, n_heads, d_head, seed, std=1.0, with_grad=True):
    """Q, K, V (and dO) iid N(0, std^2), fp32 [S, H*D], one PCG64 stream per tensor.

    Streams are seeded base+0 (Q), +1 (K), +2 (V), +3 (dO), so a config's
    inputs are identical wherever they are generated.
    """
    dm = n_heads * d_head
    names = ["q", "k", "v", "do"] if with_grad else ["q", "k", "v"]
    out = {}
    for i, name in enumerate(names):
        rng = np.random.Generator(np.random.PCG64(seed + i))
        a = rng.standard_normal((seq_len, dm), dtype=np.float32)
        if std != 1.0:
            a *= np.float32(std)
        out[name] = a
    return out
