"""The C ABI library on the CPU: it loads, exports every symbol include/*.h declares,
and rejects bad arguments on the host before any HIP call (so no GPU is needed)."""
import ctypes
import os
import re

import pytest

import dfattn
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "dfattn.h")


def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while", "for", "return")))


def test_library_loads_and_exports_every_declared_symbol():
    lib = dfattn.lib()
    declared = declared_functions(HEADER)
    assert "launch_fused_mha_forward" in declared and "dfattn_bwd" in declared
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in dfattn.h but not exported"
    assert sorted(dfattn.SYMBOLS) == declared


def test_reference_symbols_present():
    # The four launchers and the sync the reference's kernels.rs binds (kernels.rs:9-20, 689-885).
    for name in ("launch_fused_attention", "launch_fused_mha_forward", "launch_attention_backward",
                 "launch_fused_mha_backward", "darkforest_sync"):
        assert name in declared_functions(HEADER)


def test_version_and_status_strings():
    assert "gfx950" in dfattn.version()
    lib = dfattn.lib()
    assert lib.dfattn_status_string(0) == b"ok"
    assert lib.dfattn_status_string(-6) == b"workspace too small"
    assert lib.dfattn_status_string(-99) == b"unknown status"


FAKE = ctypes.c_void_p(0x10000)  # aligned, never dereferenced: validation fails first
ODD = ctypes.c_void_p(0x10002)   # not 4-byte aligned


def fwd(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=None, h=12, s=128, d=64):
    return dfattn.lib().dfattn_fwd(q, k, v, o, lse, h, s, d, 0.125, 1, None)


@pytest.mark.parametrize("kwargs,status", [
    (dict(q=None), -1), (dict(o=None), -1), (dict(v=ODD), -2), (dict(lse=ODD), -2),
    (dict(h=0), -3), (dict(s=0), -3), (dict(d=0), -4), (dict(d=129), -4),
    (dict(h=1 << 21), -5), (dict(h=65536), -5), (dict(s=(1 << 30) + 1), -5),
])
def test_forward_validation(kwargs, status):
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    assert fwd(**kwargs) == status
    assert lib.dfattn_last_error() == status
    assert lib.dfattn_last_error_message()
    lib.dfattn_clear_error()
    assert lib.dfattn_last_error() == 0


def bwd(ws=FAKE, ws_bytes=None, h=12, s=1024, d=64, lse=FAKE, o=FAKE):
    lib = dfattn.lib()
    if ws_bytes is None:
        ws_bytes = lib.dfattn_bwd_workspace_bytes(h, s, d)
    return lib.dfattn_bwd(FAKE, FAKE, FAKE, o, FAKE, lse, FAKE, FAKE, FAKE, ws, ws_bytes, h, s, d, 0.125, 1, None)


def test_backward_validation():
    lib = dfattn.lib()
    need = lib.dfattn_bwd_workspace_bytes(12, 1024, 64)
    assert bwd(ws=None) == -6
    assert bwd(ws_bytes=need - 1) == -6
    assert bwd(ws=ODD) == -6
    assert bwd(lse=None) == -1
    assert bwd(o=None) == -1
    assert bwd(d=200) == -4
    assert bwd(s=0) == -3
    lib.dfattn_clear_error()


def test_backward_workspace_is_linear_in_seq_len():
    lib = dfattn.lib()
    # The per-64-row-block dO scales [H, ceil(S/64)], two fp32 row statistics [H, S], four fp16
    # copies [H, S, 64] (c2*Q, K, V, sigma*dO) and the fp16 rounding residues of rows 0-63 of
    # sigma*dO, c2*Q and K [H, 3, 64, 64], each rounded up to 256 bytes.
    up = lambda x: (x + 255) // 256 * 256
    for h, s in ((12, 1024), (12, 4096), (1, 5), (12, 131072)):
        want = up(h * ((s + 63) // 64) * 4) + 2 * up(h * s * 4) + 4 * up(h * s * 64 * 2) + up(h * 3 * 64 * 64 * 2)
        assert lib.dfattn_bwd_workspace_bytes(h, s, 64) == want
    assert lib.dfattn_bwd_workspace_bytes(0, 10, 64) == 0
    # O(H*S*D), against the reference's O(H*S^2) probability scratch (lib.rs:2023): 1/64 of it at S = 4096.
    assert lib.dfattn_bwd_workspace_bytes(12, 4096, 64) < 12 * 2 * 4096 * 4096 * 4 // 50


def test_legacy_launcher_records_error_instead_of_launching():
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    # d_head > 128 is a device trap in the reference (attention_fused.cu:56-58); here it is
    # recorded on the host and reported by darkforest_sync().
    lib.launch_fused_mha_forward(FAKE, FAKE, FAKE, FAKE, 12, 128, 129, 0.1, 1)
    assert lib.dfattn_last_error() == -4
    lib.dfattn_clear_error()
    lib.launch_fused_mha_backward(FAKE, None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 12, 128, 64, 0.1, 1)
    assert lib.dfattn_last_error() == -1
    lib.dfattn_clear_error()


def test_sync_aborts_for_a_recorded_launcher_error_before_any_hip_call():
    """darkforest_sync aborts with the reference's "[darkforest] ..." message for an argument error
    of a void launcher (matmul.cu:21-28). The launcher records the error on the host without
    launching, and darkforest_sync checks it before touching the device, so the child process that
    aborts here never initialises HIP (its GPUs are hidden as well)."""
    import subprocess
    import sys

    pkg = os.path.join(ROOT, "dark-forest_amd")
    launcher = ("import sys; sys.path.insert(0, %r); import ctypes, dfattn; lib = dfattn.lib(); "
                "f = ctypes.c_void_p(0x10000); lib.launch_fused_mha_forward(f, f, f, f, 12, 128, 129, 0.1, 1); "
                "lib.darkforest_sync(); print('survived')") % pkg
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    out = subprocess.run([sys.executable, "-c", launcher], capture_output=True, text=True, timeout=120, env=env)
    assert out.returncode != 0 and "survived" not in out.stdout
    assert "[darkforest] attention launch error" in out.stderr, out.stderr


def test_product_path_never_touches_the_oracle():
    """Only tests/, smoke() and bench.py's cpu_baseline may use oracle/."""
    pkg = os.path.join(ROOT, "dark-forest_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".hpp", ".cpp", ".rs", "Makefile")):
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert "oracle" not in text.lower(), f"{f} mentions the oracle"


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(dfattn, "_lib", None)
    monkeypatch.setattr(dfattn, "LIB_PATH", str(tmp_path / "libdfattn.so"))
    with pytest.raises(dfattn.DfattnNotBuilt):
        dfattn.lib()


ODD4 = ctypes.c_void_p(0x10004)  # 4-byte but not 16-byte aligned


def strided(fn, stride=3 * 768, h=12, s=1024, d=64, ptr=FAKE, ws=FAKE, ws_bytes=None, flags=1):
    """One of the three row-strided training calls on fake pointers (validation fails first)."""
    lib = dfattn.lib()
    if ws_bytes is None:
        ws_bytes = lib.dfattn_bwd_workspace_bytes(h, s, 64)
    if fn == "fwd":
        return lib.dfattn_fwd_train_strided(ptr, FAKE, FAKE, FAKE, FAKE, ws, ws_bytes, h, s, d, 0.125, 1, stride, None)
    if fn == "pre":
        return lib.dfattn_bwd_preprocess_strided(ptr, FAKE, FAKE, FAKE, FAKE, FAKE, ws, ws_bytes, h, s, d, 0.125,
                                                 flags, stride, None)
    return lib.dfattn_bwd_main_strided(FAKE, ptr, FAKE, FAKE, ws, ws_bytes, h, s, d, 0.125, 1, stride, None)


@pytest.mark.parametrize("fn", ["fwd", "pre", "main"])
@pytest.mark.parametrize("kwargs,status", [
    (dict(d=32), -4), (dict(d=128), -4), (dict(stride=767), -3), (dict(stride=770), -3),
    (dict(stride=(1 << 21) + 4), -3), (dict(stride=0), -3), (dict(ptr=ODD4), -2), (dict(ptr=None), -1),
    (dict(ws=None), -6), (dict(h=0), -3),
])
def test_strided_training_pair_validation(fn, kwargs, status):
    """Row strides below the row's n_heads*64 floats, not a multiple of 4 or above 2^21, a head size
    other than 64 and tensors that are not 16-byte aligned are refused before any HIP call."""
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    assert strided(fn, **kwargs) == status
    assert lib.dfattn_last_error() == status
    assert b"strided" in lib.dfattn_last_error_message() or status in (-1, -3, -6)
    lib.dfattn_clear_error()


def test_strided_preprocess_rejects_unknown_flags():
    assert strided("pre", flags=2) == -8
    dfattn.lib().dfattn_clear_error()


def test_strided_python_helpers_validate_layouts():
    """Column blocks of one [S, 3*H*D] tensor have one row stride; other layouts are refused."""
    import torch

    wide = torch.zeros(8, 3 * 128)
    assert [dfattn._row_stride(wide[:, i * 128:(i + 1) * 128]) for i in range(3)] == [384] * 3
    assert dfattn._row_stride(torch.zeros(8, 128)) is None
    assert dfattn._row_stride(wide[:1, :128]) is None  # one row is contiguous
    for bad in (wide[:, :128].t(), wide[:, ::2], torch.zeros(8, 128, dtype=torch.float64)):
        with pytest.raises(ValueError):
            dfattn._row_stride(bad)
    with pytest.raises(ValueError):
        dfattn._same_stride("q", wide[:, :128])  # a CPU tensor


# ---------------------------------------------------------------- the context mirror (lib.rs:1949-2368)
@pytest.mark.parametrize("dims,status", [
    ((12, 128, 0), -4), ((12, 128, 129), -4), ((0, 128, 64), -3), ((12, 0, 64), -3),
    ((2 ** 32 - 1, 2 ** 32 - 1, 128), -5), ((65536, 16, 64), -5),
])
def test_context_create_validates_like_new_shared(dims, status):
    """AttentionContext::new_shared's checks (lib.rs:1981-1989) run before any device allocation."""
    lib = dfattn.lib()
    handle = ctypes.c_void_p(0x1234)
    assert lib.dfattn_context_create(*dims, ctypes.byref(handle)) == status
    assert handle.value is None  # out-pointer cleared on failure
    assert lib.dfattn_last_error() == status


def test_context_create_rejects_null_out_pointer():
    assert dfattn.lib().dfattn_context_create(12, 128, 64, None) == -1


def test_null_context_calls_fail_cleanly():
    lib = dfattn.lib()
    assert lib.dfattn_context_forward_device_into(None, FAKE, FAKE, FAKE, 0.125, 1, FAKE, 10, None) == -1
    assert lib.dfattn_context_backward_device_into(None, FAKE, FAKE, FAKE, FAKE, 0.125, 1, FAKE, FAKE, FAKE, 10,
                                                   None) == -1
    assert lib.dfattn_context_forward_device_into_strided(None, FAKE, FAKE, FAKE, 0.125, 1, FAKE, 10, 2304,
                                                          None) == -1
    assert lib.dfattn_context_backward_device_into_strided(None, FAKE, FAKE, FAKE, FAKE, 0.125, 1, FAKE, FAKE,
                                                           FAKE, 10, 2304, 2304, None) == -1
    assert lib.dfattn_context_lse(None) is None
    lib.dfattn_context_destroy(None)  # no-op


def test_host_helpers_reject_bad_shapes_before_allocating():
    """fused_attention_forward / attention_backward (lib.rs:2371-2479) shape errors."""
    import numpy as np

    with pytest.raises(dfattn.DfattnError) as e:
        dfattn.fused_attention_forward(np.zeros(10), np.zeros(10), np.zeros(10), 5, 3, 0.5, True)
    assert e.value.status == -3
    lib = dfattn.lib()
    buf = (ctypes.c_float * 16)()
    assert lib.dfattn_fused_attention_forward(buf, buf, buf, 15, 4, 4, 0.5, 1, buf) == -3
    assert lib.dfattn_fused_attention_forward(buf, buf, buf, 16, 4, 0, 0.5, 1, buf) == -4
    assert lib.dfattn_attention_backward(buf, buf, buf, buf, 15, 4, 4, 0.5, 1, buf, buf, buf) == -3
    assert b"[seq_len, d_head]" in lib.dfattn_last_error_message()


def test_context_error_is_returned_and_recorded_in_a_fresh_process():
    """A context error comes back as a status and is readable through dfattn_last_error."""
    import subprocess
    import sys

    code = ("import sys; sys.path.insert(0, %r); import ctypes, dfattn; lib = dfattn.lib(); "
            "h = ctypes.c_void_p(); assert lib.dfattn_context_create(12, 128, 0, ctypes.byref(h)) == -4; "
            "assert lib.dfattn_last_error() == -4; print('ok')") % os.path.join(ROOT, "dark-forest_amd")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "ok" in out.stdout, out.stderr


# ---------------------------------------------------------------- decode (attention_fused.cu:551-1090)
def dec(q=FAKE, k=FAKE, v=FAKE, table=None, page=1, kvt=0, out=FAKE, lse=None, h=12, n=100, d=64, ws=None,
        wsb=0):
    return dfattn.lib().dfattn_decode(q, k, v, table, page, kvt, out, lse, h, n, d, 0.125, ws, wsb, None)


@pytest.mark.parametrize("kwargs,status", [
    (dict(kvt=2), -8), (dict(d=0), -4), (dict(d=129), -4), (dict(h=0), -3), (dict(h=65536), -5),
    (dict(q=None), -1), (dict(out=None), -1), (dict(k=ODD), -2), (dict(table=FAKE, page=0), -3),
    (dict(ws=FAKE, wsb=8, n=4096), -6),
])
def test_decode_validation(kwargs, status):
    """Every case fails on the host before any launch (the pointers are fake)."""
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    assert dec(**kwargs) == status
    assert lib.dfattn_last_error() == status
    lib.dfattn_clear_error()


def test_decode_empty_cache_is_a_no_op():
    # cur_seq_len 0: nothing to compute, nothing launched (the reference's kernels return early).
    assert dec(n=0) == 0


def test_decode_workspace_formula():
    lib = dfattn.lib()
    # chunks = min(ceil(L/512), ceil(512/H)), 1 up to L = 1024; one chunk needs no workspace; else
    # H*chunks*(D+2) floats
    assert lib.dfattn_decode_workspace_bytes(12, 1024, 64) == 0
    assert lib.dfattn_decode_workspace_bytes(12, 4096, 64) == 12 * 8 * 66 * 4
    assert lib.dfattn_decode_workspace_bytes(12, 131072, 64) == 12 * 43 * 66 * 4
    assert lib.dfattn_decode_workspace_bytes(0, 100, 64) == 0


def test_legacy_decode_split_with_zero_chunk_is_recorded():
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    # the reference divides by chunk_size (attention_fused.cu:786); here it is an argument error
    lib.launch_fused_mha_decode_kv_splitk(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 12, 100, 64, 0.1, 0)
    assert lib.dfattn_last_error() == -3
    lib.dfattn_clear_error()
    lib.launch_paged_mha_decode_kv(FAKE, FAKE, FAKE, FAKE, FAKE, 12, 100, 64, 0.1, 0)
    assert lib.dfattn_last_error() == -3
    lib.dfattn_clear_error()


@pytest.mark.parametrize("call,status", [
    (lambda l: l.launch_pos_embed_interpolate(None, FAKE, 0, 10, 10, 64), -1),
    (lambda l: l.launch_pos_embed_interpolate(FAKE, FAKE, 3, 0, 10, 64), -3),   # the reference reads row 2^32-1
    (lambda l: l.launch_apply_rope(None, 1, 12, 64, 1e4), -1),
    (lambda l: l.launch_apply_rope(FAKE, 1, 0, 64, 1e4), -3),                   # grid 0: invalid launch there
    (lambda l: l.launch_apply_rope(FAKE, 1, 12, 1, 1e4), -4),                   # block 0: invalid launch there
    (lambda l: l.launch_apply_rope(FAKE, 1, 65536, 65537, 1e4), -5),
    (lambda l: l.launch_paged_copy_row(FAKE, None, 0, 0, 16, 768), -1),
    (lambda l: l.launch_paged_copy_row(FAKE, FAKE, -1, 0, 16, 768), -3),
    (lambda l: l.launch_paged_copy_row(FAKE, FAKE, 2, 16, 16, 768), -3),        # offset outside its page
    (lambda l: l.launch_paged_copy_row_f32_to_bf16(FAKE, ctypes.c_void_p(0x10001), 0, 0, 16, 768), -2),
    (lambda l: l.launch_paged_copy_row_f32_to_bf16(FAKE, FAKE, 0, 3, 2, 768), -3),
])
def test_elementwise_launchers_record_argument_errors(call, status):
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    call(lib)
    assert lib.dfattn_last_error() == status
    lib.dfattn_clear_error()


def test_elementwise_launchers_with_nothing_to_do_launch_nothing():
    lib = dfattn.lib()
    lib.dfattn_clear_error()
    lib.launch_pos_embed_interpolate(FAKE, FAKE, 3, 10, 10, 0)
    lib.launch_paged_copy_row(FAKE, FAKE, 0, 0, 16, 0)
    lib.launch_paged_copy_row_f32_to_bf16(FAKE, FAKE, 0, 0, 16, 0)
    assert lib.dfattn_last_error() == 0
