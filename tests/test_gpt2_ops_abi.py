"""The GPT-2 step ops' C ABI (include/dfgpt2.h) on the CPU: every declared symbol is exported and
typed, and bad arguments are rejected on the host before any HIP call (no GPU needed)."""
import ctypes
import os

import pytest

import dfattn
from conftest import ROOT
from dfattn import ops
from test_abi import declared_functions

HEADER = os.path.join(ROOT, "include", "dfgpt2.h")
# dfattn_status codes (include/dfattn.h)
OK, ERR_NULL, ERR_MISALIGNED, ERR_SHAPE, ERR_OVERFLOW, ERR_WORKSPACE = dfattn.DFATTN_OK, -1, -2, -3, -5, -6


def test_every_declared_symbol_is_exported_and_typed():
    lib = ops.ops_lib()
    declared = declared_functions(HEADER)
    assert "launch_layernorm" in declared and "dfgpt2_adamw_update" in declared
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in dfgpt2.h but not exported"
    assert sorted(ops.SYMBOLS) == declared


def _status(fn, *args):
    return getattr(ops.ops_lib(), fn)(*args)


BUF = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first
ODD = ctypes.c_void_p(0x1002)


@pytest.mark.parametrize("fn,args,status", [
    ("dfgpt2_layernorm_forward", (None, None, None, BUF, None, None, 4, 8, None), ERR_NULL),
    ("dfgpt2_layernorm_forward", (ODD, None, None, BUF, None, None, 4, 8, None), ERR_MISALIGNED),
    ("dfgpt2_layernorm_forward", (BUF, ODD, None, BUF, None, None, 4, 8, None), ERR_MISALIGNED),
    ("dfgpt2_layernorm_forward", (BUF, None, None, BUF, None, None, 4, 0, None), ERR_SHAPE),
    ("dfgpt2_layernorm_forward", (BUF, None, None, BUF, None, None, 2**31, 8, None), ERR_OVERFLOW),
    ("dfgpt2_layernorm_forward", (BUF, None, None, BUF, None, None, 0, 8, None), OK),
    ("dfgpt2_layernorm_backward", (BUF, BUF, None, None, BUF, BUF, None, None, 4, 8, None),
     ERR_NULL),
    ("dfgpt2_layernorm_backward", (BUF, BUF, None, BUF, BUF, BUF, ODD, None, 4, 8, None),
     ERR_MISALIGNED),
    ("dfgpt2_gelu_forward", (BUF, None, 16, None), ERR_NULL),
    ("dfgpt2_gelu_forward", (BUF, BUF, 0, None), OK),
    ("dfgpt2_gelu_forward", (None, None, 0, None), OK),
    ("dfgpt2_layernorm_backward", (None,) * 8 + (0, 8, None), OK),
    ("dfgpt2_gelu_backward", (BUF, ODD, BUF, 16, None), ERR_MISALIGNED),
    ("dfgpt2_linear_grad_bias", (BUF, None, 4, 8, 0, None), ERR_NULL),
    ("dfgpt2_linear_grad_bias", (BUF, BUF, 4, 0, 0, None), ERR_SHAPE),
    ("dfgpt2_adamw_update", (BUF, BUF, BUF, BUF, 16, 1e-3, 0.9, 0.95, 1e-8, 0.1, None, None),
     ERR_NULL),
    ("dfgpt2_logit_ce_chunk", (BUF, None, BUF, BUF, 4, 100, 4, None), ERR_NULL),
    ("dfgpt2_logit_ce_chunk", (BUF, BUF, ODD, BUF, 4, 100, 4, None), ERR_MISALIGNED),
    ("dfgpt2_logit_ce_chunk", (BUF, BUF, BUF, BUF, 4, 0, 4, None), ERR_SHAPE),
    ("dfgpt2_logit_ce_chunk", (BUF, BUF, BUF, BUF, 4, 100, 0, None), ERR_SHAPE),
    ("dfgpt2_logit_ce_chunk", (BUF, BUF, BUF, BUF, 2**31, 100, 4, None), ERR_OVERFLOW),
    ("dfgpt2_logit_ce_chunk", (None, None, None, None, 0, 100, 4, None), OK),
    ("dfgpt2_sum", (None, 4, BUF, 0, None), ERR_NULL),
    ("dfgpt2_sum", (BUF, 4, None, 0, None), ERR_NULL),
    ("dfgpt2_embedding_forward", (BUF, None, BUF, 4, 8, 10, None), ERR_NULL),
    ("dfgpt2_embedding_forward", (BUF, BUF, BUF, 4, 0, 10, None), ERR_SHAPE),
    ("dfgpt2_embedding_forward", (None, None, None, 0, 8, 10, None), OK),
    ("dfgpt2_embedding_backward", (BUF, BUF, ODD, 4, 8, 10, None), ERR_MISALIGNED),
    ("dfgpt2_embedding_backward", (BUF, BUF, BUF, 2**31, 8, 10, None), ERR_OVERFLOW),
    ("dfgpt2_add_layernorm_forward", (BUF, None, None, None, BUF, BUF, None, None, 4, 8, None), ERR_NULL),
    ("dfgpt2_add_layernorm_forward", (BUF, BUF, None, None, ODD, BUF, None, None, 4, 8, None), ERR_MISALIGNED),
    ("dfgpt2_add_layernorm_forward", (BUF, BUF, None, None, BUF, BUF, None, None, 4, 0, None), ERR_SHAPE),
    ("dfgpt2_add_layernorm_forward", (None,) * 8 + (0, 8, None), OK),
    ("dfgpt2_layernorm_backward_residual", (BUF, BUF, None, BUF, BUF, None, None, None, None, 4, 8, None),
     ERR_NULL),
    ("dfgpt2_layernorm_backward_residual", (BUF, BUF, None, BUF, BUF, ODD, BUF, None, None, 4, 8, None),
     ERR_MISALIGNED),
    ("dfgpt2_layernorm_backward_residual", (None,) * 9 + (0, 8, None), OK),
    ("dfgpt2_bias_gelu_forward", (BUF, None, BUF, 4, 8, None), ERR_NULL),
    ("dfgpt2_bias_gelu_forward", (BUF, BUF, BUF, 4, 0, None), ERR_SHAPE),
    ("dfgpt2_bias_gelu_forward", (BUF, BUF, BUF, 2**31, 8, None), ERR_OVERFLOW),
    ("dfgpt2_bias_gelu_forward", (None, None, None, 0, 8, None), OK),
    ("dfgpt2_add_bias", (BUF, None, BUF, 4, 8, None), ERR_NULL),
    ("dfgpt2_add_bias", (BUF, BUF, ODD, 4, 8, None), ERR_MISALIGNED),
    ("dfgpt2_add_bias", (BUF, BUF, BUF, 4, 0, None), ERR_SHAPE),
    ("dfgpt2_add_bias", (BUF, BUF, BUF, 2**31, 8, None), ERR_OVERFLOW),
    ("dfgpt2_add_bias", (None, None, None, 0, 8, None), OK),
    # fused LayerNorm backward: (grad_out, x, gamma, means, rstds, residual, grad_x, grad_gamma,
    # grad_beta, grad_bias, workspace, workspace_bytes, batch, features, stream)
    ("dfgpt2_layernorm_backward_fused", (BUF, BUF, None, BUF, BUF, None, None, BUF, None, None, BUF, 1 << 20, 4, 8,
                                         None), ERR_NULL),
    ("dfgpt2_layernorm_backward_fused", (BUF, BUF, None, BUF, BUF, ODD, BUF, BUF, None, None, BUF, 1 << 20, 4, 8,
                                         None), ERR_MISALIGNED),
    ("dfgpt2_layernorm_backward_fused", (BUF, BUF, None, BUF, BUF, None, BUF, BUF, None, None, BUF, 1 << 20, 4, 0,
                                         None), ERR_SHAPE),
    ("dfgpt2_layernorm_backward_fused", (BUF, BUF, None, BUF, BUF, None, BUF, BUF, None, None, None, 1 << 20, 4, 8,
                                         None), ERR_WORKSPACE),
    ("dfgpt2_layernorm_backward_fused", (BUF, BUF, None, BUF, BUF, None, BUF, BUF, BUF, None, BUF, 63, 4, 8, None),
     ERR_WORKSPACE),  # two planes of 8 sums for one workgroup need 64 bytes
    ("dfgpt2_layernorm_backward_fused", (BUF, BUF, None, BUF, BUF, None, BUF, None, None, BUF, BUF, 95, 4, 8, None),
     ERR_WORKSPACE),  # with the bias plane, 96
    ("dfgpt2_layernorm_backward_fused", (None,) * 10 + (None, 0, 0, 8, None), OK),
])
def test_argument_errors_are_caught_on_the_host(fn, args, status):
    ops.ops_lib().dfattn_clear_error()
    assert _status(fn, *args) == status
    if status != OK:
        assert ops.ops_lib().dfattn_last_error() == status
    ops.ops_lib().dfattn_clear_error()


def test_fused_layernorm_backward_workspace_formula():
    """Per workgroup of four rows, three planes (gamma, beta and bias terms) of features floats."""
    lib = ops.ops_lib()
    for rows, f in ((1024, 768), (1, 8), (5, 100), (4, 8)):
        assert lib.dfgpt2_layernorm_backward_fused_workspace_bytes(rows, f) == (rows + 3) // 4 * 3 * f * 4
    assert lib.dfgpt2_layernorm_backward_fused_workspace_bytes(0, 768) == 0


def test_reference_launcher_records_error_for_darkforest_sync():
    """The reference symbols return void: an argument error is kept for darkforest_sync (which
    aborts on it, in a subprocess in test_abi) and nothing is launched."""
    lib = ops.ops_lib()
    lib.dfattn_clear_error()
    lib.launch_layernorm(None, None, None, None, None, None, 4, 8)
    assert lib.dfattn_last_error() == ERR_NULL
    assert "dfgpt2_layernorm_forward" in lib.dfattn_last_error_message().decode()
    lib.dfattn_clear_error()
    lib.launch_adamw_update(None, BUF, BUF, BUF, 16, 1e-3, 0.9, 0.95, 1e-8, 0.1, 0.1, 0.05)
    assert lib.dfattn_last_error() == ERR_NULL
    lib.dfattn_clear_error()
    lib.launch_fused_chunked_logit_ce(BUF, BUF, BUF, None, 4, 100, 4)
    assert lib.dfattn_last_error() == ERR_NULL
    lib.dfattn_clear_error()
    lib.launch_embedding_backward(BUF, None, BUF, 4, 8)
    assert lib.dfattn_last_error() == ERR_NULL
    assert "dfgpt2_embedding_backward" in lib.dfattn_last_error_message().decode()
    lib.dfattn_clear_error()
    for call, name in ((lambda: lib.launch_add_bias(BUF, None, BUF, 4, 8), "dfgpt2_add_bias"),
                       (lambda: lib.launch_add(BUF, None, BUF, 16), "launch_add"),
                       (lambda: lib.launch_scale(None, 2.0, BUF, 16), "launch_scale"),
                       (lambda: lib.launch_fill(None, 1.0, 16), "launch_fill")):
        call()
        assert lib.dfattn_last_error() == ERR_NULL
        assert name in lib.dfattn_last_error_message().decode()
        lib.dfattn_clear_error()
    lib.launch_add(ODD, BUF, BUF, 16)
    assert lib.dfattn_last_error() == ERR_MISALIGNED
    lib.dfattn_clear_error()
    for call in (lambda: lib.launch_add(None, None, None, 0), lambda: lib.launch_scale(None, 2.0, None, 0),
                 lambda: lib.launch_fill(None, 1.0, 0), lambda: lib.launch_add_bias(None, None, None, 0, 8)):
        call()  # nothing to do: no error, nothing launched
        assert lib.dfattn_last_error() == OK
