"""GPU: zero-sized calls are no-ops, through the C ABI.

The reference's loops run zero times on empty inputs (rows, tokens, heads or
elements = 0); every entry point must then return 0 and leave every buffer as
it was (all pointers here name one guarded device buffer).
"""
import ctypes

import pytest

pytestmark = pytest.mark.gpu

F64, BF16, F16, F32 = 0, 1, 2, 3


@pytest.fixture()
def guard():
    import torch
    g = torch.arange(4096, dtype=torch.int32, device="cuda:0")
    yield g
    torch.cuda.synchronize()
    assert torch.equal(g, torch.arange(4096, dtype=torch.int32, device="cuda:0")), "a zero-sized call wrote memory"


def test_zero_sized_calls(prims, guard):
    L, h = prims.lib, prims.h
    p = ctypes.c_void_p(guard.data_ptr())
    calls = {
        "mg_rmsnorm_rows": lambda: L.mg_rmsnorm_rows(h, 1, p, 64, p, 1e-6, p, 64, 0, 64, BF16),
        "mg_residual_rmsnorm": lambda: L.mg_residual_rmsnorm(h, 0, p, 0, p, 0, p, 1e-6, p, 0, 0, 64, BF16),
        "mg_residual_rmsnorm_f64_compat": lambda: L.mg_residual_rmsnorm(h, 0, p, 0, p, 0, p, 1e-6, p, 0, 0, 64,
                                                                         0x100),
        "mg_residual_add": lambda: L.mg_residual_add(h, p, p, 0, BF16),
        "mg_swiglu": lambda: L.mg_swiglu(h, p, p, p, 0, BF16),
        "mg_sigmoid_gate": lambda: L.mg_sigmoid_gate(h, p, p, p, 0, F16),
        "mg_scale": lambda: L.mg_scale(h, p, 0, 3.87, BF16),
        "mg_softcap": lambda: L.mg_softcap(h, p, 0, 0.5, 30.0, F32),
        "mg_rope": lambda: L.mg_rope(h, p, 4, 0, p, 1, 0, 0, 64, p, p, 8, None, 0, BF16),
        "mg_qk_norm_rope": lambda: L.mg_qk_norm_rope(h, p, 4, 0, p, 1, 0, 0, 64, 1e-6, 3.87, p, p, 8, None, 0,
                                                     p, 0, p, p, 8, BF16),
        "mg_softmax_rows_heads": lambda: L.mg_softmax_rows(h, p, 0, p, 0, 0, 4, 64, 0.1, 1, 0, 0, 0.0, F32, BF16),
        "mg_softmax_rows_q": lambda: L.mg_softmax_rows(h, p, 0, p, 0, 4, 0, 64, 0.1, 1, 0, 0, 0.0, F32, BF16),
        "mg_softmax_rows_k": lambda: L.mg_softmax_rows(h, p, 0, p, 0, 4, 4, 0, 0.1, 0, 0, 0, 0.0, F64, F64),
        "mg_dequant_q8_0": lambda: L.mg_dequant_q8_0(h, p, p, p, 0, 64, BF16),
        "mg_quantize_q8_0": lambda: L.mg_quantize_q8_0(h, p, 0, 64, p, p),
        "mg_gemv_q8_0": lambda: L.mg_gemv_q8_0(h, p, p, p, 1, 0, 64, 0, p, 0, 0),
        "mg_vocab_reduce": lambda: L.mg_vocab_reduce(h, p, 0, 0, 100, F32, 4, p, p, p, p),
        "mg_vocab_reduce_tail": lambda: L.mg_vocab_reduce_tail(h, p, 0, 0, 100, F32, 1.0, 30.0, 4, p, p, p, p, p),
        "mg_sample_dist": lambda: L.mg_sample_dist(h, p, p, p, p, 0, 4, 1.0, 0.9, 0.0, p, p, p),
        "mg_sample_rows": lambda: L.mg_sample_rows(h, p, 0, 0, 100, p, 0, 1.0, 0.9, 0.0, p, p, p),
        "mg_attn_prefill": lambda: L.mg_attn_prefill(h, p, 0, p, p, 0, 8, 2, 128, 16, 0, 0, 0.1, p, 0),
    }
    failed = {}
    for name, call in calls.items():
        if call() != 0:
            failed[name] = L.mg_last_error().decode()
    prims.sync()
    assert not failed, failed


def test_zero_positions_table_is_an_error(prims, guard):
    """a RoPE table of no rows has no reference counterpart (build_rope_table(c, T) with T >= 1)"""
    L, h = prims.lib, prims.h
    p = ctypes.c_void_p(guard.data_ptr())
    assert L.mg_rope_table(h, 1e6, 64, 0, BF16, p, p) == -1
    assert b"positions" in L.mg_last_error()
