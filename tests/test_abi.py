"""The C-ABI library loads, exports what include/pocr_hip.h declares, and
rejects bad input before touching a device.  No GPU needed."""
import ctypes as C
import os

import numpy as np
import pytest

from rapidocrvl_amd import lib


def test_library_exports_every_header_symbol():
    L = lib.load()
    names = lib.header_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert set(names) == set(lib._SIGS), "ctypes signatures out of sync with the header"


def test_abi_version():
    assert lib.load().pocr_abi_version() == 1


def test_null_arguments_are_arg_errors():
    L = lib.load()
    assert L.pocr_matvec(None, None, None, 1, None) == lib.POCR_ERR_ARG
    assert L.pocr_step(None, None, None, 1, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_quantize_rows(7, 0, None, 1, 1, None, None) == lib.POCR_ERR_ARG
    assert b"pocr_step" in L.pocr_last_error()
    assert L.pocr_matvec_topk(None, None, None, 4, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_sample_topk(None, None, 8, 4, 1.0, None, None, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_sample_full(None, None, 8, 1.0, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_seq_set_sampling(None, 1.0, 4, 0) == lib.POCR_ERR_ARG
    assert L.pocr_gguf_open(None, None) == lib.POCR_ERR_ARG
    assert L.pocr_gguf_tensor_count(None) == lib.POCR_ERR_ARG
    assert L.pocr_gguf_find(None, b"x") == lib.POCR_ERR_ARG
    assert L.pocr_gguf_tensor_info(None, 0, None, None, None, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_gguf_read(None, 0, None, 4) == lib.POCR_ERR_ARG
    assert L.pocr_gguf_meta(None, 0, None, None, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_model_load_gguf(None, None, b"x", None) == lib.POCR_ERR_ARG
    # the fused sublayer mirrors and the allocation-free attention
    assert L.pocr_swiglu_down(None, None, None, None, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_swiglu_down_add_rmsnorm(None, None, None, None, None, None, None, 1e-5, 1, None) == lib.POCR_ERR_ARG
    assert L.pocr_add_rmsnorm(None, None, None, None, 4, 1e-5, 1, None) == lib.POCR_ERR_ARG
    assert L.pocr_mrope(None, None, None, None, 2, 128) == lib.POCR_ERR_ARG
    assert L.pocr_text_attention_out(None, None, None, None, 1, 16, 2, 128, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_text_attention_out_add_rmsnorm(None, None, None, None, 1, 16, 2, 128, None, None, None, 1e-5, 1,
                                                 None) == lib.POCR_ERR_ARG
    assert L.pocr_first_token_value_out_add_rmsnorm(None, None, None, 16, 2, 128, None, None, None, 1e-5, 1,
                                                    None) == lib.POCR_ERR_ARG
    assert L.pocr_text_attention_noalloc(None, None, None, None, 1, 16, 2, 128, None) == lib.POCR_ERR_ARG
    L.pocr_gguf_close(None)
    assert L.pocr_batch_create(None, None) == lib.POCR_ERR_ARG
    assert L.pocr_batch_join(None, None, 0, 0, 1, None, 0) == lib.POCR_ERR_ARG
    assert L.pocr_batch_step(None, 1) == lib.POCR_ERR_ARG
    assert L.pocr_batch_poll(None, None, None) == lib.POCR_ERR_ARG
    assert L.pocr_batch_leave(None, None, None, 0) == lib.POCR_ERR_ARG
    L.pocr_batch_destroy(None)


def test_fault_injection_is_reported_before_device_work(monkeypatch):
    monkeypatch.setenv("POCR_HIP_FAIL_OP", "ctx")
    h = C.c_void_p()
    rc = lib.load().pocr_ctx_create(0, C.byref(h))
    assert rc == lib.POCR_ERR_INJECTED
    assert b"injected" in lib.load().pocr_last_error()


@pytest.mark.skipif(lib.device_count() > 0, reason="a device is visible")
def test_no_device_is_a_device_error():
    h = C.c_void_p()
    assert lib.load().pocr_ctx_create(0, C.byref(h)) == lib.POCR_ERR_DEVICE


def test_positions_reject_grid_larger_than_placeholders():
    with pytest.raises(lib.PocrError):
        lib.mm_positions([1, 7, 7, 2], 7, (1, 4, 4))


def test_every_entry_point_rejects_null_arguments():
    # null handles and pointers, zero sizes: every status-returning entry point
    # answers POCR_ERR_ARG before touching a device; destroy/free calls accept null
    L = lib.load()
    plain = {"pocr_abi_version", "pocr_last_error", "pocr_device_count", "pocr_row_bytes"}
    for name, (res, args) in sorted(lib._SIGS.items()):
        if name in plain:
            continue
        vals = [0 if a in (C.c_int, C.c_int32, C.c_int64, C.c_uint64, C.c_uint32, C.c_size_t)
                else 0.0 if a in (C.c_float, C.c_double) else None for a in args]
        r = getattr(L, name)(*vals)
        if res is None:
            assert r is None, name
        else:
            assert r == lib.POCR_ERR_ARG, (name, r)
