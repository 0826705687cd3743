"""The C ABI library on the CPU: it loads, exports every entry point that
include/q3h.h declares, and its host-only paths (errors, the host quantizer)
behave without a GPU."""
import ctypes
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    with open(os.path.join(ROOT, "include", "q3h.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q3h_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol(q3h):
    names = declared()
    assert len(names) >= 24
    L = q3h.lib()
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(q3h.SIGNATURES), set(names) ^ set(q3h.SIGNATURES)


def test_device_open_without_gpu_fails_cleanly(q3h):
    if q3h.available():
        return  # a machine with a GPU: covered by the gpu tests
    h = ctypes.c_void_p()
    rc = q3h.lib().q3h_device_open(0, ctypes.byref(h))
    assert rc == q3h.E_NODEV
    assert q3h.lib().q3h_last_error()
    assert not h.value


def test_null_arguments_are_errors(q3h):
    L = q3h.lib()
    assert L.q3h_stack_create(None, None, None, None) == q3h.E_ARG
    assert b"NULL" in L.q3h_last_error()
    assert L.q3h_context_length(None) == q3h.E_ARG
    assert L.q3h_context_reset(None) == q3h.E_ARG
    assert L.q3h_forward_embeds(None, None, 1, -1, None, None) == q3h.E_ARG
    assert L.q3h_frame_step(None, None, None) == q3h.E_ARG
    assert L.q3h_device_close(None) == q3h.E_ARG
    assert L.q3h_device_name(None) is None
    assert L.q3h_text_create(None, None, None, None, None, None, None, None) == q3h.E_ARG
    assert L.q3h_text_project(None, None, 1, None) == q3h.E_ARG
    assert L.q3h_text_destroy(None) == 0
    assert L.q3h_frame_start_text(None, 0, None, None, None, 9, None, 5, 0) == q3h.E_ARG


def test_quantizer_rejects_ragged_rows(q3h):
    x = np.zeros(33, np.float32)
    out = np.zeros(64, np.uint8)
    rc = q3h.lib().q3h_quantize_row_q8_0(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                         out.ctypes.data_as(ctypes.c_void_p), 33)
    assert rc == q3h.E_ARG
    # the last error is per call: a good call clears it
    assert q3h.lib().q3h_quantize_row_q8_0(
        x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
        out.ctypes.data_as(ctypes.c_void_p), 32) == 0
    assert q3h.lib().q3h_last_error() == b""
