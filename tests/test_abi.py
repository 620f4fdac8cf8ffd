"""The C ABI library on a host without a GPU: it loads, exports every entry
point that include/trit_hip.h declares, and fails cleanly (an error code and
a message, no crash) when no device is there."""

import ctypes as C
import os
import re

import pytest

from trit_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "trit_hip.h")).read()
    return sorted(set(re.findall(r"\b(trit_hip_\w+)\s*\(", text)))


def test_header_names_the_seam():
    names = declared()
    for must in ["trit_hip_layer_q8_0", "trit_hip_layer_forward", "trit_hip_decoder_new",
                 "trit_hip_session_generate", "trit_hip_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(hip.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_clean_failure_without_device():
    lib = hip.lib()
    assert lib.trit_hip_version().startswith(b"trit_hip")
    try:
        import torch

        has_gpu = torch.cuda.device_count() > 0
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is visible")
    assert lib.trit_hip_init(0) == -1
    assert lib.trit_hip_last_error() != b""


def test_null_arguments_are_errors():
    lib = hip.lib()
    out = C.c_void_p()
    assert lib.trit_hip_layer_q8_0(32, 32, None, None, C.byref(out)) == -1
    assert b"NULL" in lib.trit_hip_last_error()
    assert lib.trit_hip_decoder_new(None, None, None, None, None, C.byref(out)) == -1
    assert lib.trit_hip_session_prefill(None, None, 0, None) == -1
