"""CPU checks of the C ABI: libstx.so loads, exports every function include/*.h declares, and
the Python binding covers them. Only calls that fail before touching a GPU are made here."""
import ctypes
import glob
import os
import re

import pytest

import stx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        names += re.findall(r"STX_API\s+[\w\s\*]+?\b(stx_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_functions():
    assert len(declared_functions()) >= 12


@pytest.mark.parametrize("name", declared_functions())
def test_symbol_exported_and_bound(name):
    L = stx.lib()
    assert hasattr(L, name), f"{name} not exported by libstx.so"
    assert name in stx._SIGNATURES, f"{name} has no ctypes signature in stx.py"


def test_version_and_error():
    assert stx.lib().stx_version().decode().count(".") == 2
    assert stx.lib().stx_last_error() is not None


@pytest.mark.parametrize("n,status", [(12, stx.STATUS_INVALID_ARGUMENT), (0, stx.STATUS_INVALID_ARGUMENT),
                                      (4, stx.STATUS_UNSUPPORTED), (16384, stx.STATUS_UNSUPPORTED)])
def test_fft_create_rejects(n, status):
    h = ctypes.c_void_p()
    assert stx.lib().stx_fft_create(n, ctypes.byref(h)) == status
    assert not h.value
    assert stx.lib().stx_last_error().decode() != ""


def test_fft_create_null_out():
    assert stx.lib().stx_fft_create(2048, None) == stx.STATUS_INVALID_ARGUMENT


def test_frame_counts():
    assert stx.torch_stft_frames(352800, 441) == 801
    assert stx.htdemucs_frames(4096, 343980) == 336
    assert stx.torch_stft_frames(343980, 1024) == 336


def test_null_plan_is_invalid_argument():
    rc = stx.lib().stx_torch_stft(None, None, 1, 4096, 1024, 0, None, 0, None)
    assert rc == stx.STATUS_INVALID_ARGUMENT
