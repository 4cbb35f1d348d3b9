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
                                      (1, stx.STATUS_INVALID_ARGUMENT), (1 << 25, stx.STATUS_UNSUPPORTED)])
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


def _desc(ne, addr=0x10000):
    """A dense stx_tensor descriptor at a fake address (never dereferenced: every call below is
    rejected by its argument checks before any device work)."""
    d = stx.Tensor()
    d.data = addr
    nb = 4
    for i in range(4):
        d.ne[i] = ne[i]
        d.nb[i] = nb
        nb *= ne[i]
    return d


def test_layout_argument_checks():
    L = stx.lib()
    a = _desc([4, 5, 6, 1])
    d = _desc([5, 4, 6, 1], 0x900000)
    bad_axes = L.stx_cont_permute(ctypes.byref(a), 0, 0, 1, 2, ctypes.byref(d), None)
    assert bad_axes == stx.STATUS_INVALID_ARGUMENT
    wrong_shape = L.stx_cont_permute(ctypes.byref(a), 0, 2, 1, 3, ctypes.byref(d), None)
    assert wrong_shape == stx.STATUS_INVALID_ARGUMENT
    same = _desc([4, 5, 6, 1])
    overlap = L.stx_cont_permute(ctypes.byref(a), 0, 1, 2, 3, ctypes.byref(same), None)
    assert overlap == stx.STATUS_INVALID_ARGUMENT and b"overlap" in L.stx_last_error()
    assert L.stx_cont_permute(None, 0, 1, 2, 3, ctypes.byref(d), None) == stx.STATUS_INVALID_ARGUMENT
    # dim_head 48 is not built; q/k/vt shapes are checked first.
    qkv = _desc([3 * 2 * 48, 5, 2, 1])
    q = _desc([48, 5, 2, 2], 0x1000000)
    k = _desc([48, 5, 2, 2], 0x2000000)
    vt = _desc([5, 48, 2, 2], 0x3000000)
    rc = L.stx_qkv_rope_split(ctypes.byref(qkv), ctypes.c_void_p(0x4000000), 2, 1e4, 1.0, 1.0, ctypes.byref(q),
                              ctypes.byref(k), ctypes.byref(vt), None)
    assert rc == stx.STATUS_UNSUPPORTED
    vt_bad = _desc([48, 5, 2, 2], 0x3000000)
    rc = L.stx_qkv_rope_split(ctypes.byref(qkv), ctypes.c_void_p(0x4000000), 2, 1e4, 1.0, 1.0, ctypes.byref(q),
                              ctypes.byref(k), ctypes.byref(vt_bad), None)
    assert rc == stx.STATUS_INVALID_ARGUMENT
    # concat: extents along dim must add up; other dims must match.
    s0, s1 = _desc([4, 2, 3, 1]), _desc([4, 5, 3, 1], 0x20000)
    arr = (ctypes.c_void_p * 2)(ctypes.addressof(s0), ctypes.addressof(s1))
    dst = _desc([4, 6, 3, 1], 0x800000)
    assert L.stx_concat(arr, 2, 1, ctypes.byref(dst), None) == stx.STATUS_INVALID_ARGUMENT
    assert L.stx_concat(arr, 2, 4, ctypes.byref(dst), None) == stx.STATUS_INVALID_ARGUMENT
    assert L.stx_concat(arr, 0, 1, ctypes.byref(dst), None) == stx.STATUS_INVALID_ARGUMENT
    gates = _desc([2, 6, 5, 1], 0x30000)
    o = _desc([4, 5, 6, 1])
    md = _desc([4, 6, 5, 1], 0x900000)
    assert L.stx_merge_heads(ctypes.byref(o), ctypes.byref(gates), ctypes.byref(md), None) == \
        stx.STATUS_INVALID_ARGUMENT


def test_versioned_table_from_c(tmp_path):
    """tests/cpp/abi_check.c, pure C: dlopen libstx.so, resolve only stx_get_api for the calls,
    check the V1 table (every entry is the exported function of its name), NULL for other
    versions, the size-tagged structs' frozen minimums and a few host-only calls through the
    table (src/libstems_v1.h:146-189 and tests/abi_test.c:63-101 are the model)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / "abi_check"
    subprocess.run([gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "abi_check.c"), "-o", str(exe), "-ldl"], check=True)
    r = subprocess.run([str(exe), os.path.abspath(stx.LIB_PATH)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all ok" in r.stdout


def test_table_lists_every_entry_point_in_header_order():
    """The stx_api_v1 members are the declared entry points (minus stx_get_api), in header order."""
    text = open(os.path.join(ROOT, "include", "stx.h")).read()
    head, table = text.split("typedef struct stx_api_v1 {", 1)
    decl = re.findall(r"STX_API\s+[\w\s\*]+?\b(stx_\w+)\s*\(", head)
    members = re.findall(r"\(\*(\w+)\)\(", table.split("} stx_api_v1;")[0])
    assert members == [d[4:] for d in decl]
