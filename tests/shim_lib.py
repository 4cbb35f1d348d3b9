"""ctypes access to tests/cpp/libst_shim_check.so, the compiled check of the stx::st C++
shim (include/stx_st.hpp). Each call returns (status, result): status 0, 1 for
std::invalid_argument, 2 for std::runtime_error."""
import ctypes
import os

import numpy as np

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "libst_shim_check.so")
_vp, _i = ctypes.c_void_p, ctypes.c_int
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(PATH):
            raise OSError(f"{PATH} not built (make -C tests/cpp)")
        L = ctypes.CDLL(PATH)
        L.shim_time_htdemucs_round_trip.restype = ctypes.c_double
        L.shim_time_htdemucs_round_trip.argtypes = [_i, _vp, _i, _i, _i]
        for name, args in {
            "shim_fft_create": [_i],
            "shim_fft_run": [_i, _vp, _i, _i],
            "shim_htdemucs_spec": [_i, _vp, _i, _vp, _vp],
            "shim_htdemucs_ispec": [_i, _vp, _i, _i, _vp],
            "shim_torch_stft": [_i, _vp, _i, _i, _i, _vp, _vp],
            "shim_torch_istft": [_i, _vp, _i, _i, _i, _vp],
            "shim_istft_short_spectrum": [_i],
            "shim_fft_run_prefix": [_i, _vp, _i, _i],
            "shim_fft_run_short": [_i],
        }.items():
            fn = getattr(L, name)
            fn.restype = _i
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def fft(a, inverse=False):
    a = np.ascontiguousarray(a, dtype=np.complex128).copy()
    n = a.shape[-1]
    rc = lib().shim_fft_run(n, _p(a), a.size // n, int(inverse))
    return rc, a


def fft_prefix(a, n, inverse=False):
    """st::FFT(n).run on the whole vector a (len >= n)."""
    a = np.ascontiguousarray(a, dtype=np.complex128).copy()
    rc = lib().shim_fft_run_prefix(n, _p(a), a.size, int(inverse))
    return rc, a


def htdemucs_spec(x, n_fft):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = (x.size + n_fft // 4 - 1) // (n_fft // 4)
    spec = np.zeros((n_fft // 2, T), np.complex128)
    t = ctypes.c_int(0)
    rc = lib().shim_htdemucs_spec(n_fft, _p(x), x.size, _p(spec), ctypes.byref(t))
    return rc, spec[:, : t.value] if rc == 0 else None


def htdemucs_ispec(spec, n_fft, length):
    spec = np.ascontiguousarray(spec, dtype=np.complex128)
    out = np.zeros(length, np.float32)
    rc = lib().shim_htdemucs_ispec(n_fft, _p(spec), spec.shape[1], length, _p(out))
    return rc, out


def torch_stft(x, n_fft, hop, normalized=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.size // hop + 1
    spec = np.zeros((n_fft // 2 + 1, T), np.complex128)
    t = ctypes.c_int(0)
    rc = lib().shim_torch_stft(n_fft, _p(x), x.size, hop, int(normalized), _p(spec), ctypes.byref(t))
    return rc, spec


def torch_istft(spec, n_fft, hop, normalized=False):
    spec = np.ascontiguousarray(spec, dtype=np.complex128)
    T = spec.shape[1]
    out = np.zeros(hop * (T - 1), np.float32)
    rc = lib().shim_torch_istft(n_fft, _p(spec), T, hop, int(normalized), _p(out))
    return rc, out
