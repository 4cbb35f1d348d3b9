"""ctypes access to the CPU oracle (oracle/liboracle.so) and, where it was built, to the
reference's own src/stft.h (oracle/_ref/libstft_ref.so). Test infrastructure only."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libstft_ref.so")

_vp = ctypes.c_void_p
_i = ctypes.c_int


def _np(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class _Stft:
    """The stft.h entry points with numpy in/out, over a library with prefix `pre`."""

    def __init__(self, path, pre):
        if not os.path.exists(path):
            raise OSError(f"{path} not built (make -C oracle)")
        self.L = ctypes.CDLL(path)
        self.pre = pre
        for name, args in {
            "fft": [_vp, _i, _i],
            "torch_stft": [_vp, _i, _i, _i, _i, _vp, _vp],
            "torch_istft": [_vp, _i, _i, _i, _i, _vp],
            "htdemucs_spec": [_vp, _i, _i, _vp, _vp],
            "htdemucs_ispec": [_vp, _i, _i, _i, _vp],
        }.items():
            fn = getattr(self.L, pre + name)
            fn.restype = _i
            fn.argtypes = args

    def _fn(self, name):
        return getattr(self.L, self.pre + name)

    def fft(self, a, inverse=False):
        a = np.ascontiguousarray(a, dtype=np.complex128).copy()
        rc = self._fn("fft")(_np(a), a.size, int(inverse))
        if rc:
            raise ValueError(f"fft rc={rc}")
        return a

    def torch_stft(self, x, n_fft, hop, normalized=False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.size // hop + 1
        spec = np.zeros((n_fft // 2 + 1, T), dtype=np.complex128)
        nf = ctypes.c_int(0)
        rc = self._fn("torch_stft")(_np(x), x.size, n_fft, hop, int(normalized), _np(spec), ctypes.byref(nf))
        if rc:
            raise RuntimeError(f"torch_stft rc={rc}")
        return spec

    def torch_istft(self, spec, n_fft, hop, normalized=False):
        spec = np.ascontiguousarray(spec, dtype=np.complex128)
        T = spec.shape[1]
        out = np.zeros(hop * (T - 1), dtype=np.float32)
        rc = self._fn("torch_istft")(_np(spec), T, n_fft, hop, int(normalized), _np(out))
        if rc:
            raise RuntimeError(f"torch_istft rc={rc}")
        return out

    def htdemucs_spec(self, x, n_fft):
        x = np.ascontiguousarray(x, dtype=np.float32)
        hl = n_fft // 4
        T = (x.size + hl - 1) // hl
        spec = np.zeros((n_fft // 2, T), dtype=np.complex128)
        nf = ctypes.c_int(0)
        rc = self._fn("htdemucs_spec")(_np(x), x.size, n_fft, _np(spec), ctypes.byref(nf))
        if rc:
            raise RuntimeError(f"htdemucs_spec rc={rc}")
        return spec

    def htdemucs_ispec(self, spec, n_fft, length):
        spec = np.ascontiguousarray(spec, dtype=np.complex128)
        out = np.zeros(length, dtype=np.float32)
        rc = self._fn("htdemucs_ispec")(_np(spec), spec.shape[1], n_fft, length, _np(out))
        if rc:
            raise RuntimeError(f"htdemucs_ispec rc={rc}")
        return out


_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        _oracle = _Stft(ORACLE_PATH, "orc_")
    return _oracle


def reference():
    """The reference's own stft.h (raises OSError where oracle/_ref was not built)."""
    return _Stft(REF_PATH, "ref_")


def ref_available():
    return os.path.exists(REF_PATH)


class _Bands:
    """The band-path oracle functions (oracle/band_oracle.c) with numpy in/out."""

    def __init__(self):
        self.L = ctypes.CDLL(ORACLE_PATH)
        L = self.L
        L.orc_mel_band_map.restype = _i
        L.orc_mel_band_map.argtypes = [_i, _i, _i, _vp, _vp, ctypes.c_long, _vp]
        L.orc_bands_layout.restype = _i
        L.orc_bands_layout.argtypes = [_vp, _i, _vp, ctypes.c_long, _i, _i, _vp, _vp, _vp]
        L.orc_band_gather.restype = None
        L.orc_band_gather.argtypes = [_vp, _i, _vp, _i, _i, _i, _vp, _vp]
        L.orc_band_scatter_apply.restype = None
        L.orc_band_scatter_apply.argtypes = [_vp, _i, _vp, _i, _i, _i, _vp, _i, _vp, _i, _vp]

    def mel_band_map(self, sr, n_fft, n_mels):
        sizes = np.zeros(n_mels, dtype=np.int32)
        cap = n_mels * (n_fft // 2 + 1)
        freqs = np.zeros(cap, dtype=np.int32)
        n = ctypes.c_long(0)
        rc = self.L.orc_mel_band_map(sr, n_fft, n_mels, _np(sizes), _np(freqs), cap, ctypes.byref(n))
        if rc:
            raise RuntimeError(f"mel_band_map rc={rc}")
        return sizes, freqs[: n.value].copy()

    def layout(self, sizes, freqs, n_bins, channels):
        sizes = np.ascontiguousarray(sizes, dtype=np.int32)
        freqs = np.ascontiguousarray(freqs, dtype=np.int32)
        fo = np.zeros(sizes.size + 1, dtype=np.int64)
        fe = np.zeros(sizes.size + 1, dtype=np.int64)
        bpf = np.zeros(n_bins, dtype=np.int32)
        rc = self.L.orc_bands_layout(_np(sizes), sizes.size, _np(freqs), freqs.size, n_bins, channels,
                                     _np(fo), _np(fe), _np(bpf))
        if rc:
            raise RuntimeError(f"bands_layout rc={rc}")
        return fo, fe, bpf

    def gather(self, sizes, freqs, z):
        """z: complex128 [C][F][T] -> feat float32 [total_feat * T]."""
        sizes = np.ascontiguousarray(sizes, dtype=np.int32)
        freqs = np.ascontiguousarray(freqs, dtype=np.int32)
        z = np.ascontiguousarray(z, dtype=np.complex128)
        C, F, T = z.shape
        feat = np.zeros(int(sizes.sum()) * C * 2 * T, dtype=np.float32)
        self.L.orc_band_gather(_np(sizes), sizes.size, _np(freqs), C, F, T, _np(z), _np(feat))
        return feat

    def scatter_apply(self, sizes, freqs, masks, z, zero_dc=False):
        """masks: float32 [S][total_feat * T], z: complex128 [C][F][T] -> complex128 [S][C][F][T]."""
        sizes = np.ascontiguousarray(sizes, dtype=np.int32)
        freqs = np.ascontiguousarray(freqs, dtype=np.int32)
        masks = np.ascontiguousarray(masks, dtype=np.float32)
        z = np.ascontiguousarray(z, dtype=np.complex128)
        C, F, T = z.shape
        S = masks.shape[0]
        out = np.zeros((S, C, F, T), dtype=np.complex128)
        self.L.orc_band_scatter_apply(_np(sizes), sizes.size, _np(freqs), C, F, T, _np(masks), S, _np(z),
                                      int(bool(zero_dc)), _np(out))
        return out


_bands = None


def bands():
    global _bands
    if _bands is None:
        _bands = _Bands()
    return _bands


class _Demix:
    """The demix oracle functions (oracle/demix_oracle.c) with numpy in/out."""

    def __init__(self):
        L = ctypes.CDLL(ORACLE_PATH)
        L.orc_demix_n_chunks.restype = ctypes.c_long
        L.orc_demix_n_chunks.argtypes = [ctypes.c_long, _i, _i]
        L.orc_demix_window.restype = None
        L.orc_demix_window.argtypes = [_i, _vp]
        L.orc_demix_chunks.restype = _i
        L.orc_demix_chunks.argtypes = [_vp, _i, ctypes.c_long, _i, _i, _vp]
        L.orc_demix_ola.restype = _i
        L.orc_demix_ola.argtypes = [_vp, _i, _i, ctypes.c_long, _i, _i, _vp]
        self.L = L

    def n_chunks(self, length, chunk, step):
        return self.L.orc_demix_n_chunks(length, chunk, step)

    def window(self, chunk):
        w = np.zeros(chunk, dtype=np.float32)
        self.L.orc_demix_window(chunk, _np(w))
        return w

    def chunks(self, mix, chunk, step):
        mix = np.ascontiguousarray(mix, dtype=np.float32)
        C, length = mix.shape
        n = self.n_chunks(length, chunk, step)
        parts = np.zeros((n, C, chunk), dtype=np.float32)
        rc = self.L.orc_demix_chunks(_np(mix), C, length, chunk, step, _np(parts))
        if rc:
            raise RuntimeError(f"demix_chunks rc={rc}")
        return parts

    def ola(self, y, length, chunk, step):
        y = np.ascontiguousarray(y, dtype=np.float32)
        n, S, C, _ = y.shape
        out = np.zeros((S, C, length), dtype=np.float32)
        self.L.orc_demix_ola(_np(y), S, C, length, chunk, step, _np(out))
        return out


_demix = None


def demix():
    global _demix
    if _demix is None:
        _demix = _Demix()
    return _demix
