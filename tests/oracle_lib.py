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

    def vrfft(self, a, inverse=False):
        """st::VRFFT (Bluestein, any size) of the oracle."""
        fn = self.L.orc_vrfft
        fn.restype = _i
        fn.argtypes = [_vp, _i, _i]
        a = np.ascontiguousarray(a, dtype=np.complex128).copy()
        if fn(_np(a), a.size, int(inverse)):
            raise ValueError("vrfft")
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
        L.orc_msst_window.restype = None
        L.orc_msst_window.argtypes = [_i, _vp]
        L.orc_msst_n_chunks.restype = ctypes.c_long
        L.orc_msst_n_chunks.argtypes = [ctypes.c_long, _i, _i]
        L.orc_msst_chunks.restype = _i
        L.orc_msst_chunks.argtypes = [_vp, _i, ctypes.c_long, _i, _i, _vp]
        L.orc_msst_ola.restype = _i
        L.orc_msst_ola.argtypes = [_vp, _i, _i, ctypes.c_long, _i, _i, _vp]
        L.orc_uvr_geometry.restype = ctypes.c_long
        L.orc_uvr_geometry.argtypes = [ctypes.c_long, _i, _i, ctypes.c_float, ctypes.POINTER(ctypes.c_long),
                                       ctypes.POINTER(ctypes.c_long)]
        L.orc_uvr_chunks.restype = _i
        L.orc_uvr_chunks.argtypes = [_vp, _i, ctypes.c_long, _i, _i, ctypes.c_float, _vp]
        L.orc_uvr_ola.restype = _i
        L.orc_uvr_ola.argtypes = [_vp, _i, _i, ctypes.c_long, _i, _i, ctypes.c_float, _vp]
        L.orc_tfc_post.restype = None
        L.orc_tfc_post.argtypes = [_vp, ctypes.c_long, _i, ctypes.c_float, _i, _vp]
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

    # TFC-TDF: MSST and UVR chunking (oracle/tfc_oracle.c)
    def msst_window(self, chunk):
        w = np.zeros(chunk, dtype=np.float32)
        self.L.orc_msst_window(chunk, _np(w))
        return w

    def msst_chunks(self, mix, chunk, step):
        mix = np.ascontiguousarray(mix, dtype=np.float32)
        C, length = mix.shape
        n = self.L.orc_msst_n_chunks(length, chunk, step)
        parts = np.zeros((n, C, chunk), dtype=np.float32)
        if self.L.orc_msst_chunks(_np(mix), C, length, chunk, step, _np(parts)):
            raise RuntimeError("msst_chunks")
        return parts

    def msst_ola(self, y, length, chunk, step):
        y = np.ascontiguousarray(y, dtype=np.float32)
        n, S, C, _ = y.shape
        out = np.zeros((S, C, length), dtype=np.float32)
        self.L.orc_msst_ola(_np(y), S, C, length, chunk, step, _np(out))
        return out

    def uvr_geometry(self, length, chunk, n_fft, overlap=-1.0):
        M, st = ctypes.c_long(), ctypes.c_long()
        n = self.L.orc_uvr_geometry(length, chunk, n_fft, overlap, ctypes.byref(M), ctypes.byref(st))
        return n, M.value, st.value

    def uvr_chunks(self, mix, chunk, n_fft, overlap=-1.0):
        mix = np.ascontiguousarray(mix, dtype=np.float32)
        C, length = mix.shape
        n, _, _ = self.uvr_geometry(length, chunk, n_fft, overlap)
        parts = np.zeros((n, C, chunk), dtype=np.float32)
        if self.L.orc_uvr_chunks(_np(mix), C, length, chunk, n_fft, overlap, _np(parts)):
            raise RuntimeError("uvr_chunks")
        return parts

    def uvr_ola(self, y, length, chunk, n_fft, overlap=-1.0):
        y = np.ascontiguousarray(y, dtype=np.float32)
        n, S, C, _ = y.shape
        out = np.zeros((S, C, length), dtype=np.float32)
        if self.L.orc_uvr_ola(_np(y), S, C, length, chunk, n_fft, overlap, _np(out)):
            raise RuntimeError("uvr_ola")
        return out

    def tfc_post(self, mix, est, compensate, complement):
        """est float32 [S][C][len] -> [S + complement][C][len]."""
        mix = np.ascontiguousarray(mix, dtype=np.float32)
        S = est.shape[0]
        out = np.zeros((S + (1 if complement else 0),) + est.shape[1:], np.float32)
        out[:S] = est
        self.L.orc_tfc_post(_np(mix), mix.size, S, compensate, int(bool(complement)), _np(out))
        return out


_demix = None


def demix():
    global _demix
    if _demix is None:
        _demix = _Demix()
    return _demix


def _ne(shape):
    """ggml extents of a numpy shape (torch/numpy's last dim is ne[0])."""
    s = list(shape)[::-1] + [1] * (4 - len(shape))
    return (ctypes.c_int64 * 4)(*s)


class _Ops:
    """The ggml op oracle functions (oracle/ops_oracle.c) with numpy in/out. Shapes are numpy
    shapes (last axis = ne0); broadcast operands have numpy shapes of the same rank."""

    def __init__(self):
        L = ctypes.CDLL(ORACLE_PATH)
        i64p = ctypes.POINTER(ctypes.c_int64)
        L.orc_group_norm.restype = _i
        L.orc_group_norm.argtypes = [_vp, i64p, _i, ctypes.c_float, _vp, i64p, _vp, i64p, _i, _vp]
        L.orc_norm.restype = _i
        L.orc_norm.argtypes = [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, _i, _vp, _vp, _vp]
        L.orc_soft_max.restype = _i
        L.orc_soft_max.argtypes = [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, _vp]
        L.orc_gelu_erf.restype = None
        L.orc_gelu_erf.argtypes = [_vp, ctypes.c_int64, _vp]
        L.orc_glu.restype = _i
        L.orc_glu.argtypes = [_vp, i64p, _i, _vp]
        L.orc_binary.restype = _i
        L.orc_binary.argtypes = [_i, _vp, i64p, _vp, i64p, _vp, i64p, _vp]
        L.orc_rope.restype = _i
        L.orc_rope.argtypes = [_vp, i64p, _vp, _i, _i, ctypes.c_float, ctypes.c_float, ctypes.c_float, _vp]
        L.orc_cont_permute.restype = _i
        L.orc_cont_permute.argtypes = [_vp, i64p, ctypes.POINTER(ctypes.c_int), _vp]
        L.orc_concat.restype = _i
        L.orc_concat.argtypes = [_vp, i64p, _i, _i, _vp]
        L.orc_qkv_rope_split.restype = _i
        L.orc_qkv_rope_split.argtypes = [_vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp,
                                         ctypes.c_float, ctypes.c_float, ctypes.c_float, _vp, _vp, _vp]
        L.orc_merge_heads.restype = _i
        L.orc_merge_heads.argtypes = [_vp, i64p, _vp, _vp]
        self.L = L

    @staticmethod
    def _f(a):
        return np.ascontiguousarray(a, dtype=np.float32)

    def group_norm(self, x, n_groups, eps=1e-5, w=None, b=None, gelu=False):
        x = self._f(x)
        y = np.empty_like(x)
        wa = None if w is None else self._f(w)
        ba = None if b is None else self._f(b)
        rc = self.L.orc_group_norm(_np(x), _ne(x.shape), n_groups, eps, None if wa is None else _np(wa),
                                   _ne(wa.shape if wa is not None else x.shape), None if ba is None else _np(ba),
                                   _ne(ba.shape if ba is not None else x.shape), int(gelu), _np(y))
        if rc:
            raise ValueError(f"group_norm rc={rc}")
        return y

    def norm(self, x, eps, rms=False, w=None, b=None):
        x = self._f(x)
        y = np.empty_like(x)
        wa = None if w is None else self._f(w)
        ba = None if b is None else self._f(b)
        n0 = x.shape[-1]
        rc = self.L.orc_norm(_np(x), n0, x.size // max(n0, 1), eps, int(rms), None if wa is None else _np(wa),
                             None if ba is None else _np(ba), _np(y))
        if rc:
            raise ValueError(f"norm rc={rc}")
        return y

    def soft_max(self, x, scale):
        x = self._f(x)
        y = np.empty_like(x)
        n0 = x.shape[-1]
        if self.L.orc_soft_max(_np(x), n0, x.size // n0, scale, _np(y)):
            raise ValueError("soft_max")
        return y

    def gelu(self, x):
        x = self._f(x)
        y = np.empty_like(x)
        self.L.orc_gelu_erf(_np(x), x.size, _np(y))
        return y

    def glu(self, x, dim):
        """dim is the ggml dimension (0 = last numpy axis)."""
        x = self._f(x)
        shape = list(x.shape) + []
        ax = x.ndim - 1 - dim
        shape[ax] //= 2
        y = np.empty(shape, np.float32)
        if self.L.orc_glu(_np(x), _ne(x.shape), dim, _np(y)):
            raise ValueError("glu")
        return y

    def binary(self, op, a, b, c=None):
        """op: 'add', 'mul', 'mul_add' (a + b * c) or 'add_gelu' (gelu(a + b))."""
        code = {"add": 0, "mul": 1, "mul_add": 2, "add_gelu": 3}[op]
        a, b = self._f(a), self._f(b)
        c = self._f(c) if c is not None else b
        y = np.empty_like(a)
        pad = lambda s: (1,) * (a.ndim - len(s)) + tuple(s)
        if self.L.orc_binary(code, _np(a), _ne(a.shape), _np(b), _ne(pad(b.shape)), _np(c), _ne(pad(c.shape)),
                             _np(y)):
            raise ValueError("binary")
        return y

    def rope(self, x, pos, n_dims, mode=0, freq_base=10000.0, freq_scale=1.0, attn_factor=1.0):
        x = self._f(x)
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        y = np.empty_like(x)
        if self.L.orc_rope(_np(x), _ne(x.shape), _np(pos), n_dims, mode, freq_base, freq_scale, attn_factor, _np(y)):
            raise ValueError("rope")
        return y

    def cont_permute(self, x, axes):
        """ggml_cont(ggml_permute(x, *axes)); x is a numpy array of up to 4 dims (last = ne0)."""
        x = self._f(x)
        ne = list(x.shape)[::-1] + [1] * (4 - x.ndim)
        yne = [1, 1, 1, 1]
        for i, a in enumerate(axes):
            yne[a] = ne[i]
        y = np.empty(yne[::-1], np.float32)
        if self.L.orc_cont_permute(_np(x), _ne(x.shape), (ctypes.c_int * 4)(*axes), _np(y)):
            raise ValueError("cont_permute")
        return y

    def concat(self, xs, dim):
        """ggml_concat of numpy arrays of equal rank along ggml dimension dim."""
        xs = [self._f(x) for x in xs]
        nes = []
        for x in xs:
            nes += list(_ne(x.shape))
        shape = list(xs[0].shape)
        ax = xs[0].ndim - 1 - dim
        shape[ax] = sum(x.shape[ax] for x in xs)
        y = np.empty(shape, np.float32)
        ptrs = (ctypes.c_void_p * len(xs))(*[x.ctypes.data for x in xs])
        if self.L.orc_concat(ptrs, (ctypes.c_int64 * len(nes))(*nes), len(xs), dim, _np(y)):
            raise ValueError("concat")
        return y

    def qkv_rope_split(self, qkv, pos, n_head, freq_base=10000.0, freq_scale=1.0, attn_factor=1.0):
        """qkv numpy (batch, N, 3*H*dh) -> q, k (batch, H, N, dh), vt (batch, H, dh, N)."""
        qkv = self._f(qkv)
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        batch, N, width = qkv.shape
        dh = width // (3 * n_head)
        q = np.empty((batch, n_head, N, dh), np.float32)
        k = np.empty_like(q)
        vt = np.empty((batch, n_head, dh, N), np.float32)
        if self.L.orc_qkv_rope_split(_np(qkv), dh, n_head, N, batch, _np(pos), freq_base, freq_scale, attn_factor,
                                     _np(q), _np(k), _np(vt)):
            raise ValueError("qkv_rope_split")
        return q, k, vt

    def merge_heads(self, o, gates=None):
        """o numpy (batch, H, N, dh) -> (batch, N, H, dh) [* gates (batch, N, H)]."""
        o = self._f(o)
        b, H, N, dh = o.shape
        y = np.empty((b, N, H, dh), np.float32)
        g = None if gates is None else self._f(gates)
        if self.L.orc_merge_heads(_np(o), _ne(o.shape), None if g is None else _np(g), _np(y)):
            raise ValueError("merge_heads")
        return y


_ops = None


def ops():
    global _ops
    if _ops is None:
        _ops = _Ops()
    return _ops


class _HTDemucs:
    """HTDemucs pre/post-processing and split oracle (oracle/htdemucs_oracle.c), numpy in/out."""

    def __init__(self):
        L = ctypes.CDLL(ORACLE_PATH)
        d = ctypes.c_double
        dp = ctypes.POINTER(d)
        i64 = ctypes.c_int64
        L.orc_mean_std.restype = None
        L.orc_mean_std.argtypes = [_vp, i64, dp, dp]
        L.orc_cac_normalize.restype = None
        L.orc_cac_normalize.argtypes = [_vp, _i, i64, d, d, _vp]
        L.orc_normalize.restype = None
        L.orc_normalize.argtypes = [_vp, i64, d, d, _vp]
        L.orc_cac_denormalize.restype = None
        L.orc_cac_denormalize.argtypes = [_vp, _i, _i, i64, d, d, _vp]
        L.orc_time_add.restype = None
        L.orc_time_add.argtypes = [_vp, _vp, i64, d, d, _vp]
        L.orc_mix_normalize.restype = None
        L.orc_mix_normalize.argtypes = [_vp, _i, i64, _vp, _vp]
        L.orc_split_weights.restype = None
        L.orc_split_weights.argtypes = [_i, _vp]
        L.orc_split_count.restype = _i
        L.orc_split_count.argtypes = [_i, _i, ctypes.c_float, ctypes.POINTER(_i)]
        L.orc_segments.restype = None
        L.orc_segments.argtypes = [_vp, _i, i64, i64, _i, _i, _i, _vp]
        L.orc_split_ola.restype = None
        L.orc_split_ola.argtypes = [_vp, _i, _i, _i, _i, _vp, _vp]
        L.orc_htdemucs_shift_offsets.restype = None
        L.orc_htdemucs_shift_offsets.argtypes = [ctypes.c_uint32, _i, _i, _i, _vp]
        self.L = L

    @staticmethod
    def _f(a):
        return np.ascontiguousarray(a, dtype=np.float32)

    def mean_std(self, x):
        x = self._f(x)
        m, s = ctypes.c_double(), ctypes.c_double()
        self.L.orc_mean_std(_np(x), x.size, ctypes.byref(m), ctypes.byref(s))
        return m.value, s.value

    def cac_pack(self, spec):
        """complex64 [C, F, T] -> float32 [2C, F, T] (re, im planes), no normalisation."""
        C = spec.shape[0]
        out = np.empty((2 * C,) + spec.shape[1:], np.float32)
        out[0::2] = spec.real
        out[1::2] = spec.imag
        return out

    def cac_normalize(self, spec, mean, sd):
        spec = np.ascontiguousarray(spec, dtype=np.complex64)
        C = spec.shape[0]
        ft = spec[0].size
        mag = np.empty((2 * C,) + spec.shape[1:], np.float32)
        self.L.orc_cac_normalize(_np(spec), C, ft, mean, sd, _np(mag))
        return mag

    def normalize(self, x, mean, sd):
        x = self._f(x)
        y = np.empty_like(x)
        self.L.orc_normalize(_np(x), x.size, mean, sd, _np(y))
        return y

    def cac_denormalize(self, ox, mean, sd):
        ox = self._f(ox)
        S, C2 = ox.shape[:2]
        ft = ox[0, 0].size
        spec = np.empty((S, C2 // 2) + ox.shape[2:], np.complex64)
        self.L.orc_cac_denormalize(_np(ox), S, C2 // 2, ft, mean, sd, _np(spec))
        return spec

    def time_add(self, t, y, mean, sd):
        t, y = self._f(t), self._f(y)
        out = np.empty_like(t)
        self.L.orc_time_add(_np(t), _np(y), t.size, mean, sd, _np(out))
        return out

    def mix_normalize(self, mix):
        mix = self._f(mix)
        out = np.empty_like(mix)
        stats = np.zeros(2, np.float64)
        self.L.orc_mix_normalize(_np(mix), mix.shape[0], mix.shape[1], _np(out), _np(stats))
        return out, stats

    def split_weights(self, seg):
        w = np.empty(seg, np.float32)
        self.L.orc_split_weights(seg, _np(w))
        return w

    def split_count(self, length, seg, overlap):
        st = ctypes.c_int()
        n = self.L.orc_split_count(length, seg, overlap, ctypes.byref(st))
        return st.value, n

    def segments(self, buf, offset, length, seg, stride):
        buf = self._f(buf)
        C, total = buf.shape
        n = (length + stride - 1) // stride
        parts = np.empty((n, C, seg), np.float32)
        self.L.orc_segments(_np(buf), C, total, offset, length, seg, stride, _np(parts))
        return parts

    def shift_offsets(self, seed, max_shift, n_models, shifts):
        out = np.zeros((n_models, shifts), np.int32)
        self.L.orc_htdemucs_shift_offsets(seed, max_shift, n_models, shifts, _np(out))
        return out

    def separate(self, mix, segment, bag, model, sample_rate=44100, shifts=0, overlap=-1.0, seed=0):
        """HTDemucs::separate (src/htdemucs.cpp:534-644) composed from the oracle's pieces and numpy
        float32 arithmetic; model(m, parts [n][C][seg]) -> [n][S*C][seg]."""
        C, L = mix.shape
        S = bag.shape[1]
        norm, stats = self.mix_normalize(mix)
        stride, _ = self.split_count(L, segment, overlap)

        def split(m, offset, length):
            parts = self.segments(norm, offset, length, segment, stride)
            return self.split_ola(model(m, parts), length, stride)

        est = np.zeros((S * C, L), np.float32)
        totals = np.zeros(S, np.float32)
        ms = sample_rate // 2
        offs = self.shift_offsets(seed, ms, bag.shape[0], shifts) if shifts > 0 else None
        for m in range(bag.shape[0]):
            if shifts == 0:
                res = split(m, 0, L)
            else:
                res = np.zeros((S * C, L), np.float32)
                for k in range(shifts):
                    off = int(offs[m, k])
                    o = split(m, off - ms, L + ms - off)
                    res += o[:, ms - off:ms - off + L]
                res /= np.float32(shifts)
            for s in range(S):
                w = np.float32(bag[m, s])
                totals[s] += w
                if w == 0.0:
                    continue
                est[s * C:(s + 1) * C] += w * res[s * C:(s + 1) * C]
        out = np.empty_like(est)
        for s in range(S):
            q = est[s * C:(s + 1) * C] / totals[s]
            out[s * C:(s + 1) * C] = (q.astype(np.float64) * stats[1] + stats[0]).astype(np.float32)
        return out.reshape(S, C, L)

    def split_ola(self, y, length, stride):
        y = self._f(y)
        n, tracks, seg = y.shape
        out = np.empty((tracks, length), np.float32)
        sw = np.empty(length, np.float32)
        self.L.orc_split_ola(_np(y), tracks, length, seg, stride, _np(out), _np(sw))
        return out


_htd = None


def htdemucs():
    global _htd
    if _htd is None:
        _htd = _HTDemucs()
    return _htd


class _Resample:
    """st::resample_planar oracle (oracle/resample_oracle.c)."""

    def __init__(self):
        L = ctypes.CDLL(ORACLE_PATH)
        L.orc_resample.restype = _i
        L.orc_resample.argtypes = [_vp, _i, _i, _i, _i, _vp]
        L.orc_resample_length.restype = ctypes.c_long
        L.orc_resample_length.argtypes = [ctypes.c_long, _i, _i]
        L.orc_resample_table.restype = None
        L.orc_resample_table.argtypes = [_i, _i, _vp, ctypes.POINTER(ctypes.c_double)]
        L.orc_to_channels.restype = None
        L.orc_to_channels.argtypes = [_vp, ctypes.c_long, _i, _i, _i, _vp]
        L.orc_pin_length.restype = None
        L.orc_pin_length.argtypes = [_vp, ctypes.c_long, ctypes.c_long, ctypes.c_long, _vp]
        self.L = L

    def to_channels(self, samples, n, ch, layout, want):
        """samples: flat float32 (planar [ch][n] or interleaved [n][ch]) -> [want][n]."""
        x = np.ascontiguousarray(samples, dtype=np.float32).reshape(-1)
        out = np.zeros((want, n), np.float32)
        self.L.orc_to_channels(_np(x), n, ch, layout, want, _np(out))
        return out

    def pin_length(self, x, n):
        """x [planes][back] -> [planes][n], cut or zero-padded."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        planes, back = x.shape
        out = np.zeros((planes, n), np.float32)
        self.L.orc_pin_length(_np(x), planes, back, n, _np(out))
        return out

    def separate_audio(self, samples, n, ch, layout, sr, C, R, model):
        """libstems separate() (src/libstems.cpp:160-196) around model(audio [C][len]) ->
        stems [S][C][len], composed from the oracle's steps."""
        a = self.to_channels(samples, n, ch, layout, C)
        if sr != R:
            a = self(a, sr, R)
        stems = np.ascontiguousarray(model(a), dtype=np.float32)
        if sr == R:
            return stems
        S = stems.shape[0]
        back = self(stems.reshape(S * C, -1), R, sr)
        return self.pin_length(back, n).reshape(S, C, n)

    def table(self, src, dst):
        t = np.zeros((1 << 15) + 2, np.float64)
        half = ctypes.c_double()
        self.L.orc_resample_table(src, dst, _np(t), ctypes.byref(half))
        return t, half.value

    def __call__(self, x, src, dst):
        x = np.ascontiguousarray(x, dtype=np.float32)
        C, n = x.shape
        m = self.L.orc_resample_length(n, src, dst)
        out = np.zeros((C, m), np.float32)
        self.L.orc_resample(_np(x), n, C, src, dst, _np(out))
        return out


def resample():
    return _Resample()
