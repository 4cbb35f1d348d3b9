"""ctypes binding of libstx.so, the C ABI declared in include/stx.h.

This is the Python face of the library for tests, the benchmark and Python callers. Device
buffers are torch tensors (torch is used only for device memory and streams); every call goes
straight to the HIP kernels in libstx.so. There is no fallback: if the library is missing,
loading it raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libstx.so")

STATUS_OK = 0
STATUS_INVALID_ARGUMENT = 1
STATUS_UNSUPPORTED = 2
STATUS_CANCELLED = 3
STATUS_RUNTIME_ERROR = 4
STATUS_OUT_OF_MEMORY = 6
STATUS_DEVICE_ERROR = 7

F_MAJOR = 0
T_MAJOR = 1

_c_int_p = ctypes.POINTER(ctypes.c_int)
_vp = ctypes.c_void_p
_i = ctypes.c_int

# name -> (restype, argtypes); every STX_API function of include/stx.h.
_SIGNATURES = {
    "stx_version": (ctypes.c_char_p, []),
    "stx_last_error": (ctypes.c_char_p, []),
    "stx_fft_create": (_i, [_i, ctypes.POINTER(_vp)]),
    "stx_fft_destroy": (None, [_vp]),
    "stx_fft_create_any": (_i, [_i, ctypes.POINTER(_vp)]),
    "stx_resampler_create": (_i, [_i, _i, ctypes.POINTER(_vp)]),
    "stx_resampler_destroy": (None, [_vp]),
    "stx_resample_length": (ctypes.c_int64, [_vp, ctypes.c_int64]),
    "stx_resample": (_i, [_vp, _vp, _i, ctypes.c_int64, _vp, _vp]),
    "stx_fft_size": (_i, [_vp]),
    "stx_fft_run": (_i, [_vp, _vp, _i, _i, _vp]),
    "stx_torch_stft_frames": (_i, [_i, _i]),
    "stx_htdemucs_frames": (_i, [_i, _i]),
    "stx_torch_stft": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "stx_torch_istft": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "stx_htdemucs_spec": (_i, [_vp, _vp, _i, _i, _vp, _i, _vp]),
    "stx_htdemucs_ispec": (_i, [_vp, _vp, _i, _i, _i, _vp, _i, _vp]),
    "stx_istft_workspace_size": (ctypes.c_size_t, [_vp, _i, _i]),
    "stx_torch_istft_ws": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _i, _vp, ctypes.c_size_t, _vp]),
    "stx_htdemucs_ispec_ws": (_i, [_vp, _vp, _i, _i, _i, _vp, _i, _vp, ctypes.c_size_t, _vp]),
    "stx_mel_band_map": (_i, [_i, _i, _i, _vp, _vp, ctypes.c_int64, _vp]),
    "stx_bs_band_map": (_i, [_vp, _i, _i, _vp, ctypes.c_int64, _vp]),
    "stx_bands_layout": (_i, [_vp, _i, _vp, ctypes.c_int64, _i, _i, _vp, _vp, _vp]),
    "stx_bands_create": (_i, [_vp, _i, _vp, ctypes.c_int64, _i, _i, ctypes.POINTER(_vp)]),
    "stx_bands_destroy": (None, [_vp]),
    "stx_bands_total_feat": (ctypes.c_int64, [_vp]),
    "stx_band_gather": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp]),
    "stx_band_scatter_apply": (_i, [_vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _vp]),
    "stx_band_rms_norm": (_i, [_vp, _vp, _i, _i, _vp, ctypes.c_float, _vp, _vp]),
    "stx_band_mask_glu": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "stx_demix_step": (_i, [_i, _i, ctypes.c_float]),
    "stx_demix_plan": (_i, [ctypes.c_int64, _i, _i, _vp, _vp, ctypes.c_int64]),
    "stx_demix_window": (_i, [_i, _vp]),
    "stx_demix_create": (_i, [ctypes.c_int64, _i, _i, _i, ctypes.POINTER(_vp)]),
    "stx_demix_plan_rules": (_i, [ctypes.c_int64, _i, _i, _i, _vp, _vp, ctypes.c_int64]),
    "stx_demix_window_rules": (_i, [_i, _i, _vp]),
    "stx_demix_create_rules": (_i, [ctypes.c_int64, _i, _i, _i, _i, ctypes.POINTER(_vp)]),
    "stx_uvr_demix_create": (_i, [ctypes.c_int64, _i, _i, _i, ctypes.c_float, ctypes.POINTER(_vp)]),
    "stx_uvr_demix_destroy": (None, [_vp]),
    "stx_uvr_demix_n_chunks": (ctypes.c_int64, [_vp]),
    "stx_uvr_demix_geometry": (_i, [_vp, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64), _c_int_p]),
    "stx_uvr_demix_chunks": (_i, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp]),
    "stx_uvr_demix_overlap_add": (_i, [_vp, _vp, _i, _vp, _vp]),
    "stx_tfc_tdf_separate_workspace_size": (ctypes.c_size_t, [_i, ctypes.c_int64, _i, _i, _i, _i, ctypes.c_float,
                                                              _i, _i]),
    "stx_tfc_tdf_separate": (_i, [_vp, _i, ctypes.c_int64, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i, _vp, _vp,
                                  _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "stx_demix_destroy": (None, [_vp]),
    "stx_demix_n_chunks": (ctypes.c_int64, [_vp]),
    "stx_demix_chunks": (_i, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp]),
    "stx_demix_overlap_add": (_i, [_vp, _vp, _i, _vp, _vp]),
    "stx_demix_track_workspace_size": (ctypes.c_size_t, [_i, ctypes.c_int64, _i, _i, _i, _i, _i, _i]),
    "stx_demix_track": (_i, [_vp, _i, ctypes.c_int64, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp,
                             ctypes.c_size_t, _vp]),
    "stx_htdemucs_norm_workspace_size": (ctypes.c_size_t, [ctypes.c_int64]),
    "stx_htdemucs_cac_normalize": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "stx_htdemucs_wave_normalize": (_i, [_vp, ctypes.c_int64, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "stx_htdemucs_mix_normalize": (_i, [_vp, _i, ctypes.c_int64, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "stx_htdemucs_cac_denormalize": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "stx_htdemucs_time_add": (_i, [_vp, _vp, ctypes.c_int64, _vp, _vp, _vp]),
    "stx_htdemucs_split_plan": (_i, [_i, _i, ctypes.c_float, _c_int_p, _c_int_p]),
    "stx_htdemucs_segments": (_i, [_vp, _i, ctypes.c_int64, ctypes.c_int64, _i, _i, _i, _i, _i, _vp, _vp]),
    "stx_htdemucs_split_overlap_add": (_i, [_vp, _i, _i, _i, _i, _vp, _vp]),
    "stx_htdemucs_separate_workspace_size": (ctypes.c_size_t, [_i, ctypes.c_int64, _i, _i, _i, _i, _i,
                                                               ctypes.c_float]),
    "stx_htdemucs_separate": (_i, [_vp, _i, ctypes.c_int64, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp,
                                   ctypes.c_size_t, _vp]),
    "stx_separate_options_init": (_i, [_vp]),
    "stx_get_api": (_vp, [ctypes.c_uint32]),
    "stx_group_norm_workspace_size": (ctypes.c_size_t, [_vp, _i]),
    "stx_group_norm": (_i, [_vp, _vp, _i, ctypes.c_float, _vp, _vp, _i, _vp, ctypes.c_size_t, _vp]),
    "stx_group_norm_noalloc": (_i, [_vp, _vp, _i, ctypes.c_float, _vp, _vp, _i, _vp]),
    "stx_grid_sync_fallbacks": (_i, [_vp, ctypes.POINTER(ctypes.c_uint32)]),
    "stx_norm": (_i, [_vp, _vp, ctypes.c_float, _vp]),
    "stx_norm_affine": (_i, [_vp, _vp, _vp, _vp, ctypes.c_float, _vp]),
    "stx_rms_norm": (_i, [_vp, _vp, ctypes.c_float, _vp]),
    "stx_rms_norm_mul": (_i, [_vp, _vp, _vp, ctypes.c_float, _vp]),
    "stx_soft_max_ext": (_i, [_vp, _vp, _vp, ctypes.c_float, ctypes.c_float, _vp]),
    "stx_gelu_erf": (_i, [_vp, _vp, _vp]),
    "stx_add_gelu_erf": (_i, [_vp, _vp, _vp, _vp]),
    "stx_glu": (_i, [_vp, _vp, _i, _vp]),
    "stx_add": (_i, [_vp, _vp, _vp, _vp]),
    "stx_mul": (_i, [_vp, _vp, _vp, _vp]),
    "stx_mul_add": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "stx_glu_mul_add": (_i, [_vp, _vp, _i, _vp, _vp, _vp]),
    "stx_rope_ext": (_i, [_vp, _vp, _vp, _i, _i, _i, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                          ctypes.c_float, ctypes.c_float, ctypes.c_float, _vp]),
    "stx_qkv_rope_split": (_i, [_vp, _vp, _i, ctypes.c_float, ctypes.c_float, ctypes.c_float, _vp, _vp, _vp, _vp]),
    "stx_merge_heads": (_i, [_vp, _vp, _vp, _vp]),
    "stx_cont_permute": (_i, [_vp, _i, _i, _i, _i, _vp, _vp]),
    "stx_concat": (_i, [_vp, _i, _i, _vp, _vp]),
    "stx_separate_audio_workspace_size": (ctypes.c_size_t, [_vp, _i, _i, _i]),
    "stx_separate_audio": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
}


class StxError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"stx status {status}: {message}")
        self.status = status
        self.message = message


_lib = None


def lib():
    """The loaded libstx.so (loaded on first use; raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OSError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status):
    if status != STATUS_OK:
        raise StxError(status, lib().stx_last_error().decode())


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    """hipStream_t of a torch stream (default: torch's current stream)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _require(t, dtype, what):
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{what} must be a CUDA (HIP) tensor")
    if t.dtype != dtype:
        raise TypeError(f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


class FFT:
    """st::FFT (src/stft.h:19-55) on the device: plan holding the window and twiddle tables."""

    def __init__(self, n, any_size=False):
        """any_size: st::VRFFT's sizes as well (even 2^a 3^b 5^c, stx_fft_create_any)."""
        h = ctypes.c_void_p()
        create = lib().stx_fft_create_any if any_size else lib().stx_fft_create
        check(create(int(n), ctypes.byref(h)))
        self.handle = h
        self.n = int(n)

    def close(self):
        if getattr(self, "handle", None):
            lib().stx_fft_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def size(self):
        return lib().stx_fft_size(self.handle)

    def run(self, data, inverse=False, stream=None):
        """In-place batched unnormalised FFT of complex64 data [..., n]."""
        import torch
        _require(data, torch.complex64, "data")
        if data.shape[-1] != self.n:
            raise ValueError("last dimension must be the FFT size")
        batch = data.numel() // self.n
        check(lib().stx_fft_run(self.handle, _ptr(data), batch, int(bool(inverse)), _stream(stream)))
        return data


def torch_stft_frames(length, hop):
    return lib().stx_torch_stft_frames(int(length), int(hop))


def htdemucs_frames(n_fft, length):
    return lib().stx_htdemucs_frames(int(n_fft), int(length))


def torch_stft(fft, x, hop, normalized=False, layout=F_MAJOR, out=None, stream=None):
    """x: float32 [C, len] -> complex64 [C, F, T] (F_MAJOR) or [C, T, F] (T_MAJOR)."""
    import torch
    _require(x, torch.float32, "x")
    C, L = x.shape
    T = L // hop + 1
    F = fft.n // 2 + 1
    shape = (C, F, T) if layout == F_MAJOR else (C, T, F)
    if out is None:
        out = torch.empty(shape, dtype=torch.complex64, device=x.device)
    check(lib().stx_torch_stft(fft.handle, _ptr(x), C, L, int(hop), int(bool(normalized)), _ptr(out),
                               int(layout), _stream(stream)))
    return out


def istft_workspace_size(fft, channels, n_frames):
    return lib().stx_istft_workspace_size(fft.handle, int(channels), int(n_frames))


def _ws(workspace):
    """(pointer, bytes) of an optional workspace tensor."""
    if workspace is None:
        return None, 0
    import torch
    if not isinstance(workspace, torch.Tensor) or not workspace.is_cuda:
        raise TypeError("workspace must be a CUDA (HIP) tensor")
    return ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * workspace.element_size()


def torch_istft(fft, spec, hop, normalized=False, layout=F_MAJOR, out=None, stream=None, workspace=None):
    """spec: complex64 [C, F, T] or [C, T, F] -> float32 [C, hop * (T - 1)]. A workspace tensor
    of at least istft_workspace_size() bytes is required for sizes that are not powers of two
    (two kernels); power-of-two sizes check it and run the single fused kernel."""
    import torch
    _require(spec, torch.complex64, "spec")
    C = spec.shape[0]
    T = spec.shape[2] if layout == F_MAJOR else spec.shape[1]
    if out is None:
        out = torch.empty((C, hop * (T - 1)), dtype=torch.float32, device=spec.device)
    wp, wb = _ws(workspace)
    check(lib().stx_torch_istft_ws(fft.handle, _ptr(spec), C, T, int(hop), int(bool(normalized)), _ptr(out),
                                   int(layout), wp, wb, _stream(stream)))
    return out


def htdemucs_spec(fft, x, layout=F_MAJOR, out=None, stream=None):
    """x: float32 [C, len] -> complex64 [C, n/2, T] (F_MAJOR) or [C, T, n/2]."""
    import torch
    _require(x, torch.float32, "x")
    C, L = x.shape
    T = htdemucs_frames(fft.n, L)
    F = fft.n // 2
    shape = (C, F, T) if layout == F_MAJOR else (C, T, F)
    if out is None:
        out = torch.empty(shape, dtype=torch.complex64, device=x.device)
    check(lib().stx_htdemucs_spec(fft.handle, _ptr(x), C, L, _ptr(out), int(layout), _stream(stream)))
    return out


def htdemucs_ispec(fft, spec, length, layout=F_MAJOR, out=None, stream=None, workspace=None):
    """spec: complex64 [C, n/2, T] or [C, T, n/2] -> float32 [C, length]."""
    import torch
    _require(spec, torch.complex64, "spec")
    C = spec.shape[0]
    T = spec.shape[2] if layout == F_MAJOR else spec.shape[1]
    if out is None:
        out = torch.empty((C, length), dtype=torch.float32, device=spec.device)
    wp, wb = _ws(workspace)
    check(lib().stx_htdemucs_ispec_ws(fft.handle, _ptr(spec), C, T, int(length), _ptr(out), int(layout),
                                      wp, wb, _stream(stream)))
    return out


def workspace(nbytes, device):
    """A zero-filled device workspace tensor of at least nbytes."""
    import torch
    return torch.zeros(max(1, (int(nbytes) + 3) // 4), dtype=torch.float32, device=device)


# ------------------------------------------------------------------------------- bands
def _np_ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def mel_band_map(sample_rate, n_fft, n_mels):
    """(band_sizes int32[n_mels], band_freqs int32[...]) of MelBandRoformer (host only)."""
    import numpy as np
    n = ctypes.c_int64(0)
    check(lib().stx_mel_band_map(int(sample_rate), int(n_fft), int(n_mels), None, None, 0, ctypes.byref(n)))
    sizes = np.zeros(n_mels, dtype=np.int32)
    freqs = np.zeros(max(1, n.value), dtype=np.int32)
    check(lib().stx_mel_band_map(int(sample_rate), int(n_fft), int(n_mels), _np_ptr(sizes), _np_ptr(freqs),
                                 freqs.size, ctypes.byref(n)))
    return sizes, freqs[: n.value].copy()


def bs_band_map(freqs_per_bands, n_fft):
    import numpy as np
    fpb = np.ascontiguousarray(freqs_per_bands, dtype=np.int32)
    n = ctypes.c_int64(0)
    out = np.zeros(n_fft // 2 + 1, dtype=np.int32)
    check(lib().stx_bs_band_map(_np_ptr(fpb), fpb.size, int(n_fft), _np_ptr(out), out.size, ctypes.byref(n)))
    return out[: n.value].copy()


def bands_layout(band_sizes, band_freqs, n_bins, channels):
    """(band_freq_off int64[B+1], band_feat_off int64[B+1], bands_per_freq int32[n_bins]) (host only)."""
    import numpy as np
    sizes = np.ascontiguousarray(band_sizes, dtype=np.int32)
    freqs = np.ascontiguousarray(band_freqs, dtype=np.int32)
    fo = np.zeros(sizes.size + 1, dtype=np.int64)
    fe = np.zeros(sizes.size + 1, dtype=np.int64)
    bpf = np.zeros(n_bins, dtype=np.int32)
    check(lib().stx_bands_layout(_np_ptr(sizes), sizes.size, _np_ptr(freqs), freqs.size, int(n_bins), int(channels),
                                 _np_ptr(fo), _np_ptr(fe), _np_ptr(bpf)))
    return fo, fe, bpf


class Bands:
    """Device band table of a RoFormer (src/roformer.cpp:394-411)."""

    def __init__(self, band_sizes, band_freqs, n_bins, channels):
        import numpy as np
        self.sizes = np.ascontiguousarray(band_sizes, dtype=np.int32)
        self.freqs = np.ascontiguousarray(band_freqs, dtype=np.int32)
        h = ctypes.c_void_p()
        check(lib().stx_bands_create(_np_ptr(self.sizes), self.sizes.size, _np_ptr(self.freqs), self.freqs.size,
                                     int(n_bins), int(channels), ctypes.byref(h)))
        self.handle = h
        self.n_bins = int(n_bins)
        self.channels = int(channels)
        self.total_feat = lib().stx_bands_total_feat(h)

    def close(self):
        if getattr(self, "handle", None):
            lib().stx_bands_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def gather(self, spec, n_frames, layout=T_MAJOR, out=None, stream=None):
        """spec: complex64 [batch, C, F, T] or [batch, C, T, F] -> float32 [batch, total_feat * T]."""
        import torch
        _require(spec, torch.complex64, "spec")
        batch = spec.shape[0]
        if out is None:
            out = torch.empty((batch, self.total_feat * n_frames), dtype=torch.float32, device=spec.device)
        check(lib().stx_band_gather(self.handle, _ptr(spec), batch, int(n_frames), int(layout), _ptr(out),
                                    _stream(stream)))
        return out

    def scatter_apply(self, masks, spec, n_frames, layout=T_MAJOR, zero_dc=False, out=None, stream=None):
        """masks: float32 [batch, S, total_feat * T]; spec: complex64 [batch, C, ...] ->
        complex64 [batch, S, C, ...]."""
        import torch
        _require(masks, torch.float32, "masks")
        _require(spec, torch.complex64, "spec")
        batch, S = masks.shape[0], masks.shape[1]
        if out is None:
            out = torch.empty((batch, S) + tuple(spec.shape[1:]), dtype=torch.complex64, device=spec.device)
        check(lib().stx_band_scatter_apply(self.handle, _ptr(masks), S, _ptr(spec), batch, int(n_frames), int(layout),
                                           int(bool(zero_dc)), _ptr(out), _stream(stream)))
        return out

    def rms_norm(self, feat, n_frames, gammas, eps=1e-24, out=None, stream=None):
        """The band split's RMSNorm of every band: feat float32 [batch, total_feat * T]; gammas: one
        float32 device tensor of dim_in(b) per band."""
        import torch
        _require(feat, torch.float32, "feat")
        if out is None:
            out = torch.empty_like(feat)
        table = (ctypes.c_void_p * max(len(gammas), 1))(*[g.data_ptr() for g in gammas])
        check(lib().stx_band_rms_norm(self.handle, _ptr(feat), feat.shape[0], int(n_frames), table, float(eps),
                                      _ptr(out), _stream(stream)))
        return out

    def mask_glu(self, heads, n_stems, n_frames, out=None, stream=None):
        """heads: n_stems * n_bands float32 device tensors [T, 2 * dim_in(b)] (stem-major) ->
        masks float32 [n_stems, total_feat * T]."""
        import torch
        if out is None:
            out = torch.empty((n_stems, self.total_feat * n_frames), dtype=torch.float32, device=heads[0].device)
        table = (ctypes.c_void_p * max(len(heads), 1))(*[h.data_ptr() for h in heads])
        check(lib().stx_band_mask_glu(self.handle, table, int(n_stems), int(n_frames), _ptr(out), _stream(stream)))
        return out


# ------------------------------------------------------------------------------- demix
CHUNK_FULL, CHUNK_REFLECT, CHUNK_ZERO = 0, 1, 2


class DemixGeometry(ctypes.Structure):
    """stx_demix_geometry (size tagged)."""
    _fields_ = [("size", ctypes.c_uint32), ("chunk", ctypes.c_int32), ("step", ctypes.c_int32),
                ("border", ctypes.c_int32), ("fade", ctypes.c_int32), ("reflect_border", ctypes.c_int32),
                ("len", ctypes.c_int64), ("padded_len", ctypes.c_int64), ("n_chunks", ctypes.c_int64)]


class Chunk(ctypes.Structure):
    _fields_ = [("start", ctypes.c_int64), ("length", ctypes.c_int32), ("pad_mode", ctypes.c_int32),
                ("fade_in", ctypes.c_int32), ("fade_out", ctypes.c_int32)]


SEPARATE_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                               ctypes.c_void_p, ctypes.c_void_p)
PROGRESS_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32)
CANCEL_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p)


class SeparateOptions(ctypes.Structure):
    """stx_separate_options (size tagged: size is set to the struct's size)."""
    _fields_ = [("size", ctypes.c_uint32), ("shifts", ctypes.c_int32), ("overlap", ctypes.c_float),
                ("seed", ctypes.c_uint32), ("progress", PROGRESS_FN), ("should_cancel", CANCEL_FN),
                ("user", ctypes.c_void_p)]

    def __init__(self, shifts=0, overlap=-1.0, seed=0, progress=None, should_cancel=None, user=None):
        super().__init__(ctypes.sizeof(SeparateOptions), shifts, overlap, seed,
                         progress if progress is not None else PROGRESS_FN(),
                         should_cancel if should_cancel is not None else CANCEL_FN(), user)


def demix_step(chunk, num_overlap, overlap=-1.0):
    return lib().stx_demix_step(int(chunk), int(num_overlap), float(overlap))


DEMIX_ROFORMER, DEMIX_MSST = 0, 1
TFC_MSST, TFC_UVR = 0, 1


def demix_plan(length, chunk, step, rules=DEMIX_ROFORMER):
    """(geometry dict, numpy structured chunk table) of the overlap-add demix (host only)."""
    import numpy as np
    g = DemixGeometry()
    g.size = ctypes.sizeof(DemixGeometry)
    check(lib().stx_demix_plan_rules(int(length), int(chunk), int(step), int(rules), ctypes.byref(g), None, 0))
    table = (Chunk * max(1, g.n_chunks))()
    check(lib().stx_demix_plan_rules(int(length), int(chunk), int(step), int(rules), ctypes.byref(g), table,
                                     g.n_chunks))
    geom = {f: getattr(g, f) for f, _ in DemixGeometry._fields_ if f != "size"}
    arr = np.array([(c.start, c.length, c.pad_mode, c.fade_in, c.fade_out) for c in table[: g.n_chunks]],
                   dtype=[("start", np.int64), ("length", np.int32), ("pad_mode", np.int32),
                          ("fade_in", np.int32), ("fade_out", np.int32)])
    return geom, arr


def demix_window(chunk, rules=DEMIX_ROFORMER):
    import numpy as np
    w = np.zeros(chunk, dtype=np.float32)
    check(lib().stx_demix_window_rules(int(chunk), int(rules), _np_ptr(w)))
    return w


class Demix:
    """Device plan of the overlap-add demix for one input length."""

    def __init__(self, length, channels, chunk, step, rules=DEMIX_ROFORMER):
        h = ctypes.c_void_p()
        check(lib().stx_demix_create_rules(int(length), int(channels), int(chunk), int(step), int(rules),
                                           ctypes.byref(h)))
        self.handle = h
        self.length, self.channels, self.chunk, self.step = int(length), int(channels), int(chunk), int(step)
        self.n_chunks = lib().stx_demix_n_chunks(h)

    def close(self):
        if getattr(self, "handle", None):
            lib().stx_demix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def chunks(self, mix, first=0, count=None, out=None, stream=None):
        """mix float32 [C, len] -> parts float32 [count, C, chunk]."""
        import torch
        _require(mix, torch.float32, "mix")
        count = self.n_chunks - first if count is None else count
        if out is None:
            out = torch.empty((count, self.channels, self.chunk), dtype=torch.float32, device=mix.device)
        check(lib().stx_demix_chunks(self.handle, _ptr(mix), int(first), int(count), _ptr(out), _stream(stream)))
        return out

    def overlap_add(self, y, out=None, stream=None):
        """y float32 [n_chunks, S, C, chunk] -> float32 [S, C, len]."""
        import torch
        _require(y, torch.float32, "y")
        S = y.shape[1]
        if out is None:
            out = torch.empty((S, self.channels, self.length), dtype=torch.float32, device=y.device)
        check(lib().stx_demix_overlap_add(self.handle, _ptr(y), int(S), _ptr(out), _stream(stream)))
        return out


class UvrDemix:
    """Device plan of UVR's SeperateMDX.demix chunking (TFC-TDF "uvr_mdx") for one input length."""

    def __init__(self, length, channels, chunk, n_fft, overlap=-1.0):
        h = ctypes.c_void_p()
        check(lib().stx_uvr_demix_create(int(length), int(channels), int(chunk), int(n_fft), float(overlap),
                                         ctypes.byref(h)))
        self.handle = h
        self.length, self.channels, self.chunk = int(length), int(channels), int(chunk)
        self.n_chunks = lib().stx_uvr_demix_n_chunks(h)
        M, st, tr = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
        check(lib().stx_uvr_demix_geometry(h, ctypes.byref(M), ctypes.byref(st), ctypes.byref(tr)))
        self.padded_len, self.step, self.trim = M.value, st.value, tr.value

    def close(self):
        if getattr(self, "handle", None):
            lib().stx_uvr_demix_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def chunks(self, mix, first=0, count=None, out=None, stream=None):
        import torch
        _require(mix, torch.float32, "mix")
        count = self.n_chunks - first if count is None else count
        if out is None:
            out = torch.empty((count, self.channels, self.chunk), dtype=torch.float32, device=mix.device)
        check(lib().stx_uvr_demix_chunks(self.handle, _ptr(mix), int(first), int(count), _ptr(out), _stream(stream)))
        return out

    def overlap_add(self, y, out=None, stream=None):
        import torch
        _require(y, torch.float32, "y")
        S = y.shape[1]
        if out is None:
            out = torch.empty((S, self.channels, self.length), dtype=torch.float32, device=y.device)
        check(lib().stx_uvr_demix_overlap_add(self.handle, _ptr(y), int(S), _ptr(out), _stream(stream)))
        return out


def tfc_tdf_separate(mix, chunk, n_fft, chunking, n_stems, separate, num_overlap=4, compensate=1.0,
                     complement=False, batch=4, shifts=0, overlap=-1.0, progress=None, should_cancel=None,
                     stream=None):
    """TFCTDF::separate around a Python separator (same callback as demix_track)."""
    import torch
    _require(mix, torch.float32, "mix")
    C, L = mix.shape
    ws_bytes = lib().stx_tfc_tdf_separate_workspace_size(C, L, int(chunk), int(n_fft), int(chunking),
                                                         int(num_overlap), float(overlap), int(n_stems), int(batch))
    ws = workspace(max(ws_bytes, 256), mix.device)
    out = torch.empty((n_stems + (1 if complement else 0), C, L), dtype=torch.float32, device=mix.device)

    def sep(user, parts, first, count, y, st):
        try:
            return int(separate(parts, first, count, y, st))
        except Exception:
            import traceback
            traceback.print_exc()
            return -1

    def prog(user, done, total):
        progress(done, total)

    def canc(user):
        return 1 if should_cancel() else 0

    cb = SEPARATE_FN(sep)
    opt = SeparateOptions(int(shifts), float(overlap), 0, PROGRESS_FN(prog) if progress else PROGRESS_FN(),
                          CANCEL_FN(canc) if should_cancel else CANCEL_FN(), None)
    check(lib().stx_tfc_tdf_separate(_ptr(mix), C, L, int(chunk), int(n_fft), int(chunking), int(num_overlap),
                                     int(n_stems), float(compensate), int(bool(complement)), int(batch),
                                     ctypes.cast(cb, ctypes.c_void_p), None, ctypes.byref(opt), _ptr(out), _ptr(ws),
                                     ws.numel() * 4, _stream(stream)))
    return out


def demix_track(mix, chunk, num_overlap, n_stems, separate, complement=False, sample_rate=44100, batch=8,
                shifts=0, overlap=-1.0, seed=0, progress=None, should_cancel=None, stream=None):
    """RoFormer::separate around a Python separator.

    separate(parts_ptr, first, count, y_ptr, stream_ptr) -> int gets raw device pointers:
    parts [count][C][chunk] and y [count][n_stems][C][chunk] float32."""
    import torch
    _require(mix, torch.float32, "mix")
    C, L = mix.shape
    step = demix_step(chunk, num_overlap, overlap)
    ws_bytes = lib().stx_demix_track_workspace_size(C, L, chunk, max(step, 1), n_stems, batch, shifts, sample_rate)
    ws = workspace(max(ws_bytes, 4), mix.device)
    out = torch.empty((n_stems + (1 if complement else 0), C, L), dtype=torch.float32, device=mix.device)

    def sep(user, parts, first, count, y, st):
        try:
            return int(separate(parts, first, count, y, st))
        except Exception:
            import traceback
            traceback.print_exc()
            return -1

    def prog(user, done, total):
        progress(done, total)

    def canc(user):
        return 1 if should_cancel() else 0

    cb = SEPARATE_FN(sep)
    opt = SeparateOptions(int(shifts), float(overlap), int(seed),
                          PROGRESS_FN(prog) if progress else PROGRESS_FN(),
                          CANCEL_FN(canc) if should_cancel else CANCEL_FN(), None)
    check(lib().stx_demix_track(_ptr(mix), C, L, int(chunk), int(num_overlap), int(n_stems), int(bool(complement)),
                                int(sample_rate), int(batch), ctypes.cast(cb, ctypes.c_void_p), None,
                                ctypes.byref(opt), _ptr(out), _ptr(ws), ws.numel() * 4, _stream(stream)))
    return out


# ---------------------------------------------------------------------------- resampling
class Resampler:
    """st::resample_planar (src/audio.h:17-59) on the device for one pair of rates."""

    def __init__(self, src_rate, dst_rate):
        h = ctypes.c_void_p()
        check(lib().stx_resampler_create(int(src_rate), int(dst_rate), ctypes.byref(h)))
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            lib().stx_resampler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def length(self, n):
        return lib().stx_resample_length(self.handle, int(n))

    def __call__(self, x, out=None, stream=None):
        """x float32 [C, n] -> [C, length(n)]."""
        import torch
        _require(x, torch.float32, "x")
        C, n = x.shape
        if out is None:
            out = torch.empty((C, self.length(n)), dtype=torch.float32, device=x.device)
        check(lib().stx_resample(self.handle, _ptr(x), C, n, _ptr(out), _stream(stream)))
        return out


# ------------------------------------------------------------ libstems separate() data path
AUDIO_PLANAR, AUDIO_INTERLEAVED = 0, 1
MODEL_SEPARATE_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)


class AudioView(ctypes.Structure):
    """stx_audio_view (size tagged), over device samples."""
    _fields_ = [("size", ctypes.c_uint32), ("samples", ctypes.c_void_p), ("n_samples", ctypes.c_uint64),
                ("n_channels", ctypes.c_uint32), ("sample_rate", ctypes.c_uint32), ("layout", ctypes.c_int32),
                ("reserved", ctypes.c_uint32)]


def audio_view(samples, n_samples, n_channels, sample_rate, layout):
    v = AudioView()
    v.size = ctypes.sizeof(AudioView)
    v.samples = samples if isinstance(samples, int) or samples is None else _ptr(samples)
    v.n_samples, v.n_channels, v.sample_rate, v.layout = int(n_samples), int(n_channels), int(sample_rate), int(layout)
    return v


def separate_audio(samples, n_channels, sample_rate, layout, model_channels, model_rate, n_sources, separate,
                   to_model=None, from_model=None, shifts=0, overlap=-1.0, seed=0, progress=None,
                   should_cancel=None, stream=None):
    """libstems separate() (src/libstems.cpp:135-196) around a Python model separate.

    samples: float32 device tensor, planar [n_channels, n] or interleaved [n, n_channels] (flat
    is fine). separate(audio_ptr, channels, length, options_ptr, stems_ptr, stream_ptr) -> status
    gets raw device pointers: audio [channels][length] and stems [n_sources][channels][length].
    Returns float32 [n_sources, model_channels, n]."""
    import torch
    _require(samples, torch.float32, "samples")
    n = samples.numel() // int(n_channels)
    view = audio_view(samples, n, n_channels, sample_rate, layout)
    need = lib().stx_separate_audio_workspace_size(ctypes.byref(view), int(model_channels), int(model_rate),
                                                   int(n_sources))
    ws = workspace(max(need, 4), samples.device)
    out = torch.empty((int(n_sources), int(model_channels), n), dtype=torch.float32, device=samples.device)

    def sep(user, audio, channels, length, opt, stems, st):
        try:
            return int(separate(audio, channels, length, opt, stems, st))
        except Exception:
            import traceback
            traceback.print_exc()
            return STATUS_RUNTIME_ERROR

    def prog(user, done, total):
        progress(done, total)

    def canc(user):
        return 1 if should_cancel() else 0

    cb = MODEL_SEPARATE_FN(sep)
    opt = SeparateOptions(int(shifts), float(overlap), int(seed),
                          PROGRESS_FN(prog) if progress else PROGRESS_FN(),
                          CANCEL_FN(canc) if should_cancel else CANCEL_FN(), None)
    h = lambda r: None if r is None else r.handle
    check(lib().stx_separate_audio(ctypes.byref(view), int(model_channels), int(model_rate), int(n_sources),
                                   h(to_model), h(from_model), ctypes.cast(cb, ctypes.c_void_p), None,
                                   ctypes.byref(opt), _ptr(out), _ptr(ws), ws.numel() * 4, _stream(stream)))
    return out


# ------------------------------------------------------------ HTDemucs pre/post + split
def _norm_ws(n, device, workspace):
    import torch
    need = lib().stx_htdemucs_norm_workspace_size(int(n))
    if workspace is None:
        workspace = torch.empty((need + 7) // 8, dtype=torch.float64, device=device)
    return workspace, workspace.numel() * workspace.element_size()


def htdemucs_cac_normalize(spec, out=None, stats=None, workspace=None, stream=None):
    """spec: complex64 [C, F, T] (f-major) -> (mag float32 [2C, F, T], stats float64 [2])."""
    import torch
    _require(spec, torch.complex64, "spec")
    C, F, T = spec.shape
    out = torch.empty((2 * C, F, T), dtype=torch.float32, device=spec.device) if out is None else out
    stats = torch.empty(2, dtype=torch.float64, device=spec.device) if stats is None else stats
    ws, nb = _norm_ws(2 * C * F * T, spec.device, workspace)
    check(lib().stx_htdemucs_cac_normalize(_ptr(spec), C, F, T, _ptr(out), _ptr(stats), _ptr(ws), nb, _stream(stream)))
    return out, stats


def htdemucs_wave_normalize(x, out=None, stats=None, workspace=None, stream=None):
    import torch
    _require(x, torch.float32, "x")
    out = torch.empty_like(x) if out is None else out
    stats = torch.empty(2, dtype=torch.float64, device=x.device) if stats is None else stats
    ws, nb = _norm_ws(x.numel(), x.device, workspace)
    check(lib().stx_htdemucs_wave_normalize(_ptr(x), x.numel(), _ptr(out), _ptr(stats), _ptr(ws), nb, _stream(stream)))
    return out, stats


def htdemucs_mix_normalize(mix, out=None, stats=None, workspace=None, stream=None):
    """mix float32 [C, len] -> (normalised mix, stats {ref_mean, ref_std})."""
    import torch
    _require(mix, torch.float32, "mix")
    C, L = mix.shape
    out = torch.empty_like(mix) if out is None else out
    stats = torch.empty(2, dtype=torch.float64, device=mix.device) if stats is None else stats
    ws, nb = _norm_ws(L, mix.device, workspace)
    check(lib().stx_htdemucs_mix_normalize(_ptr(mix), C, L, _ptr(out), _ptr(stats), _ptr(ws), nb, _stream(stream)))
    return out, stats


def htdemucs_cac_denormalize(ox, stats, out=None, stream=None):
    """ox float32 [S, 2C, F, T] -> complex64 [S, C, F, T]."""
    import torch
    _require(ox, torch.float32, "ox")
    S, C2, F, T = ox.shape
    out = torch.empty((S, C2 // 2, F, T), dtype=torch.complex64, device=ox.device) if out is None else out
    check(lib().stx_htdemucs_cac_denormalize(_ptr(ox), S, C2 // 2, F, T, _ptr(stats), _ptr(out), _stream(stream)))
    return out


def htdemucs_time_add(xt, y, stats, out=None, stream=None):
    import torch
    out = torch.empty_like(xt) if out is None else out
    check(lib().stx_htdemucs_time_add(_ptr(xt), _ptr(y), xt.numel(), _ptr(stats), _ptr(out), _stream(stream)))
    return out


def htdemucs_split_plan(length, segment, overlap=0.25):
    st, n = ctypes.c_int(), ctypes.c_int()
    check(lib().stx_htdemucs_split_plan(int(length), int(segment), float(overlap), ctypes.byref(st), ctypes.byref(n)))
    return st.value, n.value


def htdemucs_segments(buf, offset, length, segment, stride, first=0, count=None, out=None, stream=None):
    """Padded chunk inputs of the view [offset, offset + length) of buf float32 [C, total]."""
    import torch
    _require(buf, torch.float32, "buf")
    C, total = buf.shape
    n = (length + stride - 1) // stride
    count = n - first if count is None else count
    out = torch.empty((count, C, segment), dtype=torch.float32, device=buf.device) if out is None else out
    check(lib().stx_htdemucs_segments(_ptr(buf), C, total, int(offset), int(length), int(segment), int(stride),
                                      int(first), int(count), _ptr(out), _stream(stream)))
    return out


def htdemucs_split_overlap_add(y, length, stride, out=None, stream=None):
    """y float32 [n_chunks, tracks, segment] -> [tracks, length]."""
    import torch
    _require(y, torch.float32, "y")
    n, tracks, segment = y.shape
    out = torch.empty((tracks, length), dtype=torch.float32, device=y.device) if out is None else out
    check(lib().stx_htdemucs_split_overlap_add(_ptr(y), tracks, int(length), segment, int(stride), _ptr(out),
                                               _stream(stream)))
    return out


MODEL_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
                            ctypes.c_void_p, ctypes.c_void_p)


def htdemucs_separate(mix, segment, n_sources, bag_weights, forward, sample_rate=44100, batch=4, shifts=0,
                      overlap=-1.0, seed=0, progress=None, should_cancel=None, stream=None):
    """HTDemucs::separate around a Python model.

    forward(model, parts_ptr, count, y_ptr, stream_ptr) -> int gets raw device pointers: parts
    [count][C][segment] and y [count][n_sources][C][segment] float32. bag_weights: host
    [n_models][n_sources]."""
    import numpy as np
    import torch
    _require(mix, torch.float32, "mix")
    C, L = mix.shape
    bag = np.ascontiguousarray(bag_weights, dtype=np.float32)
    n_models = bag.shape[0]
    ws_bytes = lib().stx_htdemucs_separate_workspace_size(C, L, int(segment), int(n_sources), int(batch),
                                                          int(shifts), int(sample_rate), float(overlap))
    ws = workspace(max(ws_bytes, 4), mix.device)
    out = torch.empty((n_sources, C, L), dtype=torch.float32, device=mix.device)

    def fwd(user, model, parts, count, y, st):
        try:
            return int(forward(model, parts, count, y, st))
        except Exception:
            import traceback
            traceback.print_exc()
            return -1

    def prog(user, done, total):
        progress(done, total)

    def canc(user):
        return 1 if should_cancel() else 0

    cb = MODEL_FN(fwd)
    opt = SeparateOptions(int(shifts), float(overlap), int(seed),
                          PROGRESS_FN(prog) if progress else PROGRESS_FN(),
                          CANCEL_FN(canc) if should_cancel else CANCEL_FN(), None)
    check(lib().stx_htdemucs_separate(_ptr(mix), C, L, int(segment), int(n_sources), n_models, _np_ptr(bag),
                                      int(sample_rate), int(batch), ctypes.cast(cb, ctypes.c_void_p), None,
                                      ctypes.byref(opt), _ptr(out), _ptr(ws), ws.numel() * 4, _stream(stream)))
    return out


# --------------------------------------------------------------------------------- ops
class Tensor(ctypes.Structure):
    """stx_tensor: ggml's view of a tensor (ne[0] fastest, byte strides nb)."""
    _fields_ = [("data", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_int64 * 4)]


def as_tensor(t):
    """stx_tensor of a float32 device tensor of up to 4 dims: torch's last dim is ne[0]."""
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("operands must be CUDA (HIP) tensors")
    if t.dtype != torch.float32:
        raise TypeError(f"operands must be float32, got {t.dtype}")
    if t.dim() > 4:
        raise ValueError("at most 4 dimensions")
    shape, strides = list(t.shape)[::-1], list(t.stride())[::-1]
    d = Tensor()
    d.data = t.data_ptr()
    for i in range(4):
        if i < len(shape):
            d.ne[i] = shape[i]
            d.nb[i] = 4 * strides[i]
        else:                                   # missing leading torch dims: extent 1
            d.ne[i] = 1
            d.nb[i] = d.nb[i - 1] * d.ne[i - 1] if i else 4
    if t.dim() == 0 or shape[0] == 1:
        d.nb[0] = 4
    return d


def _t(t):
    return None if t is None else ctypes.byref(as_tensor(t))


def _out(out, like):
    import torch
    return torch.empty_like(like, memory_format=torch.contiguous_format) if out is None else out


def group_norm_workspace_size(x, n_groups):
    return lib().stx_group_norm_workspace_size(ctypes.byref(as_tensor(x)), int(n_groups))


def group_norm(x, n_groups, eps=1e-5, weight=None, bias=None, gelu=False, out=None, workspace=None, stream=None):
    """ggml_group_norm(x, n_groups, eps) [* weight + bias] [-> gelu]; weight/bias repeat into x."""
    out = _out(out, x)
    need = group_norm_workspace_size(x, n_groups)
    if workspace is None:
        workspace = globals()["workspace"](need, x.device)
    check(lib().stx_group_norm(_t(x), _t(out), int(n_groups), float(eps), _t(weight), _t(bias), int(bool(gelu)),
                               _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(stream)))
    return out


def group_norm_noalloc(x, n_groups, eps=1e-5, weight=None, bias=None, gelu=False, out=None, stream=None):
    """group_norm on the library's static per-GPU scratch (stx_group_norm_noalloc): no workspace."""
    out = _out(out, x)
    check(lib().stx_group_norm_noalloc(_t(x), _t(out), int(n_groups), float(eps), _t(weight), _t(bias),
                                       int(bool(gelu)), _stream(stream)))
    return out


def grid_sync_fallbacks(workspace=None):
    """Sticky count of grid-synchronised blocks that recomputed their statistics on `workspace`
    (None: the static scratch of group_norm_noalloc on the current GPU)."""
    n = ctypes.c_uint32(0)
    check(lib().stx_grid_sync_fallbacks(None if workspace is None else _ptr(workspace), ctypes.byref(n)))
    return int(n.value)


def norm(x, eps=1e-5, weight=None, bias=None, out=None, stream=None):
    """ggml_norm over the last torch dim (ne0) [* weight + bias]."""
    out = _out(out, x)
    if weight is None and bias is None:
        check(lib().stx_norm(_t(x), _t(out), float(eps), _stream(stream)))
    else:
        check(lib().stx_norm_affine(_t(x), _ptr(weight), _ptr(bias), _t(out), float(eps), _stream(stream)))
    return out


def rms_norm(x, eps=1e-24, gamma=None, out=None, stream=None):
    """ggml_rms_norm over the last torch dim (ne0) [* gamma]."""
    out = _out(out, x)
    if gamma is None:
        check(lib().stx_rms_norm(_t(x), _t(out), float(eps), _stream(stream)))
    else:
        check(lib().stx_rms_norm_mul(_t(x), _ptr(gamma), _t(out), float(eps), _stream(stream)))
    return out


def soft_max_ext(x, scale=1.0, mask=None, max_bias=0.0, out=None, stream=None):
    out = _out(out, x)
    check(lib().stx_soft_max_ext(_t(x), _t(mask), _t(out), float(scale), float(max_bias), _stream(stream)))
    return out


def gelu_erf(x, bias=None, out=None, stream=None):
    """ggml_gelu_erf(x), or ggml_gelu_erf(ggml_add(x, bias)) fused."""
    out = _out(out, x)
    if bias is None:
        check(lib().stx_gelu_erf(_t(x), _t(out), _stream(stream)))
    else:
        check(lib().stx_add_gelu_erf(_t(x), _t(bias), _t(out), _stream(stream)))
    return out


def glu(x, dim, out=None, stream=None):
    """GLU along ggml dimension dim (0 = torch's last dim)."""
    import torch
    if out is None:
        shape = list(x.shape)
        shape[x.dim() - 1 - dim] //= 2
        out = torch.empty(shape, dtype=x.dtype, device=x.device)
    check(lib().stx_glu(_t(x), _t(out), int(dim), _stream(stream)))
    return out


def add(a, b, out=None, stream=None):
    out = _out(out, a)
    check(lib().stx_add(_t(a), _t(b), _t(out), _stream(stream)))
    return out


def mul(a, b, out=None, stream=None):
    out = _out(out, a)
    check(lib().stx_mul(_t(a), _t(b), _t(out), _stream(stream)))
    return out


def mul_add(x, h, s, out=None, stream=None):
    """x + h * s (LayerScale + residual), rounded like ggml_add(x, ggml_mul(h, s))."""
    out = _out(out, x)
    check(lib().stx_mul_add(_t(x), _t(h), _t(s), _t(out), _stream(stream)))
    return out


def glu_mul_add(x, a, dim, s, out=None, stream=None):
    """x + glu(a along ggml dimension dim) * s: GLU + LayerScale + residual in one kernel."""
    out = _out(out, x)
    check(lib().stx_glu_mul_add(_t(x), _t(a), int(dim), _t(s), _t(out), _stream(stream)))
    return out


def rope_ext(x, pos, n_dims, mode=0, freq_base=10000.0, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0,
             n_ctx_orig=0, beta_fast=0.0, beta_slow=0.0, out=None, stream=None):
    """ggml_rope_ext; pos is an int32 device tensor with one entry per ne2 index."""
    import torch
    _require(pos, torch.int32, "pos")
    out = _out(out, x)
    check(lib().stx_rope_ext(_t(x), _ptr(pos), _t(out), int(n_dims), int(mode), int(n_ctx_orig), float(freq_base),
                             float(freq_scale), float(ext_factor), float(attn_factor), float(beta_fast),
                             float(beta_slow), _stream(stream)))
    return out


# ------------------------------------------------------------------------ layout glue
def qkv_rope_split(qkv, pos, n_head, freq_base=10000.0, freq_scale=1.0, attn_factor=1.0, out=None, stream=None):
    """The q/k/v split of RoFormer attention, fused with RoPE and the permutes.

    qkv: torch (batch, N, 3 * n_head * dh) = ggml [3*H*dh, N, batch]; pos: int32 device (N,).
    Returns (q, k, vt) with torch shapes (batch, H, N, dh), (batch, H, N, dh), (batch, H, dh, N).
    """
    import torch
    _require(pos, torch.int32, "pos")
    batch, N, width = qkv.shape
    dh = width // (3 * n_head)
    if out is None:
        q = torch.empty((batch, n_head, N, dh), dtype=qkv.dtype, device=qkv.device)
        k = torch.empty_like(q)
        vt = torch.empty((batch, n_head, dh, N), dtype=qkv.dtype, device=qkv.device)
    else:
        q, k, vt = out
    check(lib().stx_qkv_rope_split(_t(qkv), _ptr(pos), int(n_head), float(freq_base), float(freq_scale),
                                   float(attn_factor), _t(q), _t(k), _t(vt), _stream(stream)))
    return q, k, vt


def merge_heads(o, gates=None, out=None, stream=None):
    """cont(permute(o, 0, 2, 1, 3)) [* gates]: torch (batch, H, N, dh) -> (batch, N, H, dh).

    gates: torch (batch, N, H, 1) (ggml [1, H, N, batch]) or None.
    """
    import torch
    if out is None:
        b, H, N, dh = o.shape
        out = torch.empty((b, N, H, dh), dtype=o.dtype, device=o.device)
    check(lib().stx_merge_heads(_t(o), _t(gates), _t(out), _stream(stream)))
    return out


def ggml_permuted_shape(ne, axes):
    """ne of ggml_permute(a, *axes) given a's ne (ggml order): a's dim i becomes dim axes[i]."""
    out = [1, 1, 1, 1]
    for i, ax in enumerate(axes):
        out[ax] = ne[i]
    return out


def cont_permute(x, axes, out=None, stream=None):
    """ggml_cont(ggml_permute(x, *axes)) on a torch tensor of up to 4 dims (ggml order = reversed)."""
    import torch
    if out is None:
        ne = list(x.shape)[::-1] + [1] * (4 - x.dim())
        pne = ggml_permuted_shape(ne, axes)
        out = torch.empty(pne[::-1], dtype=x.dtype, device=x.device)
    check(lib().stx_cont_permute(_t(x), int(axes[0]), int(axes[1]), int(axes[2]), int(axes[3]), _t(out),
                                 _stream(stream)))
    return out


def concat(tensors, dim, out=None, stream=None):
    """ggml_concat of a list of tensors along ggml dimension dim (0 = torch's last dim)."""
    import torch
    if out is None:
        ref = tensors[0]
        shape = list(ref.shape)
        tdim = ref.dim() - 1 - dim
        shape[tdim] = sum(t.shape[tdim] for t in tensors)
        out = torch.empty(shape, dtype=ref.dtype, device=ref.device)
    descs = [as_tensor(t) for t in tensors]
    arr = (ctypes.c_void_p * len(descs))(*[ctypes.addressof(d) for d in descs])
    check(lib().stx_concat(arr, len(descs), int(dim), _t(out), _stream(stream)))
    return out
