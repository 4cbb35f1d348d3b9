// stx_st.hpp — drop-in C++ replacement for the transforms of the reference's src/stft.h.
//
// Same names, signatures, layouts and exceptions as namespace st of src/stft.h:
//   class FFT                 src/stft.h:19-55   (explicit FFT(int n), size(), run(a, inverse))
//   htdemucs_spec             src/stft.h:79-103  (spec [F = n/2][T] f-major, T returned in n_frames)
//   htdemucs_ispec            src/stft.h:106-140
//   torch_stft                src/stft.h:146-164 (spec [F = n/2 + 1][T] f-major)
//   torch_istft               src/stft.h:167-197 (hop * (T - 1) samples)
// Each call runs the gfx950 kernels of libstx.so on host data: the input is copied to the
// device, transformed there in complex64, and copied back as std::complex<double> at the edge
// (the reference's cplx). A maintainer switches a translation unit over with
//     #include "stx_st.hpp"
//     namespace st = stx::st;
// (or by replacing the include of stft.h for the transforms; reflect_pad and hann_periodic
// stay in stft.h for the code that uses them as host utilities). std::invalid_argument and
// std::runtime_error are thrown where the reference throws them; a HIP failure is a
// std::runtime_error. Calls run on the null stream and return after it has finished, like the
// reference's synchronous functions. Link with -lstx.
#pragma once

#include <hip/hip_runtime_api.h>

#include <complex>
#include <cstddef>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "stx.h"

namespace stx {
namespace st {

using cplx = std::complex<double>;

namespace detail {

[[noreturn]] inline void raise(stx_status s) {
    const std::string msg = stx_last_error();
    if (s == STX_STATUS_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

inline void check(stx_status s) {
    if (s != STX_STATUS_OK) raise(s);
}

inline void hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Device buffer owned for the duration of one call.
class Buffer {
public:
    explicit Buffer(size_t bytes) {
        if (bytes) hip(hipMalloc(&p_, bytes), "hipMalloc");
    }
    ~Buffer() {
        if (p_) (void)hipFree(p_);
    }
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;
    template <class T>
    T* as() const {
        return static_cast<T*>(p_);
    }

private:
    void* p_ = nullptr;
};

inline void to_device(void* dst, const void* src, size_t bytes) {
    if (bytes) hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

inline void to_host(void* dst, const void* src, size_t bytes) {
    if (bytes) hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

inline void sync() { hip(hipStreamSynchronize(nullptr), "hipStreamSynchronize"); }

// complex<double> host data <-> complex64 device data.
inline std::vector<float> narrow(const cplx* a, size_t n) {
    std::vector<float> f(2 * n);
    for (size_t i = 0; i < n; i++) {
        f[2 * i] = (float)a[i].real();
        f[2 * i + 1] = (float)a[i].imag();
    }
    return f;
}

inline void widen(const std::vector<float>& f, cplx* a, size_t n) {
    for (size_t i = 0; i < n; i++) a[i] = cplx(f[2 * i], f[2 * i + 1]);
}

}  // namespace detail

// st::FFT: a device plan (window and twiddle tables) for n points. Throws
// std::invalid_argument unless n is a power of two >= 2, like the reference; sizes this
// build has no kernels for (outside 16..8192) throw std::runtime_error.
class FFT {
public:
    explicit FFT(int n) {
        stx_fft* h = nullptr;
        detail::check(stx_fft_create(n, &h));
        h_.reset(h, stx_fft_destroy);
        n_ = n;
    }
    int size() const { return n_; }

    // In-place, unnormalised; inverse uses conjugate twiddles (no 1/n). a.size() may be any
    // multiple of n: each block of n values is one transform.
    void run(std::vector<cplx>& a, bool inverse) const {
        if (a.size() % (size_t)n_) throw std::invalid_argument("FFT input is not a multiple of the FFT size");
        const size_t batch = a.size() / n_;
        if (!batch) return;
        std::vector<float> f = detail::narrow(a.data(), a.size());
        detail::Buffer d(f.size() * sizeof(float));
        detail::to_device(d.as<float>(), f.data(), f.size() * sizeof(float));
        detail::check(stx_fft_run(h_.get(), d.as<float>(), (int)batch, inverse ? 1 : 0, nullptr));
        detail::to_host(f.data(), d.as<float>(), f.size() * sizeof(float));
        detail::widen(f, a.data(), a.size());
    }

    const stx_fft* handle() const { return h_.get(); }

private:
    std::shared_ptr<stx_fft> h_;
    int n_ = 0;
};

// HTDemucs._spec for one channel: `len` samples -> [F = n/2][T] complex, f-major.
inline std::vector<cplx> htdemucs_spec(const FFT& fft, const float* x, int len, int& n_frames) {
    const int T = stx_htdemucs_frames(fft.size(), len);
    if (T < 0) detail::raise(STX_STATUS_INVALID_ARGUMENT);
    const size_t F = (size_t)fft.size() / 2, bins = F * (size_t)T;
    detail::Buffer dx(sizeof(float) * (size_t)len), ds(2 * sizeof(float) * bins);
    detail::to_device(dx.as<float>(), x, sizeof(float) * (size_t)len);
    detail::check(stx_htdemucs_spec(fft.handle(), dx.as<float>(), 1, len, ds.as<float>(), STX_SPEC_F_MAJOR, nullptr));
    std::vector<float> f(2 * bins);
    detail::to_host(f.data(), ds.as<float>(), f.size() * sizeof(float));
    std::vector<cplx> spec(bins);
    detail::widen(f, spec.data(), bins);
    n_frames = T;
    return spec;
}

// HTDemucs._ispec for one channel: spec [F = n/2][T] f-major -> `length` samples.
inline std::vector<float> htdemucs_ispec(const FFT& fft, const std::vector<cplx>& spec, int n_frames, int length) {
    const size_t bins = (size_t)fft.size() / 2 * (size_t)(n_frames > 0 ? n_frames : 0);
    if (n_frames < 0 || spec.size() < bins) throw std::invalid_argument("spectrum smaller than n/2 x n_frames");
    std::vector<float> f = detail::narrow(spec.data(), bins);
    detail::Buffer ds(f.size() * sizeof(float)), dy(sizeof(float) * (size_t)(length > 0 ? length : 0));
    detail::to_device(ds.as<float>(), f.data(), f.size() * sizeof(float));
    detail::check(stx_htdemucs_ispec(fft.handle(), ds.as<float>(), 1, n_frames, length, dy.as<float>(),
                                     STX_SPEC_F_MAJOR, nullptr));
    std::vector<float> y((size_t)(length > 0 ? length : 0));
    detail::to_host(y.data(), dy.as<float>(), y.size() * sizeof(float));
    return y;
}

// torch.stft for one channel (periodic Hann, center, reflect, onesided): [F = n/2 + 1][T]
// f-major with T = len / hop + 1.
inline std::vector<cplx> torch_stft(const FFT& fft, const float* x, int len, int hop, bool normalized,
                                    int& n_frames) {
    const int T = stx_torch_stft_frames(len, hop);
    if (T < 0) detail::raise(STX_STATUS_INVALID_ARGUMENT);
    const size_t F = (size_t)fft.size() / 2 + 1, bins = F * (size_t)T;
    detail::Buffer dx(sizeof(float) * (size_t)len), ds(2 * sizeof(float) * bins);
    detail::to_device(dx.as<float>(), x, sizeof(float) * (size_t)len);
    detail::check(stx_torch_stft(fft.handle(), dx.as<float>(), 1, len, hop, normalized ? 1 : 0, ds.as<float>(),
                                 STX_SPEC_F_MAJOR, nullptr));
    std::vector<float> f(2 * bins);
    detail::to_host(f.data(), ds.as<float>(), f.size() * sizeof(float));
    std::vector<cplx> spec(bins);
    detail::widen(f, spec.data(), bins);
    n_frames = T;
    return spec;
}

// torch.istft matching torch_stft, length = None: hop * (T - 1) samples.
inline std::vector<float> torch_istft(const FFT& fft, const std::vector<cplx>& spec, int n_frames, int hop,
                                      bool normalized) {
    const size_t bins = ((size_t)fft.size() / 2 + 1) * (size_t)(n_frames > 0 ? n_frames : 0);
    if (n_frames < 0 || spec.size() < bins) throw std::invalid_argument("spectrum smaller than (n/2 + 1) x n_frames");
    const long long length = n_frames > 0 ? (long long)hop * (n_frames - 1) : 0;
    std::vector<float> f = detail::narrow(spec.data(), bins);
    detail::Buffer ds(f.size() * sizeof(float)), dy(sizeof(float) * (size_t)(length > 0 ? length : 0));
    detail::to_device(ds.as<float>(), f.data(), f.size() * sizeof(float));
    detail::check(stx_torch_istft(fft.handle(), ds.as<float>(), 1, n_frames, hop, normalized ? 1 : 0, dy.as<float>(),
                                  STX_SPEC_F_MAJOR, nullptr));
    std::vector<float> y((size_t)(length > 0 ? length : 0));
    detail::to_host(y.data(), dy.as<float>(), y.size() * sizeof(float));
    detail::sync();
    return y;
}

}  // namespace st
}  // namespace stx
