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
// (the reference's cplx). The device buffers and a pinned staging buffer belong to the FFT
// object and are reused by every call on it (allocated again only when a call needs more). A maintainer switches a translation unit over with
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
#include <mutex>
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

// A plan and the buffers its calls reuse: two device buffers and one pinned host staging
// buffer, grown on demand and kept until the FFT object is destroyed, so a call allocates only
// when it needs more than any earlier call did. The mutex makes a shared FFT object safe to
// use from several threads, as st::FFT is (calls on one object then run one at a time).
struct State {
    stx_fft* plan = nullptr;
    int n = 0;
    std::mutex mu;
    void* dev[2] = {nullptr, nullptr};
    size_t dev_bytes[2] = {0, 0};
    float* host = nullptr;
    size_t host_bytes = 0;

    ~State() {
        for (void* p : dev)
            if (p) (void)hipFree(p);
        if (host) (void)hipHostFree(host);
        if (plan) stx_fft_destroy(plan);
    }
    template <class T>
    T* device(int i, size_t bytes) {
        if (bytes > dev_bytes[i]) {
            if (dev[i]) (void)hipFree(dev[i]);
            dev[i] = nullptr;
            dev_bytes[i] = 0;
            hip(hipMalloc(&dev[i], bytes), "hipMalloc");
            dev_bytes[i] = bytes;
        }
        return static_cast<T*>(dev[i]);
    }
    float* staging(size_t floats) {
        if (floats * sizeof(float) > host_bytes) {
            if (host) (void)hipHostFree(host);
            host = nullptr;
            host_bytes = 0;
            hip(hipHostMalloc(reinterpret_cast<void**>(&host), floats * sizeof(float), 0), "hipHostMalloc");
            host_bytes = floats * sizeof(float);
        }
        return host;
    }
};

inline void to_device(void* dst, const void* src, size_t bytes) {
    if (bytes) hip(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

inline void to_host(void* dst, const void* src, size_t bytes) {
    if (bytes) hip(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

// complex<double> host data <-> interleaved float pairs (complex64).
inline void narrow(const cplx* a, size_t n, float* f) {
    for (size_t i = 0; i < n; i++) {
        f[2 * i] = (float)a[i].real();
        f[2 * i + 1] = (float)a[i].imag();
    }
}

inline void widen(const float* f, cplx* a, size_t n) {
    for (size_t i = 0; i < n; i++) a[i] = cplx(f[2 * i], f[2 * i + 1]);
}

}  // namespace detail

// st::FFT: a device plan for n points. Throws std::invalid_argument unless n is a power of
// two >= 2, like the reference (every such n up to 2^24 is supported by run(); the transforms
// below need 16 <= n <= 8192, the only sizes the reference frames at, and throw
// std::runtime_error otherwise).
class FFT {
public:
    explicit FFT(int n) : s_(std::make_shared<detail::State>()) {
        detail::check(stx_fft_create(n, &s_->plan));
        s_->n = n;
    }
    int size() const { return s_->n; }

    // In place on the first n values of a, unnormalised; inverse uses conjugate twiddles (no
    // 1/n). Values past the first n are left as they are, as the reference's loop does; a
    // vector shorter than n throws std::invalid_argument (the reference reads past its end).
    void run(std::vector<cplx>& a, bool inverse) const {
        const size_t n = (size_t)s_->n;
        if (a.size() < n) throw std::invalid_argument("FFT input shorter than the FFT size");
        std::lock_guard<std::mutex> lock(s_->mu);
        float* h = s_->staging(2 * n);
        float* d = s_->device<float>(0, 2 * n * sizeof(float));
        detail::narrow(a.data(), n, h);
        detail::to_device(d, h, 2 * n * sizeof(float));
        detail::check(stx_fft_run(s_->plan, d, 1, inverse ? 1 : 0, nullptr));
        detail::to_host(h, d, 2 * n * sizeof(float));
        detail::widen(h, a.data(), n);
    }

    const stx_fft* handle() const { return s_->plan; }
    detail::State& state() const { return *s_; }

private:
    std::shared_ptr<detail::State> s_;
};

// HTDemucs._spec for one channel: `len` samples -> [F = n/2][T] complex, f-major.
inline std::vector<cplx> htdemucs_spec(const FFT& fft, const float* x, int len, int& n_frames) {
    const int T = stx_htdemucs_frames(fft.size(), len);
    if (T < 0) detail::raise(STX_STATUS_INVALID_ARGUMENT);
    const size_t F = (size_t)fft.size() / 2, bins = F * (size_t)T;
    detail::State& st = fft.state();
    std::lock_guard<std::mutex> lock(st.mu);
    float* dx = st.device<float>(0, sizeof(float) * (size_t)(len > 0 ? len : 1));
    float* ds = st.device<float>(1, 2 * sizeof(float) * (bins ? bins : 1));
    detail::to_device(dx, x, sizeof(float) * (size_t)(len > 0 ? len : 0));
    detail::check(stx_htdemucs_spec(fft.handle(), dx, 1, len, ds, STX_SPEC_F_MAJOR, nullptr));
    float* h = st.staging(2 * bins);
    detail::to_host(h, ds, 2 * bins * sizeof(float));
    std::vector<cplx> spec(bins);
    detail::widen(h, spec.data(), bins);
    n_frames = T;
    return spec;
}

// HTDemucs._ispec for one channel: spec [F = n/2][T] f-major -> `length` samples.
inline std::vector<float> htdemucs_ispec(const FFT& fft, const std::vector<cplx>& spec, int n_frames, int length) {
    const size_t bins = (size_t)fft.size() / 2 * (size_t)(n_frames > 0 ? n_frames : 0);
    if (n_frames < 0 || spec.size() < bins) throw std::invalid_argument("spectrum smaller than n/2 x n_frames");
    detail::State& st = fft.state();
    std::lock_guard<std::mutex> lock(st.mu);
    float* h = st.staging(2 * bins);
    detail::narrow(spec.data(), bins, h);
    float* ds = st.device<float>(0, 2 * sizeof(float) * (bins ? bins : 1));
    float* dy = st.device<float>(1, sizeof(float) * (size_t)(length > 0 ? length : 1));
    detail::to_device(ds, h, 2 * bins * sizeof(float));
    detail::check(stx_htdemucs_ispec(fft.handle(), ds, 1, n_frames, length, dy, STX_SPEC_F_MAJOR, nullptr));
    std::vector<float> y((size_t)(length > 0 ? length : 0));
    detail::to_host(y.data(), dy, y.size() * sizeof(float));
    return y;
}

// torch.stft for one channel (periodic Hann, center, reflect, onesided): [F = n/2 + 1][T]
// f-major with T = len / hop + 1.
inline std::vector<cplx> torch_stft(const FFT& fft, const float* x, int len, int hop, bool normalized,
                                    int& n_frames) {
    const int T = stx_torch_stft_frames(len, hop);
    if (T < 0) detail::raise(STX_STATUS_INVALID_ARGUMENT);
    const size_t F = (size_t)fft.size() / 2 + 1, bins = F * (size_t)T;
    detail::State& st = fft.state();
    std::lock_guard<std::mutex> lock(st.mu);
    float* dx = st.device<float>(0, sizeof(float) * (size_t)(len > 0 ? len : 1));
    float* ds = st.device<float>(1, 2 * sizeof(float) * (bins ? bins : 1));
    detail::to_device(dx, x, sizeof(float) * (size_t)(len > 0 ? len : 0));
    detail::check(stx_torch_stft(fft.handle(), dx, 1, len, hop, normalized ? 1 : 0, ds, STX_SPEC_F_MAJOR, nullptr));
    float* h = st.staging(2 * bins);
    detail::to_host(h, ds, 2 * bins * sizeof(float));
    std::vector<cplx> spec(bins);
    detail::widen(h, spec.data(), bins);
    n_frames = T;
    return spec;
}

// torch.istft matching torch_stft, length = None: hop * (T - 1) samples.
inline std::vector<float> torch_istft(const FFT& fft, const std::vector<cplx>& spec, int n_frames, int hop,
                                      bool normalized) {
    const size_t bins = ((size_t)fft.size() / 2 + 1) * (size_t)(n_frames > 0 ? n_frames : 0);
    if (n_frames < 0 || spec.size() < bins) throw std::invalid_argument("spectrum smaller than (n/2 + 1) x n_frames");
    const long long length = n_frames > 0 ? (long long)hop * (n_frames - 1) : 0;
    detail::State& st = fft.state();
    std::lock_guard<std::mutex> lock(st.mu);
    float* h = st.staging(2 * bins);
    detail::narrow(spec.data(), bins, h);
    float* ds = st.device<float>(0, 2 * sizeof(float) * (bins ? bins : 1));
    float* dy = st.device<float>(1, sizeof(float) * (size_t)(length > 0 ? length : 1));
    detail::to_device(ds, h, 2 * bins * sizeof(float));
    detail::check(stx_torch_istft(fft.handle(), ds, 1, n_frames, hop, normalized ? 1 : 0, dy, STX_SPEC_F_MAJOR,
                                  nullptr));
    std::vector<float> y((size_t)(length > 0 ? length : 0));
    detail::to_host(y.data(), dy, y.size() * sizeof(float));
    return y;
}

}  // namespace st
}  // namespace stx
