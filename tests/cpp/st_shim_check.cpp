// Test helper: exposes the stx::st C++ shim (include/stx_st.hpp) to the Python parity tests
// through C functions. Each returns 0, 1 if the shim threw std::invalid_argument, 2 if it
// threw std::runtime_error, so the tests can check the reference's exception behaviour.
#include <chrono>
#include <complex>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "stx_st.hpp"

namespace st = stx::st;

namespace {

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::invalid_argument&) {
        return 1;
    } catch (const std::runtime_error&) {
        return 2;
    }
}

void put(const std::vector<st::cplx>& s, double* out) { std::memcpy(out, s.data(), s.size() * sizeof(st::cplx)); }

std::vector<st::cplx> get(const double* in, size_t n) {
    std::vector<st::cplx> s(n);
    std::memcpy(s.data(), in, n * sizeof(st::cplx));
    return s;
}

}  // namespace

extern "C" {

int shim_fft_create(int n) {
    return guarded([&] { st::FFT f(n); });
}

// In-place on `batch` interleaved complex<double> blocks of n, with one FFT object (its device
// buffers are reused by every call).
int shim_fft_run(int n, double* a, int batch, int inverse) {
    return guarded([&] {
        st::FFT f(n);
        for (int b = 0; b < batch; b++) {
            std::vector<st::cplx> v = get(a + 2 * (size_t)n * b, (size_t)n);
            f.run(v, inverse != 0);
            put(v, a + 2 * (size_t)n * b);
        }
    });
}

// run() on a vector of len >= n values: only the first n are transformed (src/stft.h:35-49).
int shim_fft_run_prefix(int n, double* a, int len, int inverse) {
    return guarded([&] {
        st::FFT f(n);
        std::vector<st::cplx> v = get(a, (size_t)len);
        f.run(v, inverse != 0);
        put(v, a);
    });
}

// run() on a vector shorter than n: std::invalid_argument.
int shim_fft_run_short(int n) {
    return guarded([&] {
        st::FFT f(n);
        std::vector<st::cplx> v((size_t)n - 1);
        f.run(v, false);
    });
}

int shim_htdemucs_spec(int n_fft, const float* x, int len, double* spec, int* n_frames) {
    return guarded([&] {
        st::FFT f(n_fft);
        int T = 0;
        put(st::htdemucs_spec(f, x, len, T), spec);
        *n_frames = T;
    });
}

int shim_htdemucs_ispec(int n_fft, const double* spec, int n_frames, int length, float* out) {
    return guarded([&] {
        st::FFT f(n_fft);
        const std::vector<float> y = st::htdemucs_ispec(f, get(spec, (size_t)n_fft / 2 * n_frames), n_frames, length);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
    });
}

int shim_torch_stft(int n_fft, const float* x, int len, int hop, int normalized, double* spec, int* n_frames) {
    return guarded([&] {
        st::FFT f(n_fft);
        int T = 0;
        put(st::torch_stft(f, x, len, hop, normalized != 0, T), spec);
        *n_frames = T;
    });
}

int shim_torch_istft(int n_fft, const double* spec, int n_frames, int hop, int normalized, float* out) {
    return guarded([&] {
        st::FFT f(n_fft);
        const std::vector<float> y =
            st::torch_istft(f, get(spec, ((size_t)n_fft / 2 + 1) * n_frames), n_frames, hop, normalized != 0);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
    });
}

// Seconds per st::htdemucs_spec + st::htdemucs_ispec round trip of `channels` channels of `len`
// samples on host buffers, one FFT object reused (after one untimed round trip), as a caller of
// src/stft.h runs them (src/htdemucs.cpp:428,470); -1 if the shim threw.
double shim_time_htdemucs_round_trip(int n_fft, const float* x, int channels, int len, int reps) {
    try {
        st::FFT f(n_fft);
        auto once = [&] {
            for (int c = 0; c < channels; c++) {
                int T = 0;
                const std::vector<st::cplx> s = st::htdemucs_spec(f, x + (size_t)c * len, len, T);
                const std::vector<float> y = st::htdemucs_ispec(f, s, T, len);
                if (y.size() != (size_t)len) throw std::runtime_error("length");
            }
        };
        once();
        const auto t0 = std::chrono::steady_clock::now();
        for (int r = 0; r < reps; r++) once();
        const auto t1 = std::chrono::steady_clock::now();
        return std::chrono::duration<double>(t1 - t0).count() / (reps > 0 ? reps : 1);
    } catch (const std::exception&) {
        return -1.0;
    }
}

// A spectrum given with fewer values than n_frames needs: the shim must throw invalid_argument.
int shim_istft_short_spectrum(int n_fft) {
    return guarded([&] {
        st::FFT f(n_fft);
        std::vector<st::cplx> s(3);
        (void)st::torch_istft(f, s, 10, n_fft / 4, false);
    });
}

}  // extern "C"
