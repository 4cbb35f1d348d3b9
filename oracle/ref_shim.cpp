// ref_shim.cpp — TEST INFRASTRUCTURE: exposes the reference's own src/stft.h through a C ABI so
// that tests/golden/make_golden.py can write golden vectors from it and the oracle can be
// checked against it. Built by oracle/Makefile into oracle/_ref/ (never committed) straight
// from the header where it lies under /root/reference/src; nothing of the reference is copied.
#include "stft.h"

#include <cstring>
#include <stdexcept>
#include <vector>

namespace {
template <class F>
int call(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::invalid_argument&) {
        return -1;
    } catch (const std::runtime_error&) {
        return -2;
    }
}
void put(const std::vector<st::cplx>& v, double* out) { std::memcpy(out, v.data(), v.size() * sizeof(st::cplx)); }
std::vector<st::cplx> get(const double* in, size_t n) {
    std::vector<st::cplx> v(n);
    std::memcpy(v.data(), in, n * sizeof(st::cplx));
    return v;
}
}  // namespace

extern "C" {
int ref_fft(double* a, int n, int inverse) {
    return call([&] {
        st::FFT fft(n);
        std::vector<st::cplx> v = get(a, n);
        fft.run(v, inverse != 0);
        put(v, a);
    });
}
int ref_torch_stft(const float* x, int len, int n_fft, int hop, int normalized, double* spec, int* n_frames) {
    return call([&] {
        st::FFT fft(n_fft);
        int T = 0;
        put(st::torch_stft(fft, x, len, hop, normalized != 0, T), spec);
        if (n_frames) *n_frames = T;
    });
}
int ref_torch_istft(const double* spec, int n_frames, int n_fft, int hop, int normalized, float* out) {
    return call([&] {
        st::FFT fft(n_fft);
        const std::vector<float> y =
            st::torch_istft(fft, get(spec, (size_t)(n_fft / 2 + 1) * n_frames), n_frames, hop, normalized != 0);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
    });
}
int ref_htdemucs_spec(const float* x, int len, int n_fft, double* spec, int* n_frames) {
    return call([&] {
        st::FFT fft(n_fft);
        int T = 0;
        put(st::htdemucs_spec(fft, x, len, T), spec);
        if (n_frames) *n_frames = T;
    });
}
int ref_htdemucs_ispec(const double* spec, int n_frames, int n_fft, int length, float* out) {
    return call([&] {
        st::FFT fft(n_fft);
        const std::vector<float> y = st::htdemucs_ispec(fft, get(spec, (size_t)(n_fft / 2) * n_frames), n_frames, length);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
    });
}
}
