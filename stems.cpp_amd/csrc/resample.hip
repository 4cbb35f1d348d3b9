// resample.hip — band-limited resampling on gfx950.
//
// Reference: st::resample_planar (src/audio.h:17-59): a Kaiser-windowed sinc (beta 8.6, 32 zero
// crossings, cutoff 0.95 of the lower Nyquist), tabulated once over |x| in [0, half] at 2^15 + 2
// points and interpolated linearly; each output sample sums, in double and in input order, the
// weighted input samples within `half` of its position. The table is computed on the host with
// the reference's formula (so it is bit-identical), kept on the device, and every per-tap
// operation is the reference's double operation in the reference's order, so the output is
// bit-identical. One thread per output sample and every channel; taps go in groups of eight
// whose loads are issued together (clamped addresses; a tap past the window, or one the
// reference skips, adds +0.0, an exact no-op on a sum that starts at +0.0). The per-tap
// division by `half` is done as a multiplication by r = RN(1/half) and one fma correction,
// q = RN(q0 + r RN(x - q0 half)) with q0 = RN(x r), which is the correctly rounded quotient
// (Markstein's theorem: r within half an ulp of 1/half, q0 within one ulp of x/half, residual
// exact by the fma), so bit-identical to IEEE division at a fraction of its cost.
#include <algorithm>
#include <cmath>
#include <vector>

#include "common.hpp"

struct stx_resampler {
    int src = 0, dst = 0;
    double ratio = 1.0, half = 0.0;
    double* d_table = nullptr;       // [kTableN + 2]
};

namespace stx {
namespace {

constexpr int kTableN = 1 << 15;
constexpr int kTapGroup = 8;

struct ResampleArgs {
    const float* in;                 // [C][n]
    float* out;                      // [C][out_n]
    const double* table;
    double ratio, half, rhalf;       // rhalf = RN(1 / half)
    int n, out_n, C;
};


template <int NC>
__global__ __launch_bounds__(256) void resample_kernel(ResampleArgs a) {
#pragma clang fp contract(off)
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i >= a.out_n) return;
    const int C = NC > 0 ? NC : a.C;
    const double c = i / a.ratio;                                   // src/audio.h:43-46
    const int lo = max(0, (int)ceil(c - a.half)), hi = min(a.n - 1, (int)floor(c + a.half));
    constexpr int MC = NC > 0 ? NC : 8;
    double acc[MC];
#pragma unroll
    for (int k = 0; k < MC; k++) acc[k] = 0.0;
    for (int j0 = lo; j0 <= hi; j0 += kTapGroup) {
        double w[kTapGroup];
        bool use[kTapGroup];
        float x[kTapGroup][MC];
#pragma unroll
        for (int q = 0; q < kTapGroup; q++) {
            const int j = min(j0 + q, hi);
            const double pos = div_rn(fabs(j - c), a.half, a.rhalf) * kTableN;
            const int t = min((int)pos, kTableN);
            const double fr = pos - t;
            const double t0 = a.table[t], t1 = a.table[t + 1];
#pragma unroll
            for (int k = 0; k < MC; k++) x[q][k] = k < C ? a.in[(size_t)k * a.n + j] : 0.0f;
            w[q] = t0 + (t1 - t0) * fr;
            use[q] = j0 + q <= hi && (int)pos < kTableN;   // past the window, or t >= table_n (:49)
        }
#pragma unroll
        for (int q = 0; q < kTapGroup; q++)
#pragma unroll
            for (int k = 0; k < MC; k++) {
                const double p = w[q] * (double)x[q][k];
                acc[k] = acc[k] + (use[q] ? p : 0.0);
            }
    }
#pragma unroll
    for (int k = 0; k < MC; k++)
        if (k < C) store_stream(a.out + (size_t)k * a.out_n + i, (float)acc[k]);
}

__global__ __launch_bounds__(256) void copy_kernel(const float* __restrict__ in, float* __restrict__ out, size_t n) {
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (size_t)gridDim.x * 256) out[e] = in[e];
}

double bessel_i0(double x) {
    double s = 1, t = 1;
    for (int k = 1; k < 30; k++) {
        t *= (x / (2 * k)) * (x / (2 * k));
        s += t;
    }
    return s;
}

void check_resampler(const stx_resampler* r) { STX_REQUIRE(r != nullptr, "null resampler"); }

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_resampler_create(int src_rate, int dst_rate, stx_resampler** out) {
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        STX_REQUIRE(src_rate > 0 && dst_rate > 0, "sample rates must be positive");
        stx_resampler* r = new stx_resampler;
        r->src = src_rate;
        r->dst = dst_rate;
        r->ratio = (double)dst_rate / src_rate;
        if (src_rate != dst_rate) {                                  // src/audio.h:20-38
            const double cutoff = 0.95 * std::min(1.0, r->ratio);
            const int zc = 32;
            const double half = zc / cutoff;
            const double beta = 8.6;
            const double i0b = bessel_i0(beta);
            std::vector<double> table(kTableN + 2);
            for (int t = 0; t <= kTableN + 1; t++) {
                const double x = std::min((double)t / kTableN, 1.0) * half;
                const double rr = x / half;
                const double arg = M_PI * x * cutoff;
                const double sinc = arg < 1e-12 ? 1.0 : std::sin(arg) / arg;
                table[t] = rr >= 1 ? 0.0 : sinc * bessel_i0(beta * std::sqrt(1 - rr * rr)) / i0b * cutoff;
            }
            r->half = half;
            hipError_t e = hipMalloc(&r->d_table, sizeof(double) * table.size());
            if (e == hipSuccess)
                e = hipMemcpy(r->d_table, table.data(), sizeof(double) * table.size(), hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                stx_resampler_destroy(r);
                hip_check(e, "stx_resampler_create");
            }
        }
        *out = r;
    });
}

STX_API void stx_resampler_destroy(stx_resampler* r) {
    if (!r) return;
    if (r->d_table) (void)hipFree(r->d_table);
    delete r;
}

STX_API int64_t stx_resample_length(const stx_resampler* r, int64_t n) {
    if (!r || n < 0) return -1;
    if (r->src == r->dst) return n;
    return (int64_t)std::llround((double)n * r->ratio);              // src/audio.h:20: llround(n * ratio) with int n
}

STX_API stx_status stx_resample(const stx_resampler* r, const float* in, int channels, int64_t n, float* out,
                                stx_stream stream) {
    return guard([&] {
        check_resampler(r);
        STX_REQUIRE(channels >= 1 && n >= 0, "bad channels/n");
        STX_REQUIRE(n < (1LL << 31) && (long long)channels * n < (1LL << 40), "input too long");
        if (n == 0) return;
        STX_REQUIRE(in && out, "NULL buffer");
        const hipStream_t s = as_stream(stream);
        if (r->src == r->dst) {                                      // src/audio.h:19: the input as it is
            const size_t count = (size_t)channels * n;
            hipLaunchKernelGGL(copy_kernel, dim3((unsigned)std::min<size_t>((count + 255) / 256, 1 << 20)), dim3(256),
                               0, s, in, out, count);
            launch_check("copy_kernel");
            return;
        }
        const int64_t out_n = stx_resample_length(r, n);
        STX_REQUIRE(out_n < (1LL << 31), "output too long");
        if (out_n == 0) return;
        if (channels > 8) fail(STX_STATUS_UNSUPPORTED, "resample: more than 8 channels");
        ResampleArgs a{in, out, r->d_table, r->ratio, r->half, 1.0 / r->half, (int)n, (int)out_n, channels};
        const dim3 grid((unsigned)((out_n + 255) / 256));
        if (channels == 1) hipLaunchKernelGGL(resample_kernel<1>, grid, dim3(256), 0, s, a);
        else if (channels == 2) hipLaunchKernelGGL(resample_kernel<2>, grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL(resample_kernel<0>, grid, dim3(256), 0, s, a);
        launch_check("resample_kernel");
    });
}

}  // extern "C"
