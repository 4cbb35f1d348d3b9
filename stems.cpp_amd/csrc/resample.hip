// resample.hip — band-limited resampling on gfx950.
//
// Reference: st::resample_planar (src/audio.h:17-59): a Kaiser-windowed sinc (beta 8.6, 32 zero
// crossings, cutoff 0.95 of the lower Nyquist), tabulated once over |x| in [0, half] at 2^15 + 2
// points and interpolated linearly; each output sample sums, in double and in input order, the
// weighted input samples within `half` of its position. Two kernels. The default one,
// resample_phase_kernel (below), weights each output by its exact phase; the per-tap one,
// resample_kernel, chosen by STX_RESAMPLE_EXACT=1, computes the table on the host with the
// reference's formula (so it is bit-identical), keeps it on the device, and does every per-tap
// operation as the reference's double operation in the reference's order, so its output is
// bit-identical. One thread per output sample and every channel; taps go in groups of eight
// whose loads are issued together (clamped addresses; a tap past the window, or one the
// reference skips, adds +0.0, an exact no-op on a sum that starts at +0.0). The per-tap
// division by `half` is done as a multiplication by r = RN(1/half) and one fma correction,
// q = RN(q0 + r RN(x - q0 half)) with q0 = RN(x r), which is the correctly rounded quotient
// (Markstein's theorem: r within half an ulp of 1/half, q0 within one ulp of x/half, residual
// exact by the fma), so bit-identical to IEEE division at a fraction of its cost.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <numeric>
#include <vector>

#include "common.hpp"
#include "resample.hpp"

struct stx_resampler {
    int src = 0, dst = 0;
    double ratio = 1.0, half = 0.0;
    double* d_table = nullptr;       // [kTableN + 2]
    // Phase table (see resample_phase_kernel): dst = up * g, src = down * g.
    int up = 0, down = 0;
    int omin = 0;                    // offset of tap 0 from floor(c)
    int npairs = 0, rs = 0;          // phase pairs (up + 1) / 2; doubles per pair row
    int width = 0, pitch = 0, lds_bytes = 0;  // staged input tile of resample_phase_kernel
    double* d_pair = nullptr;        // [npairs][rs]: the pair's two weight rows interleaved
    int4* d_prange = nullptr;        // [npairs]: each row's first and last tap
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

// The same sums over weights that depend only on the output's phase. With dst = up g and
// src = down g, output i = q + M up sits at c = i down / up = fq + M down + p / up, where
// fq = floor(q down / up) and p = q down mod up, so its taps j = fq + M down + omin + k and their
// weights (the reference's table interpolation at |j - c|) are row p of a table of up rows
// computed once on the host. Those weights differ from the reference's, which it computes per
// output from c = i / ratio with ratio rounded to double, by the rounding of c (below 1e-9 for
// three hours of 48 kHz audio), so the output is within a few float ulps of the reference's
// (SNR above 160 dB) instead of bit-identical; the per-tap division, table lookup and
// interpolation of resample_kernel are gone, leaving an fma per tap and a conversion per staged
// sample read (shared by a pair of phases, below).
//
// A workgroup takes one channel and the 64 output groups M = m0 + lane, m0 = 64 blockIdx.x: all
// outputs in [m0 up, (m0 + 64) up). It stages in LDS, for each lane, the input its outputs read:
// row l holds j = (m0 + l) down + omin + r for r < width = down + ntap + kPhaseOverread (zeros
// outside the input, which add nothing; neighbouring rows overlap by ntap + kPhaseOverread). Rows
// are `pitch` floats apart, width rounded up to odd, so the lanes of a read fall in different
// banks. 48 -> 44.1 kHz stages 62 KB: two workgroups of 16 waves, the most waves a CU holds.
//
// Each wave takes pairs of neighbouring phases q0 = 2 jp, q1 = q0 + 1 (jp = wave, wave + 16, ...).
// Their windows, at r = fq0 + s and r = fq1 + k, overlap but for a tap or two at each end, so a
// lane converts each staged sample it reads once and feeds both sums. The host interleaves the
// pair's weight rows by s (w0(s), w1(s)): eight common taps are two 64-byte scalar loads from one
// row and four paired LDS reads. Taps in only one window (the pair's ranges, lo0..hi0 and
// lo1..hi1 in s) go through a guarded loop, so no tap is summed that its phase's window lacks;
// each sum still takes its taps in order. The last 1-7 common taps load one whole chunk (at most
// 7 samples and weight pairs past them, inside the row and the padded table) and sum only their
// own under uniform branches. An odd last phase is paired with itself; its second sum is not
// stored.
struct PhaseArgs {
    const float* in;                 // [C][n]
    float* out;                      // [C][out_n]
    const double* w;                 // [npairs][rs]: (w0(s), w1(s)) for s < rs / 2
    const int4* range;               // [npairs]: lo0, hi0, lo1, hi1 in s
    long long n, out_n;
    int up, down, omin, npairs, rs;
    int width, pitch;                // staged samples per lane row; floats between rows (odd)
    FastDiv fup;                     // q down / up (below 2^20)
};

constexpr int kPhaseTile = 64;                       // output groups per workgroup, one per lane
constexpr int kPhaseWaves = 16;                      // waves per workgroup, each over every 16th phase pair
constexpr int kPhaseStage = 4;                       // staged loads in flight per lane
constexpr long long kPhaseMaxWeights = 1 << 18;      // up * ntap above this: per-tap kernel
constexpr int kPhaseOverread = 8;                    // staged samples and table weights past the last used

// The weight table and the pair ranges do not change while the kernel runs: read through the
// constant address space, a wave-uniform load of them is a scalar load into SGPRs.
typedef const __attribute__((address_space(4))) double* ConstDoubles;
typedef const __attribute__((address_space(4))) int* ConstInts;

// Taps s0..s1 of which only some lie in each window: each summed where its window has it.
__device__ __forceinline__ void pair_edge(const float* xr, ConstDoubles wp, int4 rg, int s0, int s1, double& a0,
                                          double& a1) {
    for (int s = s0; s <= s1; s++) {
        const double x = (double)xr[s];
        if (s >= rg.x && s <= rg.y) a0 = fma(wp[2 * s], x, a0);
        if (s >= rg.z && s <= rg.w) a1 = fma(wp[2 * s + 1], x, a1);
    }
}

__global__ __launch_bounds__(kPhaseWaves * 64) void resample_phase_kernel(PhaseArgs a) {
    extern __shared__ float xs[];
    const int c = (int)blockIdx.y;
    const long long m0 = (long long)blockIdx.x * kPhaseTile;
    const float* in = a.in + (size_t)c * a.n;
    const int lane = (int)threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    // Each wave stages whole rows: the row's first input index and its bounds are the same for
    // the wave, so a sample costs an offset and, at the input's ends only, a bounds test.
    for (int l = wave; l < kPhaseTile; l += kPhaseWaves) {
        const long long jb = (m0 + l) * a.down + a.omin;        // input index of r = 0
        const float* src = in + jb;
        float* dst = xs + l * a.pitch;
        const bool inside = jb >= 0 && jb + a.width <= a.n;
        const int rlo = (int)max(-jb, 0LL), rhi = (int)min(a.n - jb, (long long)a.width);   // r in [rlo, rhi) is input
        for (int r0 = 0; r0 < a.width; r0 += 64 * kPhaseStage) {
            float v[kPhaseStage];
#pragma unroll
            for (int u = 0; u < kPhaseStage; u++) {
                const int r = r0 + u * 64 + lane;
                v[u] = r < a.width && (inside || (r >= rlo && r < rhi)) ? src[r] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kPhaseStage; u++) {
                const int r = r0 + u * 64 + lane;
                if (r < a.width) dst[r] = v[u];
            }
        }
    }
    __syncthreads();
    float* outc = a.out + (size_t)c * a.out_n;
    const long long i0 = (m0 + lane) * a.up;
    for (int jp = wave; jp < a.npairs; jp += kPhaseWaves) {
        const int q0 = 2 * jp;
        const int fq0 = (int)a.fup.div((unsigned)q0 * (unsigned)a.down);
        const ConstInts rgp = (ConstInts)a.range + 4 * jp;
        const int4 rg = make_int4(rgp[0], rgp[1], rgp[2], rgp[3]);
        const ConstDoubles wp = (ConstDoubles)(a.w + (size_t)jp * a.rs);
        const float* xr = xs + lane * a.pitch + fq0;
        const int lo_u = min(rg.x, rg.z), hi_u = max(rg.y, rg.w);
        int lo_i = max(rg.x, rg.z), hi_i = min(rg.y, rg.w);
        if (lo_i > hi_i) lo_i = hi_u + 1, hi_i = hi_u;            // no common taps: all on the edge path
        double a0 = 0.0, a1 = 0.0;
        pair_edge(xr, wp, rg, lo_u, lo_i - 1, a0, a1);
        int s = lo_i;
        for (; s + 7 <= hi_i; s += 8) {
            const ConstDoubles wc = wp + 2 * s;                  // one base, constant offsets: two 64-byte loads
            const float* xc = xr + s;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const double x = (double)xc[t];
                a0 = fma(wc[2 * t], x, a0);
                a1 = fma(wc[2 * t + 1], x, a1);
            }
        }
        if (s <= hi_i) {
            const ConstDoubles wc = wp + 2 * s;
            const float* xc = xr + s;
            float x[8];
            double w[16];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                x[t] = xc[t];
                w[2 * t] = wc[2 * t];
                w[2 * t + 1] = wc[2 * t + 1];
            }
#pragma unroll
            for (int t = 0; t < 7; t++)
                if (s + t <= hi_i) {
                    a0 = fma(w[2 * t], (double)x[t], a0);
                    a1 = fma(w[2 * t + 1], (double)x[t], a1);
                }
        }
        pair_edge(xr, wp, rg, hi_i + 1, hi_u, a0, a1);
        const long long i = i0 + q0;
        if (i < a.out_n) outc[i] = (float)a0;
        if (q0 + 1 < a.up && i + 1 < a.out_n) outc[i + 1] = (float)a1;
    }
}

// LDS bytes of one staged tile (zero: the tile does not fit in `budget` bytes, the device's LDS
// per workgroup, and the per-tap kernel is used).
int phase_lds_bytes(int down, int ntap, long long budget, int* width, int* pitch) {
    const long long wd = (long long)down + ntap + kPhaseOverread;
    const long long pt = wd | 1;
    const long long bytes = kPhaseTile * pt * (long long)sizeof(float);
    if (bytes > budget) return 0;
    *width = (int)wd;
    *pitch = (int)pt;
    return (int)bytes;
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

void resampler_rates(const stx_resampler* r, int& src, int& dst) {
    check_resampler(r);
    src = r->src;
    dst = r->dst;
}

}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_resampler_create(int src_rate, int dst_rate, stx_resampler** out) {
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        STX_REQUIRE(src_rate > 0 && dst_rate > 0, "sample rates must be positive");
        // LDS per workgroup of the current device: the phase kernel's staged tile must fit.
        int dev = 0, lds_max = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        hip_check(hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev),
                  "hipDeviceGetAttribute");
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
            // Phase table: output i = q + M up has c = i down / up = floor(q down / up) + M down
            // + p / up with p = q down mod up; its taps are j = floor(c) + o for o in
            // [ceil(p/up - half), floor(p/up + half)], each weighted as the reference weights
            // |j - c| (src/audio.h:47-52), skipped where the table index reaches table_n.
            const int g = std::gcd(src_rate, dst_rate);
            const int up = dst_rate / g, down = src_rate / g;
            const int omin = -(int)std::floor(half), omax = (int)std::floor(half) + 1;
            const int ntap = omax - omin + 1;
            std::vector<double> phase;
            std::vector<int2> range;
            // The staged tile must fit in the device's LDS per workgroup; above 64 KB the kernel
            // is allowed that much dynamic LDS first.
            int width = 0, pitch = 0;
            int lds_bytes = phase_lds_bytes(down, ntap, lds_max, &width, &pitch);
            if (lds_bytes > 64 * 1024 &&
                hipFuncSetAttribute((const void*)resample_phase_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    lds_max) != hipSuccess) {
                (void)hipGetLastError();
                lds_bytes = 0;
            }
            std::vector<double> pair;
            std::vector<int4> prange;
            if ((long long)up * ntap <= kPhaseMaxWeights && lds_bytes > 0) {
                phase.assign((size_t)up * ntap, 0.0);
                range.assign(up, make_int2(0, -1));
                for (int p = 0; p < up; p++) {
                    const double frac = (double)p / up;
                    int lo = ntap, hi = -1;
                    for (int k = 0; k < ntap; k++) {
                        const int o = omin + k;
                        if (o < (int)std::ceil(frac - half) || o > (int)std::floor(frac + half)) continue;
                        const double pos = std::fabs(o - frac) / half * kTableN;
                        const int t = (int)pos;
                        if (t >= kTableN) continue;
                        phase[(size_t)p * ntap + k] = table[t] + (table[t + 1] - table[t]) * (pos - t);
                        lo = std::min(lo, k);
                        hi = std::max(hi, k);
                    }
                    range[p] = make_int2(lo, hi);
                }
                // Pairs of neighbouring phases q0 = 2 jp and q1 = q0 + 1, whose taps start at
                // floor(q down / up) + omin: q1's are d = fq1 - fq0 later, so its row goes in at
                // s = k + d. An odd last phase is paired with itself.
                auto fq = [&](int q) { return (int)((long long)q * down / up); };
                const int npairs = (up + 1) / 2;
                int dmax = 0;
                for (int jp = 0; jp < npairs; jp++)
                    if (2 * jp + 1 < up) dmax = std::max(dmax, fq(2 * jp + 1) - fq(2 * jp));
                const int rs = 2 * (ntap + dmax + kPhaseOverread);
                pair.assign((size_t)npairs * rs, 0.0);
                prange.resize(npairs);
                for (int jp = 0; jp < npairs; jp++) {
                    const int q0 = 2 * jp, q1 = q0 + 1 < up ? q0 + 1 : q0;
                    const int p0 = (int)((long long)q0 * down % up), p1 = (int)((long long)q1 * down % up);
                    const int d = fq(q1) - fq(q0);
                    double* row = pair.data() + (size_t)jp * rs;
                    for (int k = range[p0].x; k <= range[p0].y; k++) row[2 * k] = phase[(size_t)p0 * ntap + k];
                    if (q1 != q0)
                        for (int k = range[p1].x; k <= range[p1].y; k++)
                            row[2 * (k + d) + 1] = phase[(size_t)p1 * ntap + k];
                    prange[jp] = make_int4(range[p0].x, range[p0].y, d + range[p1].x, d + range[p1].y);
                }
                r->up = up;
                r->down = down;
                r->omin = omin;
                r->npairs = npairs;
                r->rs = rs;
                r->width = width;
                r->pitch = pitch;
                r->lds_bytes = lds_bytes;
            }
            hipError_t e = hipMalloc(&r->d_table, sizeof(double) * table.size());
            if (e == hipSuccess)
                e = hipMemcpy(r->d_table, table.data(), sizeof(double) * table.size(), hipMemcpyHostToDevice);
            if (e == hipSuccess && !pair.empty()) {
                e = hipMalloc(&r->d_pair, sizeof(double) * pair.size());
                if (e == hipSuccess) e = hipMalloc(&r->d_prange, sizeof(int4) * prange.size());
                if (e == hipSuccess)
                    e = hipMemcpy(r->d_pair, pair.data(), sizeof(double) * pair.size(), hipMemcpyHostToDevice);
                if (e == hipSuccess)
                    e = hipMemcpy(r->d_prange, prange.data(), sizeof(int4) * prange.size(), hipMemcpyHostToDevice);
            }
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
    if (r->d_pair) (void)hipFree(r->d_pair);
    if (r->d_prange) (void)hipFree(r->d_prange);
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
        // The phase table unless STX_RESAMPLE_EXACT=1 (read at each call) asks for the per-tap
        // kernel, which gives the reference's bits.
        const char* exact = std::getenv("STX_RESAMPLE_EXACT");
        if (r->d_pair && !(exact && exact[0] == '1')) {
            PhaseArgs pa{in, out, r->d_pair, r->d_prange, n, out_n, r->up, r->down, r->omin, r->npairs, r->rs, r->width, r->pitch,
                         FastDiv((unsigned)r->up)};
            const long long groups = (out_n + r->up - 1) / r->up;                // output groups M
            STX_REQUIRE(channels < 65536, "too many channels");
            const long long tiles = (groups + kPhaseTile - 1) / kPhaseTile;
            const dim3 pg((unsigned)tiles, (unsigned)channels);
            hipLaunchKernelGGL(resample_phase_kernel, pg, dim3(kPhaseWaves * 64), (unsigned)r->lds_bytes, s, pa);
            launch_check("resample_phase_kernel");
            return;
        }
        ResampleArgs a{in, out, r->d_table, r->ratio, r->half, 1.0 / r->half, (int)n, (int)out_n, channels};
        const dim3 grid((unsigned)((out_n + 255) / 256));
        if (channels == 1) hipLaunchKernelGGL(resample_kernel<1>, grid, dim3(256), 0, s, a);
        else if (channels == 2) hipLaunchKernelGGL(resample_kernel<2>, grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL(resample_kernel<0>, grid, dim3(256), 0, s, a);
        launch_check("resample_kernel");
    });
}

}  // extern "C"
