// tfc.hip — the TFC-TDF (MDX) chunking on gfx950: UVR's SeperateMDX.demix loop and the
// TFCTDF::separate driver (MSST or UVR chunking, compensation, complement stem).
//
// Reference: TFCTDF::Impl::demix_uvr (src/tfc_tdf.cpp:407-441) and TFCTDF::separate (:569-595).
// The MSST loop (:447-495) is the demix plan of demix.hip with STX_DEMIX_MSST rules.
//
// UVR: `trim` = n_fft / 2 zeros in front of the mix, chunks of `chunk` samples every `step`
// over M = trim + len + gen + trim - len % gen samples (gen = chunk - 2 trim), each zero-filled
// past its actual length min(chunk, M - i), weighted by np.hanning(actual) (1 when
// overlap == 0), accumulated in double and divided at the trim offset. As in demix.hip the
// whole song stays resident and the overlap-add is a gather: each output sample sums, in chunk
// order and with the reference's double products, the chunks covering it, then divides once.
// The hanning tables are computed once per plan on the host with the C library's cos, as the
// reference computes them, so the weights (and so the results) are bit-identical.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <vector>

#include "common.hpp"
#include "demix_host.hpp"

struct stx_uvr_demix {
    int64_t len = 0, M = 0, step = 0, n_chunks = 0, first_partial = 0;
    int channels = 0, chunk = 0, n_fft = 0, trim = 0;
    double* d_w = nullptr;           // [chunk] weights of full chunks, then each partial chunk's
    uint64_t w_count = 0;            // entries of d_w
};

namespace stx {
namespace {

struct UvrArgs {
    int64_t len, M, step;
    int64_t n_chunks, first_partial;
    int chunk, trim, channels;
    FastDiv sdiv;                // division by step (M < 2^32)
};

UvrArgs uvr_args(const stx_uvr_demix* d) {
    return UvrArgs{d->len, d->M, d->step, d->n_chunks, d->first_partial, d->chunk, d->trim, d->channels,
                   FastDiv((unsigned)d->step)};
}

// Offset of chunk k's weights in the plan's table: 0 for full chunks, then the partial chunks'
// tables back to back, partial chunk j holding M - j * step weights (the host layout).
__host__ __device__ __forceinline__ int64_t uvr_woff(const UvrArgs& a, int64_t k) {
    if (k < a.first_partial) return 0;
    const int64_t f = a.first_partial;
    return a.chunk + (k - f) * a.M - a.step * ((k * (k - 1) - f * (f - 1)) / 2);
}

// parts[k - first][c][t] = x[c][i + t] for t < actual, else 0, where x is the mix behind `trim`
// zeros and zeros past its end (src/tfc_tdf.cpp:416-425). Four samples per thread.
__global__ __launch_bounds__(256) void uvr_chunks_kernel(UvrArgs a, const float* __restrict__ mix, int64_t first,
                                                         int vec, float* __restrict__ parts) {
    const int c = (int)blockIdx.y;
    const int64_t k = first + (int64_t)blockIdx.z;
    const int64_t i = k * a.step;
    const int64_t actual = min((int64_t)a.chunk, a.M - i);
    const int t0 = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
    if (t0 >= a.chunk) return;
    const float* xc = mix + (size_t)c * a.len;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t t = t0 + j;
        const int64_t s = i + t - a.trim;                    // index into the mix
        const bool in = t < actual && s >= 0 && s < a.len;
        const float x = xc[in ? s : 0];
        v[j] = in ? x : 0.0f;
    }
    float* dst = parts + ((size_t)blockIdx.z * a.channels + c) * a.chunk + t0;
    if (vec && t0 + 3 < a.chunk) {
        store_stream(reinterpret_cast<float4*>(dst), make_float4(v[0], v[1], v[2], v[3]));
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (t0 + j < a.chunk) store_stream(dst + j, v[j]);
    }
}

// out[q][t] = sum_k (double)y[k][q][p - i_k] * w_k[p - i_k] / sum_k w_k[p - i_k], p = trim + t,
// over the chunks covering p in chunk order (src/tfc_tdf.cpp:427-440). NK bounds the chunks
// covering one sample. A thread takes kUvrPer samples and P planes, which share the weights and
// their sum; loads are clamped to valid addresses and issued together. U is the index type:
// uint32_t when every index fits (the usual case: 64-bit index products cost several VALU
// instructions each, which made the kernel issue-bound), uint64_t otherwise.
constexpr int kUvrMaxCover = 8;
constexpr int kUvrPer = 2;

template <class U>
__device__ __forceinline__ U umin(U x, U y) { return x < y ? x : y; }

// uvr_woff in U's arithmetic. With U = uint32_t the host has checked that the table has fewer
// than 2^32 entries and k < 65536: the halvings are then exact (k (k - 1) < 2^32) and the rest
// is ring arithmetic, so intermediate wrap-around leaves the (representable) result exact.
template <class U>
__device__ __forceinline__ U uvr_woff_u(const UvrArgs& a, U k) {
    const U f = (U)a.first_partial;
    if (k < f) return 0;
    return (U)a.chunk + (k - f) * (U)a.M - (U)a.step * (k * (k - 1) / 2 - f * (f - 1) / 2);
}

template <int NK, int P, class U>
__global__ __launch_bounds__(256) void uvr_ola_kernel(UvrArgs a, const float* __restrict__ y,
                                                      const double* __restrict__ w, int planes,
                                                      float* __restrict__ out) {
#pragma clang fp contract(off)
    const int q0 = (int)blockIdx.y * P;
    const U len = (U)a.len;
    const U t0 = (U)blockIdx.x * (kUvrPer * 256) + threadIdx.x;
    if (t0 >= len) return;
    const U step = (U)a.step, M = (U)a.M, chunk = (U)a.chunk, pc = (U)planes * chunk;
    const int last = (int)a.n_chunks - 1;
    // Where one chunk alone covers a sample and its weight is not zero (hanning weights are 0 only
    // at a window's two ends, and at least sin^2(pi / (L - 1)) > 1e-18 elsewhere), the reference's
    // result (0 + y w) / (0 + w) in double, rounded to float, is y + 0 (y itself, but +0 for -0):
    // y w is within 2^-53 of the exact product (no underflow: |y| >= 2^-149 and w > 1e-18), the
    // quotient within 2^-52 of y, far inside y's float rounding interval. A wave whose samples
    // are all such writes y + 0 for them.
    {
        bool copy = true;
        U src[kUvrPer];
#pragma unroll
        for (int e = 0; e < kUvrPer; e++) {
            const U t = t0 + (U)(256 * e);
            const U p = (U)a.trim + umin<U>(t, len - 1);
            const int kh = min((int)a.sdiv.div((unsigned)p), last);
            const U k = (U)kh, i = k * step;
            const U actual = umin<U>(chunk, M - i);
            const U r = p - i;
            const bool alone = kh == 0 || p - (k - 1) * step >= umin<U>(chunk, M - (k - 1) * step);
            copy = copy && (t >= len || (alone && r > 0 && r + 1 < actual));
            src[e] = k * pc + umin<U>(r, actual - 1);
        }
        if (__all(copy)) {
            float v[kUvrPer][P];
#pragma unroll
            for (int e = 0; e < kUvrPer; e++)
#pragma unroll
                for (int u = 0; u < P; u++) v[e][u] = y[src[e] + (U)min(q0 + u, planes - 1) * chunk];
#pragma unroll
            for (int e = 0; e < kUvrPer; e++) {
                const U t = t0 + (U)(256 * e);
#pragma unroll
                for (int u = 0; u < P; u++)
                    if (t < len && q0 + u < planes) store_stream(out + (size_t)(q0 + u) * a.len + t, v[e][u] + 0.0f);
            }
            return;
        }
    }
    // Every load of every sample first (clamped addresses), then the sums: a chunk that does not
    // cover the sample adds +0.0, an exact no-op (the sums start at +0.0 and never become -0.0),
    // so no load sits behind a branch.
    double wv[kUvrPer][NK];
    bool in[kUvrPer][NK];
    float yv[kUvrPer][P][NK];
#pragma unroll
    for (int e = 0; e < kUvrPer; e++) {
        const U t = umin<U>(t0 + (U)(256 * e), len - 1);
        const U p = (U)a.trim + t;
        const int k_hi = min((int)a.sdiv.div((unsigned)p), last);
#pragma unroll
        for (int j = 0; j < NK; j++) {                  // chunk k_hi - j
            const int kk = k_hi - j;
            const U k = (U)max(kk, 0);
            const U i = k * step;                       // <= p: k <= p / step
            const U actual = umin<U>(chunk, M - i);
            const U r = p - i;
            in[e][j] = kk >= 0 && r < actual;
            const U rc = umin<U>(r, actual - 1);
            wv[e][j] = w[uvr_woff_u<U>(a, k) + rc];
            const U base = k * pc + rc;
#pragma unroll
            for (int u = 0; u < P; u++) yv[e][u][j] = y[base + (U)min(q0 + u, planes - 1) * chunk];
        }
    }
#pragma unroll
    for (int e = 0; e < kUvrPer; e++) {
        const U t = t0 + (U)(256 * e);
        double div = 0.0;
#pragma unroll
        for (int j = NK - 1; j >= 0; j--) div = div + (in[e][j] ? wv[e][j] : 0.0);   // ascending chunk order
        // res / div for every plane as div_rn with one reciprocal per sample (the IEEE quotient);
        // a zero weight sum keeps the plain division, whose inf / NaN the identity does not give.
        const double rdiv = 1.0 / div;
#pragma unroll
        for (int u = 0; u < P; u++) {
            double res = 0.0;
#pragma unroll
            for (int j = NK - 1; j >= 0; j--) {
                const double prod = (double)yv[e][u][j] * wv[e][j];
                res = res + (in[e][j] ? prod : 0.0);
            }
            const double q = div != 0.0 ? div_rn(res, div, rdiv) : res / div;
            if (t < len && q0 + u < planes) store_stream(out + (size_t)(q0 + u) * a.len + t, (float)q);
        }
    }
}

template <int NK, class U>
void launch_uvr_ola_u(const UvrArgs& a, const float* y, const double* w, int planes, float* out, hipStream_t s) {
    const unsigned bx = (unsigned)((a.len + 256 * kUvrPer - 1) / (256 * kUvrPer));
    if (planes % 4 == 0)
        hipLaunchKernelGGL((uvr_ola_kernel<NK, 4, U>), dim3(bx, (unsigned)(planes / 4)), dim3(256), 0, s, a, y, w, planes, out);
    else if (planes % 2 == 0)
        hipLaunchKernelGGL((uvr_ola_kernel<NK, 2, U>), dim3(bx, (unsigned)(planes / 2)), dim3(256), 0, s, a, y, w, planes, out);
    else
        hipLaunchKernelGGL((uvr_ola_kernel<NK, 1, U>), dim3(bx, (unsigned)planes), dim3(256), 0, s, a, y, w, planes, out);
}

template <int NK>
void launch_uvr_ola(const UvrArgs& a, const float* y, const double* w, int planes, bool narrow, float* out,
                    hipStream_t s) {
    if (narrow) launch_uvr_ola_u<NK, uint32_t>(a, y, w, planes, out, s);
    else launch_uvr_ola_u<NK, uint64_t>(a, y, w, planes, out, s);
}

// est *= compensate (when != 1), and with `complement` rest = mix - est_0 - est_1 - ... in float
// (src/tfc_tdf.cpp:582-593). One thread per sample of the [C][len] plane.
__global__ __launch_bounds__(256) void tfc_post_kernel(const float* __restrict__ mix, int64_t plane, int n_stems,
                                                       float compensate, int complement, float* __restrict__ est) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= plane) return;
    float rest = complement ? mix[i] : 0.0f;
    for (int k = 0; k < n_stems; k++) {
        float v = est[(size_t)k * plane + i];
        if (compensate != 1.0f) {
            v = v * compensate;
            est[(size_t)k * plane + i] = v;
        }
        rest = rest - v;
    }
    if (complement) est[(size_t)n_stems * plane + i] = rest;
}

// Sets *flag when any value of x [n] is not finite (src/tfc_tdf.cpp:573-574).
__global__ __launch_bounds__(256) void nonfinite_kernel(const float* __restrict__ x, int64_t n, int* flag) {
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        bad = bad || !isfinite(x[i]);
    if (bad) flag[0] = 1;                                // plain stores of one value: the order does not matter
}

void check_uvr(const stx_uvr_demix* d) { STX_REQUIRE(d != nullptr && d->d_w != nullptr, "null UVR plan"); }

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 1 << 20); }

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_uvr_demix_create(int64_t len, int channels, int chunk, int n_fft, float overlap,
                                        stx_uvr_demix** out) {
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        STX_REQUIRE(len > 0, "empty input");
        STX_REQUIRE(channels >= 1 && chunk >= 1 && n_fft >= 1, "bad channels/chunk/n_fft");
        const int trim = n_fft / 2, gen = chunk - 2 * trim;
        if (gen <= 0) fail(STX_STATUS_RUNTIME_ERROR, "tfc_tdf: chunk shorter than the FFT");      // :410
        const int64_t M = (int64_t)trim + len + gen + trim - len % gen;
        const int64_t step = overlap < 0 ? chunk - n_fft : (int64_t)((1.0 - (double)overlap) * chunk);
        if (step <= 0) fail(STX_STATUS_INVALID_ARGUMENT, "overlap too large for this model");     // :414
        const int64_t n = (M + step - 1) / step;
        STX_REQUIRE(n < (1LL << 31) && M < (1LL << 32), "input too long");
        // Weights: one table for full chunks, one per partial chunk (np.hanning of its length).
        auto hanning = [&](int m, std::vector<double>& w) {
            const size_t o = w.size();
            w.resize(o + m, 1.0);
            if (overlap == 0.0f) return;                                                            // :428
            if (m > 1)
                for (int i = 0; i < m; i++) w[o + i] = 0.5 - 0.5 * std::cos(2.0 * M_PI * i / (m - 1));
        };
        std::vector<double> w;
        hanning(chunk, w);
        int64_t first_partial = n;
        for (int64_t k = 0; k < n; k++) {
            const int64_t actual = std::min<int64_t>(chunk, M - k * step);
            if (actual < chunk) {                   // every chunk after the first partial one is partial
                if (first_partial == n) first_partial = k;
                hanning((int)actual, w);
            }
        }
        stx_uvr_demix* d = new stx_uvr_demix;
        d->len = len;
        d->M = M;
        d->step = step;
        d->n_chunks = n;
        d->first_partial = first_partial;
        d->channels = channels;
        d->chunk = chunk;
        d->n_fft = n_fft;
        d->trim = trim;
        for (int64_t k = 0; k < n; k++)             // the device recomputes the offsets in closed form
            STX_REQUIRE(uvr_woff(uvr_args(d), k) + std::min<int64_t>(chunk, M - k * step) <= (int64_t)w.size(),
                        "UVR weight table layout");
        d->w_count = w.size();
        hipError_t e = hipMalloc(&d->d_w, sizeof(double) * w.size());
        if (e == hipSuccess) e = hipMemcpy(d->d_w, w.data(), sizeof(double) * w.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            stx_uvr_demix_destroy(d);
            hip_check(e, "stx_uvr_demix_create");
        }
        *out = d;
    });
}

STX_API void stx_uvr_demix_destroy(stx_uvr_demix* d) {
    if (!d) return;
    (void)hipFree(d->d_w);
    delete d;
}

STX_API int64_t stx_uvr_demix_n_chunks(const stx_uvr_demix* d) { return d ? d->n_chunks : 0; }

STX_API stx_status stx_uvr_demix_geometry(const stx_uvr_demix* d, int64_t* padded_len, int64_t* step, int* trim) {
    return guard([&] {
        check_uvr(d);
        if (padded_len) *padded_len = d->M;
        if (step) *step = d->step;
        if (trim) *trim = d->trim;
    });
}

STX_API stx_status stx_uvr_demix_chunks(const stx_uvr_demix* d, const float* mix, int64_t first, int64_t count,
                                        float* parts, stx_stream stream) {
    return guard([&] {
        check_uvr(d);
        STX_REQUIRE(first >= 0 && count >= 0 && first + count <= d->n_chunks, "chunk range out of the plan");
        if (count == 0) return;
        STX_REQUIRE(mix && parts, "NULL buffer");
        STX_REQUIRE(count < 65536 && d->channels < 65536, "too many chunks or channels in one call");
        const int vec = d->chunk % 4 == 0 && (reinterpret_cast<uintptr_t>(parts) & 15) == 0;
        const dim3 grid((unsigned)((d->chunk + 1023) / 1024), (unsigned)d->channels, (unsigned)count);
        hipLaunchKernelGGL(uvr_chunks_kernel, grid, dim3(256), 0, as_stream(stream), uvr_args(d), mix, first, vec, parts);
        launch_check("uvr_chunks_kernel");
    });
}

STX_API stx_status stx_uvr_demix_overlap_add(const stx_uvr_demix* d, const float* y, int n_stems, float* out,
                                             stx_stream stream) {
    return guard([&] {
        check_uvr(d);
        STX_REQUIRE(n_stems >= 1, "bad stem count");
        STX_REQUIRE(y && out, "NULL buffer");
        STX_REQUIRE((int64_t)n_stems * d->channels < 65536, "too many stems * channels");
        const int planes = n_stems * d->channels;
        const int64_t cover = (d->chunk + d->step - 1) / d->step;
        if (cover > kUvrMaxCover)
            fail(STX_STATUS_UNSUPPORTED, "UVR overlap-add: more than %d chunks cover a sample", kUvrMaxCover);
        const hipStream_t s = as_stream(stream);
        const UvrArgs a = uvr_args(d);
        // 32-bit indices when the chunk outputs, the weight table and the chunk count allow;
        // STX_UVR_WIDE_INDEX=1 (read at each call) takes the 64-bit ones for every size, so that
        // the two kernels can be compared.
        const char* wide = std::getenv("STX_UVR_WIDE_INDEX");
        const bool narrow = d->n_chunks < 65536 && (uint64_t)d->n_chunks * planes * d->chunk < (1ull << 32) &&
                            d->w_count < (1ull << 32) && !(wide && wide[0] == '1');
        switch (cover) {
        case 1: launch_uvr_ola<1>(a, y, d->d_w, planes, narrow, out, s); break;
        case 2: launch_uvr_ola<2>(a, y, d->d_w, planes, narrow, out, s); break;
        case 3: launch_uvr_ola<3>(a, y, d->d_w, planes, narrow, out, s); break;
        case 4: launch_uvr_ola<4>(a, y, d->d_w, planes, narrow, out, s); break;
        default: launch_uvr_ola<kUvrMaxCover>(a, y, d->d_w, planes, narrow, out, s); break;
        }
        launch_check("uvr_ola_kernel");
    });
}

STX_API size_t stx_tfc_tdf_separate_workspace_size(int channels, int64_t len, int chunk, int n_fft,
                                                   stx_tfc_chunking chunking, int num_overlap, float overlap,
                                                   int n_stems, int batch) {
    try {
        if (channels < 1 || len < 1 || chunk < 1 || n_stems < 1 || batch < 1) return 0;
        int64_t n = 0;
        if (chunking == STX_TFC_UVR) {
            const int trim = n_fft / 2, gen = chunk - 2 * trim;
            if (gen <= 0) return 0;
            const int64_t M = (int64_t)trim + len + gen + trim - len % gen;
            const int64_t step = overlap < 0 ? chunk - n_fft : (int64_t)((1.0 - (double)overlap) * chunk);
            if (step <= 0) return 0;
            n = (M + step - 1) / step;
        } else {
            const int step = stx_demix_step(chunk, num_overlap, overlap);
            if (step < 1) return 0;
            n = demix_geometry(len, chunk, step, STX_DEMIX_MSST).n_chunks;
        }
        auto align = [](size_t b) { return (b + 255) / 256 * 256; };
        return align(sizeof(float) * (size_t)batch * channels * chunk) +
               align(sizeof(float) * (size_t)n * n_stems * channels * chunk) + 256;
    } catch (...) {
        return 0;
    }
}

STX_API stx_status stx_tfc_tdf_separate(const float* mix, int channels, int64_t len, int chunk, int n_fft,
                                        stx_tfc_chunking chunking, int num_overlap, int n_stems, float compensate,
                                        int complement, int batch, stx_separate_fn separate, void* separate_user,
                                        const stx_separate_options* options, float* out, void* workspace,
                                        size_t workspace_bytes, stx_stream stream) {
    stx_uvr_demix* uplan = nullptr;
    stx_demix* mplan = nullptr;
    const stx_status st = guard([&] {
        const stx_separate_options opt = separate_options(options);
        if (!mix || len <= 0) fail(STX_STATUS_RUNTIME_ERROR, "tfc_tdf: empty input");                // :572
        STX_REQUIRE(chunking == STX_TFC_MSST || chunking == STX_TFC_UVR, "unknown TFC-TDF chunking %d", chunking);
        STX_REQUIRE(channels >= 1 && n_stems >= 1 && chunk >= 1 && batch >= 1, "bad channels/stems/chunk/batch");
        STX_REQUIRE(out && separate && workspace && workspace_bytes >= 256, "NULL argument or no workspace");
        const hipStream_t s = as_stream(stream);
        char* ws = static_cast<char*>(workspace);
        {   // :573-574; the flag borrows the workspace's first bytes before any chunk is built
            int* d_flag = reinterpret_cast<int*>(ws);
            int flag = 0;
            hip_check(hipMemcpyAsync(d_flag, &flag, sizeof(int), hipMemcpyHostToDevice, s), "flag");
            hipLaunchKernelGGL(nonfinite_kernel, dim3(grid_for((int64_t)channels * len)), dim3(256), 0, s, mix,
                               (int64_t)channels * len, d_flag);
            launch_check("nonfinite_kernel");
            hip_check(hipMemcpyAsync(&flag, d_flag, sizeof(int), hipMemcpyDeviceToHost, s), "flag");
            hip_check(hipStreamSynchronize(s), "flag");
            if (flag) fail(STX_STATUS_RUNTIME_ERROR, "tfc_tdf: non-finite input");
        }
        if (opt.shifts != 0) fail(STX_STATUS_RUNTIME_ERROR, "tfc_tdf: shifts are unsupported");        // :575
        if (opt.overlap >= 1.0f) fail(STX_STATUS_INVALID_ARGUMENT, "overlap must be < 1");           // :576
        if (opt.should_cancel && opt.should_cancel(opt.user)) fail(STX_STATUS_CANCELLED, "cancelled"); // :581
        int64_t n = 0;
        if (chunking == STX_TFC_UVR) {                   // the plan reports the reference's errors (:410,:414)
            const stx_status cs = stx_uvr_demix_create(len, channels, chunk, n_fft, opt.overlap, &uplan);
            if (cs != STX_STATUS_OK) fail(cs, "%s", stx_last_error());
            n = uplan->n_chunks;
        } else {
            const int step = stx_demix_step(chunk, num_overlap, opt.overlap);
            STX_REQUIRE(step >= 1, "bad num_overlap");
            const stx_status cs = stx_demix_create_rules(len, channels, chunk, step, STX_DEMIX_MSST, &mplan);
            if (cs != STX_STATUS_OK) fail(cs, "%s", stx_last_error());
            n = stx_demix_n_chunks(mplan);
        }
        const size_t need = stx_tfc_tdf_separate_workspace_size(channels, len, chunk, n_fft, chunking, num_overlap,
                                                                opt.overlap, n_stems, batch);
        STX_REQUIRE(workspace_bytes >= need, "workspace too small: %zu bytes, need %zu", workspace_bytes, need);
        const size_t parts_bytes = ((sizeof(float) * (size_t)batch * channels * chunk) + 255) / 256 * 256;
        float* d_parts = reinterpret_cast<float*>(ws);
        float* d_y = reinterpret_cast<float*>(ws + parts_bytes);
        const int total = (int)n;
        int done = 0;
        for (int64_t first = 0; first < n; first += batch) {
            const int64_t count = std::min<int64_t>(batch, n - first);
            for (int64_t k = 0; k < count; k++)                                                   // :426, :481
                if (opt.should_cancel && opt.should_cancel(opt.user)) fail(STX_STATUS_CANCELLED, "cancelled");
            const stx_status cs = uplan ? stx_uvr_demix_chunks(uplan, mix, first, count, d_parts, stream)
                                        : stx_demix_chunks(mplan, mix, first, count, d_parts, stream);
            if (cs != STX_STATUS_OK) fail(cs, "%s", stx_last_error());
            const int32_t rc = separate(separate_user, d_parts, first, count,
                                        d_y + (size_t)first * n_stems * channels * chunk, stream);
            if (rc != 0) fail(STX_STATUS_RUNTIME_ERROR, "separator failed with %d", rc);
            for (int64_t k = 0; k < count; k++)                                                   // :433, :489
                if (opt.progress) opt.progress(opt.user, ++done, total);
        }
        const stx_status os = uplan ? stx_uvr_demix_overlap_add(uplan, d_y, n_stems, out, stream)
                                    : stx_demix_overlap_add(mplan, d_y, n_stems, out, stream);
        if (os != STX_STATUS_OK) fail(os, "%s", stx_last_error());
        if (compensate != 1.0f || complement) {                                                   // :582-593
            const int64_t plane = (int64_t)channels * len;
            STX_REQUIRE((plane + 255) / 256 < (1LL << 31), "input too long");
            hipLaunchKernelGGL(tfc_post_kernel, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, s, mix, plane,
                               n_stems, compensate, complement ? 1 : 0, out);
            launch_check("tfc_post_kernel");
        }
        // The plans' tables are freed below: the queued kernels must have finished first.
        hip_check(hipStreamSynchronize(s), "tfc_tdf_separate");
    });
    if (st != STX_STATUS_OK) (void)hipStreamSynchronize(as_stream(stream));
    stx_uvr_demix_destroy(uplan);
    stx_demix_destroy(mplan);
    return st;
}

}  // extern "C"
