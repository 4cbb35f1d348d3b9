// demix.hip — chunked overlap-add demix on gfx950.
//
// Reference: RoFormer::Impl::demix (src/roformer.cpp:286-351), and with the MSST rules
// TFCTDF::Impl::demix_msst (src/tfc_tdf.cpp:447-495), which differs in the short-chunk reflect
// threshold, the chunk that drops its fade-out and the fade window (demix_host.cpp). The reference walks the chunks
// one by one and read-modify-writes a double accumulator of S*C*Lp values per chunk. Here the
// whole song stays resident (288 GB of HBM holds every chunk's output many times over) and
// the overlap-add is a single gather pass: each output sample sums, in chunk order and in
// double, the weighted outputs of the (at most ceil(chunk/step)) chunks covering it, divides
// by the summed weights and rounds once. Products of two floats are exact in double and the
// sums run in the reference's order, so the result is bit-identical to the reference for the
// same chunk outputs. The chunk inputs are built by one kernel that does the border reflect
// padding and the short-chunk reflect/zero padding as index arithmetic.
#include <algorithm>
#include <cmath>
#include <random>
#include <vector>

#include "common.hpp"
#include "demix_host.hpp"

struct stx_demix {
    stx::DemixGeometry g;
    int channels = 0;
    float* d_window = nullptr;       // [chunk]: the fade window before the per-chunk edits
};

namespace stx {
namespace {

struct DemixArgs {
    int64_t len, padded_len;
    int chunk, step, border, fade, reflect_border, channels;
    int tail_min;                // a short chunk is reflect-padded above this length
    int reach;                   // a chunk drops its fade-out when start + reach >= padded_len
};

DemixArgs args_of(const stx_demix* d) {
    const bool msst = d->g.rules == STX_DEMIX_MSST;
    return DemixArgs{d->g.len, d->g.padded_len, d->g.chunk, d->g.step, d->g.border, d->g.fade,
                     d->g.reflect_border, d->channels, d->g.chunk / 2 + (msst ? 0 : 1),
                     msst ? d->g.step : d->g.chunk};
}

// Sample p of the border-padded signal of channel row xc (src/roformer.cpp:293-301).
__device__ __forceinline__ float padded_mix(const float* __restrict__ xc, int64_t p, const DemixArgs& a) {
    if (!a.reflect_border) return xc[p];
    int64_t j = p - a.border;
    j = j < 0 ? -j : j;
    j = j >= a.len ? 2 * (a.len - 1) - j : j;
    return xc[j];
}

// parts[k - first][c][t] for chunks first .. first + count - 1. Block (x, y, z) = (tile of
// 256 * 4 * kChunkGroups samples, channel, chunk - first); each thread takes kChunkGroups
// groups of 4 consecutive samples, 1024 samples apart, and issues all their loads before the
// first store. A group inside the signal (no reflection, no tail) moves as one float4 when the
// source is 16-byte aligned (vec bit 1); the rest goes sample by sample, with no divisions.
constexpr int kChunkGroups = 4;

__global__ __launch_bounds__(256) void demix_chunks_kernel(DemixArgs a, const float* __restrict__ mix,
                                                           int64_t first, int vec, float* __restrict__ parts) {
    const int c = (int)blockIdx.y;
    const int64_t k = first + (int64_t)blockIdx.z;
    const int64_t i = k * a.step;
    const int64_t length = min((int64_t)a.chunk, a.padded_len - i);
    const bool reflect_tail = length > a.tail_min;
    const float* xc = mix + (size_t)c * a.len;
    const int64_t lead = a.reflect_border ? a.border : 0;    // padded index p is signal index p - lead
    float v[kChunkGroups][4];
#pragma unroll
    for (int g = 0; g < kChunkGroups; g++) {
        const int t0 = ((int)blockIdx.x * kChunkGroups + g) * 1024 + (int)threadIdx.x * 4;
        const int64_t s0 = i + t0 - lead;                    // signal index of sample t0
        if ((vec & 2) && t0 + 3 < length && s0 >= 0 && s0 + 3 < a.len && (s0 & 3) == 0) {
            const float4 q = *reinterpret_cast<const float4*>(xc + s0);
            v[g][0] = q.x;
            v[g][1] = q.y;
            v[g][2] = q.z;
            v[g][3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = t0 + j;
                float x = 0.f;
                if (t < length) x = padded_mix(xc, i + t, a);
                else if (t < a.chunk && reflect_tail)                       // reflect_pad(src, length, 0, chunk - length)
                    x = padded_mix(xc, i + 2 * (length - 1) - t, a);        // (src/roformer.cpp:325)
                v[g][j] = x;
            }
        }
    }
    float* dst = parts + ((size_t)blockIdx.z * a.channels + c) * a.chunk;
#pragma unroll
    for (int g = 0; g < kChunkGroups; g++) {
        const int t0 = ((int)blockIdx.x * kChunkGroups + g) * 1024 + (int)threadIdx.x * 4;
        if (t0 >= a.chunk) break;
        if ((vec & 1) && t0 + 3 < a.chunk) {
            store_stream(reinterpret_cast<float4*>(dst + t0), make_float4(v[g][0], v[g][1], v[g][2], v[g][3]));
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (t0 + j < a.chunk) store_stream(dst + t0 + j, v[g][j]);
        }
    }
}

// Weight of chunk k at offset t (src/roformer.cpp:334-336; src/tfc_tdf.cpp:484-486).
__device__ __forceinline__ float chunk_weight(const float* __restrict__ window, int64_t k, int t, const DemixArgs& a) {
    if (k == 0) return t < a.fade ? 1.0f : window[t];
    if (k * a.step + a.reach >= a.padded_len && t >= a.chunk - a.fade) return 1.0f;
    return window[t];
}

// out[s][c][t] = sum_k y[k][s][c][p - k*step] * w_k / sum_k w_k, p = off + t, chunks in order.
// Each thread takes 4 consecutive samples: their chunk weights and weight sums are formed once
// and reused for every (stem, channel) plane, then each plane sums its chunk outputs in chunk
// order in double (float x float is exact in double), divides once and rounds once.
// NK: the most chunks that cover 4 consecutive samples for the plan, ceil((chunk + 3) / step).
constexpr int kOlaMaxChunks = 8;

template <int NK>
__global__ __launch_bounds__(256) void demix_ola_kernel(DemixArgs a, const float* __restrict__ y,
                                                        const float* __restrict__ window, int planes, int vec,
                                                        float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (t0 >= a.len) return;
    const int64_t p0 = (a.reflect_border ? a.border : 0) + t0;
    const int64_t k_lo = p0 >= a.chunk ? (p0 - a.chunk) / a.step + 1 : 0;   // first chunk with p0 < k*step + chunk
    const int64_t k_hi = (p0 + 3) / a.step;                                 // last chunk starting at or before p0 + 3
    const int nk = (int)min((int64_t)NK, k_hi - k_lo + 1);
    // Window values first (clamped positions, every load before the first wait), then the
    // chunk weights of src/roformer.cpp:334-336 by selection.
    float w[NK][4];
#pragma unroll
    for (int kk = 0; kk < NK; kk++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t tt = p0 + j - (k_lo + kk) * a.step;
            w[kk][j] = window[min(max(tt, (int64_t)0), (int64_t)a.chunk - 1)];
        }
    double cnt[4] = {0.0, 0.0, 0.0, 0.0};
    bool all4 = true;                                       // every (chunk, sample) of the span valid
#pragma unroll
    for (int kk = 0; kk < NK; kk++) {
        const int64_t k = k_lo + kk;
        const int64_t i = k * a.step;
        const int64_t length = min((int64_t)a.chunk, a.padded_len - i);
        const bool last = i + a.reach >= a.padded_len;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t tt = p0 + j - i;
            const bool ok = kk < nk && t0 + j < a.len && tt >= 0 && tt < length;
            float wt = w[kk][j];
            if (k == 0) wt = tt < a.fade ? 1.0f : wt;
            else if (last && tt >= a.chunk - a.fade) wt = 1.0f;
            w[kk][j] = ok ? wt : 0.f;
            if (ok) cnt[j] += (double)w[kk][j];
            if (kk < nk && !ok) all4 = false;
        }
    }
    const size_t stride = (size_t)planes * a.chunk;          // one chunk's output
    if (vec && all4 && nk > 0) {                             // nk = 0: a gap between chunks (step > chunk)
        // Chunks past nk re-read chunk nk - 1 and add +0.0 (an exact no-op: res never holds
        // -0.0), so that every load is used and none is sunk behind a branch.
        const float* src[NK];
#pragma unroll
        for (int kk = 0; kk < NK; kk++) {
            const int64_t k = k_lo + min(kk, nk - 1);
            src[kk] = y + (size_t)k * stride + (p0 - k * a.step);
        }
        for (int sc = 0; sc < planes; sc++) {
            float4 q[NK];
#pragma unroll
            for (int kk = 0; kk < NK; kk++) q[kk] = *reinterpret_cast<const float4*>(src[kk] + (size_t)sc * a.chunk);
            double res[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int kk = 0; kk < NK; kk++) {
                const bool in = kk < nk;
                res[0] += in ? (double)q[kk].x * (double)w[kk][0] : 0.0;
                res[1] += in ? (double)q[kk].y * (double)w[kk][1] : 0.0;
                res[2] += in ? (double)q[kk].z * (double)w[kk][2] : 0.0;
                res[3] += in ? (double)q[kk].w * (double)w[kk][3] : 0.0;
            }
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const double v = res[j] / cnt[j];
                o[j] = isfinite(v) ? (float)v : 0.0f;                         // np.nan_to_num
            }
            *reinterpret_cast<float4*>(out + (size_t)sc * a.len + t0) = make_float4(o[0], o[1], o[2], o[3]);
        }
        return;
    }
    for (int sc = 0; sc < planes; sc++) {
        double res[4] = {0.0, 0.0, 0.0, 0.0};
        for (int kk = 0; kk < nk; kk++) {
            const int64_t k = k_lo + kk;
            const float* src = y + (size_t)k * stride + (size_t)sc * a.chunk + (p0 - k * a.step);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int64_t tt = p0 + j - k * a.step;
                const int64_t length = min((int64_t)a.chunk, a.padded_len - k * a.step);
                if (t0 + j < a.len && tt >= 0 && tt < length) res[j] += (double)src[j] * (double)w[kk][j];
            }
        }
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const double v = res[j] / cnt[j];
            o[j] = isfinite(v) ? (float)v : 0.0f;                             // np.nan_to_num
        }
        float* dst = out + (size_t)sc * a.len + t0;
        if (vec && t0 + 3 < a.len) {
            store_stream(reinterpret_cast<float4*>(dst), make_float4(o[0], o[1], o[2], o[3]));
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (t0 + j < a.len) store_stream(dst + j, o[j]);
        }
    }
}

// The same sum for any overlap: one thread per (sample, plane).
__global__ __launch_bounds__(256) void demix_ola_generic_kernel(DemixArgs a, const float* __restrict__ y,
                                                                const float* __restrict__ window, int n_stems,
                                                                float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= a.len) return;
    const int sc = (int)blockIdx.y;                                      // s * C + c
    const int64_t p = (a.reflect_border ? a.border : 0) + t;
    const int64_t k_hi = p / a.step;
    const int64_t k_lo = p >= a.chunk ? (p - a.chunk) / a.step + 1 : 0;  // first chunk with p < k*step + chunk
    const size_t stride = (size_t)n_stems * a.channels * a.chunk;        // one chunk's output
    const float* yc = y + (size_t)sc * a.chunk;
    double res = 0.0, cnt = 0.0;
    for (int64_t k = k_lo; k <= k_hi; k++) {
        const int64_t i = k * a.step;
        const int tt = (int)(p - i);
        const int64_t length = min((int64_t)a.chunk, a.padded_len - i);
        if (tt >= length) continue;
        const float w = chunk_weight(window, k, tt, a);
        res += (double)yc[(size_t)k * stride + tt] * (double)w;
        cnt += (double)w;
    }
    const double v = res / cnt;
    out[(size_t)sc * a.len + t] = isfinite(v) ? (float)v : 0.0f;        // np.nan_to_num
}

void check_demix(const stx_demix* d) { STX_REQUIRE(d != nullptr && d->d_window != nullptr, "null demix plan"); }

// shifted[c][t] = mix[c][t + offset - max_shift] inside the input, else 0 (src/roformer.cpp:466-472).
// blockIdx.y is the channel, so no element needs a division.
__global__ __launch_bounds__(256) void shift_kernel(const float* __restrict__ mix, int64_t len, int64_t n,
                                                    int64_t delta, float* __restrict__ shifted) {
    const int64_t c = blockIdx.y;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < n; t += (int64_t)gridDim.x * 256) {
        const int64_t src = t + delta;
        shifted[c * n + t] = (src >= 0 && src < len) ? mix[c * len + src] : 0.0f;
    }
}

// est[i][t] += y[i][t + lead] / shifts, float as the reference (:474-476); est starts at 0.
// blockIdx.y is the plane i.
__global__ __launch_bounds__(256) void shift_accumulate_kernel(const float* __restrict__ y, int64_t n, int64_t lead,
                                                               int64_t len, int shifts, int first,
                                                               float* __restrict__ est) {
#pragma clang fp contract(off)
    const int64_t i = blockIdx.y;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < len; t += (int64_t)gridDim.x * 256) {
        const float v = y[i * n + lead + t] / (float)shifts;
        est[i * len + t] = first ? 0.0f + v : est[i * len + t] + v;
    }
}

// out[c][t] = mix[c][t] - est0[c][t] (:484).
__global__ __launch_bounds__(256) void complement_kernel(const float* __restrict__ mix, const float* __restrict__ est0,
                                                         int64_t n, float* __restrict__ out) {
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256)
        store_stream(out + e, mix[e] - est0[e]);
}

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>((n + 255) / 256, 1 << 20); }

struct Cancelled {};

// The workspace layout of stx_demix_track.
struct TrackLayout {
    size_t window, parts, y, shifted, yk, total;           // byte offsets and total size
};

TrackLayout track_layout(int channels, int64_t len, int chunk, int step, int n_stems, int batch, int shifts,
                         int sample_rate) {
    const int64_t max_shift = shifts > 0 ? sample_rate / 2 : 0;
    const int64_t n_max = len + max_shift;
    const DemixGeometry g = demix_geometry(n_max, chunk, step);
    auto align = [](size_t b) { return (b + 255) / 256 * 256; };
    TrackLayout L{};
    size_t o = 0;
    L.window = o;
    o += align(sizeof(float) * chunk);
    L.parts = o;
    o += align(sizeof(float) * (size_t)batch * channels * chunk);
    L.y = o;
    o += align(sizeof(float) * (size_t)g.n_chunks * n_stems * channels * chunk);
    L.shifted = o;
    if (shifts > 0) o += align(sizeof(float) * (size_t)channels * n_max);
    L.yk = o;
    if (shifts > 0) o += align(sizeof(float) * (size_t)n_stems * channels * n_max);
    L.total = o;
    return L;
}

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_demix_create(int64_t len, int channels, int chunk, int step, stx_demix** out) {
    return stx_demix_create_rules(len, channels, chunk, step, STX_DEMIX_ROFORMER, out);
}

STX_API stx_status stx_demix_create_rules(int64_t len, int channels, int chunk, int step, stx_demix_rules rules,
                                          stx_demix** out) {
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        STX_REQUIRE(channels >= 1, "bad channel count");
        const DemixGeometry g = demix_geometry(len, chunk, step, rules);
        STX_REQUIRE(g.n_chunks < (1LL << 31), "too many chunks");
        std::vector<float> w(chunk);
        demix_window(chunk, w.data(), rules);
        stx_demix* d = new stx_demix;
        d->g = g;
        d->channels = channels;
        hipError_t e = hipMalloc(&d->d_window, sizeof(float) * chunk);
        if (e == hipSuccess) e = hipMemcpy(d->d_window, w.data(), sizeof(float) * chunk, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            stx_demix_destroy(d);
            hip_check(e, "stx_demix_create");
        }
        *out = d;
    });
}

STX_API void stx_demix_destroy(stx_demix* d) {
    if (!d) return;
    (void)hipFree(d->d_window);
    delete d;
}

STX_API int64_t stx_demix_n_chunks(const stx_demix* d) { return d ? d->g.n_chunks : 0; }

STX_API stx_status stx_demix_chunks(const stx_demix* d, const float* mix, int64_t first, int64_t count, float* parts,
                                    stx_stream stream) {
    return guard([&] {
        check_demix(d);
        STX_REQUIRE(first >= 0 && count >= 0 && first + count <= d->g.n_chunks, "chunk range out of the plan");
        if (count == 0) return;
        STX_REQUIRE(mix && parts, "NULL buffer");
        STX_REQUIRE(count < 65536 && d->channels < 65536, "too many chunks or channels in one call");
        // bit 0: float4 stores into parts; bit 1: float4 loads from the channel rows of mix.
        const int vec = (d->g.chunk % 4 == 0 && (reinterpret_cast<uintptr_t>(parts) & 15) == 0 ? 1 : 0) |
                        (d->g.len % 4 == 0 && (reinterpret_cast<uintptr_t>(mix) & 15) == 0 ? 2 : 0);
        const dim3 grid((unsigned)((d->g.chunk + 1024 * kChunkGroups - 1) / (1024 * kChunkGroups)),
                        (unsigned)d->channels, (unsigned)count);
        hipLaunchKernelGGL(demix_chunks_kernel, grid, dim3(256), 0, as_stream(stream), args_of(d), mix, first, vec, parts);
        launch_check("demix_chunks_kernel");
    });
}

STX_API stx_status stx_demix_overlap_add(const stx_demix* d, const float* y, int n_stems, float* out,
                                         stx_stream stream) {
    return guard([&] {
        check_demix(d);
        STX_REQUIRE(n_stems >= 1, "bad stem count");
        STX_REQUIRE(y && out, "NULL buffer");
        STX_REQUIRE((int64_t)n_stems * d->channels < 65536, "too many stems * channels");
        const int planes = n_stems * d->channels;
        // Chunks covering 4 consecutive samples: at most ceil((chunk + 3) / step).
        if ((d->g.chunk + 3 + (int64_t)d->g.step - 1) / d->g.step <= kOlaMaxChunks) {
            const int64_t off = d->g.reflect_border ? d->g.border : 0;
            const int vec = d->g.chunk % 4 == 0 && d->g.step % 4 == 0 && off % 4 == 0 && d->g.len % 4 == 0 &&
                            (reinterpret_cast<uintptr_t>(y) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
            const unsigned blocks = (unsigned)((d->g.len + 1023) / 1024);
            const int nk = (int)((d->g.chunk + 3 + (int64_t)d->g.step - 1) / d->g.step);
            auto go = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, as_stream(stream), args_of(d), y, d->d_window,
                                   planes, vec, out);
            };
            switch (nk) {
                case 1: go(demix_ola_kernel<1>); break;
                case 2: go(demix_ola_kernel<2>); break;
                case 3: go(demix_ola_kernel<3>); break;
                case 4: go(demix_ola_kernel<4>); break;
                case 5: go(demix_ola_kernel<5>); break;
                case 6: go(demix_ola_kernel<6>); break;
                case 7: go(demix_ola_kernel<7>); break;
                default: go(demix_ola_kernel<8>); break;
            }
            launch_check("demix_ola_kernel");
        } else {
            dim3 grid((unsigned)((d->g.len + 255) / 256), planes);
            hipLaunchKernelGGL(demix_ola_generic_kernel, grid, dim3(256), 0, as_stream(stream), args_of(d), y,
                               d->d_window, n_stems, out);
            launch_check("demix_ola_generic_kernel");
        }
    });
}

}  // extern "C"

extern "C" {

STX_API size_t stx_demix_track_workspace_size(int channels, int64_t len, int chunk, int step, int n_stems, int batch,
                                              int shifts, int sample_rate) {
    try {
        if (channels < 1 || n_stems < 1 || batch < 1 || step < 1) return 0;
        return track_layout(channels, len, chunk, step, n_stems, batch, shifts, sample_rate).total;
    } catch (...) {
        return 0;
    }
}

STX_API stx_status stx_demix_track(const float* mix, int channels, int64_t len, int chunk, int num_overlap,
                                   int n_stems, int complement, int sample_rate, int batch, stx_separate_fn separate,
                                   void* separate_user, const stx_separate_options* options, float* out,
                                   void* workspace, size_t workspace_bytes, stx_stream stream) {
    stx_status st = guard([&] {
        const stx_separate_options opt = separate_options(options);
        if (len <= 0) fail(STX_STATUS_INVALID_ARGUMENT, "empty input");                   // :439
        if (opt.overlap >= 1.0f) fail(STX_STATUS_INVALID_ARGUMENT, "overlap must be < 1"); // :440
        STX_REQUIRE(channels >= 1 && n_stems >= 1 && chunk >= 1 && batch >= 1, "bad channels/stems/chunk/batch");
        STX_REQUIRE((int64_t)n_stems * channels < 65536, "too many stems * channels");
        STX_REQUIRE(mix && out && separate && workspace, "NULL argument");
        STX_REQUIRE(opt.shifts <= 0 || sample_rate >= 2, "bad sample rate for shifts");
        const int step = stx_demix_step(chunk, num_overlap, opt.overlap);
        STX_REQUIRE(step >= 1, "bad num_overlap");
        const TrackLayout L = track_layout(channels, len, chunk, step, n_stems, batch, opt.shifts, sample_rate);
        STX_REQUIRE(workspace_bytes >= L.total, "workspace too small: %zu bytes, need %zu", workspace_bytes, L.total);
        char* ws = static_cast<char*>(workspace);
        float* d_window = reinterpret_cast<float*>(ws + L.window);
        float* d_parts = reinterpret_cast<float*>(ws + L.parts);
        float* d_y = reinterpret_cast<float*>(ws + L.y);
        const hipStream_t s = as_stream(stream);
        {
            std::vector<float> w(chunk);
            demix_window(chunk, w.data());
            hip_check(hipMemcpyAsync(d_window, w.data(), sizeof(float) * chunk, hipMemcpyHostToDevice, s), "window");
            hip_check(hipStreamSynchronize(s), "window");
        }
        const int passes = std::max(1, opt.shifts);
        const int total = (int)(passes * demix_geometry(len, chunk, step).n_chunks);
        int done = 0;
        auto tick = [&] {                                                                   // :447-451
            if (opt.should_cancel && opt.should_cancel(opt.user)) throw Cancelled{};
            if (opt.progress && done > 0) opt.progress(opt.user, done, total);
            done++;
        };
        // One demix pass (:286-351) of x [C][n] into dst [S][C][n].
        auto demix = [&](const float* x, int64_t n, float* dst) {
            stx_demix plan;
            plan.g = demix_geometry(n, chunk, step);
            plan.channels = channels;
            plan.d_window = d_window;
            for (int64_t first = 0; first < plan.g.n_chunks; first += batch) {
                const int64_t count = std::min<int64_t>(batch, plan.g.n_chunks - first);
                for (int64_t k = 0; k < count; k++) tick();
                const stx_status cs = stx_demix_chunks(&plan, x, first, count, d_parts, stream);
                if (cs != STX_STATUS_OK) fail(cs, "%s", stx_last_error());
                float* yk = d_y + (size_t)first * n_stems * channels * chunk;
                const int32_t rc = separate(separate_user, d_parts, first, count, yk, stream);
                if (rc != 0) fail(STX_STATUS_RUNTIME_ERROR, "separator failed with %d", rc);
            }
            const stx_status os = stx_demix_overlap_add(&plan, d_y, n_stems, dst, stream);
            if (os != STX_STATUS_OK) fail(os, "%s", stx_last_error());
            plan.d_window = nullptr;
        };
        try {
            if (opt.shifts <= 0) {
                demix(mix, len, out);
            } else {
                // demucs' shift trick (:459-478): average over random offsets into a zero-padded copy.
                const int max_shift = sample_rate / 2;
                std::mt19937 rng(opt.seed);
                std::uniform_int_distribution<int> dist(0, max_shift - 1);
                float* d_shifted = reinterpret_cast<float*>(ws + L.shifted);
                float* d_yk = reinterpret_cast<float*>(ws + L.yk);
                for (int k = 0; k < opt.shifts; k++) {
                    const int offset = dist(rng);
                    const int64_t n = len + max_shift - offset;
                    hipLaunchKernelGGL(shift_kernel, dim3(grid_for(n), (unsigned)channels), dim3(256), 0, s, mix, len, n,
                                       (int64_t)offset - max_shift, d_shifted);
                    launch_check("shift_kernel");
                    demix(d_shifted, n, d_yk);
                    hipLaunchKernelGGL(shift_accumulate_kernel, dim3(grid_for(len), (unsigned)(n_stems * channels)),
                                       dim3(256), 0, s, d_yk, n, (int64_t)max_shift - offset, len, opt.shifts,
                                       k == 0 ? 1 : 0, out);
                    launch_check("shift_accumulate_kernel");
                }
            }
        } catch (const Cancelled&) {
            fail(STX_STATUS_CANCELLED, "cancelled");
        }
        if (opt.progress) opt.progress(opt.user, total, total);                             // :479
        if (complement) {
            const int64_t plane = (int64_t)channels * len;
            hipLaunchKernelGGL(complement_kernel, dim3(grid_for(plane)), dim3(256), 0, s, mix, out, plane,
                               out + (size_t)n_stems * plane);
            launch_check("complement_kernel");
        }
    });
    return st;
}

}  // extern "C"
