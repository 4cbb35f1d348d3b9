// htdemucs.hip — the HTDemucs host pre/post-processing around the model graph, and the
// split of apply_model, as gfx950 kernels over device buffers.
//
// Reference: HTDemucs::Impl::run (src/htdemucs.cpp:419-474) and HTDemucs::separate (:534-644):
//   * complex-as-channels pack of the spectrum + global mean/std normalisation (:424-436), the
//     waveform's normalisation (:438-441), and the inverse: denormalise the spectral branch
//     for the iSTFT (:465-468) and denormalise + add the time branch (:469-470);
//   * the mono-mix normalisation of separate() (:539-549);
//   * split(): TensorChunk padding (:552-561), triangular weights (:566-573), center_trim and
//     the weighted overlap-add (:589-607).
//
// The moments (mean_of / std_of, :293-302: double sums of d = x - x[0], so no cancellation
// occurs, and the unbiased std) and the normalisation run as one grid-synchronised kernel when
// the input fits in the registers of blocks that are all resident at once (one segment's
// spectrum or waveform) and the output does not overlap the input: each block loads its chunk
// once, the blocks exchange their partial sums (grid_sync.hpp) and normalise from registers.
// Otherwise two kernels: pass 1 writes one (sum d, sum d^2) pair in double per 8192 floats, and
// every block of pass 2 adds them in one fixed order into {mean, sd} (the same bits in every
// block) and normalises its 8192 values. The mono mix of separate() (1 or 2 channels, as many
// 8192-sample chunks as the device holds at once: 1,024 of two channels on MI355X, 3.2 minutes
// at 44.1 kHz) has a single-pass kernel of its own that keeps pass 1's chunks, arithmetic and
// order, so it gives the two kernels' bits. The split's
// overlap-add is in gather form: each output sample sums, in chunk order and in float like the
// reference's `out += weight * seg_out`, the <= ceil(seg / stride) chunks covering it, and
// divides by the summed weights, so it is bit-exact.
#include <algorithm>
#include <cmath>
#include <random>
#include <vector>

#include "common.hpp"
#include "grid_sync.hpp"

namespace stx {
namespace {

constexpr int kMomChunk = 8192;                  // floats per pass-1 block (256 threads x 32)

enum MomKind { MOM_FLAT = 0, MOM_MONO = 1 };

struct MomArgs {
    const float* x;              // FLAT: n floats; MONO: [C][n]
    long long n;                 // FLAT: floats; MONO: samples per channel
    int C;
    double* partial;             // [blocks][2]
};

__device__ __forceinline__ float mono_at(const float* x, long long n, int C, long long i) {
    double m = 0.0;
    for (int c = 0; c < C; c++) m += x[c * n + i];
    return (float)(m / C);
}

// mono_at for NC channels known at compile time (NC = 0: C at run time), written so that the
// channel loads of all J samples are issued before the first sum.
template <int NC, int J>
__device__ __forceinline__ void mono_batch(const float* x, long long n, int C, const long long (&idx)[J],
                                           float (&out)[J]) {
    if constexpr (NC > 0) {
        float v[J][NC];
#pragma unroll
        for (int j = 0; j < J; j++)
#pragma unroll
            for (int c = 0; c < NC; c++) v[j][c] = x[c * n + idx[j]];
#pragma unroll
        for (int j = 0; j < J; j++) {
            double m = 0.0;
#pragma unroll
            for (int c = 0; c < NC; c++) m += v[j][c];
            out[j] = (float)(m / NC);
        }
    } else {
#pragma unroll
        for (int j = 0; j < J; j++) out[j] = mono_at(x, n, C, idx[j]);
    }
}

__device__ __forceinline__ double block_sum(double v, double* red) {
    v = lane_sum<64>(v);
    const int w = (int)threadIdx.x / 64, lane = (int)threadIdx.x % 64;
    __syncthreads();                             // red may still be read by a previous call
    if (lane == 0) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];    // 256 threads: 4 waves, summed in one order
}

// This thread's sums of d = v - shift over its values of the pass-1 chunk at lo (value j at
// lo + threadIdx.x + 256 j), in j order; moments_kernel and mix_fused_kernel share it, so their
// chunk sums are the same bits.
__device__ __forceinline__ void moment_add(double d, double& s, double& q) {
    s += d;
    q += d * d;
}
template <int J>
__device__ __forceinline__ void chunk_moments(const float (&v)[J], long long lo, long long n, float shift, double& s,
                                              double& q) {
    s = 0.0;
    q = 0.0;
#pragma unroll
    for (int j = 0; j < J; j++)
        if (lo + threadIdx.x + 256LL * j < n) moment_add((double)v[j] - shift, s, q);
}

// KIND: MOM_FLAT or MOM_MONO; NC: channels of the mono mix (compile time; 0 = run time).
template <int KIND, int NC>
__global__ __launch_bounds__(256) void moments_kernel(MomArgs a) {
    __shared__ double red[4];
    const long long lo = (long long)blockIdx.x * kMomChunk;
    const float shift = KIND == MOM_MONO ? mono_at(a.x, a.n, a.C, 0) : a.x[0];
    constexpr int J = kMomChunk / 256;
    float v[J];
    long long idx[J];
#pragma unroll
    for (int j = 0; j < J; j++) idx[j] = min(lo + threadIdx.x + 256LL * j, a.n - 1);   // clamped
    if (KIND == MOM_MONO) {
        mono_batch<NC, J>(a.x, a.n, a.C, idx, v);
    } else {
#pragma unroll
        for (int j = 0; j < J; j++) v[j] = a.x[idx[j]];
    }
    double s, q;
    chunk_moments(v, lo, a.n, shift, s, q);
    s = block_sum(s, red);
    q = block_sum(q, red);
    if (threadIdx.x == 0) {
        a.partial[2 * blockIdx.x] = s;
        a.partial[2 * blockIdx.x + 1] = q;
        // The shift goes after the pairs, so pass 2 never reads it from x: pass 2 may write
        // its output over x, and a block that starts late would see normalised values there.
        if (blockIdx.x == 0) a.partial[2 * gridDim.x] = (double)shift;
    }
}

enum NormKind { NORM_CAC = 0, NORM_FLAT = 1, NORM_MIX = 2 };

// {mean, den} from the pass-1 pairs, added in a fixed order (thread t takes pairs t, t + 256, ...,
// then the block sum), so every block that calls it gets the same bits; the shift is the one
// pass 1 stored after its pairs (never x[0], which an in-place call may have overwritten); the unbiased std,
// floored at 1e-8 for the mix (std::max(std, 1e-8) keeps a NaN, as here); den = 1e-5 + sd
// (spectrum, waveform) or the floored sd (mix). Block (0, 0) writes {mean, sd} to stats.
template <int KIND>
__device__ __forceinline__ void fold_stats(const MomArgs& a, int n_partial, double* stats, double& mean, double& den,
                                           double* red) {
    double s = 0.0, q = 0.0;
    for (int b = (int)threadIdx.x; b < n_partial; b += 256) {
        s += a.partial[2 * b];
        q += a.partial[2 * b + 1];
    }
    s = block_sum(s, red);
    q = block_sum(q, red);
    const double shift = a.partial[2 * n_partial];
    const double n = (double)a.n;
    double sd = sqrt(fmax(q - s * (s / n), 0.0) / (n - 1.0));
    if (KIND == NORM_MIX) sd = sd < 1e-8 ? 1e-8 : sd;
    mean = shift + s / n;
    den = KIND == NORM_MIX ? sd : 1e-5 + sd;
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
        stats[0] = mean;
        stats[1] = sd;
    }
}

constexpr int kNormPer = 8;                      // elementwise kernels: values per thread
constexpr int kFoldPer = 32;                     // normalize_kernel: values per thread (8192 per block)

// Pass 2: (v - mean) / den in double, rounded once. Each block issues its loads, then folds the
// pass-1 pairs itself (fold_stats: the same bits in every block, from the L2), so no kernel
// runs between the passes. CAC: blockIdx.y is the channel, its re and im go to planes 2c and
// 2c + 1. FLAT / MIX: a flat walk.
template <int KIND>
__global__ __launch_bounds__(256) void normalize_kernel(MomArgs m, int n_partial, const float* x, float* y,
                                                        long long count, double* stats) {
    __shared__ double red[4];
    const long long e0 = (long long)blockIdx.x * (256 * kFoldPer) + threadIdx.x;
    if (KIND == NORM_CAC) {
        const long long c = blockIdx.y;
        const float2* src = reinterpret_cast<const float2*>(x) + c * count;
        float* re = y + 2 * c * count;
        float* im = re + count;
        float2 v[kFoldPer];
#pragma unroll
        for (int k = 0; k < kFoldPer; k++) v[k] = src[min(e0 + 256LL * k, count - 1)];
        double mean, den;
        fold_stats<KIND>(m, n_partial, stats, mean, den, red);
        // den is positive (or NaN): the moments of finite floats cannot overflow, so div_rn
        // gives the IEEE quotient with one reciprocal per thread.
        const double rden = 1.0 / den;
#pragma unroll
        for (int k = 0; k < kFoldPer; k++) {
            const long long e = e0 + 256LL * k;
            if (e < count) {
                store_stream(re + e, (float)div_rn((double)v[k].x - mean, den, rden));
                store_stream(im + e, (float)div_rn((double)v[k].y - mean, den, rden));
            }
        }
    } else {
        float v[kFoldPer];
#pragma unroll
        for (int k = 0; k < kFoldPer; k++) v[k] = x[min(e0 + 256LL * k, count - 1)];
        double mean, den;
        fold_stats<KIND>(m, n_partial, stats, mean, den, red);
        const double rden = 1.0 / den;
#pragma unroll
        for (int k = 0; k < kFoldPer; k++) {
            const long long e = e0 + 256LL * k;
            if (e < count) store_stream(y + e, (float)div_rn((double)v[k] - mean, den, rden));
        }
    }
}

// This thread's values of the chunk at lo. FULL (a whole chunk, x 16-byte aligned): unconditional
// float4 loads; otherwise clamped scalar loads (always-valid addresses, issued together), counted
// only where in range. Indices are 32-bit: the single pass covers fewer than 2^32 floats.
template <int VEC, bool FULL>
__device__ __forceinline__ void norm_load(const float* x, unsigned n, unsigned lo, float (&v)[VEC][4]) {
    constexpr unsigned NT = kGridThreads;
#pragma unroll
    for (int k = 0; k < VEC; k++) {
        const unsigned p = lo + (k * NT + threadIdx.x) * 4;
        if constexpr (FULL) {
            const float4 q = *reinterpret_cast<const float4*>(x + p);
            v[k][0] = q.x;
            v[k][1] = q.y;
            v[k][2] = q.z;
            v[k][3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) v[k][j] = x[min(p + j, n - 1)];
        }
    }
}

// Block sums of d = v - shift over the chunk at lo, in every thread: each thread adds its
// values in (k, j) order, then block_sum2_n.
template <int VEC, bool FULL>
__device__ __forceinline__ void norm_sums(const float (&v)[VEC][4], unsigned n, unsigned lo, double shift, double* red,
                                          double& s1, double& s2) {
    constexpr unsigned NT = kGridThreads;
    s1 = 0.0;
    s2 = 0.0;
#pragma unroll
    for (int k = 0; k < VEC; k++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool in = FULL || lo + (k * NT + threadIdx.x) * 4 + j < n;
            const double d = in ? (double)v[k][j] - shift : 0.0;
            s1 = s1 + d;
            s2 = fma(d, d, s2);
        }
    block_sum2_n<NT>(s1, s2, red);
}

// CAC: float e of the spectrum is channel c = e / (2 ft), bin i = (e % (2 ft)) / 2, re or im by
// its parity, and goes to plane 2 c (re) or 2 c + 1 (im) at i (cdiv divides by 2 ft).
template <int KIND, int VEC, bool FULL>
__device__ __forceinline__ void norm_fused_body(const float* x, float* y, unsigned n, unsigned ft, FastDiv cdiv,
                                                bool vec, double* stats, const GridSync& f, double* red, double* tot) {
    constexpr unsigned NT = kGridThreads;
    constexpr unsigned CH = NT * 4 * VEC;
    const unsigned lo = blockIdx.x * CH;
    const int nch = (int)((n + CH - 1) / CH);
    const double shift = (double)x[0];
    float v[VEC][4];
    norm_load<VEC, FULL>(x, n, lo, v);
    double s1, s2;
    norm_sums<VEC, FULL>(v, n, lo, shift, red, s1, s2);
    // A block whose wait gave up adds every chunk's sums itself, in the collector's order.
    grid_totals<NT>(f, 0, nch, s1, s2, red, tot, [&](double* t) {
        double p1 = 0.0, p2 = 0.0;
        for (int m = 0; m < nch; m++) {
            float w[VEC][4];
            norm_load<VEC, false>(x, n, m * CH, w);
            double q1, q2;
            norm_sums<VEC, false>(w, n, m * CH, shift, red, q1, q2);
            if ((int)threadIdx.x == m % (int)NT) {
                p1 += q1;
                p2 += q2;
            }
        }
        block_sum2_n<NT>(p1, p2, red);
        if (threadIdx.x == 0) {
            t[0] = p1;
            t[1] = p2;
        }
        __syncthreads();
    });
    const double nn = (double)n, s = tot[0], q = tot[1];
    const double mean = shift + s / nn;
    const double sd = sqrt(fmax(q - s * (s / nn), 0.0) / (nn - 1.0));
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        stats[0] = mean;
        stats[1] = sd;
    }
    const double den = 1e-5 + sd, rden = 1.0 / den;
    const bool pairs = KIND == NORM_CAC && vec && ft % 2 == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0;
    const unsigned ft2 = 2 * ft;
#pragma unroll
    for (int k = 0; k < VEC; k++) {
        const unsigned p = lo + (k * NT + threadIdx.x) * 4;
        if (!FULL && p >= n) continue;
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; j++) o[j] = (float)div_rn((double)v[k][j] - mean, den, rden);   // = (v - mean) / den
        if (KIND == NORM_FLAT) {
            if (FULL || (vec && p + 3 < n)) {
                store_stream(reinterpret_cast<float4*>(y + p), make_float4(o[0], o[1], o[2], o[3]));
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (p + j < n) store_stream(y + p + j, o[j]);
            }
        } else if (pairs && (FULL || p + 3 < n)) {
            // Two whole complex values of one channel (2 ft is a multiple of 4 and p of 4).
            const unsigned c = cdiv.div(p), i = (p - c * ft2) / 2;
            store_stream(reinterpret_cast<float2*>(y + 2 * c * ft + i), make_float2(o[0], o[2]));
            store_stream(reinterpret_cast<float2*>(y + (2 * c + 1) * ft + i), make_float2(o[1], o[3]));
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const unsigned e = p + j;
                if (e >= n) continue;
                const unsigned c = cdiv.div(e), r = e - c * ft2;
                store_stream(y + (2 * c + (r & 1)) * ft + r / 2, o[j]);
            }
        }
    }
}

// One launch of moments + normalise for NORM_CAC / NORM_FLAT: x is n floats (CAC: the complex64
// spectrum [C][ft] read as 2 C ft floats), VEC float4 per thread in chunks of kGridThreads * 4 *
// VEC floats. Same statistics formulas as fold_stats and the same per-element division as
// normalize_kernel; block 0 writes {mean, sd} to stats.
template <int KIND, int VEC>
__global__ __launch_bounds__(kGridThreads) void norm_fused_kernel(const float* x, float* y, unsigned n, unsigned ft,
                                                                  FastDiv cdiv, double* stats, GridSync f) {
    __shared__ double red[2 * kGridThreads / 64];
    __shared__ double tot[2];
    constexpr unsigned CH = kGridThreads * 4 * VEC;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && n % 4 == 0;
    if (vec && blockIdx.x * CH + CH <= n)
        norm_fused_body<KIND, VEC, true>(x, y, n, ft, cdiv, vec, stats, f, red, tot);
    else
        norm_fused_body<KIND, VEC, false>(x, y, n, ft, cdiv, vec, stats, f, red, tot);
}

// One launch of the mix's moments + normalise (NORM_MIX over the mono mix of NC = 1 or 2
// channels of n samples), bit-identical to moments_kernel<MOM_MONO, NC> + normalize_kernel<NORM_MIX>:
// block b holds pass 1's chunk b (kMomChunk samples, 256 threads, every channel's values in
// registers), forms the same mono values and chunk sums (chunk_moments, block_sum), and the
// blocks' totals are folded in fold_stats' order (thread t adds chunks t, t + 256, ..., then the
// block sum) by the grid barrier; then every block normalises its values of every channel with
// the same quotient. Block 0 writes {mean, sd} to stats.
// Values j < MixKeep<NC>::regs of each channel stay in registers across the barrier, the rest in
// the block's LDS (one slot per thread and value): the 32 or 64 values per thread, with what
// the barrier needs, would not fit in the 128 registers that four blocks per CU allow, and the
// LDS kept stays within a quarter of the CU's 160 KB.
template <int NC> struct MixKeep {
    static constexpr int regs = NC == 1 ? 16 : 13;
    static constexpr int lds = kMomChunk / 256 - regs;
};

template <int NC, bool FULL>
__device__ __forceinline__ void mix_fused_body(const float* x, float* y, long long n, double* stats, const GridSync& f,
                                               double* red, double* tot, float* keep) {
    constexpr int NT = 256;
    constexpr int J = kMomChunk / NT;
    constexpr int JR = MixKeep<NC>::regs;
    const int nblk = (int)gridDim.x;
    const long long lo = (long long)blockIdx.x * kMomChunk;
    const float shift = mono_at(x, n, NC, 0);
    // Loads and stores at a uniform base (this chunk of channel c) plus a 32-bit byte offset,
    // which the compiler issues as base-register + offset-register forms instead of one 64-bit
    // address per value.
    auto at = [](auto* base, unsigned bytes) {
        using T = std::remove_pointer_t<decltype(base)>;
        return reinterpret_cast<T*>(reinterpret_cast<std::conditional_t<std::is_const_v<T>, const char*, char*>>(base) + bytes);
    };
    const unsigned tb = 4u * threadIdx.x, lastb = 4u * (unsigned)(n - 1 - lo);   // lastb: tail chunk only
    float raw[J][NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float* xc = x + c * n + lo;
#pragma unroll
        for (int j = 0; j < J; j++) raw[j][c] = *at(xc, FULL ? tb + 1024u * j : min(tb + 1024u * j, lastb));
    }
    __builtin_amdgcn_sched_barrier(0);          // every load issued before the sums start
    // mono_batch's value and chunk_moments' sums, one value at a time (the same operations in
    // the same order, so the same bits as pass 1, without a second array of J values).
    double s = 0.0, q = 0.0;
#pragma unroll
    for (int j = 0; j < J; j++) {
        double m = 0.0;
#pragma unroll
        for (int c = 0; c < NC; c++) m += raw[j][c];
        const float v = (float)(m / NC);
        if (FULL || lo + threadIdx.x + 256LL * j < n) moment_add((double)v - shift, s, q);
    }
#pragma unroll
    for (int j = JR; j < J; j++)
#pragma unroll
        for (int c = 0; c < NC; c++) keep[((j - JR) * NC + c) * NT + threadIdx.x] = raw[j][c];
    // Opaque from here: the compiler would otherwise keep the sums' double conversions of the
    // values alive across the barrier for the quotients below (twice the registers).
#pragma unroll
    for (int j = 0; j < JR; j++)
#pragma unroll
        for (int c = 0; c < NC; c++) asm volatile("" : "+v"(raw[j][c]));
    s = block_sum(s, red);
    q = block_sum(q, red);
    // A block whose wait gave up forms every chunk's sums itself, in the same order (one value
    // at a time: its registers hold this block's values meanwhile).
    grid_totals<NT>(f, 0, nblk, s, q, red, tot, [&](double* t) {
        double p1 = 0.0, p2 = 0.0;
        for (int b = 0; b < nblk; b++) {
            const long long l = (long long)b * kMomChunk;
            double q1 = 0.0, q2 = 0.0;
#pragma unroll 1
            for (int jj = 0; jj < J; jj++) {
                const long long i = min(l + threadIdx.x + 256LL * jj, n - 1);
                double m = 0.0;
#pragma unroll
                for (int c = 0; c < NC; c++) m += x[c * n + i];
                if (l + threadIdx.x + 256LL * jj < n) moment_add((double)(float)(m / NC) - shift, q1, q2);
            }
            q1 = block_sum(q1, red);
            q2 = block_sum(q2, red);
            if ((int)threadIdx.x == b % NT) {
                p1 += q1;
                p2 += q2;
            }
        }
        block_sum2_n<NT>(p1, p2, red);
        if (threadIdx.x == 0) {
            t[0] = p1;
            t[1] = p2;
        }
        __syncthreads();
    });
    // fold_stats<NORM_MIX> from the totals.
    const double nn = (double)n, ts = tot[0], tq = tot[1];
    double sd = sqrt(fmax(tq - ts * (ts / nn), 0.0) / (nn - 1.0));
    sd = sd < 1e-8 ? 1e-8 : sd;
    const double mean = (double)shift + ts / nn, den = sd, rden = 1.0 / den;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        stats[0] = mean;
        stats[1] = sd;
    }
#pragma unroll
    for (int j = JR; j < J; j++)
#pragma unroll
        for (int c = 0; c < NC; c++) raw[j][c] = keep[((j - JR) * NC + c) * NT + threadIdx.x];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        float* yc = y + c * n + lo;
#pragma unroll
        for (int j = 0; j < J; j++)
            if (FULL || tb + 1024u * j <= lastb)
                store_stream(at(yc, tb + 1024u * j), (float)div_rn((double)raw[j][c] - mean, den, rden));
    }
}

template <int NC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void mix_fused_kernel(
    const float* x, float* y, long long n, double* stats, GridSync f) {
    __shared__ double red[2 * 256 / 64];
    __shared__ double tot[2];
    __shared__ float keep[MixKeep<NC>::lds > 0 ? MixKeep<NC>::lds * NC * 256 : 1];
    if ((long long)(blockIdx.x + 1) * kMomChunk <= n) mix_fused_body<NC, true>(x, y, n, stats, f, red, tot, keep);
    else mix_fused_body<NC, false>(x, y, n, stats, f, red, tot, keep);
}

// Spectral branch denormalise: ox [S][2C][FT] -> complex64 spec [S][C][FT]; blockIdx.y = s * C + c.
__global__ __launch_bounds__(256) void cac_denorm_kernel(const float* ox, float2* spec, long long ft,
                                                         const double* stats) {
#pragma clang fp contract(off)
    const double mean = stats[0], sd = stats[1];
    const long long sc = blockIdx.y;
    const float* re = ox + 2 * sc * ft;                    // planes 2c and 2c + 1 of source s
    const float* im = re + ft;
    float2* out = spec + sc * ft;
    const long long e0 = (long long)blockIdx.x * (256 * kNormPer) + threadIdx.x;
    float vr[kNormPer], vi[kNormPer];
#pragma unroll
    for (int k = 0; k < kNormPer; k++) {
        const long long e = min(e0 + 256LL * k, ft - 1);
        vr[k] = re[e];
        vi[k] = im[e];
    }
#pragma unroll
    for (int k = 0; k < kNormPer; k++) {
        const long long e = e0 + 256LL * k;
        if (e < ft) store_stream(out + e, make_float2((float)((double)vr[k] * sd + mean), (float)((double)vi[k] * sd + mean)));
    }
}

// Time branch: out = (float)(t * sd + mean) + y, the add in float.
__global__ __launch_bounds__(256) void time_add_kernel(const float* t, const float* y, float* out, long long n,
                                                       const double* stats) {
#pragma clang fp contract(off)
    const long long e = (long long)blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const double mean = stats[0], sd = stats[1];
    const float a = (float)((double)t[e] * sd + mean);
    store_stream(out + e, a + y[e]);
}

// ------------------------------------------------------------------------------- split
struct SegArgs {
    const float* buf;            // [C][total]
    float* parts;                // [count][C][seg]
    long long total, offset;
    int length, seg, stride, first, C;
};

// parts[k][c][i] = buf[c][start_k + i] where buf has it, else 0 (TensorChunk.padded). Each
// thread writes 4 consecutive samples (one float4 when segment rows are 16-byte aligned).
template <bool V4>
__global__ __launch_bounds__(256) void segments_kernel(SegArgs a) {
    const int k = (int)blockIdx.z, c = (int)blockIdx.y;
    const int i0 = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
    if (i0 >= a.seg) return;
    const int off = (a.first + k) * a.stride;
    const int clen = min(a.seg, a.length - off);
    const long long j0 = a.offset + off - (a.seg - clen) / 2 + i0;
    const float* row = a.buf + (long long)c * a.total;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const long long j = j0 + q;
        const bool in = j >= 0 && j < a.total;
        const float t = row[in ? j : 0];
        v[q] = in ? t : 0.0f;
    }
    float* dst = a.parts + ((long long)k * a.C + c) * a.seg + i0;
    if (V4) {
        store_stream(reinterpret_cast<float4*>(dst), make_float4(v[0], v[1], v[2], v[3]));
    } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (i0 + q < a.seg) store_stream(dst + q, v[q]);
    }
}

struct OlaArgs {
    const float* y;              // [n_chunks][tracks][seg]
    float* out;                  // [tracks][length]
    int tracks, length, seg, stride, n_chunks;
    float mx;                    // the weights' maximum
    FastDiv sdiv;                // division by stride
};

constexpr int kOlaPer = 2;
constexpr int kOlaMaxCover = 8;                  // chunks covering one sample: ceil(seg / stride)

constexpr int kOlaTracks = 4;                    // tracks per thread (they share the weights)

// Gather form of split()'s overlap-add. A thread takes kOlaPer samples i and kOlaTracks tracks;
// the weights of the <= NK chunks covering i and their float sum are formed once and shared by
// the tracks (the divisions dominate the cost otherwise). The chunk values are loaded from
// clamped, always-valid addresses, all before the first use, and summed in chunk order over the
// chunks that cover i, exactly as the reference's `out += weight * seg_out`, then divided by the
// summed weights.
template <int NK>
__global__ __launch_bounds__(256) void split_ola_kernel(OlaArgs a) {
#pragma clang fp contract(off)
    const int sc0 = (int)blockIdx.y * kOlaTracks;
    const int half = a.seg / 2;
#pragma unroll
    for (int p = 0; p < kOlaPer; p++) {
        const int i = ((int)blockIdx.x * kOlaPer + p) * 256 + (int)threadIdx.x;
        if (i >= a.length) return;
        const int k_hi = (int)min(a.sdiv.div((unsigned)i), (unsigned)(a.n_chunks - 1));
        long long base[NK];                          // offset of (chunk, track 0, sample) in y
        bool in[NK];
        float w[NK];
#pragma unroll
        for (int q = 0; q < NK; q++) {               // chunk k_hi - q
            const int k = max(k_hi - q, 0);
            const int off = k * a.stride, r = i - off;
            const int clen = min(a.seg, a.length - off);
            const int trim = (a.seg - clen) / 2;
            in[q] = k_hi - q >= 0 && r < a.seg;
            base[q] = (long long)k * a.tracks * a.seg + trim + min(min(r, a.seg - 1), clen - 1);
            w[q] = (float)(r < half ? r + 1 : a.seg - r) / a.mx;
        }
        float v[kOlaTracks][NK];
#pragma unroll
        for (int t = 0; t < kOlaTracks; t++) {
            const long long sc = min(sc0 + t, a.tracks - 1);
#pragma unroll
            for (int q = 0; q < NK; q++) v[t][q] = a.y[base[q] + sc * a.seg];
        }
        float sw = 0.0f;
#pragma unroll
        for (int q = NK - 1; q >= 0; q--)            // chunk order: ascending k
            if (in[q]) sw = sw + w[q];
#pragma unroll
        for (int t = 0; t < kOlaTracks; t++) {
            if (sc0 + t >= a.tracks) break;
            float acc = 0.0f;
#pragma unroll
            for (int q = NK - 1; q >= 0; q--) {
                if (in[q]) {
                    const float prod = w[q] * v[t][q];
                    acc = acc + prod;
                }
            }
            store_stream(a.out + (long long)(sc0 + t) * a.length + i, acc / sw);
        }
    }
}

// ---------------------------------------------------------------- separate() accumulation
// res[t][i] = (first ? 0 : res[t][i]) + o[t][src_off + i]: one shift's output, added in shift order
// (src/htdemucs.cpp:622-624); blockIdx.y = t. The first shift also adds to 0.0f, as the
// reference's zeroed res does.
__global__ __launch_bounds__(256) void shift_add_kernel(float* res, const float* o, long long len, long long o_len,
                                                        long long src_off, int first) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= len) return;
    const long long t = blockIdx.y;
    const float v = o[t * o_len + src_off + i];
    const float prev = first ? 0.0f : res[t * len + i];
    res[t * len + i] = prev + v;
}

// estimates[s] += w_s * (res[s] / shifts) for every source with w_s != 0 (:625-631, the
// division by shifts of :626 when shifts > 0); the first model adds to 0.0f. blockIdx.y = s.
struct BagArgs {
    float* est;
    const float* res;
    long long plane;             // C * len
    float w[64];
    float shifts;                // 0: no division
    int first;
};

__global__ __launch_bounds__(256) void bag_add_kernel(BagArgs a) {
#pragma clang fp contract(off)
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.plane) return;
    const int s = (int)blockIdx.y;
    const long long e = (long long)s * a.plane + i;
    const float w = a.w[s];
    if (w == 0.0f) {
        if (a.first) a.est[e] = 0.0f;
        return;
    }
    const float prev = a.first ? 0.0f : a.est[e];
    float v = a.res[e];
    if (a.shifts != 0.0f) v = v / a.shifts;
    const float p = w * v;
    a.est[e] = prev + p;
}

// out = (float)(est / totals[s] * ref_std + ref_mean) (:633-638); blockIdx.y = s.
struct FinalArgs {
    float* est;
    long long plane;
    float totals[64];
    const double* stats;
};

__global__ __launch_bounds__(256) void bag_final_kernel(FinalArgs a) {
#pragma clang fp contract(off)
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.plane) return;
    const int s = (int)blockIdx.y;
    const long long e = (long long)s * a.plane + i;
    const float q = a.est[e] / a.totals[s];
    a.est[e] = (float)((double)q * a.stats[1] + a.stats[0]);
}

long long mom_blocks(long long n) { return (n + kMomChunk - 1) / kMomChunk; }

// Normalisation workspace: the single-pass kernel's area (kGridSyncBytes), then the pass-1 pairs
// and the shift (one double, padded to 16 bytes).
size_t norm_ws_bytes(long long n) { return kGridSyncBytes + (size_t)mom_blocks(n) * 16 + 16; }

unsigned grid256(long long n) { return (unsigned)((n + 255) / 256); }

struct Cancelled {};

struct SepLayout {
    size_t mix, stats, mom, parts, y, o, res, total;
    int stride, max_chunks;
    long long max_view;
};

SepLayout sep_layout(int C, long long len, int seg, int S, int batch, int shifts, int sr, float overlap) {
    SepLayout L{};
    const double ov = overlap < 0.0f ? 0.25 : (double)overlap;
    L.stride = (int)((1.0 - ov) * seg);
    const long long max_shift = shifts > 0 ? sr / 2 : 0;
    L.max_view = len + max_shift;                // a shift view's length is len + max_shift - offset
    L.max_chunks = L.stride > 0 ? (int)((L.max_view + L.stride - 1) / L.stride) : 0;
    auto align = [](size_t b) { return (b + 255) / 256 * 256; };
    size_t o = 0;
    L.mix = o;
    o += align(sizeof(float) * (size_t)C * len);
    L.stats = o;
    o += align(2 * sizeof(double));
    L.mom = o;
    o += align(norm_ws_bytes(len));
    L.parts = o;
    o += align(sizeof(float) * (size_t)batch * C * seg);
    L.y = o;
    o += align(sizeof(float) * (size_t)L.max_chunks * S * C * seg);
    L.o = o;
    o += align(sizeof(float) * (size_t)S * C * L.max_view);
    L.res = o;
    if (shifts > 0) o += align(sizeof(float) * (size_t)S * C * len);
    L.total = o;
    return L;
}

void check_ws(void* ws, size_t bytes, long long n) {
    STX_REQUIRE(ws != nullptr, "normalise: workspace is NULL");
    STX_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "normalise: workspace must be 16-byte aligned");
    STX_REQUIRE(bytes >= norm_ws_bytes(n), "normalise: workspace too small (%zu < %zu bytes)", bytes,
                norm_ws_bytes(n));
}

// The single-pass kernel at the smallest width whose blocks (at most kGridMaxBlocks) are all
// resident at once; false when none is.
template <int NK, int VEC>
bool try_norm_fused(const float* x, float* y, long long n, long long ft, double* stats, void* ws, hipStream_t s) {
    const long long ch = (long long)kGridThreads * 4 * VEC;
    const long long nch = (n + ch - 1) / ch;
    if (nch > kGridMaxBlocks) return false;
    // The single pass needs x unchanged until every block has read it (a block whose wait gives
    // up re-reads all of x): y must not overlap x (y has as many floats as x).
    if (overlaps(x, sizeof(float) * (size_t)n, y, sizeof(float) * (size_t)n)) return false;
    if (nch > resident_blocks(reinterpret_cast<const void*>(&norm_fused_kernel<NK, VEC>), s)) return false;
    // n <= kGridMaxBlocks chunks of at most 8192 floats: every index fits 32 bits.
    hipLaunchKernelGGL((norm_fused_kernel<NK, VEC>), dim3((unsigned)nch), dim3(kGridThreads), 0, s, x, y, (unsigned)n,
                       (unsigned)ft, FastDiv((unsigned)(2 * ft)), stats, grid_sync_at(ws));
    launch_check("norm_fused_kernel");
    return true;
}

// mix_fused_kernel when y does not overlap x, C is 1 or 2 and all its blocks are resident at
// once (at most kGridMaxGroups * kGridMaxBlocks: the sync area's records); false otherwise.
template <int NC>
bool try_mix_fused(const float* x, float* y, long long n, double* stats, void* ws, hipStream_t s) {
    const long long nb = mom_blocks(n);
    if (nb > (long long)kGridMaxGroups * kGridMaxBlocks) return false;
    if (overlaps(x, sizeof(float) * (size_t)(NC * n), y, sizeof(float) * (size_t)(NC * n))) return false;
    if (nb > resident_blocks(reinterpret_cast<const void*>(&mix_fused_kernel<NC>), s, 256)) return false;
    hipLaunchKernelGGL((mix_fused_kernel<NC>), dim3((unsigned)nb), dim3(256), 0, s, x, y, n, stats, grid_sync_at(ws));
    launch_check("mix_fused_kernel");
    return true;
}

template <int MK, int NK>
void normalize(const float* x, long long n_mom, long long count, int C, float* y, double* stats, void* ws,
               hipStream_t s) {
    // Pass 2 reads and writes the same indices for FLAT and MIX, so y == x is safe there; any
    // other overlap is refused, and so is any for CAC, whose planes move every value.
    const size_t bytes = sizeof(float) * (size_t)(NK == NORM_CAC ? n_mom : count);
    if (overlaps(x, bytes, y, bytes))
        STX_REQUIRE(NK != NORM_CAC && x == y, "normalise: the output overlaps the input%s",
                    NK == NORM_CAC ? "" : " without being the same buffer");
    if constexpr (NK != NORM_MIX) {
        if (try_norm_fused<NK, 1>(x, y, n_mom, count, stats, ws, s) || try_norm_fused<NK, 2>(x, y, n_mom, count, stats, ws, s) ||
            try_norm_fused<NK, 4>(x, y, n_mom, count, stats, ws, s))
            return;
    } else {
        if ((C == 1 && try_mix_fused<1>(x, y, n_mom, stats, ws, s)) || (C == 2 && try_mix_fused<2>(x, y, n_mom, stats, ws, s)))
            return;
    }
    double* partial = reinterpret_cast<double*>(static_cast<char*>(ws) + kGridSyncBytes);
    const long long nb = mom_blocks(n_mom);
    STX_REQUIRE(nb < (1LL << 31) && count < (1LL << 40), "normalise: too many elements");
    MomArgs m{x, n_mom, C, partial};
    if constexpr (MK == MOM_MONO) {
        if (C == 1) hipLaunchKernelGGL((moments_kernel<MK, 1>), dim3((unsigned)nb), dim3(256), 0, s, m);
        else if (C == 2) hipLaunchKernelGGL((moments_kernel<MK, 2>), dim3((unsigned)nb), dim3(256), 0, s, m);
        else hipLaunchKernelGGL((moments_kernel<MK, 0>), dim3((unsigned)nb), dim3(256), 0, s, m);
    } else {
        hipLaunchKernelGGL((moments_kernel<MK, 0>), dim3((unsigned)nb), dim3(256), 0, s, m);
    }
    launch_check("moments_kernel");
    const long long blocks = (count + 256 * kFoldPer - 1) / (256 * kFoldPer);
    STX_REQUIRE(blocks < (1LL << 31), "normalise: too many elements");
    hipLaunchKernelGGL((normalize_kernel<NK>), dim3((unsigned)blocks, NK == NORM_CAC ? (unsigned)C : 1u), dim3(256),
                       0, s, m, (int)nb, x, y, count, stats);
    launch_check("normalize_kernel");
}

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API size_t stx_htdemucs_norm_workspace_size(int64_t n) { return norm_ws_bytes(n > 0 ? n : 1); }

STX_API stx_status stx_htdemucs_cac_normalize(const float* spec, int channels, int n_bins, int n_frames, float* mag,
                                              double* stats, void* workspace, size_t workspace_bytes,
                                              stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(channels > 0 && n_bins > 0 && n_frames > 0, "cac_normalize: empty spectrum");
        STX_REQUIRE(spec && mag && stats, "NULL buffer");
        const long long ft = (long long)n_bins * n_frames, n = 2LL * channels * ft;
        STX_REQUIRE(n > 1, "cac_normalize: need at least two values for the unbiased std");
        STX_REQUIRE(channels < 65536, "cac_normalize: too many channels");
        check_ws(workspace, workspace_bytes, n);
        normalize<MOM_FLAT, NORM_CAC>(spec, n, ft, channels, mag, stats, workspace, as_stream(stream));
    });
}

STX_API stx_status stx_htdemucs_wave_normalize(const float* x, int64_t n, float* out, double* stats, void* workspace,
                                               size_t workspace_bytes, stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(n > 1, "wave_normalize: need at least two samples for the unbiased std");
        STX_REQUIRE(x && out && stats, "NULL buffer");
        check_ws(workspace, workspace_bytes, n);
        normalize<MOM_FLAT, NORM_FLAT>(x, n, n, 1, out, stats, workspace, as_stream(stream));
    });
}

STX_API stx_status stx_htdemucs_mix_normalize(const float* mix, int channels, int64_t len, float* out, double* stats,
                                              void* workspace, size_t workspace_bytes, stx_stream stream) {
    return guard([&] {
        if (len <= 0) fail(STX_STATUS_INVALID_ARGUMENT, "empty input");     // src/htdemucs.cpp:537
        STX_REQUIRE(channels > 0, "mix_normalize: channels must be positive");
        STX_REQUIRE(mix && out && stats, "NULL buffer");
        check_ws(workspace, workspace_bytes, len);
        normalize<MOM_MONO, NORM_MIX>(mix, len, (long long)channels * len, channels, out, stats, workspace,
                                      as_stream(stream));
    });
}

STX_API stx_status stx_htdemucs_cac_denormalize(const float* ox, int n_sources, int channels, int n_bins, int n_frames,
                                                const double* stats, float* spec, stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(n_sources >= 0 && channels > 0 && n_bins > 0 && n_frames >= 0, "cac_denormalize: bad shape");
        const long long ft = (long long)n_bins * n_frames, count = (long long)n_sources * channels * ft;
        if (count == 0) return;
        STX_REQUIRE(ox && spec && stats, "NULL buffer");
        const long long blocks = (ft + 256 * kNormPer - 1) / (256 * kNormPer);
        STX_REQUIRE(blocks < (1LL << 31) && (long long)n_sources * channels < 65536, "cac_denormalize: too large");
        hipLaunchKernelGGL(cac_denorm_kernel, dim3((unsigned)blocks, (unsigned)(n_sources * channels)), dim3(256), 0,
                           as_stream(stream), ox, reinterpret_cast<float2*>(spec), ft, stats);
        launch_check("cac_denorm_kernel");
    });
}

STX_API stx_status stx_htdemucs_time_add(const float* xt, const float* y, int64_t n, const double* stats, float* out,
                                         stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(n >= 0, "time_add: negative count");
        if (n == 0) return;
        STX_REQUIRE(xt && y && out && stats, "NULL buffer");
        const long long blocks = (n + 255) / 256;
        STX_REQUIRE(blocks < (1LL << 31), "time_add: too many elements");
        hipLaunchKernelGGL(time_add_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), xt, y, out,
                           (long long)n, stats);
        launch_check("time_add_kernel");
    });
}

STX_API stx_status stx_htdemucs_split_plan(int length, int segment, float overlap, int* stride, int* n_chunks) {
    return guard([&] {
        STX_REQUIRE(stride && n_chunks, "NULL output");
        STX_REQUIRE(length > 0 && segment > 0, "split_plan: length and segment must be positive");
        const double ov = overlap < 0.0f ? 0.25 : (double)overlap;          // src/htdemucs.cpp:564-566
        const int st = (int)((1.0 - ov) * segment);
        if (st <= 0) fail(STX_STATUS_INVALID_ARGUMENT, "overlap must be < 1");
        *stride = st;
        *n_chunks = (int)(((long long)length + st - 1) / st);
    });
}

STX_API stx_status stx_htdemucs_segments(const float* buf, int channels, int64_t total, int64_t offset, int length,
                                         int segment, int stride, int first, int count, float* parts,
                                         stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(channels > 0 && total >= 0 && length > 0 && segment > 0 && stride > 0, "segments: bad geometry");
        const int n = (int)(((long long)length + stride - 1) / stride);
        STX_REQUIRE(first >= 0 && count >= 0 && (long long)first + count <= n, "segments: chunks out of range");
        if (count == 0) return;
        STX_REQUIRE(buf && parts, "NULL buffer");
        STX_REQUIRE(total > 0, "segments: empty buffer");
        STX_REQUIRE(count < 65536 && channels < 65536, "segments: too many chunks or channels");
        SegArgs a{buf, parts, total, offset, length, segment, stride, first, channels};
        const dim3 grid((unsigned)((segment + 1023) / 1024), (unsigned)channels, (unsigned)count);
        if (segment % 4 == 0 && (reinterpret_cast<uintptr_t>(parts) & 15) == 0)
            hipLaunchKernelGGL(segments_kernel<true>, grid, dim3(256), 0, as_stream(stream), a);
        else
            hipLaunchKernelGGL(segments_kernel<false>, grid, dim3(256), 0, as_stream(stream), a);
        launch_check("segments_kernel");
    });
}

STX_API stx_status stx_htdemucs_split_overlap_add(const float* y, int tracks, int length, int segment, int stride,
                                                  float* out, stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(tracks > 0 && length > 0 && segment > 0 && stride > 0, "split_overlap_add: bad geometry");
        STX_REQUIRE(stride <= segment, "split_overlap_add: stride > segment leaves samples with no weight");
        STX_REQUIRE(y && out, "NULL buffer");
        STX_REQUIRE(tracks < 65536, "split_overlap_add: too many tracks");
        OlaArgs a{};
        a.y = y;
        a.out = out;
        a.tracks = tracks;
        a.length = length;
        a.seg = segment;
        a.stride = stride;
        a.n_chunks = (int)(((long long)length + stride - 1) / stride);
        const int half = segment / 2;
        a.mx = (float)std::max(half, segment - half);
        a.sdiv = FastDiv((unsigned)stride);
        const int cover = (segment + stride - 1) / stride;
        if (cover > kOlaMaxCover)
            fail(STX_STATUS_UNSUPPORTED, "split_overlap_add: more than %d segments cover a sample", kOlaMaxCover);
        const dim3 grid((unsigned)((length + 256 * kOlaPer - 1) / (256 * kOlaPer)),
                        (unsigned)((tracks + kOlaTracks - 1) / kOlaTracks));
        const hipStream_t s = as_stream(stream);
        switch (cover) {
        case 1: hipLaunchKernelGGL(split_ola_kernel<1>, grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL(split_ola_kernel<2>, grid, dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL(split_ola_kernel<3>, grid, dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL(split_ola_kernel<4>, grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL(split_ola_kernel<kOlaMaxCover>, grid, dim3(256), 0, s, a); break;
        }
        launch_check("split_ola_kernel");
    });
}

STX_API size_t stx_htdemucs_separate_workspace_size(int channels, int64_t len, int segment, int n_sources, int batch,
                                                   int shifts, int sample_rate, float overlap) {
    if (channels <= 0 || len <= 0 || segment <= 0 || n_sources <= 0 || batch <= 0) return 0;
    return sep_layout(channels, len, segment, n_sources, batch, std::max(0, shifts), sample_rate, overlap).total;
}

STX_API stx_status stx_htdemucs_separate(const float* mix, int channels, int64_t len, int segment, int n_sources,
                                         int n_models, const float* bag_weights, int sample_rate, int batch,
                                         stx_model_fn forward, void* forward_user,
                                         const stx_separate_options* options, float* out, void* workspace,
                                         size_t workspace_bytes, stx_stream stream) {
    return guard([&] {
        const stx_separate_options opt = separate_options(options);
        if (len <= 0) fail(STX_STATUS_INVALID_ARGUMENT, "empty input");                        // :537
        STX_REQUIRE(len < (1LL << 31) - sample_rate, "separate: input too long");
        STX_REQUIRE(channels >= 1 && n_sources >= 1 && n_sources <= 64 && n_models >= 1 && segment >= 2 && batch >= 1,
                    "separate: bad channels/sources/models/segment/batch");
        STX_REQUIRE((long long)n_sources * channels < 65536, "separate: too many tracks");
        STX_REQUIRE(mix && out && forward && workspace && bag_weights, "NULL argument");
        const int shifts = std::max(0, opt.shifts);
        STX_REQUIRE(shifts == 0 || sample_rate >= 2, "separate: bad sample rate for shifts");
        const SepLayout L = sep_layout(channels, len, segment, n_sources, batch, shifts, sample_rate, opt.overlap);
        if (L.stride <= 0) fail(STX_STATUS_INVALID_ARGUMENT, "overlap must be < 1");            // :566
        STX_REQUIRE(workspace_bytes >= L.total, "workspace too small: %zu bytes, need %zu", workspace_bytes, L.total);
        char* ws = static_cast<char*>(workspace);
        float* d_mix = reinterpret_cast<float*>(ws + L.mix);
        double* d_stats = reinterpret_cast<double*>(ws + L.stats);
        float* d_parts = reinterpret_cast<float*>(ws + L.parts);
        float* d_y = reinterpret_cast<float*>(ws + L.y);
        float* d_o = reinterpret_cast<float*>(ws + L.o);
        float* d_res = reinterpret_cast<float*>(ws + L.res);
        const hipStream_t s = as_stream(stream);
        const int S = n_sources, C = channels, tracks = S * C;
        // Normalise by the mono mix (:539-549).
        normalize<MOM_MONO, NORM_MIX>(mix, len, (long long)C * len, C, d_mix, d_stats, ws + L.mom, s);

        const int passes_per_split = (int)((len + L.stride - 1) / L.stride);                    // :577
        const int total_passes = n_models * std::max(1, shifts) * passes_per_split;
        int done = 0;
        std::mt19937 rng(opt.seed);                                                              // :580
        std::vector<float> totals(S, 0.0f);
        // split() of one view of d_mix into d_o [tracks][length] (:589-607).
        auto split = [&](int model, long long offset, int length) {
            const int n = (int)(((long long)length + L.stride - 1) / L.stride);
            for (int first = 0; first < n; first += batch) {
                const int count = std::min(batch, n - first);
                for (int k = 0; k < count; k++)
                    if (opt.should_cancel && opt.should_cancel(opt.user)) throw Cancelled{};       // :591
                const stx_status cs = stx_htdemucs_segments(d_mix, C, len, offset, length, segment, L.stride, first,
                                                            count, d_parts, stream);
                if (cs != STX_STATUS_OK) fail(cs, "%s", stx_last_error());
                float* yk = d_y + (size_t)first * tracks * segment;
                const int32_t rc = forward(forward_user, model, d_parts, count, yk, stream);
                if (rc != 0) fail(STX_STATUS_RUNTIME_ERROR, "model forward failed with %d", rc);
                for (int k = 0; k < count; k++)
                    if (opt.progress) opt.progress(opt.user, ++done, total_passes);               // :603
            }
            const stx_status os = stx_htdemucs_split_overlap_add(d_y, tracks, length, segment, L.stride, d_o, stream);
            if (os != STX_STATUS_OK) fail(os, "%s", stx_last_error());
        };
        try {
            for (int mi = 0; mi < n_models; mi++) {
                const float* res = d_o;
                if (shifts == 0) {
                    split(mi, 0, (int)len);
                } else {
                    // Shift views of the mix zero-padded by max_shift on both sides (:612-624): a view
                    // at `offset` into the padded copy is the view at offset - max_shift of the mix
                    // itself with zeros outside it, which is what the segment kernel reads.
                    const int max_shift = sample_rate / 2;
                    std::uniform_int_distribution<int> dist(0, max_shift);
                    for (int k = 0; k < shifts; k++) {
                        const int offset = dist(rng);
                        const int length = (int)len + max_shift - offset;
                        split(mi, (long long)offset - max_shift, length);
                        hipLaunchKernelGGL(shift_add_kernel, dim3(grid256(len), (unsigned)tracks), dim3(256), 0, s,
                                           d_res, d_o, (long long)len, (long long)length,
                                           (long long)(max_shift - offset), k == 0 ? 1 : 0);
                        launch_check("shift_add_kernel");
                    }
                    res = d_res;
                }
                BagArgs b{};
                b.est = out;
                b.res = res;
                b.plane = (long long)C * len;
                for (int si = 0; si < S; si++) {
                    b.w[si] = bag_weights[(size_t)mi * S + si];
                    totals[si] += b.w[si];                                                       // :627
                }
                b.shifts = shifts > 0 ? (float)shifts : 0.0f;
                b.first = mi == 0 ? 1 : 0;
                hipLaunchKernelGGL(bag_add_kernel, dim3(grid256(b.plane), (unsigned)S), dim3(256), 0, s, b);
                launch_check("bag_add_kernel");
            }
        } catch (const Cancelled&) {
            fail(STX_STATUS_CANCELLED, "cancelled");
        }
        FinalArgs f{};
        f.est = out;
        f.plane = (long long)C * len;
        for (int si = 0; si < S; si++) f.totals[si] = totals[si];
        f.stats = d_stats;
        hipLaunchKernelGGL(bag_final_kernel, dim3(grid256(f.plane), (unsigned)S), dim3(256), 0, s, f);
        launch_check("bag_final_kernel");
    });
}

}  // extern "C"
