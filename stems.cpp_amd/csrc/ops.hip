// ops.hip — the ggml normalisation, softmax, activation, broadcast and RoPE ops of the
// stems.cpp graphs, as hand-written gfx950 kernels over ggml-style tensor descriptors
// (stx_tensor: ne[4] element counts with ne[0] fastest, nb[4] byte strides, rows contiguous).
//
// Reference call sites (ggml's own sources are not part of the reference tree; what is
// restated here is the semantics those calls rely on):
//   GROUP_NORM + affine     src/htdemucs.cpp:114-128 (group_norm_rows), :223-227 (norm_out)
//   NORM (+ affine)         src/htdemucs.cpp:213-215 (layer_norm)
//   RMS_NORM * gamma        src/roformer.cpp:34,96-98 (rms)
//   SOFT_MAX_EXT            src/roformer.cpp:127, src/htdemucs.cpp:238
//   GELU (erf)              src/roformer.cpp:147, src/htdemucs.cpp:136,154,210,246
//   GLU = a * sigmoid(b)    src/htdemucs.cpp:105-110 (ne2), src/roformer.cpp:199-202 (ne0)
//   ADD / MUL broadcast     src/htdemucs.cpp:100,139,220,250-251, src/roformer.cpp:97,136,145,148
//   ROPE                    src/roformer.cpp:109-113
//
// Every op here is HBM-bound: each kernel reads its operands and writes its result once.
// Row ops keep a row in registers (a wave or a fraction of one per row) and reduce with
// cross-lane shuffles; normalisation statistics and softmax sums are accumulated in double
// (full rate on CDNA4), so results are one rounding away from the double closed form.
// ADD, MUL and x + h * s round after every operation, exactly as the separate ggml ops do, and
// are bit-exact with that definition.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "grid_sync.hpp"
#include "tensor.hpp"

namespace stx {
namespace {

constexpr int kWave = 64;

// Row r (flattened over ne1, ne2, ne3) of t.
__device__ __forceinline__ char* row_ptr(const T4& t, long long r) {
    const long long i1 = r % t.ne[1];
    const long long q = r / t.ne[1];
    const long long i2 = q % t.ne[2];
    const long long i3 = q / t.ne[2];
    return t.data + i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}

// Row r of t when the rows are equally spaced `rs` bytes apart (rs > 0), else row_ptr.
__device__ __forceinline__ char* row_ptr_flat(const T4& t, long long r, long long rs) {
    return rs > 0 ? t.data + r * rs : row_ptr(t, r);
}

// Byte distance between consecutive rows if all rows of t are equally spaced, else 0: the
// row dimensions of extent > 1 must form one chain (each stride = previous stride * extent).
long long row_spacing(const T4& t) {
    long long rs = 0, expect = 0;
    for (int i = 1; i < 4; i++) {
        if (t.ne[i] <= 1) continue;
        if (rs == 0) {
            rs = t.nb[i];
        } else if (t.nb[i] != expect) {
            return 0;
        }
        expect = t.nb[i] * t.ne[i];
    }
    return rs > 0 ? rs : 4 * t.ne[0];          // a single row: any positive spacing works
}

// Sum over a 256-thread block in a fixed order (deterministic). red holds 4 doubles.
__device__ __forceinline__ double block_sum(double v, double* red) {
    v = lane_sum<kWave>(v);
    __syncthreads();
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// 1/d from the hardware reciprocal refined by one Newton-Raphson step (d normal, finite).
__device__ __forceinline__ float rcp_nr(float d) {
    const float r = __builtin_amdgcn_rcpf(d);
    return fmaf(r, fmaf(-d, r, 1.0f), r);
}

// gelu(x) = x Phi(x), Phi(x) = (1 + erf(x/sqrt2)) / 2, without a library erf/erfc/exp call and
// without branches (~40 VALU instructions), within 9 ulp everywhere (a float32 simulation of
// these exact steps, with the hardware exp2 and reciprocal taken 1 ulp off, against erfc in
// double: at most 8.4 ulp on x < 0, 3 ulp on x > 1):
//   Q = Phi(-|x|) = exp(-x^2/2) erfcx(|x|/sqrt2) / 2, and Phi(x) = Q for x < 0, 1 - Q otherwise.
//   erfcx(u) = exp(u^2) erfc(u) = t P(t) with t = 1 / (1 + u/2) (the form of Hastings'
//     approximation, Abramowitz & Stegun 7.1.26), one reciprocal; P has degree 12, fitted for
//     this library over all u >= 0 by weighted least squares in double, its coefficients
//     rounded to float one at a time from the top with the rest refitted.
//   The exponential is 2^y with y = -(x + dx)^2 / (2 ln 2) formed as a head and tail (x^2 split
//     exactly by an fma, the constant split in two floats), so it costs one ulp instead of
//     ~x^2 ulps; 2^y = 2^n * 2^f, n = rint(y head), f in [-1/2, 1/2] on the hardware exp2.
//   x > 10: Phi(x) = 1 to float precision; x < -15: gelu underflows (0 * x keeps -0 and NaN,
//     and gives NaN at -inf like x * (1 + erf(x/sqrt2)) / 2 does).
// gelu_erf_hl takes its argument as a float head x plus a small tail dx (x + dx is the value)
// so that a fused producer can hand over a double result without rounding it first: in the
// negative tail d ln gelu / d ln x ~ 1 + x^2, so one ulp of input rounding would become ~x^2
// ulps of output error; gelu_erf_dt takes the double itself.

// Phi(-|x|) = e erfcx(|x|/sqrt2) / 2, given e = exp(-x^2/2).
__device__ __forceinline__ float gelu_phi_neg(float x, float e) {
    const float t = rcp_nr(fmaf(0.5f, fabsf(x) * 0.70710678118654752440f, 1.f));
    float p = -3.032274731e-02f;
    p = fmaf(p, t, 1.836623400e-01f);
    p = fmaf(p, t, -4.440974593e-01f);
    p = fmaf(p, t, 5.091602206e-01f);
    p = fmaf(p, t, -2.279437780e-01f);
    p = fmaf(p, t, 8.653792553e-03f);
    p = fmaf(p, t, -6.725899875e-02f);
    p = fmaf(p, t, -2.435513539e-03f);
    p = fmaf(p, t, 8.313342929e-02f);
    p = fmaf(p, t, 1.764382720e-01f);
    p = fmaf(p, t, 2.468204200e-01f);
    p = fmaf(p, t, 2.820952535e-01f);
    p = fmaf(p, t, 2.820947766e-01f);
    return 0.5f * e * (t * p);
}

__device__ __forceinline__ float gelu_erf_hl(float x, float dx) {
    // No contraction here: yh must be the rounded product that the fma residual refers to
    // (hipcc fuses a separate multiply and add by default, which would count the residual twice).
#pragma clang fp contract(off)
    constexpr float C1 = -0x1.715476p-1f;                 // -1/(2 ln 2) = C1 + C2 to 3e-16
    constexpr float C2 = -0x1.4ae0cp-27f;
    const float h = x * x;
    const float l = fmaf(x, x, -h);                       // x^2 = h + l exactly
    const float yh = h * C1;
    const float yl = fmaf(h, C1, -yh) + fmaf(h, C2, fmaf(2.f * x, dx, l) * C1);
    const float n = rintf(fmaxf(yh, -200.f));             // |x| > 15 is selected away below
    const float g = gelu_phi_neg(x, ldexpf(__builtin_amdgcn_exp2f((yh - n) + yl), (int)n));
    const float ph = x < 0.f ? g : 1.f - g;
    return x > 10.f ? x + dx : x < -15.f ? x * 0.f : fmaf(ph, dx, x * ph);
}

// gelu of a double argument t (a fused producer's result before rounding), the same
// approximation with the exponent -t^2 / (2 ln 2) formed in double instead of as a float head
// and tail, and the product of the rounded t and Phi at the end (a float multiply: in the
// simulation below the bound is unchanged, the conditioning of the tail lies in the exponent,
// which stays in double). Branch- and select-free in the ranges the
// float formula has to clamp: the 1/2 is folded into P's coefficients (exact), t > ~5.3 gives
// Q < 2^-25, so Phi = 1 - Q = 1 exactly and the result is t rounded; t < ~-13.2 underflows Q to
// 0 (the exponent is floored at -200 so that 2^n stays finite), giving t * 0 = -0 as the float
// formula's x * 0; |t| is capped at 1e30 in the reciprocal's argument so that +inf gives inf
// (not 0 * inf), -inf gives NaN like x * (1 + erf(x/sqrt2)) / 2, NaN stays NaN.
// The reciprocal is the hardware's (1 ulp) without a Newton step: the step changes the result
// by less than the polynomial's own error (measured on gfx950 over 4.2 M points in [-16, 12]
// against erfc in double: at most 5.3 ulp without the step, 5.4 with it).
// About 27 VALU instructions.
__device__ __forceinline__ float gelu_erf_dt(double t) {
    const float x = (float)t;
    const double y = t * t * -0x1.71547652b82fep-1;
    const double n = rint(fmax(y, -200.0));
    const float e = ldexpf(__builtin_amdgcn_exp2f((float)(y - n)), (int)n);
    const float r = __builtin_amdgcn_rcpf(fmaf(fminf(fabsf(x), 1e30f), 0.35355339059327376220f, 1.f));   // 1 / (1 + |x| / (2 sqrt2))
    float p = -1.5161373655e-02f;                         // P / 2 (see gelu_phi_neg)
    p = fmaf(p, r, 9.183117002e-02f);
    p = fmaf(p, r, -2.2204872965e-01f);
    p = fmaf(p, r, 2.545801103e-01f);
    p = fmaf(p, r, -1.139718890e-01f);
    p = fmaf(p, r, 4.3268962765e-03f);
    p = fmaf(p, r, -3.3629499375e-02f);
    p = fmaf(p, r, -1.2177567695e-03f);
    p = fmaf(p, r, 4.1566714645e-02f);
    p = fmaf(p, r, 8.82191360e-02f);
    p = fmaf(p, r, 1.234102100e-01f);
    p = fmaf(p, r, 1.4104762675e-01f);
    p = fmaf(p, r, 1.410473883e-01f);
    const float g = e * (r * p);                          // Phi(-|t|)
    return x * (x < 0.f ? g : 1.f - g);                   // rounded t times Phi: at most 1 ulp more
}

__device__ __forceinline__ float gelu_erf(float x) { return gelu_erf_hl(x, 0.f); }

// ------------------------------------------------------------------ NORM / RMS_NORM
// LANES lanes per row (a power of two <= 64) with VPL values per lane: rows up to LANES*VPL.
struct RowNormArgs {
    T4 src, dst;
    const float* gamma;      // * gamma[ne0] after normalising (may be NULL)
    const float* beta;       // + beta[ne0] (may be NULL)
    float eps;
    int rms;                 // 1: x / sqrt(mean x^2 + eps); 0: (x - mean) / sqrt(var + eps)
    long long rs_src, rs_dst; // row spacing in bytes when equally spaced, else 0
    int vec_params;          // gamma and beta (where given) 16-byte aligned
};

__device__ __forceinline__ float norm_out(const RowNormArgs& a, float x, double mean, double scale, int i) {
    double o = ((double)x - mean) * scale;
    if (a.gamma) o *= (double)a.gamma[i];
    if (a.beta) o += (double)a.beta[i];
    return (float)o;
}

template <int LANES, int VPL>
__global__ __launch_bounds__(256) void row_norm_kernel(RowNormArgs a) {
    const int lane = (int)threadIdx.x % LANES;
    const long long gid = ((long long)blockIdx.x * 256 + threadIdx.x) / LANES;
    const long long stride = (long long)gridDim.x * (256 / LANES);
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const int n = (int)a.src.ne[0];
    for (long long r = gid; r < rows; r += stride) {
        const float* x = reinterpret_cast<const float*>(row_ptr(a.src, r));
        float* y = reinterpret_cast<float*>(row_ptr(a.dst, r));
        float v[VPL];
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int i = lane + k * LANES;
            v[k] = i < n ? x[i] : 0.f;
        }
        double mean = 0.0, ss = 0.0;
        if (!a.rms) {
            double s = 0.0;
#pragma unroll
            for (int k = 0; k < VPL; k++) s += (double)v[k];
            mean = lane_sum<LANES>(s) / n;
        }
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const double d = (double)v[k] - mean;
            ss += lane + k * LANES < n ? d * d : 0.0;
        }
        ss = lane_sum<LANES>(ss);
        const double scale = 1.0 / sqrt(ss / n + (double)a.eps);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int i = lane + k * LANES;
            if (i < n) y[i] = norm_out(a, v[k], mean, scale, i);
        }
    }
}

// Rows longer than 2048: one block per row; the second pass re-reads the row (from cache).
__global__ __launch_bounds__(256) void row_norm_big_kernel(RowNormArgs a) {
    __shared__ double red[4];
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const int n = (int)a.src.ne[0];
    const int tid = (int)threadIdx.x;
    for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* x = reinterpret_cast<const float*>(row_ptr(a.src, r));
        float* y = reinterpret_cast<float*>(row_ptr(a.dst, r));
        double mean = 0.0;
        if (!a.rms) {
            double s = 0.0;
            for (int i = tid; i < n; i += 256) s += (double)x[i];
            mean = block_sum(s, red) / n;
        }
        double ss = 0.0;
        for (int i = tid; i < n; i += 256) {
            const double d = (double)x[i] - mean;
            ss += d * d;
        }
        ss = block_sum(ss, red);
        const double scale = 1.0 / sqrt(ss / n + (double)a.eps);
        for (int i = tid; i < n; i += 256) y[i] = norm_out(a, x[i], mean, scale, i);
    }
}

// ------------------------------------------------------------------------- SOFT_MAX
// softmax(scale * x) along ne0. exp(s*x - max) takes its argument in double from exact
// products (two floats multiply exactly in double), split into a float head and tail:
// exp(h + t) = expf(h) * (1 + t). The row sum is accumulated in double and each value divided
// once in double.
struct SoftmaxArgs {
    T4 src, dst;
    float scale;
    long long rs_src, rs_dst; // row spacing in bytes when equally spaced, else 0
};

__device__ __forceinline__ float exp_split(double d) {
    const float h = (float)d;
    const float t = isfinite(d) ? (float)(d - (double)h) : 0.f;
    return expf(h) * (1.0f + t);
}

template <int LANES, int VPL>
__global__ __launch_bounds__(256) void softmax_kernel(SoftmaxArgs a) {
    const int lane = (int)threadIdx.x % LANES;
    const long long gid = ((long long)blockIdx.x * 256 + threadIdx.x) / LANES;
    const long long stride = (long long)gridDim.x * (256 / LANES);
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const int n = (int)a.src.ne[0];
    const double sc = (double)a.scale;
    // The maximum of s*x is s*max(x) for s >= 0 and s*min(x) otherwise: negate x for s < 0.
    const float sgn = a.scale < 0.f ? -1.f : 1.f;
    for (long long r = gid; r < rows; r += stride) {
        const float* x = reinterpret_cast<const float*>(row_ptr(a.src, r));
        float* y = reinterpret_cast<float*>(row_ptr(a.dst, r));
        float v[VPL];
        float m = -INFINITY;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int i = lane + k * LANES;
            v[k] = i < n ? x[i] : 0.f;
            if (i < n) m = fmaxf(m, sgn * v[k]);
        }
        const double ms = (double)(sgn * lane_max<LANES>(m)) * sc;
        double sum = 0.0;
        float e[VPL];
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            e[k] = lane + k * LANES < n ? exp_split((double)v[k] * sc - ms) : 0.f;
            sum += (double)e[k];
        }
        const double inv = 1.0 / lane_sum<LANES>(sum);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int i = lane + k * LANES;
            if (i < n) y[i] = (float)((double)e[k] * inv);
        }
    }
}

// ------------------------------------------------------- row ops with vector loads
// The same row ops with 16-byte loads and stores: a row of n floats is split into a head up
// to the first 16-byte boundary (0..3 floats), an aligned body of float4 and a tail (0..3
// floats). LANES lanes share a row: lane l holds body float4 l, l + LANES, ... (coalesced),
// lanes 0..2 also hold the head floats and lanes 4..6 the tail floats. Used when source and
// destination rows have the same alignment (the host checks it), so stores split the same way.
struct RowSplit {
    int h, nb4, tl;
};

__device__ __forceinline__ RowSplit row_split(const float* x, int n) {
    int h = (int)((4u - ((unsigned)(reinterpret_cast<uintptr_t>(x) >> 2) & 3u)) & 3u);
    h = min(h, n);
    const int nb4 = (n - h) >> 2;
    return {h, nb4, n - h - 4 * nb4};
}

// Index of the head or tail float owned by `lane`, or -1.
__device__ __forceinline__ int row_extra(const RowSplit& sp, int lane) {
    if (lane < sp.h) return lane;
    if (lane >= 4 && lane < 4 + sp.tl) return sp.h + 4 * sp.nb4 + (lane - 4);
    return -1;
}

// The row's float4 body (slots past nb4 read as 0) and this lane's head/tail float. Every
// load is issued before the first wait: slots past nb4 re-read float4 nb4 - 1 and are zeroed
// afterwards (a row with no aligned float4 reads none), and a lane with no extra float reads
// x[0].
template <int LANES, int V4>
__device__ __forceinline__ void row_load(const float* x, const RowSplit& sp, int lane, float (&v)[4 * V4], float& e,
                                         int& ei) {
    const float4* b = reinterpret_cast<const float4*>(x + sp.h);
    ei = row_extra(sp, lane);
    e = x[max(ei, 0)];
    if (sp.nb4 > 0) {
        float4 f[V4];
#pragma unroll
        for (int k = 0; k < V4; k++) f[k] = b[min(lane + LANES * k, sp.nb4 - 1)];
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const bool in = lane + LANES * k < sp.nb4;
            v[4 * k] = in ? f[k].x : 0.f;
            v[4 * k + 1] = in ? f[k].y : 0.f;
            v[4 * k + 2] = in ? f[k].z : 0.f;
            v[4 * k + 3] = in ? f[k].w : 0.f;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4 * V4; k++) v[k] = 0.f;
    }
    if (ei < 0) e = 0.f;
}

// gamma/beta float4 of the body slots (1 and 0 where absent), loaded before the row's
// reductions so that their latency overlaps them.
template <int LANES, int V4>
__device__ __forceinline__ void row_params(const float* gamma, const float* beta, const RowSplit& sp, int lane,
                                           float4 (&g)[V4], float4 (&bb)[V4]) {
#pragma unroll
    for (int k = 0; k < V4; k++) {
        const int i0 = sp.h + 4 * min(lane + LANES * k, max(sp.nb4 - 1, 0));
        g[k] = gamma ? *reinterpret_cast<const float4*>(gamma + i0) : make_float4(1.f, 1.f, 1.f, 1.f);
        bb[k] = beta ? *reinterpret_cast<const float4*>(beta + i0) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int LANES, int V4>
__global__ __launch_bounds__(256) void row_norm_v4_kernel(RowNormArgs a) {
    const int lane = (int)threadIdx.x % LANES;
    const long long gid = ((long long)blockIdx.x * 256 + threadIdx.x) / LANES;
    const long long stride = (long long)gridDim.x * (256 / LANES);
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const int n = (int)a.src.ne[0];
    for (long long r = gid; r < rows; r += stride) {
        const float* x = reinterpret_cast<const float*>(row_ptr_flat(a.src, r, a.rs_src));
        float* y = reinterpret_cast<float*>(row_ptr_flat(a.dst, r, a.rs_dst));
        const RowSplit sp = row_split(x, n);
        float v[4 * V4], e;
        int ei;
        row_load<LANES, V4>(x, sp, lane, v, e, ei);
        const bool pvec = a.vec_params && sp.h == 0 && sp.nb4 > 0;   // parameter float4 at i0 aligned
        float4 gq[V4], bq[V4];
        if (pvec) row_params<LANES, V4>(a.gamma, a.beta, sp, lane, gq, bq);
        double mean = 0.0;
        if (!a.rms) {
            double s = ei >= 0 ? (double)e : 0.0;
#pragma unroll
            for (int k = 0; k < 4 * V4; k++) s += (double)v[k];       // invalid slots hold 0
            mean = lane_sum<LANES>(s) / n;
        }
        double ss = 0.0;
        if (ei >= 0) ss = ((double)e - mean) * ((double)e - mean);
#pragma unroll
        for (int k = 0; k < V4; k++) {
            if (lane + LANES * k < sp.nb4) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const double d = (double)v[4 * k + j] - mean;
                    ss += d * d;
                }
            }
        }
        ss = lane_sum<LANES>(ss);
        const double scale = 1.0 / sqrt(ss / n + (double)a.eps);
        const float scale_f = (float)scale;
        float4* yb = reinterpret_cast<float4*>(y + sp.h);
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const int q = lane + LANES * k;
            if (q < sp.nb4) {
                const int i0 = sp.h + 4 * q;
                float o[4];
                if (pvec && !a.beta) {
                    // No offset to cancel against: (x - mean) in double, then the scale and gamma
                    // products in float (at most ~2 ulp from the double result).
                    const float gg[4] = {gq[k].x, gq[k].y, gq[k].z, gq[k].w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float d = a.rms ? v[4 * k + j] : (float)((double)v[4 * k + j] - mean);
                        o[j] = a.gamma ? (d * scale_f) * gg[j] : d * scale_f;
                    }
                } else if (pvec) {
                    const float gg[4] = {gq[k].x, gq[k].y, gq[k].z, gq[k].w};
                    const float bv[4] = {bq[k].x, bq[k].y, bq[k].z, bq[k].w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        double t = ((double)v[4 * k + j] - mean) * scale;
                        if (a.gamma) t *= (double)gg[j];
                        t += (double)bv[j];
                        o[j] = (float)t;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++) o[j] = norm_out(a, v[4 * k + j], mean, scale, i0 + j);
                }
                store_stream(yb + q, make_float4(o[0], o[1], o[2], o[3]));
            }
        }
        if (ei >= 0) store_stream(y + ei, norm_out(a, e, mean, scale, ei));
    }
}

template <int LANES, int V4>
__global__ __launch_bounds__(256) void softmax_v4_kernel(SoftmaxArgs a) {
    const int lane = (int)threadIdx.x % LANES;
    const long long gid = ((long long)blockIdx.x * 256 + threadIdx.x) / LANES;
    const long long stride = (long long)gridDim.x * (256 / LANES);
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const int n = (int)a.src.ne[0];
    const double sc = (double)a.scale;
    const float sgn = a.scale < 0.f ? -1.f : 1.f;      // max of s*x is s*max(x) for s >= 0
    for (long long r = gid; r < rows; r += stride) {
        const float* x = reinterpret_cast<const float*>(row_ptr_flat(a.src, r, a.rs_src));
        float* y = reinterpret_cast<float*>(row_ptr_flat(a.dst, r, a.rs_dst));
        const RowSplit sp = row_split(x, n);
        float v[4 * V4], e;
        int ei;
        row_load<LANES, V4>(x, sp, lane, v, e, ei);
        float m = ei >= 0 ? sgn * e : -INFINITY;
#pragma unroll
        for (int k = 0; k < V4; k++)
            if (lane + LANES * k < sp.nb4)
#pragma unroll
                for (int j = 0; j < 4; j++) m = fmaxf(m, sgn * v[4 * k + j]);
        const double ms = (double)(sgn * lane_max<LANES>(m)) * sc;
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const bool ok = lane + LANES * k < sp.nb4;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[4 * k + j] = ok ? exp_split((double)v[4 * k + j] * sc - ms) : 0.f;
                sum += (double)v[4 * k + j];
            }
        }
        if (ei >= 0) {
            e = exp_split((double)e * sc - ms);
            sum += (double)e;
        }
        const double inv = 1.0 / lane_sum<LANES>(sum);
        float4* yb = reinterpret_cast<float4*>(y + sp.h);
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const int q = lane + LANES * k;
            if (q < sp.nb4)
                store_stream(yb + q, make_float4((float)((double)v[4 * k] * inv), (float)((double)v[4 * k + 1] * inv),
                                                 (float)((double)v[4 * k + 2] * inv), (float)((double)v[4 * k + 3] * inv)));
        }
        if (ei >= 0) store_stream(y + ei, (float)((double)e * inv));
    }
}

// Maximum over a 256-thread block (exact in any order). red holds 4 floats.
__device__ __forceinline__ float block_max(float v, float* red) {
    v = lane_max<kWave>(v);
    __syncthreads();
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Rows of 2049..8192 floats (the HTDemucs attention scores: Nk = 2,688 frequency tokens): one
// 256-thread block per row, the row held in registers (V4 float4 per thread, split as in
// softmax_v4_kernel), the maximum and the double sum reduced over the block's four waves.
template <int V4>
__global__ __launch_bounds__(256) void softmax_block_kernel(SoftmaxArgs a) {
    __shared__ float redf[4];
    __shared__ double redd[4];
    const int lane = (int)threadIdx.x;
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const int n = (int)a.src.ne[0];
    const double sc = (double)a.scale;
    const float sgn = a.scale < 0.f ? -1.f : 1.f;
    for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* x = reinterpret_cast<const float*>(row_ptr_flat(a.src, r, a.rs_src));
        float* y = reinterpret_cast<float*>(row_ptr_flat(a.dst, r, a.rs_dst));
        const RowSplit sp = row_split(x, n);
        float v[4 * V4], e;
        int ei;
        row_load<256, V4>(x, sp, lane, v, e, ei);
        float m = ei >= 0 ? sgn * e : -INFINITY;
#pragma unroll
        for (int k = 0; k < V4; k++)
            if (lane + 256 * k < sp.nb4)
#pragma unroll
                for (int j = 0; j < 4; j++) m = fmaxf(m, sgn * v[4 * k + j]);
        const double ms = (double)(sgn * block_max(m, redf)) * sc;
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const bool ok = lane + 256 * k < sp.nb4;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[4 * k + j] = ok ? exp_split((double)v[4 * k + j] * sc - ms) : 0.f;
                sum += (double)v[4 * k + j];
            }
        }
        if (ei >= 0) {
            e = exp_split((double)e * sc - ms);
            sum += (double)e;
        }
        const double inv = 1.0 / block_sum(sum, redd);
        float4* yb = reinterpret_cast<float4*>(y + sp.h);
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const int q = lane + 256 * k;
            if (q < sp.nb4)
                store_stream(yb + q, make_float4((float)((double)v[4 * k] * inv), (float)((double)v[4 * k + 1] * inv),
                                                 (float)((double)v[4 * k + 2] * inv), (float)((double)v[4 * k + 3] * inv)));
        }
        if (ei >= 0) store_stream(y + ei, (float)((double)e * inv));
    }
}

// Any row length and alignment: one block per row and three passes over it (maximum, sum,
// output), the second and third re-reading the row from the cache. Each exp is recomputed in
// the third pass from the same operands, so it has the bits the sum added.
__global__ __launch_bounds__(256) void softmax_big_kernel(SoftmaxArgs a) {
    __shared__ float redf[4];
    __shared__ double redd[4];
    const long long rows = a.src.ne[1] * a.src.ne[2] * a.src.ne[3];
    const long long n = a.src.ne[0];
    const double sc = (double)a.scale;
    const float sgn = a.scale < 0.f ? -1.f : 1.f;
    for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* x = reinterpret_cast<const float*>(row_ptr(a.src, r));
        float* y = reinterpret_cast<float*>(row_ptr(a.dst, r));
        float m = -INFINITY;
        for (long long i = threadIdx.x; i < n; i += 256) m = fmaxf(m, sgn * x[i]);
        const double ms = (double)(sgn * block_max(m, redf)) * sc;
        double sum = 0.0;
        for (long long i = threadIdx.x; i < n; i += 256) sum += (double)exp_split((double)x[i] * sc - ms);
        const double inv = 1.0 / block_sum(sum, redd);
        __syncthreads();                         // every thread has read the row before y overwrites it
        for (long long i = threadIdx.x; i < n; i += 256) y[i] = (float)((double)exp_split((double)x[i] * sc - ms) * inv);
    }
}

// --------------------------------------------------------------------- elementwise
enum EwOp { EW_GELU = 0, EW_GLU = 1, EW_ADD = 2, EW_MUL = 3, EW_MUL_ADD = 4, EW_ADD_GELU = 5, EW_GLU_MUL_ADD = 6 };

__device__ __forceinline__ float glu_value(float a, float g) { return a / (1.0f + expf(-g)); }

// GLU: x * sigmoid(y) with x and y two halves of one source. MUL_ADD: x + fl(y * z), rounded
// after each operation like ggml_add(x, ggml_mul(h, s)). ADD_GELU: gelu(fl(x + y)), a bias
// add followed by GELU. GLU_MUL_ADD: x + fl(glu(y, z) * w), the GLU + LayerScale + residual
// of a DConv branch, bit-identical to GLU followed by MUL_ADD.
template <int OP>
__device__ __forceinline__ float ew_apply(float x, float y, float z, float w) {
#pragma clang fp contract(off)
    if constexpr (OP == EW_GELU) return gelu_erf(x);
    if constexpr (OP == EW_GLU) return glu_value(x, y);
    if constexpr (OP == EW_ADD) return x + y;
    if constexpr (OP == EW_MUL) return x * y;
    if constexpr (OP == EW_MUL_ADD) {
        const float p = y * z;
        return x + p;
    }
    if constexpr (OP == EW_ADD_GELU) return gelu_erf(x + y);
    if constexpr (OP == EW_GLU_MUL_ADD) {
        const float p = glu_value(y, z) * w;
        return x + p;
    }
    return 0.f;
}

template <int OP> constexpr bool has_b() { return OP != EW_GELU; }
template <int OP> constexpr bool has_c() { return OP == EW_MUL_ADD || OP == EW_GLU_MUL_ADD; }
template <int OP> constexpr bool has_d() { return OP == EW_GLU_MUL_ADD; }

// General path. a: same shape as dst (any row strides). b, c, d repeat into dst. Work unit =
// (row, 1024-element chunk of the row).
struct EwArgs {
    T4 a, b, c, d, dst;
};

__device__ __forceinline__ const float* bcast_row(const T4& t, long long i1, long long i2, long long i3) {
    return reinterpret_cast<const float*>(t.data + (i1 % t.ne[1]) * t.nb[1] + (i2 % t.ne[2]) * t.nb[2] +
                                          (i3 % t.ne[3]) * t.nb[3]);
}

__device__ __forceinline__ float bcast_at(const float* row, long long ne0, long long n0, long long i) {
    return ne0 == n0 ? row[i] : ne0 == 1 ? row[0] : row[i % ne0];
}

template <int OP>
__global__ __launch_bounds__(256) void ew_rows_kernel(EwArgs a) {
    const long long rows = a.dst.ne[1] * a.dst.ne[2] * a.dst.ne[3];
    const long long n0 = a.dst.ne[0];
    const long long cpr = (n0 + 1023) / 1024;
    for (long long u = blockIdx.x; u < rows * cpr; u += gridDim.x) {
        const long long r = u / cpr;
        const long long base = (u - r * cpr) * 1024;
        const long long i1 = r % a.dst.ne[1], q = r / a.dst.ne[1];
        const long long i2 = q % a.dst.ne[2], i3 = q / a.dst.ne[2];
        const float* xa = reinterpret_cast<const float*>(a.a.data + i1 * a.a.nb[1] + i2 * a.a.nb[2] + i3 * a.a.nb[3]);
        const float* xb = has_b<OP>() ? bcast_row(a.b, i1, i2, i3) : nullptr;
        const float* xc = has_c<OP>() ? bcast_row(a.c, i1, i2, i3) : nullptr;
        const float* xd = has_d<OP>() ? bcast_row(a.d, i1, i2, i3) : nullptr;
        float* y = reinterpret_cast<float*>(a.dst.data + i1 * a.dst.nb[1] + i2 * a.dst.nb[2] + i3 * a.dst.nb[3]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const long long i = base + k * 256 + threadIdx.x;
            if (i < n0) {
                const float vb = has_b<OP>() ? bcast_at(xb, a.b.ne[0], n0, i) : 0.f;
                const float vc = has_c<OP>() ? bcast_at(xc, a.c.ne[0], n0, i) : 0.f;
                const float vd = has_d<OP>() ? bcast_at(xd, a.d.ne[0], n0, i) : 0.f;
                y[i] = ew_apply<OP>(xa[i], vb, vc, vd);
            }
        }
    }
}

// Flat path: a and dst contiguous and 16-byte aligned, fewer than 2^32 elements. An operand
// either has dst's shape (read as float4) or is a contiguous block that repeats: flat element
// i of dst reads p[(i / div) % mod], which covers row vectors (bias, gamma: div 1), channel
// vectors (LayerScale: div = the plane size) and any full-extent block of middle dimensions.
enum FlatMode { FLAT_NONE = 0, FLAT_SAME = 1, FLAT_ROW4 = 2, FLAT_SPLAT = 3, FLAT_GENERAL = 4 };

struct Flat {
    const float* p;
    unsigned div, mod;
    double rdiv, rmod;   // 1/div, 1/mod
    int mode;        // SAME: float4 at i; ROW4: float4 at i % mod (div 1, mod % 4 == 0);
                     // SPLAT: one value for all four (div % 4 == 0); GENERAL: per element
};

// i / d for i < 2^32 from the double reciprocal (error < 1) and one correction step: a few
// instructions instead of an integer division.
__device__ __forceinline__ unsigned fast_div(unsigned i, unsigned d, double rd) {
    unsigned q = (unsigned)((double)i * rd);
    const long long r = (long long)i - (long long)q * d;
    if (r < 0) q--;
    else if (r >= (long long)d) q++;
    return q;
}

__device__ __forceinline__ unsigned fast_mod(unsigned i, unsigned d, double rd) { return i - fast_div(i, d, rd) * d; }

__device__ __forceinline__ void flat_load(const Flat& f, unsigned i, float (&v)[4]) {
    if (f.mode == FLAT_SAME || f.mode == FLAT_ROW4) {
        const float4 q =
            *reinterpret_cast<const float4*>(f.p + (f.mode == FLAT_SAME ? i : fast_mod(i, f.mod, f.rmod)));
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    } else if (f.mode == FLAT_SPLAT) {
        v[0] = v[1] = v[2] = v[3] = f.p[fast_mod(fast_div(i, f.div, f.rdiv), f.mod, f.rmod)];
    } else if (f.mode == FLAT_GENERAL) {
        unsigned q = fast_div(i, f.div, f.rdiv);
        unsigned r = i - q * f.div;
        q = fast_mod(q, f.mod, f.rmod);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = f.p[q];
            if (++r == f.div) {
                r = 0;
                if (++q == f.mod) q = 0;
            }
        }
    } else {
        v[0] = v[1] = v[2] = v[3] = 0.f;
    }
}

__device__ __forceinline__ float flat_at(const Flat& f, unsigned i) {
    if (f.mode == FLAT_NONE) return 0.f;
    return f.mode == FLAT_SAME ? f.p[i] : f.p[fast_mod(fast_div(i, f.div, f.rdiv), f.mod, f.rmod)];
}

template <int OP>
__global__ __launch_bounds__(256) void ew_flat_kernel(const float* __restrict__ xa, Flat b, Flat c, Flat d,
                                                      float* __restrict__ y, unsigned n) {
    const unsigned n4 = n / 4;
    const unsigned stride = gridDim.x * 256;
    for (unsigned k = blockIdx.x * 256 + threadIdx.x; k < n4; k += stride) {
        const unsigned i = 4 * k;
        const float4 p = *reinterpret_cast<const float4*>(xa + i);
        float vb[4] = {0.f, 0.f, 0.f, 0.f}, vc[4] = {0.f, 0.f, 0.f, 0.f}, vd[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (has_b<OP>()) flat_load(b, i, vb);
        if constexpr (has_c<OP>()) flat_load(c, i, vc);
        if constexpr (has_d<OP>()) flat_load(d, i, vd);
        store_stream(reinterpret_cast<float4*>(y + i),
                     make_float4(ew_apply<OP>(p.x, vb[0], vc[0], vd[0]), ew_apply<OP>(p.y, vb[1], vc[1], vd[1]),
                                 ew_apply<OP>(p.z, vb[2], vc[2], vd[2]), ew_apply<OP>(p.w, vb[3], vc[3], vd[3])));
    }
    for (unsigned i = 4 * n4 + blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        store_stream(y + i, ew_apply<OP>(xa[i], has_b<OP>() ? flat_at(b, i) : 0.f, has_c<OP>() ? flat_at(c, i) : 0.f,
                                         has_d<OP>() ? flat_at(d, i) : 0.f));
}

// ----------------------------------------------------------------------- GROUP_NORM
// Groups: for each i3, channels (ne2) [g*cpg, min((g+1)*cpg, ne2)) with cpg = ceil(ne2 / G),
// normalised together over ne0 x ne1 x channels (ggml_group_norm). Contiguous tensors only,
// so a group is one contiguous span of floats (fewer than 2^32 of them).
//
// Statistics: the double sums of d and d^2, d = x - K with K the group's first element (the
// shift removes a common offset, so S2 - S1^2/N loses only ~1e-16 ((mean - K)/sigma)^2
// relative). They are added in ONE order that every path shares, so that every path gives
// the same statistics bit for bit, deterministically and without atomics:
//   - a group is cut into chunks of kGnThreads * 4 * VEC floats, VEC in {1, 2, 4} chosen from
//     the group's span alone (gn_vec); thread t of a chunk holds float4 k at
//     chunk start + (k * kGnThreads + t) * 4 and adds its values in (k, j) order;
//   - a chunk's partial sums are the threads' sums added by block_sum2_n;
//   - the totals: thread t adds the partials of chunks t, t + kGnThreads, ... from +0.0, then
//     block_sum2_n over the threads (the collector of grid_totals, gn_fold).
// The output is t = x * a + d with a = rstd * w, d = b - mean * a in double, then rounded, or
// GELU of the double t (its negative tail is ill-conditioned: d ln gelu / d ln t ~ 1 + t^2).
//
// Paths, by shape:
//   single pass (gn_fused_kernel) when the groups fit on the device at once, VEC < 4 and y
//     does not overlap x: x is read once, the blocks exchange their partial sums (grid_sync.hpp);
//   two passes otherwise: gn_partial_kernel writes each chunk's partial sums (and K), then
//     gn_apply_kernel folds its group's partials itself (or reads gn_fold_kernel's totals when
//     a group has more than kGnFoldDirect chunks) and writes its chunk.
// Affine per channel with planes of at least 256 floats (the HTDemucs shapes) takes a
// per-wave path: a wave's 256 consecutive elements lie in at most two channels, whose
// parameters it loads once (wave-uniform) before the statistics are known and turns into
// (a, d) once after; every element then costs one conversion and one fma before its GELU.
//
// Workspace: the single pass's area (kGridSyncBytes) | shift [groups] | totals [groups][2] |
// chunk partials [groups][chunks][2].
constexpr int kGnThreads = kGridThreads;
constexpr int kGnFoldDirect = 1024;
template <int VEC> constexpr unsigned gn_chunk() { return kGnThreads * 4u * VEC; }
// The smallest width whose chunks cover the group in at most kGridMaxBlocks chunks (the single
// pass's limit), else 4.
inline int gn_vec(long long span) {
    if (span <= (long long)kGridMaxBlocks * gn_chunk<1>()) return 1;
    if (span <= (long long)kGridMaxBlocks * gn_chunk<2>()) return 2;
    return 4;
}

// CHANNEL: p[c]; NE0: p[i0]; GENERAL: broadcast over all four dimensions; CHANNEL_WAVE:
// p[c] taken once per wave (per channel affine, planes of >= 256 floats).
enum AffineKind { AFF_NONE = 0, AFF_CHANNEL = 1, AFF_NE0 = 2, AFF_GENERAL = 3, AFF_CHANNEL_WAVE = 4 };

struct Affine {
    const float* p;
    long long ne[4];                     // broadcast extents (elements)
    long long nb[4];                     // strides in floats
    int kind;
};

struct GroupNormArgs {
    const float* x;
    float* y;
    Affine w, b;
    double* shift;           // [groups_total] (two passes)
    double* tot;             // [groups_total][2] (two passes, separate fold)
    double* part;            // [groups_total][nch][2] (two passes)
    unsigned ne0, ne1;       // dims of x (ne3 is folded into the group index)
    long long ne2;
    unsigned plane;          // ne0 * ne1
    double rplane, rne0;     // 1/plane, 1/ne0
    FastDiv plane_div;       // division by plane on the scalar unit
    long long cpg;           // channels per group
    int groups;              // groups per ne3 slice
    int nch;                 // chunks per group (of the largest group)
    float eps;
    int vec;                 // every group span is 16-byte aligned and a multiple of 4 floats
};

__device__ __forceinline__ void group_span(const GroupNormArgs& a, int gt, long long& begin, unsigned& count,
                                           long long& c0, long long& i3) {
    i3 = gt / a.groups;
    const long long g = gt % a.groups;
    c0 = g * a.cpg;
    const long long c1 = min(c0 + a.cpg, a.ne2);
    begin = (i3 * a.ne2 + c0) * (long long)a.plane;
    count = (unsigned)((c1 - c0) * a.plane);
}

// This thread's values of chunk [lo, hi) of base. FULL (a whole chunk of an aligned span):
// unconditional float4 loads. Otherwise clamped scalar loads (always-valid addresses, so they
// issue together) and a mask.
template <int VEC, bool FULL>
__device__ __forceinline__ void gn_load(const float* base, unsigned lo, unsigned hi, float (&v)[4 * VEC],
                                        bool (&ok)[4 * VEC]) {
#pragma unroll
    for (int k = 0; k < VEC; k++) {
        const unsigned p = lo + (k * kGnThreads + threadIdx.x) * 4;
        if constexpr (FULL) {
            const float4 q = *reinterpret_cast<const float4*>(base + p);
            v[4 * k] = q.x;
            v[4 * k + 1] = q.y;
            v[4 * k + 2] = q.z;
            v[4 * k + 3] = q.w;
#pragma unroll
            for (int j = 0; j < 4; j++) ok[4 * k + j] = true;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const unsigned e = p + j;
                const float t = base[min(e, hi - 1)];
                ok[4 * k + j] = e < hi;
                v[4 * k + j] = ok[4 * k + j] ? t : 0.f;
            }
        }
    }
}

// The thread's sums of d = v - shift over its valid values, in (k, j) order.
template <int N>
__device__ __forceinline__ void gn_thread_sums(const float (&v)[N], const bool (&ok)[N], double shift, double& s1,
                                               double& s2) {
    s1 = 0.0;
    s2 = 0.0;
#pragma unroll
    for (int k = 0; k < N; k++) {
        const double d = ok[k] ? (double)v[k] - shift : 0.0;
        s1 = s1 + d;
        s2 = fma(d, d, s2);
    }
}

// Partial sums of chunk m of a group (count floats at xg), in every thread.
template <int VEC>
__device__ __forceinline__ void gn_chunk_sums(const float* xg, unsigned m, unsigned count, double shift, double* red,
                                              double& s1, double& s2) {
    const unsigned lo = m * gn_chunk<VEC>(), hi = min(lo + gn_chunk<VEC>(), count);
    float v[4 * VEC];
    bool ok[4 * VEC];
    gn_load<VEC, false>(xg, lo, hi, v, ok);
    gn_thread_sums(v, ok, shift, s1, s2);
    block_sum2_n<kGnThreads>(s1, s2, red);
}

// A group's totals from x alone, in the collector's order (a single-pass block whose wait
// gave up): tot[0..1] (shared), then a barrier.
template <int VEC>
__device__ __forceinline__ void gn_recompute(const float* xg, unsigned count, int nblk, double shift, double* red, double* tot) {
    double p1 = 0.0, p2 = 0.0;
    for (int m = 0; m < nblk; m++) {
        double q1, q2;
        gn_chunk_sums<VEC>(xg, (unsigned)m, count, shift, red, q1, q2);
        if ((int)threadIdx.x == m % kGnThreads) {
            p1 += q1;
            p2 += q2;
        }
    }
    block_sum2_n<kGnThreads>(p1, p2, red);
    if (threadIdx.x == 0) {
        tot[0] = p1;
        tot[1] = p2;
    }
    __syncthreads();
}

// A group's totals from its nblk chunk partials (two passes), in the collector's order.
__device__ __forceinline__ void gn_fold(const double* part, int nblk, double* red, double& t1, double& t2) {
    double p1 = 0.0, p2 = 0.0;
    for (int m = threadIdx.x; m < nblk; m += kGnThreads) {
        p1 += part[2 * m];
        p2 += part[2 * m + 1];
    }
    block_sum2_n<kGnThreads>(p1, p2, red);
    t1 = p1;
    t2 = p2;
}

// mean and 1/sqrt(var + eps) from the group's totals. Every path calls this one function on the
// same totals, so every path gets the same bits. 1/N and the reciprocal square root come from
// the hardware's double approximations refined by Newton steps (each doubles the correct bits
// of the ~2^-22 start, so two reach double precision), not from IEEE division and square root:
// about 20 instructions instead of 60, on the path between a block's release and its stores.
__device__ __forceinline__ double rcp_f64_nr(double d) {
    double r = __builtin_amdgcn_rcp(d);
    r = fma(r, fma(-d, r, 1.0), r);
    return fma(r, fma(-d, r, 1.0), r);
}
__device__ __forceinline__ void gn_moments(double t1, double t2, unsigned count, double shift, float eps, double& mean,
                                           double& rstd) {
    const double rn = rcp_f64_nr((double)count), dm = t1 * rn;
    mean = shift + dm;
    const double v = fmax(t2 * rn - dm * dm, 0.0) + (double)eps;
    double y = __builtin_amdgcn_rsq(v);
    if (v > 0.0 && v < 1e300) {                       // y = y (3 - v y^2) / 2, twice
        y = y * fma(-0.5 * v, y * y, 1.5);
        y = y * fma(-0.5 * v, y * y, 1.5);
    }
    rstd = y;
}

// One affine operand at element (channel c, i0, i1, i3) under the per-element kinds.
template <int AK>
__device__ __forceinline__ float affine_at(const Affine& f, long long c, unsigned i0, unsigned i1, long long i3) {
    if constexpr (AK == AFF_CHANNEL) return f.p[c];
    if constexpr (AK == AFF_NE0) return f.p[i0];
    return f.p[(i0 % f.ne[0]) * f.nb[0] + (i1 % f.ne[1]) * f.nb[1] + (c % f.ne[2]) * f.nb[2] + (i3 % f.ne[3]) * f.nb[3]];
}

// Affine parameters of this thread's elements.
//   CHANNEL_WAVE: per float4 k, the two channels the wave's run [pw, pw + 256) can touch:
//     w0/b0 of the channel of pw, w1/b1 of the next one (clamped), and bnd, the first element
//     of the next channel (all wave-uniform).
//   other kinds: one (w, b) per element.
// The identities of a missing weight (1) and bias (0).
__device__ const float kAffineUnit[2] = {1.f, 0.f};

template <int AK, int VEC>
struct GnParams {
    static constexpr bool kWave = AK == AFF_CHANNEL_WAVE;
    float w0[kWave ? VEC : 1], w1[kWave ? VEC : 1], b0[kWave ? VEC : 1], b1[kWave ? VEC : 1];
    unsigned bnd[kWave ? VEC : 1];
    float w[kWave ? 1 : 4 * VEC], b[kWave ? 1 : 4 * VEC];
};

template <int AK, int VEC>
__device__ __forceinline__ void gn_params(const GroupNormArgs& a, unsigned lo, long long c0, long long i3,
                                          const bool (&ok)[4 * VEC], GnParams<AK, VEC>& pr) {
    constexpr int NT = kGnThreads;
    if constexpr (AK == AFF_CHANNEL_WAVE) {
        const unsigned w64 = (unsigned)__builtin_amdgcn_readfirstlane((int)threadIdx.x) & ~63u;
        const long long cl = a.ne2 - 1;
#pragma unroll
        for (int k = 0; k < VEC; k++) {
            const unsigned pw = lo + (k * NT + w64) * 4;
            const unsigned ca = a.plane_div.div(pw);
            pr.bnd[k] = (ca + 1) * a.plane;
            const long long cA = min(c0 + (long long)ca, cl), cB = min(c0 + (long long)ca + 1, cl);
            // Unconditional loads (a missing operand reads its identity from kAffineUnit), so that
            // they issue with the chunk's loads instead of after a wait in a branch.
            // Global-space pointers: a generic (flat) load would also count on the LDS counter
            // and hold up the reductions' LDS waits.
            using gfloat = __attribute__((address_space(1))) const float;
            gfloat* wp = (gfloat*)(a.w.p ? a.w.p : kAffineUnit);
            gfloat* bp = (gfloat*)(a.b.p ? a.b.p : kAffineUnit + 1);
            const long long mw = a.w.p ? -1 : 0, mb = a.b.p ? -1 : 0;
            pr.w0[k] = wp[cA & mw];
            pr.w1[k] = wp[cB & mw];
            pr.b0[k] = bp[cA & mb];
            pr.b1[k] = bp[cB & mb];
        }
    } else {
#pragma unroll
        for (int k = 0; k < VEC; k++) {
            const unsigned p = lo + (k * NT + threadIdx.x) * 4;
            long long c = 0;
            unsigned i0 = 0, i1 = 0;
            if constexpr (AK == AFF_NE0) {
                i0 = fast_mod(p, a.ne0, a.rne0);
            } else {
                const unsigned cp = fast_div(p, a.plane, a.rplane), q = p - cp * a.plane;
                c = c0 + cp;
                i1 = fast_div(q, a.ne0, a.rne0);
                i0 = q - i1 * a.ne0;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const bool in = ok[4 * k + j];
                pr.w[4 * k + j] = a.w.p && in ? affine_at<AK>(a.w, c, i0, i1, i3) : 1.f;
                pr.b[4 * k + j] = a.b.p && in ? affine_at<AK>(a.b, c, i0, i1, i3) : 0.f;
                if (++i0 == a.ne0) {
                    i0 = 0;
                    if constexpr (AK != AFF_NE0) {
                        if (++i1 == a.ne1) {
                            i1 = 0;
                            ++c;
                        }
                    }
                }
            }
        }
    }
}

template <bool GELU>
__device__ __forceinline__ float gn_out(double t) {
    if constexpr (GELU) return gelu_erf_dt(t);
    else return (float)t;
}

// Writes this thread's outputs of chunk [lo, hi) at yg.
template <int AK, bool GELU, int VEC, bool FULL>
__device__ __forceinline__ void gn_write(float* yg, unsigned lo, unsigned hi, double mean, double rstd,
                                         const float (&v)[4 * VEC], const bool (&ok)[4 * VEC],
                                         const GnParams<AK, VEC>& pr) {
    constexpr int NT = kGnThreads;
#pragma unroll
    for (int k = 0; k < VEC; k++) {
        const unsigned p = lo + (k * NT + threadIdx.x) * 4;
        float o[4];
        if constexpr (AK == AFF_CHANNEL_WAVE) {
            const double a0 = rstd * (double)pr.w0[k], d0 = fma(-mean, a0, (double)pr.b0[k]);
            const unsigned pw = (unsigned)__builtin_amdgcn_readfirstlane((int)p);
            if (pw + 255 < pr.bnd[k]) {                        // the wave's run is in one channel
#pragma unroll
                for (int j = 0; j < 4; j++) o[j] = gn_out<GELU>(fma((double)v[4 * k + j], a0, d0));
            } else {
                const double a1 = rstd * (double)pr.w1[k], d1 = fma(-mean, a1, (double)pr.b1[k]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const bool nx = p + j >= pr.bnd[k];
                    o[j] = gn_out<GELU>(fma((double)v[4 * k + j], nx ? a1 : a0, nx ? d1 : d0));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const double aj = rstd * (double)pr.w[4 * k + j];
                o[j] = gn_out<GELU>(fma((double)v[4 * k + j], aj, fma(-mean, aj, (double)pr.b[4 * k + j])));
            }
        }
        if constexpr (FULL) {
            store_stream(reinterpret_cast<float4*>(yg + p), make_float4(o[0], o[1], o[2], o[3]));
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (ok[4 * k + j]) store_stream(yg + p + j, o[j]);
        }
        // One float4 at a time: interleaving the GELUs of several would need more than the
        // 128 VGPRs that two blocks per CU leave.
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Single pass: a block keeps its chunk of x and its affine parameters in registers, sums d
// and d^2 and gets the group's totals from the other blocks through grid_totals, then writes
// y from the registers: x is read from HBM once, in one launch.
template <int AK, bool GELU, int VEC, bool FULL>
__device__ __forceinline__ void gn_fused_body(const GroupNormArgs& a, const GridSync& f, int gt, long long begin,
                                              unsigned count, long long c0, long long i3, unsigned lo, double* red,
                                              double* tot) {
    const unsigned hi = min(lo + gn_chunk<VEC>(), count);
    const int nblk = (int)((count + gn_chunk<VEC>() - 1) / gn_chunk<VEC>());
    const float* xg = a.x + begin;
    float v[4 * VEC];
    bool ok[4 * VEC];
    gn_load<VEC, FULL>(xg, lo, hi, v, ok);
    const double shift = (double)xg[0];
    GnParams<AK, VEC> pr;
    gn_params<AK, VEC>(a, lo, c0, i3, ok, pr);
    double s1, s2;
    gn_thread_sums(v, ok, shift, s1, s2);
    block_sum2_n<kGnThreads>(s1, s2, red);
    if (grid_totals<kGnThreads>(f, gt, nblk, s1, s2, red, tot,
                                [&](double* t) { gn_recompute<VEC>(xg, count, nblk, shift, red, t); })) {
        gn_load<VEC, FULL>(xg, lo, hi, v, ok);                 // x is unchanged (y does not overlap it)
        gn_params<AK, VEC>(a, lo, c0, i3, ok, pr);
    }
    double mean, rstd;
    gn_moments(tot[0], tot[1], count, shift, a.eps, mean, rstd);
    gn_write<AK, GELU, VEC, FULL>(a.y + begin, lo, hi, mean, rstd, v, ok, pr);
}

// Two blocks per CU must fit (the C = 96 and 192 op-set shapes have 504 blocks for 256 CUs):
// at least 4 waves per SIMD, i.e. at most 128 VGPRs.
template <int AK, bool GELU, int VEC>
__global__ __launch_bounds__(kGnThreads) __attribute__((amdgpu_waves_per_eu(4))) void gn_fused_kernel(GroupNormArgs a,
                                                                                                     GridSync f) {
    __shared__ double red[2 * kGnThreads / kWave];
    __shared__ double tot[2];
    const int gt = (int)blockIdx.y;
    long long begin, c0, i3;
    unsigned count;
    group_span(a, gt, begin, count, c0, i3);
    const unsigned lo = blockIdx.x * gn_chunk<VEC>();
    if (lo >= count) return;                                   // past a short group: not one of its blocks
    if (a.vec && lo + gn_chunk<VEC>() <= count)
        gn_fused_body<AK, GELU, VEC, true>(a, f, gt, begin, count, c0, i3, lo, red, tot);
    else
        gn_fused_body<AK, GELU, VEC, false>(a, f, gt, begin, count, c0, i3, lo, red, tot);
}

// Two passes, pass 1: chunk m's partial sums to part[gt][m]; chunk 0 also stores K (x may be y,
// so pass 2 must not read it back from x).
template <int VEC, bool FULL>
__device__ __forceinline__ void gn_partial_body(const GroupNormArgs& a, int gt, const float* xg, unsigned count,
                                                unsigned lo, double* red) {
    const unsigned hi = min(lo + gn_chunk<VEC>(), count);
    float v[4 * VEC];
    bool ok[4 * VEC];
    gn_load<VEC, FULL>(xg, lo, hi, v, ok);
    const double shift = (double)xg[0];
    double s1, s2;
    gn_thread_sums(v, ok, shift, s1, s2);
    block_sum2_n<kGnThreads>(s1, s2, red);
    if (threadIdx.x == 0) {
        double* p = a.part + ((size_t)gt * a.nch + blockIdx.x) * 2;
        p[0] = s1;
        p[1] = s2;
        if (blockIdx.x == 0) a.shift[gt] = shift;
    }
}

template <int VEC>
__global__ __launch_bounds__(kGnThreads) void gn_partial_kernel(GroupNormArgs a) {
    __shared__ double red[2 * kGnThreads / kWave];
    const int gt = (int)blockIdx.y;
    long long begin, c0, i3;
    unsigned count;
    group_span(a, gt, begin, count, c0, i3);
    const unsigned lo = blockIdx.x * gn_chunk<VEC>();
    if (lo >= count) return;
    if (a.vec && lo + gn_chunk<VEC>() <= count) gn_partial_body<VEC, true>(a, gt, a.x + begin, count, lo, red);
    else gn_partial_body<VEC, false>(a, gt, a.x + begin, count, lo, red);
}

// Two passes, for groups of more than kGnFoldDirect chunks: one block per group folds its
// partials into tot[gt].
__global__ __launch_bounds__(kGnThreads) void gn_fold_kernel(GroupNormArgs a, int vec) {
    __shared__ double red[2 * kGnThreads / kWave];
    const int gt = (int)blockIdx.x;
    long long begin, c0, i3;
    unsigned count;
    group_span(a, gt, begin, count, c0, i3);
    const unsigned ch = kGnThreads * 4u * (unsigned)vec;
    double t1, t2;
    gn_fold(a.part + (size_t)gt * a.nch * 2, (int)((count + ch - 1) / ch), red, t1, t2);
    if (threadIdx.x == 0) {
        a.tot[2 * gt] = t1;
        a.tot[2 * gt + 1] = t2;
    }
}

// Two passes, pass 2: loads its chunk and parameters first, then the group's totals (folded
// here from the partials, or gn_fold_kernel's), then writes its chunk.
template <int AK, bool GELU, int VEC, bool FULL>
__device__ __forceinline__ void gn_apply_body(const GroupNormArgs& a, int gt, long long begin, unsigned count,
                                              long long c0, long long i3, unsigned lo, double* red) {
    const unsigned hi = min(lo + gn_chunk<VEC>(), count);
    const int nblk = (int)((count + gn_chunk<VEC>() - 1) / gn_chunk<VEC>());
    float v[4 * VEC];
    bool ok[4 * VEC];
    gn_load<VEC, FULL>(a.x + begin, lo, hi, v, ok);
    GnParams<AK, VEC> pr;
    gn_params<AK, VEC>(a, lo, c0, i3, ok, pr);
    double t1, t2;
    if (nblk <= kGnFoldDirect) {
        gn_fold(a.part + (size_t)gt * a.nch * 2, nblk, red, t1, t2);
    } else {
        t1 = a.tot[2 * gt];
        t2 = a.tot[2 * gt + 1];
    }
    double mean, rstd;
    gn_moments(t1, t2, count, a.shift[gt], a.eps, mean, rstd);
    gn_write<AK, GELU, VEC, FULL>(a.y + begin, lo, hi, mean, rstd, v, ok, pr);
}

template <int AK, bool GELU, int VEC>
__global__ __launch_bounds__(kGnThreads) void gn_apply_kernel(GroupNormArgs a) {
    __shared__ double red[2 * kGnThreads / kWave];
    const int gt = (int)blockIdx.y;
    long long begin, c0, i3;
    unsigned count;
    group_span(a, gt, begin, count, c0, i3);
    const unsigned lo = blockIdx.x * gn_chunk<VEC>();
    if (lo >= count) return;
    if (a.vec && lo + gn_chunk<VEC>() <= count) gn_apply_body<AK, GELU, VEC, true>(a, gt, begin, count, c0, i3, lo, red);
    else gn_apply_body<AK, GELU, VEC, false>(a, gt, begin, count, c0, i3, lo, red);
}

// ----------------------------------------------------------------------------- ROPE
// ggml_rope_ext without YaRN (ext_factor 0): theta_i = freq_scale * pos * base^(-2i/n_dims),
// cos and sin scaled by attn_factor. Mode 0 rotates adjacent pairs (2i, 2i+1), mode 2 (NEOX)
// the pairs (i, i + n_dims/2); elements past n_dims are copied. Each block takes one position
// (ne2 index) and kRopeRows of its (ne1, ne3) rows; it evaluates cos/sin in double once per
// pair into LDS and rotates in double, rounding once. A thread owns a whole pair (or one
// copied element), so dst may alias src.
constexpr int kRopeRows = 128;

struct RopeArgs {
    T4 src, dst;
    const int* pos;          // [ne2]
    int n_dims, mode;
    int vec2;                // mode 0 with 8-byte aligned rows: pairs move as float2
    double freq_base, freq_scale, attn_factor;
};

__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
    extern __shared__ double cs[];                       // [n_dims/2][2]
    const long long ne0 = a.src.ne[0], ne1 = a.src.ne[1], ne3 = a.src.ne[3];
    const int half = a.n_dims / 2;
    const int units = half + (int)(ne0 - a.n_dims);     // pairs, then copied elements
    const long long i2 = blockIdx.x;
    const double p = (double)a.pos[i2];
    for (int i = (int)threadIdx.x; i < half; i += 256) {
        const double theta = a.freq_scale * p * pow(a.freq_base, -2.0 * i / a.n_dims);
        double sn, cn;
        sincos(theta, &sn, &cn);
        cs[2 * i] = cn * a.attn_factor;
        cs[2 * i + 1] = sn * a.attn_factor;
    }
    __syncthreads();
    const long long rows = ne1 * ne3;
    const long long r0 = (long long)blockIdx.y * kRopeRows;
    const long long nr = min((long long)kRopeRows, rows - r0);
    for (long long e = threadIdx.x; e < nr * units; e += 256) {
        const long long r = r0 + e / units;
        const int u = (int)(e % units);
        const long long i1 = r % ne1, i3 = r / ne1;
        const float* x = reinterpret_cast<const float*>(a.src.data + i1 * a.src.nb[1] + i2 * a.src.nb[2] + i3 * a.src.nb[3]);
        float* y = reinterpret_cast<float*>(a.dst.data + i1 * a.dst.nb[1] + i2 * a.dst.nb[2] + i3 * a.dst.nb[3]);
        if (u >= half) {
            const int i = a.n_dims + (u - half);
            y[i] = x[i];
            continue;
        }
        const int j0 = a.mode == 0 ? 2 * u : u;
        const int j1 = a.mode == 0 ? 2 * u + 1 : u + half;
        const double c = cs[2 * u], s = cs[2 * u + 1];
        double x0, x1;
        if (a.vec2) {
            const float2 v = *reinterpret_cast<const float2*>(x + j0);
            x0 = v.x;
            x1 = v.y;
        } else {
            x0 = x[j0];
            x1 = x[j1];
        }
        const float o0 = (float)(x0 * c - x1 * s), o1 = (float)(x0 * s + x1 * c);
        if (a.vec2) {
            *reinterpret_cast<float2*>(y + j0) = make_float2(o0, o1);
        } else {
            y[j0] = o0;
            y[j1] = o1;
        }
    }
}

// Mode 0 with rows of a multiple of 4 floats, 16-byte aligned: each thread moves one float4,
// i.e. two adjacent pairs (or 4 copied floats past n_dims), with 32-bit index arithmetic.
__global__ __launch_bounds__(256) void rope_v4_kernel(RopeArgs a) {
    extern __shared__ double cs[];                       // [n_dims/2][2]
    const int half = a.n_dims / 2;
    const long long i2 = blockIdx.x;
    const double p = (double)a.pos[i2];
    for (int i = (int)threadIdx.x; i < half; i += 256) {
        const double theta = a.freq_scale * p * pow(a.freq_base, -2.0 * i / a.n_dims);
        double sn, cn;
        sincos(theta, &sn, &cn);
        cs[2 * i] = cn * a.attn_factor;
        cs[2 * i + 1] = sn * a.attn_factor;
    }
    __syncthreads();
    const int ne1 = (int)a.src.ne[1];
    const int u4 = (int)(a.src.ne[0] >> 2), d4 = a.n_dims >> 2;
    const int rows = ne1 * (int)a.src.ne[3];
    const int r0 = (int)blockIdx.y * kRopeRows;
    const int total = min(kRopeRows, rows - r0) * u4;
    const char* xs = a.src.data + i2 * a.src.nb[2];
    char* ys = a.dst.data + i2 * a.dst.nb[2];
    for (int e = (int)threadIdx.x; e < total; e += 256) {
        const int rr = e / u4, q = e - rr * u4;
        const int r = r0 + rr, i1 = r % ne1, i3 = r / ne1;
        const float4 v = reinterpret_cast<const float4*>(xs + i1 * a.src.nb[1] + i3 * a.src.nb[3])[q];
        float4 o = v;
        if (q < d4) {
            const double c0 = cs[4 * q], s0 = cs[4 * q + 1], c1 = cs[4 * q + 2], s1 = cs[4 * q + 3];
            o.x = (float)((double)v.x * c0 - (double)v.y * s0);
            o.y = (float)((double)v.x * s0 + (double)v.y * c0);
            o.z = (float)((double)v.z * c1 - (double)v.w * s1);
            o.w = (float)((double)v.z * s1 + (double)v.w * c1);
        }
        store_stream(reinterpret_cast<float4*>(ys + i1 * a.dst.nb[1] + i3 * a.dst.nb[3]) + q, o);
    }
}

// ------------------------------------------------------------------------ dispatch
// Calls f(LANES, VPL) with the smallest lanes-per-row that keeps at most 16 values per lane
// (32 for rows of 1025..2048).
template <class F>
void pick_row_shape(long long n, F&& f) {
    using std::integral_constant;
    if (n <= 128) f(integral_constant<int, 8>{}, integral_constant<int, 16>{});
    else if (n <= 256) f(integral_constant<int, 16>{}, integral_constant<int, 16>{});
    else if (n <= 512) f(integral_constant<int, 32>{}, integral_constant<int, 16>{});
    else if (n <= 1024) f(integral_constant<int, 64>{}, integral_constant<int, 16>{});
    else f(integral_constant<int, 64>{}, integral_constant<int, 32>{});
}

// Calls f(LANES, V4) for the vector-load row kernels, V4 = ceil(ceil(n/4) / LANES) float4 per
// lane from {1, 2, 3, 4, 6, 8}: 8 lanes up to 32 float4, 16 lanes up to 128 (rows of up to 512
// floats: more rows per wave share each row's fixed cost of reductions and square root), 64
// lanes beyond (V4 up to 8, rows of up to 2048 floats).
template <class F>
void pick_v4_shape(long long n, F&& f) {
    using std::integral_constant;
    const long long q = (n + 3) / 4;
    auto with_lanes = [&](auto lanes) {
        constexpr int L = decltype(lanes)::value;
        const long long v = (q + L - 1) / L;
        if (v <= 1) f(lanes, integral_constant<int, 1>{});
        else if (v == 2) f(lanes, integral_constant<int, 2>{});
        else if (v == 3) f(lanes, integral_constant<int, 3>{});
        else if (v == 4) f(lanes, integral_constant<int, 4>{});
        else if (v <= 6) f(lanes, integral_constant<int, 6>{});
        else f(lanes, integral_constant<int, 8>{});
    };
    if (q <= 32) with_lanes(integral_constant<int, 8>{});
    else if (q <= 128) with_lanes(integral_constant<int, 16>{});
    else with_lanes(integral_constant<int, 64>{});
}

// Source and destination rows start at the same offset modulo 16 bytes.
bool same_row_alignment(const T4& s, const T4& d) {
    if ((reinterpret_cast<uintptr_t>(s.data) & 15) != (reinterpret_cast<uintptr_t>(d.data) & 15)) return false;
    for (int i = 1; i < 4; i++)
        if (s.ne[i] > 1 && (s.nb[i] - d.nb[i]) % 16 != 0) return false;
    return true;
}

constexpr long long kMaxRowShapeN = 2048;

unsigned row_blocks(long long rows, int lanes) {
    const long long per = 256 / lanes;
    return (unsigned)std::min<long long>((rows + per - 1) / per, 1 << 18);
}

void row_norm(const stx_tensor* a, const stx_tensor* dst, const float* gamma, const float* beta, float eps, int rms,
              stx_stream stream) {
    check_tensor(a, "a");
    check_tensor(dst, "dst");
    check_same_shape(a, dst, rms ? "rms_norm" : "norm");
    RowNormArgs args{view(a), view(dst), gamma, beta, eps, rms, 0, 0, 0};
    args.rs_src = row_spacing(args.src);
    args.rs_dst = row_spacing(args.dst);
    args.vec_params = (!gamma || aligned16(gamma)) && (!beta || aligned16(beta)) ? 1 : 0;
    const long long rows = nrows(args.src), n = args.src.ne[0];
    if (rows == 0 || n == 0) return;
    STX_REQUIRE(n < (1LL << 31), "row too long");
    const hipStream_t s = as_stream(stream);
    if (n <= kMaxRowShapeN && same_row_alignment(args.src, args.dst)) {
        pick_v4_shape(n, [&](auto lanes, auto v4) {
            constexpr int L = decltype(lanes)::value, V = decltype(v4)::value;
            hipLaunchKernelGGL((row_norm_v4_kernel<L, V>), dim3(row_blocks(rows, L)), dim3(256), 0, s, args);
        });
        launch_check("row_norm_v4_kernel");
    } else if (n <= kMaxRowShapeN) {
        pick_row_shape(n, [&](auto lanes, auto vpl) {
            constexpr int L = decltype(lanes)::value, V = decltype(vpl)::value;
            hipLaunchKernelGGL((row_norm_kernel<L, V>), dim3(row_blocks(rows, L)), dim3(256), 0, s, args);
        });
        launch_check("row_norm_kernel");
    } else {
        hipLaunchKernelGGL(row_norm_big_kernel, dim3((unsigned)std::min<long long>(rows, 1 << 18)), dim3(256), 0, s,
                           args);
        launch_check("row_norm_big_kernel");
    }
}

// How operand t (NULL: none) is read on the flat path over dst; false if it cannot be.
bool flat_operand(const stx_tensor* t, const stx_tensor* dst, Flat& f) {
    f = Flat{};
    if (!t) return true;
    const T4 v = view(t);
    if (!contiguous(v)) return false;
    f.p = reinterpret_cast<const float*>(v.data);
    bool same = true;
    for (int i = 0; i < 4; i++) same = same && t->ne[i] == dst->ne[i];
    if (same) {
        f.mode = FLAT_SAME;
        return aligned16(v.data);
    }
    // Non-unit dimensions of t must be one full-extent run [d0, d1] of dst's dimensions.
    int d0 = -1, d1 = -1;
    for (int i = 0; i < 4; i++)
        if (t->ne[i] > 1) {
            if (d0 < 0) d0 = i;
            d1 = i;
        }
    unsigned long long div = 1, mod = 1;
    if (d0 >= 0) {
        for (int i = d0; i <= d1; i++)
            if (t->ne[i] != dst->ne[i]) return false;
        for (int i = 0; i < d0; i++) div *= (unsigned long long)dst->ne[i];
        for (int i = d0; i <= d1; i++) mod *= (unsigned long long)dst->ne[i];
    }
    f.div = (unsigned)div;
    f.mod = (unsigned)mod;
    f.rdiv = 1.0 / (double)div;
    f.rmod = 1.0 / (double)mod;
    if (div == 1 && mod % 4 == 0 && aligned16(v.data)) f.mode = FLAT_ROW4;
    else if (div % 4 == 0) f.mode = FLAT_SPLAT;
    else f.mode = FLAT_GENERAL;
    return true;
}

template <int OP>
void launch_elementwise(const EwArgs& args, const stx_tensor* b, const stx_tensor* c, const stx_tensor* d,
                        const stx_tensor* dst, hipStream_t s) {
    const long long n = nelem(args.dst);
    Flat fb, fc, fd;
    const bool flat = n < (1LL << 32) - 1024 && contiguous(args.a) && contiguous(args.dst) && aligned16(args.a.data) &&
                      aligned16(args.dst.data) && flat_operand(b, dst, fb) && flat_operand(c, dst, fc) &&
                      flat_operand(d, dst, fd);
    if (flat) {
        const unsigned blocks = (unsigned)std::min<long long>((n / 4 + 255) / 256 + 1, 1 << 16);
        hipLaunchKernelGGL((ew_flat_kernel<OP>), dim3(blocks), dim3(256), 0, s,
                           reinterpret_cast<const float*>(args.a.data), fb, fc, fd,
                           reinterpret_cast<float*>(args.dst.data), (unsigned)n);
        launch_check("ew_flat_kernel");
        return;
    }
    const long long units = nrows(args.dst) * ((args.dst.ne[0] + 1023) / 1024);
    hipLaunchKernelGGL((ew_rows_kernel<OP>), dim3((unsigned)std::min<long long>(units, 1 << 20)), dim3(256), 0, s, args);
    launch_check("ew_rows_kernel");
}

void elementwise(int op, const stx_tensor* a, const stx_tensor* b, const stx_tensor* c, const stx_tensor* d,
                 const stx_tensor* dst, stx_stream stream) {
    EwArgs args{};
    args.a = view(a);
    args.dst = view(dst);
    if (b) args.b = view(b);
    if (c) args.c = view(c);
    if (d) args.d = view(d);
    if (nelem(args.dst) == 0) return;
    const hipStream_t s = as_stream(stream);
    switch (op) {
        case EW_GELU: launch_elementwise<EW_GELU>(args, b, c, d, dst, s); break;
        case EW_GLU: launch_elementwise<EW_GLU>(args, b, c, d, dst, s); break;
        case EW_ADD: launch_elementwise<EW_ADD>(args, b, c, d, dst, s); break;
        case EW_MUL: launch_elementwise<EW_MUL>(args, b, c, d, dst, s); break;
        case EW_MUL_ADD: launch_elementwise<EW_MUL_ADD>(args, b, c, d, dst, s); break;
        case EW_ADD_GELU: launch_elementwise<EW_ADD_GELU>(args, b, c, d, dst, s); break;
        default: launch_elementwise<EW_GLU_MUL_ADD>(args, b, c, d, dst, s); break;
    }
}

// Classifies an affine operand (weight or bias) that repeats into x.
Affine make_affine(const stx_tensor* t, const stx_tensor* x, const char* what) {
    Affine f{};
    if (!t) return f;
    check_tensor(t, what);
    check_repeat(t, x, what);
    f.p = static_cast<const float*>(t->data);
    for (int i = 0; i < 4; i++) {
        f.ne[i] = t->ne[i];
        f.nb[i] = t->nb[i] / 4;
    }
    const bool one1 = t->ne[1] == 1, one3 = t->ne[3] == 1;
    if (t->ne[0] == 1 && one1 && t->ne[2] == x->ne[2] && one3 && (t->ne[2] == 1 || t->nb[2] == 4))
        f.kind = AFF_CHANNEL;
    else if (t->ne[0] == x->ne[0] && one1 && t->ne[2] == 1 && one3)
        f.kind = AFF_NE0;
    else
        f.kind = AFF_GENERAL;
    return f;
}

struct GnPlan {
    long long cpg, groups, groups_total, span;
    int vec, nch;
    size_t shift_off, tot_off, part_off, bytes;          // workspace layout
};

// Every group-norm workspace starts with the single-pass kernel's area (kGridSyncBytes).
GnPlan gn_plan(const stx_tensor* a, int n_groups) {
    GnPlan p{};
    p.cpg = std::max<long long>(1, (a->ne[2] + n_groups - 1) / n_groups);
    p.groups = (a->ne[2] + p.cpg - 1) / p.cpg;
    p.groups_total = p.groups * a->ne[3];
    p.span = p.cpg * a->ne[0] * a->ne[1];
    p.vec = gn_vec(p.span);
    const long long ch = (long long)kGnThreads * 4 * p.vec;
    p.nch = (int)std::max<long long>(1, (p.span + ch - 1) / ch);
    const size_t g = (size_t)std::max<long long>(1, p.groups_total);
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    p.shift_off = kGridSyncBytes;
    p.tot_off = p.shift_off + up(sizeof(double) * g);
    p.part_off = p.tot_off + up(sizeof(double) * 2 * g);
    p.bytes = p.part_off + up(sizeof(double) * 2 * g * (size_t)p.nch);
    return p;
}

template <int AK, bool GELU, int VEC>
void launch_gn_vec(const GroupNormArgs& g, const GnPlan& p, const GridSync& sync, bool single, hipStream_t s) {
    const dim3 grid((unsigned)p.nch, (unsigned)p.groups_total);
    // VEC 4 (groups of more than kGridMaxBlocks * gn_chunk<2>() floats) takes the single pass
    // only with no or per-wave affine parameters: the per-element kinds would hold 16 weights and
    // 16 biases per thread, more than the 128 VGPRs of two blocks per CU leave without spilling.
    if constexpr (VEC < 4 || AK == AFF_NONE || AK == AFF_CHANNEL_WAVE) if (single) {
        const void* k = reinterpret_cast<const void*>(&gn_fused_kernel<AK, GELU, VEC>);
        if ((long long)p.nch * p.groups_total <= resident_blocks(k, s)) {
            hipLaunchKernelGGL((gn_fused_kernel<AK, GELU, VEC>), grid, dim3(kGnThreads), 0, s, g, sync);
            launch_check("gn_fused_kernel");
            return;
        }
    }
    hipLaunchKernelGGL(gn_partial_kernel<VEC>, grid, dim3(kGnThreads), 0, s, g);
    launch_check("gn_partial_kernel");
    if (p.nch > kGnFoldDirect) {
        hipLaunchKernelGGL(gn_fold_kernel, dim3((unsigned)p.groups_total), dim3(kGnThreads), 0, s, g, VEC);
        launch_check("gn_fold_kernel");
    }
    hipLaunchKernelGGL((gn_apply_kernel<AK, GELU, VEC>), grid, dim3(kGnThreads), 0, s, g);
    launch_check("gn_apply_kernel");
}

// Single pass when the groups fit (at most kGridMaxGroups of at most kGridMaxBlocks chunks,
// all resident together) and y does not overlap x; otherwise two passes. Both give the same
// bits.
template <int AK, bool GELU>
void launch_group_norm(const GroupNormArgs& g, const GnPlan& p, const GridSync& sync, bool single, hipStream_t s) {
    single = single && p.groups_total <= kGridMaxGroups && p.nch <= kGridMaxBlocks;
    if (p.vec == 1) launch_gn_vec<AK, GELU, 1>(g, p, sync, single, s);
    else if (p.vec == 2) launch_gn_vec<AK, GELU, 2>(g, p, sync, single, s);
    else launch_gn_vec<AK, GELU, 4>(g, p, sync, single, s);
}

// stx_group_norm on a workspace of ws_bytes at ws (checked by the caller).
void group_norm(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps, const stx_tensor* weight,
                const stx_tensor* bias, int gelu, void* ws, const GnPlan& p, hipStream_t s) {
    const T4 ta = view(a), td = view(dst);
    GroupNormArgs g{};
    g.x = reinterpret_cast<const float*>(ta.data);
    g.y = reinterpret_cast<float*>(td.data);
    g.w = make_affine(weight, a, "weight");
    g.b = make_affine(bias, a, "bias");
    char* w = static_cast<char*>(ws);
    const GridSync sync = grid_sync_at(w);
    g.shift = reinterpret_cast<double*>(w + p.shift_off);
    g.tot = reinterpret_cast<double*>(w + p.tot_off);
    g.part = reinterpret_cast<double*>(w + p.part_off);
    g.ne0 = (unsigned)ta.ne[0];
    g.ne1 = (unsigned)ta.ne[1];
    g.ne2 = ta.ne[2];
    g.plane = (unsigned)(ta.ne[0] * ta.ne[1]);
    g.rplane = 1.0 / (double)g.plane;
    g.rne0 = 1.0 / (double)g.ne0;
    g.plane_div = FastDiv(g.plane);
    g.cpg = p.cpg;
    g.groups = (int)p.groups;
    g.nch = p.nch;
    g.eps = eps;
    // Every group span starts at (i3 * ne2 + g * cpg) * plane floats.
    g.vec = aligned16(ta.data) && aligned16(td.data) && (g.cpg * (long long)g.plane) % 4 == 0 &&
                    (ta.ne[3] == 1 || (g.ne2 * (long long)g.plane) % 4 == 0)
                ? 1
                : 0;
    const size_t nbytes = (size_t)nelem(ta) * 4;
    const bool single = !overlaps(ta.data, nbytes, td.data, nbytes);
    auto fits = [&](int kind) {
        return (g.w.kind == AFF_NONE || g.w.kind == kind) && (g.b.kind == AFF_NONE || g.b.kind == kind);
    };
    int ak = fits(AFF_CHANNEL) ? AFF_CHANNEL : fits(AFF_NE0) ? AFF_NE0 : AFF_GENERAL;
    if (ak == AFF_CHANNEL && g.plane >= 256) ak = AFF_CHANNEL_WAVE;
    switch (ak * 2 + (gelu ? 1 : 0)) {
        case AFF_CHANNEL_WAVE * 2 + 1: launch_group_norm<AFF_CHANNEL_WAVE, true>(g, p, sync, single, s); break;
        case AFF_CHANNEL_WAVE * 2: launch_group_norm<AFF_CHANNEL_WAVE, false>(g, p, sync, single, s); break;
        case AFF_CHANNEL * 2 + 1: launch_group_norm<AFF_CHANNEL, true>(g, p, sync, single, s); break;
        case AFF_CHANNEL * 2: launch_group_norm<AFF_CHANNEL, false>(g, p, sync, single, s); break;
        case AFF_NE0 * 2 + 1: launch_group_norm<AFF_NE0, true>(g, p, sync, single, s); break;
        case AFF_NE0 * 2: launch_group_norm<AFF_NE0, false>(g, p, sync, single, s); break;
        case AFF_GENERAL * 2 + 1: launch_group_norm<AFF_GENERAL, true>(g, p, sync, single, s); break;
        default: launch_group_norm<AFF_GENERAL, false>(g, p, sync, single, s); break;
    }
}

// Checks shared by the group-norm entry points; the plan of a call that has work, else false.
bool group_norm_check(const stx_tensor* a, const stx_tensor* dst, int n_groups, const stx_tensor* weight,
                      const stx_tensor* bias, GnPlan& p) {
    check_tensor(a, "a");
    check_tensor(dst, "dst");
    check_same_shape(a, dst, "group_norm");
    STX_REQUIRE(n_groups >= 1, "group_norm: n_groups < 1");
    STX_REQUIRE(contiguous(view(a)) && contiguous(view(dst)), "group_norm: tensors must be contiguous");
    (void)make_affine(weight, a, "weight");
    (void)make_affine(bias, a, "bias");
    if (nelem(view(a)) == 0) return false;
    p = gn_plan(a, n_groups);
    STX_REQUIRE(p.groups_total < 65536, "group_norm: more than 65535 groups");
    STX_REQUIRE(p.span < (1LL << 32) - gn_chunk<4>(), "group_norm: groups of 2^32 floats or more are not supported");
    return true;
}

// Scratch of stx_group_norm_noalloc: a static device array, one per GPU, whose address
// hipGetSymbolAddress gives once per device (the array's name is not a device address in
// host code).
constexpr size_t kGnScratchBytes = STX_GROUP_NORM_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kGnScratchBytes];

void* scratch_address() {
    static std::mutex mu;
    static void* addr[64] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    STX_REQUIRE(dev >= 0 && dev < 64, "group_norm_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* ptr = nullptr;
        hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        STX_REQUIRE(ptr != nullptr, "group_norm_noalloc: no scratch address");
        addr[dev] = ptr;
    }
    return addr[dev];
}

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_norm(const stx_tensor* a, const stx_tensor* dst, float eps, stx_stream stream) {
    return guard([&] { row_norm(a, dst, nullptr, nullptr, eps, 0, stream); });
}

STX_API stx_status stx_norm_affine(const stx_tensor* a, const float* weight, const float* bias, const stx_tensor* dst,
                                   float eps, stx_stream stream) {
    return guard([&] { row_norm(a, dst, weight, bias, eps, 0, stream); });
}

STX_API stx_status stx_rms_norm(const stx_tensor* a, const stx_tensor* dst, float eps, stx_stream stream) {
    return guard([&] { row_norm(a, dst, nullptr, nullptr, eps, 1, stream); });
}

STX_API stx_status stx_rms_norm_mul(const stx_tensor* a, const float* gamma, const stx_tensor* dst, float eps,
                                    stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(gamma != nullptr, "rms_norm_mul: gamma is NULL");
        row_norm(a, dst, gamma, nullptr, eps, 1, stream);
    });
}

STX_API stx_status stx_soft_max_ext(const stx_tensor* a, const stx_tensor* mask, const stx_tensor* dst, float scale,
                                    float max_bias, stx_stream stream) {
    return guard([&] {
        if (mask != nullptr) fail(STX_STATUS_UNSUPPORTED, "soft_max_ext: a mask is not supported");
        if (max_bias != 0.0f) fail(STX_STATUS_UNSUPPORTED, "soft_max_ext: ALiBi (max_bias != 0) is not supported");
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "soft_max_ext");
        SoftmaxArgs args{view(a), view(dst), scale, 0, 0};
        args.rs_src = row_spacing(args.src);
        args.rs_dst = row_spacing(args.dst);
        const long long rows = nrows(args.src), n = args.src.ne[0];
        if (rows == 0 || n == 0) return;
        STX_REQUIRE(n < (1LL << 31), "soft_max_ext: row too long");
        const hipStream_t s = as_stream(stream);
        const unsigned row_grid = (unsigned)std::min<long long>(rows, 1 << 20);
        if (n > kMaxRowShapeN && n <= 4 * kMaxRowShapeN && same_row_alignment(args.src, args.dst)) {
            const long long v4 = ((n + 3) / 4 + 255) / 256;
            auto go = [&](auto k) {
                constexpr int V = decltype(k)::value;
                hipLaunchKernelGGL((softmax_block_kernel<V>), dim3(row_grid), dim3(256), 0, s, args);
            };
            using std::integral_constant;
            if (v4 <= 3) go(integral_constant<int, 3>{});
            else if (v4 == 4) go(integral_constant<int, 4>{});
            else if (v4 <= 6) go(integral_constant<int, 6>{});
            else go(integral_constant<int, 8>{});
            launch_check("softmax_block_kernel");
        } else if (n > kMaxRowShapeN) {
            hipLaunchKernelGGL(softmax_big_kernel, dim3(row_grid), dim3(256), 0, s, args);
            launch_check("softmax_big_kernel");
        } else if (same_row_alignment(args.src, args.dst)) {
            pick_v4_shape(n, [&](auto lanes, auto v4) {
                constexpr int L = decltype(lanes)::value, V = decltype(v4)::value;
                hipLaunchKernelGGL((softmax_v4_kernel<L, V>), dim3(row_blocks(rows, L)), dim3(256), 0, s, args);
            });
            launch_check("softmax_v4_kernel");
        } else {
            pick_row_shape(n, [&](auto lanes, auto vpl) {
                constexpr int L = decltype(lanes)::value, V = decltype(vpl)::value;
                hipLaunchKernelGGL((softmax_kernel<L, V>), dim3(row_blocks(rows, L)), dim3(256), 0, s, args);
            });
            launch_check("softmax_kernel");
        }
    });
}

STX_API stx_status stx_gelu_erf(const stx_tensor* a, const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "gelu_erf");
        elementwise(EW_GELU, a, nullptr, nullptr, nullptr, dst, stream);
    });
}

STX_API stx_status stx_add_gelu_erf(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst,
                                    stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(b, "b");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "add_gelu_erf");
        check_repeat(b, dst, "add_gelu_erf");
        elementwise(EW_ADD_GELU, a, b, nullptr, nullptr, dst, stream);
    });
}

STX_API stx_status stx_glu(const stx_tensor* a, const stx_tensor* dst, int dim, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        STX_REQUIRE(dim >= 0 && dim < 4, "glu: dim must be 0..3");
        STX_REQUIRE(a->ne[dim] % 2 == 0 && a->ne[dim] / 2 == dst->ne[dim], "glu: a->ne[dim] must be 2 * dst->ne[dim]");
        for (int i = 0; i < 4; i++)
            if (i != dim) STX_REQUIRE(a->ne[i] == dst->ne[i], "glu: shape mismatch in ne[%d]", i);
        // Two views of a: values (first half along dim) and gates (second half).
        stx_tensor va = *a, vg = *a;
        va.ne[dim] = vg.ne[dim] = a->ne[dim] / 2;
        vg.data = static_cast<char*>(a->data) + a->nb[dim] * (a->ne[dim] / 2);
        elementwise(EW_GLU, &va, &vg, nullptr, nullptr, dst, stream);
    });
}

STX_API stx_status stx_add(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(b, "b");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "add");
        check_repeat(b, dst, "add");
        elementwise(EW_ADD, a, b, nullptr, nullptr, dst, stream);
    });
}

STX_API stx_status stx_mul(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(b, "b");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "mul");
        check_repeat(b, dst, "mul");
        elementwise(EW_MUL, a, b, nullptr, nullptr, dst, stream);
    });
}

STX_API stx_status stx_mul_add(const stx_tensor* x, const stx_tensor* h, const stx_tensor* s, const stx_tensor* dst,
                               stx_stream stream) {
    return guard([&] {
        check_tensor(x, "x");
        check_tensor(h, "h");
        check_tensor(s, "s");
        check_tensor(dst, "dst");
        check_same_shape(x, dst, "mul_add");
        check_repeat(h, dst, "mul_add");
        check_repeat(s, dst, "mul_add");
        elementwise(EW_MUL_ADD, x, h, s, nullptr, dst, stream);
    });
}

STX_API stx_status stx_glu_mul_add(const stx_tensor* x, const stx_tensor* a, int dim, const stx_tensor* s,
                                   const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(x, "x");
        check_tensor(a, "a");
        check_tensor(s, "s");
        check_tensor(dst, "dst");
        check_same_shape(x, dst, "glu_mul_add");
        STX_REQUIRE(dim >= 0 && dim < 4, "glu_mul_add: dim must be 0..3");
        STX_REQUIRE(a->ne[dim] % 2 == 0 && a->ne[dim] / 2 == dst->ne[dim],
                    "glu_mul_add: a->ne[dim] must be 2 * dst->ne[dim]");
        for (int i = 0; i < 4; i++)
            if (i != dim) STX_REQUIRE(a->ne[i] == dst->ne[i], "glu_mul_add: shape mismatch in ne[%d]", i);
        check_repeat(s, dst, "glu_mul_add");
        stx_tensor va = *a, vg = *a;
        va.ne[dim] = vg.ne[dim] = a->ne[dim] / 2;
        vg.data = static_cast<char*>(a->data) + a->nb[dim] * (a->ne[dim] / 2);
        elementwise(EW_GLU_MUL_ADD, x, &va, &vg, s, dst, stream);
    });
}

STX_API size_t stx_group_norm_workspace_size(const stx_tensor* a, int n_groups) {
    if (!a || n_groups < 1) return 0;
    for (int i = 0; i < 4; i++)
        if (a->ne[i] < 0) return 0;
    return gn_plan(a, n_groups).bytes;
}

STX_API stx_status stx_group_norm(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps,
                                  const stx_tensor* weight, const stx_tensor* bias, int gelu, void* workspace,
                                  size_t workspace_bytes, stx_stream stream) {
    return guard([&] {
        GnPlan p;
        if (!group_norm_check(a, dst, n_groups, weight, bias, p)) return;
        STX_REQUIRE(workspace != nullptr && workspace_bytes >= p.bytes, "group_norm: workspace too small (%zu, need %zu)",
                    workspace_bytes, p.bytes);
        STX_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "group_norm: workspace must be 256-byte aligned");
        group_norm(a, dst, n_groups, eps, weight, bias, gelu, workspace, p, as_stream(stream));
    });
}

STX_API stx_status stx_group_norm_noalloc(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps,
                                          const stx_tensor* weight, const stx_tensor* bias, int gelu,
                                          stx_stream stream) {
    return guard([&] {
        GnPlan p;
        if (!group_norm_check(a, dst, n_groups, weight, bias, p)) return;
        STX_REQUIRE(p.bytes <= kGnScratchBytes,
                    "group_norm_noalloc: this shape needs %zu bytes of scratch, more than the %zu of the static "
                    "scratch (use stx_group_norm with a workspace)",
                    p.bytes, kGnScratchBytes);
        group_norm(a, dst, n_groups, eps, weight, bias, gelu, scratch_address(), p, as_stream(stream));
    });
}

STX_API stx_status stx_grid_sync_fallbacks(const void* workspace, uint32_t* count) {
    return guard([&] {
        STX_REQUIRE(count != nullptr, "grid_sync_fallbacks: count is NULL");
        const void* ws = workspace ? workspace : scratch_address();
        const char* src = static_cast<const char*>(ws) + kGridSyncFallback;
        hip_check(hipMemcpy(count, src, sizeof(uint32_t), hipMemcpyDeviceToHost), "hipMemcpy");
    });
}

STX_API stx_status stx_rope_ext(const stx_tensor* a, const int32_t* pos, const stx_tensor* dst, int n_dims, int mode,
                                int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                float beta_fast, float beta_slow, stx_stream stream) {
    return guard([&] {
        (void)n_ctx_orig;           // only used by YaRN
        (void)beta_fast;
        (void)beta_slow;
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "rope_ext");
        if (mode != 0 && mode != 2) fail(STX_STATUS_UNSUPPORTED, "rope_ext: mode %d (only 0 and 2)", mode);
        if (ext_factor != 0.0f) fail(STX_STATUS_UNSUPPORTED, "rope_ext: YaRN (ext_factor != 0) is not supported");
        STX_REQUIRE(n_dims > 0 && n_dims % 2 == 0 && n_dims <= a->ne[0], "rope_ext: n_dims must be even and <= ne0");
        const T4 ta = view(a), td = view(dst);
        if (nelem(ta) == 0) return;
        STX_REQUIRE(pos != nullptr, "rope_ext: pos is NULL");
        STX_REQUIRE(ta.ne[2] < (1LL << 31), "rope_ext: too many positions");
        bool vec2 = mode == 0 && (reinterpret_cast<uintptr_t>(ta.data) & 7) == 0 &&
                    (reinterpret_cast<uintptr_t>(td.data) & 7) == 0;
        for (int i = 1; i < 4; i++) vec2 = vec2 && ta.nb[i] % 8 == 0 && td.nb[i] % 8 == 0;
        RopeArgs r{ta, td, pos, n_dims, mode, vec2 ? 1 : 0, (double)freq_base, (double)freq_scale,
                   (double)attn_factor};
        const long long row_tiles = (ta.ne[1] * ta.ne[3] + kRopeRows - 1) / kRopeRows;
        STX_REQUIRE(row_tiles < 65536, "rope_ext: too many rows per position");
        bool v4 = mode == 0 && ta.ne[0] % 4 == 0 && n_dims % 4 == 0 && aligned16(ta.data) && aligned16(td.data) &&
                  ta.ne[1] * ta.ne[3] < (1LL << 31);
        for (int i = 1; i < 4; i++) v4 = v4 && ta.nb[i] % 16 == 0 && td.nb[i] % 16 == 0;
        if (v4) {
            hipLaunchKernelGGL(rope_v4_kernel, dim3((unsigned)ta.ne[2], (unsigned)row_tiles), dim3(256),
                               sizeof(double) * n_dims, as_stream(stream), r);
            launch_check("rope_v4_kernel");
        } else {
            hipLaunchKernelGGL(rope_kernel, dim3((unsigned)ta.ne[2], (unsigned)row_tiles), dim3(256),
                               sizeof(double) * n_dims, as_stream(stream), r);
            launch_check("rope_kernel");
        }
    });
}

}  // extern "C"
