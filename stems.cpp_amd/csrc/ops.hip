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
#include <type_traits>

#include "common.hpp"

namespace stx {
namespace {

constexpr int kWave = 64;

struct T4 {                      // device view of an stx_tensor
    char* data;
    long long ne[4];
    long long nb[4];
};

T4 view(const stx_tensor* t) {
    T4 v{};
    v.data = static_cast<char*>(t->data);
    for (int i = 0; i < 4; i++) {
        v.ne[i] = t->ne[i];
        v.nb[i] = t->nb[i];
    }
    return v;
}

long long nrows(const T4& t) { return t.ne[1] * t.ne[2] * t.ne[3]; }
long long nelem(const T4& t) { return t.ne[0] * nrows(t); }

bool contiguous(const T4& t) {
    return t.nb[0] == 4 && t.nb[1] == 4 * t.ne[0] && t.nb[2] == t.nb[1] * t.ne[1] && t.nb[3] == t.nb[2] * t.ne[2];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

void check_tensor(const stx_tensor* t, const char* what) {
    STX_REQUIRE(t != nullptr, "%s is NULL", what);
    long long n = 1;
    for (int i = 0; i < 4; i++) {
        STX_REQUIRE(t->ne[i] >= 0, "%s: negative ne[%d]", what, i);
        n *= t->ne[i];
    }
    STX_REQUIRE(t->nb[0] == 4, "%s: rows must be contiguous fp32 (nb[0] == 4)", what);
    for (int i = 1; i < 4; i++) STX_REQUIRE(t->nb[i] >= 0 && t->nb[i] % 4 == 0, "%s: bad stride nb[%d]", what, i);
    STX_REQUIRE(n < (1LL << 40), "%s too large", what);
    STX_REQUIRE(n == 0 || t->data != nullptr, "%s has no data", what);
}

void check_same_shape(const stx_tensor* a, const stx_tensor* b, const char* what) {
    for (int i = 0; i < 4; i++)
        STX_REQUIRE(a->ne[i] == b->ne[i], "%s: shape mismatch in ne[%d] (%lld vs %lld)", what, i,
                    (long long)a->ne[i], (long long)b->ne[i]);
}

// b repeats into dst (ggml_can_repeat): every dst->ne[i] is a multiple of b->ne[i].
void check_repeat(const stx_tensor* b, const stx_tensor* dst, const char* what) {
    for (int i = 0; i < 4; i++)
        STX_REQUIRE((b->ne[i] > 0 && dst->ne[i] % b->ne[i] == 0) || (b->ne[i] == 0 && dst->ne[i] == 0),
                    "%s: ne[%d] = %lld does not repeat into %lld", what, i, (long long)b->ne[i],
                    (long long)dst->ne[i]);
}

// Row r (flattened over ne1, ne2, ne3) of t.
__device__ __forceinline__ char* row_ptr(const T4& t, long long r) {
    const long long i1 = r % t.ne[1];
    const long long q = r / t.ne[1];
    const long long i2 = q % t.ne[2];
    const long long i3 = q / t.ne[2];
    return t.data + i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}

template <int LANES>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
    for (int m = LANES / 2; m >= 1; m /= 2) v += __shfl_xor(v, m, LANES);
    return v;
}

template <int LANES>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int m = LANES / 2; m >= 1; m /= 2) v = fmaxf(v, __shfl_xor(v, m, LANES));
    return v;
}

// Sum over a 256-thread block in a fixed order (deterministic). red holds 4 doubles.
__device__ __forceinline__ double block_sum(double v, double* red) {
    v = group_sum<kWave>(v);
    __syncthreads();
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// gelu(x) = x/2 * erfc(-x/sqrt2), evaluated to a few ulp everywhere.
//
// gelu_erf_hl takes its argument as a float head x plus a small tail dx (x + dx is the value),
// so that a fused producer can hand over a double result without rounding it first: in the
// negative tail d ln gelu / d ln x ~ 1 + x^2, so one ulp of input rounding would become ~x^2
// ulps of output error.
//
// x >= -1: erfcf of u = -x/sqrt2, with the rounding error du of u (from the product and from
//   1/sqrt2 itself) corrected to first order, erfc(u + du) = erfc(u) - 2/sqrt(pi) exp(-u^2) du.
// x < -1: erfc(u) = exp(-u^2) erfcx(u) with u^2 = x^2/2 split exactly into head and tail by an
//   fma, so exp(-u^2) costs one ulp instead of the 2u^2 ulps an unsplit exponent costs, and
//   erfcx from Shepherd & Laframboise's substitution (Chebyshev approximation of
//   (1 + 2u) exp(u^2) erfc(u), J. Comput. Phys. 1981): (1 + 2u) erfcx(u) = P(t),
//   t = (u - 2.5) / (u + 2.5), with P of degree 10 fitted here by weighted least squares in
//   double to relative error 1.3e-9 on u >= 0.7.
__device__ __forceinline__ float erfcx_scaled(float u) {
    constexpr float K = 2.5f;
    const float t = (u - K) / (u + K);
    float p = -1.919762726e-04f;
    p = fmaf(p, t, 5.875547067e-04f);
    p = fmaf(p, t, 5.759609630e-04f);
    p = fmaf(p, t, -4.387959838e-03f);
    p = fmaf(p, t, 9.082683246e-04f);
    p = fmaf(p, t, 3.276548162e-02f);
    p = fmaf(p, t, -1.029642969e-01f);
    p = fmaf(p, t, 1.576293558e-01f);
    p = fmaf(p, t, -9.902466089e-02f);
    p = fmaf(p, t, -1.223567501e-01f);
    p = fmaf(p, t, 1.264838219e+00f);
    return p / fmaf(2.f, u, 1.f);
}

__device__ __forceinline__ float gelu_erf_hl(float x, float dx) {
    constexpr float R = 0.70710678118654752440f;         // fl(1/sqrt2)
    constexpr float R_LO = 1.2101617e-08f;               // 1/sqrt2 - fl(1/sqrt2)
    const float u = -x * R;
    if (x < -1.f) {
        const float h = x * x;
        const float l = h < 1e37f ? fmaf(x, x, -h) : 0.f;                   // x^2 = h + l exactly
        float e = expf(-0.5f * h);
        e = fmaf(e, -fmaf(x, dx, 0.5f * l), e);          // * exp(-l/2 - x dx), first order
        const float q = 0.5f * e * erfcx_scaled(u);
        return fmaf(q, dx, q * x);
    }
    // (Past |x| = 1e30 the correction is meaningless and would turn infinities into NaN.)
    const float du = fabsf(x) < 1e30f ? fmaf(-x, R, -u) - x * R_LO - dx * R : 0.f;
    float e = erfcf(u);
    e = fmaf(-1.1283791670955126f * expf(-u * u), du, e);
    return fmaf(0.5f * dx, e, 0.5f * x * e);
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
            mean = group_sum<LANES>(s) / n;
        }
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const double d = (double)v[k] - mean;
            ss += lane + k * LANES < n ? d * d : 0.0;
        }
        ss = group_sum<LANES>(ss);
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
        const double ms = (double)(sgn * group_max<LANES>(m)) * sc;
        double sum = 0.0;
        float e[VPL];
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            e[k] = lane + k * LANES < n ? exp_split((double)v[k] * sc - ms) : 0.f;
            sum += (double)e[k];
        }
        const double inv = 1.0 / group_sum<LANES>(sum);
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const int i = lane + k * LANES;
            if (i < n) y[i] = (float)((double)e[k] * inv);
        }
    }
}

// --------------------------------------------------------------------- elementwise
enum EwOp { EW_GELU = 0, EW_GLU = 1, EW_ADD = 2, EW_MUL = 3, EW_MUL_ADD = 4, EW_ADD_GELU = 5 };

// GLU: x * sigmoid(y) with x and y two halves of one source. MUL_ADD: x + fl(y * z), rounded
// after each operation like ggml_add(x, ggml_mul(h, s)). ADD_GELU: gelu(fl(x + y)), a bias
// add followed by GELU.
__device__ __forceinline__ float ew_apply(int op, float x, float y, float z) {
#pragma clang fp contract(off)
    switch (op) {
        case EW_GELU: return gelu_erf(x);
        case EW_GLU: return x / (1.0f + expf(-y));
        case EW_ADD: return x + y;
        case EW_MUL: return x * y;
        case EW_MUL_ADD: {
            const float p = y * z;
            return x + p;
        }
        default: return gelu_erf(x + y);
    }
}

// General path. a: same shape as dst (any row strides). b, c repeat into dst. Work unit =
// (row, 1024-element chunk of the row).
struct EwArgs {
    T4 a, b, c, dst;
    int op;
};

__device__ __forceinline__ const float* bcast_row(const T4& t, long long i1, long long i2, long long i3) {
    return reinterpret_cast<const float*>(t.data + (i1 % t.ne[1]) * t.nb[1] + (i2 % t.ne[2]) * t.nb[2] +
                                          (i3 % t.ne[3]) * t.nb[3]);
}

__device__ __forceinline__ float bcast_at(const float* row, long long ne0, long long n0, long long i) {
    return ne0 == n0 ? row[i] : ne0 == 1 ? row[0] : row[i % ne0];
}

__global__ __launch_bounds__(256) void ew_rows_kernel(EwArgs a) {
    const long long rows = a.dst.ne[1] * a.dst.ne[2] * a.dst.ne[3];
    const long long n0 = a.dst.ne[0];
    const long long cpr = (n0 + 1023) / 1024;
    const bool has_b = a.op != EW_GELU, has_c = a.op == EW_MUL_ADD;
    for (long long u = blockIdx.x; u < rows * cpr; u += gridDim.x) {
        const long long r = u / cpr;
        const long long base = (u - r * cpr) * 1024;
        const long long i1 = r % a.dst.ne[1], q = r / a.dst.ne[1];
        const long long i2 = q % a.dst.ne[2], i3 = q / a.dst.ne[2];
        const float* xa = reinterpret_cast<const float*>(a.a.data + i1 * a.a.nb[1] + i2 * a.a.nb[2] + i3 * a.a.nb[3]);
        const float* xb = has_b ? bcast_row(a.b, i1, i2, i3) : nullptr;
        const float* xc = has_c ? bcast_row(a.c, i1, i2, i3) : nullptr;
        float* y = reinterpret_cast<float*>(a.dst.data + i1 * a.dst.nb[1] + i2 * a.dst.nb[2] + i3 * a.dst.nb[3]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const long long i = base + k * 256 + threadIdx.x;
            if (i < n0) {
                const float vb = has_b ? bcast_at(xb, a.b.ne[0], n0, i) : 0.f;
                const float vc = has_c ? bcast_at(xc, a.c.ne[0], n0, i) : 0.f;
                y[i] = ew_apply(a.op, xa[i], vb, vc);
            }
        }
    }
}

// Contiguous, same-shape, 16-byte aligned operands: flat float4 path.
__global__ __launch_bounds__(256) void ew_flat_kernel(int op, const float* __restrict__ xa, const float* __restrict__ xb,
                                                      const float* __restrict__ xc, float* __restrict__ y, long long n) {
    const long long n4 = n / 4;
    const float4* a4 = reinterpret_cast<const float4*>(xa);
    const float4* b4 = reinterpret_cast<const float4*>(xb);
    const float4* c4 = reinterpret_cast<const float4*>(xc);
    float4* y4 = reinterpret_cast<float4*>(y);
    const long long stride = (long long)gridDim.x * 256;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
        const float4 p = a4[i];
        const float4 q = xb ? b4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 s = xc ? c4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        y4[i] = make_float4(ew_apply(op, p.x, q.x, s.x), ew_apply(op, p.y, q.y, s.y), ew_apply(op, p.z, q.z, s.z),
                            ew_apply(op, p.w, q.w, s.w));
    }
    for (long long i = n4 * 4 + (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        y[i] = ew_apply(op, xa[i], xb ? xb[i] : 0.f, xc ? xc[i] : 0.f);
}

// ----------------------------------------------------------------------- GROUP_NORM
// Groups: for each i3, channels (ne2) [g*cpg, min((g+1)*cpg, ne2)) with cpg = ceil(ne2 / G),
// normalised together over ne0 x ne1 x channels (ggml_group_norm). Contiguous tensors only,
// so a group is one contiguous span of floats.
//   pass 1 (gn_partial_kernel): one block per 4096-float chunk of a group writes the chunk's
//     sum and its sum of squared deviations from its own mean (Chan et al.'s pairwise form,
//     no cancellation);
//   pass 2 (gn_apply_kernel): every block first combines its group's partials in a fixed
//     order (so all blocks agree bit for bit and the result is deterministic),
//     M2 = sum_k [M2_k + n_k (mean_k - mean)^2], then writes
//     ((x - mean) / sqrt(M2/N + eps)) [* w + b] [-> gelu] for 16384 floats, in double up to
//     the GELU, which takes the double as a float head and tail.
constexpr int kGnChunk = 4096;          // floats per partial (16 per thread)
constexpr int kGnApply = 4;             // chunks per apply block

enum AffineKind { AFF_NONE = 0, AFF_CHANNEL = 1, AFF_NE0 = 2, AFF_GENERAL = 3 };

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
    double* part;            // [groups_total][chunks][2]
    long long ne0, ne1, ne2; // dims of x (ne3 folded into the group index)
    long long plane;         // ne0 * ne1
    long long cpg;           // channels per group
    int groups;              // groups per ne3 slice
    int chunks;              // partials per group (max over groups)
    float eps;
    int gelu;
    int vec;                 // all group spans 16-byte aligned
};

__device__ __forceinline__ void group_span(const GroupNormArgs& a, int gt, long long& begin, long long& count,
                                           long long& c0, long long& i3) {
    i3 = gt / a.groups;
    const long long g = gt % a.groups;
    c0 = g * a.cpg;
    const long long c1 = min(c0 + a.cpg, a.ne2);
    begin = i3 * a.ne2 * a.plane + c0 * a.plane;
    count = (c1 - c0) * a.plane;
}

// Loads the 16 values of this thread in chunk [lo, hi) of base: float4 k covers positions
// lo + (k * 256 + tid) * 4 .. +3.
__device__ __forceinline__ void gn_load(const GroupNormArgs& a, const float* base, long long lo, long long hi,
                                        float (&v)[16], bool (&ok)[16]) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const long long p = lo + ((long long)k * 256 + threadIdx.x) * 4;
        if (a.vec && p + 3 < hi) {
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
                ok[4 * k + j] = p + j < hi;
                v[4 * k + j] = ok[4 * k + j] ? base[p + j] : 0.f;
            }
        }
    }
}

__global__ __launch_bounds__(256) void gn_partial_kernel(GroupNormArgs a) {
    __shared__ double red[4];
    const int gt = (int)blockIdx.y;
    long long begin, count, c0, i3;
    group_span(a, gt, begin, count, c0, i3);
    const long long lo = (long long)blockIdx.x * kGnChunk;
    if (lo >= count) return;                                   // uniform over the block
    const long long hi = min(lo + kGnChunk, count);
    float v[16];
    bool ok[16];
    gn_load(a, a.x + begin, lo, hi, v, ok);
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < 16; k++) s += (double)v[k];
    s = block_sum(s, red);
    const double mu = s / (double)(hi - lo);
    double m2 = 0.0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const double d = (double)v[k] - mu;
        m2 += ok[k] ? d * d : 0.0;
    }
    m2 = block_sum(m2, red);
    if (threadIdx.x == 0) {
        double* p = a.part + ((size_t)gt * a.chunks + blockIdx.x) * 2;
        p[0] = s;
        p[1] = m2;
    }
}

__device__ __forceinline__ float affine_at(const Affine& f, long long c, long long i0, long long i1, long long i3) {
    switch (f.kind) {
        case AFF_CHANNEL: return f.p[c];
        case AFF_NE0: return f.p[i0];
        default:
            return f.p[(i0 % f.ne[0]) * f.nb[0] + (i1 % f.ne[1]) * f.nb[1] + (c % f.ne[2]) * f.nb[2] +
                       (i3 % f.ne[3]) * f.nb[3]];
    }
}

__global__ __launch_bounds__(256) void gn_apply_kernel(GroupNormArgs a) {
    __shared__ double red[4];
    const int gt = (int)blockIdx.y;
    long long begin, count, c0, i3;
    group_span(a, gt, begin, count, c0, i3);
    const long long lo0 = (long long)blockIdx.x * kGnChunk * kGnApply;
    if (lo0 >= count) return;                                  // uniform over the block
    const int nch = (int)((count + kGnChunk - 1) / kGnChunk);
    const double* part = a.part + (size_t)gt * a.chunks * 2;
    double s = 0.0;
    for (int k = threadIdx.x; k < nch; k += 256) s += part[2 * k];
    const double N = (double)count;
    const double mean = block_sum(s, red) / N;
    double m2 = 0.0;
    for (int k = threadIdx.x; k < nch; k += 256) {
        const double nk = (double)(min((long long)(k + 1) * kGnChunk, count) - (long long)k * kGnChunk);
        const double d = part[2 * k] / nk - mean;
        m2 += part[2 * k + 1] + nk * d * d;
    }
    m2 = block_sum(m2, red);
    const double rstd = 1.0 / sqrt(m2 / N + (double)a.eps);
    const float* xg = a.x + begin;
    float* yg = a.y + begin;
    for (int cc = 0; cc < kGnApply; cc++) {
        const long long lo = lo0 + (long long)cc * kGnChunk;
        if (lo >= count) break;
        const long long hi = min(lo + kGnChunk, count);
        float v[16];
        bool ok[16];
        gn_load(a, xg, lo, hi, v, ok);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const long long p = lo + ((long long)k * 256 + threadIdx.x) * 4;
            if (p >= hi) continue;
            // Channel c and (i0, i1) inside its plane of element p, advanced element by element.
            long long c = 0, i0 = 0, i1 = 0;
            if (a.w.kind || a.b.kind) {
                c = c0 + p / a.plane;
                const long long q = p % a.plane;
                i1 = q / a.ne0;
                i0 = q % a.ne0;
            }
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                double t = ((double)v[4 * k + j] - mean) * rstd;
                if (a.w.kind) t *= (double)affine_at(a.w, c, i0, i1, i3);
                if (a.b.kind) t += (double)affine_at(a.b, c, i0, i1, i3);
                const float f = (float)t;
                o[j] = a.gelu ? gelu_erf_hl(f, (float)(t - (double)f)) : f;
                if (++i0 == a.ne0) {
                    i0 = 0;
                    if (++i1 == a.ne1) {
                        i1 = 0;
                        ++c;
                    }
                }
            }
            if (a.vec && p + 3 < hi) {
                *reinterpret_cast<float4*>(yg + p) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (ok[4 * k + j]) yg[p + j] = o[j];
            }
        }
    }
}

// ----------------------------------------------------------------------------- ROPE
// ggml_rope_ext without YaRN (ext_factor 0): theta_i = freq_scale * pos * base^(-2i/n_dims),
// cos and sin scaled by attn_factor. Mode 0 rotates adjacent pairs (2i, 2i+1), mode 2 (NEOX)
// the pairs (i, i + n_dims/2); elements past n_dims are copied. Each block takes one position
// (ne2 index) and kRopeRows of its (ne1, ne3) rows; it evaluates cos/sin in double once per
// pair into LDS and rotates in double, rounding once. A thread owns a whole pair (or one
// copied element), so dst may alias src.
constexpr int kRopeRows = 32;

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
    RowNormArgs args{view(a), view(dst), gamma, beta, eps, rms};
    const long long rows = nrows(args.src), n = args.src.ne[0];
    if (rows == 0 || n == 0) return;
    STX_REQUIRE(n < (1LL << 31), "row too long");
    const hipStream_t s = as_stream(stream);
    if (n <= kMaxRowShapeN) {
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

void elementwise(int op, const stx_tensor* a, const stx_tensor* b, const stx_tensor* c, const stx_tensor* dst,
                 stx_stream stream) {
    EwArgs args{};
    args.op = op;
    args.a = view(a);
    args.dst = view(dst);
    if (b) args.b = view(b);
    if (c) args.c = view(c);
    const long long n = nelem(args.dst);
    if (n == 0) return;
    const hipStream_t s = as_stream(stream);
    bool flat = contiguous(args.a) && contiguous(args.dst) && aligned16(args.a.data) && aligned16(args.dst.data);
    for (const stx_tensor* t : {b, c}) {
        if (!t) continue;
        const T4 v = view(t);
        flat = flat && contiguous(v) && aligned16(v.data);
        for (int i = 0; i < 4; i++) flat = flat && t->ne[i] == dst->ne[i];
    }
    if (flat) {
        const unsigned blocks = (unsigned)std::min<long long>((n / 4 + 255) / 256 + 1, 1 << 16);
        hipLaunchKernelGGL(ew_flat_kernel, dim3(blocks), dim3(256), 0, s, op,
                           reinterpret_cast<const float*>(args.a.data),
                           b ? reinterpret_cast<const float*>(args.b.data) : nullptr,
                           c ? reinterpret_cast<const float*>(args.c.data) : nullptr,
                           reinterpret_cast<float*>(args.dst.data), n);
        launch_check("ew_flat_kernel");
        return;
    }
    const long long units = nrows(args.dst) * ((args.dst.ne[0] + 1023) / 1024);
    hipLaunchKernelGGL(ew_rows_kernel, dim3((unsigned)std::min<long long>(units, 1 << 20)), dim3(256), 0, s, args);
    launch_check("ew_rows_kernel");
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
    long long cpg, groups, groups_total, chunks;
};

GnPlan gn_plan(const stx_tensor* a, int n_groups) {
    GnPlan p{};
    p.cpg = std::max<long long>(1, (a->ne[2] + n_groups - 1) / n_groups);
    p.groups = (a->ne[2] + p.cpg - 1) / p.cpg;
    p.groups_total = p.groups * a->ne[3];
    p.chunks = (p.cpg * a->ne[0] * a->ne[1] + kGnChunk - 1) / kGnChunk;
    return p;
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
        SoftmaxArgs args{view(a), view(dst), scale};
        const long long rows = nrows(args.src), n = args.src.ne[0];
        if (rows == 0 || n == 0) return;
        if (n > kMaxRowShapeN) fail(STX_STATUS_UNSUPPORTED, "soft_max_ext: rows longer than 2048 are not supported");
        const hipStream_t s = as_stream(stream);
        pick_row_shape(n, [&](auto lanes, auto vpl) {
            constexpr int L = decltype(lanes)::value, V = decltype(vpl)::value;
            hipLaunchKernelGGL((softmax_kernel<L, V>), dim3(row_blocks(rows, L)), dim3(256), 0, s, args);
        });
        launch_check("softmax_kernel");
    });
}

STX_API stx_status stx_gelu_erf(const stx_tensor* a, const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "gelu_erf");
        elementwise(EW_GELU, a, nullptr, nullptr, dst, stream);
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
        elementwise(EW_ADD_GELU, a, b, nullptr, dst, stream);
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
        elementwise(EW_GLU, &va, &vg, nullptr, dst, stream);
    });
}

STX_API stx_status stx_add(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(b, "b");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "add");
        check_repeat(b, dst, "add");
        elementwise(EW_ADD, a, b, nullptr, dst, stream);
    });
}

STX_API stx_status stx_mul(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(b, "b");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "mul");
        check_repeat(b, dst, "mul");
        elementwise(EW_MUL, a, b, nullptr, dst, stream);
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
        elementwise(EW_MUL_ADD, x, h, s, dst, stream);
    });
}

STX_API size_t stx_group_norm_workspace_size(const stx_tensor* a, int n_groups) {
    if (!a || n_groups < 1) return 0;
    for (int i = 0; i < 4; i++)
        if (a->ne[i] < 0) return 0;
    const GnPlan p = gn_plan(a, n_groups);
    return sizeof(double) * 2 * (size_t)std::max<long long>(1, p.chunks * p.groups_total);
}

STX_API stx_status stx_group_norm(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps,
                                  const stx_tensor* weight, const stx_tensor* bias, int gelu, void* workspace,
                                  size_t workspace_bytes, stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        check_same_shape(a, dst, "group_norm");
        STX_REQUIRE(n_groups >= 1, "group_norm: n_groups < 1");
        const T4 ta = view(a), td = view(dst);
        STX_REQUIRE(contiguous(ta) && contiguous(td), "group_norm: tensors must be contiguous");
        const Affine w = make_affine(weight, a, "weight");
        const Affine b = make_affine(bias, a, "bias");
        if (nelem(ta) == 0) return;
        const GnPlan p = gn_plan(a, n_groups);
        STX_REQUIRE(p.groups_total < 65536, "group_norm: more than 65535 groups");
        STX_REQUIRE(p.chunks < (1LL << 31), "group_norm: group too large");
        const size_t need = sizeof(double) * 2 * (size_t)(p.chunks * p.groups_total);
        STX_REQUIRE(workspace != nullptr && workspace_bytes >= need, "group_norm: workspace too small (%zu, need %zu)",
                    workspace_bytes, need);
        GroupNormArgs g{};
        g.x = reinterpret_cast<const float*>(ta.data);
        g.y = reinterpret_cast<float*>(td.data);
        g.w = w;
        g.b = b;
        g.part = static_cast<double*>(workspace);
        g.ne0 = ta.ne[0];
        g.ne1 = ta.ne[1];
        g.ne2 = ta.ne[2];
        g.plane = ta.ne[0] * ta.ne[1];
        g.cpg = p.cpg;
        g.groups = (int)p.groups;
        g.chunks = (int)p.chunks;
        g.eps = eps;
        g.gelu = gelu ? 1 : 0;
        // Every group span starts at (i3 * ne2 + g * cpg) * plane floats.
        g.vec = aligned16(ta.data) && aligned16(td.data) && (g.cpg * g.plane) % 4 == 0 &&
                        (ta.ne[3] == 1 || (g.ne2 * g.plane) % 4 == 0)
                    ? 1
                    : 0;
        const hipStream_t s = as_stream(stream);
        hipLaunchKernelGGL(gn_partial_kernel, dim3((unsigned)p.chunks, (unsigned)p.groups_total), dim3(256), 0, s, g);
        launch_check("gn_partial_kernel");
        const unsigned apply_blocks = (unsigned)((p.chunks + kGnApply - 1) / kGnApply);
        hipLaunchKernelGGL(gn_apply_kernel, dim3(apply_blocks, (unsigned)p.groups_total), dim3(256), 0, s, g);
        launch_check("gn_apply_kernel");
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
        hipLaunchKernelGGL(rope_kernel, dim3((unsigned)ta.ne[2], (unsigned)row_tiles), dim3(256),
                           sizeof(double) * n_dims, as_stream(stream), r);
        launch_check("rope_kernel");
    });
}

}  // extern "C"
