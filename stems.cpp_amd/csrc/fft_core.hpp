// fft_core.hpp — the complex FFT building blocks of every spectral kernel.
//
// One complex M-point transform (M a power of two, 8 <= M <= 4096) is computed by M/P
// threads holding P = 8 or 16 points each, with a self-sorting Stockham formulation: the
// first radix-P pass runs straight on registers loaded from global memory, the remaining
// passes (radix P, then one smaller radix when log_P M is not an integer) exchange through
// LDS. Input and output are in natural order, so no bit reversal is needed (the reference's
// radix-2 DIT does one, src/stft.h:36). P = 8 gives short waves (latency-bound small
// batches), P = 16 the fewest LDS passes (throughput-bound large batches).
//
// Pass with radix R after sub-transforms of length Ns: butterfly jj in [0, M/R) reads
// a[jj + r*M/R] (r < R), multiplies element r by W_{Ns*R}^{(jj mod Ns)*r}, takes an R-point
// DFT and writes element r to b[(jj / Ns)*Ns*R + (jj mod Ns) + r*Ns].
//
// Twiddles come from one table for TN points (TN = M for a complex transform, 2M for the
// half-length transform of a real one, i.e. the real transform's n_fft):
// W_TN^m = lo[m mod L] * hi[m / L] (L = 2^ceil(log2(TN)/2); at most 1.5 KB, staged in LDS at
// kernel start, every entry computed in double and rounded to float once). A butterfly looks
// up w^1, w^2, w^4, w^8 of its base twiddle and forms the other powers as products of those
// (at most three deep): about 140 dB against an exact DFT, 2 dB below exact tables.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

namespace stx {

#define STX_HD __host__ __device__ __forceinline__

STX_HD float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
STX_HD float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
STX_HD float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
STX_HD float2 cmul_mi(float2 a) { return make_float2(a.y, -a.x); }          // a * (-i)
STX_HD float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
STX_HD float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }

// Forward DFTs (kernel exp(-2*pi*i*n*k/R)) in natural order, in place on v[0..R).
template <int R> struct Dft;

template <> struct Dft<2> {
    static STX_HD void run(float2* v) {
        const float2 a = v[0], b = v[1];
        v[0] = cadd(a, b);
        v[1] = csub(a, b);
    }
};

template <> struct Dft<4> {
    static STX_HD void run(float2* v) {
        const float2 t0 = cadd(v[0], v[2]), t1 = csub(v[0], v[2]);
        const float2 t2 = cadd(v[1], v[3]), t3 = cmul_mi(csub(v[1], v[3]));
        v[0] = cadd(t0, t2);
        v[2] = csub(t0, t2);
        v[1] = cadd(t1, t3);
        v[3] = csub(t1, t3);
    }
};

template <> struct Dft<8> {
    static STX_HD void run(float2* v) {
        constexpr float r = 0.70710678118654752440f;
        float2 e[4] = {v[0], v[2], v[4], v[6]};
        float2 o[4] = {v[1], v[3], v[5], v[7]};
        Dft<4>::run(e);
        Dft<4>::run(o);
        o[1] = make_float2(r * (o[1].x + o[1].y), r * (o[1].y - o[1].x));     // * W8^1
        o[2] = cmul_mi(o[2]);                                                 // * W8^2
        o[3] = make_float2(r * (o[3].y - o[3].x), -r * (o[3].x + o[3].y));    // * W8^3
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = cadd(e[k], o[k]);
            v[k + 4] = csub(e[k], o[k]);
        }
    }
};

// 16 = 4 x 4: n = 4*n1 + n2, k = k1 + 4*k2, inner twiddles W16^(n2*k1).
template <> struct Dft<16> {
    static STX_HD void run(float2* v) {
        constexpr float c1 = 0.92387953251128675613f;   // cos(pi/8)
        constexpr float s1 = 0.38268343236508977173f;   // sin(pi/8)
        constexpr float r = 0.70710678118654752440f;
        float2 b[4][4];
#pragma unroll
        for (int n2 = 0; n2 < 4; n2++) {
            float2 t[4] = {v[n2], v[4 + n2], v[8 + n2], v[12 + n2]};
            Dft<4>::run(t);
#pragma unroll
            for (int k1 = 0; k1 < 4; k1++) b[n2][k1] = t[k1];
        }
        b[1][1] = cmul(b[1][1], make_float2(c1, -s1));   // W16^1
        b[1][2] = cmul(b[1][2], make_float2(r, -r));     // W16^2
        b[1][3] = cmul(b[1][3], make_float2(s1, -c1));   // W16^3
        b[2][1] = cmul(b[2][1], make_float2(r, -r));     // W16^2
        b[2][2] = cmul_mi(b[2][2]);                      // W16^4
        b[2][3] = cmul(b[2][3], make_float2(-r, -r));    // W16^6
        b[3][1] = cmul(b[3][1], make_float2(s1, -c1));   // W16^3
        b[3][2] = cmul(b[3][2], make_float2(-r, -r));    // W16^6
        b[3][3] = cmul(b[3][3], make_float2(-c1, s1));   // W16^9
#pragma unroll
        for (int k1 = 0; k1 < 4; k1++) {
            float2 t[4] = {b[0][k1], b[1][k1], b[2][k1], b[3][k1]};
            Dft<4>::run(t);
#pragma unroll
            for (int k2 = 0; k2 < 4; k2++) v[k1 + 4 * k2] = t[k2];
        }
    }
};

// Odd radices of the mixed-radix path (sizes 2^a 3^b 5^c). Dft<3>: X1,2 = a - (b + c)/2 -/+
// i sqrt(3)/2 (b - c). Dft<5>: with t1 = x1 + x4, t2 = x2 + x3, t3 = x1 - x4, t4 = x2 - x3,
// X1,4 = x0 + c1 t1 + c2 t2 -/+ i (s1 t3 + s2 t4), X2,3 = x0 + c2 t1 + c1 t2 -/+ i (s2 t3 - s1 t4),
// c_k = cos(2 pi k / 5), s_k = sin(2 pi k / 5).
template <> struct Dft<3> {
    static STX_HD void run(float2* v) {
        constexpr float h = 0.86602540378443864676f;     // sqrt(3) / 2
        const float2 a = v[0], t1 = cadd(v[1], v[2]), t2 = csub(v[1], v[2]);
        const float2 m = make_float2(a.x - 0.5f * t1.x, a.y - 0.5f * t1.y);
        const float2 q = make_float2(h * t2.y, -h * t2.x);  // -i h t2
        v[0] = cadd(a, t1);
        v[1] = cadd(m, q);
        v[2] = csub(m, q);
    }
};

template <> struct Dft<5> {
    static STX_HD void run(float2* v) {
        constexpr float c1 = 0.30901699437494742410f, c2 = -0.80901699437494742410f;
        constexpr float s1 = 0.95105651629515357212f, s2 = 0.58778525229247312917f;
        const float2 x0 = v[0];
        const float2 t1 = cadd(v[1], v[4]), t2 = cadd(v[2], v[3]);
        const float2 t3 = csub(v[1], v[4]), t4 = csub(v[2], v[3]);
        const float2 a1 = make_float2(x0.x + c1 * t1.x + c2 * t2.x, x0.y + c1 * t1.y + c2 * t2.y);
        const float2 a2 = make_float2(x0.x + c2 * t1.x + c1 * t2.x, x0.y + c2 * t1.y + c1 * t2.y);
        const float2 b1 = make_float2(s1 * t3.x + s2 * t4.x, s1 * t3.y + s2 * t4.y);
        const float2 b2 = make_float2(s2 * t3.x - s1 * t4.x, s2 * t3.y - s1 * t4.y);
        const float2 ib1 = make_float2(b1.y, -b1.x), ib2 = make_float2(b2.y, -b2.x);   // -i b
        v[0] = cadd(x0, cadd(t1, t2));
        v[1] = cadd(a1, ib1);
        v[4] = csub(a1, ib1);
        v[2] = cadd(a2, ib2);
        v[3] = csub(a2, ib2);
    }
};

// Dft<15>: the prime-factor algorithm (3 and 5 coprime, so no twiddles between them): input
// x[(5 n1 + 3 n2) mod 15] at a[n1][n2], 5-point DFTs along n2, 3-point DFTs along n1, output
// X[(10 k1 + 6 k2) mod 15] from b[k1][k2] (W15^(nk) = W3^(n1 k1) W5^(n2 k2) for these maps).
template <> struct Dft<15> {
    static STX_HD void run(float2* v) {
        float2 a[3][5];
#pragma unroll
        for (int n1 = 0; n1 < 3; n1++)
#pragma unroll
            for (int n2 = 0; n2 < 5; n2++) a[n1][n2] = v[(5 * n1 + 3 * n2) % 15];
#pragma unroll
        for (int n1 = 0; n1 < 3; n1++) Dft<5>::run(a[n1]);
#pragma unroll
        for (int k2 = 0; k2 < 5; k2++) {
            float2 t[3] = {a[0][k2], a[1][k2], a[2][k2]};
            Dft<3>::run(t);
#pragma unroll
            for (int k1 = 0; k1 < 3; k1++) v[(10 * k1 + 6 * k2) % 15] = t[k1];
        }
    }
};

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// cos and sin of x (|x| <= pi) by their Taylor series in double, for twiddle constants computed
// at compile time (the terms fall below 1e-17 well before the 40th).
constexpr double cx_cos(double x) {
    double t = 1.0, s = 0.0;
    for (int n = 0; n < 40; n += 2) {
        s += t;
        t *= -x * x / ((n + 1.0) * (n + 2.0));
    }
    return s;
}
constexpr double cx_sin(double x) {
    double t = x, s = 0.0;
    for (int n = 1; n < 41; n += 2) {
        s += t;
        t *= -x * x / ((n + 1.0) * (n + 2.0));
    }
    return s;
}
constexpr double kPi = 3.14159265358979323846;

// exp(-i pi r / P) for r <= P, rounded to float, as compile-time constants.
template <int P> struct HalfTurnRoots { float re[P + 1], im[P + 1]; };
template <int P> constexpr HalfTurnRoots<P> half_turn_roots() {
    HalfTurnRoots<P> t{};
    for (int r = 0; r <= P; r++) {
        t.re[r] = 2 * r == P ? 0.f : (float)cx_cos(kPi * r / P);     // exact 0 and -1 at pi/2 and pi
        t.im[r] = r == P ? 0.f : (float)-cx_sin(kPi * r / P);
    }
    return t;
}

// Two-level twiddle table for TN points: [L low entries W^m, m < L][H high entries W^(L*h)].
template <int TN> struct TwTable {
    static constexpr int LBITS = (ilog2(TN) + 1) / 2;
    static constexpr int L = 1 << LBITS;
    static constexpr int H = TN / L;
    static constexpr int SIZE = L + H;
};

inline int twiddle_table_size(int tn) {
    const int lb = (ilog2(tn) + 1) / 2;
    return (1 << lb) + tn / (1 << lb);
}

// W_TN^m (0 <= m < TN) from the LDS copy of the table.
template <int TN>
__device__ __forceinline__ float2 tw_lookup(const float2* __restrict__ twt, int m) {
    using T = TwTable<TN>;
    return cmul(twt[m & (T::L - 1)], twt[T::L + (m >> T::LBITS)]);
}

// Copies COUNT elements to LDS with NT threads, every load issued before the first LDS write
// (a loop with a thread-dependent trip count would wait for each load in turn). The caller's
// next barrier publishes the copy.
template <int COUNT, int NT, class T>
__device__ __forceinline__ void stage_lds(T* dst, const T* __restrict__ src, int tid) {
    constexpr int R = (COUNT + NT - 1) / NT;
    T v[R];
#pragma unroll
    for (int r = 0; r < R; r++) v[r] = src[min(tid + r * NT, COUNT - 1)];
#pragma unroll
    for (int r = 0; r < R; r++)
        if (tid + r * NT < COUNT) dst[tid + r * NT] = v[r];
}

// Copies the twiddle table to LDS; the caller's next barrier publishes it.
template <int TN, int NT>
__device__ __forceinline__ void stage_twiddles(float2* twt, const float2* __restrict__ g, int tid) {
    stage_lds<TwTable<TN>::SIZE, NT>(twt, g, tid);
}

// stage_lds in two halves: load() issues a thread's share of a table into registers (at the top
// of a kernel, so that the table's round trip overlaps the data loads), store() writes it to
// LDS after the data loads have been issued; the caller's next barrier publishes it.
template <int COUNT, int NT, class T>
struct Staged {
    static constexpr int R = (COUNT + NT - 1) / NT;
    T v[R];
    __device__ __forceinline__ void load(const T* __restrict__ src, int tid) {
#pragma unroll
        for (int r = 0; r < R; r++) v[r] = src[min(tid + r * NT, COUNT - 1)];
    }
    __device__ __forceinline__ void store(T* dst, int tid) const {
#pragma unroll
        for (int r = 0; r < R; r++)
            if (tid + r * NT < COUNT) dst[tid + r * NT] = v[r];
    }
};
template <int TN, int NT>
using StagedTwiddles = Staged<TwTable<TN>::SIZE, NT, float2>;

// Shape of an M-point transform with P points per thread.
template <int M, int P, int TN_> struct FftCfg {
    static_assert(P == 8 || P == 16, "P must be 8 or 16");
    static_assert(M >= P && M <= 8192 && (M & (M - 1)) == 0, "M must be a power of two in [P, 8192]");
    static_assert(TN_ % M == 0, "the twiddle table must cover the transform");
    static constexpr int TPJ = M / P;                 // threads per transform
    static constexpr int TN = TN_;                    // twiddle table size
    // LDS float2 per transform: the padded transform (one pad per P), at least M + 2 for the
    // staged half spectra, rounded to even.
    static constexpr int PADN = ((M + M / P > M + 2 ? M + M / P : M + 2) + 1) / 2 * 2;
    static STX_HD int idx(int i) { return i + i / P; }
};

// w[r] = W_{Ns*R}^{k*r} = W_TN^{k*r*scale} for r < R, scale = TN / (Ns*R).
template <int TN, int R>
__device__ __forceinline__ void twiddle_powers(const float2* __restrict__ twt, int m1, float2* w) {
    w[1] = tw_lookup<TN>(twt, m1);
    if constexpr (R > 2) {
        w[2] = tw_lookup<TN>(twt, 2 * m1);
        w[3] = cmul(w[2], w[1]);
    }
    if constexpr (R > 4) {
        w[4] = tw_lookup<TN>(twt, 4 * m1);
        w[5] = cmul(w[4], w[1]);
        w[6] = cmul(w[4], w[2]);
        w[7] = cmul(w[4], w[3]);
    }
    if constexpr (R > 8) {
        w[8] = tw_lookup<TN>(twt, 8 * m1);
#pragma unroll
        for (int r = 9; r < 16; r++) w[r] = cmul(w[8], w[r - 8]);
    }
}

// Orders the LDS accesses of one wave around an exchange among its own lanes. A wave's LDS
// instructions are performed in the order they are issued, so no wait is needed: only the
// compiler has to be kept from moving accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}
// The workgroup's barrier for data exchanged through LDS only: waits for this wave's LDS
// accesses (lgkmcnt 0; vmcnt and expcnt left at their maxima) and meets the other waves, but
// does not wait for global loads in flight, as __syncthreads' workgroup fence does. Global
// memory written before it is not made visible to the other waves.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}
// Between two passes: the workgroup's LDS barrier, or the wave's ordering when every transform
// belongs to one wave (WAVE: TPJ == 64, so no lane reads another wave's data).
template <bool WAVE>
__device__ __forceinline__ void pass_sync() {
    if constexpr (WAVE) wave_lds_sync();
    else lds_barrier();
}

struct NoPost {
    __device__ __forceinline__ float2 operator()(int, float2 v) const { return v; }
};

// Sink writing into the transform's own LDS buffer (natural order).
template <int P>
struct ToLds {
    float2* buf;
    __device__ __forceinline__ void operator()(int n, float2 v) const { buf[n + n / P] = v; }
};

// Sink writing element n at LDS index n (unpadded): for a last pass whose consecutive lanes
// write consecutive elements, so the reader of the result needs no padded index.
struct ToLdsFlat {
    float2* buf;
    __device__ __forceinline__ void operator()(int n, float2 v) const { buf[n] = v; }
};

// LDS addressing: element i of a transform lives at idx(i) = i + i / P. For a base b and a
// multiple s of P, idx(b + r s) = idx(b) + r (s + s / P), so every LDS access of a butterfly is
// one base index plus a compile-time offset (an immediate of the ds instruction) instead of an
// index computation per element.

// First pass (Ns = 1, radix P): v holds a[j + r*M/P] for r < P on entry. Writes to the LDS
// buffer (elements j*P + r, at idx = j*(P + 1) + r), or, when it is also the last pass
// (M == P), to `sink` through `post`.
template <int M, int P, int TN, class Post, class Sink>
__device__ __forceinline__ void fft_first_pass(float2* v, float2* buf, int j, const Post& post, const Sink& sink) {
    Dft<P>::run(v);
    float2* w = buf + j * (P + 1);
#pragma unroll
    for (int r = 0; r < P; r++) {
        if constexpr (M == P) sink(j * P + r, post(j * P + r, v[r]));
        else w[r] = v[r];
    }
}

// Remaining passes, in place in `buf`. Every thread of the workgroup must call this (it
// contains barriers), also threads whose transform is idle. The last pass hands every output
// element n (natural order) to sink(n, post(n, v)). With WAVE (each transform is one wave's)
// the passes are ordered per wave, and no workgroup barrier follows the last one.
template <int M, int P, int TN, int Ns, bool WAVE = false, class Post, class Sink>
__device__ __forceinline__ void fft_rest_passes(float2* buf, int j, const float2* __restrict__ twt,
                                                const Post& post, const Sink& sink) {
    if constexpr (Ns < M) {
        using C = FftCfg<M, P, TN>;
        constexpr int R = (M / Ns >= P) ? P : M / Ns;
        constexpr int TPJ = C::TPJ;
        constexpr int BPT = P / R;                    // butterflies per thread
        constexpr int SCALE = C::TN / (Ns * R);       // W_{Ns*R}^e = W_TN^(e*SCALE)
        constexpr bool LAST = (Ns * R == M);
        static_assert((M / R) % P == 0 && Ns % P == 0, "strides of the rest passes are multiples of P");
        constexpr int RS = M / R + M / R / P;         // LDS distance between a butterfly's inputs
        constexpr int WS = Ns + Ns / P;               // ... and between its outputs
        constexpr bool TO_LDS = std::is_same<Sink, ToLds<P>>::value;
        float2 v[P];
#pragma unroll
        for (int q = 0; q < BPT; q++) {
            const float2* rd = buf + C::idx(j + q * TPJ);
#pragma unroll
            for (int r = 0; r < R; r++) v[q * R + r] = rd[r * RS];
        }
        pass_sync<WAVE>();
#pragma unroll
        for (int q = 0; q < BPT; q++) {
            const int jj = j + q * TPJ;
            const int k = jj % Ns;
            float2 w[R];
            twiddle_powers<C::TN, R>(twt, k * SCALE, w);
#pragma unroll
            for (int r = 1; r < R; r++) v[q * R + r] = cmul(v[q * R + r], w[r]);
            Dft<R>::run(&v[q * R]);
            const int base = (jj / Ns) * Ns * R + k;
            float2* wr = buf + C::idx(base);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int n = base + r * Ns;
                if constexpr (LAST && TO_LDS) wr[r * WS] = post(n, v[q * R + r]);
                else if constexpr (LAST) sink(n, post(n, v[q * R + r]));
                else wr[r * WS] = v[q * R + r];
            }
        }
        pass_sync<WAVE>();
        fft_rest_passes<M, P, TN, Ns * R, WAVE>(buf, j, twt, post, sink);
    }
}

}  // namespace stx

namespace stx {

// Mixed-radix plan of an M-point complex transform, M = 2^a 3^b 5^c: radix 16 passes while 16
// divides what is left, then one of 8, 4 or 2, then 15s (a 3 and a 5 in one pass), then the
// remaining 3s and 5s.
struct MixedRadix {
    int count = 0;
    int r[24] = {};
};

inline bool mixed_plan(int m, MixedRadix& p) {
    p = MixedRadix{};
    if (m < 1) return false;
    int left = m;
    while (left % 16 == 0) { p.r[p.count++] = 16; left /= 16; }
    for (int q : {8, 4, 2})
        if (left % q == 0) { p.r[p.count++] = q; left /= q; }
    while (left % 15 == 0) { p.r[p.count++] = 15; left /= 15; }
    while (left % 3 == 0) { p.r[p.count++] = 3; left /= 3; }
    while (left % 5 == 0) { p.r[p.count++] = 5; left /= 5; }
    return left == 1 && p.count <= 24;
}

// LDS layout of the mixed-radix buffers: element i at i + i / 16, so that the first pass's
// stride-16 writes (and every other power-of-two stride of 16 or more) spread over the banks.
// A buffer for M elements holds mixed_padded(M) float2.
__host__ __device__ constexpr int mixed_pad(int i) { return i + (i >> 4); }
__host__ __device__ constexpr int mixed_padded(int m) { return m + m / 16 + 1; }

// Twiddles of the mixed-radix passes: a two-level table of W_n^m staged in LDS, lo[j] = W_n^j
// for j < kMixedTwL, then hi[h] = W_n^(h kMixedTwL) for h < ceil(n / kMixedTwL), every entry
// computed in double and rounded once; W_n^m = lo[m mod kMixedTwL] * hi[m / kMixedTwL]. Two LDS
// reads and a complex product per twiddle instead of a global load per pass (a memory round trip
// on every pass's critical path). n <= 16384.
constexpr int kMixedTwL = 128;
constexpr int kMixedTwMax = kMixedTwL + 16384 / kMixedTwL;
__device__ __forceinline__ float2 mixed_tw(const float2* twl, int m) {
    return cmul(twl[m & (kMixedTwL - 1)], twl[kMixedTwL + (m >> 7)]);
}
static_assert(kMixedTwL == 128, "mixed_tw shifts by log2(kMixedTwL)");

// One out-of-place Stockham pass of radix R after sub-transforms of length Ns over an M-point
// transform held in src (natural order, padded layout), by the NT threads of a workgroup:
// butterfly b reads src[b + r M/R], multiplies element r by W_{Ns R}^{(b mod Ns) r} =
// W_n^{(b mod Ns) r scale} (from the LDS table twl, see mixed_tw; scale = n / (Ns R); all ones
// when Ns = 1), takes an R-point DFT and writes dst[(b / Ns) Ns R + b mod Ns + r Ns]. A thread
// takes butterflies tid + i NT in batches of IT whose LDS reads are all issued before the first
// is used (clamped to a valid butterfly; the extra ones are not written). b / Ns is
// umulhi(b, inv) with inv = ceil(2^32 / Ns), exact for b, Ns < 2^18.
template <int R, int IT, int NT>
__device__ __forceinline__ void mixed_pass(const float2* src, float2* dst, int M, int Ns, int scale,
                                           const float2* twl, int tid) {
    const int B = M / R;
    const unsigned inv = Ns > 1 ? 0xffffffffu / (unsigned)Ns + 1u : 0u;
    for (int b0 = tid; b0 < B; b0 += IT * NT) {
        float2 v[IT][R];
        int base[IT];
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int b = min(b0 + it * NT, B - 1);
            const int blk = Ns > 1 ? (int)__umulhi((unsigned)b, inv) : b, k = b - blk * Ns;
#pragma unroll
            for (int r = 0; r < R; r++) v[it][r] = src[mixed_pad(b + r * B)];
            if (Ns > 1) {
#pragma unroll
                for (int r = 1; r < R; r++) v[it][r] = cmul(v[it][r], mixed_tw(twl, k * r * scale));
            }
            base[it] = blk * Ns * R + k;
        }
#pragma unroll
        for (int it = 0; it < IT; it++) {
            if (b0 + it * NT >= B) break;
            Dft<R>::run(v[it]);
#pragma unroll
            for (int r = 0; r < R; r++) dst[mixed_pad(base[it] + r * Ns)] = v[it][r];
        }
    }
}

// Butterflies per thread and batch for radix R: all of a pass of MAXM points at once, capped
// so that a batch holds at most 32 complex values.
template <int R, int MAXM, int NT>
constexpr int mixed_batch() {
    const int all = (MAXM / R + NT - 1) / NT;
    const int cap = 32 / R > 0 ? 32 / R : 1;
    return all < cap ? (all > 0 ? all : 1) : cap;
}

// All passes of plan p over the M-point transform (M <= MAXM) in buf0 (buf1: scratch; both
// padded, see mixed_pad) by NT threads; returns the buffer holding the result. Every thread of
// the workgroup must call it (it has barriers), after the LDS table twl (mixed_tw) of W_n^m, with
// n a multiple of M (tw_mul = n / M), has been published by a barrier.
template <int MAXM, int NT>
__device__ __forceinline__ float2* mixed_fft(float2* buf0, float2* buf1, int M, const MixedRadix& p, int tw_mul,
                                             const float2* twl, int tid) {
    float2* src = buf0;
    float2* dst = buf1;
    int Ns = 1;
    for (int i = 0; i < p.count; i++) {
        const int R = p.r[i];
        const int scale = (M / (Ns * R)) * tw_mul;
        switch (R) {
            case 16: mixed_pass<16, mixed_batch<16, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
            case 8: mixed_pass<8, mixed_batch<8, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
            case 4: mixed_pass<4, mixed_batch<4, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
            case 2: mixed_pass<2, mixed_batch<2, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
            case 15: mixed_pass<15, mixed_batch<15, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
            case 3: mixed_pass<3, mixed_batch<3, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
            default: mixed_pass<5, mixed_batch<5, MAXM, NT>(), NT>(src, dst, M, Ns, scale, twl, tid); break;
        }
        __syncthreads();
        float2* t = src;
        src = dst;
        dst = t;
        Ns *= R;
    }
    return src;
}

// mixed_pass with the whole pass known at compile time (M, Ns and the twiddle scale), all of a
// thread's butterflies in one batch. Every LDS access is then one padded base plus immediate
// offsets wherever the layout allows it: reads when M / R is a multiple of 16
// (pad(b + r B) = pad(b) + r (B + B / 16)), writes when Ns is (the same identity), or when
// Ns = 1 and R divides 16 (pad(b R + r) = pad(b R) + r, the run staying inside one 16-block).
// The runtime pass computes a padded index, a product and a quotient per element instead.
template <int R, int NT, int M, int Ns, int SCALE>
__device__ __forceinline__ void mixed_pass_ct(const float2* src, float2* dst, const float2* twl, int tid) {
    constexpr int B = M / R;
    constexpr int IT = (B + NT - 1) / NT;
    constexpr bool SRC_LIN = B % 16 == 0;
    constexpr bool DST_LIN = Ns % 16 == 0 || (Ns == 1 && 16 % R == 0);
    constexpr int SRC_STEP = B + B / 16, DST_STEP = Ns + Ns / 16;
    float2 v[IT][R];
    int base[IT];
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int b = min(tid + it * NT, B - 1);
        const int blk = b / Ns, k = b - blk * Ns;
        if constexpr (SRC_LIN) {
            const float2* sp = src + mixed_pad(b);
#pragma unroll
            for (int r = 0; r < R; r++) v[it][r] = sp[r * SRC_STEP];
        } else {
#pragma unroll
            for (int r = 0; r < R; r++) v[it][r] = src[mixed_pad(b + r * B)];
        }
        if constexpr (Ns > 1) {
            const int ks = k * SCALE;
#pragma unroll
            for (int r = 1; r < R; r++) v[it][r] = cmul(v[it][r], mixed_tw(twl, r * ks));
        }
        base[it] = blk * Ns * R + k;
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
        if (tid + it * NT >= B) break;
        Dft<R>::run(v[it]);
        if constexpr (DST_LIN) {
            float2* dp = dst + mixed_pad(base[it]);
#pragma unroll
            for (int r = 0; r < R; r++) dp[r * (Ns == 1 ? 1 : DST_STEP)] = v[it][r];
        } else {
#pragma unroll
            for (int r = 0; r < R; r++) dst[mixed_pad(base[it] + r * Ns)] = v[it][r];
        }
    }
}

// The passes of radices R, Rest... after sub-transforms of length Ns, ping-ponging between
// src and dst (barrier after each); returns the buffer holding the result.
template <int NT, int M, int TWMUL, int Ns, int R, int... Rest>
__device__ __forceinline__ float2* mixed_fft_ct(float2* src, float2* dst, const float2* twl, int tid) {
    mixed_pass_ct<R, NT, M, Ns, (M / (Ns * R)) * TWMUL>(src, dst, twl, tid);
    __syncthreads();
    if constexpr (sizeof...(Rest) == 0) return dst;
    else return mixed_fft_ct<NT, M, TWMUL, Ns * R, Rest...>(dst, src, twl, tid);
}

// A transform size whose plan (the radices mixed_plan gives) is compiled in: mixed_fft_ct over
// M points. The host checks that the plan object it built has the same radices.
template <int M_, int... Rs>
struct MixedCt {
    static constexpr int M = M_;
    static constexpr int count = sizeof...(Rs);
    static constexpr int radix[sizeof...(Rs)] = {Rs...};
    template <int NT, int TWMUL>
    static __device__ __forceinline__ float2* run(float2* b0, float2* b1, const float2* twl, int tid) {
        return mixed_fft_ct<NT, M, TWMUL, 1, Rs...>(b0, b1, twl, tid);
    }
};
// Kim_Vocal_2's n_fft 7680: the real transform's 3840-point half.
using MixedCt3840 = MixedCt<3840, 16, 16, 15>;

inline bool mixed_plan_is(const MixedRadix& p, const int* radix, int count) {
    if (p.count != count) return false;
    for (int i = 0; i < count; i++)
        if (p.r[i] != radix[i]) return false;
    return true;
}

}  // namespace stx
