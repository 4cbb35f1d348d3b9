// fft_core.hpp — the complex FFT building blocks of every spectral kernel.
//
// One complex N-point transform (N a power of two, 16 <= N <= 8192) is computed by N/16
// threads with a self-sorting Stockham formulation: the first radix-16 pass runs straight on
// registers loaded from global memory, the remaining passes (radix 16, then one radix 2/4/8
// pass when log2 N is not a multiple of 4) exchange through LDS. Input and output are in
// natural order, so no bit reversal is needed (the reference's radix-2 DIT does one,
// src/stft.h:36). Twiddles come from a table of W_N^m = exp(-2*pi*i*m/N) computed once in
// double precision and rounded to float, never from recurrences.
//
// Pass with radix R after sub-transforms of length Ns: butterfly jj in [0, N/R) reads
// a[jj + r*N/R] (r < R), multiplies element r by W_{Ns*R}^{(jj mod Ns)*r}, takes an R-point
// DFT and writes element r to b[(jj / Ns)*Ns*R + (jj mod Ns) + r*Ns].
#pragma once

#include <hip/hip_runtime.h>

namespace stx {

#define STX_HD __host__ __device__ __forceinline__

STX_HD float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
STX_HD float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
STX_HD float2 cmul(float2 a, float2 b) {
    return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
STX_HD float2 cmul_mi(float2 a) { return make_float2(a.y, -a.x); }          // a * (-i)
STX_HD float2 cconj(float2 a) { return make_float2(a.x, -a.y); }

// Forward DFTs (kernel exp(-2*pi*i*n*k/R)) in natural order, in place on v[0..R).
template <int R> struct Dft;

template <> struct Dft<1> {
    static STX_HD void run(float2*) {}
};

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

// LDS index with one float2 of padding every 16: spreads the radix-16 scatter of the first
// pass (stride 16 float2 = 128 B) over all banks.
STX_HD int lds_idx(int i) { return i + (i >> 4); }

template <int N> struct FftShape {
    static_assert(N >= 16 && N <= 8192 && (N & (N - 1)) == 0, "N must be a power of two in [16, 8192]");
    static constexpr int TPJ = N / 16;               // threads per transform
    static constexpr int PADN = N + N / 16;          // LDS float2 per transform
};

// First pass (Ns = 1, radix 16): v holds a[j + r*N/16] for r < 16 on entry. Writes the
// result to LDS buffer `buf` (of one transform). No twiddles: jj mod 1 == 0.
template <int N>
__device__ __forceinline__ void fft_first_pass(float2* v, float2* buf, int j) {
    Dft<16>::run(v);
#pragma unroll
    for (int r = 0; r < 16; r++) buf[lds_idx(j * 16 + r)] = v[r];
}

// Remaining passes, in place in `buf`. Every thread of the workgroup must call this (it
// contains barriers), also threads whose transform is idle.
template <int N, int Ns>
__device__ __forceinline__ void fft_rest_passes(float2* buf, int j, const float2* __restrict__ tw) {
    if constexpr (Ns < N) {
        constexpr int R = (N / Ns >= 16) ? 16 : N / Ns;
        constexpr int TPJ = N / 16;
        constexpr int BPT = 16 / R;                  // butterflies per thread
        constexpr int TSTRIDE = N / (Ns * R);        // W_{Ns*R}^e = W_N^(e*TSTRIDE)
        float2 v[16];
#pragma unroll
        for (int q = 0; q < BPT; q++) {
            const int jj = j + q * TPJ;
#pragma unroll
            for (int r = 0; r < R; r++) v[q * R + r] = buf[lds_idx(jj + r * (N / R))];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < BPT; q++) {
            const int jj = j + q * TPJ;
            const int k = jj % Ns;
#pragma unroll
            for (int r = 1; r < R; r++) v[q * R + r] = cmul(v[q * R + r], tw[k * r * TSTRIDE]);
            Dft<R>::run(&v[q * R]);
            const int base = (jj / Ns) * Ns * R + k;
#pragma unroll
            for (int r = 0; r < R; r++) buf[lds_idx(base + r * Ns)] = v[q * R + r];
        }
        __syncthreads();
        fft_rest_passes<N, Ns * R>(buf, j, tw);
    }
}

}  // namespace stx
