// stft.hip — batched STFT / iSTFT for gfx950, behind the stft.h entry points of stx.h.
//
// Reference: src/stft.h (torch_stft :146-164, torch_istft :167-197, htdemucs_spec :79-103,
// htdemucs_ispec :106-140). The reference runs one double-precision radix-2 FFT per frame on
// the host. Here:
//   * every real frame of N samples is one complex N/2-point FFT of z[n] = x[2n] + i x[2n+1]
//     followed by the split X[k] = E[k] + W_N^k O[k] with E = (Z[k] + conj Z[N/2-k]) / 2,
//     O = (Z[k] - conj Z[N/2-k]) / 2i, which halves the arithmetic of a real transform and
//     makes one job per frame;
//   * the reflect padding of both modes (torch's center pad, and HTDemucs' extra pad before
//     it) is index arithmetic on the load, so the padded signal is never materialised;
//     frames that touch no padding skip it;
//   * the inverse transform is the forward one on conjugated data (ifft(X) = conj fft conj X),
//     after the inverse split Z' = (X[k] + conj X[N/2-k]) + i W_N^-k (X[k] - conj X[N/2-k]);
//   * the iSTFT overlap-add is in gather form, without atomics, in one of two ways:
//       - fused (no workspace): one workgroup owns a tile of output samples (several tiles in
//         turn when they outnumber the workgroups the device holds), inverse-transforms every
//         frame that overlaps it (frames shared by two tiles are transformed by both), sums the
//         windowed frames in frame order in registers and divides by the window-squared
//         envelope, evaluated in closed form per sample;
//       - two kernels (the mixed-radix sizes, with a workspace of C*T*N floats): one
//         inverse-transforms each frame once and writes it windowed to the workspace, the
//         next sums and divides. Power-of-two sizes run the fused kernel with or without a
//         workspace (measured faster at every size).
#include <algorithm>
#include <type_traits>
#include <memory>
#include <cmath>
#include <vector>

#include "common.hpp"
#include "fft_core.hpp"

struct stx_fft {
    int n = 0;
    int device = 0;
    float2* twt = nullptr;   // device: two-level twiddle table for n points (fft_core.hpp)
    float* win = nullptr;    // device [n]: periodic Hann
    float* win_hs = nullptr; // device [2][n]: the Hann window times 1/2 and times 1/(2 sqrt n) (power-of-two STFT)
    int mixed = 0;           // n = 2^a 3^b 5^c, not a power of two: the mixed-radix kernels
    float2* twn = nullptr;   // mixed: device [n], W_n^m
    float2* twm = nullptr;   // mixed: device [kMixedTwMax], the passes' two-level table (fft_core.hpp)
    stx::MixedRadix half;    // mixed: plan of the n/2-point transform of real frames
    stx::MixedRadix full;    // mixed: plan of the n-point complex transform
    // Powers of two without STFT kernels (stx_fft_run only): 2, 4, 8 are register transforms;
    // above 8192 the transform runs in four steps as n1 x n2 with the plans sub1, sub2 and a
    // scratch of n complex values.
    int run_only = 0;
    int n1 = 0, n2 = 0;
    stx_fft* sub1 = nullptr;
    stx_fft* sub2 = nullptr;
    float2* scratch = nullptr;
};

namespace stx {
namespace {

// floor(x / h) and ceil(x / h) for h > 0 and x of either sign.
__device__ __forceinline__ int floordiv(int x, int h) { return x >= 0 ? x / h : -((-x + h - 1) / h); }
__device__ __forceinline__ int ceildiv(int x, int h) { return -floordiv(-x, h); }

// --------------------------------------------------------------------------------- STFT
struct StftArgs {
    const float* x;          // [C][len]
    float2* spec;            // [C][F][T] or [C][T][F]
    const float* win;        // [N]
    const float* win_hs;     // [N]: win * scale / 2 (power-of-two kernel: the split's 1/2 and the norm)
    const float2* twt;       // twiddle table for N
    int len;                 // samples per channel
    int len1;                // length of the pre-padded signal (len when there is no pre-pad)
    int pre_left;            // left size of the pre-pad (HTDemucs' pad, 0 for torch)
    int hop;
    int frame0;              // padded index of frame 0's first sample
    int T;                   // frames per channel
    int F;                   // bins written per frame
    int jobs;                // channels * T
    int nblocks;             // real (logical) block count
    int layout;              // STX_SPEC_*
    float scale;             // normalisation
};

// torch reflect (edge not repeated): j < 0 -> -j; j >= n -> 2(n - 1) - j (src/stft.h:58-68).
__device__ __forceinline__ int reflect(int j, int n) {
    j = j < 0 ? -j : j;
    j = j >= n ? 2 * (n - 1) - j : j;
    return j;
}

// Signal index of sample m of the fully padded signal (center pad N/2 around the pre-padded
// one).
template <int N>
__device__ __forceinline__ int padded_index(int m, const StftArgs& a) {
    int j = reflect(m - N / 2, a.len1) - a.pre_left;
    j = reflect(j, a.len);
    return min(max(j, 0), a.len - 1);   // host validation keeps j in range; this only guards memory
}

// One workgroup transforms JOBS consecutive frames (one per N/2/P threads), then writes them so
// that neighbouring lanes store neighbouring addresses: consecutive frames of one bin row
// (F-major) or consecutive bins of one frame (T-major).
template <int N, int P, int JOBS>
__global__ __launch_bounds__(JOBS * (N / 2 / P)) void stft_kernel(StftArgs a) {
    constexpr int M = N / 2;
    using C = FftCfg<M, P, N>;
    constexpr int TPJ = C::TPJ;
    constexpr int NT = JOBS * TPJ;
    // Slots one float2 longer than the transform's buffer, so that the same element of
    // neighbouring slots (the lanes of one bin in the f-major stores) lies in different banks.
    constexpr int SLOT = C::PADN + 1;
    __shared__ float2 lds[JOBS * SLOT];
    __shared__ float2 twt[TwTable<N>::SIZE];

    const int lb = xcd_block();
    if (lb >= a.nblocks) return;                       // whole block idle: no barrier reached
    const int tid = (int)threadIdx.x;
    const int slot = tid / TPJ;
    const int j = tid % TPJ;
    const int f = lb * JOBS + slot;
    const bool active = f < a.jobs;
    float2* buf = lds + slot * SLOT;

    StagedTwiddles<N, NT> tws;
    tws.load(a.twt, tid);                              // overlaps the frame's loads
    const int c = active ? f / a.T : 0;
    const int t = active ? f - c * a.T : 0;
    const float* xc = a.x + (size_t)c * a.len;
    const int m0 = a.frame0 + t * a.hop;               // padded index of the first sample
    const int base = m0 - N / 2 - a.pre_left;          // its signal index when nothing reflects
    const bool interior = base >= 0 && base + N <= a.len;
    const float2* win2 = reinterpret_cast<const float2*>(a.win_hs);   // times scale / 2

    // Every load issued before the first wait (an inactive job reads frame 0 of channel 0,
    // always in range; its slot is transformed but never written). `interior` is uniform over
    // the job's threads, so only one of the two index paths runs.
    float2 v[P];
    if (interior) {
#pragma unroll
        for (int r = 0; r < P; r++) {
            const int n = j + r * TPJ;
            v[r] = make_float2(xc[base + 2 * n], xc[base + 2 * n + 1]);
        }
    } else {
        int ix[2 * P];
#pragma unroll
        for (int r = 0; r < P; r++) {
            const int n = j + r * TPJ;
            ix[2 * r] = padded_index<N>(m0 + 2 * n, a);
            ix[2 * r + 1] = padded_index<N>(m0 + 2 * n + 1, a);
        }
#pragma unroll
        for (int r = 0; r < P; r++) v[r] = make_float2(xc[ix[2 * r]], xc[ix[2 * r + 1]]);
    }
    float2 w[P];
#pragma unroll
    for (int r = 0; r < P; r++) w[r] = win2[j + r * TPJ];
#pragma unroll
    for (int r = 0; r < P; r++) v[r] = make_float2(v[r].x * w[r].x, v[r].y * w[r].y);
    tws.store(twt, tid);
    fft_first_pass<M, P, N>(v, buf, j, NoPost{}, ToLds<P>{buf});
    __syncthreads();
    fft_rest_passes<M, P, N, P>(buf, j, twt, NoPost{}, ToLds<P>{buf});

    // X[k] = E[k] + W_N^k O[k] for frame g of the block, k <= N/2 (the frame was windowed with
    // win * scale / 2, which folds the split's 1/2 and the norm in). Bins k = k0 + i*KS are read
    // at idx(k) = idx(k0) + i*(KS + KS/P), their mirrors M - k at idx(M - k0) - i*(KS + KS/P);
    // k = 0 and k = M pair with element 0 (k & (M - 1)). KS = TPJ in both layouts, so
    // W_N^k = W_N^k0 * exp(-i pi i / P): one table lookup per thread, then compile-time roots.
    const int f0 = lb * JOBS;
    const int c0 = f0 / a.T, t0 = f0 - c0 * a.T;
    constexpr int MP = M + M / P;
    // ik, im: idx(k) and idx(M - k) kept incrementally when the bin stride KS is a multiple of
    // P (every size from 32 up), computed directly otherwise.
    auto bin = [&](const float2* bs, int k, int ik, int im, float2 w, auto ks) {
        const bool inc = decltype(ks)::value % P == 0;
        const float2 zk = bs[inc ? (k < M ? ik : ik - MP) : C::idx(k & (M - 1))];
        const float2 zm = bs[(k & (M - 1)) == 0 ? 0 : inc ? im : C::idx(M - k)];
        const float er = zk.x + zm.x, ei = zk.y - zm.y;       // 2E
        const float orr = zk.y + zm.y, oi = zm.x - zk.x;      // 2O
        return make_float2(er + w.x * orr - w.y * oi, ei + w.x * oi + w.y * orr);
    };
    constexpr HalfTurnRoots<P> rot = half_turn_roots<P>();
    auto rotate = [&](float2 w0, int i) { return i == 0 ? w0 : cmul(w0, make_float2(rot.re[i], rot.im[i])); };
    if (a.layout == STX_SPEC_F_MAJOR) {
        // Element e = k*JOBS + g: with NT a multiple of JOBS every thread keeps one frame
        // g = tid % JOBS and takes bins tid / JOBS + i * NT / JOBS, so that the JOBS lanes of a
        // bin write consecutive frames of its row.
        constexpr int KS = NT / JOBS, KSP = KS + KS / P;
        static_assert(KS == TPJ, "bin stride");
        const int g = tid % JOBS, k0 = tid / JOBS;
        int tt = t0 + g, cc = c0;
        while (tt >= a.T) { tt -= a.T; cc++; }
        if (f0 + g < a.jobs) {
            const float2* bs = lds + g * SLOT;
            float2* col = a.spec + (size_t)cc * a.F * a.T + tt;
            const unsigned rs = (unsigned)a.T * KS;           // row step of one bin stride
            unsigned off = (unsigned)k0 * a.T;
            int ik = C::idx(k0), im = C::idx(M - k0);
            const float2 w0 = tw_lookup<N>(twt, k0);
#pragma unroll
            for (int i = 0; i <= P; i++, off += rs, ik += KSP, im -= KSP) {   // k0 + P*KS > M
                const int k = k0 + i * KS;
                // A plain store: the rows' short runs from neighbouring workgroups meet in the
                // XCD's L2 and leave as whole lines (with the non-temporal bit, c1 13.2 -> 18.2 us
                // and c3 13.2 -> 31.1 us).
                if (k < a.F) col[off] = bin(bs, k, ik, im, rotate(w0, i), std::integral_constant<int, KS>{});
            }
        }
    } else {
        // Row of frame g, then each bin's twiddle once for all JOBS frames.
        constexpr int KSP = NT + NT / P;
        float2* rows[JOBS];
#pragma unroll
        for (int g = 0; g < JOBS; g++) {
            int tt = t0 + g, cc = c0;
            while (tt >= a.T) { tt -= a.T; cc++; }
            rows[g] = f0 + g < a.jobs ? a.spec + ((size_t)cc * a.T + tt) * a.F : nullptr;
        }
        // Bin stride NT = JOBS * TPJ: W_N^(i*NT) = exp(-i pi i JOBS / P).
        static_assert(P % JOBS == 0, "t-major bin stride");
        int ik = C::idx(tid), im = C::idx(M - tid);
        const float2 w0 = tw_lookup<N>(twt, tid);
#pragma unroll
        for (int i = 0; i <= P / JOBS; i++, ik += KSP, im -= KSP) {   // tid + (P / JOBS) * NT >= M
            const int k = tid + i * NT;
            if (k >= a.F) continue;
            const float2 w = rotate(w0, i * JOBS);
#pragma unroll
            for (int g = 0; g < JOBS; g++)
                if (rows[g]) store_stream(rows[g] + k, bin(lds + g * SLOT, k, ik, im, w, std::integral_constant<int, NT>{}));
        }
    }
}

// -------------------------------------------------------------------------------- iSTFT
struct IstftArgs {
    const float2* spec;
    float* out;              // [C][out_len]
    const float* win;
    const float2* twt;
    float* frames;           // two-kernel path: [C][T][N] windowed frames
    int T;                   // spectrum frames
    int F;                   // bins per frame in spec
    int layout;
    int hop;
    int env_frames;          // frames that add win^2 to the envelope
    int frame_off;           // spectrum frame = envelope frame - frame_off
    int out_off;             // full-signal index of out[0]
    int out_len;             // samples per channel
    int valid_end;           // out[i] = 0 where out_off + i >= valid_end
    int keep_nyquist;        // 1: Nyquist real part used (torch); 0: Nyquist zeroed (HTDemucs)
    int tile_origin;         // fused: full-signal index where tile 0 starts
    int tile_len;            // fused: full-signal samples per tile
    int tiles;               // fused: tiles per channel
    int jobs;                // two-kernel: channels * T
    int nblocks;             // fused: tiles over all channels
    int grid;                // fused: workgroups launched (a multiple of the XCD count)
    float norm;
};

__device__ __forceinline__ float2 spec_bin(const IstftArgs& a, const float2* __restrict__ sc, int st, int k) {
    return a.layout == STX_SPEC_F_MAJOR ? sc[(size_t)k * a.T + st] : sc[(size_t)st * a.F + k];
}

// conj Z'[k] for k < N/2 from X[k] and X[N/2 - k] of one frame: the inverse split, with the
// DC and Nyquist imaginary parts ignored (src/stft.h:121,177,182) and the Nyquist bin zeroed
// for HTDemucs (:126).
__device__ __forceinline__ float2 inverse_split_w(float2 xk, float2 xm, int k, int keep_nyquist, float2 w) {
    if (k == 0) {
        xk = make_float2(xk.x, 0.f);
        xm = keep_nyquist ? make_float2(xm.x, 0.f) : make_float2(0.f, 0.f);
    }
    const float er = xk.x + xm.x, ei = xk.y - xm.y;          // X[k] + conj X[M-k]
    const float dr = xk.x - xm.x, di = xk.y + xm.y;          // X[k] - conj X[M-k]
    const float orr = dr * w.x + di * w.y, oi = di * w.x - dr * w.y;   // times conj(W_N^k)
    return make_float2(er - oi, -(ei + orr));                // conj(E' + i O')
}

template <int N>
__device__ __forceinline__ float2 inverse_split(float2 xk, float2 xm, int k, int keep_nyquist,
                                                const float2* __restrict__ twt) {
    return inverse_split_w(xk, xm, k, keep_nyquist, tw_lookup<N>(twt, k));
}

// Windowed output of the inverse transform: z[n] = conj(fft(conj Z'))[n] holds samples
// 2n (real) and 2n + 1 (imaginary); returns them times win * norm.
struct WindowPost {
    const float2* win2;
    float norm;
    __device__ __forceinline__ float2 operator()(int n, float2 r) const {
        const float2 w = win2[n];
        return make_float2(r.x * w.x * norm, -r.y * w.y * norm);
    }
};

// The same without the norm, which the fused kernel applies with the envelope's reciprocal.
struct WindowMul {
    const float2* win2;
    __device__ __forceinline__ float2 operator()(int n, float2 r) const {
        const float2 w = win2[n];
        return make_float2(r.x * w.x, -r.y * w.y);
    }
};

// Two-kernel path (mixed-radix sizes), step 2: out = sum of the windowed frames over the frames covering each
// sample, in frame order, divided by the window-squared envelope.
__global__ __launch_bounds__(256) void istft_ola_kernel(IstftArgs a, int N) {
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    const int c = (int)blockIdx.y;
    if (i >= a.out_len) return;
    const int J = a.out_off + i;
    float y = 0.f;
    if (J < a.valid_end) {
        const int hop = a.hop;
        const int lo = max(0, ceildiv(J - N + 1, hop));
        const int hi = min(a.env_frames - 1, J / hop);
        const float* fc = a.frames + (size_t)c * a.T * N;
        float env = 0.f, sum = 0.f;
        // Up to 8 covering frames per step, every load issued before the first sum (the frame
        // count varies, so a plain loop would wait for each load in turn); the sums stay in
        // frame order and skip what the loop skipped.
        for (int tf0 = lo; tf0 <= hi; tf0 += 8) {
            float wv[8], xv[8];
            bool in[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int tf = tf0 + u, st = tf - a.frame_off;
                const bool ok = tf <= hi;
                const int s = ok ? J - tf * hop : 0;
                in[u] = ok && st >= 0 && st < a.T;
                wv[u] = ok ? a.win[s] : 0.f;
                xv[u] = in[u] ? fc[(size_t)st * N + s] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (tf0 + u <= hi) env += wv[u] * wv[u];
                if (in[u]) sum += xv[u];
            }
        }
        y = env > 1e-11f ? sum / env : 0.f;
    }
    store_stream(a.out + (size_t)c * a.out_len + i, y);
}

// Fused path: one workgroup owns a tile of output samples and inverse-transforms, JOBS frames
// at a time (normally all at once), every frame that overlaps it; the last FFT pass applies
// window * norm; each thread sums its samples over the overlapping frames in frame order and
// divides by the window-squared envelope. PERSIST: fewer workgroups than tiles, each taking
// several (launches whose tiles outnumber the workgroups the device holds at once).
template <int N, int P, int JOBS, int PER, bool PERSIST>
__global__ __launch_bounds__(JOBS * (N / 2 / P)) void istft_kernel(IstftArgs a) {
    constexpr int M = N / 2;
    using C = FftCfg<M, P, N>;
    constexpr int TPJ = C::TPJ;
    constexpr int NT = JOBS * TPJ;
    // Slots KPW float2 apart modulo 32 (256 bytes of banks): the f-major staging's lanes write
    // bin tr / JOBS of slot tr % JOBS, KPW = ceil(64 / JOBS) bins per wave, so the JOBS slots'
    // runs fall on different banks (with slots a multiple of 32 float2 apart they shared them:
    // 5x the LDS bank-conflict cycles of the t-major staging at c1).
    constexpr int KPW = (64 + JOBS - 1) / JOBS;                  // a wave is 64 lanes
    constexpr int SLOT = C::PADN < 512 ? C::PADN : C::PADN + ((KPW - C::PADN % 32) % 32 + 32) % 32;  // short slots: as is
    // One wave per transform: between the split and the last pass every lane touches only its
    // own wave's slot, so those passes need no workgroup barrier.
    constexpr bool WAVE = TPJ == 64;
    constexpr bool WIN_LDS = (size_t)JOBS * SLOT * 8 + TwTable<N>::SIZE * 8 + N * 4 <= 160 * 1024;
    // Reciprocal window-squared envelope per position R = J mod hop where every covering
    // frame exists (R < N suffices: positions past N have no frame).
    constexpr bool ENV_LDS = WIN_LDS && (size_t)JOBS * SLOT * 8 + TwTable<N>::SIZE * 8 + N * 8 <= 160 * 1024;
    __shared__ float2 lds[JOBS * SLOT];
    __shared__ float2 twt[TwTable<N>::SIZE];
    __shared__ float wl[WIN_LDS ? N : 2];
    __shared__ float inv_env[ENV_LDS ? N : 2];

    // Workgroup lb takes tile lb of the a.nblocks tiles over all channels, and with PERSIST also
    // tiles lb + G, lb + 2G, ... (G = a.grid, the workgroups launched); at every step each XCD
    // holds a contiguous run of tiles.
    const int lb = xcd_block();
    if (lb >= a.nblocks) return;
    const int tid = (int)threadIdx.x;
    const int slot = tid / TPJ;
    const int j = tid % TPJ;
    float2* buf = lds + slot * SLOT;
    const int hop = a.hop;

    // The twiddle and window tables are loaded into registers here and written to LDS after the
    // first tile's spectrum loads are issued, so that their round trips overlap.
    StagedTwiddles<N, NT> tws;
    Staged<WIN_LDS ? N : 1, NT, float> wins;
    tws.load(a.twt, tid);
    if constexpr (WIN_LDS) wins.load(a.win, tid);
    const float* win = WIN_LDS ? wl : a.win;
    const WindowMul post{reinterpret_cast<const float2*>(win)};

    struct Tile {
        int c, J0, J1, st_lo, st_hi;
        const float2* sc;
    };
    auto tile_at = [&](int ti) {
        Tile t;
        t.c = ti / a.tiles;
        const int tile = ti - t.c * a.tiles;
        t.J0 = max(a.out_off, a.tile_origin + tile * a.tile_len);
        t.J1 = min(a.out_off + a.out_len, a.tile_origin + (tile + 1) * a.tile_len);
        // Spectrum frames overlapping [J0, J1): envelope frame tf covers [tf*hop, tf*hop + N).
        t.st_lo = max(0, max(0, ceildiv(t.J0 - N + 1, hop)) - a.frame_off);
        t.st_hi = min(a.T - 1, floordiv(t.J1 - 1, hop) - a.frame_off);
        t.sc = a.spec + (size_t)t.c * a.T * a.F;
        return t;
    };
    // X[0..M] of frames s0 .. s0 + JOBS - 1 into registers, neighbouring lanes on neighbouring
    // addresses in either layout: bins k < M are P per thread (M * JOBS = P * NT), the Nyquist
    // bins one per slot; frames past st_hi read frame st_hi again (finite values, transformed
    // but never summed: the walk stops at st_hi). F-major: element e = tr + i*NT is slot
    // e % JOBS = tr % JOBS, bin tr / JOBS + i*TPJ. T-major: thread jr of a slot takes bins
    // jr + i*TPJ of the slot's frame, the FFT's own element order (one row address, then
    // constant offsets), and the Nyquist bin.
    auto load_frames = [&](const Tile& t, int s0, int tr, int jr, float2 (&sv)[P], float2& nyq) {
        if (a.layout == STX_SPEC_F_MAJOR) {
            const float2* col = t.sc + min(s0 + tr % JOBS, t.st_hi);
#pragma unroll
            for (int i = 0; i < P; i++) sv[i] = col[(size_t)(tr / JOBS + i * TPJ) * a.T];
            nyq = t.sc[(size_t)min(M, a.F - 1) * a.T + min(s0 + min(tr, JOBS - 1), t.st_hi)];
        } else {
            const float2* row = t.sc + (size_t)min(s0 + tr / TPJ, t.st_hi) * a.F;
#pragma unroll
            for (int i = 0; i < P; i++) sv[i] = row[jr + i * TPJ];
            nyq = row[min(M, a.F - 1)];
        }
    };
    auto stage_frames = [&](int tr, int jr, const float2 (&sv)[P], float2 nyq) {
        if (a.layout == STX_SPEC_F_MAJOR) {
            const int g = tr % JOBS, k0 = tr / JOBS;
#pragma unroll
            for (int i = 0; i < P; i++) lds[g * SLOT + k0 + i * TPJ] = sv[i];
            if (tr < JOBS) lds[tr * SLOT + M] = M < a.F ? nyq : make_float2(0.f, 0.f);
        } else {
            float2* bs = lds + (tr / TPJ) * SLOT;
#pragma unroll
            for (int i = 0; i < P; i++) bs[jr + i * TPJ] = sv[i];
            if (jr == 0) bs[M] = M < a.F ? nyq : make_float2(0.f, 0.f);
        }
    };

    bool staged = false;
    auto stage_tables = [&]() {
        tws.store(twt, tid);
        if constexpr (WIN_LDS) wins.store(wl, tid);
        staged = true;
    };
    Tile t = tile_at(lb);
    float2 sv[P], nyq = make_float2(0.f, 0.f);
    if constexpr (PERSIST) {
        if (t.st_lo <= t.st_hi) load_frames(t, t.st_lo, tid, j, sv, nyq);
        stage_tables();
    }

    // Samples J = J0 + q*NT + tid (q < PER). With J = A*hop + R (0 <= R < hop), the frames
    // covering J are tf = A - K .. A at positions s = R + K*hop .. R, where K = K0 when
    // R <= rK and K0 - 1 otherwise (K0 = (N-1)/hop, rK = N-1 - K0*hop). One division per
    // walk; A and R then advance by NT = dA*hop + dR per q. The walk is redone after each
    // round's transform rather than held in registers across it.
    const int K0 = (N - 1) / hop, rK = N - 1 - K0 * hop;
    const int dA = NT / hop, dR = NT - dA * hop;
    auto walk = [&](int J0, int lane, auto&& body) {
        int A = (J0 + lane) / hop, R = J0 + lane - A * hop;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int K = R <= rK ? K0 : K0 - 1;
            body(q, A - K, R + K * hop, K);    // first covering envelope frame, its position, K
            R += dR;
            A += dA;
            if (R >= hop) { R -= hop; A++; }
        }
    };

    // Envelope: win^2 summed over the envelope frames 0 <= tf < env_frames covering J, in frame
    // order (src/stft.h:130,187); out = acc * (norm / env) where env > 1e-11, else 0 (the sums
    // hold frames times the window only: the transform's norm is applied here, once per
    // sample). Where all K + 1 frames of J exist, env depends on R = J mod hop only: norm / env
    // (0 for env <= 1e-11) comes from a table built once per workgroup when the LDS has room;
    // elsewhere (and at the signal's ends) the same sum and quotient run here, so the table
    // changes no bit. Barriers here and below wait for LDS traffic only (lds_barrier), so the
    // spectrum loads issued before them stay in flight.
    auto build_env = [&]() {
        const int nr = min(hop, N);
        for (int R = tid; R < nr; R += NT) {
            const int K = R <= rK ? K0 : K0 - 1;
            float env = 0.f;
            for (int i = K; i >= 0; i--) {               // frame order: position R + K*hop first
                const float w = win[R + i * hop];
                env += w * w;
            }
            inv_env[R] = env > 1e-11f ? a.norm / env : 0.f;
        }
    };
    if constexpr (ENV_LDS && PERSIST) {
        lds_barrier();                                // the window table written
        build_env();                                  // read after the first tile's rounds
    }
    const float* ldsf = reinterpret_cast<const float*>(lds);

    for (int ti = lb;; ti += a.grid) {
        const int tn = ti + a.grid;                     // this workgroup's next tile
        float acc[PER];
#pragma unroll
        for (int q = 0; q < PER; q++) acc[q] = 0.f;
        for (int s0 = t.st_lo; s0 <= t.st_hi; s0 += JOBS) {
            // An opaque copy of the lane index: keeps the compiler from hoisting the (round
            // invariant) twiddle reads, staging addresses and sample walk out of this loop,
            // which would hold them in registers across the transform.
            int jr = j, tr = tid;
            asm volatile("" : "+v"(jr), "+v"(tr));
            __builtin_assume(jr >= 0 && jr < TPJ && tr >= 0 && tr < NT);
            if constexpr (PERSIST) {
                stage_frames(tr, jr, sv, nyq);
                // The next round's loads (or the next tile's first), in flight through this round.
                if (s0 + JOBS <= t.st_hi) {
                    load_frames(t, s0 + JOBS, tr, jr, sv, nyq);
                } else if (tn < a.nblocks) {
                    const Tile u = tile_at(tn);
                    if (u.st_lo <= u.st_hi) load_frames(u, u.st_lo, tr, jr, sv, nyq);
                }
            } else {
                // One tile: each round's frames are loaded at its start, so that no registers are
                // held across the transform; the tables go to LDS while the first round's loads
                // are in flight.
                load_frames(t, s0, tr, jr, sv, nyq);
                if (!staged) stage_tables();
                stage_frames(tr, jr, sv, nyq);
            }
            lds_barrier();
            // Split twiddles W_N^k for k = jr + r*TPJ: W_N^jr from the table times the
            // constant W_N^(r*TPJ) = exp(-i pi r / P).
            constexpr HalfTurnRoots<P> rot = half_turn_roots<P>();
            const float2 w0 = tw_lookup<N>(twt, jr);
            float2 v[P];
#pragma unroll
            for (int r = 0; r < P; r++) {
                const int k = jr + r * TPJ;
                const float2 wr = r == 0 ? w0 : cmul(w0, make_float2(rot.re[r], rot.im[r]));
                v[r] = inverse_split_w(buf[k], buf[M - k], k, a.keep_nyquist, wr);
            }
            pass_sync<WAVE>();                          // staging read before the FFT overwrites it
            fft_first_pass<M, P, N>(v, buf, jr, post, ToLdsFlat{buf});
            pass_sync<WAVE>();
            fft_rest_passes<M, P, N, P, WAVE>(buf, jr, twt, post, ToLdsFlat{buf});
            if constexpr (WAVE) lds_barrier();          // every slot written before the sums read them
            // Slot g now holds samples (2n, 2n + 1) of frame s0 + g at LDS index n (unpadded:
            // the last pass's lanes write consecutive n), windowed: add the frames of this
            // round that cover each sample, in frame order.
            const int s_end = min(t.st_hi, s0 + JOBS - 1);
            walk(t.J0, tr, [&](int q, int tf0, int s_first, int K) {
                if (q * NT + tr >= t.J1 - t.J0) return;
                const int first = tf0 - a.frame_off;              // spectrum frame of tf0
                const int i0 = max(0, s0 - first), i1 = min(K, s_end - first);
                // Sample pos (0 <= pos < N) of slot g is float pos of the slot.
                const float* sl = ldsf + 2 * SLOT * (first + i0 - s0) + (s_first - i0 * hop);
                float sum = acc[q];
                for (int i = i0; i <= i1; i++, sl += 2 * SLOT - hop) sum += *sl;
                acc[q] = sum;
            });
            lds_barrier();
        }
        if constexpr (PERSIST) {
            if (t.st_lo > t.st_hi) lds_barrier();      // no frame overlaps the tile (uniform): tables
        } else {
            if (!staged) {                             // no frame overlaps the tile (uniform)
                stage_tables();
                lds_barrier();
            }
            if constexpr (ENV_LDS) {
                build_env();
                lds_barrier();
            }
        }
        float* oc = a.out + (size_t)t.c * a.out_len;
        walk(t.J0, tid, [&](int q, int tf0, int s_first, int K) {
            const int J = t.J0 + q * NT + tid;
            if (J >= t.J1) return;
            float y = 0.f;
            if (ENV_LDS && J < a.valid_end && tf0 >= 0 && tf0 + K < a.env_frames) {
                const float r = inv_env[s_first - K * hop];
                y = r > 0.f ? acc[q] * r : 0.f;
            } else if (J < a.valid_end) {
                const int i0 = max(0, -tf0), i1 = min(K, a.env_frames - 1 - tf0);
                unsigned pos = (unsigned)(s_first - i0 * hop);
                float env = 0.f;
                for (int i = i0; i <= i1; i++, pos -= (unsigned)hop) {
                    const float w = win[pos];
                    env += w * w;
                }
                y = env > 1e-11f ? acc[q] * (a.norm / env) : 0.f;   // as the table's product
            }
            store_stream(oc + (J - a.out_off), y);
        });
        if (!PERSIST || tn >= a.nblocks) break;
        t = tile_at(tn);
    }
}

// ------------------------------------------------------------------ mixed-radix sizes
// n = 2^a 3^b 5^c that is not a power of two (VRFFT's sizes: Kim_Vocal_2's 7680, VR's 320, 640,
// 960; src/vr_dsp.h:11-37, src/tfc_tdf.cpp:85-86,551-552). The reference reaches these sizes with
// Bluestein (three power-of-two transforms of at least 2n - 1 points); here one workgroup runs
// the n/2-point transform of a real frame directly, radix 16 / 8 / 4 / 2 / 15 / 3 / 5 Stockham passes
// ping-ponging between two LDS buffers with twiddles W_n^m from a table computed in double.
// Frames are packed and split as in the power-of-two kernels; the iSTFT always takes the
// two-kernel path (frames to the workspace, then istft_ola_kernel). One frame per workgroup,
// numbered XCD-aware (xcd_block): consecutive frames run on one XCD, so the F-major spectrum's
// rows, where each frame owns 8 bytes of a 128-byte line, are written (or read) through one L2
// that merges the 16 frames of a line, instead of as partial lines from eight XCDs.
constexpr int kMixedThreads = 512;

__device__ __forceinline__ int padded_index_rt(int m, const StftArgs& a, int n) {
    int j = reflect(m - n / 2, a.len1) - a.pre_left;
    j = reflect(j, a.len);
    return min(max(j, 0), a.len - 1);
}

// CT: a size whose plan is compiled in (MixedCt: constant trip counts, LDS offsets as
// immediates), or void for the plan p at run time.
template <class CT> struct MixedM { static constexpr int value = CT::M; };
template <> struct MixedM<void> { static constexpr int value = 0; };

// FPB frames per block, as in istft_frames_mixed_kernel: with FPB = 2 (f-major, T even, 16-byte
// aligned spectrum) the two frames t and t + 1 of one channel are transformed by the two halves
// of the block, and every bin row gets both frames' values as one 16-byte store.
template <int MAXM, class CT, int FPB>
__global__ __launch_bounds__(kMixedThreads * FPB) void stft_mixed_kernel(StftArgs a, MixedRadix p,
                                                                         const float2* __restrict__ twn,
                                                                         const float2* __restrict__ twm, int n_rt) {
    __shared__ float2 b0s[FPB][mixed_padded(MAXM)], b1s[FPB][mixed_padded(MAXM)];
    __shared__ float2 twl[kMixedTwMax];
    constexpr int NT = kMixedThreads;
    constexpr int CTM = MixedM<CT>::value;
    const int n = CTM ? 2 * CTM : n_rt;
    const int M = n / 2, tall = (int)threadIdx.x, half = tall / NT, tid = tall - half * NT;
    const int f0 = xcd_block() * FPB;                  // first frame (channel * T + frame) of the block
    if (f0 >= a.jobs) return;                          // whole block idle: no barrier reached
    const int f = f0 + half;
    float2* b0 = b0s[half];
    float2* b1 = b1s[half];
    Staged<kMixedTwMax, NT * FPB, float2> tws;
    tws.load(twm, tall);
    const int c = f / a.T, t = f - c * a.T;
    const float* xc = a.x + (size_t)c * a.len;
    const int m0 = a.frame0 + t * a.hop;
    for (int i = tid; i < M; i += NT) {
        const float x0 = xc[padded_index_rt(m0 + 2 * i, a, n)], x1 = xc[padded_index_rt(m0 + 2 * i + 1, a, n)];
        b0[mixed_pad(i)] = make_float2(x0 * a.win[2 * i], x1 * a.win[2 * i + 1]);
    }
    tws.store(twl, tall);
    __syncthreads();
    const float2* z;
    if constexpr (CTM != 0) z = CT::template run<NT, 2>(b0, b1, twl, tid);
    else z = mixed_fft<MAXM, NT>(b0, b1, M, p, 2, twl, tid);
    // X[k] = E[k] + W_n^k O[k], k <= n/2, as in stft_kernel.
    const float hs = 0.5f * a.scale;
    auto bin = [&](const float2* zz, int k, float2 w) {
        const float2 zk = zz[mixed_pad(k == M ? 0 : k)], zm = zz[mixed_pad(k == 0 ? 0 : M - k)];
        const float er = zk.x + zm.x, ei = zk.y - zm.y;
        const float orr = zk.y + zm.y, oi = zm.x - zk.x;
        return make_float2((er + w.x * orr - w.y * oi) * hs, (ei + w.x * oi + w.y * orr) * hs);
    };
    if constexpr (FPB == 2) {
        // Both halves ran the same passes, so both results are in the same buffer of their half;
        // the last pass ended with a barrier.
        const bool in0 = z == b0;
        const float2* z0 = in0 ? b0s[0] : b1s[0];
        const float2* z1 = in0 ? b0s[1] : b1s[1];
        const int t0 = t - half;                       // even
        for (int k = tall; k < a.F; k += 2 * NT) {
            const float2 w = twn[k];
            const float2 v0 = bin(z0, k, w), v1 = bin(z1, k, w);
            *reinterpret_cast<float4*>(a.spec + ((size_t)c * a.F + k) * a.T + t0) = make_float4(v0.x, v0.y, v1.x, v1.y);
        }
    } else {
        for (int k = tid; k < a.F; k += NT) {
            const float2 val = bin(z, k, twn[k]);
            if (a.layout == STX_SPEC_F_MAJOR) a.spec[((size_t)c * a.F + k) * a.T + t] = val;
            else store_stream(a.spec + ((size_t)c * a.T + t) * a.F + k, val);
        }
    }
}

// FPB frames per block. FPB = 2 (f-major, T even, 16-byte aligned spectrum): the block's frames
// are st and st + 1 of one channel, adjacent in every bin row, so each bin of both arrives in one
// 16-byte load, half the L2 requests of one frame per block; each half of the block (512 threads)
// then runs its frame's inverse split, transform and windowed store in its own buffers.
template <int MAXM, class CT, int FPB>
__global__ __launch_bounds__(kMixedThreads * FPB) void istft_frames_mixed_kernel(IstftArgs a, MixedRadix p,
                                                                                 const float2* __restrict__ twn,
                                                                                 const float2* __restrict__ twm,
                                                                                 int n_rt, int jobs) {
    __shared__ float2 b0s[FPB][mixed_padded(MAXM)], b1s[FPB][mixed_padded(MAXM)];
    __shared__ float2 twl[kMixedTwMax];
    constexpr int NT = kMixedThreads;
    constexpr int CTM = MixedM<CT>::value;
    const int n = CTM ? 2 * CTM : n_rt;
    const int M = n / 2, tall = (int)threadIdx.x, half = tall / NT, tid = tall - half * NT;
    const int f0 = xcd_block() * FPB;                  // first frame (channel * T + frame) of the block
    if (f0 >= jobs) return;                            // whole block idle: no barrier reached
    const int f = f0 + half;
    float2* b0 = b0s[half];
    float2* b1 = b1s[half];
    Staged<kMixedTwMax, NT * FPB, float2> tws;
    tws.load(twm, tall);
    const int c = f / a.T, st = f - c * a.T;
    const float2* sc = a.spec + (size_t)c * a.T * a.F;
    // Bins 0..M, each loaded once (clamped to valid bins) and staged in b1, and the twiddles, all
    // issued before the first LDS write; the inverse split then takes X[k] and X[M - k] from
    // LDS. In the f-major layout each bin is its own request to the L2, so loading X[k] and
    // X[M - k] from memory, as two loads per bin, doubled the requests the kernel waits on.
    constexpr int RL = (MAXM + NT - 1) / NT;
    float2 tw[RL];
    if constexpr (FPB == 2) {
        constexpr int RB = (MAXM + 1 + 2 * NT - 1) / (2 * NT);
        const float2* sp = sc + st - half;             // frame st of half 0 (even)
        float4 xb[RB];
#pragma unroll
        for (int q = 0; q < RB; q++) {
            const int k = min(min(tall + q * 2 * NT, M), a.F - 1);
            xb[q] = *reinterpret_cast<const float4*>(sp + (size_t)k * a.T);
        }
#pragma unroll
        for (int q = 0; q < RL; q++) tw[q] = twn[min(tid + q * NT, M - 1)];
#pragma unroll
        for (int q = 0; q < RB; q++) {
            const int k = tall + q * 2 * NT;
            if (k > M) break;
            b1s[0][mixed_pad(k)] = make_float2(xb[q].x, xb[q].y);
            b1s[1][mixed_pad(k)] = make_float2(xb[q].z, xb[q].w);
        }
    } else {
        constexpr int RB = (MAXM + 1 + NT - 1) / NT;
        float2 xb[RB];
#pragma unroll
        for (int q = 0; q < RB; q++) xb[q] = spec_bin(a, sc, st, min(min(tid + q * NT, M), a.F - 1));
#pragma unroll
        for (int q = 0; q < RL; q++) tw[q] = twn[min(tid + q * NT, M - 1)];
#pragma unroll
        for (int q = 0; q < RB; q++) {
            const int k = tid + q * NT;
            if (k > M) break;
            b1[mixed_pad(k)] = xb[q];
        }
    }
    tws.store(twl, tall);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RL; q++) {
        const int k = tid + q * NT;
        if (k >= M) break;
        const float2 m = k == 0 && !a.keep_nyquist ? make_float2(0.f, 0.f) : b1[mixed_pad(M - k)];
        b0[mixed_pad(k)] = inverse_split_w(b1[mixed_pad(k)], m, k, a.keep_nyquist, tw[q]);
    }
    __syncthreads();                                   // b1 read before the first pass writes it
    const float2* r;
    if constexpr (CTM != 0) r = CT::template run<NT, 2>(b0, b1, twl, tid);
    else r = mixed_fft<MAXM, NT>(b0, b1, M, p, 2, twl, tid);
    float* dst = a.frames + (size_t)f * n;
    const float2* win2 = reinterpret_cast<const float2*>(a.win);
    float2 wv[RL];
#pragma unroll
    for (int q = 0; q < RL; q++) wv[q] = win2[min(tid + q * NT, M - 1)];
    // Windowed as WindowPost, streamed out: the overlap-add kernel reads these frames across
    // XCDs, so they come back from memory whatever the store; with the non-temporal bit they
    // leave during the kernel instead of as dirty L2 lines at its end (Kim 7680 iSTFT
    // 25.3 -> 24.2 us). 8-byte stores where the workspace allows them (n is even).
    const bool pairs = (reinterpret_cast<uintptr_t>(a.frames) & 7) == 0;
#pragma unroll
    for (int q = 0; q < RL; q++) {
        const int i = tid + q * NT;
        if (i >= M) break;
        const float2 ri = r[mixed_pad(i)];
        const float2 o = make_float2(ri.x * wv[q].x * a.norm, -ri.y * wv[q].y * a.norm);
        if (pairs) {
            store_stream(reinterpret_cast<float2*>(dst + 2 * i), o);
        } else {
            store_stream(dst + 2 * i, o.x);
            store_stream(dst + 2 * i + 1, o.y);
        }
    }
}

template <int MAXM>
__global__ __launch_bounds__(kMixedThreads) void fft_mixed_kernel(float2* data, int inverse, MixedRadix p,
                                                                  const float2* __restrict__ twm, int n) {
    __shared__ float2 b0[mixed_padded(MAXM)], b1[mixed_padded(MAXM)];
    __shared__ float2 twl[kMixedTwMax];
    const int tid = (int)threadIdx.x;
    Staged<kMixedTwMax, kMixedThreads, float2> tws;
    tws.load(twm, tid);
    float2* d = data + (size_t)blockIdx.x * n;
    constexpr int RL = (MAXM + kMixedThreads - 1) / kMixedThreads;
    float2 v[RL];
#pragma unroll
    for (int q = 0; q < RL; q++) v[q] = d[min(tid + q * kMixedThreads, n - 1)];   // every load first
#pragma unroll
    for (int q = 0; q < RL; q++)
        if (tid + q * kMixedThreads < n) b0[mixed_pad(tid + q * kMixedThreads)] = inverse ? cconj(v[q]) : v[q];
    tws.store(twl, tid);
    __syncthreads();
    const float2* r = mixed_fft<MAXM, kMixedThreads>(b0, b1, n, p, 1, twl, tid);
    for (int i = tid; i < n; i += kMixedThreads) d[i] = inverse ? cconj(r[mixed_pad(i)]) : r[mixed_pad(i)];
}

__global__ __launch_bounds__(256) void zero_kernel(float* out, size_t count) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) out[i] = 0.f;
}

// ------------------------------------------------------------------------ plain FFT
template <int N, int P, int JOBS>
__global__ __launch_bounds__(JOBS * (N / P)) void fft_kernel(float2* data, int batch, int inverse,
                                                             const float2* __restrict__ gtw, int nblocks) {
    using C = FftCfg<N, P, N>;
    constexpr int TPJ = C::TPJ;
    __shared__ float2 lds[JOBS * C::PADN];
    __shared__ float2 twt[TwTable<N>::SIZE];
    const int lb = xcd_block();
    if (lb >= nblocks) return;
    const int tid = (int)threadIdx.x;
    const int slot = tid / TPJ;
    const int j = tid % TPJ;
    const int job = lb * JOBS + slot;
    const bool active = job < batch;
    float2* buf = lds + slot * C::PADN;
    float2* d = data + (size_t)(active ? job : 0) * N;
    StagedTwiddles<N, JOBS * TPJ> tws;
    tws.load(gtw, tid);
    float2 v[P];
#pragma unroll
    for (int r = 0; r < P; r++) {
        const float2 x = active ? d[j + r * TPJ] : make_float2(0.f, 0.f);
        v[r] = inverse ? cconj(x) : x;
    }
    tws.store(twt, tid);
    auto sink = [&](int k, float2 y) {
        if (active) d[k] = inverse ? cconj(y) : y;
    };
    fft_first_pass<N, P, N>(v, buf, j, NoPost{}, sink);
    __syncthreads();
    fft_rest_passes<N, P, N, P>(buf, j, twt, NoPost{}, sink);
}

// Transforms of N = 2, 4 or 8 points, one per thread, in registers (the inverse as conj, forward
// DFT, conj).
template <int N>
__global__ __launch_bounds__(256) void fft_small_kernel(float2* data, int batch, int inverse) {
    const int b = (int)(blockIdx.x * 256 + threadIdx.x);
    if (b >= batch) return;
    float2* d = data + (size_t)b * N;
    float2 v[N];
#pragma unroll
    for (int r = 0; r < N; r++) v[r] = inverse ? cconj(d[r]) : d[r];
    Dft<N>::run(v);
#pragma unroll
    for (int r = 0; r < N; r++) d[r] = inverse ? cconj(v[r]) : v[r];
}

// Four-step transforms (n = n1 n2 > 8192): dst[c][r] = src[r][c] for a rows x cols complex
// matrix, times W_n^(r c) (conjugated for the inverse) when `twiddle`, with W evaluated in
// double; 32 x 32 tiles through LDS (one float2 of padding per row).
__global__ __launch_bounds__(256) void transpose_c64_kernel(const float2* __restrict__ src, float2* __restrict__ dst,
                                                            int rows, int cols, int twiddle, int n, int inverse) {
    __shared__ float2 tile[32][33];
    const int c0 = (int)blockIdx.x * 32, r0 = (int)blockIdx.y * 32;
    const int tx = (int)threadIdx.x % 32, ty = (int)threadIdx.x / 32;
#pragma unroll
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) {
            float2 v = src[(size_t)r * cols + c];
            if (twiddle) {
                double sn, cs;
                sincospi(2.0 * (double)((long long)r * c % n) / (double)n, &sn, &cs);
                v = cmul(v, make_float2((float)cs, inverse ? (float)sn : (float)-sn));
            }
            tile[i][tx] = v;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) dst[(size_t)c * rows + r] = tile[tx][i];
    }
}

__global__ __launch_bounds__(256) void copy_c64_kernel(const float2* __restrict__ src, float2* __restrict__ dst,
                                                       long long count) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < count) dst[i] = src[i];
}

// ------------------------------------------------------------------------ dispatch
constexpr int block_jobs(int tpj, int threads) { return tpj >= threads ? 1 : threads / tpj; }
constexpr int kIstftPer = 6;                           // fused: output samples per thread per tile

// Points per thread: 8 keeps waves short for the small, latency-bound batches of one
// segment (16 measured slower for the STFT at n_fft 2048, faster from 4096); the fused iSTFT
// uses 16 so that one workgroup holds as many frames as possible.
constexpr int kStftP = 8;
constexpr int fused_p(int n) { return n / 2 >= 16 ? 16 : 8; }

// One frame per workgroup in the T-major layout (the most workgroups); two in the F-major
// layout, whose bins then leave as 16-byte runs of two frames per row instead of 8.
template <int N, int JOBS>
void launch_stft_jobs(StftArgs a, hipStream_t s) {
    constexpr int P = kStftP;
    constexpr int TPJ = N / 2 / P;
    a.nblocks = (a.jobs + JOBS - 1) / JOBS;
    hipLaunchKernelGGL((stft_kernel<N, P, JOBS>), dim3(xcd_grid(a.nblocks)), dim3(JOBS * TPJ), 0, s, a);
    launch_check("stft_kernel");
}

template <int N>
void launch_stft(const StftArgs& a, hipStream_t s) {
    constexpr int TPJ = N / 2 / kStftP;
    constexpr int J2 = TPJ * 2 <= 1024 ? 2 : 1;
    if (a.layout == STX_SPEC_T_MAJOR) launch_stft_jobs<N, 1>(a, s);
    else launch_stft_jobs<N, J2>(a, s);
}

// Tiles of m hops need m + ceil(N/hop) - 1 frames; m is chosen so that they fit one round of
// JOBS frames, within the PER*NT samples the threads accumulate. Returns the block count.
template <int N, int JOBS>
long long plan_istft_tiles(IstftArgs& a, int channels) {
    constexpr int NT = JOBS * (N / 2 / fused_p(N));
    const int span = (N + a.hop - 1) / a.hop;
    const long long m = std::max(1, JOBS - span + 1);
    const long long tile_len = std::min<long long>(m * a.hop, (long long)kIstftPer * NT);
    a.tile_len = (int)tile_len;
    a.tile_origin = (tile_len % a.hop == 0) ? a.out_off - a.out_off % a.hop : a.out_off;
    const long long end = (long long)a.out_off + a.out_len;
    a.tiles = (int)((end - a.tile_origin + tile_len - 1) / tile_len);
    return (long long)a.tiles * channels;
}

// One workgroup per tile while the device holds them all at once; past that (MAY_PERSIST), as
// many workgroups as it holds, each taking every grid-th tile.
template <int N, int JOBS, bool MAY_PERSIST>
void launch_istft_fused_jobs(IstftArgs a, int channels, hipStream_t s) {
    constexpr int P = fused_p(N);
    constexpr int NT = JOBS * (N / 2 / P);
    a.nblocks = (int)plan_istft_tiles<N, JOBS>(a, channels);
    if constexpr (MAY_PERSIST) {
        const void* k = reinterpret_cast<const void*>(istft_kernel<N, P, JOBS, kIstftPer, true>);
        const int resident = device_blocks(k, NT);
        if (resident > 0 && a.nblocks > resident) {
            a.grid = (int)xcd_grid(resident);
            hipLaunchKernelGGL((istft_kernel<N, P, JOBS, kIstftPer, true>), dim3(a.grid), dim3(NT), 0, s, a);
            launch_check("istft_kernel");
            return;
        }
    }
    a.grid = (int)xcd_grid(a.nblocks);
    hipLaunchKernelGGL((istft_kernel<N, P, JOBS, kIstftPer, false>), dim3(a.grid), dim3(NT), 0, s, a);
    launch_check("istft_kernel");
}

// One workgroup per CU at most (the frames fill the LDS), so when the full-size tiles leave
// CUs idle, tiles of 3/4 the frames (more of them, each frame transformed by more tiles) are
// taken if they still fit in one round.
template <int N>
void launch_istft_fused(IstftArgs a, int channels, hipStream_t s) {
    constexpr int JOBS = block_jobs(N / 2 / fused_p(N), 1024);
    constexpr int ALT = JOBS * 3 / 4;
    if constexpr (N >= 2048 && ALT >= 2) {
        const int span = (N + a.hop - 1) / a.hop;
        IstftArgs t = a;
        const long long cus = device_cus();
        if (ALT - span >= 1 && plan_istft_tiles<N, JOBS>(t, channels) < cus &&
            plan_istft_tiles<N, ALT>(t, channels) <= cus) {
            launch_istft_fused_jobs<N, ALT, false>(a, channels, s);
            return;
        }
    }
    launch_istft_fused_jobs<N, JOBS, true>(a, channels, s);
}

template <int N>
void launch_fft(float2* data, int batch, int inverse, const float2* twt, hipStream_t s) {
    constexpr int P = N >= 16 ? 16 : 8;
    constexpr int TPJ = N / P;
    constexpr int JOBS = block_jobs(TPJ, 256);
    const int nblocks = (batch + JOBS - 1) / JOBS;
    hipLaunchKernelGGL((fft_kernel<N, P, JOBS>), dim3(xcd_grid(nblocks)), dim3(JOBS * TPJ), 0, s,
                       data, batch, inverse, twt, nblocks);
    launch_check("fft_kernel");
}

template <template <int> class L, class... Args>
void by_size(int n, Args&&... args) {
    switch (n) {
        case 16: L<16>::go(args...); break;
        case 32: L<32>::go(args...); break;
        case 64: L<64>::go(args...); break;
        case 128: L<128>::go(args...); break;
        case 256: L<256>::go(args...); break;
        case 512: L<512>::go(args...); break;
        case 1024: L<1024>::go(args...); break;
        case 2048: L<2048>::go(args...); break;
        case 4096: L<4096>::go(args...); break;
        case 8192: L<8192>::go(args...); break;
        default: fail(STX_STATUS_UNSUPPORTED, "FFT size %d has no kernel (supported: 16..8192)", n);
    }
}
template <int N> struct StftL { static void go(const StftArgs& a, hipStream_t s) { launch_stft<N>(a, s); } };
template <int N> struct IstftL {
    static void go(const IstftArgs& a, int ch, hipStream_t s) { launch_istft_fused<N>(a, ch, s); }
};
template <int N> struct FftL {
    static void go(float2* d, int b, int inv, const float2* tw, hipStream_t s) { launch_fft<N>(d, b, inv, tw, s); }
};

// Largest power of two stx_fft_create accepts (its four-step scratch is n complex values).
constexpr int kFftMaxRun = 1 << 24;

void check_fft(const stx_fft* f) {
    STX_REQUIRE(f != nullptr && f->n >= 2, "null FFT plan");
}

// A plan the STFT / iSTFT kernels can use (n_fft from 16 to 8192, or a mixed-radix size).
void check_stft_plan(const stx_fft* f) {
    check_fft(f);
    if (f->run_only)
        fail(STX_STATUS_UNSUPPORTED, "no STFT kernel for n_fft %d (power-of-two STFT sizes: 16..8192)", f->n);
}

void check_layout(int layout) {
    STX_REQUIRE(layout == STX_SPEC_F_MAJOR || layout == STX_SPEC_T_MAJOR, "unknown spectrum layout %d", layout);
}

// The spectrum and signal sizes are addressed with 32-bit ints inside the kernels.
void check_extent(long long elems, const char* what) {
    STX_REQUIRE(elems >= 0 && elems < (1LL << 31), "%s too large (%lld elements)", what, elems);
}

size_t istft_workspace_bytes(int n, int channels, int n_frames) {
    return sizeof(float) * (size_t)n * (size_t)std::max(channels, 0) * (size_t)std::max(n_frames, 0);
}

// Shared body of the four iSTFT entry points.
void run_istft(const stx_fft* f, IstftArgs a, int channels, void* workspace, size_t ws_bytes, hipStream_t s) {
    const bool two_step = workspace != nullptr;
    if (f->mixed) {
        if (!two_step) fail(STX_STATUS_UNSUPPORTED, "iSTFT of size %d needs the workspace variant", f->n);
        const size_t need = istft_workspace_bytes(f->n, channels, a.T);
        STX_REQUIRE(ws_bytes >= need, "workspace too small: %zu bytes, need %zu", ws_bytes, need);
        check_extent((long long)channels * a.T * f->n, "workspace");
        a.frames = static_cast<float*>(workspace);
        const int jobs = channels * a.T;
        // Two frames per block where a bin's two frames are one aligned 16-byte load (f-major, T
        // even) and both frames' buffers fit in LDS (n / 2 <= 4096).
        const bool pair = a.layout == STX_SPEC_F_MAJOR && a.T % 2 == 0 && f->n / 2 <= 4096 &&
                          (reinterpret_cast<uintptr_t>(a.spec) & 15) == 0;
        const int blocks = pair ? jobs / 2 : jobs;
        const unsigned grid = (unsigned)((blocks + kXcds - 1) / kXcds * kXcds);   // xcd_block's multiple
        const dim3 bd(kMixedThreads * (pair ? 2 : 1));
        const bool ct = f->n == 2 * MixedCt3840::M && mixed_plan_is(f->half, MixedCt3840::radix, MixedCt3840::count);
        if (ct && pair)
            hipLaunchKernelGGL((istft_frames_mixed_kernel<4096, MixedCt3840, 2>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        else if (ct)
            hipLaunchKernelGGL((istft_frames_mixed_kernel<4096, MixedCt3840, 1>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        else if (f->n / 2 <= 1024 && pair)
            hipLaunchKernelGGL((istft_frames_mixed_kernel<1024, void, 2>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        else if (f->n / 2 <= 1024)
            hipLaunchKernelGGL((istft_frames_mixed_kernel<1024, void, 1>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        else if (f->n / 2 <= 4096 && pair)
            hipLaunchKernelGGL((istft_frames_mixed_kernel<4096, void, 2>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        else if (f->n / 2 <= 4096)
            hipLaunchKernelGGL((istft_frames_mixed_kernel<4096, void, 1>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        else
            hipLaunchKernelGGL((istft_frames_mixed_kernel<8192, void, 1>), dim3(grid), bd, 0, s, a, f->half, f->twn,
                               f->twm, f->n, jobs);
        launch_check("istft_frames_mixed_kernel");
        hipLaunchKernelGGL(istft_ola_kernel, dim3((a.out_len + 255) / 256, channels), dim3(256), 0, s, a, f->n);
        launch_check("istft_ola_kernel");
        return;
    }
    // Power-of-two sizes: the fused kernel with or without a workspace (a two-kernel path that
    // transforms each frame once into the workspace measured slower at every size here: it
    // writes and re-reads every windowed frame). A workspace passed in is still checked.
    if (two_step) {
        const size_t need = istft_workspace_bytes(f->n, channels, a.T);
        STX_REQUIRE(ws_bytes >= need, "workspace too small: %zu bytes, need %zu", ws_bytes, need);
    }
    by_size<IstftL>(f->n, a, channels, s);
}

stx_status torch_istft_impl(const stx_fft* f, const float* spec, int channels, int n_frames, int hop,
                            int normalized, float* out, stx_spec_layout layout, void* ws, size_t ws_bytes,
                            stx_stream stream) {
    return guard([&] {
        check_stft_plan(f);
        check_layout(layout);
        const int n = f->n;
        STX_REQUIRE(channels >= 0 && hop > 0 && n_frames >= 1, "bad channels/hop/n_frames");
        const long long length = (long long)hop * (n_frames - 1);
        check_extent(length + n, "signal");
        check_extent((long long)channels * n_frames * (n / 2 + 1), "spectrum");
        check_extent((long long)channels * length, "output");
        if (channels == 0 || length == 0) return;
        STX_REQUIRE(spec && out, "NULL buffer");
        IstftArgs a{};
        a.spec = reinterpret_cast<const float2*>(spec);
        a.out = out;
        a.win = f->win;
        a.twt = f->twt;
        a.T = n_frames;
        a.F = n / 2 + 1;
        a.layout = layout;
        a.hop = hop;
        a.env_frames = n_frames;
        a.frame_off = 0;
        a.out_off = n / 2;
        a.out_len = (int)length;
        a.valid_end = (int)(n + (long long)hop * (n_frames - 1));
        a.keep_nyquist = 1;
        a.norm = (float)((normalized ? std::sqrt((double)n) : 1.0) / n);
        run_istft(f, a, channels, ws, ws_bytes, as_stream(stream));
    });
}

stx_status htdemucs_ispec_impl(const stx_fft* f, const float* spec, int channels, int n_frames, int length,
                               float* out, stx_spec_layout layout, void* ws, size_t ws_bytes, stx_stream stream) {
    return guard([&] {
        check_stft_plan(f);
        if (f->mixed) fail(STX_STATUS_UNSUPPORTED, "htdemucs_ispec needs a power-of-two FFT size");
        check_layout(layout);
        const int n = f->n, hl = n / 4, pad = hl / 2 * 3;
        STX_REQUIRE(channels >= 0 && n_frames >= 0 && length >= 0, "bad channels/n_frames/length");
        const long long frames = (long long)n_frames + 4;             // two zero frames each side
        const long long full = n + (long long)hl * (frames - 1);
        const long long le_out = (long long)hl * ((length + hl - 1) / hl) + 2 * pad;
        check_extent(full + length, "signal");
        check_extent((long long)channels * n_frames * (n / 2), "spectrum");
        check_extent((long long)channels * length, "output");
        if (channels == 0 || length == 0) return;
        STX_REQUIRE(spec && out, "NULL buffer");
        if (n_frames == 0) {   // no frames: silence (a fill kernel, which graph capture records safely)
            const size_t count = (size_t)channels * length;
            hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, as_stream(stream),
                               out, count);
            launch_check("zero_kernel");
            return;
        }
        IstftArgs a{};
        a.spec = reinterpret_cast<const float2*>(spec);
        a.out = out;
        a.win = f->win;
        a.twt = f->twt;
        a.T = n_frames;
        a.F = n / 2;
        a.layout = layout;
        a.hop = hl;
        a.env_frames = (int)frames;
        a.frame_off = 2;
        a.out_off = n / 2 + pad;
        a.out_len = length;
        // out[i] = 0 where j - n/2 >= le_out or j >= full (src/stft.h:135-136), j = n/2 + pad + i.
        a.valid_end = (int)std::min(full, le_out + n / 2);
        a.keep_nyquist = 0;
        a.norm = (float)(std::sqrt((double)n) / n);
        run_istft(f, a, channels, ws, ws_bytes, as_stream(stream));
    });
}

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_fft_create(int n, stx_fft** out) {
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        // st::FFT's own check (src/stft.h:22).
        if (n < 2 || (n & (n - 1))) fail(STX_STATUS_INVALID_ARGUMENT, "FFT size must be a power of two");
        if (n > kFftMaxRun)
            fail(STX_STATUS_UNSUPPORTED, "FFT size %d is above %d (the four-step scratch limit)", n, kFftMaxRun);
        if (n < 16 || n > 8192) {
            std::unique_ptr<stx_fft, void (*)(stx_fft*)> f(new stx_fft, stx_fft_destroy);
            f->n = n;
            f->run_only = 1;
            hip_check(hipGetDevice(&f->device), "hipGetDevice");
            if (n > 8192) {
                const int b = ilog2(n);
                f->n1 = 1 << ((b + 1) / 2);
                f->n2 = n / f->n1;
                stx_fft* s1 = nullptr;
                stx_fft* s2 = nullptr;
                const stx_status st1 = stx_fft_create(f->n1, &s1);
                f->sub1 = s1;
                if (st1 != STX_STATUS_OK) fail(st1, "%s", stx_last_error());
                const stx_status st2 = stx_fft_create(f->n2, &s2);
                f->sub2 = s2;
                if (st2 != STX_STATUS_OK) fail(st2, "%s", stx_last_error());
                hip_check(hipMalloc(&f->scratch, sizeof(float2) * (size_t)n), "hipMalloc(FFT scratch)");
            }
            *out = f.release();
            return;
        }
        const int lbits = (ilog2(n) + 1) / 2, L = 1 << lbits, H = n / L;
        std::vector<float2> twt(L + H);
        auto w_n = [n](long long m) {
            const double th = 2.0 * M_PI * (double)m / n;
            return make_float2((float)std::cos(th), (float)-std::sin(th));
        };
        for (int m = 0; m < L; m++) twt[m] = w_n(m);
        for (int h = 0; h < H; h++) twt[L + h] = w_n((long long)h * L);
        std::vector<float> win(n), win_hs(2 * (size_t)n);
        for (int m = 0; m < n; m++) {
            const double w = 0.5 - 0.5 * std::cos(2.0 * M_PI * m / n);   // hann_periodic (src/stft.h:70-74)
            win[m] = (float)w;
            win_hs[m] = (float)(0.5 * w);                                  // STFT scale 1
            win_hs[n + m] = (float)(0.5 * w / std::sqrt((double)n));       // STFT scale 1 / sqrt(n)
        }
        stx_fft* f = new stx_fft;
        f->n = n;
        hipError_t e = hipGetDevice(&f->device);
        if (e == hipSuccess) e = hipMalloc(&f->twt, sizeof(float2) * twt.size());
        if (e == hipSuccess) e = hipMalloc(&f->win, sizeof(float) * n);
        if (e == hipSuccess) e = hipMalloc(&f->win_hs, sizeof(float) * win_hs.size());
        if (e == hipSuccess) e = hipMemcpy(f->twt, twt.data(), sizeof(float2) * twt.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(f->win, win.data(), sizeof(float) * n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(f->win_hs, win_hs.data(), sizeof(float) * win_hs.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            stx_fft_destroy(f);
            hip_check(e, "stx_fft_create");
        }
        *out = f;
    });
}

STX_API stx_status stx_fft_create_any(int n, stx_fft** out) {
    if (n >= 16 && n <= 8192 && (n & (n - 1)) == 0) return stx_fft_create(n, out);
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        STX_REQUIRE(n >= 1, "FFT size must be positive");
        MixedRadix half, full;
        if (n % 2 != 0 || n < 16 || n > 16384 || !mixed_plan(n / 2, half) || !mixed_plan(n, full))
            fail(STX_STATUS_UNSUPPORTED, "FFT size %d has no kernel (even sizes 2^a 3^b 5^c from 16 to 16384)", n);
        std::vector<float2> twn(n);
        for (int m = 0; m < n; m++) {
            const double th = 2.0 * M_PI * (double)m / n;
            twn[m] = make_float2((float)std::cos(th), (float)-std::sin(th));
        }
        // The passes' two-level table: W_n^j for j < kMixedTwL, then W_n^(h kMixedTwL).
        std::vector<float2> twm(kMixedTwMax, make_float2(0.f, 0.f));
        for (int j = 0; j < kMixedTwL; j++) twm[j] = twn[j % n];
        for (int h = 0; h * kMixedTwL < n; h++) twm[kMixedTwL + h] = twn[h * kMixedTwL];
        std::vector<float> win(n);
        for (int m = 0; m < n; m++) win[m] = (float)(0.5 - 0.5 * std::cos(2.0 * M_PI * m / n));   // hann_periodic (src/stft.h:70-74)
        stx_fft* f = new stx_fft;
        f->n = n;
        f->mixed = 1;
        f->half = half;
        f->full = full;
        hipError_t e = hipGetDevice(&f->device);
        if (e == hipSuccess) e = hipMalloc(&f->twn, sizeof(float2) * n);
        if (e == hipSuccess) e = hipMalloc(&f->win, sizeof(float) * n);
        if (e == hipSuccess) e = hipMemcpy(f->twn, twn.data(), sizeof(float2) * n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMalloc(&f->twm, sizeof(float2) * twm.size());
        if (e == hipSuccess) e = hipMemcpy(f->twm, twm.data(), sizeof(float2) * twm.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(f->win, win.data(), sizeof(float) * n, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            stx_fft_destroy(f);
            hip_check(e, "stx_fft_create_any");
        }
        *out = f;
    });
}

STX_API void stx_fft_destroy(stx_fft* f) {
    if (!f) return;
    if (f->sub1) stx_fft_destroy(f->sub1);
    if (f->sub2) stx_fft_destroy(f->sub2);
    if (f->scratch) (void)hipFree(f->scratch);
    if (f->twt) (void)hipFree(f->twt);
    if (f->win) (void)hipFree(f->win);
    if (f->win_hs) (void)hipFree(f->win_hs);
    if (f->twn) (void)hipFree(f->twn);
    if (f->twm) (void)hipFree(f->twm);
    delete f;
}

STX_API int stx_fft_size(const stx_fft* f) { return f ? f->n : 0; }

STX_API stx_status stx_fft_run(const stx_fft* f, float* data, int batch, int inverse, stx_stream stream) {
    return guard([&] {
        check_fft(f);
        STX_REQUIRE(batch >= 0, "batch < 0");
        if (batch == 0) return;
        STX_REQUIRE(data != nullptr, "data is NULL");
        check_extent((long long)batch * f->n, "FFT batch");
        const hipStream_t st = as_stream(stream);
        float2* d2 = reinterpret_cast<float2*>(data);
        const int inv = inverse ? 1 : 0;
        if (f->run_only && f->n <= 8) {
            const unsigned grid = (unsigned)((batch + 255) / 256);
            if (f->n == 2) hipLaunchKernelGGL(fft_small_kernel<2>, dim3(grid), dim3(256), 0, st, d2, batch, inv);
            else if (f->n == 4) hipLaunchKernelGGL(fft_small_kernel<4>, dim3(grid), dim3(256), 0, st, d2, batch, inv);
            else hipLaunchKernelGGL(fft_small_kernel<8>, dim3(grid), dim3(256), 0, st, d2, batch, inv);
            launch_check("fft_small_kernel");
            return;
        }
        if (f->run_only) {
            // x[n2 m1 + m2] as A[m1][m2] (n1 x n2): transpose, n2 transforms of n1 points, twiddle
            // W_n^(m2 k1) and transpose, n1 transforms of n2 points, transpose: X[k1 + n1 k2].
            const int n1 = f->n1, n2 = f->n2;
            auto transpose = [&](const float2* src, float2* dst, int rows, int cols, int tw) {
                hipLaunchKernelGGL(transpose_c64_kernel, dim3((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32)),
                                   dim3(256), 0, st, src, dst, rows, cols, tw, f->n, inv);
                launch_check("transpose_c64_kernel");
            };
            for (int b = 0; b < batch; b++) {
                float2* d = d2 + (size_t)b * f->n;
                transpose(d, f->scratch, n1, n2, 0);
                by_size<FftL>(n1, f->scratch, n2, inv, f->sub1->twt, st);
                transpose(f->scratch, d, n2, n1, 1);
                by_size<FftL>(n2, d, n1, inv, f->sub2->twt, st);
                transpose(d, f->scratch, n1, n2, 0);
                hipLaunchKernelGGL(copy_c64_kernel, dim3((unsigned)((f->n + 255) / 256)), dim3(256), 0, st,
                                   f->scratch, d, (long long)f->n);
                launch_check("copy_c64_kernel");
            }
            return;
        }
        if (f->mixed) {
            if (f->n > 8192) fail(STX_STATUS_UNSUPPORTED, "complex transforms of %d points (at most 8192)", f->n);
            if (f->n <= 1024)
                hipLaunchKernelGGL(fft_mixed_kernel<1024>, dim3((unsigned)batch), dim3(kMixedThreads), 0,
                                   as_stream(stream), reinterpret_cast<float2*>(data), inverse ? 1 : 0, f->full, f->twm,
                                   f->n);
            else if (f->n <= 4096)
                hipLaunchKernelGGL(fft_mixed_kernel<4096>, dim3((unsigned)batch), dim3(kMixedThreads), 0,
                                   as_stream(stream), reinterpret_cast<float2*>(data), inverse ? 1 : 0, f->full, f->twm,
                                   f->n);
            else
                hipLaunchKernelGGL(fft_mixed_kernel<8192>, dim3((unsigned)batch), dim3(kMixedThreads), 0,
                                   as_stream(stream), reinterpret_cast<float2*>(data), inverse ? 1 : 0, f->full, f->twm,
                                   f->n);
            launch_check("fft_mixed_kernel");
            return;
        }
        by_size<FftL>(f->n, reinterpret_cast<float2*>(data), batch, inverse ? 1 : 0, f->twt, as_stream(stream));
    });
}

STX_API int stx_torch_stft_frames(int len, int hop) { return hop > 0 && len >= 0 ? len / hop + 1 : 0; }

STX_API int stx_htdemucs_frames(int n_fft, int len) {
    const int hl = n_fft / 4;
    return hl > 0 && len >= 0 ? (len + hl - 1) / hl : 0;
}

STX_API stx_status stx_torch_stft(const stx_fft* f, const float* x, int channels, int len, int hop,
                                  int normalized, float* spec, stx_spec_layout layout, stx_stream stream) {
    return guard([&] {
        check_stft_plan(f);
        check_layout(layout);
        const int n = f->n;
        STX_REQUIRE(channels >= 0 && hop > 0 && len >= 0, "bad channels/hop/len");
        // reflect_pad(x, len, n/2, n/2) throws unless len > n/2 (src/stft.h:59).
        if (len <= n / 2) fail(STX_STATUS_RUNTIME_ERROR, "reflect pad larger than the signal");
        if (channels == 0) return;
        STX_REQUIRE(x && spec, "NULL buffer");
        StftArgs a{};
        a.x = x;
        a.spec = reinterpret_cast<float2*>(spec);
        a.win = f->win;
        a.twt = f->twt;
        a.len = len;
        a.len1 = len;
        a.pre_left = 0;
        a.hop = hop;
        a.frame0 = 0;
        a.T = len / hop + 1;
        a.F = n / 2 + 1;
        a.jobs = channels * a.T;
        a.layout = layout;
        a.scale = normalized ? (float)(1.0 / std::sqrt((double)n)) : 1.0f;
        a.win_hs = f->win_hs ? f->win_hs + (normalized ? n : 0) : nullptr;
        check_extent((long long)channels * a.T * a.F, "spectrum");
        check_extent((long long)channels * len + n, "signal");
        if (f->mixed) {
            // Two frames per block where a bin row's two values are one aligned 16-byte store
            // (f-major, T even) and both frames' buffers fit in LDS (n / 2 <= 4096).
            const bool pair = layout == STX_SPEC_F_MAJOR && a.T % 2 == 0 && n / 2 <= 4096 &&
                              (reinterpret_cast<uintptr_t>(spec) & 15) == 0;
            const int blocks = pair ? a.jobs / 2 : a.jobs;
            const unsigned grid = (unsigned)((blocks + kXcds - 1) / kXcds * kXcds);   // xcd_block's multiple
            const dim3 bd(kMixedThreads * (pair ? 2 : 1));
            const hipStream_t st = as_stream(stream);
            const bool ct = n == 2 * MixedCt3840::M && mixed_plan_is(f->half, MixedCt3840::radix, MixedCt3840::count);
            if (ct && pair)
                hipLaunchKernelGGL((stft_mixed_kernel<4096, MixedCt3840, 2>), dim3(grid), bd, 0, st, a, f->half, f->twn,
                                   f->twm, n);
            else if (ct)
                hipLaunchKernelGGL((stft_mixed_kernel<4096, MixedCt3840, 1>), dim3(grid), bd, 0, st, a, f->half, f->twn,
                                   f->twm, n);
            else if (n / 2 <= 1024 && pair)
                hipLaunchKernelGGL((stft_mixed_kernel<1024, void, 2>), dim3(grid), bd, 0, st, a, f->half, f->twn, f->twm, n);
            else if (n / 2 <= 1024)
                hipLaunchKernelGGL((stft_mixed_kernel<1024, void, 1>), dim3(grid), bd, 0, st, a, f->half, f->twn, f->twm, n);
            else if (n / 2 <= 4096 && pair)
                hipLaunchKernelGGL((stft_mixed_kernel<4096, void, 2>), dim3(grid), bd, 0, st, a, f->half, f->twn, f->twm, n);
            else if (n / 2 <= 4096)
                hipLaunchKernelGGL((stft_mixed_kernel<4096, void, 1>), dim3(grid), bd, 0, st, a, f->half, f->twn, f->twm, n);
            else
                hipLaunchKernelGGL((stft_mixed_kernel<8192, void, 1>), dim3(grid), bd, 0, st, a, f->half, f->twn, f->twm, n);
            launch_check("stft_mixed_kernel");
            return;
        }
        by_size<StftL>(n, a, as_stream(stream));
    });
}

STX_API stx_status stx_htdemucs_spec(const stx_fft* f, const float* x, int channels, int len, float* spec,
                                     stx_spec_layout layout, stx_stream stream) {
    return guard([&] {
        check_stft_plan(f);
        if (f->mixed) fail(STX_STATUS_UNSUPPORTED, "htdemucs_spec needs a power-of-two FFT size");
        check_layout(layout);
        const int n = f->n, hl = n / 4;
        STX_REQUIRE(channels >= 0 && len >= 0, "bad channels/len");
        const int le = (len + hl - 1) / hl;
        const int pad = hl / 2 * 3;
        const int rpad = pad + le * hl - len;
        // reflect_pad(x, len, pad, rpad) then reflect_pad(xf, len1, n/2, n/2) (src/stft.h:86-89).
        if (len <= pad || len <= rpad) fail(STX_STATUS_RUNTIME_ERROR, "reflect pad larger than the signal");
        const int len1 = len + pad + rpad;
        if (len1 <= n / 2) fail(STX_STATUS_RUNTIME_ERROR, "reflect pad larger than the signal");
        if (channels == 0) return;
        STX_REQUIRE(x && spec, "NULL buffer");
        StftArgs a{};
        a.x = x;
        a.spec = reinterpret_cast<float2*>(spec);
        a.win = f->win;
        a.twt = f->twt;
        a.len = len;
        a.len1 = len1;
        a.pre_left = pad;
        a.hop = hl;
        a.frame0 = 2 * hl;                                    // skip the first two frames (:97)
        a.T = le;
        a.F = n / 2;                                          // Nyquist dropped (:100)
        a.jobs = channels * a.T;
        a.layout = layout;
        a.scale = (float)(1.0 / std::sqrt((double)n));
        a.win_hs = f->win_hs ? f->win_hs + n : nullptr;   // power-of-two plans only
        check_extent((long long)channels * a.T * a.F, "spectrum");
        check_extent((long long)channels * len1 + n, "signal");
        by_size<StftL>(n, a, as_stream(stream));
    });
}

STX_API size_t stx_istft_workspace_size(const stx_fft* f, int channels, int n_frames) {
    return f ? istft_workspace_bytes(f->n, channels, n_frames) : 0;
}

STX_API stx_status stx_torch_istft(const stx_fft* f, const float* spec, int channels, int n_frames, int hop,
                                   int normalized, float* out, stx_spec_layout layout, stx_stream stream) {
    return torch_istft_impl(f, spec, channels, n_frames, hop, normalized, out, layout, nullptr, 0, stream);
}

STX_API stx_status stx_torch_istft_ws(const stx_fft* f, const float* spec, int channels, int n_frames, int hop,
                                      int normalized, float* out, stx_spec_layout layout, void* workspace,
                                      size_t workspace_bytes, stx_stream stream) {
    return torch_istft_impl(f, spec, channels, n_frames, hop, normalized, out, layout, workspace,
                            workspace_bytes, stream);
}

STX_API stx_status stx_htdemucs_ispec(const stx_fft* f, const float* spec, int channels, int n_frames,
                                      int length, float* out, stx_spec_layout layout, stx_stream stream) {
    return htdemucs_ispec_impl(f, spec, channels, n_frames, length, out, layout, nullptr, 0, stream);
}

STX_API stx_status stx_htdemucs_ispec_ws(const stx_fft* f, const float* spec, int channels, int n_frames,
                                         int length, float* out, stx_spec_layout layout, void* workspace,
                                         size_t workspace_bytes, stx_stream stream) {
    return htdemucs_ispec_impl(f, spec, channels, n_frames, length, out, layout, workspace, workspace_bytes,
                               stream);
}

}  // extern "C"
