// stft.hip — batched STFT / iSTFT for gfx950, behind the stft.h entry points of stx.h.
//
// Reference: src/stft.h (torch_stft :146-164, torch_istft :167-197, htdemucs_spec :79-103,
// htdemucs_ispec :106-140). The reference runs one double-precision radix-2 FFT per frame on
// the host. Here:
//   * two real frames of one channel (t, t+1) share one complex N-point FFT
//     (z = a + i*b, A[k] = (Z[k] + conj Z[N-k]) / 2, B[k] = (Z[k] - conj Z[N-k]) / 2i),
//     which halves the arithmetic of a real transform;
//   * the reflect padding of both modes (torch's center pad, and HTDemucs' extra pad before
//     it) is index arithmetic on the load, so the padded signal is never materialised;
//   * the inverse transform is the forward one on conjugated data (ifft(X) = conj fft conj X);
//   * the iSTFT is an overlap-add in gather form: each workgroup owns a tile of output
//     samples, inverse-transforms every frame that overlaps it (frames shared by two tiles
//     are transformed by both, their spectra re-read from L2), accumulates the windowed
//     frames in registers in frame order, and divides by the window-squared envelope, which
//     is data independent and evaluated in closed form per sample. No atomics, no scratch,
//     one pass over the spectrum and one over the output.
#include <cmath>
#include <vector>

#include "common.hpp"
#include "fft_core.hpp"

struct stx_fft {
    int n = 0;
    int device = 0;
    float2* tw = nullptr;    // device [n]: W_n^m = exp(-2*pi*i*m/n)
    float* win = nullptr;    // device [n]: periodic Hann
};

namespace stx {
namespace {

// --------------------------------------------------------------------------------- STFT
struct StftArgs {
    const float* x;          // [C][len]
    float2* spec;            // [C][F][T] or [C][T][F]
    const float* win;        // [N]
    const float2* tw;        // [N]
    int len;                 // samples per channel
    int len1;                // length of the pre-padded signal (len when there is no pre-pad)
    int pre_left;            // left size of the pre-pad (HTDemucs' pad, 0 for torch)
    int hop;
    int frame0;              // padded index of frame 0's first sample
    int T;                   // frames per channel
    int F;                   // bins written per frame
    int pairs;               // ceil(T / 2)
    int jobs;                // channels * pairs
    int nblocks;             // real (logical) block count
    int layout;              // STX_SPEC_*
    int vec4;                // F-major pair stores may use one 16-byte store
    float half_scale;        // 0.5 * normalisation
};

// torch reflect (edge not repeated): j < 0 -> -j; j >= n -> 2(n - 1) - j (src/stft.h:58-68).
__device__ __forceinline__ int reflect(int j, int n) {
    j = j < 0 ? -j : j;
    j = j >= n ? 2 * (n - 1) - j : j;
    return j;
}

// Sample m of the fully padded signal (center pad N/2 around the pre-padded one).
template <int N>
__device__ __forceinline__ float padded_sample(const float* __restrict__ xc, int m, const StftArgs& a) {
    int j = reflect(m - N / 2, a.len1) - a.pre_left;
    j = reflect(j, a.len);
    j = min(max(j, 0), a.len - 1);   // host validation keeps j in range; this only guards memory
    return xc[j];
}

template <int N, int JOBS>
__global__ __launch_bounds__(JOBS * (N / 16)) void stft_kernel(StftArgs a) {
    using S = FftShape<N>;
    constexpr int TPJ = S::TPJ;
    __shared__ float2 lds[JOBS * S::PADN];

    const int lb = xcd_block();
    if (lb >= a.nblocks) return;                       // whole block idle: no barrier reached
    const int slot = (int)threadIdx.x / TPJ;
    const int j = (int)threadIdx.x % TPJ;
    const int job = lb * JOBS + slot;
    const bool active = job < a.jobs;
    float2* buf = lds + slot * S::PADN;

    const int c = active ? job / a.pairs : 0;
    const int t = active ? 2 * (job % a.pairs) : 0;
    const bool has_b = active && (t + 1 < a.T);
    const float* xc = a.x + (size_t)c * a.len;
    const int m0 = a.frame0 + t * a.hop;

    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int n = j + r * TPJ;
        const float w = a.win[n];
        float re = 0.f, im = 0.f;
        if (active) {
            re = padded_sample<N>(xc, m0 + n, a) * w;
            if (has_b) im = padded_sample<N>(xc, m0 + a.hop + n, a) * w;
        }
        v[r] = make_float2(re, im);
    }
    fft_first_pass<N>(v, buf, j);
    __syncthreads();
    fft_rest_passes<N, 16>(buf, j, a.tw);

    if (!active) return;
    // Separate the two real spectra and store bins k = j + q*TPJ (+ Nyquist).
    const float hs = a.half_scale;
    auto store = [&](int k) {
        const float2 zk = buf[lds_idx(k)];
        const float2 zm = buf[lds_idx((N - k) & (N - 1))];
        const float2 A = make_float2((zk.x + zm.x) * hs, (zk.y - zm.y) * hs);
        const float2 B = make_float2((zk.y + zm.y) * hs, (zm.x - zk.x) * hs);
        if (a.layout == STX_SPEC_F_MAJOR) {
            float2* p = a.spec + ((size_t)c * a.F + k) * a.T + t;
            if (has_b && a.vec4) {
                *reinterpret_cast<float4*>(p) = make_float4(A.x, A.y, B.x, B.y);
            } else {
                p[0] = A;
                if (has_b) p[1] = B;
            }
        } else {
            float2* p = a.spec + ((size_t)c * a.T + t) * a.F + k;
            p[0] = A;
            if (has_b) p[a.F] = B;
        }
    };
#pragma unroll
    for (int q = 0; q < 8; q++) store(j + q * TPJ);    // 8 * TPJ = N/2 bins
    if (a.F > N / 2 && j == 0) store(N / 2);
}

// -------------------------------------------------------------------------------- iSTFT
struct IstftArgs {
    const float2* spec;
    float* out;              // [C][out_len]
    const float* win;
    const float2* tw;
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
    int tiles;               // tiles per channel
    int nblocks;             // channels * tiles
    float norm;
};

template <int N>
__device__ __forceinline__ float2 load_bin(const IstftArgs& a, const float2* __restrict__ sc, int st, int k) {
    if (a.layout == STX_SPEC_F_MAJOR) return sc[(size_t)k * a.T + st];
    return sc[(size_t)st * a.F + k];
}

// conj(Z[k]) where Z = A + iB is the full (Hermitian-extended) spectrum of frames sa, sb.
template <int N>
__device__ __forceinline__ float2 load_pair_bin(const IstftArgs& a, const float2* __restrict__ sc,
                                                int sa, bool ha, int sb, bool hb, int k) {
    float2 A = make_float2(0.f, 0.f), B = make_float2(0.f, 0.f);
    float2 z;
    if (k == 0) {
        if (ha) A = load_bin<N>(a, sc, sa, 0);
        if (hb) B = load_bin<N>(a, sc, sb, 0);
        z = make_float2(A.x, B.x);                       // DC imaginary parts ignored
    } else if (k < N / 2) {
        if (ha) A = load_bin<N>(a, sc, sa, k);
        if (hb) B = load_bin<N>(a, sc, sb, k);
        z = make_float2(A.x - B.y, A.y + B.x);
    } else if (k == N / 2) {
        if (a.keep_nyquist) {
            if (ha) A = load_bin<N>(a, sc, sa, k);
            if (hb) B = load_bin<N>(a, sc, sb, k);
        }
        z = make_float2(A.x, B.x);                       // Nyquist imaginary parts ignored
    } else {
        const int m = N - k;
        if (ha) A = load_bin<N>(a, sc, sa, m);
        if (hb) B = load_bin<N>(a, sc, sb, m);
        z = make_float2(A.x + B.y, B.x - A.y);
    }
    return cconj(z);
}

template <int N, int JOBS, int PER>
__global__ __launch_bounds__(JOBS * (N / 16)) void istft_kernel(IstftArgs a) {
    using S = FftShape<N>;
    constexpr int TPJ = S::TPJ;
    constexpr int NT = JOBS * TPJ;
    constexpr int OT = PER * NT;                         // output samples per tile
    __shared__ float2 lds[JOBS * S::PADN];

    const int lb = xcd_block();
    if (lb >= a.nblocks) return;
    const int c = lb / a.tiles;
    const int tile = lb % a.tiles;
    const int tid = (int)threadIdx.x;
    const int slot = tid / TPJ;
    const int j = tid % TPJ;
    float2* buf = lds + slot * S::PADN;

    const int i0 = tile * OT;
    const int i1 = min(i0 + OT, a.out_len);
    const int J0 = a.out_off + i0, J1 = a.out_off + i1;
    // Spectrum frames overlapping [J0, J1): envelope frame tf covers [tf*hop, tf*hop + N).
    const int tf_lo = max(0, (J0 - N + 1 + a.hop - 1) / a.hop);   // J0 - N + 1 may be < 0: clamped
    const int tf_hi = (J1 - 1) / a.hop;
    const int st_lo = max(0, max(tf_lo, 0) - a.frame_off);
    const int st_hi = min(a.T - 1, tf_hi - a.frame_off);
    const float2* sc = a.spec + (size_t)c * a.T * a.F;

    float acc[PER];
#pragma unroll
    for (int q = 0; q < PER; q++) acc[q] = 0.f;

    for (int s0 = st_lo; s0 <= st_hi; s0 += 2 * JOBS) {
        const int sa = s0 + 2 * slot, sb = sa + 1;
        const bool ha = sa <= st_hi, hb = sb <= st_hi;
        float2 v[16];
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = load_pair_bin<N>(a, sc, sa, ha, sb, hb, j + r * TPJ);
        fft_first_pass<N>(v, buf, j);
        __syncthreads();
        fft_rest_passes<N, 16>(buf, j, a.tw);
        // buf[n] = fft(conj Z)[n]: frame sa is Re, frame sb is -Im (times N).
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int J = J0 + q * NT + tid;
#pragma unroll
            for (int s = 0; s < JOBS; s++) {
                const int fa = s0 + 2 * s;
                const float2* bs = lds + s * S::PADN;
                const int na = J - (fa + a.frame_off) * a.hop;
                if (fa <= st_hi && na >= 0 && na < N) acc[q] += bs[lds_idx(na)].x * a.win[na];
                const int nb = na - a.hop;
                if (fa + 1 <= st_hi && nb >= 0 && nb < N) acc[q] -= bs[lds_idx(nb)].y * a.win[nb];
            }
        }
        __syncthreads();
    }

    float* oc = a.out + (size_t)c * a.out_len;
#pragma unroll
    for (int q = 0; q < PER; q++) {
        const int i = i0 + q * NT + tid;
        if (i >= i1) continue;
        const int J = a.out_off + i;
        float y = 0.f;
        if (J < a.valid_end) {
            // Envelope: sum of win^2 over every frame covering J (src/stft.h:130,187).
            const int lo = max(0, (J - N + a.hop) / a.hop);
            const int hi = min(a.env_frames - 1, J / a.hop);
            float env = 0.f;
            for (int tf = lo; tf <= hi; tf++) {
                const int n = J - tf * a.hop;
                if (n >= 0 && n < N) {
                    const float w = a.win[n];
                    env += w * w;
                }
            }
            y = env > 1e-11f ? acc[q] * a.norm / env : 0.f;
        }
        oc[i] = y;
    }
}

// ------------------------------------------------------------------------ plain FFT
template <int N, int JOBS>
__global__ __launch_bounds__(JOBS * (N / 16)) void fft_kernel(float2* data, int batch, int inverse,
                                                              const float2* __restrict__ tw, int nblocks) {
    using S = FftShape<N>;
    constexpr int TPJ = S::TPJ;
    __shared__ float2 lds[JOBS * S::PADN];
    const int lb = xcd_block();
    if (lb >= nblocks) return;
    const int slot = (int)threadIdx.x / TPJ;
    const int j = (int)threadIdx.x % TPJ;
    const int job = lb * JOBS + slot;
    const bool active = job < batch;
    float2* buf = lds + slot * S::PADN;
    float2* d = data + (size_t)(active ? job : 0) * N;
    float2 v[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        float2 x = active ? d[j + r * TPJ] : make_float2(0.f, 0.f);
        v[r] = inverse ? cconj(x) : x;
    }
    fft_first_pass<N>(v, buf, j);
    __syncthreads();
    fft_rest_passes<N, 16>(buf, j, tw);
    if (!active) return;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int k = j + r * TPJ;
        const float2 y = buf[lds_idx(k)];
        d[k] = inverse ? cconj(y) : y;
    }
}

// ------------------------------------------------------------------------ dispatch
constexpr int jobs_per_block(int n) { return n >= 4096 ? 1 : 4096 / n; }

template <int N>
void launch_stft(const StftArgs& a0, hipStream_t s) {
    constexpr int JOBS = jobs_per_block(N);
    StftArgs a = a0;
    a.nblocks = (a.jobs + JOBS - 1) / JOBS;
    hipLaunchKernelGGL((stft_kernel<N, JOBS>), dim3(xcd_grid(a.nblocks)), dim3(JOBS * (N / 16)), 0, s, a);
    launch_check("stft_kernel");
}

constexpr int kIstftPer = 16;

template <int N>
void launch_istft(IstftArgs a, int channels, hipStream_t s) {
    constexpr int JOBS = jobs_per_block(N);
    constexpr int OT = kIstftPer * JOBS * (N / 16);
    a.tiles = (a.out_len + OT - 1) / OT;
    a.nblocks = a.tiles * channels;
    hipLaunchKernelGGL((istft_kernel<N, JOBS, kIstftPer>), dim3(xcd_grid(a.nblocks)),
                       dim3(JOBS * (N / 16)), 0, s, a);
    launch_check("istft_kernel");
}

template <int N>
void launch_fft(float2* data, int batch, int inverse, const float2* tw, hipStream_t s) {
    constexpr int JOBS = jobs_per_block(N);
    const int nblocks = (batch + JOBS - 1) / JOBS;
    hipLaunchKernelGGL((fft_kernel<N, JOBS>), dim3(xcd_grid(nblocks)), dim3(JOBS * (N / 16)), 0, s,
                       data, batch, inverse, tw, nblocks);
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
    static void go(const IstftArgs& a, int ch, hipStream_t s) { launch_istft<N>(a, ch, s); }
};
template <int N> struct FftL {
    static void go(float2* d, int b, int inv, const float2* tw, hipStream_t s) { launch_fft<N>(d, b, inv, tw, s); }
};

void check_fft(const stx_fft* f) {
    STX_REQUIRE(f != nullptr && f->n >= 16, "null FFT plan");
}

void check_layout(int layout) {
    STX_REQUIRE(layout == STX_SPEC_F_MAJOR || layout == STX_SPEC_T_MAJOR, "unknown spectrum layout %d", layout);
}

// The spectrum and signal sizes are addressed with 32-bit ints inside the kernels.
void check_extent(long long elems, const char* what) {
    STX_REQUIRE(elems >= 0 && elems < (1LL << 31), "%s too large (%lld elements)", what, elems);
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
        if (n < 16 || n > 8192) fail(STX_STATUS_UNSUPPORTED, "FFT size %d has no kernel (supported: 16..8192)", n);
        std::vector<float2> tw(n);
        std::vector<float> win(n);
        for (int m = 0; m < n; m++) {
            const double th = 2.0 * M_PI * m / n;
            tw[m] = make_float2((float)std::cos(th), (float)-std::sin(th));
            // hann_periodic (src/stft.h:70-74), in double, rounded once.
            win[m] = (float)(0.5 - 0.5 * std::cos(2.0 * M_PI * m / n));
        }
        stx_fft* f = new stx_fft;
        f->n = n;
        hipError_t e = hipGetDevice(&f->device);
        if (e == hipSuccess) e = hipMalloc(&f->tw, sizeof(float2) * n);
        if (e == hipSuccess) e = hipMalloc(&f->win, sizeof(float) * n);
        if (e == hipSuccess) e = hipMemcpy(f->tw, tw.data(), sizeof(float2) * n, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(f->win, win.data(), sizeof(float) * n, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            stx_fft_destroy(f);
            hip_check(e, "stx_fft_create");
        }
        *out = f;
    });
}

STX_API void stx_fft_destroy(stx_fft* f) {
    if (!f) return;
    if (f->tw) (void)hipFree(f->tw);
    if (f->win) (void)hipFree(f->win);
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
        by_size<FftL>(f->n, reinterpret_cast<float2*>(data), batch, inverse ? 1 : 0, f->tw, as_stream(stream));
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
        check_fft(f);
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
        a.tw = f->tw;
        a.len = len;
        a.len1 = len;
        a.pre_left = 0;
        a.hop = hop;
        a.frame0 = 0;
        a.T = len / hop + 1;
        a.F = n / 2 + 1;
        a.pairs = (a.T + 1) / 2;
        a.jobs = channels * a.pairs;
        a.layout = layout;
        a.vec4 = (a.T % 2 == 0) && ((uintptr_t)spec % 16 == 0);
        a.half_scale = 0.5f * (normalized ? (float)(1.0 / std::sqrt((double)n)) : 1.0f);
        check_extent((long long)channels * a.T * a.F, "spectrum");
        check_extent((long long)channels * len, "signal");
        by_size<StftL>(n, a, as_stream(stream));
    });
}

STX_API stx_status stx_htdemucs_spec(const stx_fft* f, const float* x, int channels, int len, float* spec,
                                     stx_spec_layout layout, stx_stream stream) {
    return guard([&] {
        check_fft(f);
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
        a.tw = f->tw;
        a.len = len;
        a.len1 = len1;
        a.pre_left = pad;
        a.hop = hl;
        a.frame0 = 2 * hl;                                    // skip the first two frames (:97)
        a.T = le;
        a.F = n / 2;                                          // Nyquist dropped (:100)
        a.pairs = (a.T + 1) / 2;
        a.jobs = channels * a.pairs;
        a.layout = layout;
        a.vec4 = (a.T % 2 == 0) && ((uintptr_t)spec % 16 == 0);
        a.half_scale = (float)(0.5 / std::sqrt((double)n));
        check_extent((long long)channels * a.T * a.F, "spectrum");
        check_extent((long long)channels * len1 + n, "signal");
        by_size<StftL>(n, a, as_stream(stream));
    });
}

STX_API stx_status stx_torch_istft(const stx_fft* f, const float* spec, int channels, int n_frames, int hop,
                                   int normalized, float* out, stx_spec_layout layout, stx_stream stream) {
    return guard([&] {
        check_fft(f);
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
        a.tw = f->tw;
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
        by_size<IstftL>(n, a, channels, as_stream(stream));
    });
}

STX_API stx_status stx_htdemucs_ispec(const stx_fft* f, const float* spec, int channels, int n_frames,
                                      int length, float* out, stx_spec_layout layout, stx_stream stream) {
    return guard([&] {
        check_fft(f);
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
        IstftArgs a{};
        a.spec = reinterpret_cast<const float2*>(spec);
        a.out = out;
        a.win = f->win;
        a.tw = f->tw;
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
        if (n_frames == 0) {
            hip_check(hipMemsetAsync(out, 0, sizeof(float) * (size_t)channels * length, as_stream(stream)),
                      "hipMemsetAsync");
            return;
        }
        by_size<IstftL>(n, a, channels, as_stream(stream));
    });
}

}  // extern "C"
