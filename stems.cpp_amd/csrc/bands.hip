// bands.hip — RoFormer band gather and mask scatter-average + complex mask apply on gfx950.
//
// Reference: RoFormer::Impl::run, src/roformer.cpp:226-241 (gather) and :251-278 (scatter,
// average, apply, zero_dc). Both are rewritten in gather form so that no two threads write
// one element:
//   * band gather: band b's features are one contiguous block [T][size_b * C] of complex
//     values (feat[t][(j*C + c)*2 + {re,im}]). T-major spectra: one workgroup per frame stages
//     the frame's C rows in LDS with its first loads and writes every (band, position) entry's
//     C values from there, guided by one 8-byte record per entry (no table search before the
//     spectrum loads); frames too wide for LDS walk the output flat, 8 values per thread,
//     finding their band by a binary search over the band starts. F-major spectra: one
//     workgroup per (band, tile of frames) through an LDS transpose, so that both sides stay
//     coalesced.
//   * scatter + apply: a thread per (bin, channel) and tile of frames (T-major) or per frame
//     (F-major) sums the mask values of the (band, position) pairs that cover its bin in the
//     reference's band-then-position order, in double, divides by the band count and
//     multiplies the spectrum, all in double like the reference, and rounds once. The pairs
//     come from one 16-byte record per bin when no bin has more than two (the mel and
//     band-split maps), else from a CSR table built once per band table. Neighbouring lanes
//     take neighbouring (bin, channel) pairs, which are neighbouring floats of the mask rows,
//     so mask reads are coalesced in T-major layout, and each thread issues its frames' loads
//     together.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "bands_host.hpp"
#include "common.hpp"

namespace stx {
struct BandInfo {
    long long feat_off;      // band_feat_off[b]: first float of the band's block, per frame
    int freq_off;            // band_freq_off[b]
    int size;                // band_sizes[b]
};
struct CsrEntry {
    long long feat_off;      // band_feat_off[b] of the covering band
    int din;                 // dim_in(b) = size * C * 2
    int col;                 // j * C * 2: the bin's column inside the band's rows
};
// A bin's covering (band, position) pairs when there are at most two, in CSR order: one 16-byte
// load instead of the CSR offsets, the entries and the denominator. din[1] == 0: one pair;
// din[0] == 0: none. A missing pair repeats a valid address (entry 0, or the first mask value)
// and is not added.
struct BinBands {
    int feat_off[2];
    unsigned short din[2];
    unsigned short col[2];
};
static_assert(sizeof(BinBands) == 16, "BinBands is one 16-byte load");
// One (band, position) entry of the band table, in feature order.
struct GatherRec {
    int first;               // freq_off[b]: the band's first entry
    unsigned short size;     // band_sizes[b]
    unsigned short bin;      // band_freqs[entry]
};
static_assert(sizeof(GatherRec) == 8, "GatherRec is one 8-byte load");
}  // namespace stx

struct stx_bands {
    int n_bands = 0, n_bins = 0, channels = 0;
    long long n_freqs = 0, total_feat = 0;
    int max_pairs = 0;                               // max band size * channels
    std::vector<int64_t> freq_off, feat_off;
    std::vector<int32_t> bpf;
    stx::BandInfo* d_bands = nullptr;
    int* d_band_freqs = nullptr;
    int* d_csr_off = nullptr;                        // [n_bins + 1]
    stx::CsrEntry* d_csr = nullptr;                  // [n_freqs]
    double* d_denom = nullptr;                       // [n_bins]: max(bands_per_freq, 1)
    stx::BinBands* d_bin_bands = nullptr;            // [n_bins] when every bin has at most two pairs
    stx::GatherRec* d_gather_rec = nullptr;          // [n_freqs] when sizes and bins fit 16 bits
    int* d_pair_off = nullptr;                       // [n_bands + 1]: first (bin, channel) pair of band b
    int* d_pair_code = nullptr;                      // [total_feat / 2]: (channel << 16) | bin of each pair
    int* d_freq_lo = nullptr;                        // [n_bands]: first bin of each band
    stx::FastDiv* d_pair_div = nullptr;              // [n_bands]: division by the band's pairs per frame
    bool ranges = false;                             // every band is a range of consecutive bins
};

namespace stx {
namespace {

struct GatherArgs {
    const float2* spec;      // [batch][C][F][T] or [batch][C][T][F]
    float2* feat;            // [batch][total_feat * T / 2]
    const BandInfo* bands;
    const int* band_freqs;
    const int* pair_off;     // [n_bands + 1]
    const int* pair_code;    // [total_feat / 2]
    const int* freq_lo;      // [n_bands]: first bin of each band when every band is a bin range
    const stx::FastDiv* pair_div;   // [n_bands]: division by the band's pairs per frame
    stx::FastDiv cdiv;       // division by C
    const GatherRec* rec;    // [n_entries] (band_gather_frame_kernel)
    int n_entries;           // n_freqs
    stx::FastDiv fdiv;       // division by F
    int C, F, T;
    int n_bands;
    long long total_feat;    // floats per frame of one batch item
    int TT;                  // F-major: frames per tile
};

constexpr int kGatherPer = 8;                        // T-major: outputs per thread

// T-major: the batch item's features, n = (total_feat / 2) * T complex values, walked flat in
// blocks of 256 * kGatherPer. Band b covers [pair_off[b] * T, pair_off[b + 1] * T); inside it,
// value r is frame r / pairs_b, pair r % pairs_b. Reads of one band row are neighbouring bins
// of two channel rows; writes are contiguous.
// RANGES: every band is a range of consecutive bins, so pair q of band b is channel q % C of
// bin freq_lo[b] + q / C and the pair table is not read.
template <bool RANGES>
__global__ __launch_bounds__(256) void band_gather_t_kernel(GatherArgs a) {
    // LDS: [n_bands + 1] pair offsets, [n_bands] first bins, [n_bands] dividers by the pairs.
    extern __shared__ int po[];
    int* flo = po + a.n_bands + 1;
    stx::FastDiv* fd = reinterpret_cast<stx::FastDiv*>(flo + a.n_bands);
    const int tid = (int)threadIdx.x;
    for (int b = tid; b <= a.n_bands; b += 256) po[b] = a.pair_off[b];
    for (int b = tid; b < a.n_bands; b += 256) {
        if constexpr (RANGES) flo[b] = a.freq_lo[b];
        fd[b] = a.pair_div[b];
    }
    __syncthreads();
    const int bt = (int)blockIdx.y;
    const int n = po[a.n_bands] * a.T;
    const int e0 = (int)blockIdx.x * (256 * kGatherPer) + tid;
    if (e0 >= n) return;
    int lo = 0, hi = a.n_bands;                      // po[lo] * T <= e0 < po[hi] * T
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (po[mid] * a.T <= e0) lo = mid;
        else hi = mid;
    }
    int b = lo;
    int pair[kGatherPer], t[kGatherPer], code[kGatherPer];
#pragma unroll
    for (int k = 0; k < kGatherPer; k++) {
        const int e = min(e0 + k * 256, n - 1);
        while (po[b + 1] * a.T <= e) b++;
        const int pairs = po[b + 1] - po[b];
        const int r = e - po[b] * a.T;
        t[k] = (int)fd[b].div((unsigned)r);                   // r / pairs
        const int q = r - t[k] * pairs;
        pair[k] = po[b] + q;
        if constexpr (RANGES) {
            const int j = (int)a.cdiv.div((unsigned)q);       // q / C
            code[k] = ((q - j * a.C) << 16) | (flo[b] + j);
        }
    }
    if constexpr (!RANGES) {
#pragma unroll
        for (int k = 0; k < kGatherPer; k++) code[k] = a.pair_code[pair[k]];
    }
    const float2* sb = a.spec + (size_t)bt * a.C * a.T * a.F;
    float2 v[kGatherPer];
#pragma unroll
    for (int k = 0; k < kGatherPer; k++)
        v[k] = sb[((size_t)(code[k] >> 16) * a.T + t[k]) * a.F + (code[k] & 0xffff)];
    float2* fb = a.feat + (size_t)bt * n;
#pragma unroll
    for (int k = 0; k < kGatherPer; k++)
        if (e0 + k * 256 < n) fb[e0 + k * 256] = v[k];
}

// T-major, one workgroup per frame: the frame's C rows of F bins (contiguous in this layout)
// are loaded into LDS with the first loads of the kernel, together with the thread's entry
// records; each thread then takes entries e (band b, position j) and writes the C values of
// bin band_freqs[e] to feat[C * (first_b * T + t * size_b + j) + c], one contiguous C * 8-byte
// store (16 bytes at C = 2). Nothing waits on a table lookup before the spectrum is in flight,
// and each spectrum value is read from HBM once however many bands cover its bin.
// Workgroups are dealt to the XCDs in runs of consecutive frames, so the partial lines where
// band rows of neighbouring frames meet merge in one L2.
template <int CC, int NT, int ROW, int OUT>          // channels (0: a.C at run time); threads;
__global__ __launch_bounds__(NT) void band_gather_frame_kernel(GatherArgs a) {   // per thread
    extern __shared__ float2 row[];                  // [C][F]
    const int t = xcd_block();
    if (t >= a.T) return;                            // uniform per workgroup
    const int C = CC > 0 ? CC : a.C;
    const int tid = (int)threadIdx.x;
    const int F = a.F, E = a.n_entries, n = C * F;
    const size_t plane = (size_t)a.T * F;
    const size_t bt = blockIdx.y;
    const float2* sb = a.spec + bt * C * plane + (size_t)t * F;
    GatherRec r[OUT];
    auto load_recs = [&](int e0) {
#pragma unroll
        for (int k = 0; k < OUT; k++) r[k] = a.rec[min(e0 + tid + k * NT, E - 1)];
    };
    load_recs(0);
    for (int i0 = 0; i0 < n; i0 += NT * ROW) {
        float2 v[ROW];
#pragma unroll
        for (int k = 0; k < ROW; k++) {
            const int i = min(i0 + tid + k * NT, n - 1);
            const int c = CC == 1 ? 0 : CC == 2 ? (i >= F ? 1 : 0) : (int)a.fdiv.div((unsigned)i);
            v[k] = sb[(size_t)c * plane + (i - c * F)];
        }
#pragma unroll
        for (int k = 0; k < ROW; k++)
            if (i0 + tid + k * NT < n) row[i0 + tid + k * NT] = v[k];
    }
    __syncthreads();
    float2* fb = a.feat + bt * ((size_t)E * C * a.T);
    for (int e0 = 0; e0 < E; e0 += NT * OUT) {
        if (e0 > 0) load_recs(e0);
#pragma unroll
        for (int k = 0; k < OUT; k++) {
            const int e = e0 + tid + k * NT;
            if (e >= E) break;
            const GatherRec R = r[k];
            float2* d = fb + (size_t)C * ((size_t)R.first * a.T + (size_t)t * R.size + (e - R.first));
            if constexpr (CC == 2) {
                const float2 v0 = row[R.bin], v1 = row[F + R.bin];
                store_stream(reinterpret_cast<float4*>(d), make_float4(v0.x, v0.y, v1.x, v1.y));
            } else {
                for (int c = 0; c < C; c++) store_stream(d + c, row[c * F + R.bin]);
            }
        }
    }
}

// The frame gather's shape: 256 threads, 9 row values (C * F = 2050 at n_fft 2048 stereo in one
// batch of 2304) and 8 entries (2048 >= the 1,979 of the 60-band mel map) per thread per batch.
template <int CC>
void launch_gather_frame(const GatherArgs& a, dim3 grid, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((band_gather_frame_kernel<CC, 256, 9, 8>), grid, dim3(256), lds, s, a);
}

// F-major: a tile [pairs][TT] is read along t (coalesced) into LDS and written along the
// band rows (coalesced).
__global__ __launch_bounds__(256) void band_gather_f_kernel(GatherArgs a) {
    extern __shared__ float2 tile[];                 // [pairs][TT + 1]
    const int b = (int)blockIdx.x;
    const int t0 = (int)blockIdx.y * a.TT;
    const int bt = (int)blockIdx.z;
    const BandInfo bi = a.bands[b];
    const int pairs = bi.size * a.C;
    const int TT = a.TT, ld = TT + 1;
    const float2* sb = a.spec + (size_t)bt * a.C * a.F * a.T;
    float2* fb = a.feat + ((size_t)bt * a.total_feat * a.T + (size_t)bi.feat_off * a.T) / 2;
    for (int e = (int)threadIdx.x; e < pairs * TT; e += 256) {
        const int q = e / TT, tt = e - q * TT;
        const int t = t0 + tt;
        if (t < a.T) {
            const int j = q / a.C, c = q - j * a.C;
            const int f = a.band_freqs[bi.freq_off + j];
            tile[q * ld + tt] = sb[((size_t)c * a.F + f) * a.T + t];
        }
    }
    __syncthreads();
    for (int e = (int)threadIdx.x; e < pairs * TT; e += 256) {
        const int tt = e / pairs, q = e - tt * pairs;
        const int t = t0 + tt;
        if (t < a.T) fb[(size_t)t * pairs + q] = tile[q * ld + tt];
    }
}

struct ScatterArgs {
    const float* masks;      // [batch][S][total_feat * T]
    const float2* spec;      // [batch][C][F][T] or [batch][C][T][F]
    float2* out;             // [batch][S][C][F][T] or [batch][S][C][T][F]
    const int* csr_off;
    const CsrEntry* csr;
    const double* denom;
    const BinBands* rec;     // per-bin pairs (band_scatter_rec_kernel)
    stx::FastDiv fc_div, c_div;   // by F * C and by C (band_scatter_rec_kernel)
    int C, F, T, S, zero_dc;
    long long total_feat;
};

// out = spec * (sum of the covering masks / band count), one rounding, src/roformer.cpp:266-278.
__device__ __forceinline__ float2 masked_bin(const ScatterArgs& a, const float* __restrict__ mb, float2 z,
                                             int f, int c, int t) {
#pragma clang fp contract(off)
    if (a.zero_dc && f == 0) return make_float2(0.f, 0.f);
    double ar = 0.0, ai = 0.0;
    const int e1 = a.csr_off[f + 1];
    for (int e = a.csr_off[f]; e < e1; e++) {
        const CsrEntry E = a.csr[e];
        const float2 m = *reinterpret_cast<const float2*>(mb + (size_t)E.feat_off * a.T + (size_t)t * E.din + E.col + 2 * c);
        ar += (double)m.x;
        ai += (double)m.y;
    }
    const double d = a.denom[f], rd = 1.0 / d;
    const double qr = div_rn(ar, d, rd), qi = div_rn(ai, d, rd);   // = ar / d, ai / d
    const double zr = z.x, zi = z.y;
    return make_float2((float)(zr * qr - zi * qi), (float)(zr * qi + zi * qr));
}

// T-major: thread = (bin, channel) for kScatterFrames frames; lanes cover consecutive mask
// floats. The CSR entries are read once; the frames' spectrum and mask loads are issued
// together, one covering band at a time, and each frame's sum runs in CSR order.
constexpr int kScatterFrames = 8;

__global__ __launch_bounds__(256) void band_scatter_t_kernel(ScatterArgs a) {
#pragma clang fp contract(off)
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i >= a.F * a.C) return;
    const int f = i / a.C, c = i - f * a.C;
    const int t0 = (int)blockIdx.y * kScatterFrames;
    const int bt = (int)blockIdx.z / a.S, s = (int)blockIdx.z % a.S;
    const float* mb = a.masks + ((size_t)bt * a.S + s) * a.total_feat * a.T;
    const float2* zc = a.spec + (((size_t)bt * a.C + c) * a.T) * a.F + f;
    int tt[kScatterFrames];
    float2 z[kScatterFrames];
#pragma unroll
    for (int k = 0; k < kScatterFrames; k++) {
        tt[k] = min(t0 + k, a.T - 1);
        z[k] = zc[(size_t)tt[k] * a.F];
    }
    double ar[kScatterFrames], ai[kScatterFrames];
#pragma unroll
    for (int k = 0; k < kScatterFrames; k++) ar[k] = ai[k] = 0.0;
    // Covering bands two at a time (a bin is in one or two bands of a mel map): both CSR
    // entries, then both bands' mask loads, then the sums in CSR order.
    const int e1 = a.csr_off[f + 1];
    for (int e = a.csr_off[f]; e < e1; e += 2) {
        const bool two = e + 1 < e1;
        const CsrEntry E0 = a.csr[e], E1 = a.csr[two ? e + 1 : e];
        const float* r0 = mb + (size_t)E0.feat_off * a.T + E0.col + 2 * c;
        const float* r1 = mb + (size_t)E1.feat_off * a.T + E1.col + 2 * c;
        float2 m0[kScatterFrames], m1[kScatterFrames];
#pragma unroll
        for (int k = 0; k < kScatterFrames; k++) {
            m0[k] = *reinterpret_cast<const float2*>(r0 + (size_t)tt[k] * E0.din);
            m1[k] = *reinterpret_cast<const float2*>(r1 + (size_t)tt[k] * E1.din);
        }
#pragma unroll
        for (int k = 0; k < kScatterFrames; k++) {
            ar[k] += (double)m0[k].x;
            ai[k] += (double)m0[k].y;
        }
        if (two) {
#pragma unroll
            for (int k = 0; k < kScatterFrames; k++) {
                ar[k] += (double)m1[k].x;
                ai[k] += (double)m1[k].y;
            }
        }
    }
    // ar / d and ai / d as div_rn with one reciprocal per thread (the IEEE quotients).
    const double d = a.denom[f], rd = 1.0 / d;
    float2* oc = a.out + (((size_t)bt * a.S + s) * a.C + c) * a.T * a.F + f;
#pragma unroll
    for (int k = 0; k < kScatterFrames; k++) {
        if (t0 + k >= a.T) break;
        float2 o = make_float2(0.f, 0.f);
        if (!(a.zero_dc && f == 0)) {
            const double qr = div_rn(ar[k], d, rd), qi = div_rn(ai[k], d, rd);
            const double zr = z[k].x, zi = z[k].y;
            o = make_float2((float)(zr * qr - zi * qi), (float)(zr * qi + zi * qr));
        }
        oc[(size_t)(t0 + k) * a.F] = o;
    }
}

// T-major with per-bin records (every bin in at most two (band, position) pairs, as in the mel
// and band-split maps): thread = (tile of kScatterRecFrames frames, bin, channel), numbered with
// (bin, channel) fastest so that no workgroup idles at the end of a tile. The record load is
// issued with the spectrum loads, so the masks are one memory trip behind, not two. With no
// table walk to amortise, 2 frames per thread (twice the workgroups of 4, 4x those of 8) hides
// the most latency; the output is stored with the non-temporal hint.
constexpr int kScatterRecFrames = 2;

__global__ __launch_bounds__(256) void band_scatter_rec_kernel(ScatterArgs a, unsigned n) {
#pragma clang fp contract(off)
    const unsigned i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const int tile = (int)a.fc_div.div(i);
    const int fc = (int)(i - (unsigned)tile * a.fc_div.d);
    const int f = (int)a.c_div.div((unsigned)fc), c = fc - f * a.C;
    const int t0 = tile * kScatterRecFrames;
    const int bt = (int)blockIdx.y / a.S, s = (int)blockIdx.y % a.S;
    const BinBands R = a.rec[f];
    const float* mb = a.masks + ((size_t)bt * a.S + s) * a.total_feat * a.T + 2 * c;
    const float2* zc = a.spec + (((size_t)bt * a.C + c) * a.T) * a.F + f;
    int tt[kScatterRecFrames];
    float2 z[kScatterRecFrames];
#pragma unroll
    for (int k = 0; k < kScatterRecFrames; k++) {
        tt[k] = min(t0 + k, a.T - 1);
        z[k] = zc[(size_t)tt[k] * a.F];
    }
    const float* r0 = mb + (size_t)R.feat_off[0] * a.T + R.col[0];
    const float* r1 = mb + (size_t)R.feat_off[1] * a.T + R.col[1];
    float2 m0[kScatterRecFrames], m1[kScatterRecFrames];
#pragma unroll
    for (int k = 0; k < kScatterRecFrames; k++) {
        m0[k] = *reinterpret_cast<const float2*>(r0 + (size_t)tt[k] * R.din[0]);
        m1[k] = *reinterpret_cast<const float2*>(r1 + (size_t)tt[k] * R.din[1]);
    }
    const int count = R.din[0] == 0 ? 0 : R.din[1] == 0 ? 1 : 2;
    // The sums in CSR order from +0.0; the quotient by max(count, 1) as div_rn, the IEEE quotient.
    const double d = count > 1 ? 2.0 : 1.0, rd = count > 1 ? 0.5 : 1.0;
    float2* oc = a.out + (((size_t)bt * a.S + s) * a.C + c) * a.T * a.F + f;
#pragma unroll
    for (int k = 0; k < kScatterRecFrames; k++) {
        if (t0 + k >= a.T) break;
        double ar = 0.0, ai = 0.0;
        if (count > 0) {
            ar += (double)m0[k].x;
            ai += (double)m0[k].y;
        }
        if (count > 1) {
            ar += (double)m1[k].x;
            ai += (double)m1[k].y;
        }
        float2 o = make_float2(0.f, 0.f);
        if (!(a.zero_dc && f == 0)) {
            const double qr = div_rn(ar, d, rd), qi = div_rn(ai, d, rd);
            const double zr = z[k].x, zi = z[k].y;
            o = make_float2((float)(zr * qr - zi * qi), (float)(zr * qi + zi * qr));
        }
        store_stream(oc + (size_t)(t0 + k) * a.F, o);
    }
}

// F-major: thread = frame of one (bin, channel); spectrum and output coalesced along t.
__global__ __launch_bounds__(256) void band_scatter_f_kernel(ScatterArgs a) {
    const int t = (int)(blockIdx.x * 256 + threadIdx.x);
    if (t >= a.T) return;
    const int f = (int)blockIdx.y;
    const int z3 = (int)blockIdx.z;                   // (bt * S + s) * C + c
    const int c = z3 % a.C, s = (z3 / a.C) % a.S, bt = z3 / (a.C * a.S);
    const float* mb = a.masks + ((size_t)bt * a.S + s) * a.total_feat * a.T;
    const float2 z = a.spec[(((size_t)bt * a.C + c) * a.F + f) * a.T + t];
    a.out[(((size_t)bt * a.S + s) * a.C + c) * a.F * a.T + (size_t)f * a.T + t] = masked_bin(a, mb, z, f, c, t);
}

// ----------------------------------------------------------------- band-split RMSNorm
// RMSNorm * gamma of every band's block at once (src/roformer.cpp:169-175 with rms at :96-98,
// eps kRmsEps = 1e-24 at :34): row t of band b is feat[feat_off[b] * T + t * dim_in(b) + i],
// i < dim_in(b) = size_b * C * 2. Band widths differ a lot (28 to 520 floats for the 60 mel
// bands), so each band gets its own shape: L_b lanes per frame (a power of two, enough for at
// most kBandNormPer float2 per lane, at most a wave) and 256 / L_b frames per block, which
// gives every block a similar payload. Blocks are numbered band after band; a block finds its
// band by binary search over the bands' first block. Each lane keeps its float2 in registers;
// the sum of squares is accumulated in double and reduced across the row's lanes, and
// y = (x * scale) * gamma in float with scale = 1 / sqrt(mean + eps) rounded once, the
// arithmetic of stx_rms_norm_mul.
constexpr int kBandNormPer = 4;
constexpr int kBandTable = 160;                      // bands per launch

struct BandNormArgs {
    const float* gamma[kBandTable];
    int first_block[kBandTable + 1];                 // of each band; [nb] = blocks of the launch
    unsigned char lanes_log2[kBandTable];
    const float* feat;
    float* out;
    const BandInfo* bands;
    long long total_feat;
    int T, C, b0, nb;                                // bands b0 .. b0 + nb - 1 in this launch
    float eps;
};
static_assert(sizeof(BandNormArgs) <= 4096, "band table exceeds the kernel argument space");

template <int V>
__global__ __launch_bounds__(256) void band_rms_norm_kernel(BandNormArgs a) {
    const int blk = (int)blockIdx.x;
    int lo = 0, hi = a.nb - 1;                       // last band whose first block <= blk
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.first_block[mid] <= blk) lo = mid;
        else hi = mid - 1;
    }
    const int bi = lo;
    const BandInfo info = a.bands[a.b0 + bi];
    const int d = info.size * a.C;                   // float2 per row
    const int lg = a.lanes_log2[bi], L = 1 << lg;
    const int lane = (int)threadIdx.x & (L - 1), rr = (int)threadIdx.x >> lg;
    const int t = (blk - a.first_block[bi]) * (256 >> lg) + rr;
    const long long base = (long long)blockIdx.y * a.total_feat * a.T + info.feat_off * a.T +
                           (long long)min(t, a.T - 1) * 2 * d;
    const float2* x = reinterpret_cast<const float2*>(a.feat + base);
    const float2* g = reinterpret_cast<const float2*>(a.gamma[bi]);
    const int nk = (d + L - 1) >> lg;                // float2 per lane, uniform over the block
    float2 v[V], gv[V];
#pragma unroll
    for (int k = 0; k < V; k++) {                    // clamped loads, all issued up front;
        if (k < nk) {                                // slots past nk are skipped uniformly
            const int q = min(lane + (k << lg), d - 1);
            v[k] = x[q];
            gv[k] = g[q];
        } else {
            v[k] = gv[k] = make_float2(0.f, 0.f);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < V; k++) {
        if (lane + (k << lg) < d) ss += (double)v[k].x * v[k].x + (double)v[k].y * v[k].y;
    }
    ss = lane_sum_dyn(ss, L);                        // stays inside the row's lanes
    const float scale = (float)(1.0 / sqrt(ss / (2.0 * d) + (double)a.eps));
    if (t >= a.T) return;
    float2* y = reinterpret_cast<float2*>(a.out + base);
#pragma unroll
    for (int k = 0; k < V; k++) {
        const int q = lane + (k << lg);
        if (k < nk && q < d) store_stream(y + q, make_float2((v[k].x * scale) * gv[k].x, (v[k].y * scale) * gv[k].y));
    }
}

// The same with 16-byte accesses, for an even channel count (every row and band block then
// starts on a float4) and 16-byte aligned buffers: L_b lanes per frame with at most
// kBandNormPer / 2 float4 per lane. Half the memory instructions of the float2 form for the same
// payload per lane; the sum of squares is added in (lane, float4) order instead of (lane,
// float2), so its rounding differs from that form's.
template <int V>
__global__ __launch_bounds__(256) void band_rms_norm_v4_kernel(BandNormArgs a) {
    const int blk = (int)blockIdx.x;
    int lo = 0, hi = a.nb - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.first_block[mid] <= blk) lo = mid;
        else hi = mid - 1;
    }
    const int bi = lo;
    const BandInfo info = a.bands[a.b0 + bi];
    const int d = info.size * a.C / 2;               // float4 per row
    const int lg = a.lanes_log2[bi], L = 1 << lg;
    const int lane = (int)threadIdx.x & (L - 1), rr = (int)threadIdx.x >> lg;
    const int t = (blk - a.first_block[bi]) * (256 >> lg) + rr;
    const long long base = (long long)blockIdx.y * a.total_feat * a.T + info.feat_off * a.T +
                           (long long)min(t, a.T - 1) * 4 * d;
    const float4* x = reinterpret_cast<const float4*>(a.feat + base);
    const float4* g = reinterpret_cast<const float4*>(a.gamma[bi]);
    const int nk = (d + L - 1) >> lg;
    float4 v[V], gv[V];
#pragma unroll
    for (int k = 0; k < V; k++) {
        if (k < nk) {
            const int q = min(lane + (k << lg), d - 1);
            v[k] = x[q];
            gv[k] = g[q];
        } else {
            v[k] = gv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < V; k++) {
        if (lane + (k << lg) < d)
            ss += ((double)v[k].x * v[k].x + (double)v[k].y * v[k].y) + ((double)v[k].z * v[k].z + (double)v[k].w * v[k].w);
    }
    ss = lane_sum_dyn(ss, L);
    const float scale = (float)(1.0 / sqrt(ss / (4.0 * d) + (double)a.eps));
    if (t >= a.T) return;
    float4* y = reinterpret_cast<float4*>(a.out + base);
#pragma unroll
    for (int k = 0; k < V; k++) {
        const int q = lane + (k << lg);
        if (k < nk && q < d)
            store_stream(y + q, make_float4((v[k].x * scale) * gv[k].x, (v[k].y * scale) * gv[k].y,
                                            (v[k].z * scale) * gv[k].z, (v[k].w * scale) * gv[k].w));
    }
}

// ------------------------------------------------------------------- mask-head GLU
// The GLU that ends every mask estimator (src/roformer.cpp:199-204): for stem s and band b the
// last layer's output h [T][2 * dim_in(b)] becomes m[t][i] = h[t][i] * sigmoid(h[t][dim_in + i]),
// written straight into the band's block of the stem's mask buffer, the layout the
// scatter-average reads. The stem's buffer is walked flat, kGluPer float2 per thread, each
// finding its band by binary search over the band starts staged in LDS; the sigmoid is the
// one of stx_glu, a / (1 + expf(-g)), so each band's result equals stx_glu on that band.
constexpr int kGluPer = 4;
constexpr int kGluTable = 448;                       // head pointers per launch

struct BandGluArgs {
    const float2* heads[kGluTable];                  // [stem - s0][band]
    float2* masks;                                   // [n_stems][total_feat * T / 2]
    const int* pair_off;                             // [n_bands + 1]
    const FastDiv* pair_div;                         // [n_bands]
    int total_pairs, T, n_bands, s0;
};
static_assert(sizeof(BandGluArgs) <= 4096, "head table exceeds the kernel argument space");

__device__ __forceinline__ float glu_gate(float a, float g) { return a / (1.0f + expf(-g)); }

// LDS: band starts [n_bands + 1] ints, then the stem's head pointers and the bands' divisors.
size_t glu_lds_bytes(int n_bands) {
    return (sizeof(int) * (n_bands + 1) + 7) / 8 * 8 + (sizeof(void*) + sizeof(FastDiv)) * n_bands;
}

__global__ __launch_bounds__(256) void band_mask_glu_kernel(BandGluArgs a) {
    extern __shared__ __align__(8) unsigned char lds[];
    const int B = a.n_bands;
    int* start = reinterpret_cast<int*>(lds);                                   // first float2 of each band
    const float2** ptr = reinterpret_cast<const float2**>(lds + (sizeof(int) * (B + 1) + 7) / 8 * 8);
    FastDiv* div = reinterpret_cast<FastDiv*>(ptr + B);
    const int si = (int)blockIdx.y;
    for (int b = (int)threadIdx.x; b <= B; b += 256) {
        start[b] = a.pair_off[b] * a.T;
        if (b < B) {
            ptr[b] = a.heads[si * B + b];
            div[b] = a.pair_div[b];
        }
    }
    __syncthreads();
    const int n = a.total_pairs * a.T;
    float2* out = a.masks + (long long)(a.s0 + si) * n;
    const int e0 = (int)blockIdx.x * (256 * kGluPer) + (int)threadIdx.x;
    if (e0 >= n) return;
    // Pointers read back from LDS are generic to the compiler; flat loads would also count on the
    // LDS counter and serialise against the next search, so they are cast back to global.
    typedef float f2 __attribute__((ext_vector_type(2)));
    using gf2 = __attribute__((address_space(1))) const f2;
    gf2* src0[kGluPer];
    gf2* src1[kGluPer];
#pragma unroll
    for (int k = 0; k < kGluPer; k++) {                // LDS only: band, frame and column
        const int e = min(e0 + 256 * k, n - 1);
        int lo = 0, hi = B - 1;                      // last band with start <= e
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (start[mid] <= e) lo = mid;
            else hi = mid - 1;
        }
        const FastDiv dv = div[lo];
        const unsigned local = (unsigned)(e - start[lo]);
        const unsigned t = dv.div(local), j = local - t * dv.d;
        gf2* row = (gf2*)(ptr[lo] + (size_t)t * 2 * dv.d);
        src0[k] = row + j;
        src1[k] = row + dv.d + j;
    }
    f2 h0[kGluPer], h1[kGluPer];
#pragma unroll
    for (int k = 0; k < kGluPer; k++) {                // then every load at once
        h0[k] = *src0[k];
        h1[k] = *src1[k];
    }
#pragma unroll
    for (int k = 0; k < kGluPer; k++) {
        const int e = e0 + 256 * k;
        if (e < n) store_stream(out + e, make_float2(glu_gate(h0[k].x, h1[k].x), glu_gate(h0[k].y, h1[k].y)));
    }
}

void check_bands(const stx_bands* b) { STX_REQUIRE(b != nullptr && b->d_bands != nullptr, "null band table"); }

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_bands_create(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs,
                                    int64_t n_freqs, int n_bins, int channels, stx_bands** out) {
    return guard([&] {
        STX_REQUIRE(out != nullptr, "out is NULL");
        *out = nullptr;
        std::vector<int64_t> fo, fe;
        std::vector<int32_t> bpf;
        check_band_tables(band_sizes, n_bands, band_freqs, n_freqs, n_bins, channels, fo, fe, bpf);
        STX_REQUIRE(fe.back() < (1LL << 40) && n_freqs < (1LL << 31), "band table too large");
        std::vector<BandInfo> bi(n_bands);
        int max_pairs = 0;
        for (int b = 0; b < n_bands; b++) {
            bi[b] = BandInfo{(long long)fe[b], (int)fo[b], band_sizes[b]};
            max_pairs = std::max(max_pairs, band_sizes[b] * channels);
        }
        // CSR of (band, position) pairs per bin, in band then position order.
        std::vector<int> csr_off(n_bins + 1, 0);
        for (int64_t i = 0; i < n_freqs; i++) csr_off[band_freqs[i] + 1]++;
        for (int f = 0; f < n_bins; f++) csr_off[f + 1] += csr_off[f];
        std::vector<CsrEntry> csr(std::max<int64_t>(n_freqs, 1));
        std::vector<int> fill(csr_off.begin(), csr_off.end() - 1);
        for (int b = 0; b < n_bands; b++)
            for (int j = 0; j < band_sizes[b]; j++) {
                const int f = band_freqs[fo[b] + j];
                csr[fill[f]++] = CsrEntry{(long long)fe[b], band_sizes[b] * channels * 2, j * channels * 2};
            }
        // Per (bin, channel) pair of every band, in feature order: (channel << 16) | bin.
        STX_REQUIRE(n_bins < 65536 && channels < 32768, "band table: n_bins or channels too large");
        std::vector<int> pair_off(n_bands + 1, 0), pair_code;
        pair_code.reserve((size_t)(fe.back() / 2));
        for (int b = 0; b < n_bands; b++) {
            pair_off[b] = (int)(fe[b] / 2);
            for (int j = 0; j < band_sizes[b]; j++)
                for (int c = 0; c < channels; c++) pair_code.push_back((c << 16) | band_freqs[fo[b] + j]);
        }
        pair_off[n_bands] = (int)(fe.back() / 2);
        std::vector<int> freq_lo(n_bands, 0);
        bool ranges = true;
        for (int b = 0; b < n_bands; b++) {
            freq_lo[b] = band_sizes[b] > 0 ? band_freqs[fo[b]] : 0;
            for (int j = 1; j < band_sizes[b]; j++) ranges = ranges && band_freqs[fo[b] + j] == freq_lo[b] + j;
        }
        std::vector<double> denom(n_bins);
        for (int f = 0; f < n_bins; f++) denom[f] = (double)std::max(bpf[f], 1);   // src/roformer.cpp:272
        // Per-bin records when every bin has at most two pairs and the offsets fit their fields.
        bool records = fe.back() >= 2LL * channels && fe.back() < (1LL << 31);
        for (int f = 0; f < n_bins && records; f++) records = bpf[f] <= 2;
        for (int b = 0; b < n_bands && records; b++) records = band_sizes[b] * (long long)channels * 2 < 65536;
        std::vector<GatherRec> grec;
        bool gather_records = fe.back() / 2 / channels < (1LL << 31);
        for (int b = 0; b < n_bands && gather_records; b++) gather_records = band_sizes[b] < 65536;
        if (gather_records) {
            grec.reserve((size_t)n_freqs);
            for (int b = 0; b < n_bands; b++)
                for (int j = 0; j < band_sizes[b]; j++)
                    grec.push_back(GatherRec{(int)fo[b], (unsigned short)band_sizes[b],
                                             (unsigned short)band_freqs[fo[b] + j]});
        }
        std::vector<BinBands> rec;
        if (records) {
            rec.assign(n_bins, BinBands{{0, 0}, {0, 0}, {0, 0}});
            for (int f = 0; f < n_bins; f++) {
                BinBands& r = rec[f];
                for (int k = 0; k < 2; k++) {
                    const int e = std::min(csr_off[f] + k, csr_off[f + 1] - 1);   // a missing pair repeats entry 0
                    if (e < csr_off[f]) break;
                    r.feat_off[k] = (int)csr[e].feat_off;
                    r.col[k] = (unsigned short)csr[e].col;
                    r.din[k] = csr_off[f] + k < csr_off[f + 1] ? (unsigned short)csr[e].din : 0;
                }
            }
        }

        stx_bands* h = new stx_bands;
        h->n_bands = n_bands;
        h->n_bins = n_bins;
        h->channels = channels;
        h->n_freqs = n_freqs;
        h->total_feat = fe.back();
        h->max_pairs = max_pairs;
        h->freq_off = fo;
        h->feat_off = fe;
        h->bpf = bpf;
        hipError_t e = hipSuccess;
        auto up = [&](auto** dst, const auto& v) {
            using T = std::remove_reference_t<decltype(v[0])>;
            if (e == hipSuccess) e = hipMalloc(dst, sizeof(T) * std::max<size_t>(v.size(), 1));
            if (e == hipSuccess && !v.empty())
                e = hipMemcpy(*dst, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice);
        };
        std::vector<int> bf(band_freqs, band_freqs + n_freqs);
        up(&h->d_bands, bi);
        up(&h->d_band_freqs, bf);
        up(&h->d_csr_off, csr_off);
        up(&h->d_csr, csr);
        up(&h->d_denom, denom);
        if (records) up(&h->d_bin_bands, rec);
        if (gather_records && n_freqs > 0) up(&h->d_gather_rec, grec);
        up(&h->d_pair_off, pair_off);
        up(&h->d_pair_code, pair_code);
        up(&h->d_freq_lo, freq_lo);
        std::vector<FastDiv> pair_div(n_bands);
        for (int b = 0; b < n_bands; b++) pair_div[b] = FastDiv((unsigned)std::max(band_sizes[b] * channels, 1));
        up(&h->d_pair_div, pair_div);
        h->ranges = ranges;
        if (e != hipSuccess) {
            stx_bands_destroy(h);
            hip_check(e, "stx_bands_create");
        }
        *out = h;
    });
}

STX_API void stx_bands_destroy(stx_bands* h) {
    if (!h) return;
    (void)hipFree(h->d_bands);
    (void)hipFree(h->d_band_freqs);
    (void)hipFree(h->d_csr_off);
    (void)hipFree(h->d_csr);
    (void)hipFree(h->d_denom);
    (void)hipFree(h->d_bin_bands);
    (void)hipFree(h->d_gather_rec);
    (void)hipFree(h->d_pair_off);
    (void)hipFree(h->d_pair_code);
    (void)hipFree(h->d_freq_lo);
    (void)hipFree(h->d_pair_div);
    delete h;
}

STX_API int64_t stx_bands_total_feat(const stx_bands* h) { return h ? h->total_feat : 0; }

STX_API stx_status stx_band_gather(const stx_bands* h, const float* spec, int batch, int n_frames,
                                   stx_spec_layout layout, float* feat, stx_stream stream) {
    return guard([&] {
        check_bands(h);
        STX_REQUIRE(layout == STX_SPEC_F_MAJOR || layout == STX_SPEC_T_MAJOR, "unknown spectrum layout");
        STX_REQUIRE(batch >= 0 && n_frames >= 0, "bad batch/n_frames");
        if (batch == 0 || n_frames == 0 || h->total_feat == 0) return;
        STX_REQUIRE(spec && feat, "NULL buffer");
        STX_REQUIRE(n_frames < 65536 && batch < 65536, "too many frames or batch items");
        GatherArgs a{};
        a.spec = reinterpret_cast<const float2*>(spec);
        a.feat = reinterpret_cast<float2*>(feat);
        a.bands = h->d_bands;
        a.band_freqs = h->d_band_freqs;
        a.C = h->channels;
        a.F = h->n_bins;
        a.T = n_frames;
        a.total_feat = h->total_feat;
        a.pair_off = h->d_pair_off;
        a.pair_code = h->d_pair_code;
        a.freq_lo = h->d_freq_lo;
        a.n_bands = h->n_bands;
        const hipStream_t s = as_stream(stream);
        const size_t row_bytes = sizeof(float2) * (size_t)a.C * a.F;
        const bool aligned = a.C != 2 || reinterpret_cast<uintptr_t>(feat) % 16 == 0;
        if (layout == STX_SPEC_T_MAJOR && h->d_gather_rec && row_bytes <= 65536 && aligned) {
            a.rec = h->d_gather_rec;
            a.n_entries = (int)h->n_freqs;
            a.fdiv = FastDiv((unsigned)a.F);
            const dim3 grid(xcd_grid(n_frames), batch);
            if (a.C == 1) launch_gather_frame<1>(a, grid, row_bytes, s);
            else if (a.C == 2) launch_gather_frame<2>(a, grid, row_bytes, s);
            else launch_gather_frame<0>(a, grid, row_bytes, s);
            launch_check("band_gather_frame_kernel");
            return;
        }
        if (layout == STX_SPEC_T_MAJOR) {
            const long long n = h->total_feat / 2 * (long long)n_frames;
            STX_REQUIRE(n < (1LL << 31) - 256 * kGatherPer, "band gather: too many features per chunk");
            if (h->n_bands > 8191) fail(STX_STATUS_UNSUPPORTED, "T-major band gather: more than 8191 bands");
            dim3 grid((unsigned)((n + 256 * kGatherPer - 1) / (256 * kGatherPer)), batch);
            const size_t lds = sizeof(int) * (2 * (size_t)h->n_bands + 1) + sizeof(FastDiv) * (size_t)h->n_bands;
            a.pair_div = h->d_pair_div;
            a.cdiv = FastDiv((unsigned)a.C);
            if (h->ranges) hipLaunchKernelGGL(band_gather_t_kernel<true>, grid, dim3(256), lds, s, a);
            else hipLaunchKernelGGL(band_gather_t_kernel<false>, grid, dim3(256), lds, s, a);
            launch_check("band_gather_t_kernel");
            return;
        }
        // LDS tile [max_pairs][TT + 1] float2 within 64 KB.
        int TT = 32;
        while (TT > 1 && (size_t)h->max_pairs * (TT + 1) * sizeof(float2) > 65536) TT /= 2;
        if ((size_t)h->max_pairs * (TT + 1) * sizeof(float2) > 65536)
            fail(STX_STATUS_UNSUPPORTED, "band of %d (bin, channel) pairs is too wide for the F-major gather",
                 h->max_pairs);
        a.TT = TT;
        dim3 grid(h->n_bands, (n_frames + TT - 1) / TT, batch);
        hipLaunchKernelGGL(band_gather_f_kernel, grid, dim3(256), (size_t)h->max_pairs * (TT + 1) * sizeof(float2),
                           s, a);
        launch_check("band_gather_f_kernel");
    });
}

STX_API stx_status stx_band_scatter_apply(const stx_bands* h, const float* masks, int n_stems, const float* spec,
                                          int batch, int n_frames, stx_spec_layout layout, int zero_dc, float* out,
                                          stx_stream stream) {
    return guard([&] {
        check_bands(h);
        STX_REQUIRE(layout == STX_SPEC_F_MAJOR || layout == STX_SPEC_T_MAJOR, "unknown spectrum layout");
        STX_REQUIRE(batch >= 0 && n_frames >= 0 && n_stems >= 0, "bad batch/n_frames/n_stems");
        if (batch == 0 || n_frames == 0 || n_stems == 0) return;
        STX_REQUIRE(masks && spec && out, "NULL buffer");
        STX_REQUIRE(n_frames < 65536 && (long long)batch * n_stems * h->channels < 65536, "grid too large");
        ScatterArgs a{};
        a.masks = masks;
        a.spec = reinterpret_cast<const float2*>(spec);
        a.out = reinterpret_cast<float2*>(out);
        a.csr_off = h->d_csr_off;
        a.csr = h->d_csr;
        a.denom = h->d_denom;
        a.C = h->channels;
        a.F = h->n_bins;
        a.T = n_frames;
        a.S = n_stems;
        a.zero_dc = zero_dc ? 1 : 0;
        a.total_feat = h->total_feat;
        const hipStream_t s = as_stream(stream);
        const long long tiles = (n_frames + kScatterFrames - 1) / kScatterFrames;
        const long long rec_tiles = (n_frames + kScatterRecFrames - 1) / kScatterRecFrames;
        if (layout == STX_SPEC_T_MAJOR && h->d_bin_bands && rec_tiles * a.F * a.C < (1LL << 32) - 256) {
            const unsigned n = (unsigned)(rec_tiles * a.F * a.C);
            a.rec = h->d_bin_bands;
            a.fc_div = FastDiv((unsigned)(a.F * a.C));
            a.c_div = FastDiv((unsigned)a.C);
            const dim3 grid((n + 255) / 256, batch * n_stems);
            hipLaunchKernelGGL(band_scatter_rec_kernel, grid, dim3(256), 0, s, a, n);
            launch_check("band_scatter_rec_kernel");
        } else if (layout == STX_SPEC_T_MAJOR) {
            dim3 grid((a.F * a.C + 255) / 256, (unsigned)tiles, batch * n_stems);
            hipLaunchKernelGGL(band_scatter_t_kernel, grid, dim3(256), 0, s, a);
            launch_check("band_scatter_t_kernel");
        } else {
            dim3 grid((n_frames + 255) / 256, a.F, batch * n_stems * a.C);
            hipLaunchKernelGGL(band_scatter_f_kernel, grid, dim3(256), 0, s, a);
            launch_check("band_scatter_f_kernel");
        }
    });
}

STX_API stx_status stx_band_rms_norm(const stx_bands* h, const float* feat, int batch, int n_frames,
                                     const float* const* gammas, float eps, float* out, stx_stream stream) {
    return guard([&] {
        check_bands(h);
        STX_REQUIRE(batch >= 0 && n_frames >= 0, "bad batch/n_frames");
        if (batch == 0 || n_frames == 0 || h->total_feat == 0) return;
        STX_REQUIRE(feat && out && gammas, "NULL buffer");
        STX_REQUIRE(batch < 65536, "too many batch items");
        for (int b = 0; b < h->n_bands; b++) {
            const long long d = (h->feat_off[b + 1] - h->feat_off[b]) / 2;
            STX_REQUIRE(d == 0 || gammas[b] != nullptr, "band_rms_norm: gamma of band %d is NULL", b);
            if (d > 64LL * 16)
                fail(STX_STATUS_UNSUPPORTED, "band_rms_norm: band %d has %lld floats per frame (at most 2048)", b,
                     2 * d);
        }
        const hipStream_t s = as_stream(stream);
        for (int b0 = 0; b0 < h->n_bands; b0 += kBandTable) {
            BandNormArgs a{};
            a.feat = feat;
            a.out = out;
            a.bands = h->d_bands;
            a.total_feat = h->total_feat;
            a.T = n_frames;
            a.C = h->channels;
            a.b0 = b0;
            a.eps = eps;
            long long blocks = 0;
            int max_nk = 1;
            const int nb = std::min(kBandTable, h->n_bands - b0);
            // 16-byte accesses when every row starts on a float4 (an even channel count) and
            // every buffer is 16-byte aligned.
            bool v4 = h->channels % 2 == 0 && (reinterpret_cast<uintptr_t>(feat) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(out) & 15) == 0;
            for (int i = 0; i < nb; i++) v4 = v4 && (reinterpret_cast<uintptr_t>(gammas[b0 + i]) & 15) == 0;
            const int unit = v4 ? 4 : 2;                 // floats per access
            const int per = v4 ? kBandNormPer / 2 : kBandNormPer;
            for (int i = 0; i < nb; i++) {
                const int d = (int)((h->feat_off[b0 + i + 1] - h->feat_off[b0 + i]) / unit);
                int lg = 0;
                while ((1 << lg) < 64 && (1 << lg) * per < d) lg++;
                a.gamma[i] = gammas[b0 + i];
                a.lanes_log2[i] = (unsigned char)lg;
                a.first_block[i] = (int)blocks;      // an empty band gets no blocks: the search skips it
                if (d > 0) blocks += (n_frames + (256 >> lg) - 1) / (256 >> lg);
                max_nk = std::max(max_nk, (d + (1 << lg) - 1) >> lg);
            }
            if (blocks == 0) continue;
            STX_REQUIRE(blocks < (1LL << 31), "band_rms_norm: too many frames");
            a.first_block[nb] = (int)blocks;
            a.nb = nb;
            const dim3 grid((unsigned)blocks, (unsigned)batch);
            if (v4) {
                if (max_nk <= 2) hipLaunchKernelGGL(band_rms_norm_v4_kernel<2>, grid, dim3(256), 0, s, a);
                else if (max_nk <= 4) hipLaunchKernelGGL(band_rms_norm_v4_kernel<4>, grid, dim3(256), 0, s, a);
                else hipLaunchKernelGGL(band_rms_norm_v4_kernel<8>, grid, dim3(256), 0, s, a);
            } else if (max_nk <= 4) {
                hipLaunchKernelGGL(band_rms_norm_kernel<4>, grid, dim3(256), 0, s, a);
            } else if (max_nk <= 8) {
                hipLaunchKernelGGL(band_rms_norm_kernel<8>, grid, dim3(256), 0, s, a);
            } else {
                hipLaunchKernelGGL(band_rms_norm_kernel<16>, grid, dim3(256), 0, s, a);
            }
            launch_check("band_rms_norm_kernel");
        }
    });
}

STX_API stx_status stx_band_mask_glu(const stx_bands* h, const float* const* heads, int n_stems, int n_frames,
                                     float* masks, stx_stream stream) {
    return guard([&] {
        check_bands(h);
        STX_REQUIRE(n_stems >= 0 && n_frames >= 0, "bad n_stems/n_frames");
        if (n_stems == 0 || n_frames == 0 || h->total_feat == 0) return;
        STX_REQUIRE(heads && masks, "NULL buffer");
        const int B = h->n_bands;
        for (long long i = 0; i < (long long)n_stems * B; i++) {
            const bool empty = h->feat_off[i % B + 1] == h->feat_off[i % B];
            STX_REQUIRE(empty || heads[i] != nullptr, "band_mask_glu: head %lld is NULL", i);
        }
        const long long n = h->total_feat / 2 * (long long)n_frames;
        STX_REQUIRE(n < (1LL << 31) - 256 * kGluPer, "band_mask_glu: too many features per stem");
        if (B > kGluTable) fail(STX_STATUS_UNSUPPORTED, "band_mask_glu: more than %d bands", kGluTable);
        const int per_launch = kGluTable / B;
        const hipStream_t s = as_stream(stream);
        for (int s0 = 0; s0 < n_stems; s0 += per_launch) {
            const int ns = std::min(per_launch, n_stems - s0);
            STX_REQUIRE(ns < 65536, "too many stems");
            BandGluArgs a{};
            for (int i = 0; i < ns * B; i++) a.heads[i] = reinterpret_cast<const float2*>(heads[(long long)s0 * B + i]);
            a.masks = reinterpret_cast<float2*>(masks);
            a.pair_off = h->d_pair_off;
            a.pair_div = h->d_pair_div;
            a.total_pairs = (int)(h->total_feat / 2);
            a.T = n_frames;
            a.n_bands = B;
            a.s0 = s0;
            const dim3 grid((unsigned)((n + 256 * kGluPer - 1) / (256 * kGluPer)), (unsigned)ns);
            hipLaunchKernelGGL(band_mask_glu_kernel, grid, dim3(256), glu_lds_bytes(B), s, a);
            launch_check("band_mask_glu_kernel");
        }
    });
}

}  // extern "C"
