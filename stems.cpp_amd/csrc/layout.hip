// layout.hip — the layout glue around RoFormer attention and the band split, as gfx950
// kernels that move each element through HBM once instead of once per ggml node:
//
//   qkv split + RoPE + permute   src/roformer.cpp:101-112 (part(i) = cont(view), rope_ext,
//                                cont(permute(.., 0,2,1,3)) for q and k, cont(permute(.., 1,2,0,3))
//                                for v)
//   head merge (* gates)         src/roformer.cpp:132-137 (cont(permute(o, 0,2,1,3)), mul by
//                                reshape_4d(gates, 1, H, N, batch))
//   cont(permute(a, ...))        src/roformer.cpp:112,133,182,184,190
//   concat of many tensors       src/roformer.cpp:52-60 (concat_all: a tree of ggml_concat),
//                                :132 (attention batch groups), :178 (band split)
//
// All of it is pure data movement plus the RoPE rotation, so every kernel is HBM-bound: loads
// and stores are whole 64-float runs per wave (256 contiguous bytes), and the transposes go
// through an LDS tile with one float of padding per row so that both the row-wise write and
// the column-wise read hit 64 different banks.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.hpp"
#include "tensor.hpp"

namespace stx {
namespace {

// ------------------------------------------------------------------- qkv split + RoPE
// qkv is the output of the fused q/k/v projection, [3*H*dh, N, batch]: each position's row
// holds q (heads 0..H-1), then k, then v, dh floats per head ('b n (qkv h d)'). Outputs, all
// dense:
//   q, k  [dh, N, H, batch]  rope_ext(part(i), pos, n_dims = dh, mode 0) permuted (0,2,1,3)
//   vt    [N, dh, H, batch]  part(2) permuted (1,2,0,3)
// A block takes kSplitTile positions and a run of (head, batch) units. Each thread owns one
// float4 (two rotation pairs) of kSplitTile / RPP rows, so the cos/sin of its pairs are
// evaluated once per block and kept in registers for every unit; q and k rows go straight out
// (256 contiguous bytes per head row), v goes through a double-buffered LDS tile and leaves
// along N. The rotation is the one of stx_rope_ext (theta = freq_scale * pos *
// freq_base^(-2i/dh), cos/sin in double times attn_factor, rotated in double and rounded
// once), so q and k are bit-identical to rope_ext on the view followed by the permute.
constexpr int kSplitTile = 64;
constexpr int kSplitBlocksPerCu = 16;

struct QkvArgs {
    const char* qkv;
    long long nb1, nb2;          // qkv byte strides of a position and of a batch entry
    float* q;
    float* k;
    float* vt;
    const int* pos;              // [N]
    int n, heads, units;         // units = heads * batch
    int units_per_block;
    int tiles, blocks;           // position tiles; tiles * unit groups
    double freq_base, freq_scale, attn_factor;
};

__device__ __forceinline__ float4 rotate_pairs(float4 v, double c0, double s0, double c1, double s1) {
    float4 o;
    o.x = (float)((double)v.x * c0 - (double)v.y * s0);
    o.y = (float)((double)v.x * s0 + (double)v.y * c0);
    o.z = (float)((double)v.z * c1 - (double)v.w * s1);
    o.w = (float)((double)v.z * s1 + (double)v.w * c1);
    return o;
}

template <int DH>
__global__ __launch_bounds__(256) void qkv_rope_split_kernel(QkvArgs a) {
    constexpr int R4 = DH / 4;                  // float4s per head row
    constexpr int RPP = 256 / R4;               // rows per pass of the block
    constexpr int P = kSplitTile / RPP;         // passes over the tile
    constexpr int NBUF = DH <= 64 ? 2 : 1;     // LDS buffers for the v tile (64 KB of static LDS at most)
    static_assert(DH % 4 == 0 && 256 % R4 == 0 && kSplitTile % RPP == 0, "tile shape");
    __shared__ float tile[NBUF][DH][kSplitTile + 1];

    // Logical block = unit group * tiles + tile, laid out so each XCD runs a contiguous range:
    // the tiles of one unit group then share an L2, which merges the partial 128-byte lines
    // where neighbouring tiles meet in a vt row.
    const int lb = xcd_block();
    if (lb >= a.blocks) return;
    const int t = (int)threadIdx.x;
    const int q4 = t % R4, rr = t / R4;
    const int group = lb / a.tiles;
    const int n0 = (lb - group * a.tiles) * kSplitTile;
    const int u0 = group * a.units_per_block;
    const int u1 = min(u0 + a.units_per_block, a.units);
    const int H = a.heads, N = a.n;

    int row[P];
    bool ok[P];
    int pv[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int n = n0 + rr + RPP * p;
        ok[p] = n < N;
        row[p] = min(n, N - 1);
        pv[p] = a.pos[row[p]];                  // issued before the first unit's data
    }
    double c0[P], s0[P], c1[P], s1[P];
    const int nn = t % kSplitTile, dd = t / kSplitTile;

    for (int u = u0; u < u1; u++) {
        const int b = u / H, h = u - b * H;
        const char* base = a.qkv + (long long)b * a.nb2;
        float4 xq[P], xk[P], xv[P];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const float4* r = reinterpret_cast<const float4*>(base + (long long)row[p] * a.nb1);
            xq[p] = r[h * R4 + q4];
            xk[p] = r[(H + h) * R4 + q4];
            xv[p] = r[(2 * H + h) * R4 + q4];
        }
        if (u == u0) {                          // overlaps the first unit's loads
            const double pw0 = pow(a.freq_base, -2.0 * (2 * q4) / DH);
            const double pw1 = pow(a.freq_base, -2.0 * (2 * q4 + 1) / DH);
#pragma unroll
            for (int p = 0; p < P; p++) {
                const double fp = a.freq_scale * (double)pv[p];
                double sn, cn;
                sincos(fp * pw0, &sn, &cn);
                c0[p] = cn * a.attn_factor;
                s0[p] = sn * a.attn_factor;
                sincos(fp * pw1, &sn, &cn);
                c1[p] = cn * a.attn_factor;
                s1[p] = sn * a.attn_factor;
            }
        }
        const long long head = (long long)u * N;     // (b * H + h) * N
        float* qo = a.q + head * DH + 4 * q4;
        float* ko = a.k + head * DH + 4 * q4;
        const int buf = NBUF == 2 ? (u - u0) & 1 : 0;
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int n = n0 + rr + RPP * p;
            if (ok[p]) {
                store_stream(reinterpret_cast<float4*>(qo + (long long)n * DH), rotate_pairs(xq[p], c0[p], s0[p], c1[p], s1[p]));
                store_stream(reinterpret_cast<float4*>(ko + (long long)n * DH), rotate_pairs(xk[p], c0[p], s0[p], c1[p], s1[p]));
            }
            tile[buf][4 * q4 + 0][rr + RPP * p] = xv[p].x;
            tile[buf][4 * q4 + 1][rr + RPP * p] = xv[p].y;
            tile[buf][4 * q4 + 2][rr + RPP * p] = xv[p].z;
            tile[buf][4 * q4 + 3][rr + RPP * p] = xv[p].w;
        }
        __syncthreads();                        // with two buffers, one is rewritten only after the next barrier
        float* vo = a.vt + (long long)u * DH * N + n0 + nn;
        if (n0 + nn < N) {
#pragma unroll
            for (int j = 0; j < DH / 4; j++) {
                const int d = dd + 4 * j;
                store_stream(vo + (long long)d * N, tile[buf][d][nn]);
            }
        }
        if (NBUF == 1) __syncthreads();
    }
}

template <int DH>
void launch_qkv_split(QkvArgs a, hipStream_t s) {
    const int tiles = (a.n + kSplitTile - 1) / kSplitTile;
    const long long target = (long long)device_cus() * kSplitBlocksPerCu;
    long long per = std::max<long long>(1, ((long long)tiles * a.units + target - 1) / target);
    a.units_per_block = (int)per;
    a.tiles = tiles;
    const long long blocks = (long long)tiles * ((a.units + per - 1) / per);
    STX_REQUIRE(blocks < (1LL << 31) - kXcds, "qkv_rope_split: too many blocks");
    a.blocks = (int)blocks;
    hipLaunchKernelGGL((qkv_rope_split_kernel<DH>), dim3(xcd_grid(blocks)), dim3(256), 0, s, a);
    launch_check("qkv_rope_split_kernel");
}

// ------------------------------------------------------------------ permute (rows kept)
// dst = cont(permute(src)) when dimension 0 stays in place: every dst row (i1, i2, i3) is a
// src row, found through the src strides of the dimensions that land on dst 1..3. Optionally
// each row is multiplied by a per-row scalar gate[i1, i2, i3] (ggml_mul with a [1, ...]
// operand: one rounding). Each thread moves kRowUnits float4s (or floats) of consecutive
// blocks of 256, all loaded before any is stored.
constexpr int kRowUnits = 4;

struct RowPermArgs {
    const char* src;
    long long s1, s2, s3;        // src byte stride of the dimension that lands on dst 1, 2, 3
    char* dst;
    long long d1, d2, d3;        // dst byte strides
    const char* gate;            // NULL or [1, ne1, ne2, ne3]
    long long g1, g2, g3;
    unsigned count;              // units (float4 or float) in dst
    FastDiv dq, dn1, dn2;        // units per row, dst ne1, dst ne2
};

template <bool V4, bool GATE>
__global__ __launch_bounds__(256) void permute_rows_kernel(RowPermArgs a) {
    using U = typename std::conditional<V4, float4, float>::type;
    constexpr int W = V4 ? 16 : 4;
    const unsigned e0 = blockIdx.x * (256u * kRowUnits) + threadIdx.x;
    U v[kRowUnits];
    long long doff[kRowUnits];
    float g[kRowUnits];
#pragma unroll
    for (int u = 0; u < kRowUnits; u++) {
        const unsigned e = min(e0 + 256u * u, a.count - 1);      // clamped; stores are skipped
        const unsigned r = a.dq.div(e), q = e - r * a.dq.d;
        const unsigned r2 = a.dn1.div(r), i1 = r - r2 * a.dn1.d;
        const unsigned i3 = a.dn2.div(r2), i2 = r2 - i3 * a.dn2.d;
        v[u] = *reinterpret_cast<const U*>(a.src + i1 * a.s1 + i2 * a.s2 + i3 * a.s3 + (long long)q * W);
        doff[u] = i1 * a.d1 + i2 * a.d2 + i3 * a.d3 + (long long)q * W;
        if (GATE) g[u] = *reinterpret_cast<const float*>(a.gate + i1 * a.g1 + i2 * a.g2 + i3 * a.g3);
    }
#pragma unroll
    for (int u = 0; u < kRowUnits; u++) {
        if (e0 + 256u * u >= a.count) break;
        U o = v[u];
        if constexpr (GATE) {
            if constexpr (V4) {
                o.x *= g[u];
                o.y *= g[u];
                o.z *= g[u];
                o.w *= g[u];
            } else {
                o *= g[u];
            }
        }
        store_stream(reinterpret_cast<U*>(a.dst + doff[u]), o);
    }
}

// -------------------------------------------------------------- permute (transposing)
// dst = cont(permute(src)) when src dimension 0 moves to dst dimension `pa` != 0 and dst
// dimension 0 comes from src dimension `s`: 64 x 64 tiles of (src 0, src s) go through LDS,
// read along src 0 and written along dst 0, one float per lane, 256 contiguous bytes per wave
// on both sides. Logical blocks run over (tile along s, tile along 0, the two remaining
// dimensions), fastest first, each XCD taking a contiguous range, so the tiles that meet inside
// a dst row (where a 64-float run rarely starts on a 128-byte line) share an L2.
constexpr int kTile = 64;

struct TransArgs {
    const char* src;
    char* dst;
    int na, nbb;                 // extents of src dim 0 (A) and src dim s (B)
    int tiles_a, tiles_b, blocks;
    long long sb, da;            // src byte stride of B, dst byte stride of A
    int nc1, nc2;                // extents of the two other dims
    long long sc1, sc2, dc1, dc2;
};

__global__ __launch_bounds__(256) void transpose_kernel(TransArgs a) {
    __shared__ float tile[kTile][kTile + 1];     // [b][a]
    const int lb = xcd_block();
    if (lb >= a.blocks) return;                    // uniform over the block
    const int lane = (int)threadIdx.x % kTile, w = (int)threadIdx.x / kTile;
    int rest = lb;
    const int tb = rest % a.tiles_b;
    rest /= a.tiles_b;
    const int ta = rest % a.tiles_a;
    rest /= a.tiles_a;
    const int c1 = rest % a.nc1, c2 = rest / a.nc1;
    const int a0 = ta * kTile, b0 = tb * kTile;
    const char* s = a.src + c1 * a.sc1 + c2 * a.sc2;
    char* d = a.dst + c1 * a.dc1 + c2 * a.dc2;
    float v[kTile / 4];
    const int ia = min(a0 + lane, a.na - 1);
#pragma unroll
    for (int j = 0; j < kTile / 4; j++) {
        const int ib = min(b0 + w + 4 * j, a.nbb - 1);
        v[j] = *reinterpret_cast<const float*>(s + ib * a.sb + (long long)ia * 4);
    }
#pragma unroll
    for (int j = 0; j < kTile / 4; j++) tile[w + 4 * j][lane] = v[j];
    __syncthreads();
    const int ob = b0 + lane;
    if (ob < a.nbb) {
#pragma unroll
        for (int j = 0; j < kTile / 4; j++) {
            const int oa = a0 + w + 4 * j;
            if (oa < a.na) store_stream(reinterpret_cast<float*>(d + oa * a.da + (long long)ob * 4), tile[lane][w + 4 * j]);
        }
    }
}

// --------------------------------------------------------------------------- concat
// ggml_concat along `dim` of up to kConcatMax sources per launch: each source is copied into its slice of dst, element (i0, i1, i2, i3) to the same
// index shifted along `dim`, so a tree of pairwise concats (concat_all) becomes one pass. The
// sources share every extent but the one along `dim`, so each carries only its own divisor for
// that one; the table fits the 4 KB of kernel arguments.
constexpr int kConcatMax = 64;
constexpr int kConcatUnits = 4;

struct ConcatSrc {
    const char* data;
    long long nb1, nb2, nb3;
    long long dst_off;           // byte offset of this source's slice in dst
    FastDiv along;               // this source's extent along dim (in units when dim is 0)
    unsigned count;              // units (float4 or float)
};

struct ConcatArgs {
    char* dst;
    long long d1, d2, d3;
    FastDiv dq, dn1, dn2;        // units per row, ne1, ne2 shared by every source (but along dim)
    int dim;
    unsigned n_src;
    ConcatSrc src[kConcatMax];
};
static_assert(sizeof(ConcatArgs) <= 4096, "concat table exceeds the kernel argument space");

template <bool V4>
__global__ __launch_bounds__(256) void concat_kernel(ConcatArgs a) {
    using U = typename std::conditional<V4, float4, float>::type;
    constexpr int W = V4 ? 16 : 4;
    // Source fastest: the blocks in flight at once cover every source's slice of a few dst
    // rows, so the writes sweep dst nearly in order.
    const unsigned src = blockIdx.x % a.n_src, chunk = blockIdx.x / a.n_src;
    const ConcatSrc& s = a.src[src];
    const unsigned e0 = chunk * (256u * kConcatUnits) + threadIdx.x;
    if (e0 >= s.count) return;
    const FastDiv& f0 = a.dim == 0 ? s.along : a.dq;
    const FastDiv& f1 = a.dim == 1 ? s.along : a.dn1;
    const FastDiv& f2 = a.dim == 2 ? s.along : a.dn2;
    U v[kConcatUnits];
    long long doff[kConcatUnits];
#pragma unroll
    for (int u = 0; u < kConcatUnits; u++) {
        const unsigned e = min(e0 + 256u * u, s.count - 1);
        const unsigned r = f0.div(e), q = e - r * f0.d;
        const unsigned r2 = f1.div(r), i1 = r - r2 * f1.d;
        const unsigned i3 = f2.div(r2), i2 = r2 - i3 * f2.d;
        v[u] = *reinterpret_cast<const U*>(s.data + i1 * s.nb1 + i2 * s.nb2 + i3 * s.nb3 + (long long)q * W);
        doff[u] = s.dst_off + i1 * a.d1 + i2 * a.d2 + i3 * a.d3 + (long long)q * W;
    }
#pragma unroll
    for (int u = 0; u < kConcatUnits; u++) {
        if (e0 + 256u * u >= s.count) break;
        store_stream(reinterpret_cast<U*>(a.dst + doff[u]), v[u]);
    }
}

// ------------------------------------------------------------------------- host side
bool aligned16_strides(const T4& t) {
    return aligned16(t.data) && t.nb[1] % 16 == 0 && t.nb[2] % 16 == 0 && t.nb[3] % 16 == 0;
}

void check_dense(const stx_tensor* t, const char* what) {
    STX_REQUIRE(contiguous(view(t)), "%s must be contiguous", what);
}

void require_shape(const stx_tensor* t, long long n0, long long n1, long long n2, long long n3, const char* what) {
    STX_REQUIRE(t->ne[0] == n0 && t->ne[1] == n1 && t->ne[2] == n2 && t->ne[3] == n3,
                "%s: expected shape [%lld, %lld, %lld, %lld], got [%lld, %lld, %lld, %lld]", what, n0, n1, n2, n3,
                (long long)t->ne[0], (long long)t->ne[1], (long long)t->ne[2], (long long)t->ne[3]);
}

// dst = cont(permute(src, ax)) with ggml's meaning: src dimension i lands on dst dimension
// ax[i]. gate (may be NULL) is a [1, dst ne1, ne2, ne3] tensor multiplied into each row; it
// needs ax[0] == 0.
void permute(const stx_tensor* src, const int ax[4], const stx_tensor* dst, const stx_tensor* gate,
             hipStream_t stream) {
    const T4 ts = view(src), td = view(dst);
    int from[4];                                  // dst dim j comes from src dim from[j]
    for (int i = 0; i < 4; i++) from[ax[i]] = i;
    if (nelem(td) == 0) return;
    if (ax[0] == 0) {
        const bool v4 = ts.ne[0] % 4 == 0 && aligned16_strides(ts) && aligned16_strides(td);
        const long long units_per_row = v4 ? ts.ne[0] / 4 : ts.ne[0];
        const long long count = units_per_row * nrows(td);
        if (count >= (1LL << 32) - 256LL * kRowUnits)
            fail(STX_STATUS_UNSUPPORTED, "cont_permute: more than 2^32 elements per call");
        STX_REQUIRE(td.ne[1] < (1LL << 32) && td.ne[2] < (1LL << 32), "cont_permute: dimension too large");
        RowPermArgs a{};
        a.src = ts.data;
        a.s1 = ts.nb[from[1]];
        a.s2 = ts.nb[from[2]];
        a.s3 = ts.nb[from[3]];
        a.dst = td.data;
        a.d1 = td.nb[1];
        a.d2 = td.nb[2];
        a.d3 = td.nb[3];
        a.count = (unsigned)count;
        a.dq = FastDiv((unsigned)units_per_row);
        a.dn1 = FastDiv((unsigned)td.ne[1]);
        a.dn2 = FastDiv((unsigned)td.ne[2]);
        if (gate != nullptr) {
            const T4 tg = view(gate);
            a.gate = tg.data;
            a.g1 = tg.nb[1];
            a.g2 = tg.nb[2];
            a.g3 = tg.nb[3];
        }
        const unsigned blocks = (unsigned)((count + 256 * kRowUnits - 1) / (256 * kRowUnits));
        if (v4) {
            if (gate) hipLaunchKernelGGL((permute_rows_kernel<true, true>), dim3(blocks), dim3(256), 0, stream, a);
            else hipLaunchKernelGGL((permute_rows_kernel<true, false>), dim3(blocks), dim3(256), 0, stream, a);
        } else {
            if (gate) hipLaunchKernelGGL((permute_rows_kernel<false, true>), dim3(blocks), dim3(256), 0, stream, a);
            else hipLaunchKernelGGL((permute_rows_kernel<false, false>), dim3(blocks), dim3(256), 0, stream, a);
        }
        launch_check("permute_rows_kernel");
        return;
    }
    STX_REQUIRE(gate == nullptr, "cont_permute: a gate needs dimension 0 in place");
    const int s = from[0];                       // src dim that becomes dst dim 0
    int others[2], k = 0;
    for (int i = 1; i < 4; i++)
        if (i != s) others[k++] = i;
    for (int i = 0; i < 4; i++) STX_REQUIRE(ts.ne[i] < (1LL << 31), "cont_permute: dimension too large");
    TransArgs a{};
    a.src = ts.data;
    a.dst = td.data;
    a.na = (int)ts.ne[0];
    a.nbb = (int)ts.ne[s];
    a.tiles_a = (a.na + kTile - 1) / kTile;
    a.tiles_b = (a.nbb + kTile - 1) / kTile;
    a.sb = ts.nb[s];
    a.da = td.nb[ax[0]];
    a.nc1 = (int)ts.ne[others[0]];
    a.nc2 = (int)ts.ne[others[1]];
    a.sc1 = ts.nb[others[0]];
    a.sc2 = ts.nb[others[1]];
    a.dc1 = td.nb[ax[others[0]]];
    a.dc2 = td.nb[ax[others[1]]];
    const long long blocks = (long long)a.tiles_a * a.tiles_b * a.nc1 * a.nc2;
    STX_REQUIRE(blocks < (1LL << 31) - kXcds, "cont_permute: too many tiles");
    a.blocks = (int)blocks;
    hipLaunchKernelGGL(transpose_kernel, dim3(xcd_grid(blocks)), dim3(256), 0, stream, a);
    launch_check("transpose_kernel");
}

void check_axes(const int ax[4]) {
    bool seen[4] = {false, false, false, false};
    for (int i = 0; i < 4; i++) {
        STX_REQUIRE(ax[i] >= 0 && ax[i] < 4 && !seen[ax[i]], "cont_permute: axes must be a permutation of 0..3");
        seen[ax[i]] = true;
    }
}

// dst must not overlap src: a permute reorders, so an in-place call would read overwritten data.
void check_disjoint(const stx_tensor* a, const stx_tensor* b, const char* what) {
    for (int i = 0; i < 4; i++)
        if (a->ne[i] == 0 || b->ne[i] == 0) return;
    auto span = [](const stx_tensor* t, uintptr_t& lo, uintptr_t& hi) {
        lo = reinterpret_cast<uintptr_t>(t->data);
        long long last = 0;
        for (int i = 0; i < 4; i++) last += (t->ne[i] - 1) * t->nb[i];
        hi = lo + (uintptr_t)last + 4;
    };
    uintptr_t alo, ahi, blo, bhi;
    span(a, alo, ahi);
    span(b, blo, bhi);
    STX_REQUIRE(ahi <= blo || bhi <= alo, "%s: source and destination overlap", what);
}

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_qkv_rope_split(const stx_tensor* qkv, const int32_t* pos, int n_head, float freq_base,
                                      float freq_scale, float attn_factor, const stx_tensor* q,
                                      const stx_tensor* k, const stx_tensor* vt, stx_stream stream) {
    return guard([&] {
        check_tensor(qkv, "qkv");
        check_tensor(q, "q");
        check_tensor(k, "k");
        check_tensor(vt, "vt");
        STX_REQUIRE(n_head > 0, "qkv_rope_split: n_head must be positive");
        const long long dh = q->ne[0], N = qkv->ne[1], batch = qkv->ne[2];
        STX_REQUIRE(qkv->ne[3] == 1, "qkv_rope_split: qkv must be [3 * n_head * dim_head, N, batch]");
        STX_REQUIRE(qkv->ne[0] == 3LL * n_head * dh, "qkv_rope_split: qkv ne0 (%lld) != 3 * n_head * dim_head (%lld)",
                    (long long)qkv->ne[0], 3LL * n_head * dh);
        require_shape(q, dh, N, n_head, batch, "qkv_rope_split: q");
        require_shape(k, dh, N, n_head, batch, "qkv_rope_split: k");
        require_shape(vt, N, dh, n_head, batch, "qkv_rope_split: vt");
        check_dense(q, "qkv_rope_split: q");
        check_dense(k, "qkv_rope_split: k");
        check_dense(vt, "qkv_rope_split: vt");
        if (N == 0 || batch == 0 || dh == 0) return;
        if (dh != 32 && dh != 64 && dh != 128)
            fail(STX_STATUS_UNSUPPORTED, "qkv_rope_split: dim_head %lld (32, 64 and 128 are built)", dh);
        STX_REQUIRE(pos != nullptr, "qkv_rope_split: pos is NULL");
        const T4 tq = view(qkv);
        STX_REQUIRE(aligned16(tq.data) && tq.nb[1] % 16 == 0 && tq.nb[2] % 16 == 0,
                    "qkv_rope_split: qkv rows must be 16-byte aligned");
        STX_REQUIRE(aligned16(q->data) && aligned16(k->data), "qkv_rope_split: q and k must be 16-byte aligned");
        STX_REQUIRE(N < (1LL << 31) && (long long)n_head * batch < (1LL << 31), "qkv_rope_split: too large");
        check_disjoint(qkv, q, "qkv_rope_split (q)");
        check_disjoint(qkv, k, "qkv_rope_split (k)");
        check_disjoint(qkv, vt, "qkv_rope_split (vt)");
        QkvArgs a{};
        a.qkv = tq.data;
        a.nb1 = tq.nb[1];
        a.nb2 = tq.nb[2];
        a.q = static_cast<float*>(q->data);
        a.k = static_cast<float*>(k->data);
        a.vt = static_cast<float*>(vt->data);
        a.pos = pos;
        a.n = (int)N;
        a.heads = n_head;
        a.units = (int)(n_head * batch);
        a.freq_base = freq_base;
        a.freq_scale = freq_scale;
        a.attn_factor = attn_factor;
        const hipStream_t s = as_stream(stream);
        if (dh == 32) launch_qkv_split<32>(a, s);
        else if (dh == 64) launch_qkv_split<64>(a, s);
        else launch_qkv_split<128>(a, s);
    });
}

STX_API stx_status stx_merge_heads(const stx_tensor* o, const stx_tensor* gates, const stx_tensor* dst,
                                   stx_stream stream) {
    return guard([&] {
        check_tensor(o, "o");
        check_tensor(dst, "dst");
        require_shape(dst, o->ne[0], o->ne[2], o->ne[1], o->ne[3], "merge_heads: dst");
        if (gates != nullptr) {
            check_tensor(gates, "gates");
            require_shape(gates, 1, o->ne[2], o->ne[1], o->ne[3], "merge_heads: gates");
        }
        check_disjoint(o, dst, "merge_heads");
        const int ax[4] = {0, 2, 1, 3};
        permute(o, ax, dst, gates, as_stream(stream));
    });
}

STX_API stx_status stx_cont_permute(const stx_tensor* a, int ax0, int ax1, int ax2, int ax3, const stx_tensor* dst,
                                    stx_stream stream) {
    return guard([&] {
        check_tensor(a, "a");
        check_tensor(dst, "dst");
        const int ax[4] = {ax0, ax1, ax2, ax3};
        check_axes(ax);
        for (int i = 0; i < 4; i++)
            STX_REQUIRE(dst->ne[ax[i]] == a->ne[i], "cont_permute: dst ne[%d] = %lld, expected a->ne[%d] = %lld", ax[i],
                        (long long)dst->ne[ax[i]], i, (long long)a->ne[i]);
        check_disjoint(a, dst, "cont_permute");
        permute(a, ax, dst, nullptr, as_stream(stream));
    });
}

STX_API stx_status stx_concat(const stx_tensor* const* srcs, int n_srcs, int dim, const stx_tensor* dst,
                              stx_stream stream) {
    return guard([&] {
        STX_REQUIRE(n_srcs >= 1 && srcs != nullptr, "concat: need at least one source");
        STX_REQUIRE(dim >= 0 && dim < 4, "concat: dim must be 0..3");
        check_tensor(dst, "dst");
        long long along = 0;
        bool v4 = aligned16_strides(view(dst));
        for (int i = 0; i < n_srcs; i++) {
            check_tensor(srcs[i], "concat source");
            for (int j = 0; j < 4; j++)
                if (j != dim)
                    STX_REQUIRE(srcs[i]->ne[j] == dst->ne[j], "concat: source %d ne[%d] = %lld, dst has %lld", i, j,
                                (long long)srcs[i]->ne[j], (long long)dst->ne[j]);
            along += srcs[i]->ne[dim];
            check_disjoint(srcs[i], dst, "concat");
            const T4 ts = view(srcs[i]);
            v4 = v4 && ts.ne[0] % 4 == 0 && aligned16_strides(ts);
        }
        STX_REQUIRE(along == dst->ne[dim], "concat: sources add up to %lld along dim %d, dst has %lld", along, dim,
                    (long long)dst->ne[dim]);
        if (dim == 0) v4 = v4 && dst->ne[0] % 4 == 0;
        const T4 td = view(dst);
        const hipStream_t s = as_stream(stream);
        STX_REQUIRE(td.ne[1] < (1LL << 32) && td.ne[2] < (1LL << 32), "concat: dimension too large");
        const long long dst_upr = v4 ? td.ne[0] / 4 : td.ne[0];
        long long off = 0;                       // elements along dim already placed
        for (int first = 0; first < n_srcs; first += kConcatMax) {
            const int m = std::min(kConcatMax, n_srcs - first);
            ConcatArgs a{};
            a.dst = td.data;
            a.d1 = td.nb[1];
            a.d2 = td.nb[2];
            a.d3 = td.nb[3];
            a.dq = FastDiv((unsigned)std::max<long long>(dst_upr, 1));
            a.dn1 = FastDiv((unsigned)std::max<long long>(td.ne[1], 1));
            a.dn2 = FastDiv((unsigned)std::max<long long>(td.ne[2], 1));
            a.dim = dim;
            long long max_units = 0;
            for (int i = 0; i < m; i++) {
                const T4 ts = view(srcs[first + i]);
                ConcatSrc& c = a.src[i];
                const long long upr = v4 ? ts.ne[0] / 4 : ts.ne[0];
                const long long count = upr * nrows(ts);
                if (count >= (1LL << 32) - 256LL * kConcatUnits)
                    fail(STX_STATUS_UNSUPPORTED, "concat: more than 2^32 elements in one source");
                c.data = ts.data;
                c.nb1 = ts.nb[1];
                c.nb2 = ts.nb[2];
                c.nb3 = ts.nb[3];
                c.dst_off = off * td.nb[dim];
                c.count = (unsigned)count;
                c.along = FastDiv((unsigned)std::max<long long>(dim == 0 ? upr : ts.ne[dim], 1));
                off += ts.ne[dim];
                max_units = std::max(max_units, count);
            }
            if (max_units == 0) continue;
            const long long chunks = (max_units + 256 * kConcatUnits - 1) / (256 * kConcatUnits);
            a.n_src = (unsigned)m;
            const unsigned blocks = (unsigned)(chunks * m);
            if (v4) hipLaunchKernelGGL((concat_kernel<true>), dim3(blocks), dim3(256), 0, s, a);
            else hipLaunchKernelGGL((concat_kernel<false>), dim3(blocks), dim3(256), 0, s, a);
            launch_check("concat_kernel");
        }
    });
}

}  // extern "C"
