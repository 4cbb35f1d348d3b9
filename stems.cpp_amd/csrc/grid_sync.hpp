// grid_sync.hpp — totals of per-block partial sums across the blocks of one launch, for
// single-pass kernels that normalise by statistics of data they keep in registers
// (GroupNorm in ops.hip, the HTDemucs normalisations in htdemucs.hip).
//
// Every block of a group publishes its partial sums (s1, s2); block 0 of the group waits for
// all of them (one record per block, polled by one thread each: no same-address atomics), adds
// them in a fixed order and publishes the totals; the other blocks wait for the totals. Every
// block thus gets the same totals bit for bit, and the data is read from HBM once in one launch.
// The host checks first that all blocks of a launch can be resident at once (resident_blocks)
// and takes a multi-kernel path when they cannot.
//
// Records are (s1, s2, tag) with tag = s1 ^ rotl(s2, 29) ^ the launch's key (as bits). The key
// is a 64-bit hash of the hardware's name for this dispatch: the AQL packet's dispatch id (its
// index in its queue, 64 bits, never reused by that queue) and the queue's address, and of the
// group. Every block of a launch reads the same key, graph replays get new ones, and a record
// of an earlier launch, a torn record or garbage in a fresh workspace fails the check: the
// workspace needs no initialisation and no per-launch state. Cross-block words are device-scope relaxed atomics, which gfx950
// performs at the device's coherence point, past the XCD's own L2.
//
// Every wait is bounded (spin_limit polls). A block whose wait gives up (blocks that never
// became resident: another process or a concurrent kernel holding CUs, a CU-masked queue)
// computes its group's totals itself from the input, chunk by chunk in the same order and with
// the same arithmetic as the blocks and the collector, so its output is bit-identical to the
// normal path's; it counts itself in the workspace's fallback word (stx_grid_sync_fallbacks).
// That needs the input unchanged until every block has read it: the callers take the single
// pass only when the output does not overlap the input.
#pragma once

#include <atomic>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "common.hpp"

// The AQL packet's dispatch id (user SGPRs set up by the command processor).
extern "C" __device__ unsigned long long stx_amdgcn_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

namespace stx {

constexpr int kGridThreads = 512;                    // threads per block of the single-pass kernels
constexpr int kGridMaxBlocks = 512;                  // per group (one collector thread per block)
constexpr int kGridMaxGroups = 8;
constexpr int kGridStatCopies = 8;                   // waiters poll copy (block % 8)
constexpr int kGridStatStride = 128;                 // unsigned long longs between copies (1 KB)
constexpr unsigned kGridSpinLimit = 1u << 16;        // polls of 0.1 to 1 us each

// Workspace area: [8 KB) totals records, 8 per group at 1 KB apart | [256 B) the fallback
// counter | partial sums records, 3 words per block.
constexpr size_t kGridSyncStat = 0;
constexpr size_t kGridSyncFallback = sizeof(unsigned long long) * kGridStatCopies * kGridStatStride;
constexpr size_t kGridSyncPart = kGridSyncFallback + 256;
constexpr size_t kGridSyncBytes =
    (kGridSyncPart + sizeof(unsigned long long) * 3 * kGridMaxGroups * kGridMaxBlocks + 255) / 256 * 256;
static_assert(3 * kGridMaxGroups <= kGridStatStride, "grid sync area layout");

struct GridSync {
    unsigned long long* stat;        // [kGridStatCopies][kGridStatStride]: group g's totals record at 3g
    unsigned long long* part;        // [kGridMaxGroups][kGridMaxBlocks][3]: partial sums records
    unsigned* fallbacks;             // blocks that computed their totals themselves (sticky)
    unsigned spin_limit;
};

// Sums of two doubles over an NT-thread block: wave sums (lane_sum<64>), then the wave totals
// added in wave order by every thread (the same order in every block). red holds 2 * NT / 64
// doubles. Returns the OR of `flag` over the block (a ballot per wave, passed beside the sums).
template <int NT>
__device__ __forceinline__ bool block_sum2_or(double& a, double& b, double* red, bool flag) {
    constexpr int W = NT / 64;
    __shared__ int wflag[W];
    a = lane_sum<64>(a);
    b = lane_sum<64>(b);
    const bool wany = __ballot(flag) != 0;
    __syncthreads();                                   // readers of a previous call's red are done
    if (threadIdx.x % 64 == 0) {
        red[threadIdx.x / 64] = a;
        red[W + threadIdx.x / 64] = b;
        wflag[threadIdx.x / 64] = wany ? 1 : 0;
    }
    __syncthreads();
    a = 0.0;
    b = 0.0;
    int any = 0;
#pragma unroll
    for (int w = 0; w < W; w++) {
        a += red[w];
        b += red[W + w];
        any |= wflag[w];
    }
    return any != 0;
}

template <int NT>
__device__ __forceinline__ void block_sum2_n(double& a, double& b, double* red) {
    (void)block_sum2_or<NT>(a, b, red, false);
}

__device__ __forceinline__ void sync_store(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long sync_load(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// MurmurHash3's 64-bit finaliser.
__device__ __forceinline__ unsigned long long fmix64(unsigned long long k) {
    k ^= k >> 33;
    k *= 0xff51afd7ed558ccdull;
    k ^= k >> 33;
    k *= 0xc4ceb9fe1a85ec53ull;
    k ^= k >> 33;
    return k;
}
// Key of group gt in this launch.
__device__ __forceinline__ unsigned long long launch_key(int gt) {
    const unsigned long long q = (unsigned long long)__builtin_amdgcn_queue_ptr();
    return fmix64(fmix64(stx_amdgcn_dispatch_id() ^ fmix64(q)) + (unsigned long long)gt);
}
// A record's check word. The key is already a 64-bit hash, so the check needs no mixing of its
// own: a record of another launch, or one whose words come from two launches, passes only if
// the two launches' keys differ by exactly what their words differ by (probability 2^-64), and
// the check costs three instructions per poll instead of three 64-bit multiply chains.
__device__ __forceinline__ unsigned long long record_tag(unsigned long long a, unsigned long long b,
                                                         unsigned long long key) {
    return a ^ ((b << 29) | (b >> 35)) ^ key;
}
// Publishes (s1, s2) at r[0..2] under key.
__device__ __forceinline__ void record_store(unsigned long long* r, double s1, double s2, unsigned long long key) {
    const unsigned long long a = (unsigned long long)__double_as_longlong(s1);
    const unsigned long long b = (unsigned long long)__double_as_longlong(s2);
    sync_store(r, a);
    sync_store(r + 1, b);
    sync_store(r + 2, record_tag(a, b, key));
}
// Polls r (at most limit times after the first look) until it holds a record under key; false
// if it never did. One poll in flight, issued as soon as the previous one has been checked (a
// pause of 64 or 128 clocks between polls, or a second poll in flight, measured slower).
__device__ __forceinline__ bool record_wait(const unsigned long long* r, unsigned long long key, unsigned limit,
                                            double& s1, double& s2) {
    for (unsigned spins = 0;;) {
        const unsigned long long a = sync_load(r), b = sync_load(r + 1), h = sync_load(r + 2);
        if (h == record_tag(a, b, key)) {
            s1 = __longlong_as_double((long long)a);
            s2 = __longlong_as_double((long long)b);
            return true;
        }
        if (++spins > limit) return false;
    }
}

// Totals over the nblk blocks of group gt (this block is blockIdx.x) of the block sums s1, s2
// (the same values in every thread): tot[0..1] (shared) holds them in every block on return.
// The collector's order: thread t adds the sums of blocks t, t + NT, t + 2 NT, ... in that
// order, starting from +0.0, then the block adds the threads' sums (block_sum2_or).
// recompute(tot) is called by every thread of a block whose wait gave up: it must leave the
// same totals in tot[0..1] from the input, in that order, and end with a barrier. Returns
// whether it was called (uniform over the block), so that the caller can reload what it kept
// in registers instead of holding it across the recompute.
template <int NT, class Recompute>
__device__ __forceinline__ bool grid_totals(const GridSync& f, int gt, int nblk, double s1, double s2, double* red,
                                            double* tot, Recompute&& recompute) {
    const unsigned long long key = launch_key(gt);
    unsigned long long* part = f.part + 3 * (size_t)gt * kGridMaxBlocks;
    bool late = false;
    if (blockIdx.x != 0) {
        __shared__ int wait_late;
        if (threadIdx.x == 0) {
            record_store(part + 3 * blockIdx.x, s1, s2, key);
            double t1 = 0.0, t2 = 0.0;                         // the group's totals, from block 0
            const bool l = !record_wait(f.stat + (blockIdx.x % kGridStatCopies) * kGridStatStride + 3 * gt, key,
                                        f.spin_limit, t1, t2);
            tot[0] = t1;
            tot[1] = t2;
            wait_late = l ? 1 : 0;
        }
        __syncthreads();
        late = wait_late != 0;
    } else {
        double p1 = 0.0, p2 = 0.0;
        if (threadIdx.x == 0) {
            p1 += s1;
            p2 += s2;
        }
        for (int b = threadIdx.x == 0 ? NT : (int)threadIdx.x; b < nblk && !late; b += NT) {
            double q1 = 0.0, q2 = 0.0;
            late = !record_wait(part + 3 * b, key, f.spin_limit, q1, q2);
            p1 += q1;
            p2 += q2;
        }
        late = block_sum2_or<NT>(p1, p2, red, late);
        if (!late) {
            if (threadIdx.x < kGridStatCopies) {              // one copy per thread
                tot[0] = p1;
                tot[1] = p2;
                record_store(f.stat + threadIdx.x * kGridStatStride + 3 * gt, p1, p2, key);
            }
            __syncthreads();
        }
    }
    if (late) {                                                // uniform over the block
        recompute(tot);
        if (threadIdx.x == 0) {
            if (blockIdx.x == 0) {                             // blocks still waiting take these
#pragma unroll
                for (int c = 0; c < kGridStatCopies; c++)
                    record_store(f.stat + c * kGridStatStride + 3 * gt, tot[0], tot[1], key);
            }
            __hip_atomic_fetch_add(f.fallbacks, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
    return late;
}

// Polls per wait: kGridSpinLimit, or STX_GRID_SYNC_SPIN_LIMIT when set (read at every call;
// a small value forces the recompute path, for tests).
inline unsigned grid_spin_limit() {
    const char* s = std::getenv("STX_GRID_SYNC_SPIN_LIMIT");
    if (!s || !s[0]) return kGridSpinLimit;
    char* end = nullptr;
    const unsigned long v = std::strtoul(s, &end, 10);
    return end && *end == 0 ? (unsigned)std::min<unsigned long>(v, 1ul << 30) : kGridSpinLimit;
}

// The sync area of a workspace that starts at ws (8-byte aligned), for one call.
inline GridSync grid_sync_at(void* ws) {
    char* b = static_cast<char*>(ws);
    GridSync f;
    f.stat = reinterpret_cast<unsigned long long*>(b + kGridSyncStat);
    f.fallbacks = reinterpret_cast<unsigned*>(b + kGridSyncFallback);
    f.part = reinterpret_cast<unsigned long long*>(b + kGridSyncPart);
    f.spin_limit = grid_spin_limit();
    return f;
}

// Whether the single-pass kernels may run on `stream`: not when STX_NO_GRID_SYNC is set to
// anything but "0" (read at every call), not when the process's queues carry a CU mask
// (HSA_CU_MASK, ROC_GLOBAL_CU_MASK), and not on a stream created with a CU mask
// (hipExtStreamCreateWithCUMask): those leave fewer CUs than the occupancy check counts. The
// single pass stays correct without them (see above), only slower.
inline bool grid_sync_enabled(hipStream_t stream) {
    const char* off = std::getenv("STX_NO_GRID_SYNC");
    if (off && off[0] && !(off[0] == '0' && off[1] == 0)) return false;
    static const bool masked = std::getenv("HSA_CU_MASK") || std::getenv("ROC_GLOBAL_CU_MASK");
    if (masked) return false;
    if (stream == nullptr) return true;
    uint32_t mask[32] = {};
    if (hipExtStreamGetCUMask(stream, 32, mask) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    int set = 0;
    for (uint32_t m : mask) set += __builtin_popcount(m);
    return set >= device_cus();
}

// device_blocks for the single-pass kernels; 0 when grid_sync_enabled() is false, so that
// callers take their multi-kernel path.
inline int resident_blocks(const void* kernel, hipStream_t stream, int threads = kGridThreads) {
    if (!grid_sync_enabled(stream)) return 0;
    return device_blocks(kernel, threads);
}

// Whether [a, a + an) and [b, b + bn) (bytes) overlap.
inline bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + bn && y < x + an;
}

}  // namespace stx
