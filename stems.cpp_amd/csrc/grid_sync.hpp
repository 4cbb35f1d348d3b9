// grid_sync.hpp — totals of per-block partial sums across the blocks of one launch, for
// single-pass kernels that normalise by statistics of data they keep in registers
// (GroupNorm in ops.hip, the HTDemucs normalisations in htdemucs.hip).
//
// Every block of a group publishes its partial sums (s1, s2); block 0 of the group waits for
// all of them (one record per block, polled by one thread each: no same-address atomics), adds
// them in block order and publishes the totals; the other blocks wait for the totals. Every
// block thus gets the same totals bit for bit, and the data is read from HBM once in one launch.
// All blocks of a launch must be resident at once: the host checks the occupancy first
// (resident_blocks) and takes another path when they would not be.
//
// Records are (s1, s2, tag) with tag = a 64-bit hash of s1, s2 and the call's key (token << 32 |
// gen + 1): the token is a per-call random number from the host, gen a per-group generation
// number kept in the workspace that block 0 advances once every block has read it. A reader
// takes a record only when its tag matches the values it read under the current key, so the
// three words need no write ordering (a torn or stale record fails the check), graph replays
// of one call (same token) wait for a new gen each time, and neither a record of another call
// nor garbage in a fresh workspace passes: the workspace needs no initialisation or clearing.
// Cross-block words are device-scope relaxed atomics, which gfx950 performs at the device's
// coherence point (sc1), past the XCD's own L2: no L2 write-back or invalidation, which a
// release/acquire pair would cost per block. Every wait is bounded: a block that gives up
// (which needs blocks that never become resident, e.g. two such kernels sharing the device)
// reports it, and the kernels then write NaN instead of hanging.
#pragma once

#include <atomic>
#include <chrono>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace stx {

constexpr int kGridThreads = 512;                    // threads per block of the single-pass kernels
constexpr int kGridMaxBlocks = 512;                  // per group
constexpr int kGridMaxGroups = 8;
constexpr int kGridStatCopies = 8;                   // waiters poll copy (block % 8)
constexpr int kGridStatStride = 128;                 // unsigned long longs between copies (1 KB)
constexpr unsigned kGridSpinLimit = 1u << 18;        // polls of about 1 us each

// Workspace area, at a fixed offset with a fixed size so that a workspace shared by calls of
// different shapes keeps each group slot's generation number consistent: [8 KB) totals
// records, 8 per group at 1 KB apart | [256 B) generation numbers | partial sums records,
// 3 words per block.
constexpr size_t kGridSyncStat = 0;
constexpr size_t kGridSyncGen = sizeof(unsigned long long) * kGridStatCopies * kGridStatStride;
constexpr size_t kGridSyncPart = kGridSyncGen + 256;
constexpr size_t kGridSyncBytes =
    (kGridSyncPart + sizeof(unsigned long long) * 3 * kGridMaxGroups * kGridMaxBlocks + 255) / 256 * 256;
static_assert(3 * kGridMaxGroups <= kGridStatStride && 4 * kGridMaxGroups <= 256, "grid sync area layout");

struct GridSync {
    unsigned* gen;                   // [kGridMaxGroups]
    unsigned long long* stat;        // [kGridStatCopies][kGridStatStride]: group g's totals record at 3g
    unsigned long long* part;        // [kGridMaxGroups][kGridMaxBlocks][3]: partial sums records
    unsigned token;
    unsigned spin_limit;
};

// Sums of two doubles over an NT-thread block: wave sums, then the wave totals added in wave
// order by every thread (the same order in every block). red holds 2 * NT / 64 doubles.
template <int NT>
__device__ __forceinline__ void block_sum2_n(double& a, double& b, double* red) {
    constexpr int W = NT / 64;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        a += __shfl_xor(a, m, 64);
        b += __shfl_xor(b, m, 64);
    }
    __syncthreads();
    if (threadIdx.x % 64 == 0) {
        red[threadIdx.x / 64] = a;
        red[W + threadIdx.x / 64] = b;
    }
    __syncthreads();
    a = 0.0;
    b = 0.0;
#pragma unroll
    for (int w = 0; w < W; w++) {
        a += red[w];
        b += red[W + w];
    }
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
__device__ __forceinline__ unsigned long long record_tag(unsigned long long a, unsigned long long b,
                                                         unsigned long long key) {
    return fmix64(a ^ fmix64(b ^ fmix64(key)));
}
// Publishes (s1, s2) at r[0..2] under key.
__device__ __forceinline__ void record_store(unsigned long long* r, double s1, double s2, unsigned long long key) {
    const unsigned long long a = (unsigned long long)__double_as_longlong(s1);
    const unsigned long long b = (unsigned long long)__double_as_longlong(s2);
    sync_store(r, a);
    sync_store(r + 1, b);
    sync_store(r + 2, record_tag(a, b, key));
}
// Polls r (at most limit times) until it holds a record under key; false if it never did.
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
        __builtin_amdgcn_s_sleep(1);
    }
}

// Generation number of group gt for this call, plus one (read at the start of the kernel,
// before the block publishes anything).
__device__ __forceinline__ unsigned grid_gen1(const GridSync& f, int gt) {
    return __hip_atomic_load(f.gen + gt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}

// Totals over the nblk blocks of group gt (this block is blockIdx.x) of the block sums s1, s2
// (the same values in every thread): tot[0..1] (shared) gets them in every block. gen1 is
// grid_gen1() read at the start. Returns true when a wait gave up (every thread agrees).
template <int NT>
__device__ __forceinline__ bool grid_totals(const GridSync& f, int gt, int nblk, unsigned gen1, double s1, double s2,
                                            double* red, double* tot) {
    const unsigned long long key = (unsigned long long)f.token << 32 | gen1;
    unsigned long long* part = f.part + 3 * (size_t)gt * kGridMaxBlocks;
    bool late = false;
    if (blockIdx.x != 0) {
        if (threadIdx.x == 0) {
            record_store(part + 3 * blockIdx.x, s1, s2, key);
            double t1 = 0.0, t2 = 0.0;                         // the group's totals, from block 0
            late = !record_wait(f.stat + (blockIdx.x % kGridStatCopies) * kGridStatStride + 3 * gt, key,
                                f.spin_limit, t1, t2);
            tot[0] = t1;
            tot[1] = t2;
        }
    } else {
        // Block 0 collects: thread t waits for the records of blocks t, t + NT, ... and adds
        // them in that order (block 0's own sums first), then the block adds the threads' sums
        // in thread order and publishes the totals, one record per copy.
        double p1 = threadIdx.x == 0 ? s1 : 0.0, p2 = threadIdx.x == 0 ? s2 : 0.0;
        for (int b = threadIdx.x == 0 ? NT : (int)threadIdx.x; b < nblk && !late; b += NT) {
            double q1 = 0.0, q2 = 0.0;
            late = !record_wait(part + 3 * b, key, f.spin_limit, q1, q2);
            p1 += q1;
            p2 += q2;
        }
        block_sum2_n<NT>(p1, p2, red);
        if (threadIdx.x == 0) {
            tot[0] = p1;
            tot[1] = p2;
#pragma unroll
            for (int c = 0; c < kGridStatCopies; c++)
                record_store(f.stat + c * kGridStatStride + 3 * gt, p1, p2, key);
            // Every block has read gen before it published its record.
            __hip_atomic_store(f.gen + gt, gen1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    return __syncthreads_or(late);
}

// A per-call random number: murmur3's 32-bit finaliser of a call counter offset by a
// per-process seed from the clock.
inline unsigned grid_call_token() {
    static const unsigned seed = (unsigned)std::chrono::steady_clock::now().time_since_epoch().count();
    static std::atomic<unsigned> calls{0};
    unsigned h = seed + 0x9e3779b9u * calls.fetch_add(1, std::memory_order_relaxed);
    h ^= h >> 16;
    h *= 0x85ebca6bu;
    h ^= h >> 13;
    h *= 0xc2b2ae35u;
    h ^= h >> 16;
    return h;
}

// The sync area of a workspace that starts at ws (8-byte aligned), for one call.
inline GridSync grid_sync_at(void* ws) {
    char* b = static_cast<char*>(ws);
    GridSync f;
    f.gen = reinterpret_cast<unsigned*>(b + kGridSyncGen);
    f.stat = reinterpret_cast<unsigned long long*>(b + kGridSyncStat);
    f.part = reinterpret_cast<unsigned long long*>(b + kGridSyncPart);
    f.token = grid_call_token();
    f.spin_limit = kGridSpinLimit;
    return f;
}

// Whether the single-pass kernels may run: not when STX_NO_GRID_SYNC is set to anything but
// "0" (read at every call, for callers that run such kernels concurrently on one device), and
// not when the process's queues carry a CU mask (HSA_CU_MASK, ROC_GLOBAL_CU_MASK), which would
// leave fewer CUs than the occupancy check counts.
inline bool grid_sync_enabled() {
    const char* off = std::getenv("STX_NO_GRID_SYNC");
    if (off && off[0] && !(off[0] == '0' && off[1] == 0)) return false;
    static const bool masked = std::getenv("HSA_CU_MASK") || std::getenv("ROC_GLOBAL_CU_MASK");
    return !masked;
}

// Blocks of `kernel` (kGridThreads threads, no dynamic LDS) that the current device holds at
// once; 0 when grid_sync_enabled() is false, so that callers take their multi-kernel path.
inline int resident_blocks(const void* kernel) {
    if (!grid_sync_enabled()) return 0;
    struct Entry {
        const void* k;
        int dev, blocks;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
        if (e.k == kernel && e.dev == dev) return e.blocks;
    int cus = 0, per_cu = 0;
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGridThreads, 0),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    cache.push_back({kernel, dev, cus * per_cu});
    return cus * per_cu;
}

}  // namespace stx
