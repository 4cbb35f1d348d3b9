// common.hpp — status/error plumbing and launch helpers shared by every translation unit.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "stx.h"

namespace stx {

// An error that maps onto one stx_status; thrown inside the library, caught at the C ABI.
struct Error : std::exception {
    stx_status code;
    std::string msg;
    Error(stx_status c, std::string m) : code(c), msg(std::move(m)) {}
    const char* what() const noexcept override { return msg.c_str(); }
};

[[noreturn]] inline void fail(stx_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw Error(code, buf);
}

void set_last_error(const char* msg);

// Runs f, converting every exception into a status and the thread's last-error message.
template <class F>
stx_status guard(F&& f) noexcept {
    try {
        f();
        set_last_error("");
        return STX_STATUS_OK;
    } catch (const Error& e) {
        set_last_error(e.msg.c_str());
        return e.code;
    } catch (const std::bad_alloc&) {
        set_last_error("out of host memory");
        return STX_STATUS_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return STX_STATUS_RUNTIME_ERROR;
    } catch (...) {
        set_last_error("unknown C++ exception");
        return STX_STATUS_RUNTIME_ERROR;
    }
}

inline void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory)
        fail(STX_STATUS_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    fail(STX_STATUS_DEVICE_ERROR, "%s: %s", what, hipGetErrorString(e));
}

// Call right after a kernel launch: reports launch-configuration errors.
inline void launch_check(const char* kernel) { hip_check(hipGetLastError(), kernel); }

#define STX_REQUIRE(cond, ...) \
    do { if (!(cond)) ::stx::fail(STX_STATUS_INVALID_ARGUMENT, __VA_ARGS__); } while (0)

inline hipStream_t as_stream(stx_stream s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kXcds = 8;   // MI355X: 8 XCDs; workgroups are dealt to them round-robin

// Grid size rounded up to a multiple of the XCD count, for xcd_block().
inline unsigned xcd_grid(long long blocks) {
    return (unsigned)((blocks + kXcds - 1) / kXcds * kXcds);
}

// Maps the hardware block id to a logical one so that each XCD receives a contiguous run of
// logical blocks: neighbouring tiles (which share halo data and partial cache lines) then
// meet in the same L2. gridDim.x must be a multiple of kXcds; callers skip ids >= the real
// block count.
__device__ __forceinline__ int xcd_block() {
    const int per = (int)gridDim.x / kXcds;
    return ((int)blockIdx.x % kXcds) * per + (int)blockIdx.x / kXcds;
}

inline bool is_pow2(long long n) { return n >= 1 && (n & (n - 1)) == 0; }

// Wave reductions on DPP lane permutations (VALU moves, no LDS round trip). The controls used
// here read lanes of the same 16-lane row only, so every source lane exists:
//   0xB1 quad_perm [1,0,3,2] (lane ^ 1), 0x4E quad_perm [2,3,0,1] (lane ^ 2),
//   0x141 row_half_mirror (7 - i within 8 lanes), 0x140 row_mirror (15 - i within 16 lanes).
// Each step adds a lane's value to its partner's; IEEE addition is commutative, so both
// partners hold the same bits after every step and the result is the same in every lane.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Sum over aligned groups of LANES lanes (a power of two <= 64), the same bits in every lane of
// a group. Up to 16 lanes: DPP steps inside the row. 32: the row sums, then one exchange
// between the two rows of the group. 64: the four row sums read into scalars and added as
// (r0 + r1) + (r2 + r3), uniform over the wave.
template <int LANES>
__device__ __forceinline__ double lane_sum(double v) {
    static_assert(LANES >= 1 && LANES <= 64 && (LANES & (LANES - 1)) == 0, "lane_sum: LANES");
    if constexpr (LANES >= 2) v += dpp_f64<0xB1>(v);
    if constexpr (LANES >= 4) v += dpp_f64<0x4E>(v);
    if constexpr (LANES >= 8) v += dpp_f64<0x141>(v);
    if constexpr (LANES >= 16) v += dpp_f64<0x140>(v);
    if constexpr (LANES == 32) v += __shfl_xor(v, 16, 32);
    if constexpr (LANES == 64)
        v = (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
    return v;
}

// lane_sum with a run-time group size L (a power of two <= 64, uniform over the wave).
__device__ __forceinline__ double lane_sum_dyn(double v, int L) {
    if (L >= 2) v += dpp_f64<0xB1>(v);
    if (L >= 4) v += dpp_f64<0x4E>(v);
    if (L >= 8) v += dpp_f64<0x141>(v);
    if (L >= 16) v += dpp_f64<0x140>(v);
    if (L >= 32) v += __shfl_xor(v, 16, 64);
    if (L >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Maximum over aligned groups of LANES lanes, in every lane of a group (max is exact, so any
// order gives the same value).
template <int LANES>
__device__ __forceinline__ float lane_max(float v) {
    static_assert(LANES >= 1 && LANES <= 64 && (LANES & (LANES - 1)) == 0, "lane_max: LANES");
    if constexpr (LANES >= 2) v = fmaxf(v, dpp_f32<0xB1>(v));
    if constexpr (LANES >= 4) v = fmaxf(v, dpp_f32<0x4E>(v));
    if constexpr (LANES >= 8) v = fmaxf(v, dpp_f32<0x141>(v));
    if constexpr (LANES >= 16) v = fmaxf(v, dpp_f32<0x140>(v));
    if constexpr (LANES >= 32) v = fmaxf(v, __shfl_xor(v, 16, LANES));
    if constexpr (LANES == 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// Vector stores with the non-temporal hint (the store's nt bit), for outputs the kernel does not
// read back. Measured on outputs of tens of MB written once (the band gather's features): the
// cold call is ~20 % faster, since the written lines no longer displace dirty lines of earlier
// work from the caches; when the same buffers are rewritten while still cached it costs ~2 %.
// Not for stores of short runs that other workgroups complete to whole lines (the F-major STFT
// rows): those must meet in L2 first, and streamed they cost 1.4-2.4x.
typedef float stx_v2f __attribute__((ext_vector_type(2)));
typedef float stx_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_stream(float2* p, float2 v) {
    __builtin_nontemporal_store(stx_v2f{v.x, v.y}, reinterpret_cast<stx_v2f*>(p));
}
__device__ __forceinline__ void store_stream(float4* p, float4 v) {
    __builtin_nontemporal_store(stx_v4f{v.x, v.y, v.z, v.w}, reinterpret_cast<stx_v4f*>(p));
}

// x / h correctly rounded, for h finite and nonzero, given r = RN(1/h): q0 = RN(x r), then
// RN(q0 + r RN(x - q0 h)), which by Markstein's theorem (r within half an ulp of 1/h, q0 within
// one ulp of x/h, the residual exact by the fma) is the IEEE quotient when nothing overflows or
// underflows on the way. When q0 is not finite (x infinite or NaN, or x/h overflowing) the
// residual would be inf - inf = NaN; the IEEE quotient is then q0 itself (+-inf or NaN).
__device__ __forceinline__ double div_rn(double x, double h, double r) {
#pragma clang fp contract(off)
    const double q0 = x * r;
    const double q = fma(fma(-q0, h, x), r, q0);
    return isfinite(q0) ? q : q0;
}

// Division of any n < 2^32 by a fixed d >= 1 with one high multiply, one add and one shift:
// the round-up method of Granlund and Montgomery, "Division by invariant integers using
// multiplication" (PLDI 1994), Fig. 4.1 with N = 32: l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1 (fits 32 bits), q = (mulhi(m, n) + n) >> l, with the
// add done in 64 bits so it cannot overflow.
struct FastDiv {
    unsigned d = 1, m = 1, l = 0;
    FastDiv() = default;
    explicit FastDiv(unsigned divisor) : d(divisor) {
        while ((1ull << l) < d) l++;
        m = (unsigned)((((1ull << l) - d) << 32) / d + 1);
    }
    __host__ __device__ __forceinline__ unsigned div(unsigned n) const {
#ifdef __HIP_DEVICE_COMPILE__
        const unsigned hi = __umulhi(m, n);
#else
        const unsigned hi = (unsigned)(((unsigned long long)m * n) >> 32);
#endif
        return (unsigned)(((unsigned long long)hi + n) >> l);
    }
    __host__ __device__ __forceinline__ unsigned mod(unsigned n) const { return n - div(n) * d; }
};

// The defaults of stx_separate_options (src/separator.h:19-32): no shifts, the model's overlap.
inline stx_separate_options default_separate_options() {
    stx_separate_options o{};
    o.size = sizeof o;
    o.overlap = -1.0f;
    return o;
}

// A caller's separate options (NULL: the defaults), checked against the frozen V1 prefix; the
// fields past the caller's size keep their defaults.
inline stx_separate_options separate_options(const stx_separate_options* in) {
    stx_separate_options o = default_separate_options();
    if (!in) return o;
    STX_REQUIRE(in->size >= STX_SEPARATE_OPTIONS_MIN_SIZE, "separate options: size %u is below the V1 minimum %u",
                in->size, STX_SEPARATE_OPTIONS_MIN_SIZE);
    std::memcpy(&o, in, in->size < sizeof o ? in->size : sizeof o);
    o.size = sizeof o;
    return o;
}

// Compute units of the current device (cached per device id).
inline int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64) dev = 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Blocks of `kernel` (`threads` threads, no dynamic LDS) that the current device holds at
// once (occupancy times CUs, cached per kernel and device).
inline int device_blocks(const void* kernel, int threads) {
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
    hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0),
              "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    cache.push_back({kernel, dev, cus * per_cu});
    return cus * per_cu;
}

}  // namespace stx
