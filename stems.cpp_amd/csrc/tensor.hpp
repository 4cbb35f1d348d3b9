// tensor.hpp — ggml-style tensor descriptors (stx_tensor) on the host and the device, and the
// argument checks shared by the op entry points.
#pragma once

#include <cstdint>

#include "common.hpp"

namespace stx {

struct T4 {                      // device view of an stx_tensor
    char* data;
    long long ne[4];
    long long nb[4];
};

inline T4 view(const stx_tensor* t) {
    T4 v{};
    v.data = static_cast<char*>(t->data);
    for (int i = 0; i < 4; i++) {
        v.ne[i] = t->ne[i];
        v.nb[i] = t->nb[i];
    }
    return v;
}

inline long long nrows(const T4& t) { return t.ne[1] * t.ne[2] * t.ne[3]; }
inline long long nelem(const T4& t) { return t.ne[0] * nrows(t); }

// Dense row-major layout; the stride of a dimension of extent 1 is never used and may be anything.
inline bool contiguous(const T4& t) {
    long long expect = 4;
    for (int i = 0; i < 4; i++) {
        if (t.ne[i] > 1 && t.nb[i] != expect) return false;
        expect *= t.ne[i];
    }
    return true;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline void check_tensor(const stx_tensor* t, const char* what) {
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

inline void check_same_shape(const stx_tensor* a, const stx_tensor* b, const char* what) {
    for (int i = 0; i < 4; i++)
        STX_REQUIRE(a->ne[i] == b->ne[i], "%s: shape mismatch in ne[%d] (%lld vs %lld)", what, i,
                    (long long)a->ne[i], (long long)b->ne[i]);
}

// b repeats into dst (ggml_can_repeat): every dst->ne[i] is a multiple of b->ne[i].
inline void check_repeat(const stx_tensor* b, const stx_tensor* dst, const char* what) {
    for (int i = 0; i < 4; i++)
        STX_REQUIRE((b->ne[i] > 0 && dst->ne[i] % b->ne[i] == 0) || (b->ne[i] == 0 && dst->ne[i] == 0),
                    "%s: ne[%d] = %lld does not repeat into %lld", what, i, (long long)b->ne[i],
                    (long long)dst->ne[i]);
}

}  // namespace stx
