// demix_host.cpp — host-side bookkeeping of the chunked overlap-add demix.
//
// Reference: RoFormer::Impl::demix (src/roformer.cpp:286-351), n_chunks (:353-357) and the step
// rule of RoFormer::separate (:442-443); with the MSST rules, TFCTDF::Impl::demix_msst
// (src/tfc_tdf.cpp:447-495), ZFTurbo's loop with three differences: short chunks are
// reflect-padded above chunk / 2 samples (not chunk / 2 + 1), only the chunk after which the
// loop ends drops its fade-out (not every chunk reaching the end), and the fades are
// linspace(0, 1, fade) and linspace(1, 0, fade) (:56-63,465-469). Everything here is integer or
// single float operations in the reference's order, so the chunk table and the fade window are
// bit-identical to the reference's.
#include <cmath>
#include <vector>

#include "common.hpp"
#include "demix_host.hpp"

namespace stx {

DemixGeometry demix_geometry(int64_t len, int chunk, int step, int rules) {
    STX_REQUIRE(len > 0, "empty input");
    STX_REQUIRE(chunk > 0 && step > 0, "bad chunk/step");
    STX_REQUIRE(rules == STX_DEMIX_ROFORMER || rules == STX_DEMIX_MSST, "unknown demix rules %d", rules);
    DemixGeometry g;
    g.rules = rules;
    g.len = len;
    g.chunk = chunk;
    g.step = step;
    g.fade = chunk / 10;
    g.border = chunk - step;
    g.reflect_border = (len > 2LL * g.border && g.border > 0) ? 1 : 0;      // :290
    g.padded_len = g.reflect_border ? len + 2LL * g.border : len;           // :291
    g.n_chunks = (g.padded_len + step - 1) / step;                          // :353-357
    return g;
}

stx_chunk demix_chunk(const DemixGeometry& g, int64_t k) {
    stx_chunk c{};
    const int64_t i = k * g.step;
    c.start = i;
    c.length = (int32_t)std::min<int64_t>(g.chunk, g.padded_len - i);      // :318
    const bool msst = g.rules == STX_DEMIX_MSST;
    if (c.length == g.chunk) c.pad_mode = STX_CHUNK_FULL;
    else if (c.length > g.chunk / 2 + (msst ? 0 : 1)) c.pad_mode = STX_CHUNK_REFLECT;  // :324; tfc_tdf :474
    else c.pad_mode = STX_CHUNK_ZERO;
    // :335-336: the first chunk drops its fade-in, otherwise a chunk reaching the end drops its
    // fade-out; MSST (tfc_tdf :485-486): only the chunk after which i + step >= Lp.
    c.fade_in = i == 0 ? 0 : 1;
    const int64_t reach = msst ? i + g.step : i + g.chunk;
    c.fade_out = (i != 0 && reach >= g.padded_len) ? 0 : 1;
    return c;
}

// torch.linspace(a, b, n) in float32, from both ends (src/tfc_tdf.cpp:55-63).
static void linspace(float a, float b, int n, float* v) {
    if (n == 1) v[0] = a;
    if (n < 2) return;
    const float step = (b - a) / (float)(n - 1);
    for (int i = 0; i < n; i++) v[i] = i < n / 2 ? a + step * (float)i : b - step * (float)(n - 1 - i);
}

void demix_window(int chunk, float* window, int rules) {
    const int fade = chunk / 10;
    for (int t = 0; t < chunk; t++) window[t] = 1.0f;
    if (rules == STX_DEMIX_MSST) {                                          // tfc_tdf :465-469
        if (fade > 0) {
            linspace(1.0f, 0.0f, fade, window + chunk - fade);
            linspace(0.0f, 1.0f, fade, window);
        }
        return;
    }
    // torch.linspace(0, 1, fade) in float32, from both ends (:303-309); fade_in stays zero when
    // fade == 1 (only fade > 1 fills it).
    std::vector<float> fade_in(std::max(fade, 0), 0.0f);
    if (fade > 1) {
        const float stp = 1.0f / (float)(fade - 1);
        for (int i = 0; i < fade; i++)
            fade_in[i] = i < fade / 2 ? (float)i * stp : 1.0f - (float)(fade - 1 - i) * stp;
    }
    for (int i = 0; i < fade; i++) {                                        // :310-313
        window[i] *= fade_in[i];
        window[chunk - 1 - i] *= fade_in[i];
    }
}

}  // namespace stx

using namespace stx;

extern "C" {

STX_API int stx_demix_step(int chunk, int num_overlap, float overlap) {
    if (chunk <= 0) return 0;
    if (overlap < 0.0f) return num_overlap > 0 ? chunk / num_overlap : 0;                  // :442
    if (overlap >= 1.0f) return 0;                                                          // :440
    return std::max(1, (int)std::lround(chunk * (1.0 - overlap)));                          // :443
}

STX_API stx_status stx_demix_plan(int64_t len, int chunk, int step, stx_demix_geometry* geom, stx_chunk* chunks,
                                  int64_t capacity) {
    return stx_demix_plan_rules(len, chunk, step, STX_DEMIX_ROFORMER, geom, chunks, capacity);
}

STX_API stx_status stx_demix_plan_rules(int64_t len, int chunk, int step, stx_demix_rules rules,
                                        stx_demix_geometry* geom, stx_chunk* chunks, int64_t capacity) {
    return guard([&] {
        const DemixGeometry g = demix_geometry(len, chunk, step, rules);
        if (geom) {
            STX_REQUIRE(geom->size >= STX_DEMIX_GEOMETRY_MIN_SIZE, "demix geometry: size %u is below the V1 minimum %u",
                        geom->size, STX_DEMIX_GEOMETRY_MIN_SIZE);
            stx_demix_geometry o{};
            o.size = geom->size;
            o.len = g.len;
            o.padded_len = g.padded_len;
            o.chunk = g.chunk;
            o.step = g.step;
            o.border = g.border;
            o.fade = g.fade;
            o.reflect_border = g.reflect_border;
            o.n_chunks = g.n_chunks;
            std::memcpy(geom, &o, std::min<size_t>(geom->size, sizeof o));
        }
        if (!chunks) return;
        STX_REQUIRE(capacity >= g.n_chunks, "chunk table capacity %lld < %lld", (long long)capacity,
                    (long long)g.n_chunks);
        for (int64_t k = 0; k < g.n_chunks; k++) chunks[k] = demix_chunk(g, k);
    });
}

STX_API stx_status stx_demix_window(int chunk, float* window) {
    return stx_demix_window_rules(chunk, STX_DEMIX_ROFORMER, window);
}

STX_API stx_status stx_demix_window_rules(int chunk, stx_demix_rules rules, float* window) {
    return guard([&] {
        STX_REQUIRE(chunk > 0 && window, "bad chunk/window");
        STX_REQUIRE(rules == STX_DEMIX_ROFORMER || rules == STX_DEMIX_MSST, "unknown demix rules %d", rules);
        demix_window(chunk, window, rules);
    });
}

}  // extern "C"
