// demix_host.hpp — chunk geometry of the overlap-add demix, shared by demix_host.cpp and demix.hip.
#pragma once

#include <cstdint>

#include "stx.h"

namespace stx {

struct DemixGeometry {
    int64_t len = 0;             // samples per channel of the input
    int64_t padded_len = 0;      // Lp: len + 2 * border when the borders are reflect-padded
    int64_t n_chunks = 0;
    int chunk = 0, step = 0;
    int border = 0;              // chunk - step
    int fade = 0;                // chunk / 10
    int reflect_border = 0;      // len > 2 * border && border > 0
    int rules = 0;               // STX_DEMIX_ROFORMER or STX_DEMIX_MSST
};

DemixGeometry demix_geometry(int64_t len, int chunk, int step, int rules = STX_DEMIX_ROFORMER);   // throws stx::Error
stx_chunk demix_chunk(const DemixGeometry& g, int64_t k);
void demix_window(int chunk, float* window, int rules = STX_DEMIX_ROFORMER);

}  // namespace stx
