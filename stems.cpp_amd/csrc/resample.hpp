// resample.hpp — what other translation units need of resample.hip's plans.
#pragma once

#include "stx.h"

namespace stx {

// The source and destination rates of a plan (INVALID_ARGUMENT for NULL).
void resampler_rates(const stx_resampler* r, int& src, int& dst);

}  // namespace stx
