// bands_host.hpp — host-side band tables shared by bands_host.cpp and bands.hip.
#pragma once

#include <cstdint>
#include <vector>

namespace stx {

// Bin lists of the mel bands (see bands_host.cpp).
void mel_band_lists(int sr, int n_fft, int n_mels, std::vector<std::vector<int>>& bands);

// The RoFormer constructor's checks and tables (src/roformer.cpp:394-411); throws stx::Error.
void check_band_tables(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs, int64_t n_freqs,
                       int n_bins, int channels, std::vector<int64_t>& freq_off, std::vector<int64_t>& feat_off,
                       std::vector<int32_t>& bpf);

}  // namespace stx
