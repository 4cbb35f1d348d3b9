// bands_host.cpp — host-side band maps and band tables of the RoFormer spectral path.
//
//   stx_mel_band_map: MelBandRoformer's freqs_per_band, i.e. tools/convert_roformer.py:107-115:
//     librosa.filters.mel(sr, n_fft, n_mels) (Slaney scale, fmin 0, fmax sr/2, htk=False,
//     norm='slaney'), then fb[0][0] = 1 and fb[-1][-1] = 1, and band b holds the bins k with
//     fb[b][k] > 0. A triangle weight is positive exactly when the bin frequency lies strictly
//     between the band's outer mel vertices (the Slaney normalisation only scales by a positive
//     factor), so the map is computed from those comparisons in double precision.
//   stx_bs_band_map: BSRoformer's contiguous bands, tools/convert_roformer.py:118-124.
//   stx_bands_layout: the constructor's tables and checks, src/roformer.cpp:394-411 (offsets
//     band_freq_off, band_feat_off with dim_in(b) = size * channels * 2 (:85), and
//     bands_per_freq), without touching a device.
#include <cmath>
#include <cstring>
#include <vector>

#include "bands_host.hpp"
#include "common.hpp"

namespace stx {

// librosa's Slaney mel scale (hz_to_mel / mel_to_hz with htk=False).
static double hz_to_mel(double f) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    return f >= min_log_hz ? min_log_mel + std::log(f / min_log_hz) / logstep : f / f_sp;
}

static double mel_to_hz(double m) {
    const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / f_sp;
    const double logstep = std::log(6.4) / 27.0;
    return m >= min_log_mel ? min_log_hz * std::exp(logstep * (m - min_log_mel)) : f_sp * m;
}

void mel_band_lists(int sr, int n_fft, int n_mels, std::vector<std::vector<int>>& bands) {
    const int n_bins = n_fft / 2 + 1;
    // mel_frequencies(n_mels + 2, 0, sr/2): numpy linspace of mels (last point exact), to Hz.
    const int np = n_mels + 2;
    const double mmin = hz_to_mel(0.0), mmax = hz_to_mel(sr / 2.0);
    const double step = (mmax - mmin) / (np - 1);
    std::vector<double> mel_f(np);
    for (int i = 0; i < np; i++) mel_f[i] = mel_to_hz(i == np - 1 ? mmax : i * step + mmin);
    bands.assign(n_mels, {});
    for (int b = 0; b < n_mels; b++) {
        for (int k = 0; k < n_bins; k++) {
            const double fk = (double)k * sr / n_fft;            // fft_frequencies
            bool on = fk > mel_f[b] && fk < mel_f[b + 2];
            if (b == 0 && k == 0) on = true;                     // fb[0][0] = 1
            if (b == n_mels - 1 && k == n_bins - 1) on = true;   // fb[-1, -1] = 1
            if (on) bands[b].push_back(k);
        }
    }
}

void check_band_tables(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs, int64_t n_freqs,
                       int n_bins, int channels, std::vector<int64_t>& freq_off, std::vector<int64_t>& feat_off,
                       std::vector<int32_t>& bpf) {
    STX_REQUIRE(n_bands >= 1 && n_bins >= 1 && channels >= 1 && n_freqs >= 0, "bad band table sizes");
    STX_REQUIRE(band_sizes && (band_freqs || n_freqs == 0), "NULL band table");
    freq_off.assign(1, 0);
    feat_off.assign(1, 0);
    for (int b = 0; b < n_bands; b++) {
        STX_REQUIRE(band_sizes[b] >= 0, "negative band size");
        freq_off.push_back(freq_off.back() + band_sizes[b]);
        feat_off.push_back(feat_off.back() + (int64_t)band_sizes[b] * channels * 2);
    }
    if (freq_off.back() != n_freqs)
        fail(STX_STATUS_RUNTIME_ERROR, "roformer.band_sizes does not match roformer.band_freqs");
    bpf.assign(n_bins, 0);
    for (int64_t i = 0; i < n_freqs; i++) {
        const int f = band_freqs[i];
        if (f < 0 || f >= n_bins) fail(STX_STATUS_RUNTIME_ERROR, "band frequency out of range");
        bpf[f]++;
    }
}

}  // namespace stx

using namespace stx;

extern "C" {

STX_API stx_status stx_mel_band_map(int sample_rate, int n_fft, int n_mels, int32_t* band_sizes,
                                    int32_t* band_freqs, int64_t capacity, int64_t* n_freqs) {
    return guard([&] {
        STX_REQUIRE(sample_rate > 0 && n_fft >= 2 && n_mels >= 1, "bad mel parameters");
        std::vector<std::vector<int>> bands;
        mel_band_lists(sample_rate, n_fft, n_mels, bands);
        int64_t total = 0;
        std::vector<int> covered(n_fft / 2 + 1, 0);
        for (const auto& b : bands) {
            total += (int64_t)b.size();
            for (int k : b) covered[k] = 1;
        }
        // assert mask.any(axis=0).all() (tools/convert_roformer.py:114)
        for (int c : covered)
            if (!c) fail(STX_STATUS_RUNTIME_ERROR, "every frequency must be covered by a band");
        if (n_freqs) *n_freqs = total;
        if (!band_sizes && !band_freqs) return;                  // size query
        STX_REQUIRE(band_sizes && band_freqs, "NULL output");
        STX_REQUIRE(capacity >= total, "band_freqs capacity %lld < %lld", (long long)capacity, (long long)total);
        int64_t o = 0;
        for (int b = 0; b < n_mels; b++) {
            band_sizes[b] = (int32_t)bands[b].size();
            for (int k : bands[b]) band_freqs[o++] = k;
        }
    });
}

STX_API stx_status stx_bs_band_map(const int32_t* freqs_per_bands, int n_bands, int n_fft, int32_t* band_freqs,
                                   int64_t capacity, int64_t* n_freqs) {
    return guard([&] {
        STX_REQUIRE(freqs_per_bands && n_bands >= 1 && n_fft >= 2, "bad band parameters");
        int64_t f = 0;
        for (int b = 0; b < n_bands; b++) {
            STX_REQUIRE(freqs_per_bands[b] >= 0, "negative band size");
            f += freqs_per_bands[b];
        }
        // assert f == stft_n_fft // 2 + 1 (tools/convert_roformer.py:123)
        if (f != n_fft / 2 + 1) fail(STX_STATUS_RUNTIME_ERROR, "freqs_per_bands sum to %lld", (long long)f);
        if (n_freqs) *n_freqs = f;
        if (!band_freqs) return;
        STX_REQUIRE(capacity >= f, "band_freqs capacity too small");
        for (int64_t i = 0; i < f; i++) band_freqs[i] = (int32_t)i;
    });
}

STX_API stx_status stx_bands_layout(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs,
                                    int64_t n_freqs, int n_bins, int channels, int64_t* band_freq_off,
                                    int64_t* band_feat_off, int32_t* bands_per_freq) {
    return guard([&] {
        std::vector<int64_t> fo, fe;
        std::vector<int32_t> bpf;
        check_band_tables(band_sizes, n_bands, band_freqs, n_freqs, n_bins, channels, fo, fe, bpf);
        if (band_freq_off) std::memcpy(band_freq_off, fo.data(), fo.size() * sizeof(int64_t));
        if (band_feat_off) std::memcpy(band_feat_off, fe.data(), fe.size() * sizeof(int64_t));
        if (bands_per_freq) std::memcpy(bands_per_freq, bpf.data(), bpf.size() * sizeof(int32_t));
    });
}

}  // extern "C"
