/* band_oracle.c — TEST INFRASTRUCTURE: CPU restatement of the RoFormer band path.
 *
 *   orc_mel_band_map: tools/convert_roformer.py:107-115 (librosa.filters.mel, Slaney scale,
 *     fmin 0, fmax sr/2, then fb[0][0] = fb[-1][-1] = 1 and mask = fb > 0).
 *   orc_bands_layout: RoFormer constructor tables, src/roformer.cpp:394-411.
 *   orc_band_gather: src/roformer.cpp:226-241.
 *   orc_band_scatter_apply: src/roformer.cpp:251-278 (acc in double, / max(bpf, 1), times z).
 * Spectra are complex double [C][F][T] (the reference's z[c][f * T + t]).
 */
#include "stx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static double hz_to_mel(double f) {
    const double f_min = 0.0, f_sp = 200.0 / 3, min_log_hz = 1000.0;
    const double min_log_mel = (min_log_hz - f_min) / f_sp, logstep = log(6.4) / 27.0;
    double mels = (f - f_min) / f_sp;
    if (f >= min_log_hz) mels = min_log_mel + log(f / min_log_hz) / logstep;
    return mels;
}

static double mel_to_hz(double m) {
    const double f_min = 0.0, f_sp = 200.0 / 3, min_log_hz = 1000.0;
    const double min_log_mel = (min_log_hz - f_min) / f_sp, logstep = log(6.4) / 27.0;
    double hz = f_min + f_sp * m;
    if (m >= min_log_mel) hz = min_log_hz * exp(logstep * (m - min_log_mel));
    return hz;
}

int orc_mel_band_map(int sr, int n_fft, int n_mels, int* band_sizes, int* band_freqs, long cap, long* n_total) {
    const int n_bins = n_fft / 2 + 1, np = n_mels + 2;
    double* mel_f = (double*)malloc(sizeof(double) * np);
    const double lo = hz_to_mel(0.0), hi = hz_to_mel(sr / 2.0), step = (hi - lo) / (np - 1);
    for (int i = 0; i < np; i++) mel_f[i] = mel_to_hz(i == np - 1 ? hi : i * step + lo);
    long o = 0;
    int rc = 0;
    char* covered = (char*)calloc(n_bins, 1);
    for (int b = 0; b < n_mels; b++) {
        int size = 0;
        for (int k = 0; k < n_bins; k++) {
            const double fk = (double)k * sr / n_fft;
            /* weight = max(0, min((fk - mel_f[b]) / fdiff[b], (mel_f[b+2] - fk) / fdiff[b+1])) */
            const double lower = (fk - mel_f[b]) / (mel_f[b + 1] - mel_f[b]);
            const double upper = (mel_f[b + 2] - fk) / (mel_f[b + 2] - mel_f[b + 1]);
            int on = (lower < upper ? lower : upper) > 0.0;
            if ((b == 0 && k == 0) || (b == n_mels - 1 && k == n_bins - 1)) on = 1;
            if (on) {
                if (o < cap) band_freqs[o] = k;
                o++;
                size++;
                covered[k] = 1;
            }
        }
        band_sizes[b] = size;
    }
    for (int k = 0; k < n_bins; k++)
        if (!covered[k]) rc = -2;
    if (n_total) *n_total = o;
    free(mel_f);
    free(covered);
    return o > cap ? -1 : rc;
}

int orc_bands_layout(const int* band_sizes, int n_bands, const int* band_freqs, long n_freqs, int n_bins,
                     int channels, long* freq_off, long* feat_off, int* bpf) {
    freq_off[0] = 0;
    feat_off[0] = 0;
    for (int b = 0; b < n_bands; b++) {
        freq_off[b + 1] = freq_off[b] + band_sizes[b];
        feat_off[b + 1] = feat_off[b] + (long)band_sizes[b] * channels * 2;
    }
    if (freq_off[n_bands] != n_freqs) return -2;
    for (int f = 0; f < n_bins; f++) bpf[f] = 0;
    for (long i = 0; i < n_freqs; i++) {
        if (band_freqs[i] < 0 || band_freqs[i] >= n_bins) return -2;
        bpf[band_freqs[i]]++;
    }
    return 0;
}

void orc_band_gather(const int* band_sizes, int n_bands, const int* band_freqs, int C, int F, int T,
                     const double* z, float* feat) {
    long foff = 0, eoff = 0;
    for (int b = 0; b < n_bands; b++) {
        float* blk = feat + eoff * T;
        const int din = band_sizes[b] * C * 2;
        for (int j = 0; j < band_sizes[b]; j++) {
            const int f = band_freqs[foff + j];
            for (int c = 0; c < C; c++)
                for (int t = 0; t < T; t++) {
                    const double* v = z + 2 * (((size_t)c * F + f) * T + t);
                    float* p = blk + (size_t)t * din + (j * C + c) * 2;
                    p[0] = (float)v[0];
                    p[1] = (float)v[1];
                }
        }
        foff += band_sizes[b];
        eoff += din;
    }
}

void orc_band_scatter_apply(const int* band_sizes, int n_bands, const int* band_freqs, int C, int F, int T,
                            const float* masks, int S, const double* z, int zero_dc, double* out) {
    long total = 0, nf = 0;
    for (int b = 0; b < n_bands; b++) {
        total += (long)band_sizes[b] * C * 2;
        nf += band_sizes[b];
    }
    int* bpf = (int*)calloc(F, sizeof(int));
    for (long i = 0; i < nf; i++) bpf[band_freqs[i]]++;
    double* acc = (double*)malloc(sizeof(double) * 2 * (size_t)C * F * T);
    for (int s = 0; s < S; s++) {
        const float* m = masks + (size_t)s * total * T;
        memset(acc, 0, sizeof(double) * 2 * (size_t)C * F * T);
        long foff = 0, eoff = 0;
        for (int b = 0; b < n_bands; b++) {
            const int din = band_sizes[b] * C * 2;
            const float* mb = m + eoff * T;
            for (int j = 0; j < band_sizes[b]; j++) {
                const int f = band_freqs[foff + j];
                for (int c = 0; c < C; c++)
                    for (int t = 0; t < T; t++) {
                        const float* p = mb + (size_t)t * din + (j * C + c) * 2;
                        double* a = acc + 2 * (((size_t)c * F + f) * T + t);
                        a[0] += p[0];
                        a[1] += p[1];
                    }
            }
            foff += band_sizes[b];
            eoff += din;
        }
        for (int c = 0; c < C; c++) {
            for (int f = 0; f < F; f++) {
                const double denom = bpf[f] > 1 ? bpf[f] : 1;
                for (int t = 0; t < T; t++) {
                    const size_t i = ((size_t)c * F + f) * T + t;
                    const double qr = acc[2 * i] / denom, qi = acc[2 * i + 1] / denom;
                    const double zr = z[2 * i], zi = z[2 * i + 1];
                    double* o = out + 2 * ((size_t)s * C * F * T + i);
                    o[0] = zr * qr - zi * qi;
                    o[1] = zr * qi + zi * qr;
                }
            }
            if (zero_dc)
                for (int t = 0; t < T; t++) {
                    double* o = out + 2 * ((size_t)s * C * F * T + (size_t)c * F * T + t);
                    o[0] = 0.0;
                    o[1] = 0.0;
                }
        }
    }
    free(bpf);
    free(acc);
}
