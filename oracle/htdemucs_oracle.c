/* htdemucs_oracle.c — CPU oracle (test infrastructure) for the HTDemucs host pre/post-processing
 * around the model graph: the complex-as-channels pack and the global mean/std normalisation
 * of one segment, the inverse (denormalise + time-branch add), and apply_model's split: the
 * mono-mix normalisation, TensorChunk padding, triangular weights, center_trim and the
 * weighted overlap-add, all in the reference's arithmetic and order. */
#include <math.h>
#include <stdint.h>

#include "stx_oracle.h"

/* mean_of / std_of (src/htdemucs.cpp:293-302): double sums in index order, unbiased std. */
void orc_mean_std(const float* x, int64_t n, double* mean, double* sd) {
    double s = 0;
    for (int64_t i = 0; i < n; i++) s += x[i];
    const double m = s / (double)n;
    double q = 0;
    for (int64_t i = 0; i < n; i++) {
        const double d = x[i] - m;
        q += d * d;
    }
    *mean = m;
    *sd = sqrt(q / (double)(n - 1));
}

/* Complex-as-channels pack (src/htdemucs.cpp:424-432): spec is interleaved complex64
 * [C][F*T] (the f-major spectrum); mag[2c] = re, mag[2c+1] = im, each [F*T]. Then
 * (v - mean) / (1e-5 + sd) with the moments of all of mag (:434-436). */
void orc_cac_normalize(const float* spec, int C, int64_t FT, double mean, double sd, float* mag) {
    for (int c = 0; c < C; c++)
        for (int64_t i = 0; i < FT; i++) {
            mag[(2 * c) * FT + i] = (float)((spec[2 * (c * FT + i)] - mean) / (1e-5 + sd));
            mag[(2 * c + 1) * FT + i] = (float)((spec[2 * (c * FT + i) + 1] - mean) / (1e-5 + sd));
        }
}

/* The waveform branch's normalisation (src/htdemucs.cpp:438-441). */
void orc_normalize(const float* x, int64_t n, double mean, double sd, float* y) {
    for (int64_t i = 0; i < n; i++) y[i] = (float)((x[i] - mean) / (1e-5 + sd));
}

/* Denormalise the spectral branch (src/htdemucs.cpp:465-468): ox [S][2C][F*T] ->
 * spec [S][C][F*T] complex, re * sd + mean and im * sd + mean in double, stored as complex64
 * (the precision the device iSTFT takes). */
void orc_cac_denormalize(const float* ox, int S, int C, int64_t FT, double mean, double sd, float* spec) {
    for (int s = 0; s < S; s++)
        for (int c = 0; c < C; c++) {
            const float* re = ox + (int64_t)(s * 2 * C + 2 * c) * FT;
            const float* im = ox + (int64_t)(s * 2 * C + 2 * c + 1) * FT;
            float* o = spec + 2 * (int64_t)(s * C + c) * FT;
            for (int64_t i = 0; i < FT; i++) {
                o[2 * i] = (float)(re[i] * sd + mean);
                o[2 * i + 1] = (float)(im[i] * sd + mean);
            }
        }
}

/* Time branch denormalise + add of the spectral branch's iSTFT (src/htdemucs.cpp:469-470):
 * out = (float)(t * sd + mean) + y, the add in float. */
void orc_time_add(const float* t, const float* y, int64_t n, double mean, double sd, float* out) {
    for (int64_t i = 0; i < n; i++) {
        const float a = (float)(t[i] * sd + mean);
        out[i] = a + y[i];
    }
}

/* Mono-mix normalisation of separate() (src/htdemucs.cpp:539-549): mono[i] = (float)(sum_c x / C),
 * ref_mean / ref_std = max(std, 1e-8) of mono, mix = (float)((x - ref_mean) / ref_std).
 * stats[0] = ref_mean, stats[1] = ref_std. */
void orc_mix_normalize(const float* mix, int C, int64_t len, float* out, double* stats) {
    double s = 0;
    for (int64_t i = 0; i < len; i++) {
        double m = 0;
        for (int c = 0; c < C; c++) m += mix[c * len + i];
        s += (float)(m / C);
    }
    const double mean = s / (double)len;
    double q = 0;
    for (int64_t i = 0; i < len; i++) {
        double m = 0;
        for (int c = 0; c < C; c++) m += mix[c * len + i];
        const double d = (float)(m / C) - mean;
        q += d * d;
    }
    double sd = sqrt(q / (double)(len - 1));
    if (sd < 1e-8) sd = 1e-8;
    for (int64_t i = 0; i < C * len; i++) out[i] = (float)((mix[i] - mean) / sd);
    stats[0] = mean;
    stats[1] = sd;
}

/* Triangular split weights (src/htdemucs.cpp:566-573): i + 1 up to seg/2, then seg - i, over
 * their float maximum. */
void orc_split_weights(int seg, float* w) {
    const int half = seg / 2;
    for (int i = 0; i < half; i++) w[i] = (float)(i + 1);
    for (int i = half; i < seg; i++) w[i] = (float)(seg - i);
    float mx = w[0];
    for (int i = 1; i < seg; i++)
        if (w[i] > mx) mx = w[i];
    for (int i = 0; i < seg; i++) w[i] /= mx;
}

/* Stride and chunk count of split() (src/htdemucs.cpp:565-566,589): stride = (int)((1 -
 * overlap) * seg) with overlap 0.25 when negative; chunks start at 0, stride, ... < length. */
int orc_split_count(int length, int seg, float overlap, int* stride) {
    const double ov = overlap < 0.0f ? 0.25 : (double)overlap;
    const int st = (int)((1.0 - ov) * seg);
    if (st <= 0) return -1;
    *stride = st;
    return (length + st - 1) / st;
}

/* The padded segments of one view (src/htdemucs.cpp:552-561, :589-593): chunk k of the view
 * [offset, offset + length) of buf [C][total] starts at off = k * stride, has
 * min(seg, length - off) samples, and is centre-padded to seg by reading buf around it where
 * buf has samples and zeros beyond: parts[k][c][i] = buf[c][start + i] with
 * start = offset + off - (seg - chunk_len) / 2. */
void orc_segments(const float* buf, int C, int64_t total, int64_t offset, int length, int seg, int stride,
                  float* parts) {
    const int n = (length + stride - 1) / stride;
    for (int k = 0; k < n; k++) {
        const int off = k * stride;
        const int clen = seg < length - off ? seg : length - off;
        const int64_t start = offset + off - (seg - clen) / 2;
        for (int c = 0; c < C; c++)
            for (int i = 0; i < seg; i++) {
                const int64_t j = start + i;
                parts[((int64_t)k * C + c) * seg + i] = (j >= 0 && j < total) ? buf[c * total + j] : 0.0f;
            }
    }
}

/* The weighted overlap-add of split() (src/htdemucs.cpp:594-606): y [n_chunks][tracks][seg]
 * are the model outputs of the chunks (tracks = S * C); each is center-trimmed by
 * (seg - chunk_len) / 2, weighted and summed in chunk order in float, then divided by the
 * summed weights. out [tracks][length]. */
void orc_split_ola(const float* y, int tracks, int length, int seg, int stride, float* out, float* sum_w) {
    const int n = (length + stride - 1) / stride;
    for (int64_t i = 0; i < (int64_t)tracks * length; i++) out[i] = 0.0f;
    for (int i = 0; i < length; i++) sum_w[i] = 0.0f;
    const int half = seg / 2;
    const float mx = (float)(seg - half > half ? seg - half : half);
    for (int k = 0; k < n; k++) {
        const int off = k * stride;
        const int clen = seg < length - off ? seg : length - off;
        const int trim = (seg - clen) / 2;
        for (int sc = 0; sc < tracks; sc++)
            for (int i = 0; i < clen; i++) {
                const float wi = (float)(i < half ? i + 1 : seg - i) / mx;
                const float p = wi * y[((int64_t)k * tracks + sc) * seg + trim + i];
                out[(int64_t)sc * length + off + i] += p;
            }
        for (int i = 0; i < clen; i++) sum_w[off + i] += (float)(i < half ? i + 1 : seg - i) / mx;
    }
    for (int sc = 0; sc < tracks; sc++)
        for (int i = 0; i < length; i++) out[(int64_t)sc * length + i] /= sum_w[i];
}
