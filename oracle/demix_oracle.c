/* demix_oracle.c — TEST INFRASTRUCTURE: CPU restatement of RoFormer::Impl::demix
 * (src/roformer.cpp:286-351) and n_chunks (:353-357), split at the separator call so that any
 * separator can sit between orc_demix_chunks and orc_demix_ola:
 *   orc_demix_chunks: the chunk inputs part[k][c][chunk] the reference hands to run()
 *     (:289-331: border reflect pad rounded to float, short chunks reflect- or zero-padded);
 *   orc_demix_ola: the weighted accumulation into result/counter in double, chunk by chunk,
 *     the division at the border offset and nan_to_num (:334-350).
 */
#include "stx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static long padded_len(long len, int chunk, int step, int* border, int* pad) {
    *border = chunk - step;
    *pad = len > 2L * *border && *border > 0;
    return *pad ? len + 2L * *border : len;
}

long orc_demix_n_chunks(long len, int chunk, int step) {
    int border, pad;
    const long Lp = padded_len(len, chunk, step, &border, &pad);
    return (Lp + step - 1) / step;
}

void orc_demix_window(int chunk, float* window) {
    const int fade = chunk / 10;
    float* fade_in = (float*)calloc(fade > 0 ? fade : 1, sizeof(float));
    if (fade > 1) {
        const float stp = 1.0f / (float)(fade - 1);
        for (int i = 0; i < fade; i++)
            fade_in[i] = i < fade / 2 ? (float)i * stp : 1.0f - (float)(fade - 1 - i) * stp;
    }
    for (int i = 0; i < chunk; i++) window[i] = 1.0f;
    for (int i = 0; i < fade; i++) {
        window[i] *= fade_in[i];
        window[chunk - 1 - i] *= fade_in[i];
    }
    free(fade_in);
}

int orc_demix_chunks(const float* mix, int C, long len, int chunk, int step, float* parts) {
    int border, pad;
    const long Lp = padded_len(len, chunk, step, &border, &pad);
    float* x = (float*)malloc(sizeof(float) * (size_t)C * Lp);
    double* tmp = (double*)malloc(sizeof(double) * (Lp > chunk ? Lp : chunk));
    for (int c = 0; c < C; c++) {
        const float* src = mix + (size_t)c * len;
        if (pad) {
            if (orc_reflect_pad(src, (int)len, border, border, tmp)) {
                free(x);
                free(tmp);
                return -2;
            }
            for (long i = 0; i < Lp; i++) x[(size_t)c * Lp + i] = (float)tmp[i];
        } else {
            memcpy(x + (size_t)c * Lp, src, sizeof(float) * len);
        }
    }
    long k = 0;
    for (long i = 0; i < Lp; i += step, k++) {
        const int length = (int)(chunk < Lp - i ? chunk : Lp - i);
        for (int c = 0; c < C; c++) {
            const float* src = x + (size_t)c * Lp + i;
            float* dst = parts + ((size_t)k * C + c) * chunk;
            memcpy(dst, src, sizeof(float) * length);
            if (length < chunk) {
                if (length > chunk / 2 + 1) {
                    orc_reflect_pad(src, length, 0, chunk - length, tmp);
                    for (int t = 0; t < chunk; t++) dst[t] = (float)tmp[t];
                } else {
                    for (int t = length; t < chunk; t++) dst[t] = 0.0f;
                }
            }
        }
    }
    free(x);
    free(tmp);
    return 0;
}

int orc_demix_ola(const float* y, int S, int C, long len, int chunk, int step, float* out) {
    int border, pad;
    const long Lp = padded_len(len, chunk, step, &border, &pad);
    const int fade = chunk / 10;
    float* window = (float*)malloc(sizeof(float) * chunk);
    float* w = (float*)malloc(sizeof(float) * chunk);
    orc_demix_window(chunk, window);
    double* result = (double*)calloc((size_t)S * C * Lp, sizeof(double));
    double* counter = (double*)calloc(Lp, sizeof(double));
    long k = 0;
    for (long i = 0; i < Lp; i += step, k++) {
        const int length = (int)(chunk < Lp - i ? chunk : Lp - i);
        const float* yk = y + (size_t)k * S * C * chunk;
        memcpy(w, window, sizeof(float) * chunk);
        if (i == 0) {
            for (int t = 0; t < fade; t++) w[t] = 1.0f;
        } else if (i + chunk >= Lp) {
            for (int t = chunk - fade; t < chunk; t++) w[t] = 1.0f;
        }
        for (int q = 0; q < S * C; q++)
            for (int t = 0; t < length; t++) result[(size_t)q * Lp + i + t] += (double)yk[(size_t)q * chunk + t] * w[t];
        for (int t = 0; t < length; t++) counter[i + t] += w[t];
    }
    const long off = pad ? border : 0;
    for (int q = 0; q < S * C; q++)
        for (long t = 0; t < len; t++) {
            const double v = result[(size_t)q * Lp + off + t] / counter[off + t];
            out[(size_t)q * len + t] = isfinite(v) ? (float)v : 0.0f;
        }
    free(window);
    free(w);
    free(result);
    free(counter);
    return 0;
}
