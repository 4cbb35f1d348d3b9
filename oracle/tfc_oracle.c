/* tfc_oracle.c — TEST INFRASTRUCTURE: CPU restatement of the TFC-TDF (MDX) chunking loops,
 * split at the model call so any model can sit between the chunk builder and the overlap-add:
 *   MSST (TFCTDF::Impl::demix_msst, src/tfc_tdf.cpp:447-495): ZFTurbo's loop with
 *     linspace fades (:55-63,465-469), short chunks reflect-padded above chunk / 2 (:474-478), the
 *     first chunk without fade-in and the chunk after which i >= Lp without fade-out (:484-486);
 *   UVR (TFCTDF::Impl::demix_uvr, :407-441): `trim` zeros in front, chunks of `chunk` every
 *     `step` over M samples zero-filled past the mix, np.hanning of each chunk's actual length
 *     (or 1 when overlap == 0), double accumulation, and the division at the trim offset;
 *   the post-processing of TFCTDF::separate (:569-595): compensation and the complement stem.
 */
#include "stx_oracle.h"

#include <math.h>

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif
#include <stdlib.h>
#include <string.h>

/* torch.linspace in float32, from both ends (src/tfc_tdf.cpp:55-63). */
static void linspace_f(float a, float b, int n, float* v) {
    if (n == 1) v[0] = a;
    if (n < 2) return;
    const float step = (b - a) / (float)(n - 1);
    for (int i = 0; i < n; i++) v[i] = i < n / 2 ? a + step * (float)i : b - step * (float)(n - 1 - i);
}

void orc_msst_window(int chunk, float* window) {
    const int fade = chunk / 10;
    for (int i = 0; i < chunk; i++) window[i] = 1.0f;
    if (fade > 0) {
        linspace_f(1.0f, 0.0f, fade, window + chunk - fade);
        linspace_f(0.0f, 1.0f, fade, window);
    }
}

static long msst_padded(long len, int chunk, int step, int* border, int* pad) {
    *border = chunk - step;
    *pad = len > 2L * *border && *border > 0;
    return *pad ? len + 2L * *border : len;
}

long orc_msst_n_chunks(long len, int chunk, int step) {
    int border, pad;
    const long Lp = msst_padded(len, chunk, step, &border, &pad);
    return (Lp + step - 1) / step;
}

int orc_msst_chunks(const float* mix, int C, long len, int chunk, int step, float* parts) {
    int border, pad;
    const long Lp = msst_padded(len, chunk, step, &border, &pad);
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
        const int n = (int)(chunk < Lp - i ? chunk : Lp - i);
        for (int c = 0; c < C; c++) {
            const float* src = x + (size_t)c * Lp + i;
            float* dst = parts + ((size_t)k * C + c) * chunk;
            memcpy(dst, src, sizeof(float) * n);
            if (n < chunk) {
                if (n > chunk / 2) {
                    orc_reflect_pad(src, n, 0, chunk - n, tmp);
                    for (int t = 0; t < chunk; t++) dst[t] = (float)tmp[t];
                } else {
                    for (int t = n; t < chunk; t++) dst[t] = 0.0f;
                }
            }
        }
    }
    free(x);
    free(tmp);
    return 0;
}

int orc_msst_ola(const float* y, int S, int C, long len, int chunk, int step, float* out) {
    int border, pad;
    const long Lp = msst_padded(len, chunk, step, &border, &pad);
    const int fade = chunk / 10;
    float* window = (float*)malloc(sizeof(float) * chunk);
    float* w = (float*)malloc(sizeof(float) * chunk);
    orc_msst_window(chunk, window);
    double* result = (double*)calloc((size_t)S * C * Lp, sizeof(double));
    double* counter = (double*)calloc(Lp, sizeof(double));
    long k = 0;
    for (long i = 0; i < Lp; k++) {
        const long start = i;
        const int n = (int)(chunk < Lp - i ? chunk : Lp - i);
        i += step;
        memcpy(w, window, sizeof(float) * chunk);
        if (i - step == 0) {
            for (int t = 0; t < fade; t++) w[t] = 1.0f;
        } else if (i >= Lp) {
            for (int t = chunk - fade; t < chunk; t++) w[t] = 1.0f;
        }
        const float* yk = y + (size_t)k * S * C * chunk;
        for (int q = 0; q < S * C; q++)
            for (int t = 0; t < n; t++) result[(size_t)q * Lp + start + t] += (double)yk[(size_t)q * chunk + t] * w[t];
        for (int t = 0; t < n; t++) counter[start + t] += w[t];
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

/* UVR geometry (src/tfc_tdf.cpp:410-415): trim = n_fft / 2, gen = chunk - 2 trim,
 * M = trim + len + gen + trim - len % gen, step = chunk - n_fft for overlap < 0, else
 * (int64)((1 - overlap) * chunk). Returns the number of chunks, -1 for gen <= 0 (the
 * reference's runtime_error) and -2 for step <= 0 (its invalid_argument). */
long orc_uvr_geometry(long len, int chunk, int n_fft, float overlap, long* M, long* step) {
    const int trim = n_fft / 2, gen = chunk - 2 * trim;
    if (gen <= 0) return -1;
    *M = (long)trim + len + gen + trim - len % gen;
    *step = overlap < 0 ? chunk - n_fft : (long)((1.0 - (double)overlap) * chunk);
    if (*step <= 0) return -2;
    return (*M + *step - 1) / *step;
}

int orc_uvr_chunks(const float* mix, int C, long len, int chunk, int n_fft, float overlap, float* parts) {
    long M, step;
    const long n = orc_uvr_geometry(len, chunk, n_fft, overlap, &M, &step);
    if (n < 0) return (int)n;
    const int trim = n_fft / 2;
    float* x = (float*)calloc((size_t)C * M, sizeof(float));
    for (int c = 0; c < C; c++) memcpy(x + (size_t)c * M + trim, mix + (size_t)c * len, sizeof(float) * len);
    long k = 0;
    for (long i = 0; i < M; i += step, k++) {
        const int actual = (int)(chunk < M - i ? chunk : M - i);
        for (int c = 0; c < C; c++) {
            float* dst = parts + ((size_t)k * C + c) * chunk;
            for (int t = 0; t < chunk; t++) dst[t] = 0.0f;
            memcpy(dst, x + (size_t)c * M + i, sizeof(float) * actual);
        }
    }
    free(x);
    return 0;
}

/* np.hanning(n) (src/tfc_tdf.cpp:65-71). */
static void hanning_d(int n, double* w) {
    for (int i = 0; i < n; i++) w[i] = 1.0;
    if (n > 1)
        for (int i = 0; i < n; i++) w[i] = 0.5 - 0.5 * cos(2.0 * M_PI * i / (n - 1));
}

int orc_uvr_ola(const float* y, int S, int C, long len, int chunk, int n_fft, float overlap, float* out) {
    long M, step;
    const long n = orc_uvr_geometry(len, chunk, n_fft, overlap, &M, &step);
    if (n < 0) return (int)n;
    const int trim = n_fft / 2;
    double* result = (double*)calloc((size_t)S * C * M, sizeof(double));
    double* divider = (double*)calloc(M, sizeof(double));
    double* w = (double*)malloc(sizeof(double) * chunk);
    long k = 0;
    for (long i = 0; i < M; i += step, k++) {
        const int actual = (int)(chunk < M - i ? chunk : M - i);
        if (overlap == 0) {
            for (int t = 0; t < actual; t++) w[t] = 1.0;
        } else {
            hanning_d(actual, w);
        }
        const float* yk = y + (size_t)k * S * C * chunk;
        for (int q = 0; q < S * C; q++)
            for (int t = 0; t < actual; t++) result[(size_t)q * M + i + t] += (double)yk[(size_t)q * chunk + t] * w[t];
        for (int t = 0; t < actual; t++) divider[i + t] += w[t];
    }
    for (int q = 0; q < S * C; q++)
        for (long t = 0; t < len; t++) out[(size_t)q * len + t] = (float)(result[(size_t)q * M + trim + t] / divider[trim + t]);
    free(result);
    free(divider);
    free(w);
    return 0;
}

/* TFCTDF::separate's post-processing (src/tfc_tdf.cpp:582-595): est *= compensate (when != 1),
 * then with `complement` one more plane: mix - stem 0 - stem 1 - ... in float. est holds
 * [S][plane] and, with complement, room for [S + 1][plane]. */
void orc_tfc_post(const float* mix, long plane, int S, float compensate, int complement, float* est) {
    if (compensate != 1.0f)
        for (long i = 0; i < (long)S * plane; i++) est[i] *= compensate;
    if (complement) {
        float* rest = est + (size_t)S * plane;
        for (long i = 0; i < plane; i++) {
            float v = mix[i];
            for (int k = 0; k < S; k++) v -= est[(size_t)k * plane + i];
            rest[i] = v;
        }
    }
}
