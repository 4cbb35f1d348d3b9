/* stft_oracle.c — TEST INFRASTRUCTURE: CPU restatement of src/stft.h in plain C.
 *
 * The operation order follows the reference exactly (complex products as (ac - bd, ad + bc),
 * scalar factors applied left to right, envelope and signal accumulated frame by frame), and
 * the file is built with -ffp-contract=off, so on x86-64 its results are bit-identical to
 * the reference header compiled with g++. tests/test_oracle_stft.py checks exactly that
 * against the golden vectors in tests/golden/.
 */
#include "stx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

static int is_pow2(int n) { return n >= 2 && (n & (n - 1)) == 0; }

/* st::FFT::FFT + run (src/stft.h:21-49). */
int orc_fft(double* a, int n, int inverse) {
    if (!is_pow2(n)) return -1;
    int bits = 0;
    while ((1 << bits) < n) bits++;
    double* twr = (double*)malloc(sizeof(double) * (n / 2));
    double* twi = (double*)malloc(sizeof(double) * (n / 2));
    for (int i = 0; i < n / 2; i++) {           /* std::polar(1.0, -2 pi i / n) (:30) */
        const double th = -2.0 * M_PI * i / n;
        twr[i] = 1.0 * cos(th);
        twi[i] = 1.0 * sin(th);
    }
    for (int i = 0; i < n; i++) {               /* bit reversal (:25-29, :36) */
        int r = 0;
        for (int b = 0; b < bits; b++) r |= ((i >> b) & 1) << (bits - 1 - b);
        if (i < r) {
            double t0 = a[2 * i], t1 = a[2 * i + 1];
            a[2 * i] = a[2 * r];
            a[2 * i + 1] = a[2 * r + 1];
            a[2 * r] = t0;
            a[2 * r + 1] = t1;
        }
    }
    for (int len = 2; len <= n; len <<= 1) {    /* butterflies (:37-48) */
        const int step = n / len, h = len / 2;
        for (int i = 0; i < n; i += len) {
            for (int j = 0; j < h; j++) {
                const double wr = twr[j * step];
                const double wi = inverse ? -twi[j * step] : twi[j * step];
                double* pu = a + 2 * (i + j);
                double* pv = a + 2 * (i + j + h);
                const double ur = pu[0], ui = pu[1];
                const double vr = pv[0] * wr - pv[1] * wi;
                const double vi = pv[0] * wi + pv[1] * wr;
                pu[0] = ur + vr;
                pu[1] = ui + vi;
                pv[0] = ur - vr;
                pv[1] = ui - vi;
            }
        }
    }
    free(twr);
    free(twi);
    return 0;
}

/* st::VRFFT (src/vr_dsp.h:11-37): Bluestein's transform for any n on top of the radix-2 FFT of
 * m >= 2n - 1 points: chirp c[i] = polar(1, -pi i^2 / n), kernel conj(c) wrapped around and
 * transformed once, then x -> (x c) * FFT -> * kernel -> inverse FFT -> * c / m; the inverse
 * transform conjugates on the way in and out. Unnormalised, like orc_fft. */
int orc_vrfft(double* x, int n, int inverse) {
    if (n < 1) return -1;
    int m = 1;
    while (m < 2 * n - 1) m *= 2;
    double* chirp = (double*)malloc(sizeof(double) * 2 * n);
    double* kern = (double*)calloc(2 * (size_t)m, sizeof(double));
    double* a = (double*)calloc(2 * (size_t)m, sizeof(double));
    for (int i = 0; i < n; i++) {
        const double th = -M_PI * (double)i * i / n;
        chirp[2 * i] = 1.0 * cos(th);
        chirp[2 * i + 1] = 1.0 * sin(th);
        kern[2 * i] = chirp[2 * i];
        kern[2 * i + 1] = -chirp[2 * i + 1];
        if (i) {
            kern[2 * (m - i)] = kern[2 * i];
            kern[2 * (m - i) + 1] = kern[2 * i + 1];
        }
    }
    orc_fft(kern, m, 0);
    for (int i = 0; i < n; i++) {
        const double xr = x[2 * i], xi = inverse ? -x[2 * i + 1] : x[2 * i + 1];
        const double cr = chirp[2 * i], ci = chirp[2 * i + 1];
        a[2 * i] = xr * cr - xi * ci;
        a[2 * i + 1] = xr * ci + xi * cr;
    }
    orc_fft(a, m, 0);
    for (int i = 0; i < m; i++) {
        const double ar = a[2 * i], ai = a[2 * i + 1], kr = kern[2 * i], ki = kern[2 * i + 1];
        a[2 * i] = ar * kr - ai * ki;
        a[2 * i + 1] = ar * ki + ai * kr;
    }
    orc_fft(a, m, 1);
    for (int i = 0; i < n; i++) {
        const double ar = a[2 * i], ai = a[2 * i + 1], cr = chirp[2 * i], ci = chirp[2 * i + 1];
        const double vr = (ar * cr - ai * ci) / (double)m, vi = (ar * ci + ai * cr) / (double)m;
        x[2 * i] = vr;
        x[2 * i + 1] = inverse ? -vi : vi;
    }
    free(chirp);
    free(kern);
    free(a);
    return 0;
}

/* The FFT the reference's torch_stft / torch_istft template is instantiated with: st::FFT for
 * powers of two, st::VRFFT otherwise (src/tfc_tdf.cpp:551-552). */
static int any_fft(double* a, int n, int inverse) { return is_pow2(n) ? orc_fft(a, n, inverse) : orc_vrfft(a, n, inverse); }

int orc_hann_periodic(double* w, int n) {
    for (int i = 0; i < n; i++) w[i] = 0.5 - 0.5 * cos(2.0 * M_PI * i / n);
    return 0;
}

int orc_reflect_pad(const float* x, int n, int left, int right, double* y) {
    if (n <= left || n <= right) return -2;
    const int total = n + left + right;
    for (int i = 0; i < total; i++) {
        int j = i - left;
        if (j < 0) j = -j;
        if (j >= n) j = 2 * (n - 1) - j;
        y[i] = x[j];
    }
    return 0;
}

/* Frames of a padded signal xp through the FFT: out[f * T + t] = FFT(xp[start..] * win)[f] * norm. */
static int frames_fft(const double* xp, int n_fft, int T, long first, long hop, int F, double norm,
                      double* out) {
    double* win = (double*)malloc(sizeof(double) * n_fft);
    double* buf = (double*)malloc(sizeof(double) * 2 * n_fft);
    orc_hann_periodic(win, n_fft);
    for (int t = 0; t < T; t++) {
        const long start = first + (long)t * hop;
        for (int i = 0; i < n_fft; i++) {
            buf[2 * i] = xp[start + i] * win[i];
            buf[2 * i + 1] = 0.0;
        }
        any_fft(buf, n_fft, 0);
        for (int f = 0; f < F; f++) {
            out[2 * ((size_t)f * T + t)] = buf[2 * f] * norm;
            out[2 * ((size_t)f * T + t) + 1] = buf[2 * f + 1] * norm;
        }
    }
    free(win);
    free(buf);
    return 0;
}

int orc_torch_stft(const float* x, int len, int n_fft, int hop, int normalized, double* spec, int* n_frames) {
    if (n_fft < 2) return -1;
    const int F = n_fft / 2 + 1;
    double* xp = (double*)malloc(sizeof(double) * ((size_t)len + n_fft));
    if (orc_reflect_pad(x, len, n_fft / 2, n_fft / 2, xp)) {
        free(xp);
        return -2;
    }
    const double norm = normalized ? 1.0 / sqrt((double)n_fft) : 1.0;
    const int T = len / hop + 1;
    if (n_frames) *n_frames = T;
    frames_fft(xp, n_fft, T, 0, hop, F, norm, spec);
    free(xp);
    return 0;
}

int orc_htdemucs_spec(const float* x, int len, int n_fft, double* spec, int* n_frames) {
    if (!is_pow2(n_fft)) return -1;
    const int hl = n_fft / 4;
    const int le = (len + hl - 1) / hl;
    const int pad = hl / 2 * 3;
    const int right = pad + le * hl - len;
    const int n1 = len + pad + right;
    double* p = (double*)malloc(sizeof(double) * n1);
    float* xf = (float*)malloc(sizeof(float) * n1);
    double* xp = (double*)malloc(sizeof(double) * ((size_t)n1 + n_fft));
    int rc = orc_reflect_pad(x, len, pad, right, p);
    if (!rc) {
        for (int i = 0; i < n1; i++) xf[i] = (float)p[i];      /* rounded to float (:84-88) */
        rc = orc_reflect_pad(xf, n1, n_fft / 2, n_fft / 2, xp);
    }
    if (!rc) {
        if (n_frames) *n_frames = le;
        frames_fft(xp, n_fft, le, 2L * hl, hl, n_fft / 2, 1.0 / sqrt((double)n_fft), spec);
    }
    free(p);
    free(xf);
    free(xp);
    return rc;
}

int orc_torch_istft(const double* spec, int n_frames, int n_fft, int hop, int normalized, float* out) {
    if (n_fft < 2 || n_fft % 2) return -1;
    const int F = n_fft / 2 + 1;
    double* win = (double*)malloc(sizeof(double) * n_fft);
    orc_hann_periodic(win, n_fft);
    const size_t full = (size_t)n_fft + (size_t)hop * (n_frames - 1);
    double* y = (double*)calloc(full, sizeof(double));
    double* env = (double*)calloc(full, sizeof(double));
    double* buf = (double*)malloc(sizeof(double) * 2 * n_fft);
    const double norm = (normalized ? sqrt((double)n_fft) : 1.0) / n_fft;
    for (int t = 0; t < n_frames; t++) {
        buf[0] = spec[2 * t];
        buf[1] = 0.0;
        for (int f = 1; f < F - 1; f++) {
            const double re = spec[2 * ((size_t)f * n_frames + t)], im = spec[2 * ((size_t)f * n_frames + t) + 1];
            buf[2 * f] = re;
            buf[2 * f + 1] = im;
            buf[2 * (n_fft - f)] = re;
            buf[2 * (n_fft - f) + 1] = -im;
        }
        buf[2 * (F - 1)] = spec[2 * ((size_t)(F - 1) * n_frames + t)];
        buf[2 * (F - 1) + 1] = 0.0;
        any_fft(buf, n_fft, 1);
        const size_t off = (size_t)t * hop;
        for (int i = 0; i < n_fft; i++) {
            y[off + i] += buf[2 * i] * norm * win[i];
            env[off + i] += win[i] * win[i];
        }
    }
    const int length = hop * (n_frames - 1);
    for (int i = 0; i < length; i++) {
        const size_t j = (size_t)n_fft / 2 + i;
        out[i] = env[j] > 1e-11 ? (float)(y[j] / env[j]) : 0.0f;
    }
    free(win);
    free(y);
    free(env);
    free(buf);
    return 0;
}

int orc_htdemucs_ispec(const double* spec, int n_frames, int n_fft, int length, float* out) {
    if (!is_pow2(n_fft)) return -1;
    const int hl = n_fft / 4, F = n_fft / 2;
    const int pad = hl / 2 * 3;
    const int le_out = hl * ((length + hl - 1) / hl) + 2 * pad;
    const int frames = n_frames + 4;
    double* win = (double*)malloc(sizeof(double) * n_fft);
    orc_hann_periodic(win, n_fft);
    const size_t full = (size_t)n_fft + (size_t)hl * (frames - 1);
    double* y = (double*)calloc(full, sizeof(double));
    double* env = (double*)calloc(full, sizeof(double));
    double* buf = (double*)malloc(sizeof(double) * 2 * n_fft);
    const double norm = sqrt((double)n_fft) / n_fft;
    for (int t = 0; t < frames; t++) {
        const int st = t - 2;
        const size_t off = (size_t)t * hl;
        if (st >= 0 && st < n_frames) {
            buf[0] = spec[2 * st];
            buf[1] = 0.0;
            for (int f = 1; f < F; f++) {
                const double re = spec[2 * ((size_t)f * n_frames + st)], im = spec[2 * ((size_t)f * n_frames + st) + 1];
                buf[2 * f] = re;
                buf[2 * f + 1] = im;
                buf[2 * (n_fft - f)] = re;
                buf[2 * (n_fft - f) + 1] = -im;
            }
            buf[2 * F] = 0.0;
            buf[2 * F + 1] = 0.0;
            orc_fft(buf, n_fft, 1);
            for (int i = 0; i < n_fft; i++) y[off + i] += buf[2 * i] * norm * win[i];
        }
        for (int i = 0; i < n_fft; i++) env[off + i] += win[i] * win[i];
    }
    for (int i = 0; i < length; i++) {
        const size_t j = (size_t)n_fft / 2 + pad + i;
        if ((int)(j - n_fft / 2) >= le_out || j >= full) {
            out[i] = 0.0f;
            continue;
        }
        out[i] = env[j] > 1e-11 ? (float)(y[j] / env[j]) : 0.0f;
    }
    free(win);
    free(y);
    free(env);
    free(buf);
    return 0;
}
