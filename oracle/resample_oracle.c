/* resample_oracle.c — TEST INFRASTRUCTURE: CPU restatement of st::resample_planar
 * (src/audio.h:17-59): a Kaiser-windowed sinc (beta 8.6, 32 zero crossings, cutoff 0.95 of the
 * lower Nyquist) tabulated over |x| in [0, half] at 2^15 + 2 points and interpolated linearly,
 * accumulated in double over the input samples within half of each output position. */
#include "stx_oracle.h"

#include <math.h>
#include <stdlib.h>

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

static double bessel_i0(double x) {
    double s = 1, t = 1;
    for (int k = 1; k < 30; k++) {
        t *= (x / (2 * k)) * (x / (2 * k));
        s += t;
    }
    return s;
}

/* The kernel table of src/audio.h:25-38: table[table_n + 2], and half and ratio. */
void orc_resample_table(int src_rate, int dst_rate, double* table, double* half_out) {
    const double ratio = (double)dst_rate / src_rate;
    const double cutoff = 0.95 * (ratio < 1.0 ? ratio : 1.0);
    const int zc = 32;
    const double half = zc / cutoff;
    const double beta = 8.6;
    const double i0b = bessel_i0(beta);
    const int table_n = 1 << 15;
    for (int t = 0; t <= table_n + 1; t++) {
        const double x = ((double)t / table_n < 1.0 ? (double)t / table_n : 1.0) * half;
        const double r = x / half;
        const double arg = M_PI * x * cutoff;
        const double sinc = arg < 1e-12 ? 1.0 : sin(arg) / arg;
        table[t] = r >= 1 ? 0.0 : sinc * bessel_i0(beta * sqrt(1 - r * r)) / i0b * cutoff;
    }
    *half_out = half;
}

/* out_n = llround(n * ratio); in [ch][n] -> out [ch][out_n]. */
long orc_resample_length(long n, int src_rate, int dst_rate) {
    if (src_rate == dst_rate) return n;
    return llround(n * ((double)dst_rate / src_rate));
}

int orc_resample(const float* in, int n, int ch, int src_rate, int dst_rate, float* out) {
    if (src_rate == dst_rate) {
        for (long i = 0; i < (long)n * ch; i++) out[i] = in[i];
        return 0;
    }
    const double ratio = (double)dst_rate / src_rate;
    const int out_n = (int)llround(n * ratio);
    const int table_n = 1 << 15;
    double half;
    double* table = (double*)malloc(sizeof(double) * (table_n + 2));
    double* acc = (double*)malloc(sizeof(double) * ch);
    orc_resample_table(src_rate, dst_rate, table, &half);
    for (int i = 0; i < out_n; i++) {
        const double c = i / ratio;
        int lo = (int)ceil(c - half), hi = (int)floor(c + half);
        if (lo < 0) lo = 0;
        if (hi > n - 1) hi = n - 1;
        for (int k = 0; k < ch; k++) acc[k] = 0.0;
        for (int j = lo; j <= hi; j++) {
            const double pos = fabs(j - c) / half * table_n;
            const int t = (int)pos;
            if (t >= table_n) continue;
            const double fr = pos - t;
            const double w = table[t] + (table[t + 1] - table[t]) * fr;
            for (int k = 0; k < ch; k++) acc[k] += w * in[(size_t)k * n + j];
        }
        for (int k = 0; k < ch; k++) out[(size_t)k * out_n + i] = (float)acc[k];
    }
    free(table);
    free(acc);
    return 0;
}

/* The request's audio in planar model channels (src/libstems.cpp:160-167, then st::to_channels,
 * src/audio.h:62-71): planar in[c * n + i] or interleaved in[i * ch + c] copied to a planar
 * buffer, then model channel c takes input channel 0 when the input is mono, else
 * min(c, ch - 1) (an unchanged copy when ch == want). */
void orc_to_channels(const float* in, long n, int ch, int layout, int want, float* out) {
    for (int c = 0; c < want; c++) {
        const int src = ch == want ? c : (ch == 1 ? 0 : (c < ch - 1 ? c : ch - 1));
        for (long i = 0; i < n; i++)
            out[(size_t)c * n + i] = layout == 0 ? in[(size_t)src * n + i] : in[(size_t)i * ch + src];
    }
}

/* Each of `planes` planes of `back` samples cut or zero-padded to n samples
 * (src/libstems.cpp:188-193). */
void orc_pin_length(const float* in, long planes, long back, long n, float* out) {
    for (long k = 0; k < planes; k++)
        for (long i = 0; i < n; i++) out[(size_t)k * n + i] = i < back ? in[(size_t)k * back + i] : 0.0f;
}
