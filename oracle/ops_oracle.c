/* ops_oracle.c — CPU oracle (test infrastructure) for the ggml ops of the HTDemucs and
 * RoFormer graphs. ggml's sources are absent from the reference tree, so each op is the
 * textbook closed form, in double and rounded once, with the parameters the reference passes
 * at its call sites (cited per function). ADD, MUL and x + h*s are the float operations
 * themselves, rounded after every operation as separate ggml ops round (this file is built
 * with -ffp-contract=off).
 *
 * Tensors are contiguous with ggml's shape convention: ne[0] fastest, ne[3] slowest. A
 * broadcast operand with extents bne repeats into ne (index i -> i mod bne per dimension).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "stx_oracle.h"

/* Offset of element (i0, i1, i2, i3) of a contiguous tensor with extents bne, broadcast. */
static int64_t bidx(const int64_t bne[4], int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    return (((i3 % bne[3]) * bne[2] + (i2 % bne[2])) * bne[1] + (i1 % bne[1])) * bne[0] + (i0 % bne[0]);
}

static double gelu_d(double x) { return 0.5 * x * erfc(-x / sqrt(2.0)); }

/* ggml_group_norm(x, G, eps) (src/htdemucs.cpp:118,124,224) + mul/add (:127,:226) + GELU
 * (:136): channels ne2 in groups of cpg = ceil(ne2 / G); each (group, i3) normalised over
 * ne0 x ne1 x its channels with the biased variance (two passes in double). The fused GELU
 * is applied to the unrounded double value: gelu(GN(x) * w + b). */
int orc_group_norm(const float* x, const int64_t ne[4], int n_groups, float eps, const float* w, const int64_t wne[4],
                   const float* b, const int64_t bne[4], int gelu, float* y) {
    if (n_groups < 1) return -1;
    const int64_t cpg = (ne[2] + n_groups - 1) / n_groups;
    const int64_t plane = ne[0] * ne[1];
    for (int64_t i3 = 0; i3 < ne[3]; i3++) {
        for (int64_t c0 = 0; c0 < ne[2]; c0 += cpg) {
            const int64_t c1 = c0 + cpg < ne[2] ? c0 + cpg : ne[2];
            const int64_t off = (i3 * ne[2] + c0) * plane, n = (c1 - c0) * plane;
            double s = 0.0;
            for (int64_t i = 0; i < n; i++) s += x[off + i];
            const double mean = s / (double)n;
            double ss = 0.0;
            for (int64_t i = 0; i < n; i++) {
                const double d = x[off + i] - mean;
                ss += d * d;
            }
            const double rstd = 1.0 / sqrt(ss / (double)n + (double)eps);
            for (int64_t i = 0; i < n; i++) {
                const int64_t c = c0 + i / plane, i1 = (i % plane) / ne[0], i0 = i % ne[0];
                double t = (x[off + i] - mean) * rstd;
                if (w) t *= (double)w[bidx(wne, i0, i1, c, i3)];
                if (b) t += (double)b[bidx(bne, i0, i1, c, i3)];
                y[off + i] = gelu ? (float)gelu_d(t) : (float)t;
            }
        }
    }
    return 0;
}

/* ggml_norm (src/htdemucs.cpp:215; rms = 0) and ggml_rms_norm (src/roformer.cpp:34,96-98;
 * rms = 1) over rows of ne0, then * w[ne0] + b[ne0] when given (layer_norm :213-215, rms ·γ). */
int orc_norm(const float* x, int64_t ne0, int64_t rows, float eps, int rms, const float* w, const float* b, float* y) {
    if (ne0 < 1) return -1;
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * ne0;
        double mean = 0.0;
        if (!rms) {
            for (int64_t i = 0; i < ne0; i++) mean += xr[i];
            mean /= (double)ne0;
        }
        double ss = 0.0;
        for (int64_t i = 0; i < ne0; i++) ss += (xr[i] - mean) * (xr[i] - mean);
        const double scale = 1.0 / sqrt(ss / (double)ne0 + (double)eps);
        for (int64_t i = 0; i < ne0; i++) {
            double t = (xr[i] - mean) * scale;
            if (w) t *= (double)w[i];
            if (b) t += (double)b[i];
            y[r * ne0 + i] = (float)t;
        }
    }
    return 0;
}

/* ggml_soft_max_ext(x, NULL, scale, 0) (src/roformer.cpp:127, src/htdemucs.cpp:238):
 * softmax(scale * x) over rows of ne0. */
int orc_soft_max(const float* x, int64_t ne0, int64_t rows, float scale, float* y) {
    if (ne0 < 1) return -1;
    double* e = (double*)malloc(sizeof(double) * (size_t)ne0);
    if (!e) return -2;
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * ne0;
        double m = -INFINITY;
        for (int64_t i = 0; i < ne0; i++) {
            const double v = (double)scale * xr[i];
            if (v > m) m = v;
        }
        double s = 0.0;
        for (int64_t i = 0; i < ne0; i++) {
            e[i] = exp((double)scale * xr[i] - m);
            s += e[i];
        }
        for (int64_t i = 0; i < ne0; i++) y[r * ne0 + i] = (float)(e[i] / s);
    }
    free(e);
    return 0;
}

/* ggml_gelu_erf (src/roformer.cpp:147, src/htdemucs.cpp:136,154,210,246):
 * x/2 * (1 + erf(x/sqrt2)) = x/2 * erfc(-x/sqrt2). */
void orc_gelu_erf(const float* x, int64_t n, float* y) {
    for (int64_t i = 0; i < n; i++) y[i] = (float)gelu_d(x[i]);
}

/* GLU (src/htdemucs.cpp:105-110, src/roformer.cpp:199-202): first half along `dim` times the
 * sigmoid of the second half. x has extents ne; y has ne with ne[dim] halved. */
int orc_glu(const float* x, const int64_t ne[4], int dim, float* y) {
    if (dim < 0 || dim > 3 || ne[dim] % 2) return -1;
    int64_t yne[4] = {ne[0], ne[1], ne[2], ne[3]};
    yne[dim] /= 2;
    int64_t i[4];
    for (i[3] = 0; i[3] < yne[3]; i[3]++)
        for (i[2] = 0; i[2] < yne[2]; i[2]++)
            for (i[1] = 0; i[1] < yne[1]; i[1]++)
                for (i[0] = 0; i[0] < yne[0]; i[0]++) {
                    int64_t g[4] = {i[0], i[1], i[2], i[3]};
                    g[dim] += yne[dim];
                    const double a = x[bidx(ne, i[0], i[1], i[2], i[3])];
                    const double gate = x[bidx(ne, g[0], g[1], g[2], g[3])];
                    y[bidx(yne, i[0], i[1], i[2], i[3])] = (float)(a / (1.0 + exp(-gate)));
                }
    return 0;
}

/* Broadcast binary ops: op 0 ADD a + b, 1 MUL a * b, 2 MUL_ADD a + fl(b * c)
 * (src/htdemucs.cpp:139,250-251), 3 ADD_GELU gelu(fl(a + b)) (the FF bias + GELU,
 * src/roformer.cpp:147). b and c repeat into a's extents ne. */
int orc_binary(int op, const float* a, const int64_t ne[4], const float* b, const int64_t bne[4], const float* c,
               const int64_t cne[4], float* y) {
    if (op < 0 || op > 3) return -1;
    for (int k = 0; k < 4; k++)
        if (bne[k] < 1 || ne[k] % bne[k] || (op == 2 && (cne[k] < 1 || ne[k] % cne[k]))) return -1;
    int64_t n = 0;
    for (int64_t i3 = 0; i3 < ne[3]; i3++)
        for (int64_t i2 = 0; i2 < ne[2]; i2++)
            for (int64_t i1 = 0; i1 < ne[1]; i1++)
                for (int64_t i0 = 0; i0 < ne[0]; i0++, n++) {
                    const float x = a[n], v = b[bidx(bne, i0, i1, i2, i3)];
                    switch (op) {
                        case 0: y[n] = x + v; break;
                        case 1: y[n] = x * v; break;
                        case 2: {
                            const float p = v * c[bidx(cne, i0, i1, i2, i3)];
                            y[n] = x + p;
                            break;
                        }
                        default: {
                            const float s = x + v;
                            y[n] = (float)gelu_d(s);
                        }
                    }
                }
    return 0;
}

/* ggml_rope_ext without YaRN (src/roformer.cpp:109-113): rows of ne0 at position pos[i2]
 * rotated by theta_k = freq_scale * pos * freq_base^(-2k/n_dims), scaled by attn_factor;
 * mode 0 pairs (2k, 2k+1), mode 2 pairs (k, k + n_dims/2); elements past n_dims copied. */
int orc_rope(const float* x, const int64_t ne[4], const int32_t* pos, int n_dims, int mode, float freq_base,
             float freq_scale, float attn_factor, float* y) {
    if (n_dims < 2 || n_dims % 2 || n_dims > ne[0] || (mode != 0 && mode != 2)) return -1;
    const int half = n_dims / 2;
    for (int64_t i3 = 0; i3 < ne[3]; i3++)
        for (int64_t i2 = 0; i2 < ne[2]; i2++)
            for (int64_t i1 = 0; i1 < ne[1]; i1++) {
                const int64_t off = ((i3 * ne[2] + i2) * ne[1] + i1) * ne[0];
                const float* xr = x + off;
                float* yr = y + off;
                for (int k = 0; k < half; k++) {
                    const double th = (double)freq_scale * (double)pos[i2] * pow((double)freq_base, -2.0 * k / n_dims);
                    const double c = cos(th) * attn_factor, s = sin(th) * attn_factor;
                    const int j0 = mode == 0 ? 2 * k : k, j1 = mode == 0 ? 2 * k + 1 : k + half;
                    const double x0 = xr[j0], x1 = xr[j1];
                    yr[j0] = (float)(x0 * c - x1 * s);
                    yr[j1] = (float)(x0 * s + x1 * c);
                }
                for (int64_t i = n_dims; i < ne[0]; i++) yr[i] = xr[i];
            }
    return 0;
}
