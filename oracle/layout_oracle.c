/* layout_oracle.c — CPU oracle (test infrastructure) for the layout glue around RoFormer
 * attention: ggml_cont(ggml_permute(...)), ggml_concat, and the q/k/v split of
 * src/roformer.cpp:101-112 composed exactly as the reference's graph composes it (cont of a
 * view, rope_ext, cont of a permute). Tensors are contiguous with ggml extents ne[4] (ne[0]
 * fastest). */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "stx_oracle.h"

/* ggml_cont(ggml_permute(x, ax[0..3])): dimension i of x becomes dimension ax[i] of y
 * (src/roformer.cpp:112,133,182,184,190 use (0,2,1,3) and (1,2,0,3)). */
int orc_cont_permute(const float* x, const int64_t ne[4], const int ax[4], float* y) {
    int seen[4] = {0, 0, 0, 0};
    for (int i = 0; i < 4; i++) {
        if (ax[i] < 0 || ax[i] > 3 || seen[ax[i]]) return -1;
        seen[ax[i]] = 1;
    }
    int64_t yne[4], ynb[4];                    /* y extents, and y's element stride per x dim */
    for (int i = 0; i < 4; i++) yne[ax[i]] = ne[i];
    int64_t st[4];
    st[0] = 1;
    for (int j = 1; j < 4; j++) st[j] = st[j - 1] * yne[j - 1];
    for (int i = 0; i < 4; i++) ynb[i] = st[ax[i]];
    int64_t e = 0;
    for (int64_t i3 = 0; i3 < ne[3]; i3++)
        for (int64_t i2 = 0; i2 < ne[2]; i2++)
            for (int64_t i1 = 0; i1 < ne[1]; i1++)
                for (int64_t i0 = 0; i0 < ne[0]; i0++)
                    y[i0 * ynb[0] + i1 * ynb[1] + i2 * ynb[2] + i3 * ynb[3]] = x[e++];
    return 0;
}

/* ggml_concat of n tensors along dim, in order (concat_all of src/roformer.cpp:52-60 is a tree
 * of pairwise concats, which places every source in the same slice). */
int orc_concat(const float* const* xs, const int64_t* nes, int n, int dim, float* y) {
    if (n < 1 || dim < 0 || dim > 3) return -1;
    int64_t yne[4];
    for (int j = 0; j < 4; j++) yne[j] = nes[j];
    yne[dim] = 0;
    for (int s = 0; s < n; s++) {
        for (int j = 0; j < 4; j++)
            if (j != dim && nes[4 * s + j] != yne[j]) return -1;
        yne[dim] += nes[4 * s + dim];
    }
    int64_t off = 0;
    for (int s = 0; s < n; s++) {
        const int64_t* ne = nes + 4 * s;
        int64_t e = 0;
        for (int64_t i3 = 0; i3 < ne[3]; i3++)
            for (int64_t i2 = 0; i2 < ne[2]; i2++)
                for (int64_t i1 = 0; i1 < ne[1]; i1++)
                    for (int64_t i0 = 0; i0 < ne[0]; i0++) {
                        int64_t j[4] = {i0, i1, i2, i3};
                        j[dim] += off;
                        y[((j[3] * yne[2] + j[2]) * yne[1] + j[1]) * yne[0] + j[0]] = xs[s][e++];
                    }
        off += ne[dim];
    }
    return 0;
}

/* src/roformer.cpp:101-112. qkv [3*H*dh, N, batch]; part(i) = cont(view_4d(qkv, dh, H, N,
 * batch, offset i*H*dh)); q = cont(permute(rope_ext(part(0), pos, dh, mode 0), 0,2,1,3)),
 * k likewise, vt = cont(permute(part(2), 1,2,0,3)). */
int orc_qkv_rope_split(const float* qkv, int64_t dh, int64_t H, int64_t N, int64_t batch, const int32_t* pos,
                       float freq_base, float freq_scale, float attn_factor, float* q, float* k, float* vt) {
    const int64_t n = dh * H * N * batch, width = 3 * H * dh;
    float* part = malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    float* rot = malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    if (!part || !rot) {
        free(part);
        free(rot);
        return -2;
    }
    const int64_t ne[4] = {dh, H, N, batch};
    const int qk_axes[4] = {0, 2, 1, 3}, v_axes[4] = {1, 2, 0, 3};
    float* outs[2] = {q, k};
    int rc = 0;
    for (int i = 0; i < 3 && rc == 0; i++) {
        for (int64_t b = 0; b < batch; b++)
            for (int64_t t = 0; t < N; t++)
                memcpy(part + (b * N + t) * H * dh, qkv + (b * N + t) * width + i * H * dh, sizeof(float) * H * dh);
        if (i < 2) {
            rc = orc_rope(part, ne, pos, (int)dh, 0, freq_base, freq_scale, attn_factor, rot);
            if (rc == 0) rc = orc_cont_permute(rot, ne, qk_axes, outs[i]);
        } else {
            rc = orc_cont_permute(part, ne, v_axes, vt);
        }
    }
    free(part);
    free(rot);
    return rc;
}

/* src/roformer.cpp:133-137: y = cont(permute(o, 0,2,1,3)) [* reshape_4d(gates, 1, H, N, batch)],
 * o [dh, N, H, batch] -> y [dh, H, N, batch]; gates (may be NULL) is [H, N, batch]. */
int orc_merge_heads(const float* o, const int64_t ne[4], const float* gates, float* y) {
    const int axes[4] = {0, 2, 1, 3};
    int rc = orc_cont_permute(o, ne, axes, y);
    if (rc || !gates) return rc;
    const int64_t rows = ne[1] * ne[2] * ne[3];
    for (int64_t r = 0; r < rows; r++)
        for (int64_t i = 0; i < ne[0]; i++) y[r * ne[0] + i] *= gates[r];
    return 0;
}
