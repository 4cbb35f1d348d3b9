/* stx_oracle.h — CPU oracle for the stems.cpp spectral + elementwise hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference algorithms
 * (betweentwomidnights/stems.cpp v0.1.7), used as the parity checker and as the timed CPU
 * baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product library (stems.cpp_amd/libstx.so) never calls it and has no CPU fallback.
 *
 * Each function cites the reference file:line it follows. Complex arrays are interleaved
 * doubles (re, im), i.e. the memory layout of std::complex<double>. Every function returns 0
 * on success, -1 where the reference throws std::invalid_argument and -2 where it throws
 * std::runtime_error.
 *
 * How each part is pinned (beyond restating the formula):
 *   orc_fft, orc_torch_stft/istft, orc_htdemucs_spec/ispec: bit-exact against golden vectors
 *     written by the reference's own src/stft.h (tests/golden/), plus closed forms (impulse
 *     known answer, brute-force DFT, Parseval) and the reference's round-trip tolerances
 *     (tests/dsp_test.cpp:63,76-77,95).
 *   orc_vrfft: a brute-force DFT in double (closed form) at the reference's sizes 7680, 960, 640
 *     and 320, and the torch STFT -> iSTFT round trip at n_fft 7680 (Kim_Vocal_2).
 *   orc_mel_band_map: the counts the survey of the reference restated independently (60 bands,
 *     1,979 entries, sizes 7, 6, 6, ..., 122, 130, 71 bins in one band and 954 in two), an
 *     independent vectorised float32 restatement of librosa's filterbank in the test, and the
 *     margin between every bin frequency and every mel vertex (>= 0.098 Hz), which shows that
 *     ulp-level differences in log/exp cannot change the map. Exact librosa-version behaviour
 *     is parity unpinned (librosa is not installed).
 *   orc_bands_layout / orc_band_gather / orc_band_scatter_apply: brute force against
 *     independent numpy formulations on small tables, and invariants (gather then scatter of
 *     bin-constant masks returns the spectrum times that constant; band counts sum to the
 *     table size).
 *   orc_group_norm, orc_norm, orc_soft_max, orc_gelu_erf, orc_glu, orc_rope: torch's own
 *     float64 implementations (F.group_norm, F.layer_norm, F.rms_norm, softmax, F.gelu, F.glu)
 *     as an independent library, a complex-multiplication restatement of RoPE, and invariants
 *     (normalised groups have mean 0 and variance var/(var+eps); softmax rows sum to 1;
 *     gelu(x) - gelu(-x) = x; RoPE preserves pair norms and q.k depends only on the position
 *     difference). ggml-specific rounding (the float theta recurrence of ggml's RoPE, its float
 *     softmax and norm arithmetic) is parity unpinned: ggml's sources are not in the reference.
 *   orc_binary: numpy's float32 arithmetic on explicitly tiled operands, bit for bit.
 *   orc_msst_* / orc_uvr_* / orc_tfc_post: the closed forms of their windows (linspace ends at
 *     exactly 0 and 1; np.hanning against numpy's own), numpy restatements of both loops on
 *     small inputs, the identity model (both must return the mix), and the UVR geometry of the
 *     reference's defaults (trim n_fft / 2, step chunk - n_fft).
 *   orc_to_channels / orc_pin_length: numpy's transpose (interleaved to planar), fancy indexing
 *     by the channel map and slicing / zero padding, on every layout and channel count case.
 *   orc_resample: src == dst returns the input; a numpy restatement of the tabulated kernel,
 *     bit for bit; the direct Kaiser-sinc formula (no table) to the interpolation error; and
 *     the closed forms of a band-limited sine (passband gain 1) and of DC.
 *   orc_mean_std / orc_*normalize / orc_time_add / orc_split_*: torch.std's unbiased estimator
 *     and numpy float32 arithmetic on the same formulas, the weights' closed form (symmetric
 *     up to the centre sample, maximum 1), the identity model (a split of a model that returns
 *     its input gives the input back), and the TensorChunk rule that the last segment is
 *     centre-padded with the audio before it, not with zeros (src/htdemucs.cpp:530-533).
 *   orc_cont_permute / orc_concat / orc_merge_heads: numpy's transpose, concatenate and
 *     multiply, bit for bit, and the shapes the reference's own comments give for its permutes
 *     (src/roformer.cpp:112-114,133: [dh, N, H, batch] and [N, dh, H, batch] from
 *     [dh, H, N, batch]). orc_qkv_rope_split: its q and k against the complex-multiplication
 *     RoPE on numpy's slices of qkv, and its vt bit for bit against numpy's transpose.
 *   orc_demix_*: the chunk table the survey of the reference derived for 180 s at chunk 352,800
 *     and step 88,200 (96 chunks, four without fade-out, short chunks of 264,600 (reflect),
 *     176,400 and 88,200 (zero) samples), torch.linspace(0, 1, fade) in float32 for the fade
 *     (the reference computes "the way torch does"), and the identity separator, which must
 *     return the input (sum of w * x over sum of w).
 */
#ifndef STX_ORACLE_H
#define STX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* st::FFT (src/stft.h:19-55): in-place radix-2 DIT, unnormalised; inverse = conj twiddles. */
int orc_fft(double* a, int n, int inverse);

/* st::VRFFT (src/vr_dsp.h:11-37): Bluestein for any n, unnormalised. orc_torch_stft and
 * orc_torch_istft use it for sizes that are not powers of two, as the reference's TFC-TDF does. */
int orc_vrfft(double* a, int n, int inverse);

/* st::hann_periodic (src/stft.h:70-74). */
int orc_hann_periodic(double* w, int n);

/* st::reflect_pad (src/stft.h:58-68). y has n + left + right doubles. */
int orc_reflect_pad(const float* x, int n, int left, int right, double* y);

/* st::torch_stft (src/stft.h:146-164) for one channel: spec [F = n/2+1][T = len/hop+1]. */
int orc_torch_stft(const float* x, int len, int n_fft, int hop, int normalized, double* spec, int* n_frames);

/* st::torch_istft (src/stft.h:166-197): out has hop * (n_frames - 1) floats. */
int orc_torch_istft(const double* spec, int n_frames, int n_fft, int hop, int normalized, float* out);

/* st::htdemucs_spec (src/stft.h:76-103): spec [F = n/2][T = ceil(len / (n/4))]. */
int orc_htdemucs_spec(const float* x, int len, int n_fft, double* spec, int* n_frames);

/* st::htdemucs_ispec (src/stft.h:105-140): out has `length` floats. */
int orc_htdemucs_ispec(const double* spec, int n_frames, int n_fft, int length, float* out);

/* Mel band map of tools/convert_roformer.py:107-115. Returns -2 if a bin is uncovered. */
int orc_mel_band_map(int sr, int n_fft, int n_mels, int* band_sizes, int* band_freqs, long cap, long* n_total);

/* RoFormer constructor tables (src/roformer.cpp:394-411); -2 where the constructor throws. */
int orc_bands_layout(const int* band_sizes, int n_bands, const int* band_freqs, long n_freqs, int n_bins,
                     int channels, long* freq_off, long* feat_off, int* bpf);

/* Band gather, src/roformer.cpp:226-241: z complex [C][F][T] -> feat [total_feat * T]. */
void orc_band_gather(const int* band_sizes, int n_bands, const int* band_freqs, int C, int F, int T,
                     const double* z, float* feat);

/* Scatter-average + complex mask apply, src/roformer.cpp:251-278: masks [S][total_feat * T],
 * z complex [C][F][T] -> out complex [S][C][F][T] (before the iSTFT). */
void orc_band_scatter_apply(const int* band_sizes, int n_bands, const int* band_freqs, int C, int F, int T,
                            const float* masks, int S, const double* z, int zero_dc, double* out);

/* Chunk count of src/roformer.cpp:353-357. */
long orc_demix_n_chunks(long len, int chunk, int step);

/* Fade window of src/roformer.cpp:303-313 (window[chunk]). */
void orc_demix_window(int chunk, float* window);

/* Chunk inputs of src/roformer.cpp:289-331: mix [C][len] -> parts [n_chunks][C][chunk]. */
int orc_demix_chunks(const float* mix, int C, long len, int chunk, int step, float* parts);

/* Overlap-add of src/roformer.cpp:334-350: y [n_chunks][S][C][chunk] -> out [S][C][len]. */
int orc_demix_ola(const float* y, int S, int C, long len, int chunk, int step, float* out);

/* TFC-TDF chunking (tfc_oracle.c): MSST (src/tfc_tdf.cpp:447-495) and UVR (:407-441) chunk
 * inputs [n_chunks][C][chunk] and overlap-adds of y [n_chunks][S][C][chunk] -> out [S][C][len],
 * and separate()'s compensation + complement (:582-595). */
void orc_msst_window(int chunk, float* window);
long orc_msst_n_chunks(long len, int chunk, int step);
int orc_msst_chunks(const float* mix, int C, long len, int chunk, int step, float* parts);
int orc_msst_ola(const float* y, int S, int C, long len, int chunk, int step, float* out);
long orc_uvr_geometry(long len, int chunk, int n_fft, float overlap, long* M, long* step);
int orc_uvr_chunks(const float* mix, int C, long len, int chunk, int n_fft, float overlap, float* parts);
int orc_uvr_ola(const float* y, int S, int C, long len, int chunk, int n_fft, float overlap, float* out);
void orc_tfc_post(const float* mix, long plane, int S, float compensate, int complement, float* est);

/* st::resample_planar (src/audio.h:17-59) (resample_oracle.c). */
void orc_resample_table(int src_rate, int dst_rate, double* table, double* half);
long orc_resample_length(long n, int src_rate, int dst_rate);
int orc_resample(const float* in, int n, int ch, int src_rate, int dst_rate, float* out);
/* libstems separate()'s audio steps (src/libstems.cpp:160-196) (resample_oracle.c): layout 0
 * planar, 1 interleaved. */
void orc_to_channels(const float* in, long n, int ch, int layout, int want, float* out);
void orc_pin_length(const float* in, long planes, long back, long n, float* out);

/* ggml ops (ops_oracle.c). Contiguous tensors, ggml extents ne[4] (ne[0] fastest); broadcast
 * operands repeat into ne. */
int orc_group_norm(const float* x, const int64_t ne[4], int n_groups, float eps, const float* w, const int64_t wne[4],
                   const float* b, const int64_t bne[4], int gelu, float* y);
int orc_norm(const float* x, int64_t ne0, int64_t rows, float eps, int rms, const float* w, const float* b, float* y);
int orc_soft_max(const float* x, int64_t ne0, int64_t rows, float scale, float* y);
void orc_gelu_erf(const float* x, int64_t n, float* y);
int orc_glu(const float* x, const int64_t ne[4], int dim, float* y);
int orc_binary(int op, const float* a, const int64_t ne[4], const float* b, const int64_t bne[4], const float* c,
               const int64_t cne[4], float* y);
int orc_rope(const float* x, const int64_t ne[4], const int32_t* pos, int n_dims, int mode, float freq_base,
             float freq_scale, float attn_factor, float* y);

/* Layout glue (layout_oracle.c). x and y contiguous; nes holds 4 extents per source. */
int orc_cont_permute(const float* x, const int64_t ne[4], const int ax[4], float* y);
int orc_concat(const float* const* xs, const int64_t* nes, int n, int dim, float* y);
int orc_qkv_rope_split(const float* qkv, int64_t dh, int64_t H, int64_t N, int64_t batch, const int32_t* pos,
                       float freq_base, float freq_scale, float attn_factor, float* q, float* k, float* vt);
int orc_merge_heads(const float* o, const int64_t ne[4], const float* gates, float* y);

/* HTDemucs pre/post-processing and apply_model's split (htdemucs_oracle.c). */
void orc_mean_std(const float* x, int64_t n, double* mean, double* sd);
void orc_cac_normalize(const float* spec, int C, int64_t FT, double mean, double sd, float* mag);
void orc_normalize(const float* x, int64_t n, double mean, double sd, float* y);
void orc_cac_denormalize(const float* ox, int S, int C, int64_t FT, double mean, double sd, float* spec);
void orc_time_add(const float* t, const float* y, int64_t n, double mean, double sd, float* out);
void orc_mix_normalize(const float* mix, int C, int64_t len, float* out, double* stats);
void orc_split_weights(int seg, float* w);
int orc_split_count(int length, int seg, float overlap, int* stride);
void orc_segments(const float* buf, int C, int64_t total, int64_t offset, int length, int seg, int stride,
                  float* parts);
void orc_split_ola(const float* y, int tracks, int length, int seg, int stride, float* out, float* sum_w);

#ifdef __cplusplus
}
#endif

#endif /* STX_ORACLE_H */
