/* stx.h — C ABI of the MI355X (gfx950) spectral + elementwise hot path of stems.cpp.
 *
 * Every entry point here replaces one host function or ggml op of the reference
 * (betweentwomidnights/stems.cpp v0.1.7); the comment above each declaration cites the
 * reference interface it replaces as file:line.
 *
 * Conventions (after the libstems V1 ABI, src/libstems_v1.h:53-63 and :18-20):
 *   - Every call returns an stx_status. On failure stx_last_error() holds a message for the
 *     calling thread. No C++ exception crosses this boundary.
 *   - STX_STATUS_INVALID_ARGUMENT is what the reference reports with std::invalid_argument,
 *     STX_STATUS_RUNTIME_ERROR what it reports with std::runtime_error.
 *   - Buffers marked "device" are caller-owned device memory (hipMalloc or any allocator);
 *     the hot calls never allocate. Work is enqueued on `stream` (a hipStream_t; NULL is the
 *     null stream) and runs asynchronously; results are valid once the stream is synchronised.
 *   - Complex arrays are interleaved float pairs (re, im), i.e. complex64.
 *   - Spectra use layout STX_SPEC_F_MAJOR, the reference's own (spec[(c * F + f) * T + t],
 *     src/stft.h:76-78), or STX_SPEC_T_MAJOR (spec[(c * T + t) * F + f]), which keeps every
 *     frame contiguous and is what the device pipeline prefers.
 *   - Handles (stx_fft, stx_bands) are immutable after creation and may be shared between
 *     threads and streams, as st::FFT is (src/stft.h:19-55).
 *   - Versioned table (libstems V1's model, src/libstems_v1.h:146-189): a consumer that loads
 *     the library at run time resolves only stx_get_api(STX_ABI_VERSION_1) and calls every
 *     entry point through the returned table. Structs that may grow (stx_separate_options,
 *     stx_demix_geometry) are size tagged and checked against frozen *_MIN_SIZE prefixes;
 *     stx_tensor (ggml's descriptor) and stx_chunk (an element of a caller-sized array) are
 *     frozen by-value types.
 */
#ifndef STX_H
#define STX_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#  define STX_API __attribute__((visibility("default")))
#else
#  define STX_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t stx_status;
enum {
    STX_STATUS_OK               = 0,
    STX_STATUS_INVALID_ARGUMENT = 1,   /* std::invalid_argument in the reference */
    STX_STATUS_UNSUPPORTED      = 2,   /* valid for the reference, not implemented here */
    STX_STATUS_CANCELLED        = 3,   /* st::Cancelled (src/separator.h:34-36) */
    STX_STATUS_RUNTIME_ERROR    = 4,   /* std::runtime_error in the reference */
    STX_STATUS_OUT_OF_MEMORY    = 6,
    STX_STATUS_DEVICE_ERROR     = 7    /* a HIP call failed */
};

typedef int32_t stx_spec_layout;
enum {
    STX_SPEC_F_MAJOR = 0,              /* spec[(c * F + f) * T + t]: stft.h's layout */
    STX_SPEC_T_MAJOR = 1               /* spec[(c * T + t) * F + f] */
};

typedef void* stx_stream;              /* a hipStream_t */

/* Library version string, e.g. "0.1.0". */
STX_API const char* stx_version(void);

/* Message of the last failed call on this thread ("" if none). */
STX_API const char* stx_last_error(void);

/* ------------------------------------------------------------------------------------------
 * FFT plan. Replaces st::FFT (src/stft.h:19-55).
 * ---------------------------------------------------------------------------------------- */
typedef struct stx_fft stx_fft;

/* st::FFT::FFT(int n) (src/stft.h:21-31): INVALID_ARGUMENT unless n is a power of two >= 2,
 * exactly like the reference; every such n up to 2^24 gives a plan (UNSUPPORTED above: the
 * plan's scratch). Sizes 16..8192 serve every call below; 2, 4, 8 (register transforms) and
 * sizes above 8192 (four steps: n1 x n2 transforms around transposes, scratch of n complex
 * values owned by the plan) serve stx_fft_run only, and the STFT/iSTFT calls return
 * UNSUPPORTED for them (the reference frames only at 2048 and 4096). Allocates the plan's
 * device tables on the current device. */
STX_API stx_status stx_fft_create(int n, stx_fft** out);
/* st::VRFFT::VRFFT(int n) (src/vr_dsp.h:11-37), the plan the reference uses for sizes that are
 * not powers of two (TFC-TDF's n_fft 7680, src/tfc_tdf.cpp:85-86,551-552; VR's 320/640/960): any
 * even n = 2^a 3^b 5^c in [16, 16384] (powers of two in [16, 8192] give the stx_fft_create plan),
 * UNSUPPORTED otherwise. The plan serves stx_fft_run (complex transforms up to 8192 points),
 * stx_torch_stft and the workspace iSTFT (stx_torch_istft_ws); the reference's Bluestein
 * transform is computed exactly (a DFT), so results agree to rounding. */
STX_API stx_status stx_fft_create_any(int n, stx_fft** out);
STX_API void       stx_fft_destroy(stx_fft* fft);
/* st::FFT::size() (src/stft.h:32). */
STX_API int        stx_fft_size(const stx_fft* fft);

/* st::FFT::run(a, inverse) (src/stft.h:34-49), batched: data is device [batch][n] complex,
 * transformed in place, unnormalised; inverse uses conjugate twiddles (no 1/n). Calls with a
 * plan above 8192 points must not overlap (they share the plan's scratch). */
STX_API stx_status stx_fft_run(const stx_fft* fft, float* data, int batch, int inverse,
                               stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * STFT / iSTFT. Replace src/stft.h:79-197, batched over channels. Input signals are
 * contiguous device [channels][len] float32.
 * ---------------------------------------------------------------------------------------- */

/* Frame count of torch_stft: len / hop + 1 (src/stft.h:153). */
STX_API int stx_torch_stft_frames(int len, int hop);
/* Frame count of htdemucs_spec: ceil(len / (n_fft / 4)) (src/stft.h:81,93). */
STX_API int stx_htdemucs_frames(int n_fft, int len);

/* torch_stft (src/stft.h:146-164): hann_window(n) periodic, center=True reflect pad,
 * onesided, F = n/2 + 1 bins, T = len/hop + 1 frames, optional 1/sqrt(n) normalisation.
 * spec: device [channels][F][T] (F_MAJOR) or [channels][T][F] (T_MAJOR) complex.
 * RUNTIME_ERROR if len <= n/2 (the reference's reflect_pad check, src/stft.h:59). */
STX_API stx_status stx_torch_stft(const stx_fft* fft, const float* x, int channels, int len,
                                  int hop, int normalized, float* spec, stx_spec_layout layout,
                                  stx_stream stream);

/* torch_istft (src/stft.h:166-197): DC and Nyquist imaginary parts ignored, window-squared
 * overlap-add normalisation, length = hop * (n_frames - 1). out: device [channels][length]. */
STX_API stx_status stx_torch_istft(const stx_fft* fft, const float* spec, int channels,
                                   int n_frames, int hop, int normalized, float* out,
                                   stx_spec_layout layout, stx_stream stream);

/* htdemucs_spec (src/stft.h:76-103): HTDemucs._spec; hop n/4, F = n/2 bins (Nyquist dropped),
 * T = ceil(len / hop) frames, 1/sqrt(n) normalised. spec: device [channels][F][T] or
 * [channels][T][F]. RUNTIME_ERROR where the reference's reflect pads would throw. */
STX_API stx_status stx_htdemucs_spec(const stx_fft* fft, const float* x, int channels, int len,
                                     float* spec, stx_spec_layout layout, stx_stream stream);

/* htdemucs_ispec (src/stft.h:105-140): HTDemucs._ispec; spec has F = n/2 bins and n_frames
 * frames; out: device [channels][length]. */
STX_API stx_status stx_htdemucs_ispec(const stx_fft* fft, const float* spec, int channels,
                                      int n_frames, int length, float* out,
                                      stx_spec_layout layout, stx_stream stream);

/* Bytes of device workspace for the *_ws iSTFT variants: channels * n_frames * n floats. */
STX_API size_t stx_istft_workspace_size(const stx_fft* fft, int channels, int n_frames);

/* stx_torch_istft / stx_htdemucs_ispec with a caller-owned device workspace of at least
 * stx_istft_workspace_size() bytes (INVALID_ARGUMENT if smaller). Sizes that are not powers of
 * two (stx_fft_create_any) need it: they inverse-transform each frame once into the workspace
 * and overlap-add in a second kernel. Power-of-two sizes run the same single kernel as the plain
 * entry points (the workspace is checked, not used): at every size measured that kernel, which
 * transforms frames shared by two output tiles twice, was faster than writing and re-reading
 * every windowed frame. A NULL workspace selects the plain path. */
STX_API stx_status stx_torch_istft_ws(const stx_fft* fft, const float* spec, int channels,
                                      int n_frames, int hop, int normalized, float* out,
                                      stx_spec_layout layout, void* workspace,
                                      size_t workspace_bytes, stx_stream stream);
STX_API stx_status stx_htdemucs_ispec_ws(const stx_fft* fft, const float* spec, int channels,
                                         int n_frames, int length, float* out,
                                         stx_spec_layout layout, void* workspace,
                                         size_t workspace_bytes, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * RoFormer band maps, band tables, band gather and mask scatter-average + apply.
 * Replace the host loops of RoFormer::Impl (src/roformer.cpp:217-283) and the band-map rules
 * of tools/convert_roformer.py:107-124. Layout of band features, per batch item (one chunk):
 * feat[band_feat_off[b] * T + t * dim_in(b) + (j * C + c) * 2 + {re, im}], dim_in(b) =
 * band_sizes[b] * C * 2 (src/roformer.cpp:85,226-241); masks of S stems use the same layout,
 * stem-major ([S][total_feat * T]).
 * ---------------------------------------------------------------------------------------- */
typedef struct stx_bands stx_bands;

/* MelBandRoformer's band map, tools/convert_roformer.py:107-115: librosa.filters.mel(sr, n_fft,
 * n_mels) (Slaney, fmin 0, fmax sr/2) with fb[0][0] = fb[-1][-1] = 1; band b holds the bins with
 * a positive weight, ascending. Writes band_sizes[n_mels] and band_freqs[*n_freqs]; with both
 * outputs NULL only *n_freqs is set (size query). RUNTIME_ERROR if a bin is left uncovered
 * (the converter's assertion, :114). Host only. */
STX_API stx_status stx_mel_band_map(int sample_rate, int n_fft, int n_mels, int32_t* band_sizes,
                                    int32_t* band_freqs, int64_t capacity, int64_t* n_freqs);

/* BSRoformer's contiguous bands, tools/convert_roformer.py:118-124: RUNTIME_ERROR unless the
 * sizes sum to n_fft/2 + 1. Host only. */
STX_API stx_status stx_bs_band_map(const int32_t* freqs_per_bands, int n_bands, int n_fft,
                                   int32_t* band_freqs, int64_t capacity, int64_t* n_freqs);

/* The RoFormer constructor's band tables and checks (src/roformer.cpp:394-411): RUNTIME_ERROR
 * if the sizes do not sum to n_freqs or a bin is out of [0, n_bins). Writes
 * band_freq_off[n_bands + 1], band_feat_off[n_bands + 1] (floats per frame) and
 * bands_per_freq[n_bins]; any output may be NULL. Host only. */
STX_API stx_status stx_bands_layout(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs,
                                    int64_t n_freqs, int n_bins, int channels, int64_t* band_freq_off,
                                    int64_t* band_feat_off, int32_t* bands_per_freq);

/* Device band table for `channels` channels and n_bins STFT bins, same checks as
 * stx_bands_layout. */
STX_API stx_status stx_bands_create(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs,
                                    int64_t n_freqs, int n_bins, int channels, stx_bands** out);
STX_API void       stx_bands_destroy(stx_bands* bands);
/* band_feat_off.back() = sum of dim_in(b): feature floats per frame (src/roformer.cpp:86). */
STX_API int64_t    stx_bands_total_feat(const stx_bands* bands);

/* Band gather (src/roformer.cpp:226-241) for `batch` chunks: spec is device
 * [batch][C][F][T] (F_MAJOR) or [batch][C][T][F] complex64; feat is device
 * [batch][total_feat * T] float, each value the spectrum's float re/im. */
STX_API stx_status stx_band_gather(const stx_bands* bands, const float* spec, int batch, int n_frames,
                                   stx_spec_layout layout, float* feat, stx_stream stream);

/* Mask scatter-average and complex mask apply (src/roformer.cpp:251-278) for `batch` chunks and
 * n_stems stems: out[b][s][c] = spec[b][c] * (sum of the stem's band masks covering each bin /
 * max(bands_per_freq, 1)), accumulated and applied in double and rounded once; bin 0 is zeroed
 * when zero_dc (:278). masks: device [batch][n_stems][total_feat * T]; spec: device
 * [batch][C][...] and out: device [batch][n_stems][C][...] complex64 in `layout`. */
STX_API stx_status stx_band_scatter_apply(const stx_bands* bands, const float* masks, int n_stems,
                                          const float* spec, int batch, int n_frames,
                                          stx_spec_layout layout, int zero_dc, float* out,
                                          stx_stream stream);

/* The band split's RMSNorm (src/roformer.cpp:169-175, rms at :96-98) for every band in one
 * launch: row t of band b, feat[batch][feat_off[b] * T + t * dim_in(b) + i] for
 * i < dim_in(b), becomes x / sqrt(mean(x^2) + eps) * gammas[b][i] (ggml_mul(ggml_rms_norm(view,
 * eps), gamma_b); the reference's eps is 1e-24, src/roformer.cpp:34). feat and out are device
 * [batch][total_feat * T] in the layout stx_band_gather writes; out may be feat. gammas is a host
 * array of n_bands device pointers, gammas[b] holding dim_in(b) floats. Bands of more than 1,024
 * floats per frame are UNSUPPORTED. */
STX_API stx_status stx_band_rms_norm(const stx_bands* bands, const float* feat, int batch, int n_frames,
                                     const float* const* gammas, float eps, float* out, stx_stream stream);

/* The GLU at the end of every mask estimator (src/roformer.cpp:193-204): heads[s * n_bands + b]
 * is device [T][2 * dim_in(b)], the last layer's output for stem s and band b; masks gets
 * a * sigmoid(gate) of its two halves, device [n_stems][total_feat * T] in the layout
 * stx_band_scatter_apply reads (pass batch * n_stems as n_stems for several chunks, heads in
 * the same order). heads is a host array of n_stems * n_bands device pointers. Each band's
 * result equals stx_glu(dim 0) on that band. */
STX_API stx_status stx_band_mask_glu(const stx_bands* bands, const float* const* heads, int n_stems, int n_frames,
                                     float* masks, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * Chunked overlap-add demix. Replaces RoFormer::Impl::demix (src/roformer.cpp:286-351),
 * n_chunks (:353-357) and RoFormer::separate (:436-486): chunks of `chunk` samples every `step`
 * over the input reflect-padded by border = chunk - step on both sides (when
 * len > 2 * border > 0), linear fades of chunk / 10 samples at both ends of every chunk's
 * weight (none at the start of the first chunk, none at the end of a chunk reaching the end),
 * sum of weight * output over chunks in double, divided by the summed weights; non-finite
 * results become 0 (np.nan_to_num).
 * ---------------------------------------------------------------------------------------- */
enum {
    STX_CHUNK_FULL    = 0,     /* length == chunk */
    STX_CHUNK_REFLECT = 1,     /* short chunk reflect-padded to `chunk` (length > chunk/2 + 1) */
    STX_CHUNK_ZERO    = 2      /* short chunk zero-padded (src/roformer.cpp:323-330) */
};

typedef struct {
    int64_t start;             /* first sample in the padded signal (k * step) */
    int32_t length;            /* samples taken from the padded signal, <= chunk */
    int32_t pad_mode;          /* STX_CHUNK_* */
    int32_t fade_in;           /* 1: the weight keeps its fade-in (0 for the first chunk) */
    int32_t fade_out;          /* 1: the weight keeps its fade-out (0 for chunks reaching the end) */
} stx_chunk;

/* Size tagged: set size = sizeof(stx_demix_geometry) before the call; the library writes the
 * fields that fit in `size` (at least STX_DEMIX_GEOMETRY_MIN_SIZE). */
typedef struct {
    uint32_t size;
    int32_t chunk, step, border, fade, reflect_border;
    int64_t len;               /* samples per channel */
    int64_t padded_len;        /* Lp */
    int64_t n_chunks;
} stx_demix_geometry;

/* Step of RoFormer::separate (src/roformer.cpp:442-443): chunk / num_overlap for overlap < 0,
 * else max(1, lround(chunk * (1 - overlap))); 0 for overlap >= 1 (the reference rejects it). */
STX_API int stx_demix_step(int chunk, int num_overlap, float overlap);

/* The integer chunk table (host only): geometry (unless NULL), and chunks[n_chunks] unless
 * chunks is NULL. INVALID_ARGUMENT for len <= 0 ("empty input"), chunk/step <= 0 or a geometry
 * whose size is below STX_DEMIX_GEOMETRY_MIN_SIZE. */
STX_API stx_status stx_demix_plan(int64_t len, int chunk, int step, stx_demix_geometry* geom,
                                  stx_chunk* chunks, int64_t capacity);

/* The chunking rules of a plan. STX_DEMIX_MSST is TFCTDF::Impl::demix_msst
 * (src/tfc_tdf.cpp:447-495), ZFTurbo's loop as the MDX/TFC-TDF models run it: short chunks are
 * reflect-padded when longer than chunk / 2 (not chunk / 2 + 1), only the chunk after which the
 * loop ends (start + step >= Lp) keeps full weight at its end, and the fades are
 * linspace(0, 1, fade) and linspace(1, 0, fade) (:56-63,465-469). */
typedef int32_t stx_demix_rules;
enum {
    STX_DEMIX_ROFORMER = 0,
    STX_DEMIX_MSST     = 1
};
/* stx_demix_plan / stx_demix_window / stx_demix_create with explicit rules. */
STX_API stx_status stx_demix_plan_rules(int64_t len, int chunk, int step, stx_demix_rules rules,
                                        stx_demix_geometry* geom, stx_chunk* chunks, int64_t capacity);

/* The fade window of src/roformer.cpp:303-313 (host only): window[chunk] floats, before the
 * first/last chunk edits. */
STX_API stx_status stx_demix_window(int chunk, float* window);
STX_API stx_status stx_demix_window_rules(int chunk, stx_demix_rules rules, float* window);

typedef struct stx_demix stx_demix;

/* Device plan for one input length: geometry and window on the device. */
STX_API stx_status stx_demix_create(int64_t len, int channels, int chunk, int step, stx_demix** out);
STX_API stx_status stx_demix_create_rules(int64_t len, int channels, int chunk, int step, stx_demix_rules rules,
                                          stx_demix** out);
STX_API void       stx_demix_destroy(stx_demix* demix);
STX_API int64_t    stx_demix_n_chunks(const stx_demix* demix);

/* Chunk inputs first .. first+count-1 (src/roformer.cpp:289-331): mix is device [C][len],
 * parts is device [count][C][chunk]; the border and short-chunk padding are done on the fly. */
STX_API stx_status stx_demix_chunks(const stx_demix* demix, const float* mix, int64_t first, int64_t count,
                                    float* parts, stx_stream stream);

/* Overlap-add of every chunk's separated output (src/roformer.cpp:334-350): y is device
 * [n_chunks][n_stems][C][chunk], out is device [n_stems][C][len]. Bit-identical to the
 * reference for identical chunk outputs. */
STX_API stx_status stx_demix_overlap_add(const stx_demix* demix, const float* y, int n_stems, float* out,
                                         stx_stream stream);

/* Separator callback of stx_demix_track: separates chunks first .. first+count-1. parts is
 * device [count][C][chunk] (read only), y is device [count][n_stems][C][chunk] (to fill).
 * Work may be enqueued on `stream`; return 0 on success. */
typedef int32_t (*stx_separate_fn)(void* user, const float* parts, int64_t first, int64_t count, float* y,
                                   stx_stream stream);
typedef void (*stx_progress_fn)(void* user, int32_t done, int32_t total);
typedef int32_t (*stx_cancel_fn)(void* user);

/* st::SeparateOptions (src/separator.h:19-32). Size tagged: zero it, set size = sizeof,
 * call stx_separate_options_init for the defaults, then set fields. A NULL options pointer
 * means the defaults; a size below STX_SEPARATE_OPTIONS_MIN_SIZE is INVALID_ARGUMENT. */
typedef struct {
    uint32_t size;
    int32_t shifts;                /* random time shifts averaged; 0 = one deterministic pass */
    float overlap;                 /* [0, 1); negative = the model's num_overlap */
    uint32_t seed;                 /* for the shift offsets (std::mt19937) */
    stx_progress_fn progress;      /* (done, total) chunk passes; may be NULL */
    stx_cancel_fn should_cancel;   /* polled before every chunk; non-zero cancels; may be NULL */
    void* user;
} stx_separate_options;

/* Writes the defaults (no shifts, overlap -1: the model's own, seed 0, no callbacks) into the
 * fields that fit in options->size. INVALID_ARGUMENT for NULL or a size below
 * STX_SEPARATE_OPTIONS_MIN_SIZE. Host only. */
STX_API stx_status stx_separate_options_init(stx_separate_options* options);

/* Bytes of device workspace stx_demix_track needs (batch = chunks per separator call). */
STX_API size_t stx_demix_track_workspace_size(int channels, int64_t len, int chunk, int step, int n_stems,
                                              int batch, int shifts, int sample_rate);

/* RoFormer::separate (src/roformer.cpp:436-486) around any separator: step from
 * num_overlap/overlap (:442-443), demix (:286-351) through `separate` in batches of `batch`
 * chunks, demucs' shift averaging (:456-478, offsets from std::mt19937(seed)), and, when
 * `complement`, one more output plane mix - stem 0 (:481-485). mix is device [C][len]; out is
 * device [n_stems + complement][C][len]. CANCELLED when should_cancel returns non-zero;
 * INVALID_ARGUMENT for len <= 0 ("empty input") or overlap >= 1. Progress and cancel callbacks
 * run on the calling thread, before each chunk. */
STX_API stx_status stx_demix_track(const float* mix, int channels, int64_t len, int chunk, int num_overlap,
                                   int n_stems, int complement, int sample_rate, int batch,
                                   stx_separate_fn separate, void* separate_user,
                                   const stx_separate_options* options, float* out, void* workspace,
                                   size_t workspace_bytes, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * TFC-TDF (MDX) chunking. Replaces TFCTDF::Impl::demix_uvr (src/tfc_tdf.cpp:407-441) and
 * TFCTDF::separate (:569-595); the MSST loop (:447-495) is an stx_demix plan with
 * STX_DEMIX_MSST rules.
 * ---------------------------------------------------------------------------------------- */
typedef struct stx_uvr_demix stx_uvr_demix;

/* UVR's SeperateMDX.demix geometry (src/tfc_tdf.cpp:410-415): trim = n_fft / 2 zeros in front,
 * gen = chunk - 2 trim, M = trim + len + gen + trim - len % gen samples, step = chunk - n_fft for
 * overlap < 0, else (int64)((1 - overlap) * chunk); chunks start at 0, step, ... < M. Weights
 * are np.hanning of each chunk's actual length min(chunk, M - start), or 1 when overlap == 0,
 * held by the plan on the device. RUNTIME_ERROR "tfc_tdf: chunk shorter than the FFT" for
 * gen <= 0, INVALID_ARGUMENT "overlap too large for this model" for step <= 0. */
STX_API stx_status stx_uvr_demix_create(int64_t len, int channels, int chunk, int n_fft, float overlap,
                                        stx_uvr_demix** out);
STX_API void       stx_uvr_demix_destroy(stx_uvr_demix* demix);
STX_API int64_t    stx_uvr_demix_n_chunks(const stx_uvr_demix* demix);
/* M, step and trim of a plan (each pointer may be NULL). */
STX_API stx_status stx_uvr_demix_geometry(const stx_uvr_demix* demix, int64_t* padded_len, int64_t* step, int* trim);
/* Model inputs of chunks first .. first + count - 1 (:416-425): mix device [C][len] ->
 * parts device [count][C][chunk], zero past each chunk's actual length. */
STX_API stx_status stx_uvr_demix_chunks(const stx_uvr_demix* demix, const float* mix, int64_t first, int64_t count,
                                        float* parts, stx_stream stream);
/* The weighted overlap-add (:427-440): y device [n_chunks][n_stems][C][chunk] -> out device
 * [n_stems][C][len], double products and sums in chunk order, one division, bit-identical to the
 * reference for the same model outputs. Indices are 32-bit when every one fits, else 64-bit;
 * STX_UVR_WIDE_INDEX=1 (read at each call) forces the 64-bit kernel, which gives the same bits. */
STX_API stx_status stx_uvr_demix_overlap_add(const stx_uvr_demix* demix, const float* y, int n_stems, float* out,
                                             stx_stream stream);

typedef int32_t stx_tfc_chunking;
enum {
    STX_TFC_MSST = 0,          /* the model's chunking "msst" (ZFTurbo's demix) */
    STX_TFC_UVR  = 1           /* "uvr_mdx" (UVR's SeperateMDX.demix) */
};

/* Bytes of device workspace stx_tfc_tdf_separate needs (0 for a geometry it rejects). */
STX_API size_t stx_tfc_tdf_separate_workspace_size(int channels, int64_t len, int chunk, int n_fft,
                                                   stx_tfc_chunking chunking, int num_overlap, float overlap,
                                                   int n_stems, int batch);

/* TFCTDF::separate (src/tfc_tdf.cpp:569-595) around any separator (parts [count][C][chunk] ->
 * y [count][n_stems][C][chunk], the model's run_chunk): RUNTIME_ERROR for empty or non-finite
 * input or shifts != 0, INVALID_ARGUMENT for overlap >= 1, CANCELLED when should_cancel returns
 * non-zero (polled before the loop and before each chunk); MSST or UVR chunking (MSST step:
 * stx_demix_step(chunk, num_overlap, overlap)); the stems times `compensate` when it is not 1;
 * with `complement`, one more plane mix - stem 0 - stem 1 - ... in float. out is device
 * [n_stems + complement][C][len]. Returns after the stream has drained. */
STX_API stx_status stx_tfc_tdf_separate(const float* mix, int channels, int64_t len, int chunk, int n_fft,
                                        stx_tfc_chunking chunking, int num_overlap, int n_stems, float compensate,
                                        int complement, int batch, stx_separate_fn separate, void* separate_user,
                                        const stx_separate_options* options, float* out, void* workspace,
                                        size_t workspace_bytes, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * Resampling. Replaces st::resample_planar (src/audio.h:17-59), used when the input is not at
 * the model's rate.
 * ---------------------------------------------------------------------------------------- */
typedef struct stx_resampler stx_resampler;

/* The reference's Kaiser-windowed sinc (beta 8.6, 32 zero crossings, cutoff 0.95 of the lower
 * Nyquist), tabulated at 2^15 + 2 points on the device, for src_rate -> dst_rate. */
STX_API stx_status stx_resampler_create(int src_rate, int dst_rate, stx_resampler** out);
STX_API void       stx_resampler_destroy(stx_resampler* resampler);
/* Output samples per channel for n input samples: llround(n * dst / src), n when the rates are
 * equal (src/audio.h:19-20); -1 for a NULL plan or n < 0. */
STX_API int64_t    stx_resample_length(const stx_resampler* resampler, int64_t n);
/* in: device [channels][n]; out: device [channels][stx_resample_length(n)]. By default each output
 * uses the weights of its exact phase (dst / gcd rows computed once by the reference's formula),
 * which differ from the reference's per-output weights by the rounding of its position i / ratio:
 * measured within 2.0e-7 of the output's rms, 167 dB SNR, on 180 s of stereo at 48 kHz.
 * STX_RESAMPLE_EXACT=1 in the environment (read at each call) selects the per-tap kernel,
 * bit-identical to the reference (double sums in its order). That kernel is also used when the
 * phase path does not fit: more than 2^18 phase-table weights, or a staged input tile (64 rows of
 * down + taps + 8 samples) above the device's LDS per workgroup. Equal rates copy. More than 8
 * channels is UNSUPPORTED. */
STX_API stx_status stx_resample(const stx_resampler* resampler, const float* in, int channels, int64_t n, float* out,
                                stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * HTDemucs pre/post-processing around the model graph, and apply_model's split. Replace the
 * host loops of HTDemucs::Impl::run (src/htdemucs.cpp:419-474) and HTDemucs::separate
 * (:534-644). Statistics are device double[2] {mean, sd}, written by the normalise calls and
 * read by the denormalise calls, so nothing returns to the host between them.
 * ---------------------------------------------------------------------------------------- */

/* Bytes of device workspace for a normalise call over n values (a fixed area for the
 * single-pass kernel, 16 bytes per 8192 values and 16 more). */
STX_API size_t stx_htdemucs_norm_workspace_size(int64_t n);

/* Complex-as-channels pack and normalisation of one segment's spectrum
 * (src/htdemucs.cpp:424-436): spec is device complex64 [C][F][T] (f-major, as
 * stx_htdemucs_spec writes it); mag is device [2C][F][T] with mag[2c] = re and mag[2c+1] = im,
 * each (v - mean) / (1e-5 + sd) over all 2 C F T values (mean_of and the unbiased std_of,
 * :293-302, in double). stats gets {mean, sd}. workspace: device, 16-byte aligned,
 * stx_htdemucs_norm_workspace_size(2 C F T) bytes, no initialisation needed; calls that share one
 * must not overlap. mag must not overlap spec (INVALID_ARGUMENT). A segment that fits on the
 * device at once is normalised by one grid-synchronised kernel, with the bounded waits and
 * the same-bits fallback of stx_group_norm; the rest take two kernels (moments, then the
 * normalisation, each of whose blocks adds the moments' partial sums itself). */
STX_API stx_status stx_htdemucs_cac_normalize(const float* spec, int channels, int n_bins, int n_frames, float* mag,
                                              double* stats, void* workspace, size_t workspace_bytes,
                                              stx_stream stream);

/* The waveform branch's normalisation (src/htdemucs.cpp:438-441): out = (x - mean) / (1e-5 + sd)
 * over n values. stats gets {mean, sd}. out may be x (in place, two kernels); any other
 * overlap of out and x is INVALID_ARGUMENT. */
STX_API stx_status stx_htdemucs_wave_normalize(const float* x, int64_t n, float* out, double* stats, void* workspace,
                                               size_t workspace_bytes, stx_stream stream);

/* separate()'s normalisation by the mono mix (src/htdemucs.cpp:539-549): mono = sum_c x / C
 * (rounded to float), ref_mean and ref_std = max(std, 1e-8) of mono, out = (x - ref_mean) /
 * ref_std for every channel of mix [C][len]. stats gets {ref_mean, ref_std}. INVALID_ARGUMENT
 * "empty input" when len <= 0, as the reference throws. workspace: norm_workspace_size(len).
 * out may be mix (in place); any other overlap is INVALID_ARGUMENT. With 1 or 2 channels and
 * out not overlapping mix, a mix whose 8192-sample chunks the device holds at once (1,024
 * chunks of two channels on MI355X, 3.2 minutes at 44.1 kHz) is normalised by one
 * grid-synchronised kernel with the same bits as the two kernels that every other call takes. */
STX_API stx_status stx_htdemucs_mix_normalize(const float* mix, int channels, int64_t len, float* out, double* stats,
                                              void* workspace, size_t workspace_bytes, stx_stream stream);

/* The spectral branch's denormalisation (src/htdemucs.cpp:465-468): ox is the model's
 * [S][2C][F][T] output; spec gets complex64 [S][C][F][T] with re * sd + mean and
 * im * sd + mean (double, rounded once), stats being the cac_normalize ones. Feed spec to
 * stx_htdemucs_ispec with S * C channels. */
STX_API stx_status stx_htdemucs_cac_denormalize(const float* ox, int n_sources, int channels, int n_bins, int n_frames,
                                                const double* stats, float* spec, stx_stream stream);

/* The time branch's denormalisation plus the spectral branch (src/htdemucs.cpp:469-470):
 * out = (float)(xt * sd + mean) + y over n values, with the wave_normalize stats. */
STX_API stx_status stx_htdemucs_time_add(const float* xt, const float* y, int64_t n, const double* stats, float* out,
                                         stx_stream stream);

/* split()'s chunking (src/htdemucs.cpp:564-566,589): stride = (int)((1 - overlap) * segment)
 * (overlap < 0 means 0.25) and the number of chunks of a view of `length` samples.
 * INVALID_ARGUMENT "overlap must be < 1" when stride <= 0. */
STX_API stx_status stx_htdemucs_split_plan(int length, int segment, float overlap, int* stride, int* n_chunks);

/* The padded model inputs of chunks first .. first + count - 1 of the view [offset, offset +
 * length) of buf (device [C][total]) (TensorChunk.padded, src/htdemucs.cpp:552-561,589-593):
 * chunk k starts at k * stride, keeps min(segment, length - k * stride) samples and is
 * centre-padded to `segment` with buf's own samples around it where they exist, zeros beyond.
 * parts: device [count][C][segment]. */
STX_API stx_status stx_htdemucs_segments(const float* buf, int channels, int64_t total, int64_t offset, int length,
                                         int segment, int stride, int first, int count, float* parts,
                                         stx_stream stream);

/* split()'s weighted overlap-add (src/htdemucs.cpp:566-573,594-606): y is device
 * [n_chunks][tracks][segment], the model outputs of every chunk (tracks = S * C); each is
 * center-trimmed, weighted by the triangular window and summed in chunk order in float, then
 * divided by the summed weights: out device [tracks][length], bit-identical to the reference. */
STX_API stx_status stx_htdemucs_split_overlap_add(const float* y, int tracks, int length, int segment, int stride,
                                                  float* out, stx_stream stream);

/* Model callback of stx_htdemucs_separate: runs model `model` of the bag on `count` segments.
 * parts is device [count][C][segment] (normalised by the mono mix, read only); y is device
 * [count][n_sources][C][segment] (to fill): HTDemucs::forward / Impl::run per segment
 * (src/htdemucs.cpp:419-474, whose pre/post-processing the calls above provide). Work may be
 * enqueued on `stream`; return 0 on success. */
typedef int32_t (*stx_model_fn)(void* user, int32_t model, const float* parts, int64_t count, float* y,
                                stx_stream stream);

/* Bytes of device workspace stx_htdemucs_separate needs (batch = segments per model call). */
STX_API size_t stx_htdemucs_separate_workspace_size(int channels, int64_t len, int segment, int n_sources, int batch,
                                                   int shifts, int sample_rate, float overlap);

/* HTDemucs::separate (src/htdemucs.cpp:534-644) around any model: normalise by the mono mix,
 * for each model of the bag split() the mix (or, with shifts > 0, `shifts` views at offsets
 * drawn from one std::mt19937(seed) with uniform_int_distribution(0, sample_rate / 2) per
 * model, into the mix zero-padded by sample_rate / 2) through `forward` in batches of `batch`
 * segments, average the shifts, weight the models by bag_weights (host [n_models][n_sources];
 * a zero weight skips the source), divide by the weight totals and denormalise. mix is device
 * [C][len]; out is device [n_sources][C][len]. Float arithmetic and orders as the reference's.
 * options->overlap < 0 means 0.25. CANCELLED when should_cancel returns non-zero (polled before
 * each segment); progress reports (done, n_models * max(1, shifts) * ceil(len / stride)) after
 * each segment, as the reference does. INVALID_ARGUMENT for len <= 0 ("empty input") or
 * overlap >= 1. n_sources is at most 64. */
STX_API stx_status stx_htdemucs_separate(const float* mix, int channels, int64_t len, int segment, int n_sources,
                                         int n_models, const float* bag_weights, int sample_rate, int batch,
                                         stx_model_fn forward, void* forward_user,
                                         const stx_separate_options* options, float* out, void* workspace,
                                         size_t workspace_bytes, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * ggml ops of the HTDemucs and RoFormer graphs. ggml's sources are not in the reference tree
 * (an un-vendored submodule), so each entry point cites the call sites whose semantics it
 * implements. Tensors are fp32 with ggml's shape convention: ne[0] is the fastest dimension,
 * nb[] are byte strides, and rows must be contiguous (nb[0] == 4). Unused trailing dimensions
 * have ne = 1. A broadcast operand "repeats into" dst when every dst->ne[i] is a multiple of
 * its ne[i] (ggml_can_repeat). Normalisations and softmax compute their statistics in double
 * and round once; ADD, MUL and MUL_ADD round after every operation like the separate ggml ops.
 * ---------------------------------------------------------------------------------------- */
typedef struct {
    void* data;                    /* device */
    int64_t ne[4];                 /* elements per dimension, ne[0] fastest */
    int64_t nb[4];                 /* byte strides; nb[0] must be 4 */
} stx_tensor;

/* ggml_group_norm(a, n_groups, eps) (src/htdemucs.cpp:118,124,224), fused with the affine
 * mul/add that follows it (:127,:226) and optionally with the GELU after that (:136). Channels
 * (ne2) are split into groups of ceil(ne2 / n_groups); each group of each ne3 slice is
 * normalised over ne0 x ne1 x its channels with the biased variance. weight and bias (either
 * may be NULL) repeat into a; gelu != 0 applies GELU-erf last. a and dst must be contiguous
 * (dst may be a). workspace: device, 256-byte aligned, stx_group_norm_workspace_size() bytes,
 * no initialisation needed; calls that share a workspace must not run concurrently.
 * Results are deterministic and the same bits whichever path a call takes:
 *   - groups of at most 2^21 floats that fit on the device at once (at most 8 groups, all
 *     blocks resident together) with dst not overlapping a run as one grid-synchronised kernel. Its blocks wait for one
 *     another with bounded waits; a block whose wait gives up (blocks that never became
 *     resident: another process or a concurrent kernel holding CUs) computes its group's
 *     statistics itself from a, in the same order, and counts itself in the workspace's
 *     fallback word (stx_grid_sync_fallbacks). Streams created with a CU mask, HSA_CU_MASK,
 *     ROC_GLOBAL_CU_MASK and STX_NO_GRID_SYNC=1 select the two-kernel path;
 *   - everything else runs as two kernels (three for groups of more than 2^23 floats). */
STX_API size_t     stx_group_norm_workspace_size(const stx_tensor* a, int n_groups);
STX_API stx_status stx_group_norm(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps,
                                  const stx_tensor* weight, const stx_tensor* bias, int gelu, void* workspace,
                                  size_t workspace_bytes, stx_stream stream);

/* Bytes of the static scratch of stx_group_norm_noalloc, per GPU. */
#define STX_GROUP_NORM_SCRATCH_BYTES (1u << 20)

/* stx_group_norm without a workspace argument and without any allocation: no counterpart in
 * the reference. It is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Its scratch is a static
 * device array of STX_GROUP_NORM_SCRATCH_BYTES per GPU, held until the process ends; shapes
 * whose stx_group_norm_workspace_size() exceeds it return INVALID_ARGUMENT. Every call on a
 * GPU shares that GPU's scratch: calls that overlap on one GPU (other streams, other threads)
 * race; calls in one stream are ordered and safe. Same kernels and results as stx_group_norm. */
STX_API stx_status stx_group_norm_noalloc(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps,
                                          const stx_tensor* weight, const stx_tensor* bias, int gelu,
                                          stx_stream stream);

/* Blocks of grid-synchronised kernels that ran on `workspace` (a group-norm or HTDemucs
 * normalisation workspace; NULL: the calling GPU's stx_group_norm_noalloc scratch) and
 * computed their statistics themselves because a wait gave up: a sticky count, read
 * synchronously (the caller synchronises the streams that used the workspace first). The
 * count is a 32-bit word inside the workspace that no call clears: it starts from whatever the
 * workspace held, so it means something only from a workspace the caller zeroed (all of it:
 * the kernels accept a zeroed workspace) before the calls to be counted. The noalloc scratch
 * starts zeroed when the library loads. Not part of the reference; a diagnostic for callers
 * that share the device. */
STX_API stx_status stx_grid_sync_fallbacks(const void* workspace, uint32_t* count);

/* ggml_norm(a, eps) over ne0 (src/htdemucs.cpp:215): (x - mean) / sqrt(var + eps). */
STX_API stx_status stx_norm(const stx_tensor* a, const stx_tensor* dst, float eps, stx_stream stream);
/* layer_norm of src/htdemucs.cpp:213-215: ggml_norm then * weight[ne0] + bias[ne0], fused.
 * weight or bias may be NULL. */
STX_API stx_status stx_norm_affine(const stx_tensor* a, const float* weight, const float* bias, const stx_tensor* dst,
                                   float eps, stx_stream stream);

/* ggml_rms_norm(a, eps) over ne0 (src/roformer.cpp:34): x / sqrt(mean(x^2) + eps). */
STX_API stx_status stx_rms_norm(const stx_tensor* a, const stx_tensor* dst, float eps, stx_stream stream);
/* Graph::rms (src/roformer.cpp:96-98): ggml_rms_norm then * gamma[ne0], fused. */
STX_API stx_status stx_rms_norm_mul(const stx_tensor* a, const float* gamma, const stx_tensor* dst, float eps,
                                    stx_stream stream);

/* ggml_soft_max_ext(a, mask, scale, max_bias) along ne0 (src/roformer.cpp:127,
 * src/htdemucs.cpp:238): softmax(scale * x). The reference passes mask = NULL and
 * max_bias = 0; anything else is UNSUPPORTED. Any row length: rows of up to 2048 floats share
 * a wave, rows of up to 8192 (the HTDemucs scores, Nk = 1,344 or 2,688 tokens) take one block
 * each with the row in registers, longer or unevenly aligned ones one block and three passes.
 * dst may be a. */
STX_API stx_status stx_soft_max_ext(const stx_tensor* a, const stx_tensor* mask, const stx_tensor* dst, float scale,
                                    float max_bias, stx_stream stream);

/* ggml_gelu_erf(a) (src/roformer.cpp:147, src/htdemucs.cpp:136,154,210,246):
 * x/2 * (1 + erf(x / sqrt2)). */
STX_API stx_status stx_gelu_erf(const stx_tensor* a, const stx_tensor* dst, stx_stream stream);
/* ggml_gelu_erf(ggml_add(a, b)) with b repeating into a: the bias add + GELU of the
 * feed-forward layers (src/roformer.cpp:147, src/htdemucs.cpp:246), fused. */
STX_API stx_status stx_add_gelu_erf(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst,
                                    stx_stream stream);

/* GLU, ggml_mul(first half, ggml_sigmoid(second half)) along dimension dim of a
 * (src/htdemucs.cpp:105-110 splits ne2, src/roformer.cpp:199-202 splits ne0). dst has
 * ne[dim] = a->ne[dim] / 2. */
STX_API stx_status stx_glu(const stx_tensor* a, const stx_tensor* dst, int dim, stx_stream stream);

/* ggml_add / ggml_mul with b repeating into a (src/htdemucs.cpp:100,139,220,
 * src/roformer.cpp:97,136,145,148). */
STX_API stx_status stx_add(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst, stx_stream stream);
STX_API stx_status stx_mul(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst, stx_stream stream);
/* ggml_add(x, ggml_mul(h, s)): LayerScale + residual (src/htdemucs.cpp:139,250-251), fused,
 * with the same two roundings. h and s repeat into x. */
STX_API stx_status stx_mul_add(const stx_tensor* x, const stx_tensor* h, const stx_tensor* s, const stx_tensor* dst,
                               stx_stream stream);
/* ggml_add(x, ggml_mul(glu(a), s)): the GLU + LayerScale + residual of a DConv branch
 * (src/htdemucs.cpp:137-139), fused; bit-identical to stx_glu then stx_mul_add. a is split
 * along `dim` as in stx_glu; x, dst have the GLU output's shape; s repeats into dst. */
STX_API stx_status stx_glu_mul_add(const stx_tensor* x, const stx_tensor* a, int dim, const stx_tensor* s,
                                   const stx_tensor* dst, stx_stream stream);

/* ggml_rope_ext(a, pos, NULL, n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor,
 * attn_factor, beta_fast, beta_slow) (src/roformer.cpp:109-113): rotates each ne0 row of
 * position pos[i2] (pos: device int32[ne2]) by theta_i = freq_scale * pos * freq_base^(-2i/n_dims).
 * Mode 0 (the reference's) rotates adjacent pairs, mode 2 (NEOX) pairs (i, i + n_dims/2).
 * ext_factor != 0 (YaRN) and other modes are UNSUPPORTED. */
STX_API stx_status stx_rope_ext(const stx_tensor* a, const int32_t* pos, const stx_tensor* dst, int n_dims, int mode,
                                int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                float beta_fast, float beta_slow, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * Layout glue around attention and the band split: each replaces a chain of ggml view / cont /
 * permute / concat nodes by one pass over HBM, with results identical to that chain.
 * ---------------------------------------------------------------------------------------- */

/* The q/k/v split of RoFormer attention (src/roformer.cpp:101-112): qkv is the projection
 * output [3 * n_head * dh, N, batch] ('b n (qkv h d)'); pos is device int32[N]. Writes
 *   q  = cont(permute(rope_ext(part(0), pos, dh, mode 0, ...), 0, 2, 1, 3))   [dh, N, n_head, batch]
 *   k  = the same for part(1)
 *   vt = cont(permute(part(2), 1, 2, 0, 3))                                  [N, dh, n_head, batch]
 * where part(i) is the dh x n_head slice at i * n_head * dh of each row. dh is q->ne[0]; 32, 64
 * and 128 are built (others are UNSUPPORTED). The rotation is stx_rope_ext's, bit for bit. q, k
 * and vt are dense and must not overlap qkv; qkv rows and q, k are 16-byte aligned. */
STX_API stx_status stx_qkv_rope_split(const stx_tensor* qkv, const int32_t* pos, int n_head, float freq_base,
                                      float freq_scale, float attn_factor, const stx_tensor* q,
                                      const stx_tensor* k, const stx_tensor* vt, stx_stream stream);

/* The head merge after attention (src/roformer.cpp:133-137): dst = cont(permute(o, 0, 2, 1, 3)),
 * o [dh, N, H, batch] -> dst [dh, H, N, batch], times reshape_4d(gates, 1, H, N, batch) when
 * gates (the sigmoid output, [1, H, N, batch]) is not NULL, rounded once like ggml_mul. */
STX_API stx_status stx_merge_heads(const stx_tensor* o, const stx_tensor* gates, const stx_tensor* dst,
                                   stx_stream stream);

/* ggml_cont(ggml_permute(a, ax0, ax1, ax2, ax3)) (src/roformer.cpp:112,133,182,184,190):
 * dimension i of a becomes dimension ax_i of dst. dst must not overlap a. */
STX_API stx_status stx_cont_permute(const stx_tensor* a, int ax0, int ax1, int ax2, int ax3, const stx_tensor* dst,
                                    stx_stream stream);

/* ggml_concat of n_srcs tensors along dim, in order (src/roformer.cpp:52-60 concat_all, :132,
 * :178; n_srcs = 2 is ggml_concat itself): every other dimension of the sources equals dst's,
 * and their extents along dim add up to dst's. srcs is a host array of n_srcs descriptors. */
STX_API stx_status stx_concat(const stx_tensor* const* srcs, int n_srcs, int dim, const stx_tensor* dst,
                              stx_stream stream);


/* ------------------------------------------------------------------------------------------
 * libstems' separate() data path (src/libstems.cpp:135-196) around a model's separate: the
 * request's audio (planar or interleaved, any channel count and rate) is brought to the model's
 * channels (st::to_channels, src/audio.h:62-71) and rate (st::resample_planar, :17-59), the
 * model separates it, and the stems are resampled back with their length pinned to the input's.
 * The GGUF loader and the model graphs stay with the caller, behind the callback.
 * ---------------------------------------------------------------------------------------- */
typedef int32_t stx_audio_layout;
enum {
    STX_AUDIO_PLANAR      = 0,     /* samples[channel * n_samples + sample] (STEMS_AUDIO_PLANAR_V1) */
    STX_AUDIO_INTERLEAVED = 1      /* samples[sample * n_channels + channel] (STEMS_AUDIO_INTERLEAVED_V1) */
};

/* stems_audio_view_v1 (src/libstems_v1.h:84-93) over device samples. Size tagged like the
 * reference's view: a size below STX_AUDIO_VIEW_MIN_SIZE is INVALID_ARGUMENT. */
typedef struct {
    uint32_t size;
    const float* samples;          /* device */
    uint64_t n_samples;            /* per channel */
    uint32_t n_channels;
    uint32_t sample_rate;
    stx_audio_layout layout;
    uint32_t reserved;
} stx_audio_view;

/* The model's Separator::separate at its own rate and channel count (src/separator.h:53,
 * src/libstems.cpp:184): audio device [channels][len] -> stems device [n_sources][channels][len],
 * e.g. stx_demix_track, stx_htdemucs_separate or stx_tfc_tdf_separate around the model's graph.
 * options carries the request's shifts, overlap, seed and callbacks. Work may be enqueued on
 * `stream`. Return STX_STATUS_OK, or a status that stx_separate_audio returns as it is. */
typedef stx_status (*stx_model_separate_fn)(void* user, const float* audio, int channels, int64_t len,
                                            const stx_separate_options* options, float* stems,
                                            stx_stream stream);

/* Bytes of device workspace stx_separate_audio needs for this input and model (0 for an input
 * it rejects). */
STX_API size_t stx_separate_audio_workspace_size(const stx_audio_view* input, int model_channels, int model_rate,
                                                 int n_sources);

/* separate() of libstems V1 (src/libstems.cpp:135-196) on the device. Checks as the reference's
 * (:141-155): INVALID_ARGUMENT for a missing or short view, no samples, a zero count, channel count
 * or rate, an unknown layout, more than INT32_MAX / 4 samples, shifts outside 0..10 or
 * overlap >= 1. Then: the input in planar model channels (:160-167; input channel
 * min(c, n_channels - 1) for model channel c, channel 0 for mono), resampled to model_rate when
 * the rates differ through to_model (a plan for sample_rate -> model_rate), the model's separate,
 * and each stem resampled back through from_model (model_rate -> sample_rate), its length pinned
 * to n_samples: cut, or padded with zeros (:186-196). The plans are unused (may be NULL) when
 * the rates are equal. out: device [n_sources][model_channels][n_samples]. The resampling is
 * stx_resample's (STX_RESAMPLE_EXACT=1 gives the reference's bits). */
STX_API stx_status stx_separate_audio(const stx_audio_view* input, int model_channels, int model_rate, int n_sources,
                                      const stx_resampler* to_model, const stx_resampler* from_model,
                                      stx_model_separate_fn separate, void* separate_user,
                                      const stx_separate_options* options, float* out, void* workspace,
                                      size_t workspace_bytes, stx_stream stream);

/* ------------------------------------------------------------------------------------------
 * Versioned function table (after libstems V1, src/libstems_v1.h:146-189). Every entry point
 * above, in header order; a later revision of V1 may append entries (never reorder them), so
 * a consumer checks `size` against the prefix it needs.
 * ---------------------------------------------------------------------------------------- */
#define STX_ABI_VERSION_1 1u

typedef struct stx_api_v1 {
    uint32_t size;                 /* sizeof the library's table */
    uint32_t abi_version;          /* STX_ABI_VERSION_1 */
    const char*(*version)(void);
    const char*(*last_error)(void);
    stx_status (*fft_create)(int n, stx_fft** out);
    stx_status (*fft_create_any)(int n, stx_fft** out);
    void (*fft_destroy)(stx_fft* fft);
    int (*fft_size)(const stx_fft* fft);
    stx_status (*fft_run)(const stx_fft* fft, float* data, int batch, int inverse,
                          stx_stream stream);
    int (*torch_stft_frames)(int len, int hop);
    int (*htdemucs_frames)(int n_fft, int len);
    stx_status (*torch_stft)(const stx_fft* fft, const float* x, int channels, int len, int hop,
                             int normalized, float* spec, stx_spec_layout layout,
                             stx_stream stream);
    stx_status (*torch_istft)(const stx_fft* fft, const float* spec, int channels, int n_frames,
                              int hop, int normalized, float* out, stx_spec_layout layout,
                              stx_stream stream);
    stx_status (*htdemucs_spec)(const stx_fft* fft, const float* x, int channels, int len,
                                float* spec, stx_spec_layout layout, stx_stream stream);
    stx_status (*htdemucs_ispec)(const stx_fft* fft, const float* spec, int channels, int n_frames,
                                 int length, float* out, stx_spec_layout layout, stx_stream stream);
    size_t (*istft_workspace_size)(const stx_fft* fft, int channels, int n_frames);
    stx_status (*torch_istft_ws)(const stx_fft* fft, const float* spec, int channels, int n_frames,
                                 int hop, int normalized, float* out, stx_spec_layout layout,
                                 void* workspace, size_t workspace_bytes, stx_stream stream);
    stx_status (*htdemucs_ispec_ws)(const stx_fft* fft, const float* spec, int channels,
                                    int n_frames, int length, float* out, stx_spec_layout layout,
                                    void* workspace, size_t workspace_bytes, stx_stream stream);
    stx_status (*mel_band_map)(int sample_rate, int n_fft, int n_mels, int32_t* band_sizes,
                               int32_t* band_freqs, int64_t capacity, int64_t* n_freqs);
    stx_status (*bs_band_map)(const int32_t* freqs_per_bands, int n_bands, int n_fft,
                              int32_t* band_freqs, int64_t capacity, int64_t* n_freqs);
    stx_status (*bands_layout)(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs,
                               int64_t n_freqs, int n_bins, int channels, int64_t* band_freq_off,
                               int64_t* band_feat_off, int32_t* bands_per_freq);
    stx_status (*bands_create)(const int32_t* band_sizes, int n_bands, const int32_t* band_freqs,
                               int64_t n_freqs, int n_bins, int channels, stx_bands** out);
    void (*bands_destroy)(stx_bands* bands);
    int64_t (*bands_total_feat)(const stx_bands* bands);
    stx_status (*band_gather)(const stx_bands* bands, const float* spec, int batch, int n_frames,
                              stx_spec_layout layout, float* feat, stx_stream stream);
    stx_status (*band_scatter_apply)(const stx_bands* bands, const float* masks, int n_stems,
                                     const float* spec, int batch, int n_frames,
                                     stx_spec_layout layout, int zero_dc, float* out,
                                     stx_stream stream);
    stx_status (*band_rms_norm)(const stx_bands* bands, const float* feat, int batch, int n_frames,
                                const float* const* gammas, float eps, float* out,
                                stx_stream stream);
    stx_status (*band_mask_glu)(const stx_bands* bands, const float* const* heads, int n_stems,
                                int n_frames, float* masks, stx_stream stream);
    int (*demix_step)(int chunk, int num_overlap, float overlap);
    stx_status (*demix_plan)(int64_t len, int chunk, int step, stx_demix_geometry* geom,
                             stx_chunk* chunks, int64_t capacity);
    stx_status (*demix_plan_rules)(int64_t len, int chunk, int step, stx_demix_rules rules,
                                   stx_demix_geometry* geom, stx_chunk* chunks, int64_t capacity);
    stx_status (*demix_window)(int chunk, float* window);
    stx_status (*demix_window_rules)(int chunk, stx_demix_rules rules, float* window);
    stx_status (*demix_create)(int64_t len, int channels, int chunk, int step, stx_demix** out);
    stx_status (*demix_create_rules)(int64_t len, int channels, int chunk, int step,
                                     stx_demix_rules rules, stx_demix** out);
    void (*demix_destroy)(stx_demix* demix);
    int64_t (*demix_n_chunks)(const stx_demix* demix);
    stx_status (*demix_chunks)(const stx_demix* demix, const float* mix, int64_t first,
                               int64_t count, float* parts, stx_stream stream);
    stx_status (*demix_overlap_add)(const stx_demix* demix, const float* y, int n_stems,
                                    float* out, stx_stream stream);
    stx_status (*separate_options_init)(stx_separate_options* options);
    size_t (*demix_track_workspace_size)(int channels, int64_t len, int chunk, int step,
                                         int n_stems, int batch, int shifts, int sample_rate);
    stx_status (*demix_track)(const float* mix, int channels, int64_t len, int chunk,
                              int num_overlap, int n_stems, int complement, int sample_rate,
                              int batch, stx_separate_fn separate, void* separate_user,
                              const stx_separate_options* options, float* out, void* workspace,
                              size_t workspace_bytes, stx_stream stream);
    stx_status (*uvr_demix_create)(int64_t len, int channels, int chunk, int n_fft, float overlap,
                                   stx_uvr_demix** out);
    void (*uvr_demix_destroy)(stx_uvr_demix* demix);
    int64_t (*uvr_demix_n_chunks)(const stx_uvr_demix* demix);
    stx_status (*uvr_demix_geometry)(const stx_uvr_demix* demix, int64_t* padded_len,
                                     int64_t* step, int* trim);
    stx_status (*uvr_demix_chunks)(const stx_uvr_demix* demix, const float* mix, int64_t first,
                                   int64_t count, float* parts, stx_stream stream);
    stx_status (*uvr_demix_overlap_add)(const stx_uvr_demix* demix, const float* y, int n_stems,
                                        float* out, stx_stream stream);
    size_t (*tfc_tdf_separate_workspace_size)(int channels, int64_t len, int chunk, int n_fft,
                                              stx_tfc_chunking chunking, int num_overlap,
                                              float overlap, int n_stems, int batch);
    stx_status (*tfc_tdf_separate)(const float* mix, int channels, int64_t len, int chunk,
                                   int n_fft, stx_tfc_chunking chunking, int num_overlap,
                                   int n_stems, float compensate, int complement, int batch,
                                   stx_separate_fn separate, void* separate_user,
                                   const stx_separate_options* options, float* out,
                                   void* workspace, size_t workspace_bytes, stx_stream stream);
    stx_status (*resampler_create)(int src_rate, int dst_rate, stx_resampler** out);
    void (*resampler_destroy)(stx_resampler* resampler);
    int64_t (*resample_length)(const stx_resampler* resampler, int64_t n);
    stx_status (*resample)(const stx_resampler* resampler, const float* in, int channels,
                           int64_t n, float* out, stx_stream stream);
    size_t (*htdemucs_norm_workspace_size)(int64_t n);
    stx_status (*htdemucs_cac_normalize)(const float* spec, int channels, int n_bins, int n_frames,
                                         float* mag, double* stats, void* workspace,
                                         size_t workspace_bytes, stx_stream stream);
    stx_status (*htdemucs_wave_normalize)(const float* x, int64_t n, float* out, double* stats,
                                          void* workspace, size_t workspace_bytes,
                                          stx_stream stream);
    stx_status (*htdemucs_mix_normalize)(const float* mix, int channels, int64_t len, float* out,
                                         double* stats, void* workspace, size_t workspace_bytes,
                                         stx_stream stream);
    stx_status (*htdemucs_cac_denormalize)(const float* ox, int n_sources, int channels,
                                           int n_bins, int n_frames, const double* stats,
                                           float* spec, stx_stream stream);
    stx_status (*htdemucs_time_add)(const float* xt, const float* y, int64_t n,
                                    const double* stats, float* out, stx_stream stream);
    stx_status (*htdemucs_split_plan)(int length, int segment, float overlap, int* stride,
                                      int* n_chunks);
    stx_status (*htdemucs_segments)(const float* buf, int channels, int64_t total, int64_t offset,
                                    int length, int segment, int stride, int first, int count,
                                    float* parts, stx_stream stream);
    stx_status (*htdemucs_split_overlap_add)(const float* y, int tracks, int length, int segment,
                                             int stride, float* out, stx_stream stream);
    size_t (*htdemucs_separate_workspace_size)(int channels, int64_t len, int segment,
                                               int n_sources, int batch, int shifts,
                                               int sample_rate, float overlap);
    stx_status (*htdemucs_separate)(const float* mix, int channels, int64_t len, int segment,
                                    int n_sources, int n_models, const float* bag_weights,
                                    int sample_rate, int batch, stx_model_fn forward,
                                    void* forward_user, const stx_separate_options* options,
                                    float* out, void* workspace, size_t workspace_bytes,
                                    stx_stream stream);
    size_t (*group_norm_workspace_size)(const stx_tensor* a, int n_groups);
    stx_status (*group_norm)(const stx_tensor* a, const stx_tensor* dst, int n_groups, float eps,
                             const stx_tensor* weight, const stx_tensor* bias, int gelu,
                             void* workspace, size_t workspace_bytes, stx_stream stream);
    stx_status (*group_norm_noalloc)(const stx_tensor* a, const stx_tensor* dst, int n_groups,
                                     float eps, const stx_tensor* weight, const stx_tensor* bias,
                                     int gelu, stx_stream stream);
    stx_status (*grid_sync_fallbacks)(const void* workspace, uint32_t* count);
    stx_status (*norm)(const stx_tensor* a, const stx_tensor* dst, float eps, stx_stream stream);
    stx_status (*norm_affine)(const stx_tensor* a, const float* weight, const float* bias,
                              const stx_tensor* dst, float eps, stx_stream stream);
    stx_status (*rms_norm)(const stx_tensor* a, const stx_tensor* dst, float eps,
                           stx_stream stream);
    stx_status (*rms_norm_mul)(const stx_tensor* a, const float* gamma, const stx_tensor* dst,
                               float eps, stx_stream stream);
    stx_status (*soft_max_ext)(const stx_tensor* a, const stx_tensor* mask, const stx_tensor* dst,
                               float scale, float max_bias, stx_stream stream);
    stx_status (*gelu_erf)(const stx_tensor* a, const stx_tensor* dst, stx_stream stream);
    stx_status (*add_gelu_erf)(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst,
                               stx_stream stream);
    stx_status (*glu)(const stx_tensor* a, const stx_tensor* dst, int dim, stx_stream stream);
    stx_status (*add)(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst,
                      stx_stream stream);
    stx_status (*mul)(const stx_tensor* a, const stx_tensor* b, const stx_tensor* dst,
                      stx_stream stream);
    stx_status (*mul_add)(const stx_tensor* x, const stx_tensor* h, const stx_tensor* s,
                          const stx_tensor* dst, stx_stream stream);
    stx_status (*glu_mul_add)(const stx_tensor* x, const stx_tensor* a, int dim,
                              const stx_tensor* s, const stx_tensor* dst, stx_stream stream);
    stx_status (*rope_ext)(const stx_tensor* a, const int32_t* pos, const stx_tensor* dst,
                           int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
                           float ext_factor, float attn_factor, float beta_fast, float beta_slow,
                           stx_stream stream);
    stx_status (*qkv_rope_split)(const stx_tensor* qkv, const int32_t* pos, int n_head,
                                 float freq_base, float freq_scale, float attn_factor,
                                 const stx_tensor* q, const stx_tensor* k, const stx_tensor* vt,
                                 stx_stream stream);
    stx_status (*merge_heads)(const stx_tensor* o, const stx_tensor* gates, const stx_tensor* dst,
                              stx_stream stream);
    stx_status (*cont_permute)(const stx_tensor* a, int ax0, int ax1, int ax2, int ax3,
                               const stx_tensor* dst, stx_stream stream);
    stx_status (*concat)(const stx_tensor* const* srcs, int n_srcs, int dim, const stx_tensor* dst,
                         stx_stream stream);
    /* Appended to V1 after STX_API_V1_MIN_SIZE: check `size` before using these. */
    size_t (*separate_audio_workspace_size)(const stx_audio_view* input, int model_channels,
                                            int model_rate, int n_sources);
    stx_status (*separate_audio)(const stx_audio_view* input, int model_channels, int model_rate,
                                 int n_sources, const stx_resampler* to_model,
                                 const stx_resampler* from_model, stx_model_separate_fn separate,
                                 void* separate_user, const stx_separate_options* options,
                                 float* out, void* workspace, size_t workspace_bytes,
                                 stx_stream stream);
    void (*reserved[16])(void);
} stx_api_v1;

/* Frozen V1 prefixes: each names the last field of the initial V1 contract. */
#define STX_FIELD_END(type, field) ((uint32_t)(offsetof(type, field) + sizeof(((type*)0)->field)))
#define STX_SEPARATE_OPTIONS_MIN_SIZE STX_FIELD_END(stx_separate_options, user)
#define STX_DEMIX_GEOMETRY_MIN_SIZE   STX_FIELD_END(stx_demix_geometry, n_chunks)
#define STX_API_V1_MIN_SIZE           STX_FIELD_END(stx_api_v1, concat)
#define STX_AUDIO_VIEW_MIN_SIZE       STX_FIELD_END(stx_audio_view, reserved)

/* The one symbol a dynamically loading consumer resolves: the static V1 table (owned by the
 * library for the lifetime of the module) for abi_version STX_ABI_VERSION_1, NULL for any other
 * version. */
STX_API const stx_api_v1* stx_get_api(uint32_t abi_version);

#ifdef __cplusplus
}
#endif

#endif /* STX_H */
