/* abi_check: the V1 table contract a run-time loading consumer relies on. libstx.so (argv[1],
 * an absolute path) is dlopen'ed and only stx_get_api is resolved through dlsym for the calls;
 * the other dlsym lookups only cross-check that each table entry is the function of its name.
 * Pure C on purpose: the public header must stay C-clean. Every call here is host-only or
 * fails its argument checks before any device work, so this runs without a GPU.
 * Exit status 0 when every check passes. */
#include "stx.h"

#include <dlfcn.h>
#include <stdio.h>
#include <string.h>

typedef const stx_api_v1* (*get_api_fn)(uint32_t);

static int failures = 0;

static void check(int ok, const char* what) {
    printf("  %-66s %s\n", what, ok ? "ok" : "FAIL");
    if (!ok) failures++;
}

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: abi_check LIBRARY\n");
        return 2;
    }
    void* lib = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!lib) {
        printf("FAIL: dlopen(%s): %s\n", argv[1], dlerror());
        return 1;
    }
    get_api_fn get_api = (get_api_fn)dlsym(lib, "stx_get_api");
    if (!get_api) {
        printf("FAIL: no stx_get_api\n");
        return 1;
    }

    printf("table\n");
    const stx_api_v1* api = get_api(STX_ABI_VERSION_1);
    check(api != NULL, "stx_get_api(1) returns the V1 table");
    if (!api) return 1;
    check(get_api(0) == NULL && get_api(2) == NULL && get_api(0x10001u) == NULL,
          "stx_get_api(0), (2) and (0x10001) return NULL");
    check(api->abi_version == STX_ABI_VERSION_1 && api->size >= STX_API_V1_MIN_SIZE,
          "abi_version 1, size covers the frozen V1 table");
    check(get_api(STX_ABI_VERSION_1) == api, "the table is one static object");
    int all = 1;
#define CHECK_FN(field, name)                                                       \
    do {                                                                            \
        void* sym = dlsym(lib, name);                                               \
        if (api->field == NULL || sym == NULL || (void*)api->field != sym) {        \
            printf("    table entry %s does not match %s\n", #field, name);        \
            all = 0;                                                                \
        }                                                                           \
    } while (0)
    CHECK_FN(version, "stx_version");
    CHECK_FN(last_error, "stx_last_error");
    CHECK_FN(fft_create, "stx_fft_create");
    CHECK_FN(fft_create_any, "stx_fft_create_any");
    CHECK_FN(fft_destroy, "stx_fft_destroy");
    CHECK_FN(fft_size, "stx_fft_size");
    CHECK_FN(fft_run, "stx_fft_run");
    CHECK_FN(torch_stft_frames, "stx_torch_stft_frames");
    CHECK_FN(htdemucs_frames, "stx_htdemucs_frames");
    CHECK_FN(torch_stft, "stx_torch_stft");
    CHECK_FN(torch_istft, "stx_torch_istft");
    CHECK_FN(htdemucs_spec, "stx_htdemucs_spec");
    CHECK_FN(htdemucs_ispec, "stx_htdemucs_ispec");
    CHECK_FN(istft_workspace_size, "stx_istft_workspace_size");
    CHECK_FN(torch_istft_ws, "stx_torch_istft_ws");
    CHECK_FN(htdemucs_ispec_ws, "stx_htdemucs_ispec_ws");
    CHECK_FN(mel_band_map, "stx_mel_band_map");
    CHECK_FN(bs_band_map, "stx_bs_band_map");
    CHECK_FN(bands_layout, "stx_bands_layout");
    CHECK_FN(bands_create, "stx_bands_create");
    CHECK_FN(bands_destroy, "stx_bands_destroy");
    CHECK_FN(bands_total_feat, "stx_bands_total_feat");
    CHECK_FN(band_gather, "stx_band_gather");
    CHECK_FN(band_scatter_apply, "stx_band_scatter_apply");
    CHECK_FN(band_rms_norm, "stx_band_rms_norm");
    CHECK_FN(band_mask_glu, "stx_band_mask_glu");
    CHECK_FN(demix_step, "stx_demix_step");
    CHECK_FN(demix_plan, "stx_demix_plan");
    CHECK_FN(demix_plan_rules, "stx_demix_plan_rules");
    CHECK_FN(demix_window, "stx_demix_window");
    CHECK_FN(demix_window_rules, "stx_demix_window_rules");
    CHECK_FN(demix_create, "stx_demix_create");
    CHECK_FN(demix_create_rules, "stx_demix_create_rules");
    CHECK_FN(demix_destroy, "stx_demix_destroy");
    CHECK_FN(demix_n_chunks, "stx_demix_n_chunks");
    CHECK_FN(demix_chunks, "stx_demix_chunks");
    CHECK_FN(demix_overlap_add, "stx_demix_overlap_add");
    CHECK_FN(separate_options_init, "stx_separate_options_init");
    CHECK_FN(demix_track_workspace_size, "stx_demix_track_workspace_size");
    CHECK_FN(demix_track, "stx_demix_track");
    CHECK_FN(uvr_demix_create, "stx_uvr_demix_create");
    CHECK_FN(uvr_demix_destroy, "stx_uvr_demix_destroy");
    CHECK_FN(uvr_demix_n_chunks, "stx_uvr_demix_n_chunks");
    CHECK_FN(uvr_demix_geometry, "stx_uvr_demix_geometry");
    CHECK_FN(uvr_demix_chunks, "stx_uvr_demix_chunks");
    CHECK_FN(uvr_demix_overlap_add, "stx_uvr_demix_overlap_add");
    CHECK_FN(tfc_tdf_separate_workspace_size, "stx_tfc_tdf_separate_workspace_size");
    CHECK_FN(tfc_tdf_separate, "stx_tfc_tdf_separate");
    CHECK_FN(resampler_create, "stx_resampler_create");
    CHECK_FN(resampler_destroy, "stx_resampler_destroy");
    CHECK_FN(resample_length, "stx_resample_length");
    CHECK_FN(resample, "stx_resample");
    CHECK_FN(htdemucs_norm_workspace_size, "stx_htdemucs_norm_workspace_size");
    CHECK_FN(htdemucs_cac_normalize, "stx_htdemucs_cac_normalize");
    CHECK_FN(htdemucs_wave_normalize, "stx_htdemucs_wave_normalize");
    CHECK_FN(htdemucs_mix_normalize, "stx_htdemucs_mix_normalize");
    CHECK_FN(htdemucs_cac_denormalize, "stx_htdemucs_cac_denormalize");
    CHECK_FN(htdemucs_time_add, "stx_htdemucs_time_add");
    CHECK_FN(htdemucs_split_plan, "stx_htdemucs_split_plan");
    CHECK_FN(htdemucs_segments, "stx_htdemucs_segments");
    CHECK_FN(htdemucs_split_overlap_add, "stx_htdemucs_split_overlap_add");
    CHECK_FN(htdemucs_separate_workspace_size, "stx_htdemucs_separate_workspace_size");
    CHECK_FN(htdemucs_separate, "stx_htdemucs_separate");
    CHECK_FN(group_norm_workspace_size, "stx_group_norm_workspace_size");
    CHECK_FN(group_norm, "stx_group_norm");
    CHECK_FN(group_norm_noalloc, "stx_group_norm_noalloc");
    CHECK_FN(grid_sync_fallbacks, "stx_grid_sync_fallbacks");
    CHECK_FN(norm, "stx_norm");
    CHECK_FN(norm_affine, "stx_norm_affine");
    CHECK_FN(rms_norm, "stx_rms_norm");
    CHECK_FN(rms_norm_mul, "stx_rms_norm_mul");
    CHECK_FN(soft_max_ext, "stx_soft_max_ext");
    CHECK_FN(gelu_erf, "stx_gelu_erf");
    CHECK_FN(add_gelu_erf, "stx_add_gelu_erf");
    CHECK_FN(glu, "stx_glu");
    CHECK_FN(add, "stx_add");
    CHECK_FN(mul, "stx_mul");
    CHECK_FN(mul_add, "stx_mul_add");
    CHECK_FN(glu_mul_add, "stx_glu_mul_add");
    CHECK_FN(rope_ext, "stx_rope_ext");
    CHECK_FN(qkv_rope_split, "stx_qkv_rope_split");
    CHECK_FN(merge_heads, "stx_merge_heads");
    CHECK_FN(cont_permute, "stx_cont_permute");
    CHECK_FN(concat, "stx_concat");
    check(all, "every entry is set and is the exported function of its name");
    /* Entries appended after the frozen V1 prefix: present when size covers them. */
    check(api->size >= offsetof(stx_api_v1, separate_audio) + sizeof(api->separate_audio),
          "the table covers the appended separate_audio entries");
    all = 1;
    CHECK_FN(separate_audio_workspace_size, "stx_separate_audio_workspace_size");
    CHECK_FN(separate_audio, "stx_separate_audio");
    check(all, "appended entries are the exported functions of their names");
    {
        stx_audio_view view;
        memset(&view, 0, sizeof view);
        view.size = sizeof view;
        check(api->separate_audio_workspace_size(&view, 2, 44100, 4) == 0,
              "separate_audio_workspace_size is 0 for an empty view");
        view.size = 4;
        check(api->separate_audio(&view, 2, 44100, 4, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL) ==
                  STX_STATUS_INVALID_ARGUMENT && api->last_error()[0] != '\0',
              "separate_audio with a too-small view is INVALID_ARGUMENT");
        check(STX_AUDIO_VIEW_MIN_SIZE == sizeof view, "STX_AUDIO_VIEW_MIN_SIZE is the V1 view");
    }
    const char* v = api->version();
    check(v != NULL && strchr(v, '.') != NULL, "version() through the table");
    printf("  version: %s\n", v ? v : "(null)");

    printf("size-tagged structs\n");
    check(api->separate_options_init(NULL) == STX_STATUS_INVALID_ARGUMENT, "separate_options_init(NULL)");
    stx_separate_options opt;
    memset(&opt, 0, sizeof opt);
    opt.size = 4;
    check(api->separate_options_init(&opt) == STX_STATUS_INVALID_ARGUMENT && api->last_error()[0] != '\0',
          "separate_options_init with a too-small size is INVALID_ARGUMENT");
    memset(&opt, 0, sizeof opt);
    opt.size = sizeof opt;
    opt.shifts = 7;
    check(api->separate_options_init(&opt) == STX_STATUS_OK && opt.shifts == 0 && opt.overlap == -1.0f &&
              opt.seed == 0 && opt.progress == NULL && opt.should_cancel == NULL && opt.size == sizeof opt,
          "separate_options_init writes the defaults, keeps size");
    stx_separate_options small = opt;
    small.size = 4;
    float dummy = 0.f;
    check(api->demix_track(&dummy, 2, 1000, 352800, 4, 4, 0, 44100, 1, NULL, NULL, &small, &dummy, &dummy, 1 << 20,
                           NULL) == STX_STATUS_INVALID_ARGUMENT,
          "demix_track with truncated options is INVALID_ARGUMENT");
    check(api->demix_track(NULL, 2, 1000, 352800, 4, 4, 0, 44100, 1, NULL, NULL, &opt, NULL, NULL, 0, NULL) ==
              STX_STATUS_INVALID_ARGUMENT,
          "demix_track with NULL buffers is INVALID_ARGUMENT");

    stx_demix_geometry g;
    memset(&g, 0, sizeof g);
    g.size = 8;
    check(api->demix_plan(7938000, 352800, 88200, &g, NULL, 0) == STX_STATUS_INVALID_ARGUMENT,
          "demix_plan with a too-small geometry is INVALID_ARGUMENT");
    memset(&g, 0, sizeof g);
    g.size = sizeof g;
    check(api->demix_plan(7938000, 352800, 88200, &g, NULL, 0) == STX_STATUS_OK && g.n_chunks == 96 &&
              g.padded_len == 8467200 && g.border == 264600 && g.fade == 35280 && g.size == sizeof g,
          "demix_plan: the 180 s geometry (96 chunks, Lp 8,467,200)");
    stx_chunk chunks[96];
    check(api->demix_plan(7938000, 352800, 88200, &g, chunks, 96) == STX_STATUS_OK && chunks[95].start == 95 * 88200LL &&
              chunks[95].pad_mode == STX_CHUNK_ZERO && chunks[0].fade_in == 0,
          "demix_plan: chunk table through the table");
    check(api->demix_plan(0, 352800, 88200, &g, NULL, 0) == STX_STATUS_INVALID_ARGUMENT, "demix_plan(len 0)");

    printf("host-only calls through the table\n");
    int64_t nf = 0;
    int32_t sizes[60];
    int32_t freqs[4096];
    check(api->mel_band_map(44100, 2048, 60, sizes, freqs, 4096, &nf) == STX_STATUS_OK && nf == 1979 &&
              sizes[0] == 7 && sizes[59] == 130,
          "mel_band_map: 60 bands, 1,979 entries");
    check(api->torch_stft_frames(352800, 441) == 801 && api->htdemucs_frames(4096, 343980) == 336, "frame counts");
    check(api->demix_step(352800, 4, -1.0f) == 88200, "demix_step");
    stx_fft* f = NULL;
    check(api->fft_create(12, &f) == STX_STATUS_INVALID_ARGUMENT && f == NULL, "fft_create(12) is INVALID_ARGUMENT");
    check(api->group_norm(NULL, NULL, 1, 1e-5f, NULL, NULL, 0, NULL, 0, NULL) == STX_STATUS_INVALID_ARGUMENT,
          "group_norm(NULL) is INVALID_ARGUMENT");

    printf(failures ? "FAILED (%d)\n" : "all ok\n", failures);
    return failures ? 1 : 0;
}
