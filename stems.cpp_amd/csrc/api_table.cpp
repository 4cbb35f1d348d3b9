// api_table.cpp — the versioned function table (stx_get_api) and the initialiser of the size-tagged
// separate options of the C ABI.
#include <algorithm>
#include <cstring>

#include "common.hpp"

namespace {
const stx_api_v1 kApiV1 = {
    sizeof(stx_api_v1),
    STX_ABI_VERSION_1,
    &stx_version,
    &stx_last_error,
    &stx_fft_create,
    &stx_fft_create_any,
    &stx_fft_destroy,
    &stx_fft_size,
    &stx_fft_run,
    &stx_torch_stft_frames,
    &stx_htdemucs_frames,
    &stx_torch_stft,
    &stx_torch_istft,
    &stx_htdemucs_spec,
    &stx_htdemucs_ispec,
    &stx_istft_workspace_size,
    &stx_torch_istft_ws,
    &stx_htdemucs_ispec_ws,
    &stx_mel_band_map,
    &stx_bs_band_map,
    &stx_bands_layout,
    &stx_bands_create,
    &stx_bands_destroy,
    &stx_bands_total_feat,
    &stx_band_gather,
    &stx_band_scatter_apply,
    &stx_band_rms_norm,
    &stx_band_mask_glu,
    &stx_demix_step,
    &stx_demix_plan,
    &stx_demix_plan_rules,
    &stx_demix_window,
    &stx_demix_window_rules,
    &stx_demix_create,
    &stx_demix_create_rules,
    &stx_demix_destroy,
    &stx_demix_n_chunks,
    &stx_demix_chunks,
    &stx_demix_overlap_add,
    &stx_separate_options_init,
    &stx_demix_track_workspace_size,
    &stx_demix_track,
    &stx_uvr_demix_create,
    &stx_uvr_demix_destroy,
    &stx_uvr_demix_n_chunks,
    &stx_uvr_demix_geometry,
    &stx_uvr_demix_chunks,
    &stx_uvr_demix_overlap_add,
    &stx_tfc_tdf_separate_workspace_size,
    &stx_tfc_tdf_separate,
    &stx_resampler_create,
    &stx_resampler_destroy,
    &stx_resample_length,
    &stx_resample,
    &stx_htdemucs_norm_workspace_size,
    &stx_htdemucs_cac_normalize,
    &stx_htdemucs_wave_normalize,
    &stx_htdemucs_mix_normalize,
    &stx_htdemucs_cac_denormalize,
    &stx_htdemucs_time_add,
    &stx_htdemucs_split_plan,
    &stx_htdemucs_segments,
    &stx_htdemucs_split_overlap_add,
    &stx_htdemucs_separate_workspace_size,
    &stx_htdemucs_separate,
    &stx_group_norm_workspace_size,
    &stx_group_norm,
    &stx_group_norm_noalloc,
    &stx_grid_sync_fallbacks,
    &stx_norm,
    &stx_norm_affine,
    &stx_rms_norm,
    &stx_rms_norm_mul,
    &stx_soft_max_ext,
    &stx_gelu_erf,
    &stx_add_gelu_erf,
    &stx_glu,
    &stx_add,
    &stx_mul,
    &stx_mul_add,
    &stx_glu_mul_add,
    &stx_rope_ext,
    &stx_qkv_rope_split,
    &stx_merge_heads,
    &stx_cont_permute,
    &stx_concat,
    &stx_separate_audio_workspace_size,
    &stx_separate_audio,
    {},
};
}  // namespace

extern "C" {

STX_API const stx_api_v1* stx_get_api(uint32_t abi_version) {
    return abi_version == STX_ABI_VERSION_1 ? &kApiV1 : nullptr;
}

STX_API stx_status stx_separate_options_init(stx_separate_options* options) {
    return stx::guard([&] {
        STX_REQUIRE(options != nullptr, "separate options: NULL");
        STX_REQUIRE(options->size >= STX_SEPARATE_OPTIONS_MIN_SIZE, "separate options: size %u is below the V1 minimum %u",
                    options->size, STX_SEPARATE_OPTIONS_MIN_SIZE);
        const stx_separate_options d = stx::default_separate_options();
        std::memcpy(reinterpret_cast<char*>(options) + sizeof(uint32_t), reinterpret_cast<const char*>(&d) + sizeof(uint32_t),
                    std::min<size_t>(options->size, sizeof d) - sizeof(uint32_t));
    });
}

}  // extern "C"
