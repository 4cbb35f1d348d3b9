// rng_oracle.cpp — CPU oracle (test infrastructure): the shift offsets of the reference's
// separate() loops, drawn with the C++ standard library exactly as the reference draws them
// (std::mt19937 seeded once, std::uniform_int_distribution<int> per model).
#include <cstdint>
#include <random>

extern "C" {

// HTDemucs::separate (src/htdemucs.cpp:580,616-619): one rng for all models, dist(0, max_shift)
// per model, `shifts` draws each. offsets: [n_models][shifts].
void orc_htdemucs_shift_offsets(uint32_t seed, int max_shift, int n_models, int shifts, int32_t* offsets) {
    std::mt19937 rng(seed);
    for (int m = 0; m < n_models; m++) {
        std::uniform_int_distribution<int> dist(0, max_shift);
        for (int k = 0; k < shifts; k++) offsets[m * shifts + k] = dist(rng);
    }
}

}  // extern "C"
