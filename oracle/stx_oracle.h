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
 */
#ifndef STX_ORACLE_H
#define STX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* st::FFT (src/stft.h:19-55): in-place radix-2 DIT, unnormalised; inverse = conj twiddles. */
int orc_fft(double* a, int n, int inverse);

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

#ifdef __cplusplus
}
#endif

#endif /* STX_ORACLE_H */
