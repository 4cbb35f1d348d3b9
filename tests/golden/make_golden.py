"""Writes the STFT golden vectors in this directory from the reference's own src/stft.h.

Run where /root/reference exists after `make -C oracle` has built oracle/_ref/libstft_ref.so:
    python tests/golden/make_golden.py
Each case is an .npz of inputs and the reference's outputs (float64 spectra, float32 signals),
at small seeded sizes following the reference's own tests (tests/dsp_test.cpp:53-96): the
FFT round trip at 4096, torch_stft/istft at n_fft 2048 / hop 441 (both `normalized`
values), and htdemucs_spec/ispec at 4096 / 1024, plus ragged lengths and tiny sizes.
Inputs come from stems.cpp_amd/synth.py (splitmix64 + Box-Muller, sigma 0.1).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "stems.cpp_amd"))

import oracle_lib  # noqa: E402
import synth  # noqa: E402


def main():
    ref = oracle_lib.reference()
    cases = {}
    # FFT: random complex vectors, forward then inverse (dsp_test.cpp:53-64), and an impulse.
    for n, seed in [(16, 11), (2048, 12), (4096, 13)]:
        v = synth.normal(seed, (2 * n,), 0.5).astype(np.float64)
        a = v[0::2] + 1j * v[1::2]
        X = ref.fft(a, False)
        cases[f"fft_{n}"] = dict(x=a, X=X, x_back=ref.fft(X, True))
    imp = np.zeros(4096, dtype=np.complex128)
    imp[7] = 1.0
    cases["fft_impulse_4096"] = dict(x=imp, X=ref.fft(imp, False))
    # torch_stft / torch_istft (dsp_test.cpp:66-78 uses n_fft 2048, hop 441).
    for name, n_fft, hop, length, seed in [
        ("torch_2048_441", 2048, 441, 441 * 20, 21),
        ("torch_2048_441_ragged", 2048, 441, 441 * 20 + 100, 22),
        ("torch_16_4", 16, 4, 40, 23),
        ("torch_4096_1024", 4096, 1024, 1024 * 8 + 7, 24),
    ]:
        x = synth.normal(seed, (length,), 0.1)
        for norm in (0, 1):
            spec = ref.torch_stft(x, n_fft, hop, bool(norm))
            y = ref.torch_istft(spec, n_fft, hop, bool(norm))
            cases[f"{name}_n{norm}"] = dict(x=x, spec=spec, y=y, n_fft=n_fft, hop=hop, normalized=norm)
    # htdemucs_spec / htdemucs_ispec (dsp_test.cpp:80-96 uses 4096 / 1024).
    for name, n_fft, length, seed in [
        ("htdemucs_4096", 4096, 1024 * 12, 31),
        ("htdemucs_4096_ragged", 4096, 1024 * 12 - 300, 32),
        ("htdemucs_64", 64, 16 * 9 + 5, 33),
    ]:
        x = synth.normal(seed, (length,), 0.1)
        spec = ref.htdemucs_spec(x, n_fft)
        y = ref.htdemucs_ispec(spec, n_fft, length)
        cases[name] = dict(x=x, spec=spec, y=y, n_fft=n_fft)
    for name, arrays in cases.items():
        np.savez_compressed(os.path.join(HERE, f"stft_{name}.npz"), **{k: np.asarray(v) for k, v in arrays.items()})
        print("wrote", name)


if __name__ == "__main__":
    main()
