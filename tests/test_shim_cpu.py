"""The C++ shim's test helper loads and maps the reference's argument errors to
std::invalid_argument without touching a GPU (the checks run before any device call)."""
import shim_lib


def test_shim_helper_loads_and_rejects_bad_sizes():
    L = shim_lib.lib()
    assert L.shim_fft_create(3) == 1       # not a power of two: std::invalid_argument
    assert L.shim_fft_create(0) == 1
    assert L.shim_fft_create(1 << 25) == 2   # a power of two above the plan limit: runtime_error
