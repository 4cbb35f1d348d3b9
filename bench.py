"""Benchmark of the spectral hot path on one MI355X.

Headline workload (one "step"): the HTDemucs-spec STFT -> iSTFT round trip on stereo fp32,
343,980 samples per channel (7.8 s at 44.1 kHz), n_fft 4096, hop 1024, periodic Hann, reflect
pad, center=True: stx_htdemucs_spec then stx_htdemucs_ispec, the drop-in replacements of
src/stft.h:79-140, spectrum in the reference's f-major layout. Inputs are resident in HBM
before timing and rotate over enough copies (> 512 MB) that the 256 MB Infinity Cache cannot
hold them, so the numbers are cold-cache numbers.

value = Msamples/s = 2 * 343,980 samples per step / step time.
roofline: the slower of the two kernels, algorithmic bytes per launch (fp32 signal read or
written once + complex64 spectrum written or read once = 13,761,888 B) / its average
duration, timed with HIP events on the stream the kernels run on.
cpu_baseline: the reference's own stft.h (oracle/_ref, built from the reference sources) or,
where that is absent, the C oracle restating it, single-threaded as the reference runs it,
on a bounded number of round trips of the same input.

Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stems.cpp_amd"))

METRIC = "STFT+iSTFT Msamples/s; norm/softmax/elementwise HBM GB/s (% of 8 TB/s)"
HBM_PEAK_GBS = 8000.0
C1_LEN, C1_NFFT = 343980, 4096


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def traffic_for(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    a copy kernel of known size), if that measurement was committed under profiles/."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(kernel)


def cpu_baseline(x, budget_s):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    kind = "reference" if oracle_lib.ref_available() else "port"
    lib = oracle_lib.reference() if kind == "reference" else oracle_lib.oracle()
    C, L = x.shape
    reps = 0
    t0 = time.perf_counter()
    while True:
        for c in range(C):
            s = lib.htdemucs_spec(x[c], C1_NFFT)
            lib.htdemucs_ispec(s, C1_NFFT, L)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {
        "value": round(reps * C * L / el / 1e6, 3),
        "unit": "Msamples/s",
        "cores": 1,
        "kind": kind,
        "sample": f"{reps} HTDemucs-spec STFT->iSTFT round trips of the same stereo {L}-sample input "
                  f"({el:.1f} s, single thread, double precision, "
                  + ("src/stft.h built from the reference sources" if kind == "reference"
                     else "C restatement of src/stft.h") + ")",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus N > 1 is not supported "
              "(no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import stx
    import synth

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    fft = stx.FFT(C1_NFFT)
    C, L = 2, C1_LEN
    T = stx.htdemucs_frames(C1_NFFT, L)
    F = C1_NFFT // 2
    x_host = synth.normal(2024, (C, L), 0.1)
    x0 = torch.from_numpy(x_host).to(dev)
    per_copy = (C * L * 4) * 2 + C * F * T * 8
    copies = max(2, int(np.ceil(512e6 / per_copy)) + 1)
    xs = [x0.clone() for _ in range(copies)]
    specs = [torch.empty((C, F, T), dtype=torch.complex64, device=dev) for _ in range(copies)]
    ys = [torch.empty((C, L), dtype=torch.float32, device=dev) for _ in range(copies)]

    def step(i, ev=None):
        k = i % copies
        if ev is not None:
            ev[0].record(stream)
        stx.htdemucs_spec(fft, xs[k], out=specs[k], stream=stream)
        if ev is not None:
            ev[1].record(stream)
        stx.htdemucs_ispec(fft, specs[k], L, out=ys[k], stream=stream)
        if ev is not None:
            ev[2].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # Timed region 1: the steps alone.
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(args.steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps

    # Timed region 2: the same steps with HIP events around each kernel.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    stft_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    istft_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))

    samples = C * L
    alg_bytes = samples * 4 + C * F * T * 8           # 13,761,888 B, same for both kernels
    kernels = {"stft_kernel<4096,1>": stft_ms, "istft_kernel<4096,1,16>": istft_ms}
    dom = max(kernels, key=kernels.get)
    achieved = alg_bytes / (kernels[dom] * 1e-3) / 1e9
    traffic = traffic_for(dom)

    # Parity of the measured output against the oracle (one channel), reported alongside.
    out = {
        "metric": METRIC,
        "value": round(samples / (ms_per_step * 1e-3) / 1e6, 3),
        "unit": "Msamples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "htdemucs_spec_ispec_round_trip",
            "channels": C,
            "samples_per_channel": L,
            "n_fft": C1_NFFT,
            "hop": C1_NFFT // 4,
            "frames": T,
            "bins": F,
            "layout": "f_major",
            "input": "N(0, 0.1^2) fp32 from seed 2024",
            "input_copies_rotated": copies,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": alg_bytes,
            "avg_us": round(kernels[dom] * 1e3, 3),
        },
        "kernels_us": {k: round(v * 1e3, 3) for k, v in kernels.items()},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(x_host, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
