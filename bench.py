"""Benchmark of the spectral + elementwise hot path on one MI355X. Prints ONE JSON line.

Headline workload (one "step"): the HTDemucs elementwise/reduction op set on fp32 inputs drawn
N(0, 1) from a seed, for each (C, T) in (48, 85995), (96, 21499), (192, 5375), (384, 1344):
  1. GroupNorm(num_groups=1) over [1, C, T], * w[C] + b[C], then GELU (erf), one call:
     stx_group_norm (src/htdemucs.cpp:114-128,136);
  2. GLU over 2C channels of a [1, 2C, T] input, then LayerScale broadcast MUL plus residual
     ADD, x + glu(h) * scale[C], one call: stx_glu_mul_add (src/htdemucs.cpp:105-110,137-139).
The 8 calls (8 kernels) of a step are captured once into a HIP graph per buffer set and
replayed on one stream; buffer sets rotate so that more than 512 MB is touched between reuses,
larger than the 256 MB Infinity Cache: cold-cache numbers.

value = algorithmic bytes per step / step time, in GB/s (cold), with the algorithmic bytes of the
reference's decomposition of the op set (one unit per op, each reading its inputs and writing
its output once): GroupNorm+affine 8, GELU 8, GLU 12 and LayerScale MUL + residual ADD 12 bytes
per element of [C, T] (40 in all, plus the parameters). Fusion moves fewer bytes than that:
config.bytes_moved_per_step gives the minimum these kernels move (24 per element); moved_GBps is
that over the same step time (the bytes the kernels really move), warm the same step replayed on
one buffer set that stays in the Infinity Cache.
roofline: the op with the largest share of the step (GroupNorm+GELU): its algorithmic bytes
(8 per element) / its duration (gn_fused_kernel, one grid-synchronised pass, at C = 96, 192, 384;
gn_partial_kernel + gn_apply_kernel at C = 48), from a graph of instances
of that op on more than 512 MB of distinct buffers (cold, like the step) replayed between two
HIP events on the stream the kernels run on. traffic: HBM bytes of that op
per step measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter
on a plain copy of known size), read from profiles/pmc_traffic.json when present.
cpu_baseline: the C oracle (a double-precision restatement; ggml's CPU backend is not in the
reference tree) on whole steps of the same workload for a bounded time, on as many threads as
physical cores (ggml's default; capped by OMP_NUM_THREADS where the job sets it), with the
single-thread figure beside it.

The same line carries the spectral half of the metric, STFT+iSTFT Msamples/s:
  spectral.htdemucs_round_trip: stx_htdemucs_spec + stx_htdemucs_ispec (src/stft.h:76-140) on
    stereo 343,980 samples, n_fft 4096 (hop 1024), reference f-major layout; its CPU baseline is
    the reference's own src/stft.h compiled from the reference sources (oracle/_ref) or, where
    that is absent, the C oracle, single-threaded as the reference runs it, with a second figure
    spreading channel round trips over the physical cores;
  spectral.roformer_chunk: stx_torch_stft (n_fft 2048, hop 441) -> stx_band_scatter_apply with
    60 mel bands and uniform [-1, 1] masks (one stem) -> stx_torch_istft on one stereo chunk of
    352,800 samples (src/roformer.cpp:217-283).
rows: every other hot-path kernel at its config shape (c1 HTDemucs spec/ispec, c3 band gather /
scatter-apply / STFT / iSTFT, c4 RMSNorm, RoPE, softmax, bias+GELU, c5 demix chunk build and
overlap-add), each timed cold (a graph of calls on more than 512 MB of distinct buffers) against
its algorithmic bytes and against a plain device copy of the same bytes at the same size
(copy_us; frac_of_copy = copy_us / us), the practical ceiling for small, launch-bound sizes.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stems.cpp_amd"))

METRIC = "STFT+iSTFT Msamples/s; norm/softmax/elementwise HBM GB/s (% of 8 TB/s)"
HBM_PEAK_GBS = 8000.0
SHAPES = [(48, 85995), (96, 21499), (192, 5375), (384, 1344)]
EPS = 1e-5


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on each CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-spectral", action="store_true")
    p.add_argument("--no-rows", action="store_true", help="skip the per-kernel timings of the other configs")
    p.add_argument("--pmc-pass", action="store_true",
                   help="for rocprofv3 --pmc: run each timed op on two buffer sets eagerly, once, no timing")
    p.add_argument("--rows", default="", help="comma-separated prefixes of the rows to run (default: all)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="end with one 256 MiB device copy (the reference kernel for PMC byte counters)")
    return p.parse_args()


PMC_PASS = False            # --pmc-pass: every op once per buffer set, eagerly (no graphs, no timing)
ROW_PREFIXES = []           # --rows


def traffic_for(name):
    """HBM bytes per step of op `name` from the committed PMC measurement, or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get("ops", {}).get(name)
    return None if entry is None else entry.get("bytes_per_step")


def spin(torch, us=3000):
    """Occupies the stream for about `us` microseconds so that the host can enqueue ahead."""
    torch.cuda._sleep(int(us * 2400))


class OpSet:
    """Buffers and calls of the headline workload."""

    def __init__(self, torch, stx, dev, copies):
        g = torch.Generator(device=dev)
        g.manual_seed(2025)
        rn = lambda *s: torch.randn(s, generator=g, device=dev, dtype=torch.float32)
        self.torch = torch
        self.stx = stx
        self.params = []
        for C, T in SHAPES:
            w, b, s = rn(C, 1, 1), rn(C, 1, 1), rn(C, 1, 1) * 0.1
            ws = stx.workspace(stx.group_norm_workspace_size(torch.empty((C, 1, T), device=dev), 1), dev)
            self.params.append((w, b, s, ws))
        self.sets = []
        for _ in range(copies):
            bufs = []
            for C, T in SHAPES:
                bufs.append({"x": rn(C, 1, T), "y": torch.empty((C, 1, T), device=dev), "h": rn(2 * C, 1, T),
                             "r": rn(C, 1, T), "o": torch.empty((C, 1, T), device=dev)})
            self.sets.append(bufs)

    def gn(self, k, i, stream=None):
        w, b, _, ws = self.params[i]
        B = self.sets[k][i]
        self.stx.group_norm(B["x"], 1, EPS, w, b, gelu=True, out=B["y"], workspace=ws, stream=stream)

    def glu_scale_residual(self, k, i, stream=None):
        B = self.sets[k][i]
        self.stx.glu_mul_add(B["r"], B["h"], 2, self.params[i][2], out=B["o"], stream=stream)

    def instance(self, name, i):
        """A call of op `name` at shape i on freshly allocated buffers of its own."""
        torch, stx = self.torch, self.stx
        C, T = SHAPES[i]
        w, b, s, ws = self.params[i]
        dev = w.device
        if name == "gn":
            x, y = torch.randn((C, 1, T), device=dev), torch.empty((C, 1, T), device=dev)
            return lambda st: stx.group_norm(x, 1, EPS, w, b, gelu=True, out=y, workspace=ws, stream=st)
        h, r, o = torch.randn((2 * C, 1, T), device=dev), torch.randn((C, 1, T), device=dev), torch.empty((C, 1, T), device=dev)
        return lambda st: stx.glu_mul_add(r, h, 2, s, out=o, stream=st)

    def step(self, k, stream=None):
        for i in range(len(SHAPES)):
            self.gn(k, i, stream)
            self.glu_scale_residual(k, i, stream)


def op_bytes():
    """Algorithmic bytes per op and shape, in the reference's decomposition: GroupNorm+affine
    and GELU 8 each, GLU 12, LayerScale + residual 12 per element (+ parameters)."""
    per = {"gn": [], "glu_scale_residual": []}
    for C, T in SHAPES:
        per["gn"].append(16 * C * T + 8 * C)
        per["glu_scale_residual"].append(24 * C * T + 4 * C)
    return per


def moved_bytes():
    """Minimum bytes the fused kernels move per op and shape: GroupNorm+GELU reads x and writes
    y (8 per element), GLU + LayerScale + residual reads 2C rows and x and writes (16)."""
    return {"gn": [8 * C * T for C, T in SHAPES], "glu_scale_residual": [16 * C * T for C, T in SHAPES]}


def run_ops(args, torch, stx, dev):
    elems = sum(C * T for C, T in SHAPES)
    per_set = 20 * elems
    copies = 2 if PMC_PASS else max(2, int(512e6 // per_set) + 1)
    ops = OpSet(torch, stx, dev, copies)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    if PMC_PASS:
        with torch.cuda.stream(stream):
            for k in range(copies):
                ops.step(k, stream)
        torch.cuda.synchronize()
        return None, ops

    # One graph per buffer set: the 8 calls (8 kernels) of a step.
    graphs = []
    with torch.cuda.stream(stream):
        for k in range(copies):
            ops.step(k, stream)                        # eager run before capture
        torch.cuda.synchronize()
        for k in range(copies):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                ops.step(k, stream)
            graphs.append(gr)
    torch.cuda.synchronize()

    for i in range(args.warmup):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    t0.record(cur)
    for i in range(args.steps):
        graphs[i % copies].replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    # Warm: the same step replayed on one buffer set (its 155 MB stay in the Infinity Cache).
    t0.record(cur)
    for i in range(args.steps):
        graphs[0].replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ms_per_step_warm = t0.elapsed_time(t1) / args.steps

    # Per-op durations, cold like the step: per (op, shape), one graph of instances on their
    # own buffers, more than 512 MB of them, replayed between two HIP events on the stream the
    # kernels run on (no launch gaps between kernels, graph launch cost amortised).
    REPLAYS = 3
    names = ["gn", "glu_scale_residual"]
    nbytes = moved_bytes()
    us = {}
    with torch.cuda.stream(stream):
        for name in names:
            for i in range(len(SHAPES)):
                n_inst = int(512e6 // nbytes[name][i]) + 2
                calls = [ops.instance(name, i) for _ in range(n_inst)]
                for c in calls:
                    c(stream)
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, stream=stream):
                    for c in calls:
                        c(stream)
                gr.replay()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(REPLAYS):
                    gr.replay()
                e1.record(stream)
                e1.synchronize()
                us[(name, i)] = e0.elapsed_time(e1) * 1e3 / (REPLAYS * n_inst)
                del gr, calls
    torch.cuda.synchronize()
    ops_us = {f"{n}[C={SHAPES[i][0]},T={SHAPES[i][1]}]": round(us[(n, i)], 3) for n in names for i in range(len(SHAPES))}
    share = {n: sum(us[(n, i)] for i in range(len(SHAPES))) for n in names}
    dom = max(share, key=share.get)
    # The roofline credits the dominant op with the bytes it must move itself (its fused
    # minimum), not with the reference decomposition's bytes.
    dom_bytes = sum(nbytes[dom])
    achieved = dom_bytes / (share[dom] * 1e-6) / 1e9
    step_bytes = sum(sum(v) for v in op_bytes().values())
    kernel_names = {"gn": "group_norm+affine+gelu (gn_fused_kernel<channel,gelu,width>, one grid-synchronised pass "
                          "at each of the four shapes)",
                    "glu_scale_residual": "glu + layer scale + residual (ew_flat_kernel<GLU_MUL_ADD>)"}
    moved = sum(sum(v) for v in moved_bytes().values())
    res = {
        "value": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "ms_per_step": round(ms_per_step, 6),
        "moved_GBps": round(moved / (ms_per_step * 1e-3) / 1e9, 1),
        "moved_frac_of_peak": round(moved / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "warm": {"ms_per_step": round(ms_per_step_warm, 6),
                 "value": round(step_bytes / (ms_per_step_warm * 1e-3) / 1e9, 1),
                 "moved_GBps": round(moved / (ms_per_step_warm * 1e-3) / 1e9, 1)},
        "config": {
            "workload": "htdemucs_op_set: GroupNorm(1)+affine then GELU on [1,C,T]; GLU 2C->C then LayerScale MUL + residual ADD",
            "shapes_CT": [list(s) for s in SHAPES],
            "bytes_per_step": step_bytes,
            "bytes_moved_per_step": sum(sum(v) for v in moved_bytes().values()),
            "execution": "one HIP graph per step (8 kernels), one stream",
            "buffer_sets_rotated": copies,
            "input": "N(0,1) fp32 from seed 2025",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_names[dom],
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_for(dom),
            "algorithmic_bytes_per_step": dom_bytes,
            "us_per_step": round(share[dom], 3),
        },
        "ops_us": ops_us,
        "ops_share_us": {k: round(v, 3) for k, v in share.items()},
    }
    return res, ops


def physical_cores():
    """Physical cores as the reference counts them (src/backend_loader.cpp:57-95, Linux branch):
    one per distinct thread_siblings_list over the logical CPUs, else the logical count."""
    logical = os.cpu_count() or 1
    cores = set()
    for i in range(logical):
        try:
            with open(f"/sys/devices/system/cpu/cpu{i}/topology/thread_siblings_list") as f:
                cores.add(f.readline().strip())
        except OSError:
            pass
    return len(cores) if cores else logical


def host_cpu():
    """The CPU baseline's host: model name, physical cores, logical CPUs, the CPUs this process
    may run on and the job's thread cap (OMP_NUM_THREADS)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    return {"cpu_model": model, "physical_cores": physical_cores(), "logical_cpus": os.cpu_count() or 1,
            "affinity_cpus": affinity, "thread_cap": int(omp) if omp and omp.isdigit() else None}


def cpu_threads():
    """Threads for the multi-core CPU figures: the physical cores (ggml's default thread count in
    the reference), capped by the CPUs this process may use and the job's OMP_NUM_THREADS."""
    h = host_cpu()
    n = min(h["physical_cores"], h["affinity_cpus"])
    if h["thread_cap"]:
        n = min(n, h["thread_cap"])
    return max(1, n)


def timed_threads(n, unit, budget_s):
    """Runs unit() repeatedly on n threads for about budget_s seconds; (units done, seconds). The
    oracle is called through ctypes, which releases the GIL, so the threads run in parallel."""
    import threading
    counts = [0] * n
    deadline = time.perf_counter() + budget_s

    def work(i):
        while True:
            unit()
            counts[i] += 1
            if time.perf_counter() >= deadline:
                break
    t0 = time.perf_counter()
    th = [threading.Thread(target=work, args=(i,)) for i in range(n)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    return sum(counts), time.perf_counter() - t0


def cpu_ops_baseline(budget_s):
    """The C oracle (a double-precision restatement; ggml's CPU backend is absent) on whole steps
    of the op set: one step per thread at a time, on as many threads as physical cores (ggml's
    default thread count), and on one thread."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    import synth
    o = oracle_lib.ops()
    data = []
    for C, T in SHAPES:
        data.append((synth.normal(C, (C, 1, T), 1.0), synth.normal(C + 1, (C, 1, 1), 1.0),
                     synth.normal(C + 2, (C, 1, 1), 1.0), synth.normal(C + 3, (2 * C, 1, T), 1.0),
                     synth.normal(C + 4, (C, 1, T), 1.0), synth.normal(C + 5, (C, 1, 1), 0.1)))

    def step():
        for x, w, b, h, r, s in data:
            o.group_norm(x, 1, EPS, w, b, gelu=True)
            g = o.glu(h, 2)
            o.binary("mul_add", r, g, s)
    step_bytes = sum(sum(v) for v in op_bytes().values())
    n = cpu_threads()
    steps, el = timed_threads(n, step, budget_s / 2)
    steps1, el1 = timed_threads(1, step, budget_s / 2)
    return {
        "value": round(steps * step_bytes / el / 1e9, 3),
        "unit": "GB/s",
        "cores": n,
        "kind": "port",
        "sample": f"{steps} whole steps of the same op set in {el:.1f} s on {n} threads (one step per thread at a "
                  "time): the C oracle, a double-precision restatement of the ops (ggml's CPU backend is absent "
                  "from the reference)",
        "single_thread": {"value": round(steps1 * step_bytes / el1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                          "sample": f"{steps1} steps in {el1:.1f} s"},
        "host": host_cpu(),
    }


def run_spectral(args, torch, stx, dev):
    import numpy as np
    import synth
    out = {}
    steps = max(20, args.steps)
    # HTDemucs spec round trip, reference layout.
    n_fft, L, C = 4096, 343980, 2
    fft = stx.FFT(n_fft)
    T = stx.htdemucs_frames(n_fft, L)
    F = n_fft // 2
    x_host = synth.normal(2024, (C, L), 0.1)
    per = C * L * 4 * 2 + C * F * T * 8
    copies = max(2, int(512e6 // per) + 1)
    xs = [torch.from_numpy(x_host).to(dev) for _ in range(copies)]
    specs = [torch.empty((C, F, T), dtype=torch.complex64, device=dev) for _ in range(copies)]
    ys = [torch.empty((C, L), device=dev) for _ in range(copies)]
    stream = torch.cuda.Stream()

    def rt(k):
        stx.htdemucs_spec(fft, xs[k], out=specs[k], stream=stream)
        stx.htdemucs_ispec(fft, specs[k], L, out=ys[k], stream=stream)
    out["htdemucs_round_trip"] = time_graphs(torch, stream, rt, copies, steps, C * L, args.warmup)
    out["htdemucs_round_trip"]["config"] = {"channels": C, "samples": L, "n_fft": n_fft, "hop": n_fft // 4,
                                            "frames": T, "layout": "f_major", "buffer_sets_rotated": copies}
    # Per-kernel durations behind a spin kernel.
    evs = []
    with torch.cuda.stream(stream):
        for r in range(20):
            spin(torch, 500)
            k = r % copies
            e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
            e[0].record(stream)
            stx.htdemucs_spec(fft, xs[k], out=specs[k], stream=stream)
            e[1].record(stream)
            stx.htdemucs_ispec(fft, specs[k], L, out=ys[k], stream=stream)
            e[2].record(stream)
            evs.append(e)
    torch.cuda.synchronize()
    alg = C * L * 4 + C * F * T * 8
    for name, a, b in (("stft", 0, 1), ("istft", 1, 2)):
        t = float(np.median([e[a].elapsed_time(e[b]) * 1e3 for e in evs]))
        out["htdemucs_round_trip"][f"{name}_us"] = round(t, 3)
        out["htdemucs_round_trip"][f"{name}_GBps"] = round(alg / (t * 1e-6) / 1e9, 1)
    del xs, specs, ys
    # The same round trip through the drop-in C++ shim (include/stx_st.hpp) on host buffers, as
    # src/htdemucs.cpp:428,470 call src/stft.h: one st::FFT reused, per channel htdemucs_spec then
    # htdemucs_ispec; includes the PCIe copies and the complex<double> <-> complex64 conversion.
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    try:
        import shim_lib
        sec = shim_lib.lib().shim_time_htdemucs_round_trip(n_fft, x_host.ctypes.data_as(ctypes.c_void_p), C, L, 10)
        if sec > 0:
            out["htdemucs_round_trip_st_shim"] = {
                "metric": "Msamples/s", "value": round(C * L / sec / 1e6, 3), "ms_per_step": round(sec * 1e3, 6),
                "note": "stx_st.hpp on host vectors: st::htdemucs_spec + st::htdemucs_ispec per channel, one FFT "
                        "object reused, PCIe copies and complex<double> conversion included"}
    except OSError as e:
        out["htdemucs_round_trip_st_shim"] = {"skipped": str(e)}

    # RoFormer chunk: STFT -> mask scatter-average + apply -> iSTFT.
    n_fft, hop, L, C, S = 2048, 441, 352800, 2, 1
    fft2 = stx.FFT(n_fft)
    sizes, freqs = stx.mel_band_map(44100, n_fft, 60)
    bands = stx.Bands(sizes, freqs, n_fft // 2 + 1, C)
    T = stx.torch_stft_frames(L, hop)
    F = n_fft // 2 + 1
    per = C * L * 8 + C * F * T * 16 + S * bands.total_feat * T * 4
    copies = max(2, int(512e6 // per) + 1)
    x_host = synth.normal(2026, (C, L), 0.1)
    xs = [torch.from_numpy(x_host).to(dev) for _ in range(copies)]
    ms = [torch.from_numpy(synth.uniform(7 + k, (1, S, bands.total_feat * T))).to(dev) for k in range(copies)]
    specs = [torch.empty((C, T, F), dtype=torch.complex64, device=dev) for _ in range(copies)]
    masked = [torch.empty((1, S, C, T, F), dtype=torch.complex64, device=dev) for _ in range(copies)]
    ys = [torch.empty((S * C, hop * (T - 1)), device=dev) for _ in range(copies)]

    def chunk(k):
        stx.torch_stft(fft2, xs[k], hop, layout=stx.T_MAJOR, out=specs[k], stream=stream)
        bands.scatter_apply(ms[k], specs[k].view(1, C, T, F), T, layout=stx.T_MAJOR, out=masked[k], stream=stream)
        stx.torch_istft(fft2, masked[k].view(S * C, T, F), hop, layout=stx.T_MAJOR, out=ys[k], stream=stream)
    out["roformer_chunk"] = time_graphs(torch, stream, chunk, copies, steps, C * L, args.warmup)
    out["roformer_chunk"]["config"] = {"channels": C, "samples": L, "n_fft": n_fft, "hop": hop, "frames": T,
                                       "bins": F, "bands": 60, "stems": S, "layout": "t_major",
                                       "buffer_sets_rotated": copies}
    return out


def time_graphs(torch, stream, fn, copies, steps, samples, warmup):
    graphs = []
    with torch.cuda.stream(stream):
        for k in range(copies):
            fn(k)
        torch.cuda.synchronize()
        for k in range(copies):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=stream):
                fn(k)
            graphs.append(gr)
    for i in range(warmup):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    t0.record(cur)
    for i in range(steps):
        graphs[i % copies].replay()
    t1.record(cur)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    t0.record(cur)
    for i in range(steps):
        graphs[0].replay()                             # warm: one buffer set, kept in the Infinity Cache
    t1.record(cur)
    torch.cuda.synchronize()
    warm = t0.elapsed_time(t1) / steps
    return {"metric": "Msamples/s", "value": round(samples / (ms * 1e-3) / 1e6, 3), "ms_per_step": round(ms, 6),
            "steps": steps, "warm_value": round(samples / (warm * 1e-3) / 1e6, 3),
            "warm_ms_per_step": round(warm, 6)}


def time_call(torch, stream, make, nbytes, replays=3):
    """Cold timing of one op: a graph of calls on distinct buffers (more than 512 MB of them in
    total) replayed `replays` times between two HIP events; microseconds per call."""
    if PMC_PASS:
        calls = [make() for _ in range(2)]
        with torch.cuda.stream(stream):
            for c in calls:
                c()
        torch.cuda.synchronize()
        del calls
        torch.cuda.empty_cache()
        return {"us": 0.0, "algorithmic_bytes": int(nbytes)}
    n_inst = max(1, int(512e6 // max(nbytes, 1)) + 1) if nbytes < 512e6 else 1
    calls = [make() for _ in range(n_inst)]
    with torch.cuda.stream(stream):
        for c in calls:
            c()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=stream):
            for c in calls:
                c()
        gr.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            gr.replay()
        e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * n_inst)
    del gr
    # Warm: one instance's buffers, which stay in the 256 MB Infinity Cache when they fit,
    # captured WARM_REPS times into one graph and replayed.
    WARM_REPS = 20
    with torch.cuda.stream(stream):
        gw = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gw, stream=stream):
            for _ in range(WARM_REPS):
                calls[0]()
        gw.replay()
        e0.record(stream)
        for _ in range(replays):
            gw.replay()
        e1.record(stream)
    e1.synchronize()
    warm = e0.elapsed_time(e1) * 1e3 / (replays * WARM_REPS)
    del gw, calls
    torch.cuda.empty_cache()
    return {"us": round(us, 3), "algorithmic_bytes": int(nbytes), "GBps": round(nbytes / us / 1e3, 1),
            "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "warm_us": round(warm, 3)}


def row(out, name, torch, stream, make, nbytes):
    """Times one row (time_call) unless --rows excludes it."""
    if ROW_PREFIXES and not any(name.startswith(p) for p in ROW_PREFIXES):
        return
    out[name] = time_call(torch, stream, make, nbytes)


def run_rows(torch, stx, dev):
    """Every other hot-path kernel at its config shape, cold, against its algorithmic bytes and
    against a plain device copy of the same bytes (copy_us, frac_of_copy = copy_us / us)."""
    import synth
    stream = torch.cuda.Stream()
    rn = lambda *shape: torch.randn(shape, device=dev)
    out = {}
    # c3: RoFormer chunk spectral path (stereo 352,800, n_fft 2048, hop 441; 60 mel bands).
    n_fft, hop, L, C = 2048, 441, 352800, 2
    fft = stx.FFT(n_fft)
    sizes, freqs = stx.mel_band_map(44100, n_fft, 60)
    bands = stx.Bands(sizes, freqs, n_fft // 2 + 1, C)
    T, F = stx.torch_stft_frames(L, hop), n_fft // 2 + 1
    feat = bands.total_feat * T

    def mk_stft():
        x, y = rn(C, L), torch.empty((C, T, F), dtype=torch.complex64, device=dev)
        return lambda: stx.torch_stft(fft, x, hop, layout=stx.T_MAJOR, out=y, stream=stream)
    row(out, "c3_stft_t_major", torch, stream, mk_stft, C * L * 4 + C * T * F * 8)

    def mk_stft_f():
        x, y = rn(C, L), torch.empty((C, F, T), dtype=torch.complex64, device=dev)
        return lambda: stx.torch_stft(fft, x, hop, layout=stx.F_MAJOR, out=y, stream=stream)
    row(out, "c3_stft_f_major", torch, stream, mk_stft_f, C * L * 4 + C * T * F * 8)

    def mk_gather():
        z, f = torch.randn((1, C, T, F), dtype=torch.complex64, device=dev), torch.empty((1, feat), device=dev)
        return lambda: bands.gather(z, T, layout=stx.T_MAJOR, out=f, stream=stream)
    row(out, "c3_band_gather", torch, stream, mk_gather, C * T * F * 8 + feat * 4)

    def mk_scatter():
        m = torch.from_numpy(synth.uniform(3, (1, 1, feat))).to(dev)
        z = torch.randn((1, C, T, F), dtype=torch.complex64, device=dev)
        o = torch.empty((1, 1, C, T, F), dtype=torch.complex64, device=dev)
        return lambda: bands.scatter_apply(m, z, T, layout=stx.T_MAJOR, out=o, stream=stream)
    row(out, "c3_scatter_apply", torch, stream, mk_scatter, feat * 4 + 2 * C * T * F * 8)

    # The band split's RMSNorm of all 60 bands, and the mask heads' GLU for 4 stems, one launch each.
    gammas = [rn(int(s) * C * 2) for s in sizes]

    def mk_band_norm():
        f, o = rn(1, feat), torch.empty((1, feat), device=dev)
        return lambda: bands.rms_norm(f, T, gammas, 1e-24, out=o, stream=stream)
    row(out, "c3_band_rms_norm", torch, stream, mk_band_norm, 2 * feat * 4 + bands.total_feat * 4)

    def mk_mask_glu():
        heads = [rn(T, 2 * int(s) * C * 2) for _ in range(4) for s in sizes]
        m = torch.empty((4, feat), device=dev)
        return lambda: bands.mask_glu(heads, 4, T, out=m, stream=stream)
    row(out, "c3_band_mask_glu", torch, stream, mk_mask_glu, 4 * 3 * feat * 4)

    def mk_istft():
        z, y = torch.randn((C, T, F), dtype=torch.complex64, device=dev), torch.empty((C, hop * (T - 1)), device=dev)
        return lambda: stx.torch_istft(fft, z, hop, layout=stx.T_MAJOR, out=y, stream=stream)
    row(out, "c3_istft_t_major", torch, stream, mk_istft, C * L * 4 + C * T * F * 8)

    def mk_istft_f():
        z, y = torch.randn((C, F, T), dtype=torch.complex64, device=dev), torch.empty((C, hop * (T - 1)), device=dev)
        return lambda: stx.torch_istft(fft, z, hop, layout=stx.F_MAJOR, out=y, stream=stream)
    row(out, "c3_istft_f_major", torch, stream, mk_istft_f, C * L * 4 + C * T * F * 8)

    def mk_istft_ws():
        z, y = torch.randn((C, T, F), dtype=torch.complex64, device=dev), torch.empty((C, hop * (T - 1)), device=dev)
        ws = stx.workspace(stx.istft_workspace_size(fft, C, T), dev)
        return lambda: stx.torch_istft(fft, z, hop, layout=stx.T_MAJOR, out=y, stream=stream, workspace=ws)
    row(out, "c3_istft_t_major_ws", torch, stream, mk_istft_ws, C * L * 4 + C * T * F * 8)

    # Launch-amortised: one call over the 180 s song's 96 chunks x 2 channels at the c3 geometry
    # (192 channels of 352,800 samples, T-major, the device pipeline's layout): the kernels'
    # throughput once launch and ramp costs vanish.
    CB = 96 * C

    def mk_stft_b():
        x, y = rn(CB, L), torch.empty((CB, T, F), dtype=torch.complex64, device=dev)
        return lambda: stx.torch_stft(fft, x, hop, layout=stx.T_MAJOR, out=y, stream=stream)
    row(out, "c5_stft_batched", torch, stream, mk_stft_b, CB * L * 4 + CB * T * F * 8)

    def mk_istft_b(with_ws):
        def mk():
            z = torch.randn((CB, T, F), dtype=torch.complex64, device=dev)
            y = torch.empty((CB, hop * (T - 1)), device=dev)
            ws = stx.workspace(stx.istft_workspace_size(fft, CB, T), dev) if with_ws else None
            return lambda: stx.torch_istft(fft, z, hop, layout=stx.T_MAJOR, out=y, stream=stream, workspace=ws)
        return mk
    row(out, "c5_istft_batched", torch, stream, mk_istft_b(False), CB * L * 4 + CB * T * F * 8)
    del bands, fft

    # c1: HTDemucs spectrogram of one stereo segment (343,980 samples, n_fft 4096, hop 1024).
    n1, L1 = 4096, 343980
    fft1 = stx.FFT(n1)
    T1, F1 = stx.htdemucs_frames(n1, L1), n1 // 2
    c1_bytes = C * L1 * 4 + C * T1 * F1 * 8

    def mk_spec1():
        x, y = rn(C, L1), torch.empty((C, F1, T1), dtype=torch.complex64, device=dev)
        return lambda: stx.htdemucs_spec(fft1, x, out=y, stream=stream)
    row(out, "c1_htdemucs_spec", torch, stream, mk_spec1, c1_bytes)

    def mk_spec1_t():
        x, y = rn(C, L1), torch.empty((C, T1, F1), dtype=torch.complex64, device=dev)
        return lambda: stx.htdemucs_spec(fft1, x, layout=stx.T_MAJOR, out=y, stream=stream)
    row(out, "c1_htdemucs_spec_t_major", torch, stream, mk_spec1_t, c1_bytes)

    def mk_ispec1(with_ws):
        def mk():
            z, y = torch.randn((C, F1, T1), dtype=torch.complex64, device=dev), torch.empty((C, L1), device=dev)
            ws = stx.workspace(stx.istft_workspace_size(fft1, C, T1), dev) if with_ws else None
            return lambda: stx.htdemucs_ispec(fft1, z, L1, out=y, stream=stream, workspace=ws)
        return mk
    row(out, "c1_htdemucs_ispec", torch, stream, mk_ispec1(False), c1_bytes)
    row(out, "c1_htdemucs_ispec_ws", torch, stream, mk_ispec1(True), c1_bytes)

    def mk_ispec1_t():
        z, y = torch.randn((C, T1, F1), dtype=torch.complex64, device=dev), torch.empty((C, L1), device=dev)
        return lambda: stx.htdemucs_ispec(fft1, z, L1, layout=stx.T_MAJOR, out=y, stream=stream)
    row(out, "c1_htdemucs_ispec_t_major", torch, stream, mk_ispec1_t, c1_bytes)
    del fft1

    # c1 pre/post-processing around the HTDemucs graph (4 sources): CaC pack + normalise of the
    # spectrum, the waveform's normalise, the spectral denormalise and the time branch + add.
    spec_bytes = C * F1 * T1 * 8

    def mk_cac():
        z, m = torch.randn((C, F1, T1), dtype=torch.complex64, device=dev), torch.empty((2 * C, F1, T1), device=dev)
        st = torch.empty(2, dtype=torch.float64, device=dev)
        return lambda: stx.htdemucs_cac_normalize(z, out=m, stats=st, stream=stream)
    row(out, "c1_cac_normalize", torch, stream, mk_cac, 2 * spec_bytes)

    def mk_wave():
        x, y = rn(C, L1), torch.empty((C, L1), device=dev)
        st = torch.empty(2, dtype=torch.float64, device=dev)
        return lambda: stx.htdemucs_wave_normalize(x, out=y, stats=st, stream=stream)
    row(out, "c1_wave_normalize", torch, stream, mk_wave, 2 * C * L1 * 4)

    def mk_denorm():
        ox, z = rn(4, 2 * C, F1, T1), torch.empty((4, C, F1, T1), dtype=torch.complex64, device=dev)
        st = torch.tensor([0.01, 0.5], dtype=torch.float64, device=dev)
        return lambda: stx.htdemucs_cac_denormalize(ox, st, out=z, stream=stream)
    row(out, "c1_cac_denormalize", torch, stream, mk_denorm, 2 * 4 * spec_bytes)

    def mk_tadd():
        xt, y, o = rn(4 * C, L1), rn(4 * C, L1), torch.empty((4 * C, L1), device=dev)
        st = torch.tensor([0.01, 0.5], dtype=torch.float64, device=dev)
        return lambda: stx.htdemucs_time_add(xt, y, st, out=o, stream=stream)
    row(out, "c1_time_add", torch, stream, mk_tadd, 3 * 4 * C * L1 * 4)


    # Kim_Vocal_2's transform (n_fft 7680, not a power of two; hop 1024) on one TFC-TDF chunk of
    # 1024 x 255 = 261,120 stereo samples -> [2][3841][256]: the mixed-radix STFT and iSTFT.
    fk, Lk, Tk, Fk = stx.FFT(7680, any_size=True), 261120, 256, 3841
    kim_bytes = C * Lk * 4 + C * Tk * Fk * 8

    def mk_kim_stft():
        x, y = rn(C, Lk), torch.empty((C, Fk, Tk), dtype=torch.complex64, device=dev)
        return lambda: stx.torch_stft(fk, x, 1024, out=y, stream=stream)
    row(out, "kim_stft_7680", torch, stream, mk_kim_stft, kim_bytes)

    def mk_kim_istft():
        z, y = torch.randn((C, Fk, Tk), dtype=torch.complex64, device=dev), torch.empty((C, 1024 * 255), device=dev)
        ws = stx.workspace(stx.istft_workspace_size(fk, C, Tk), dev)
        return lambda: stx.torch_istft(fk, z, 1024, out=y, stream=stream, workspace=ws)
    row(out, "kim_istft_7680", torch, stream, mk_kim_istft, kim_bytes)
    del fk

    # c4: RoFormer transformer ops (dim 384, 8 heads x 64, 60 bands x 801 frames).
    def mk_rms():
        x, g, y = rn(48060, 384), rn(384), torch.empty((48060, 384), device=dev)
        return lambda: stx.rms_norm(x, 1e-24, gamma=g, out=y, stream=stream)
    row(out, "c4_rms_norm_mul", torch, stream, mk_rms, 2 * 48060 * 384 * 4 + 384 * 4)
    for name, shape, n in (("c4_rope_time", (60, 801, 8, 64), 801), ("c4_rope_band", (801, 60, 8, 64), 60)):
        def mk_rope(shape=shape, n=n):
            x, y = rn(*shape), torch.empty(shape, device=dev)
            pos = torch.arange(n, dtype=torch.int32, device=dev)
            return lambda: stx.rope_ext(x, pos, 64, mode=0, freq_base=10000.0, out=y, stream=stream)
        row(out, name, torch, stream, mk_rope, 2 * 64 * 8 * 801 * 60 * 4 + n * 4)
    for name, shape in (("c4_softmax_time", (60, 8, 801, 801)), ("c4_softmax_band", (801, 8, 60, 60))):
        def mk_sm(shape=shape):
            x, y = rn(*shape), torch.empty(shape, device=dev)
            return lambda: stx.soft_max_ext(x, 0.125, out=y, stream=stream)
        n = 1
        for d in shape:
            n *= d
        row(out, name, torch, stream, mk_sm, 8 * n)
    # HTDemucs cross-transformer scores, frequency self-attention: kq [Nk = 2688, Nq = 2688, 8 heads],
    # scale 1/sqrt(48) (src/htdemucs.cpp:236-238; rows longer than 2048 take one block each).
    def mk_sm_htd():
        x, y = rn(8, 2688, 2688), torch.empty((8, 2688, 2688), device=dev)
        return lambda: stx.soft_max_ext(x, 1.0 / 48 ** 0.5, out=y, stream=stream)
    row(out, "htd_softmax_freq", torch, stream, mk_sm_htd, 8 * 8 * 2688 * 2688)

    def mk_ff():
        h, bb, y = rn(60, 801, 1536), rn(1536), torch.empty((60, 801, 1536), device=dev)
        return lambda: stx.gelu_erf(h, bias=bb, out=y, stream=stream)
    row(out, "c4_gelu_ff_bias", torch, stream, mk_ff, 2 * 60 * 801 * 1536 * 4 + 1536 * 4)

    # c4 layout glue: the q/k/v split + RoPE + permutes of one attention layer (time axis: 60
    # sequences of 801 frames; band axis: 801 sequences of 60 bands), the head merge, the
    # [D, B, T] -> [D, T, B] transpose between the two transformers and the band-split concat.
    for name, (b, n) in (("c4_qkv_rope_split_time", (60, 801)), ("c4_qkv_rope_split_band", (801, 60))):
        def mk_split(b=b, n=n):
            qkv = rn(b, n, 1536)
            q, k = torch.empty((b, 8, n, 64), device=dev), torch.empty((b, 8, n, 64), device=dev)
            vt = torch.empty((b, 8, 64, n), device=dev)
            pos = torch.arange(n, dtype=torch.int32, device=dev)
            return lambda: stx.qkv_rope_split(qkv, pos, 8, 10000.0, out=(q, k, vt), stream=stream)
        row(out, name, torch, stream, mk_split, 2 * b * n * 1536 * 4 + n * 4)

    def mk_merge():
        o, y = rn(60, 8, 801, 64), torch.empty((60, 801, 8, 64), device=dev)
        return lambda: stx.merge_heads(o, out=y, stream=stream)
    row(out, "c4_merge_heads_time", torch, stream, mk_merge, 2 * 60 * 8 * 801 * 64 * 4)

    def mk_transpose():
        x, y = rn(801, 60, 384), torch.empty((60, 801, 384), device=dev)
        return lambda: stx.cont_permute(x, (0, 2, 1, 3), out=y, stream=stream)
    row(out, "c4_permute_dbt", torch, stream, mk_transpose, 2 * 60 * 801 * 384 * 4)

    def mk_concat():
        xs, y = [rn(801, 1, 384) for _ in range(60)], torch.empty((801, 60, 384), device=dev)
        return lambda: stx.concat(xs, 1, out=y, stream=stream)
    row(out, "c4_band_concat", torch, stream, mk_concat, 2 * 60 * 801 * 384 * 4)

    # c5: full-song demix (180 s stereo, chunk 352,800, step 88,200, 4 stems).
    Lsong, chunk, step, S = 7938000, 352800, 88200, 4
    plan = stx.Demix(Lsong, C, chunk, step)
    _, table = stx.demix_plan(Lsong, chunk, step)
    lens = int(table["length"].astype("int64").sum())
    mix = torch.from_numpy(synth.sines_plus_pink(5, C, Lsong)).to(dev)

    def mk_chunks():
        m, parts = mix.clone(), torch.empty((plan.n_chunks, C, chunk), device=dev)
        return lambda: plan.chunks(m, out=parts, stream=stream)
    row(out, "c5_demix_chunks", torch, stream, mk_chunks, C * Lsong * 4 + plan.n_chunks * C * chunk * 4)

    def mk_ola():
        y, o = rn(plan.n_chunks, S, C, chunk), torch.empty((S, C, Lsong), device=dev)
        return lambda: plan.overlap_add(y, out=o, stream=stream)
    row(out, "c5_demix_overlap_add", torch, stream, mk_ola, lens * S * C * 4 + S * C * Lsong * 4)
    del plan

    # The song arriving at 48 kHz: resampled to the models' 44.1 kHz (src/audio.h:17-59).
    rsm = stx.Resampler(48000, 44100)
    n48 = 8640000

    def mk_resample():
        x, y = rn(C, n48), torch.empty((C, rsm.length(n48)), device=dev)
        return lambda: rsm(x, out=y, stream=stream)
    row(out, "c5_resample_48k", torch, stream, mk_resample, C * (n48 + rsm.length(n48)) * 4)
    # The per-tap kernel, bit-identical to the reference (chosen by the variable at each call,
    # so also when a graph is captured).
    prev = os.environ.get("STX_RESAMPLE_EXACT")
    os.environ["STX_RESAMPLE_EXACT"] = "1"
    try:
        row(out, "c5_resample_48k_exact", torch, stream, mk_resample, C * (n48 + rsm.length(n48)) * 4)
    finally:
        if prev is None:
            del os.environ["STX_RESAMPLE_EXACT"]
        else:
            os.environ["STX_RESAMPLE_EXACT"] = prev
    del rsm

    # The same song through the TFC-TDF UVR chunking (Kim_Vocal_2: n_fft 7680, chunk 261,120,
    # step 253,440, one stem): chunk inputs and the hanning-weighted overlap-add.
    uvr = stx.UvrDemix(Lsong, C, 261120, 7680)

    def mk_uvr_chunks():
        m, p = mix.clone(), torch.empty((uvr.n_chunks, C, 261120), device=dev)
        return lambda: uvr.chunks(m, out=p, stream=stream)
    row(out, "c5_uvr_chunks", torch, stream, mk_uvr_chunks, C * Lsong * 4 + uvr.n_chunks * C * 261120 * 4)

    def mk_uvr_ola():
        y, o = rn(uvr.n_chunks, 1, C, 261120), torch.empty((1, C, Lsong), device=dev)
        return lambda: uvr.overlap_add(y, out=o, stream=stream)
    uvr_read = sum(min(261120, uvr.padded_len - k * uvr.step) for k in range(uvr.n_chunks))
    row(out, "c5_uvr_overlap_add", torch, stream, mk_uvr_ola, (uvr_read + Lsong) * C * 4)
    del uvr

    # The same song through HTDemucs' apply_model split: mono-mix normalise, the 31 padded
    # segments of 343,980 samples (stride 257,985) and the triangular-weight overlap-add.
    seg = 343980
    stride, n_seg = stx.htdemucs_split_plan(Lsong, seg, 0.25)

    def mk_mixnorm():
        m, o = mix.clone(), torch.empty((C, Lsong), device=dev)
        st = torch.empty(2, dtype=torch.float64, device=dev)
        return lambda: stx.htdemucs_mix_normalize(m, out=o, stats=st, stream=stream)
    row(out, "c5_htdemucs_mix_normalize", torch, stream, mk_mixnorm, 2 * C * Lsong * 4)

    def mk_segments():
        m, p = mix.clone(), torch.empty((n_seg, C, seg), device=dev)
        return lambda: stx.htdemucs_segments(m, 0, Lsong, seg, stride, out=p, stream=stream)
    row(out, "c5_htdemucs_segments", torch, stream, mk_segments, C * Lsong * 4 + n_seg * C * seg * 4)

    def mk_split_ola():
        y, o = rn(n_seg, S * C, seg), torch.empty((S * C, Lsong), device=dev)
        return lambda: stx.htdemucs_split_overlap_add(y, Lsong, stride, out=o, stream=stream)
    last = Lsong - (n_seg - 1) * stride
    valid = (n_seg - 1) * seg + last
    row(out, "c5_htdemucs_split_ola", torch, stream, mk_split_ola, (valid + Lsong) * S * C * 4)
    torch.cuda.empty_cache()
    if PMC_PASS:
        return out
    # The practical ceiling at each row's size: a plain device copy (torch's copy_) moving the
    # same bytes (half read, half written), timed the same cold way.
    for name, r in out.items():
        n = max(1, r["algorithmic_bytes"] // 8)

        def mk_copy(n=n):
            x, y = torch.empty(n, device=dev), torch.empty(n, device=dev)
            return lambda: y.copy_(x)
        cp = time_call(torch, stream, mk_copy, 8 * n)
        r["copy_us"] = cp["us"]
        r["frac_of_copy"] = round(cp["us"] / r["us"], 3)
    return out


def cpu_spectral_baseline(budget_s):
    """The reference's own src/stft.h (oracle/_ref; the C restatement where that is absent) on the
    c1 round trip: single-threaded as the reference runs it, and with the channels' round trips
    spread over as many threads as physical cores."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    import synth
    kind = "reference" if oracle_lib.ref_available() else "port"
    lib = oracle_lib.reference() if kind == "reference" else oracle_lib.oracle()
    C, L, n_fft = 2, 343980, 4096
    x = synth.normal(2024, (C, L), 0.1)

    def channel_round_trip(c=0):
        s = lib.htdemucs_spec(x[c], n_fft)
        lib.htdemucs_ispec(s, n_fft, L)
    what = "src/stft.h compiled from the reference sources" if kind == "reference" else "C restatement of src/stft.h"
    reps1, el1 = timed_threads(1, channel_round_trip, budget_s / 2)
    n = cpu_threads()
    repsn, eln = timed_threads(n, channel_round_trip, budget_s / 2)
    return {"value": round(reps1 * L / el1 / 1e6, 3), "unit": "Msamples/s", "cores": 1, "kind": kind,
            "sample": f"{reps1} single-channel HTDemucs-spec STFT->iSTFT round trips of {L} samples ({el1:.1f} s, "
                      f"single thread, double precision, {what})",
            "multi_core": {"value": round(repsn * L / eln / 1e6, 3), "unit": "Msamples/s", "cores": n,
                           "sample": f"{repsn} channel round trips in {eln:.1f} s on {n} threads"},
            "host": host_cpu()}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build runs on one GPU; there is no multi-GPU path "
              "(the workload shards by independent channels/chunks, see the design notes)", file=sys.stderr)
        sys.exit(2)
    import torch

    import stx

    dev = torch.device("cuda:0")
    global PMC_PASS, ROW_PREFIXES
    PMC_PASS = args.pmc_pass
    ROW_PREFIXES = [p for p in args.rows.split(",") if p]
    if PMC_PASS:
        run_ops(args, torch, stx, dev)
        rows = run_rows(torch, stx, dev) if not args.no_rows else {}
        if args.copy_calibration:
            a = torch.empty(64 << 20, device=dev)
            b = torch.empty_like(a)
            b.copy_(a)
            torch.cuda.synchronize()
        print(json.dumps({"pmc_pass": True, "rows": sorted(rows)}), flush=True)
        return
    res, _ = run_ops(args, torch, stx, dev)
    out = {
        "metric": METRIC,
        "value": res["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": res["config"],
        "roofline": res["roofline"],
        "effective_frac_of_peak": round(res["value"] / HBM_PEAK_GBS, 4),
        "moved_GBps": res["moved_GBps"],
        "moved_frac_of_peak": res["moved_frac_of_peak"],
        "warm": res["warm"],
        "ops_us": res["ops_us"],
        "ops_share_us": res["ops_share_us"],
    }
    torch.cuda.empty_cache()
    if not args.no_spectral:
        out["spectral"] = run_spectral(args, torch, stx, dev)
    if not args.no_rows:
        out["rows"] = run_rows(torch, stx, dev)
    if args.copy_calibration:
        a = torch.empty(64 << 20, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_ops_baseline(args.cpu_seconds)
        if "spectral" in out:
            out["spectral"]["htdemucs_round_trip"]["cpu_baseline"] = cpu_spectral_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
