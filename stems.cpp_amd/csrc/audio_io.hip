// audio_io.hip — libstems' separate() data path (src/libstems.cpp:135-196) on the device, around
// a model's separate.
//
// The reference copies the request's audio into a planar host buffer (de-interleaving when
// asked, :160-167), maps it to the model's channel count (st::to_channels, src/audio.h:62-71),
// resamples it to the model's rate (st::resample_planar, :17-59), separates, and resamples the
// stems back, cutting or zero-padding each to the input's length (:186-196). Here the layout and
// the channel mapping are one gather kernel reading the caller's device buffer (skipped when the
// input already is planar at the model's channel count), the resampling is stx_resample (in
// groups of at most 8 planes, its per-launch limit), and the length pinning is a copy kernel,
// skipped when the back-resampled length already equals the input's (the resampler then writes
// into `out` itself). Everything is enqueued on the caller's stream.
#include <algorithm>
#include <climits>
#include <cmath>

#include "common.hpp"
#include "resample.hpp"

namespace stx {
namespace {

constexpr unsigned kIoThreads = 256;
constexpr long long kIoMaxBlocks = 4096;           // per plane: grid-stride beyond

// out[c][i] = input channel src(c) at sample i, src(c) = 0 for mono, else min(c, ch - 1)
// (src/audio.h:66); the input is read planar (in[src * n + i]) or interleaved (in[i * ch + src],
// src/libstems.cpp:165).
__global__ __launch_bounds__(kIoThreads) void to_channels_kernel(const float* __restrict__ in, long long n, int ch,
                                                                  int layout, float* __restrict__ out) {
    const int c = (int)blockIdx.y;
    const long long src = ch == 1 ? 0 : min(c, ch - 1);
    float* oc = out + (long long)c * n;
    for (long long i = (long long)blockIdx.x * kIoThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kIoThreads)
        oc[i] = layout == STX_AUDIO_PLANAR ? in[src * n + i] : in[i * ch + src];
}

// out[p][i] = i < back ? e[p][i] : 0 for i < n: each plane of back samples cut or zero-padded to
// n (src/libstems.cpp:188-193).
__global__ __launch_bounds__(kIoThreads) void pin_length_kernel(const float* __restrict__ e, long long back,
                                                                 float* __restrict__ out, long long n) {
    const long long p = blockIdx.y;
    const float* ep = e + p * back;
    float* op = out + p * n;
    for (long long i = (long long)blockIdx.x * kIoThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kIoThreads)
        op[i] = i < back ? ep[i] : 0.f;
}

unsigned io_blocks(long long n) { return (unsigned)std::min<long long>((n + kIoThreads - 1) / kIoThreads, kIoMaxBlocks); }

// llround(n * dst / src) as st::resample_planar computes it (src/audio.h:20-21).
long long resampled_length(long long n, int src, int dst) {
    if (src == dst) return n;
    return std::llround((double)n * ((double)dst / src));
}

struct AudioPlan {
    long long n = 0, len = 0, back = 0;
    int ch = 0, sr = 0, layout = 0, C = 0, R = 0, S = 0;
    bool convert = false;      // the input is not planar [C][n] already
    bool resample = false;     // sample_rate != model_rate
    size_t off_a = 0, off_b = 0, off_d = 0, off_e = 0, bytes = 0;
};

// The request checks of src/libstems.cpp:141-146, the model's shape, and the workspace layout:
// A [C][n] model-channel input | B [C][len] at the model's rate | D [S][C][len] stems at the
// model's rate | E [S][C][back] stems back at the input's rate (each present only when needed).
AudioPlan audio_plan(const stx_audio_view* in, int C, int R, int S) {
    STX_REQUIRE(in != nullptr && in->size >= STX_AUDIO_VIEW_MIN_SIZE && in->samples != nullptr && in->n_samples != 0 &&
                    in->n_channels != 0 && in->sample_rate != 0,
                "request.input needs samples, n_samples, n_channels and sample_rate");
    STX_REQUIRE(in->layout == STX_AUDIO_PLANAR || in->layout == STX_AUDIO_INTERLEAVED,
                "request.input.layout is not a known layout");
    STX_REQUIRE(in->n_samples <= (uint64_t)INT32_MAX / 4, "input is too long");
    STX_REQUIRE(in->n_channels <= (uint32_t)INT32_MAX && in->sample_rate <= (uint32_t)INT32_MAX,
                "request.input: channel count or rate out of range");
    STX_REQUIRE(C >= 1 && C <= 65535 && R >= 1 && S >= 1, "model_channels (1..65535), model_rate and n_sources must be positive");
    STX_REQUIRE((long long)S * C <= 65535, "n_sources * model_channels above 65535");
    AudioPlan p;
    p.n = (long long)in->n_samples;
    p.ch = (int)in->n_channels;
    p.sr = (int)in->sample_rate;
    p.layout = in->layout;
    p.C = C;
    p.R = R;
    p.S = S;
    p.convert = !(p.layout == STX_AUDIO_PLANAR && p.ch == C);
    p.resample = p.sr != R;
    p.len = resampled_length(p.n, p.sr, R);
    p.back = resampled_length(p.len, R, p.sr);
    STX_REQUIRE(p.len >= 1 && p.len <= (long long)INT32_MAX / 2, "input resampled to the model's rate is empty or too long");
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    size_t off = 0;
    if (p.convert) {
        p.off_a = off;
        off += up(sizeof(float) * (size_t)C * p.n);
    }
    if (p.resample) {
        p.off_b = off;
        off += up(sizeof(float) * (size_t)C * p.len);
        p.off_d = off;
        off += up(sizeof(float) * (size_t)S * C * p.len);
        if (p.back != p.n) {
            p.off_e = off;
            off += up(sizeof(float) * (size_t)S * C * p.back);
        }
    }
    p.bytes = off;
    return p;
}

// stx_resample over `planes` planes of n samples, at most 8 per launch.
void resample_planes(const stx_resampler* r, const float* in, long long planes, long long n, long long n_out, float* out,
                     hipStream_t s) {
    for (long long q = 0; q < planes; q += 8) {
        const int k = (int)std::min<long long>(8, planes - q);
        const stx_status st = stx_resample(r, in + q * n, k, n, out + q * n_out, s);
        if (st != STX_STATUS_OK) fail(st, "%s", stx_last_error());
    }
}

void check_rates(const stx_resampler* r, int src, int dst, const char* name) {
    STX_REQUIRE(r != nullptr, "%s is NULL but the rates differ (%d -> %d Hz)", name, src, dst);
    int a = 0, b = 0;
    resampler_rates(r, a, b);
    STX_REQUIRE(a == src && b == dst, "%s resamples %d -> %d Hz, not %d -> %d Hz", name, a, b, src, dst);
}

}  // namespace
}  // namespace stx

using namespace stx;

extern "C" {

STX_API size_t stx_separate_audio_workspace_size(const stx_audio_view* input, int model_channels, int model_rate,
                                                 int n_sources) {
    size_t bytes = 0;
    const stx_status st = guard([&] { bytes = audio_plan(input, model_channels, model_rate, n_sources).bytes; });
    return st == STX_STATUS_OK ? bytes : 0;
}

STX_API stx_status stx_separate_audio(const stx_audio_view* input, int model_channels, int model_rate, int n_sources,
                                      const stx_resampler* to_model, const stx_resampler* from_model,
                                      stx_model_separate_fn separate, void* separate_user,
                                      const stx_separate_options* options, float* out, void* workspace,
                                      size_t workspace_bytes, stx_stream stream) {
    return guard([&] {
        const stx_separate_options opt = separate_options(options);
        const AudioPlan p = audio_plan(input, model_channels, model_rate, n_sources);
        STX_REQUIRE(opt.shifts >= 0 && opt.shifts <= 10, "shifts must be 0..10");                       // :149-150
        STX_REQUIRE(opt.overlap < 1.0f, "overlap must be < 1 (negative = model default)");             // :151-152
        STX_REQUIRE(separate != nullptr, "separate is NULL");
        STX_REQUIRE(out != nullptr, "out is NULL");
        STX_REQUIRE(p.bytes == 0 || (workspace != nullptr && workspace_bytes >= p.bytes),
                    "workspace of %zu bytes, %zu needed", workspace_bytes, p.bytes);
        if (p.resample) {
            check_rates(to_model, p.sr, p.R, "to_model");
            check_rates(from_model, p.R, p.sr, "from_model");
        }
        const hipStream_t s = as_stream(stream);
        char* ws = static_cast<char*>(workspace);
        const float* audio = input->samples;
        if (p.convert) {                                       // :160-167 and st::to_channels
            float* a = reinterpret_cast<float*>(ws + p.off_a);
            hipLaunchKernelGGL(to_channels_kernel, dim3(io_blocks(p.n), (unsigned)p.C), dim3(kIoThreads), 0, s,
                               input->samples, p.n, p.ch, p.layout, a);
            launch_check("to_channels_kernel");
            audio = a;
        }
        float* stems = out;
        if (p.resample) {                                      // :169
            float* b = reinterpret_cast<float*>(ws + p.off_b);
            resample_planes(to_model, audio, p.C, p.n, p.len, b, s);
            audio = b;
            stems = reinterpret_cast<float*>(ws + p.off_d);
        }
        set_last_error("");
        const stx_status rc = separate(separate_user, audio, p.C, p.len, &opt, stems, stream);   // :184
        if (rc != STX_STATUS_OK) {
            const char* why = stx_last_error();
            fail(rc, "model separate failed (status %d)%s%s", (int)rc, why[0] ? ": " : "", why);
        }
        if (p.resample) {                                      // :185-196
            const long long planes = (long long)p.S * p.C;
            if (p.back == p.n) {
                resample_planes(from_model, stems, planes, p.len, p.back, out, s);
            } else {
                float* e = reinterpret_cast<float*>(ws + p.off_e);
                resample_planes(from_model, stems, planes, p.len, p.back, e, s);
                hipLaunchKernelGGL(pin_length_kernel, dim3(io_blocks(p.n), (unsigned)planes), dim3(kIoThreads), 0, s, e,
                                   p.back, out, p.n);
                launch_check("pin_length_kernel");
            }
        }
    });
}

}  // extern "C"
