// k_embed.hip -- time/noise embeddings.
// Reference maths: mp_fourier src/kernels.cu:385-394 (launcher 416-423) and
// sinusoidal src/kernels.cu:444-456 (launcher 569-575).
//
// Both outputs are tiny ([batch, C], <= a few hundred KB) and latency-bound.
// The float arguments are formed exactly as the reference forms them; the
// transcendental step (cos, sin, exp) is evaluated in double and rounded once
// to float, i.e. the correctly rounded value of the float function, so the
// result does not depend on a float libm's last-ulp behaviour.
#include "nnk_common.h"

namespace {

constexpr int kTpb = 256;

__global__ __launch_bounds__(kTpb) void mp_fourier_kernel(float* __restrict__ out,
    const float* __restrict__ x, const float* __restrict__ freqs,
    const float* __restrict__ phases, int total, nnk::FastDiv divC) {
    const int i = blockIdx.x * kTpb + threadIdx.x;
    if (i >= total) return;
    uint32_t b, k;
    divC.divmod((uint32_t)i, b, k);
    const float arg = 6.28318530718f * (x[b] * freqs[k] + phases[k]);
    out[i] = 1.41421356237f * (float)cos((double)arg);
}

__global__ __launch_bounds__(kTpb) void sinusoidal_kernel(float* __restrict__ out,
    const float* __restrict__ t, int total, int half, nnk::FastDiv divC, float log_max_period) {
    const int i = blockIdx.x * kTpb + threadIdx.x;
    if (i >= total) return;
    uint32_t b, c;
    divC.divmod((uint32_t)i, b, c);
    const int j = (int)c < half ? (int)c : (int)c - half;
    const float e = -log_max_period * (float)j / (float)half;
    const float freq = (float)exp((double)e);
    const float arg = t[b] * freq;
    out[i] = (int)c < half ? (float)sin((double)arg) : (float)cos((double)arg);
}

}  // namespace

extern "C" {

void launch_mp_fourier(float* out, const float* x, const float* freqs, const float* phases,
    int batch, int C, hipStream_t s) {
    const char* what = "launch_mp_fourier";
    NNK_REQUIRE(batch >= 0 && C > 0, what, "%s: bad shape batch=%d C=%d", what, batch, C);
    const long long total = (long long)batch * C;
    NNK_REQUIRE(total < (1LL << 31), what, "%s: too many elements", what);
    if (total == 0) return;
    NNK_REQUIRE(out && x && freqs && phases, what, "%s: null pointer", what);
    mp_fourier_kernel<<<(unsigned)((total + kTpb - 1) / kTpb), kTpb, 0, s>>>(out, x, freqs, phases,
        (int)total, nnk::FastDiv((uint32_t)C));
    nnk_after_launch(what, s);
}

void launch_sinusoidal(float* out, const float* t, int batch, int C, float log_max_period,
    hipStream_t s) {
    const char* what = "launch_sinusoidal";
    NNK_REQUIRE(batch >= 0 && C >= 2, what, "%s: bad shape batch=%d C=%d", what, batch, C);
    const long long total = (long long)batch * C;
    NNK_REQUIRE(total < (1LL << 31), what, "%s: too many elements", what);
    if (total == 0) return;
    NNK_REQUIRE(out && t, what, "%s: null pointer", what);
    sinusoidal_kernel<<<(unsigned)((total + kTpb - 1) / kTpb), kTpb, 0, s>>>(out, t, (int)total,
        C / 2, nnk::FastDiv((uint32_t)C), log_max_period);
    nnk_after_launch(what, s);
}

}  // extern "C"
