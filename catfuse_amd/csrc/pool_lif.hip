// AvgPool2d(2, stride 2) -> LIF over T steps, one thread per output neuron,
// v in a VGPR across the time loop.  z = (p00 + p01 + p10 + p11) * 0.25 in
// that order (catfuse/kernels/avgpool_lif.py:131-132; equal to torch's
// avg_pool2d for a 2x2 window since 0.25 is a power of two).
// Algorithmic bytes per output neuron: 16T (4 inputs) + 4T (spike) + 8 (v).
#include "cf_common.h"

namespace {

template <typename S>
__global__ __launch_bounds__(256) void avgpool2_lif_kernel(
    const float* __restrict__ x, const float* __restrict__ v_in, S* __restrict__ spike,
    float* __restrict__ v_out, int T, int64_t NC, int H, int W, int Ho, int Wo, LifParams p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (nc, oh, ow)
  const int64_t per_step = NC * Ho * Wo;
  if (i >= per_step) return;
  const int ow = (int)(i % Wo);
  const int oh = (int)((i / Wo) % Ho);
  const int64_t nc = i / ((int64_t)Wo * Ho);
  float v = v_in ? v_in[i] : lif_initial_v(p);
  const int64_t in_step = NC * H * W;
  const int64_t base = nc * H * W + (int64_t)(2 * oh) * W + 2 * ow;
  for (int t = 0; t < T; ++t) {
    const float* xt = x + (int64_t)t * in_step + base;
    const float p00 = xt[0], p01 = xt[1], p10 = xt[W], p11 = xt[W + 1];
    const float z = (((p00 + p01) + p10) + p11) * 0.25f;
    v = lif_charge(v, z, p);
    const float s = lif_fire_reset(v, p);
    spike[(int64_t)t * per_step + i] = (S)s;
  }
  if (v_out) v_out[i] = v;
}

}  // namespace

CF_API int cf_avgpool2x2_lif(const float* x, const float* v_in, void* spike, int spike_dtype,
                             float* v_out, int64_t T, int64_t NC, int64_t H, int64_t W,
                             double tau, double v_th, double v_reset, int hard_reset,
                             int decay_input, void* stream) {
  if (!x || !spike || T < 0 || NC < 0 || H < 2 || W < 2) return (int)hipErrorInvalidValue;
  const int64_t Ho = H / 2, Wo = W / 2;
  const int64_t n = NC * Ho * Wo;
  if (T == 0 || n == 0) return 0;
  const LifParams p = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  hipStream_t st = (hipStream_t)stream;
  if (spike_dtype == 0)
    hipLaunchKernelGGL(avgpool2_lif_kernel<float>, dim3(cf_blocks(n, 256)), dim3(256), 0, st, x,
                       v_in, (float*)spike, v_out, (int)T, NC, (int)H, (int)W, (int)Ho, (int)Wo, p);
  else if (spike_dtype == 1)
    hipLaunchKernelGGL(avgpool2_lif_kernel<uint8_t>, dim3(cf_blocks(n, 256)), dim3(256), 0, st, x,
                       v_in, (uint8_t*)spike, v_out, (int)T, NC, (int)H, (int)W, (int)Ho, (int)Wo,
                       p);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}
