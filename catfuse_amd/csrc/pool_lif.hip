// AvgPool2d(2, stride 2) -> LIF over T steps, v in a VGPR across the time
// loop.  z = (p00 + p01 + p10 + p11) * 0.25 in that order
// (catfuse/kernels/avgpool_lif.py:131-132; equal to torch's avg_pool2d for a
// 2x2 window since 0.25 is a power of two).
// Algorithmic bytes per output neuron: 16T (4 inputs) + 4T (spike) + 8 (v).
// When W is a multiple of 4 (and the pointers allow it) a thread owns two
// horizontally adjacent outputs: one 16-byte load per input row and step,
// and the loads of up to four steps in flight before the first is used;
// every access of that kernel is non-temporal (on inputs that are not
// cache-resident: 59 -> 65 % of HBM peak at the VGG shape).
#include "cf_common.h"

namespace {

typedef float f32x4_nt __attribute__((ext_vector_type(4)));
typedef float f32x2_nt __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float4 load4_nt(const float* p) {
  const f32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_nt*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store2_nt(float* p, float a, float b) {
  const f32x2_nt v = {a, b};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x2_nt*>(p));
}

template <typename S> struct Pair;
template <> struct Pair<float> { typedef float2 type; };
template <> struct Pair<uint8_t> { typedef uchar2 type; };

template <typename S, int LM>
__global__ __launch_bounds__(256) void avgpool2_lif_pair_kernel(
    const float* __restrict__ x, const float* __restrict__ v_in, S* __restrict__ spike,
    float* __restrict__ v_out, int T, int64_t NC, int H, int W, int Ho, int Wo, LifParams p) {
  const int64_t i2 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (nc, oh, ow pair)
  const int Wp = Wo / 2;
  const int64_t pairs = NC * Ho * Wp;
  if (i2 >= pairs) return;
  const int owp = (int)(i2 % Wp);
  const int oh = (int)((i2 / Wp) % Ho);
  const int64_t nc = i2 / ((int64_t)Wp * Ho);
  const int64_t i = (nc * Ho + oh) * Wo + 2 * owp;   // first output of the pair
  const int64_t per_step = NC * Ho * Wo;
  float v0, v1;
  if (v_in) {
    const float2 vi = *reinterpret_cast<const float2*>(v_in + i);
    v0 = vi.x;
    v1 = vi.y;
  } else {
    v0 = v1 = lif_initial_v(p);
  }
  const int64_t in_step = NC * H * W;
  const int64_t base = nc * H * W + (int64_t)(2 * oh) * W + 4 * owp;
  constexpr int TC = 4;
  for (int t0 = 0; t0 < T; t0 += TC) {
    float4 r0[TC], r1[TC];
#pragma unroll
    for (int u = 0; u < TC; ++u) {
      r0[u] = r1[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (t0 + u < T) {
        const float* xt = x + (int64_t)(t0 + u) * in_step + base;
        r0[u] = load4_nt(xt);
        r1[u] = load4_nt(xt + W);
      }
    }
#pragma unroll
    for (int u = 0; u < TC; ++u) {
      if (t0 + u >= T) break;
      const float z0 = (((r0[u].x + r0[u].y) + r1[u].x) + r1[u].y) * 0.25f;
      const float z1 = (((r0[u].z + r0[u].w) + r1[u].z) + r1[u].w) * 0.25f;
      v0 = lif_charge_m<LM>(v0, z0, p);
      const bool f0 = lif_fire_reset_bit<LM>(v0, p);
      v1 = lif_charge_m<LM>(v1, z1, p);
      const bool f1 = lif_fire_reset_bit<LM>(v1, p);
      S* const sp = spike + (int64_t)(t0 + u) * per_step + i;
      if constexpr (sizeof(S) == 4) {
        store2_nt(sp, f0 ? 1.0f : 0.0f, f1 ? 1.0f : 0.0f);
      } else {
        typename Pair<S>::type o;
        o.x = f0 ? (S)1 : (S)0;
        o.y = f1 ? (S)1 : (S)0;
        *reinterpret_cast<typename Pair<S>::type*>(sp) = o;
      }
    }
  }
  if (v_out) store2_nt(v_out + i, v0, v1);
}

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
  if (spike_dtype != 0 && spike_dtype != 1) return (int)hipErrorInvalidValue;
  const size_t sb = spike_dtype == 0 ? 4 : 1;
  const bool pair = W % 4 == 0 && (uintptr_t)x % 16 == 0 &&
                    (uintptr_t)spike % (2 * sb) == 0 && (!v_in || (uintptr_t)v_in % 8 == 0) &&
                    (!v_out || (uintptr_t)v_out % 8 == 0);
  if (pair) {
    const dim3 grid(cf_blocks(n / 2, 256)), block(256);
    const int lm = cf_lif_mode(p);
#define CF_POOL_PAIR(SV, LMV)                                                                  \
  hipLaunchKernelGGL((avgpool2_lif_pair_kernel<SV, LMV>), grid, block, 0, st, x, v_in,         \
                     (SV*)spike, v_out, (int)T, NC, (int)H, (int)W, (int)Ho, (int)Wo, p)
    if (spike_dtype == 0) {
      if (lm == LM_HARD0_DECAY_P2) CF_POOL_PAIR(float, LM_HARD0_DECAY_P2);
      else if (lm == LM_HARD_DECAY_P2) CF_POOL_PAIR(float, LM_HARD_DECAY_P2);
      else CF_POOL_PAIR(float, LM_GENERIC);
    } else {
      if (lm == LM_HARD0_DECAY_P2) CF_POOL_PAIR(uint8_t, LM_HARD0_DECAY_P2);
      else if (lm == LM_HARD_DECAY_P2) CF_POOL_PAIR(uint8_t, LM_HARD_DECAY_P2);
      else CF_POOL_PAIR(uint8_t, LM_GENERIC);
    }
#undef CF_POOL_PAIR
    return (int)hipGetLastError();
  }
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
