// Streaming multi-step LIF family (HBM-bound tails).
//
// One thread owns 4 consecutive neurons for all T steps: the membrane
// potential v stays in VGPRs across the time loop (TimeBlock(K=T) with
// StateCarry through v_in/v_out), z is read once per step with dwordx4
// loads, spikes are written once per step.  The loads of up to four steps
// are issued before the first of them is used, so a thread waits for one
// memory latency per four steps, not one per step.  Algorithmic bytes per neuron:
//   mode 0/1 : (8T + 8)  (z, spike, v_in, v_out)
//   mode 2-4 : (12T + 8) (z, z2, spike, v_in, v_out)
//
// Reference kernels this family replaces (behaviour, not code):
//   catfuse/sparseflow/lif_seq_kernel.py:12-90          (mode 0)
//   catfuse/kernels/partial_fusion_conv_lif_impl.py:91-156     (mode 0, v0=0)
//   catfuse/kernels/partial_fusion_conv_bn_lif_impl.py:110-189 (mode 1)
//   catfuse/kernels/partial_fusion_conv_bn_add_lif_impl.py:76-158 (mode 2)
//   catfuse/kernels/add_lif.py:63-151                   (mode 3)
//   benchmarks/add_bn_lif_min.py:72-129                 (mode 4)
// The LIF op order follows SpikingJelly (lif_charge in cf_common.h), not the
// reference's Triton reformulation v*DECAY + z*RT (lif_seq_kernel.py:37).
#include "cf_common.h"
#include <math.h>

namespace {

enum { M_PLAIN = 0, M_BN = 1, M_BN_ADD = 2, M_ADD = 3, M_ADD_BN = 4 };

template <int MODE>
__device__ __forceinline__ float input_current(float z, float z2, float s, float b) {
  if (MODE == M_PLAIN) return z;
  if (MODE == M_BN) return z * s + b;
  if (MODE == M_BN_ADD) return (z * s + b) + z2;
  if (MODE == M_ADD) return z + z2;
  return (z + z2) * s + b;  // M_ADD_BN
}

template <typename S> __device__ __forceinline__ S to_spike(float s);
template <> __device__ __forceinline__ float to_spike<float>(float s) { return s; }
template <> __device__ __forceinline__ uint8_t to_spike<uint8_t>(float s) { return (uint8_t)s; }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Streamed operands (read or written once per launch), accessed
// non-temporally: on buffers that are not cache-resident (the tails' inputs
// are a conv's output, written long before in a large layer) non-temporal
// loads and stores, the final potential's included, measured 66-67 -> 77 %
// of HBM peak for the one-input modes and 77-80 % for the two-input ones.
template <bool NT>
__device__ __forceinline__ float4 load_stream(const float* p) {
  if constexpr (NT) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
  } else {
    return *reinterpret_cast<const float4*>(p);
  }
}
template <bool NT>
__device__ __forceinline__ void store_stream(float* p, float a, float b, float c, float d) {
  if constexpr (NT) {
    const f32x4 v = {a, b, c, d};
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
  }
}

template <int MODE, typename S, int LM>
__global__ __launch_bounds__(256) void lif_stream_vec4(
    const float* __restrict__ z, const float* __restrict__ z2,
    const float* __restrict__ scale, const float* __restrict__ shift,
    const float* __restrict__ v_in, S* __restrict__ spike, float* __restrict__ v_out,
    int T, int64_t N, int C, int64_t HW, LifParams p) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // quad index
  const int64_t n0 = q * 4;
  if (n0 >= N) return;
  float sc[4], sh[4];
  if (MODE == M_BN || MODE == M_BN_ADD || MODE == M_ADD_BN) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = (int)(((n0 + j) / HW) % C);
      sc[j] = scale[c];
      sh[j] = shift[c];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) { sc[j] = 1.0f; sh[j] = 0.0f; }
  }
  float v[4];
  if (v_in) {
    const float4 vi = *reinterpret_cast<const float4*>(v_in + n0);
    v[0] = vi.x; v[1] = vi.y; v[2] = vi.z; v[3] = vi.w;
  } else {
    const float v0 = lif_initial_v(p);
    v[0] = v[1] = v[2] = v[3] = v0;
  }
  constexpr bool TWO = MODE == M_BN_ADD || MODE == M_ADD || MODE == M_ADD_BN;
  constexpr int TC = 4;   // steps whose loads are in flight together
  for (int t0 = 0; t0 < T; t0 += TC) {
    float4 zz[TC], z2v[TC];
#pragma unroll
    for (int u = 0; u < TC; ++u) {
      zz[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      z2v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (t0 + u < T) {
        const int64_t off = (int64_t)(t0 + u) * N + n0;
        zz[u] = load_stream<true>(z + off);
        if (TWO) z2v[u] = load_stream<true>(z2 + off);
      }
    }
#pragma unroll
    for (int u = 0; u < TC; ++u) {
      if (t0 + u >= T) break;
      const int64_t off = (int64_t)(t0 + u) * N + n0;
      const float zi[4] = {zz[u].x, zz[u].y, zz[u].z, zz[u].w};
      const float z2i[4] = {z2v[u].x, z2v[u].y, z2v[u].z, z2v[u].w};
      float s[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = input_current<MODE>(zi[j], z2i[j], sc[j], sh[j]);
        v[j] = lif_charge_m<LM>(v[j], x, p);
        s[j] = lif_fire_reset_bit<LM>(v[j], p) ? 1.0f : 0.0f;
      }
      if constexpr (sizeof(S) == 4) {
        store_stream<true>(spike + off, s[0], s[1], s[2], s[3]);
      } else {
        uchar4 o;
        o.x = (uint8_t)s[0]; o.y = (uint8_t)s[1]; o.z = (uint8_t)s[2]; o.w = (uint8_t)s[3];
        *reinterpret_cast<uchar4*>(spike + off) = o;
      }
    }
  }
  if (v_out) store_stream<true>(v_out + n0, v[0], v[1], v[2], v[3]);
}

template <int MODE, typename S, int LM>
__global__ __launch_bounds__(256) void lif_stream_scalar(
    const float* __restrict__ z, const float* __restrict__ z2,
    const float* __restrict__ scale, const float* __restrict__ shift,
    const float* __restrict__ v_in, S* __restrict__ spike, float* __restrict__ v_out,
    int T, int64_t N, int C, int64_t HW, LifParams p) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float sc = 1.0f, sh = 0.0f;
  if (MODE == M_BN || MODE == M_BN_ADD || MODE == M_ADD_BN) {
    const int c = (int)((n / HW) % C);
    sc = scale[c];
    sh = shift[c];
  }
  float v = v_in ? v_in[n] : lif_initial_v(p);
  for (int t = 0; t < T; ++t) {
    const int64_t off = (int64_t)t * N + n;
    const float b = (MODE == M_BN_ADD || MODE == M_ADD || MODE == M_ADD_BN) ? z2[off] : 0.0f;
    const float x = input_current<MODE>(z[off], b, sc, sh);
    v = lif_charge_m<LM>(v, x, p);
    spike[off] = to_spike<S>(lif_fire_reset_bit<LM>(v, p) ? 1.0f : 0.0f);
  }
  if (v_out) v_out[n] = v;
}

template <int MODE, typename S, int LM>
hipError_t launch_lif_m(const float* z, const float* z2, const float* scale, const float* shift,
                        const float* v_in, S* spike, float* v_out, int T, int64_t N, int C,
                        int64_t HW, const LifParams& p, hipStream_t st) {
  const bool aligned = ((uintptr_t)z % 16 == 0) && (!z2 || (uintptr_t)z2 % 16 == 0) &&
                       ((uintptr_t)spike % (4 * sizeof(S)) == 0) &&
                       (!v_in || (uintptr_t)v_in % 16 == 0) &&
                       (!v_out || (uintptr_t)v_out % 16 == 0);
  if (N % 4 == 0 && aligned) {
    hipLaunchKernelGGL((lif_stream_vec4<MODE, S, LM>), dim3(cf_blocks(N / 4, 256)), dim3(256), 0,
                       st, z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p);
  } else {
    hipLaunchKernelGGL((lif_stream_scalar<MODE, S, LM>), dim3(cf_blocks(N, 256)), dim3(256), 0,
                       st, z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p);
  }
  return hipGetLastError();
}

template <int MODE, typename S>
hipError_t launch_lif(const float* z, const float* z2, const float* scale, const float* shift,
                      const float* v_in, S* spike, float* v_out, int T, int64_t N, int C,
                      int64_t HW, const LifParams& p, hipStream_t st) {
  switch (cf_lif_mode(p)) {
    case LM_HARD0_DECAY_P2:
      return launch_lif_m<MODE, S, LM_HARD0_DECAY_P2>(z, z2, scale, shift, v_in, spike, v_out, T,
                                                      N, C, HW, p, st);
    case LM_HARD_DECAY_P2:
      return launch_lif_m<MODE, S, LM_HARD_DECAY_P2>(z, z2, scale, shift, v_in, spike, v_out, T,
                                                     N, C, HW, p, st);
    default:
      return launch_lif_m<MODE, S, LM_GENERIC>(z, z2, scale, shift, v_in, spike, v_out, T, N, C,
                                               HW, p, st);
  }
}

template <typename S>
hipError_t dispatch_mode(int mode, const float* z, const float* z2, const float* scale,
                         const float* shift, const float* v_in, S* spike, float* v_out, int T,
                         int64_t N, int C, int64_t HW, const LifParams& p, hipStream_t st) {
  switch (mode) {
    case M_PLAIN: return launch_lif<M_PLAIN, S>(z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p, st);
    case M_BN: return launch_lif<M_BN, S>(z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p, st);
    case M_BN_ADD: return launch_lif<M_BN_ADD, S>(z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p, st);
    case M_ADD: return launch_lif<M_ADD, S>(z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p, st);
    case M_ADD_BN: return launch_lif<M_ADD_BN, S>(z, z2, scale, shift, v_in, spike, v_out, T, N, C, HW, p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Builds the LIF parameter block from the SpikingJelly-level (double)
// parameters: tau/v_th/v_reset are rounded to fp32 exactly as torch does when
// a Python float meets an fp32 tensor; 1 - 1/tau is evaluated in double first.
LifParams cf_make_lif_params(double tau, double v_th, double v_reset, int hard, int decay_input) {
  LifParams p;
  p.tau = (float)tau;
  p.v_th = (float)v_th;
  p.v_reset = hard ? (float)v_reset : 0.0f;
  p.decay_coef = (float)(1.0 - 1.0 / tau);
  int e2 = 0;
  const double m = frexp((double)p.tau, &e2);  // |tau| = |m| * 2^e2, |m| in [0.5, 1)
  p.tau_pow2 = (m == 0.5 || m == -0.5) && e2 - 1 >= -125 && e2 - 1 <= 126 ? 1 : 0;
  p.inv_tau = p.tau_pow2 ? (float)(1.0 / (double)p.tau) : 0.0f;
  p.hard = hard ? 1 : 0;
  p.decay_input = decay_input ? 1 : 0;
  return p;
}

CF_API int cf_lif_multistep(const float* z, const float* z2, const float* scale, const float* shift,
                            int mode, const float* v_in, void* spike, int spike_dtype,
                            float* v_out, int64_t T, int64_t N, int64_t C, int64_t HW,
                            double tau, double v_th, double v_reset, int hard_reset,
                            int decay_input, void* stream) {
  if (!z || !spike || T < 0 || N < 0 || mode < 0 || mode > 4) return (int)hipErrorInvalidValue;
  const bool need_z2 = (mode == M_BN_ADD || mode == M_ADD || mode == M_ADD_BN);
  const bool need_aff = (mode == M_BN || mode == M_BN_ADD || mode == M_ADD_BN);
  if (need_z2 && !z2) return (int)hipErrorInvalidValue;
  if (need_aff && (!scale || !shift || C <= 0 || HW <= 0)) return (int)hipErrorInvalidValue;
  if (T == 0 || N == 0) return 0;
  if (C <= 0) C = 1;
  if (HW <= 0) HW = 1;
  if (T > INT32_MAX || C > INT32_MAX) return (int)hipErrorInvalidValue;
  const LifParams p = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (spike_dtype == 0)
    e = dispatch_mode<float>(mode, z, z2, scale, shift, v_in, (float*)spike, v_out, (int)T, N,
                             (int)C, HW, p, st);
  else if (spike_dtype == 1)
    e = dispatch_mode<uint8_t>(mode, z, z2, scale, shift, v_in, (uint8_t*)spike, v_out, (int)T, N,
                               (int)C, HW, p, st);
  else
    return (int)hipErrorInvalidValue;
  return (int)e;
}
