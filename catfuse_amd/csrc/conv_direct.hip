// Fused Conv -> BN -> LIF for analog (non-spike) inputs, in fp32 on the VALU.
//
// Used for the network's first layer (e.g. the SEW-ResNet 7x7/2 stem over
// an image, VGG's first 3x3), where x is not exactly representable in fp16
// and the channel count is tiny (C_in = 3), so an MFMA tile would be mostly
// padding.  Each thread owns one output pixel and COB output channels;
// weight indices are wave-uniform (scalar loads), products are fused
// multiply-adds in fp32.
//
// Direct encoding: when the caller's input repeats one image over T (a
// stride-0 time axis, x_img_tstride == 0), the convolution is evaluated once
// and its z feeds all T LIF steps, which is exact because z is identical.
//
// Reference behaviour replaced: catfuse/implementations/dense_keep.py:97-155
// applied to the stem (catfuse/patterns.py:237-387 PartialFusionConvBNLIF).
#include "cf_common.h"

namespace {

enum { EPI_LIF = 0, EPI_Z = 1 };

struct DirectArgs {
  const float* x;  // [img][Cin][H][W], img = t*x_img_tstride + b
  const float* w;  // [Cout][Cin][KH][KW]
  const float* alpha;
  const float* beta;
  const float* v_in;
  float* v_out;
  float* out;  // [T][B][Cout][Ho][Wo] or null (then out_nhwc is set)
  _Float16* out_nhwc;  // [T*B][Ho][Wo][cp_out] or null
  int cp_out;
  int T, B, Cin, Cout, H, W, Ho, Wo, KH, KW, stride, pad, x_img_tstride;
  LifParams lif;
};

template <int COB>
__device__ __forceinline__ void conv_pixel(const DirectArgs& a, int img, int oh, int ow, int co0,
                                           float (&acc)[COB]) {
#pragma unroll
  for (int j = 0; j < COB; ++j) acc[j] = 0.0f;
  const int ih0 = oh * a.stride - a.pad, iw0 = ow * a.stride - a.pad;
  const float* xb = a.x + (size_t)img * a.Cin * a.H * a.W;
  const int KK = a.KH * a.KW;
  for (int ci = 0; ci < a.Cin; ++ci) {
    const float* xc = xb + (size_t)ci * a.H * a.W;
    for (int kh = 0; kh < a.KH; ++kh) {
      const int ih = ih0 + kh;
      const bool hok = ih >= 0 && ih < a.H;
      for (int kw = 0; kw < a.KW; ++kw) {
        const int iw = iw0 + kw;
        const float xv = (hok && iw >= 0 && iw < a.W) ? xc[(size_t)ih * a.W + iw] : 0.0f;
        const float* wp = a.w + ((size_t)co0 * a.Cin + ci) * KK + kh * a.KW + kw;
#pragma unroll
        for (int j = 0; j < COB; ++j) acc[j] = fmaf(xv, wp[(size_t)j * a.Cin * KK], acc[j]);
      }
    }
  }
}

template <int COB, int EPI>
__global__ __launch_bounds__(256) void conv_direct_kernel(DirectArgs a) {
  const int HoWo = a.Ho * a.Wo;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  const int co0 = blockIdx.z * COB;  // host guarantees Cout % COB == 0
  if (p >= HoWo) return;
  const int oh = p / a.Wo, ow = p % a.Wo;
  float acc[COB], v[COB];
  if (EPI == EPI_LIF) {
#pragma unroll
    for (int j = 0; j < COB; ++j)
      v[j] = a.v_in ? a.v_in[((size_t)b * a.Cout + co0 + j) * HoWo + p] : lif_initial_v(a.lif);
  }
  const bool dedupe = a.x_img_tstride == 0;
  if (dedupe) conv_pixel<COB>(a, b, oh, ow, co0, acc);
  for (int t = 0; t < a.T; ++t) {
    if (!dedupe) conv_pixel<COB>(a, t * a.x_img_tstride + b, oh, ow, co0, acc);
    typedef _Float16 h8v __attribute__((ext_vector_type(8)));
    h8v oh16[(COB + 7) / 8];
#pragma unroll
    for (int j = 0; j < COB; ++j) {
      const int co = co0 + j;
      const float z = acc[j] * a.alpha[co] + a.beta[co];
      const size_t o = ((size_t)(t * a.B + b) * a.Cout + co) * HoWo + p;
      float ov;
      if (EPI == EPI_Z) {
        ov = z;
      } else {
        float vv = lif_charge(v[j], z, a.lif);
        ov = lif_fire_reset(vv, a.lif);
        v[j] = vv;
      }
      if (a.out) a.out[o] = ov;
      oh16[j / 8][j % 8] = (_Float16)ov;
    }
    if (a.out_nhwc) {
      _Float16* dst = a.out_nhwc + ((size_t)(t * a.B + b) * HoWo + p) * a.cp_out + co0;
      if constexpr (COB % 8 == 0) {
        // the pixel's COB channels as 16-byte chunks (co0 and cp_out are
        // multiples of 8)
#pragma unroll
        for (int j = 0; j < COB; j += 8) *reinterpret_cast<h8v*>(dst + j) = oh16[j / 8];
      } else {
#pragma unroll
        for (int j = 0; j < COB; ++j) dst[j] = oh16[j / 8][j % 8];
      }
    }
    if (a.out_nhwc && co0 + COB == a.Cout)
      for (int co = a.Cout; co < a.cp_out; ++co)
        store_nhwc(a.out_nhwc, a.cp_out, (size_t)t * a.B + b, HoWo, p, co, 0.0f);
  }
  if (EPI == EPI_LIF && a.v_out) {
#pragma unroll
    for (int j = 0; j < COB; ++j) a.v_out[((size_t)b * a.Cout + co0 + j) * HoWo + p] = v[j];
  }
}

template <int COB>
hipError_t launch_direct(const DirectArgs& a, int epi, hipStream_t st) {
  dim3 grid(cf_blocks((int64_t)a.Ho * a.Wo, 256), (unsigned)a.B, (unsigned)(a.Cout / COB));
  if (epi == EPI_Z) hipLaunchKernelGGL((conv_direct_kernel<COB, EPI_Z>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((conv_direct_kernel<COB, EPI_LIF>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

CF_API int cf_conv_direct(const float* x, const float* w, const float* alpha, const float* beta,
                          const float* v_in, float* v_out, float* out, void* out_nhwc,
                          int64_t cp_out, int64_t T, int64_t B,
                          int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
                          int64_t KH, int64_t KW, int64_t stride, int64_t pad,
                          int64_t x_img_tstride, int epilogue, double tau, double v_th,
                          double v_reset, int hard_reset, int decay_input, void* stream) {
  if (!x || !w || !alpha || !beta || (!out && !out_nhwc) || T <= 0 || B <= 0 || Cin <= 0 || Cout <= 0 ||
      H <= 0 || W <= 0 || KH <= 0 || KW <= 0 || stride <= 0 || pad < 0 || x_img_tstride < 0 ||
      B > 65535)
    return (int)hipErrorInvalidValue;
  if (Ho != (H + 2 * pad - KH) / stride + 1 || Wo != (W + 2 * pad - KW) / stride + 1 || Ho <= 0 ||
      Wo <= 0)
    return (int)hipErrorInvalidValue;
  if (epilogue != EPI_LIF && epilogue != EPI_Z) return (int)hipErrorInvalidValue;
  DirectArgs a;
  a.x = x; a.w = w; a.alpha = alpha; a.beta = beta; a.v_in = v_in; a.v_out = v_out; a.out = out;
  a.out_nhwc = (_Float16*)out_nhwc; a.cp_out = (int)cp_out;
  if (out_nhwc && (cp_out < Cout || cp_out % 8 != 0)) return (int)hipErrorInvalidValue;
  a.T = (int)T; a.B = (int)B; a.Cin = (int)Cin; a.Cout = (int)Cout; a.H = (int)H; a.W = (int)W;
  a.Ho = (int)Ho; a.Wo = (int)Wo; a.KH = (int)KH; a.KW = (int)KW; a.stride = (int)stride;
  a.pad = (int)pad; a.x_img_tstride = (int)x_img_tstride;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  hipStream_t st = (hipStream_t)stream;
  if (Cout % 16 == 0) return (int)launch_direct<16>(a, epilogue, st);
  if (Cout % 4 == 0) return (int)launch_direct<4>(a, epilogue, st);
  return (int)launch_direct<1>(a, epilogue, st);
}
