// Fused grouped Conv -> BN -> LIF (groups > 1, depthwise included) over all
// T steps, on the fp16 NHWC copies the fused layers exchange.
//
// A grouped convolution computes Cin/groups * k * k products per output
// element (9 for a depthwise 3 x 3), so it is bound by HBM traffic, not by
// arithmetic: each thread owns one output channel of one pixel of one image,
// accumulates its group's taps in fp32 (one fma per product, order kh, kw,
// then the group's input channels), applies the folded BN affine and runs
// the LIF over T with the membrane in a register.  Consecutive threads take
// consecutive channels, so the NHWC input reads, the NHWC spike writes and
// the channels-last membrane accesses of a wave are contiguous.  An all-zero
// input (count block published as zero) takes the StaticZero route: no input
// reads, z is the channel's BN bias.
//
// Reference: catfuse/sparseflow/sparse_grouped_conv2d_kernel.py:93-364
// (groups run as independent sparse conv sub-problems, depthwise is
// groups == C; Conv only, the LIF separate).
#include "cf_common.h"

namespace {

struct GroupedArgs {
  const _Float16* x;      // [T*B][H][W][Cp] fp16 NHWC copy, or null
  const float* x32;       // [T*tstride + B][Cin][H][W] fp32 NCHW (analog input), or null
  int tstride;            // images between time steps of x32 (0: direct encoding)
  int Cin;
  const float* w;         // [Cout][Cg][K][K]
  const float* alpha;     // [Cout] folded BN scale
  const float* beta;      // [Cout] folded BN shift (+ bias * scale)
  const float* v_in;      // [B][Ho][Wo][Cout] or null
  float* v_out;           // [B][Ho][Wo][Cout] or null
  _Float16* out;          // [T*B][Ho][Wo][cp_out]
  const unsigned long long* nnz;   // count block of the input (routing), or null
  unsigned long long* nz_out;      // count block of the output, or null
  int T, B, Cp, Cout, cp_out, Cg, cout_per_group, H, W, Ho, Wo, K, stride, pad;
  LifParams lif;
};

template <int LM, bool DW3, bool XF32>
__global__ __launch_bounds__(256) void grouped_conv_lif_kernel(GroupedArgs a) {
  __shared__ unsigned any_sh[4];
  const uint32_t HoWo = (uint32_t)(a.Ho * a.Wo);
  const uint32_t total = (uint32_t)a.B * HoWo * (uint32_t)a.cp_out;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  uint32_t anyw = 0u;
  if (i < total) {
    const uint32_t co = i % (uint32_t)a.cp_out;
    const uint32_t pix = i / (uint32_t)a.cp_out;            // b * HoWo + p
    const uint32_t b = pix / HoWo, p = pix - b * HoWo;
    const int oh = (int)(p / (uint32_t)a.Wo), ow = (int)(p - (uint32_t)oh * (uint32_t)a.Wo);
    const bool real = co < (uint32_t)a.Cout;
    const bool zero_in = a.nnz != nullptr && cf_count_read(a.nnz) == 0ull;
    float v = lif_initial_v(a.lif);
    float al = 0.0f, be = 0.0f;
    int g0 = 0;
    if (real) {
      al = a.alpha[co];
      be = a.beta[co];
      g0 = (int)(co / (uint32_t)a.cout_per_group) * a.Cg;   // first input channel
      if (a.v_in) v = a.v_in[(size_t)pix * a.Cout + co];
    }
    const float* wc = a.w + (size_t)co * a.Cg * a.K * a.K;
    // depthwise 3 x 3: the nine weights stay in registers across the steps
    float w9[9];
    if constexpr (DW3) {
#pragma unroll
      for (int k = 0; k < 9; ++k) w9[k] = real ? wc[k] : 0.0f;
    }
    const int ih0 = oh * a.stride - a.pad, iw0 = ow * a.stride - a.pad;
    for (int t = 0; t < a.T; ++t) {
      float acc = 0.0f;
      if (real && !zero_in) {
        const _Float16* xb = XF32 ? nullptr : a.x + (size_t)((size_t)t * a.B + b) * a.H * a.W * a.Cp + g0;
        const float* xf = XF32 ? a.x32 + ((size_t)((size_t)t * a.tstride + b) * a.Cin + g0) * a.H * a.W
                               : nullptr;
        if constexpr (DW3) {
#pragma unroll
          for (int kh = 0; kh < 3; ++kh) {
            const int ih = ih0 + kh;
#pragma unroll
            for (int kw = 0; kw < 3; ++kw) {
              const int iw = iw0 + kw;
              const bool in = ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
              float xv = 0.0f;
              if (in) xv = XF32 ? xf[(size_t)ih * a.W + iw] : (float)xb[((size_t)ih * a.W + iw) * a.Cp];
              acc = __builtin_fmaf(xv, w9[kh * 3 + kw], acc);
            }
          }
        } else {
          for (int kh = 0; kh < a.K; ++kh) {
            const int ih = ih0 + kh;
            for (int kw = 0; kw < a.K; ++kw) {
              const int iw = iw0 + kw;
              const bool in = ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
              const size_t pos = (size_t)(in ? ih : 0) * a.W + (in ? iw : 0);
              for (int ci = 0; ci < a.Cg; ++ci) {
                float xv = 0.0f;
                if (in) xv = XF32 ? xf[(size_t)ci * a.H * a.W + pos] : (float)xb[pos * a.Cp + ci];
                acc = __builtin_fmaf(xv, wc[(ci * a.K + kh) * a.K + kw], acc);
              }
            }
          }
        }
      }
      const float z = __builtin_fmaf(acc, al, be);
      float vv = lif_charge_m<LM>(v, z, a.lif);
      const bool f = lif_fire_reset_bit<LM>(vv, a.lif) && real;
      v = vv;
      a.out[((size_t)((size_t)t * a.B + b) * HoWo + p) * a.cp_out + co] =
          f ? (_Float16)1.0f : (_Float16)0.0f;
      anyw |= f ? 1u : 0u;
    }
    if (real && a.v_out) a.v_out[(size_t)pix * a.Cout + co] = v;
  }
  if (a.nz_out) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (threadIdx.x == 0) cf_count_publish(a.nz_out, any ? 1ull : 0ull, blockIdx.x, gridDim.x);
  }
}

}  // namespace

CF_API int cf_conv_grouped_lif(const void* x, const float* x32, int64_t x_img_tstride,
                               const float* w, const float* alpha,
                               const float* beta, const float* v_in, float* v_out,
                               void* out_nhwc, int64_t cp_out, const unsigned long long* nnz,
                               unsigned long long* nz_out, int64_t T, int64_t B, int64_t Cin,
                               int64_t Cp, int64_t Cout, int64_t groups, int64_t H, int64_t W,
                               int64_t Ho, int64_t Wo, int64_t ksize, int64_t stride, int64_t pad,
                               double tau, double v_th, double v_reset, int hard_reset,
                               int decay_input, void* stream) {
  if ((!x) == (!x32) || !w || !alpha || !beta || !out_nhwc || x_img_tstride < 0)
    return (int)hipErrorInvalidValue;
  if (T <= 0 || B <= 0 || Cin <= 0 || Cout <= 0 || groups <= 0 || Cin % groups != 0 ||
      Cout % groups != 0 || (x && (Cp < Cin || Cp % 8 != 0)) || cp_out < Cout || cp_out % 8 != 0 ||
      H <= 0 || W <= 0 || ksize <= 0 || stride <= 0 || pad < 0)
    return (int)hipErrorInvalidValue;
  if (Ho != (H + 2 * pad - ksize) / stride + 1 || Wo != (W + 2 * pad - ksize) / stride + 1 ||
      Ho <= 0 || Wo <= 0)
    return (int)hipErrorInvalidValue;
  // 32-bit thread indices (B * Ho * Wo * cp_out) and a count block's tally
  const int64_t total = B * Ho * Wo * cp_out;
  if (total >= ((int64_t)1 << 32) - 256 || T * B * H * W * Cp > ((int64_t)1 << 40) ||
      (total + 255) / 256 >= (int64_t)CF_MAX_COUNT_WG)
    return (int)hipErrorInvalidValue;
  GroupedArgs a;
  a.x = (const _Float16*)x; a.x32 = x32; a.tstride = (int)x_img_tstride; a.Cin = (int)Cin;
  a.w = w; a.alpha = alpha; a.beta = beta; a.v_in = v_in;
  a.v_out = v_out; a.out = (_Float16*)out_nhwc; a.nnz = nnz; a.nz_out = nz_out;
  a.T = (int)T; a.B = (int)B; a.Cp = (int)Cp; a.Cout = (int)Cout; a.cp_out = (int)cp_out;
  a.Cg = (int)(Cin / groups); a.cout_per_group = (int)(Cout / groups);
  a.H = (int)H; a.W = (int)W; a.Ho = (int)Ho; a.Wo = (int)Wo; a.K = (int)ksize;
  a.stride = (int)stride; a.pad = (int)pad;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  const dim3 grid((unsigned)((total + 255) / 256)), block(256);
  const bool dw3 = a.Cg == 1 && ksize == 3, f32 = x32 != nullptr;
  const int lm = cf_lif_mode(a.lif);
  hipStream_t st = (hipStream_t)stream;
#define CF_GROUPED_X(LMV, DWV)                                                             \
  do {                                                                                     \
    if (f32) hipLaunchKernelGGL((grouped_conv_lif_kernel<LMV, DWV, true>), grid, block, 0, st, a); \
    else hipLaunchKernelGGL((grouped_conv_lif_kernel<LMV, DWV, false>), grid, block, 0, st, a);    \
  } while (0)
#define CF_GROUPED(LMV)                                                                    \
  do {                                                                                     \
    if (dw3) CF_GROUPED_X(LMV, true);                                                      \
    else CF_GROUPED_X(LMV, false);                                                         \
  } while (0)
  if (lm == LM_HARD0_DECAY_P2) CF_GROUPED(LM_HARD0_DECAY_P2);
  else if (lm == LM_HARD_DECAY_P2) CF_GROUPED(LM_HARD_DECAY_P2);
  else CF_GROUPED(LM_GENERIC);
#undef CF_GROUPED
#undef CF_GROUPED_X
  return (int)hipGetLastError();
}
