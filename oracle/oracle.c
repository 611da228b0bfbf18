/* CPU oracle for the catfuse_amd hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline);
 * the product path never calls it.
 *
 * Plain scalar C, compiled with -O2 -ffp-contract=off (no fused
 * multiply-add) so every float operation rounds exactly once, in the order
 * written.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Multi-step LIF in SpikingJelly 0.0.0.0.14 eval-mode order (the
 * jit_eval_multi_step_forward_{hard,soft}_reset_{decay,no_decay}_input
 * recurrences that LIFNode.multi_step_forward uses with the torch backend),
 * as restated by the reference at tests/check_lif_parity.py:16-22 and
 * catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:425-445:
 *   hard, decay   : h = v + (x - (v - v_reset)) / tau
 *   hard, no decay: h = v - (v - v_reset) / tau + x
 *   soft, decay   : h = v + (x - v) / tau
 *   soft, no decay: h = v * (1 - 1/tau) + x       [(1 - 1/tau) in double]
 *   s = (h >= v_th)
 *   hard: v = v_reset * s + (1 - s) * h      soft: v = h - s * v_th
 * Input current x per mode (channel c = (n / HW) % C):
 *   0: z   1: z*scale + shift   2: (z*scale + shift) + z2
 *   3: z + z2   4: (z + z2)*scale + shift
 * (catfuse/kernels/partial_fusion_conv_bn_lif_impl.py:110-155,
 *  partial_fusion_conv_bn_add_lif_impl.py:76-123, kernels/add_lif.py:63-110,
 *  benchmarks/add_bn_lif_min.py:72-129).
 * h_seq (nullable) receives the charged potential h before fire/reset. */
void oracle_lif_multistep(const float* z, const float* z2, const float* scale,
                          const float* shift, int mode, const float* v_in, float* spike,
                          float* v_out, float* h_seq, int64_t T, int64_t N, int64_t C,
                          int64_t HW, double tau_d, double v_th_d, double v_reset_d, int hard,
                          int decay_input) {
  const float tau = (float)tau_d, v_th = (float)v_th_d;
  const float v_reset = hard ? (float)v_reset_d : 0.0f;
  const float coef = (float)(1.0 - 1.0 / tau_d);
  if (C <= 0) C = 1;
  if (HW <= 0) HW = 1;
  for (int64_t n = 0; n < N; ++n) {
    float v = v_in ? v_in[n] : (hard ? v_reset : 0.0f);
    const int64_t c = (n / HW) % C;
    for (int64_t t = 0; t < T; ++t) {
      const int64_t o = t * N + n;
      float x;
      switch (mode) {
        case 0: x = z[o]; break;
        case 1: x = z[o] * scale[c] + shift[c]; break;
        case 2: x = (z[o] * scale[c] + shift[c]) + z2[o]; break;
        case 3: x = z[o] + z2[o]; break;
        default: x = (z[o] + z2[o]) * scale[c] + shift[c]; break;
      }
      float h;
      if (hard) h = decay_input ? v + (x - (v - v_reset)) / tau : (v - (v - v_reset) / tau) + x;
      else h = decay_input ? v + (x - v) / tau : v * coef + x;
      if (h_seq) h_seq[o] = h;
      const float s = (h >= v_th) ? 1.0f : 0.0f;
      v = hard ? v_reset * s + (1.0f - s) * h : h - s * v_th;
      spike[o] = s;
    }
    if (v_out) v_out[n] = v;
  }
}

/* Prescan by brute force from the definition (catfuse/sparseflow/prescan.py
 * :153-189 _prescan_2d_impl, :57-109 _classify_tiles; tile geometry
 * sparse_conv2d_kernel.py:80-84): for tile (n, gh, gw), bit g is set iff
 * there is a valid output pixel (oh, ow) of the tile, a tap (kh, kw) with
 * (ih, iw) = (oh*s - p + kh, ow*s - p + kw) inside the image, and a channel
 * c of group g (c / gs == g) with |x[n][c][ih][iw]| > threshold.
 * tile_class: 0 ZERO (no bit), 2 DENSEISH (all num_groups bits), else 1. */
void oracle_prescan2d(const float* x, int64_t N, int64_t C, int64_t H, int64_t W, int64_t Ho,
                      int64_t Wo, int64_t ks, int64_t stride, int64_t pad, int64_t BH,
                      int64_t BW, int64_t gs, float threshold, int32_t* ag_mask,
                      int32_t* tile_class) {
  const int64_t GH = (Ho + BH - 1) / BH, GW = (Wo + BW - 1) / BW;
  const int64_t G = (C + gs - 1) / gs;
  const uint32_t all = G >= 32 ? 0xffffffffu : ((1u << G) - 1u);
  for (int64_t n = 0; n < N; ++n)
    for (int64_t gh = 0; gh < GH; ++gh)
      for (int64_t gw = 0; gw < GW; ++gw) {
        uint32_t m = 0;
        for (int64_t oh = gh * BH; oh < gh * BH + BH && oh < Ho; ++oh)
          for (int64_t ow = gw * BW; ow < gw * BW + BW && ow < Wo; ++ow)
            for (int64_t kh = 0; kh < ks; ++kh)
              for (int64_t kw = 0; kw < ks; ++kw) {
                const int64_t ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                for (int64_t c = 0; c < C; ++c)
                  if (fabsf(x[((n * C + c) * H + ih) * W + iw]) > threshold)
                    m |= 1u << (uint32_t)(c / gs);
              }
        const int64_t t = (n * GH + gh) * GW + gw;
        ag_mask[t] = (int32_t)m;
        tile_class[t] = m == 0 ? 0 : (m == all ? 2 : 1);
      }
}

/* Direct convolution in double (textbook definition), rounded to fp32 at
 * the end.  Used to pin the torch CPU convolution on tiny shapes.
 * x [N][Cin][H][W], w [Cout][Cin][KH][KW], y [N][Cout][Ho][Wo]. */
void oracle_conv2d_f64(const float* x, const float* w, float* y, int64_t N, int64_t Cin,
                       int64_t H, int64_t W, int64_t Cout, int64_t KH, int64_t KW,
                       int64_t stride, int64_t pad) {
  const int64_t Ho = (H + 2 * pad - KH) / stride + 1, Wo = (W + 2 * pad - KW) / stride + 1;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t co = 0; co < Cout; ++co)
      for (int64_t oh = 0; oh < Ho; ++oh)
        for (int64_t ow = 0; ow < Wo; ++ow) {
          double acc = 0.0;
          for (int64_t ci = 0; ci < Cin; ++ci)
            for (int64_t kh = 0; kh < KH; ++kh)
              for (int64_t kw = 0; kw < KW; ++kw) {
                const int64_t ih = oh * stride - pad + kh, iw = ow * stride - pad + kw;
                if (ih < 0 || ih >= H || iw < 0 || iw >= W) continue;
                acc += (double)x[((n * Cin + ci) * H + ih) * W + iw] *
                       (double)w[((co * Cin + ci) * KH + kh) * KW + kw];
              }
          y[((n * Cout + co) * Ho + oh) * Wo + ow] = (float)acc;
        }
}
