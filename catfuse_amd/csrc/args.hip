// Argument-block forms of the fused conv entry points: cf_conv_mfma_args and
// cf_conv_halo_pair_args take the blocks laid out in include/catfuse_amd.h
// and forward every field, unchanged and in parameter order, to
// cf_conv_mfma / cf_conv_halo_pair.  This file includes the C-ABI header
// itself (the kernels' shared header restates its route and count constants
// as enumerators), so it defines the export attribute on its own.
#include <hip/hip_runtime.h>

#include "catfuse_amd.h"

#define CF_ARGS_API extern "C" __attribute__((visibility("default")))

CF_ARGS_API int cf_conv_mfma_args(const CfConvMfmaArgs* a) {
  if (!a) return (int)hipErrorInvalidValue;
  return cf_conv_mfma(a->x, a->w_packed, a->alpha, a->beta, a->v_in, a->v_out, a->out,
                      a->out_nhwc, a->cp_out, a->identity, a->identity_nhwc, a->cp_id,
                      (int)a->identity_mode, a->ag_mask, a->tile_order, a->nnz, a->nz_out,
                      a->x_desc, a->id_desc, a->out_desc, (int)a->bias_info, a->id_nnz, a->numel,
                      a->sparse_threshold, a->T, a->B, a->Cp, a->Cout, a->Coutp, a->H, a->W,
                      a->Ho, a->Wo, a->KH, a->KW, a->stride, a->pad, a->x_img_tstride, a->tile_h,
                      a->tile_w, a->group_size, (int)a->epilogue, a->tau, a->v_th, a->v_reset,
                      (int)a->hard_reset, (int)a->decay_input, a->stream);
}

CF_ARGS_API int cf_conv_halo_pair_args(const CfConvHaloPairArgs* a) {
  if (!a) return (int)hipErrorInvalidValue;
  return cf_conv_halo_pair(a->x, a->nnz, a->x_desc, a->numel, a->T, a->B, a->Cp, a->H, a->W,
                           a->Ho, a->Wo, a->w_a, a->alpha_a, a->beta_a, a->v_in_a, a->v_out_a,
                           a->out_a, a->cp_out_a, a->nz_a, a->desc_a, (int)a->bias_info_a,
                           a->Cout_a, a->Coutp_a, a->pad_a, a->w_b, a->alpha_b, a->beta_b,
                           a->v_in_b, a->v_out_b, a->out_b, a->cp_out_b, a->nz_b, a->desc_b,
                           (int)a->bias_info_b, a->Cout_b, a->Coutp_b, a->pad_b, a->tau, a->v_th,
                           a->v_reset, (int)a->hard_reset, (int)a->decay_input, a->stream);
}

CF_ARGS_API int cf_conv_args_sizes(int64_t* sizes) {
  if (!sizes) return (int)hipErrorInvalidValue;
  sizes[0] = (int64_t)sizeof(CfConvMfmaArgs);
  sizes[1] = (int64_t)sizeof(CfConvHaloPairArgs);
  return 0;
}
