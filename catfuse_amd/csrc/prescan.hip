// SparseFlow prescan, spatial half: per-output-tile active-group bitmask and
// tile class from the per-pixel group bits produced by pack.hip.
//
// Definition (catfuse/sparseflow/prescan.py:153-189 _prescan_2d_impl and
// :57-109 _classify_tiles): bit g of tile (n, gh, gw) is set iff some input
// pixel inside the receptive field of some *valid* output pixel of the tile
// has a channel of group g with |x| > threshold.  max_pool2d pads with -inf,
// so out-of-image positions never contribute; ceil_mode tiles only contain
// output pixels < (Ho, Wo).  Class: ZERO (0) if no group, DENSEISH (2) if all
// NUM_GROUPS groups, SPARSE (1) otherwise.
//
// One wave64 per tile: lanes stride over the receptive-field rectangle and
// the OR is reduced with cross-lane shuffles.
#include "cf_common.h"

namespace {

__global__ __launch_bounds__(256) void prescan_tiles_kernel(
    const uint32_t* __restrict__ act, int64_t n_tiles, int H, int W, int Ho, int Wo, int ks,
    int stride, int pad, int BH, int BW, int GH, int GW, uint32_t all_ones,
    int32_t* __restrict__ ag_mask, int32_t* __restrict__ tile_class) {
  const int lane = threadIdx.x & 63;
  const int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= n_tiles) return;
  const int gw = (int)(tile % GW);
  const int gh = (int)((tile / GW) % GH);
  const int64_t n = tile / ((int64_t)GW * GH);
  const int oh0 = gh * BH, oh1 = min(oh0 + BH, Ho) - 1;
  const int ow0 = gw * BW, ow1 = min(ow0 + BW, Wo) - 1;
  const int ih0 = max(oh0 * stride - pad, 0), ih1 = min(oh1 * stride - pad + ks - 1, H - 1);
  const int iw0 = max(ow0 * stride - pad, 0), iw1 = min(ow1 * stride - pad + ks - 1, W - 1);
  const int rw = iw1 - iw0 + 1;
  const int cnt = (ih1 >= ih0 && rw > 0) ? (ih1 - ih0 + 1) * rw : 0;
  uint32_t m = 0;
  const uint32_t* a = act + n * (int64_t)H * W;
  const bool gaps = stride > ks;  // receptive fields do not tile the rectangle
  for (int i = lane; i < cnt; i += 64) {
    const int ih = ih0 + i / rw, iw = iw0 + i % rw;
    if (gaps && (((ih + pad) % stride) >= ks || ((iw + pad) % stride) >= ks)) continue;
    m |= a[(int64_t)ih * W + iw];
  }
  for (int off = 32; off > 0; off >>= 1) m |= (uint32_t)__shfl_xor((int)m, off, 64);
  if (lane == 0) {
    m &= all_ones;
    ag_mask[tile] = (int32_t)m;
    tile_class[tile] = (m == 0) ? 0 : ((m == all_ones) ? 2 : 1);
  }
}

}  // namespace

CF_API int cf_prescan_tiles(const uint32_t* act, int64_t NB, int64_t H, int64_t W, int64_t Ho,
                            int64_t Wo, int64_t kernel_size, int64_t stride, int64_t padding,
                            int64_t block_h, int64_t block_w, int64_t num_groups,
                            int32_t* ag_mask, int32_t* tile_class, void* stream) {
  if (!act || !ag_mask || !tile_class || NB < 0 || H <= 0 || W <= 0 || Ho <= 0 || Wo <= 0 ||
      kernel_size <= 0 || stride <= 0 || padding < 0 || block_h <= 0 || block_w <= 0 ||
      num_groups <= 0 || num_groups > 32)
    return (int)hipErrorInvalidValue;
  const int64_t GH = (Ho + block_h - 1) / block_h, GW = (Wo + block_w - 1) / block_w;
  const int64_t n_tiles = NB * GH * GW;
  if (n_tiles == 0) return 0;
  const uint32_t all_ones = num_groups == 32 ? 0xffffffffu : ((1u << num_groups) - 1u);
  hipLaunchKernelGGL(prescan_tiles_kernel, dim3(cf_blocks(n_tiles, 4)), dim3(256), 0,
                     (hipStream_t)stream, act, n_tiles, (int)H, (int)W, (int)Ho, (int)Wo,
                     (int)kernel_size, (int)stride, (int)padding, (int)block_h, (int)block_w,
                     (int)GH, (int)GW, all_ones, ag_mask, tile_class);
  return (int)hipGetLastError();
}
