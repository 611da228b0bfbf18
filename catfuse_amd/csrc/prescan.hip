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

namespace {

// One workgroup: tiles active at some step (any bit of ag_mask[t][tile] for
// t < T) in ascending order, then the inactive ones in ascending order.
// Scanned in passes of 1024 tiles: per-wave ballots and popcounts give each
// tile its rank among the active (or inactive) tiles of the pass, offset by
// the counts of the earlier passes.  The first pass also sums the group
// bits active at some step of every tile for the dispatch score.
__global__ __launch_bounds__(1024) void compact_tiles_kernel(const int32_t* __restrict__ ag_mask,
                                                             int T, int ntiles, int num_groups,
                                                             double macs_per_tile, double tau,
                                                             double r_min,
                                                             int32_t* __restrict__ n_active,
                                                             int32_t* __restrict__ order) {
  __shared__ int wave_act[16];
  __shared__ unsigned long long wave_pop[16];
  __shared__ int base_sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // total active tiles first (the inactive ones go after them)
  int cnt = 0;
  unsigned long long pop = 0ull;
  for (int i = tid; i < ntiles; i += 1024) {
    uint32_t m = 0u;
    for (int t = 0; t < T; ++t) m |= (uint32_t)ag_mask[(size_t)t * ntiles + i];
    pop += (unsigned long long)__popc(m);
    cnt += m != 0u;
  }
  for (int off = 32; off > 0; off >>= 1) {
    cnt += __shfl_xor(cnt, off, 64);
    pop += __shfl_xor(pop, off, 64);
  }
  if (lane == 0) {
    wave_act[wave] = cnt;
    wave_pop[wave] = pop;
  }
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    unsigned long long ps = 0ull;
    for (int w = 0; w < 16; ++w) {
      s += wave_act[w];
      ps += wave_pop[w];
    }
    base_sh = s;
    // Dispatch score (catfuse/sparseflow/dispatch.py:868-1000): R = 1 - AGR,
    // S = R * macs_per_tile; SparseFlow iff R >= 0.99, or R >= r_min and
    // S > tau; else the conv takes the dense route (n_active = -1).  The
    // conv stages the steps of a tile together and skips a group's products
    // only where it is silent at all of them, so R here is the fraction of
    // (tile, group) pairs silent at every step (the reference counts
    // (image, tile, group) triples, its kernel running one image per tile).
    bool keep = true;
    if (tau >= 0.0) {
      const double total = (double)ntiles * (double)num_groups;
      const double R = 1.0 - (double)ps / total;
      keep = R >= 0.99 || (R >= r_min && R * macs_per_tile > tau);
    }
    *n_active = keep ? s : -1;
  }
  __syncthreads();
  const int total_active = base_sh;
  int act_before = 0;   // active tiles of earlier passes
  for (int p0 = 0; p0 < ntiles; p0 += 1024) {
    const int i = p0 + tid;
    uint32_t m = 0u;
    if (i < ntiles)
      for (int t = 0; t < T; ++t) m |= (uint32_t)ag_mask[(size_t)t * ntiles + i];
    const bool act = i < ntiles && m != 0u;
    const unsigned long long bal = __ballot(act ? 1 : 0);
    const int rank_w = __popcll(bal & ((1ull << lane) - 1ull));
    __syncthreads();   // wave_act of the previous pass has been read
    if (lane == 0) wave_act[wave] = __popcll(bal);
    __syncthreads();
    int before_w = 0, pass_act = 0;
    for (int w = 0; w < 16; ++w) {
      before_w += w < wave ? wave_act[w] : 0;
      pass_act += wave_act[w];
    }
    if (i < ntiles) {
      const int ra = act_before + before_w + rank_w;   // rank among active tiles
      order[act ? ra : total_active + (i - ra)] = i;
    }
    act_before += pass_act;
  }
}

}  // namespace

// Reference: catfuse/sparseflow/sparse_conv2d_kernel.py:113-123 (the
// active tiles of tile_class, host-synchronising torch.nonzero there).
CF_API int cf_compact_tiles(const int32_t* ag_mask, int64_t T, int64_t ntiles,
                            int64_t num_groups, double macs_per_tile, double tau, double r_min,
                            int32_t* order, void* stream) {
  if (!ag_mask || !order || T <= 0 || ntiles <= 0 || ntiles >= ((int64_t)1 << 30) ||
      T * ntiles >= ((int64_t)1 << 40) || num_groups <= 0 || num_groups > 32 ||
      !(macs_per_tile >= 0.0) || tau != tau || !(r_min <= 1.0))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(compact_tiles_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, ag_mask,
                     (int)T, (int)ntiles, (int)num_groups, macs_per_tile, tau, r_min, order,
                     order + 1);
  return (int)hipGetLastError();
}
