// Input staging for the MFMA conv path, plus the per-pixel half of the
// SparseFlow prescan and the StaticZero/SparseFlow/DenseKeep route count.
//
// One pass over the fp32 NCHW boundary tensor x[NB][C][H][W] produces:
//   xp   fp16 NHWC x[NB][H][W][Cp] (channels C..Cp-1 zero) — MFMA B operand
//   act  uint32 [NB][H][W]: bit g set iff |x[c]| > thr for some c in
//        channel group g (channels g*GS .. g*GS+GS-1)
//   nnz  count_nonzero(x), published in a count block (cf_count_publish)
//   status |= CF_STATUS_INEXACT_FP16 if some x is not exactly representable
//        in fp16 (the MFMA path multiplies fp16 x by split fp32 weights, so
//        exactness of x is what keeps the contraction fp32-faithful)
// The group-OR per pixel is the channel reduction of the reference prescan
// (catfuse/sparseflow/prescan.py:32-45 _groupwise_amax_last_dim, then
// `> threshold` at :184); the spatial (receptive field, tile) reduction is in
// prescan.hip.  HBM traffic: 4 B read + 2 B (xp) + 4/C B (act) per element.
#include "cf_common.h"

namespace {

constexpr int PX = 64;   // pixels per block
constexpr int CC = 32;   // channels per chunk

__global__ __launch_bounds__(256) void pack_kernel(
    const float* __restrict__ x, int64_t C, int64_t HW, int64_t Cp,
    _Float16* __restrict__ xp, uint32_t* __restrict__ act, int gs, float thr,
    unsigned long long* __restrict__ nnz, uint32_t* __restrict__ status) {
  __shared__ _Float16 tile[CC][PX + 2];
  __shared__ uint32_t bits_sh[4][PX];
  __shared__ unsigned int cnt_sh;
  __shared__ unsigned int inexact_sh;
  const int tid = threadIdx.x;
  const int64_t n = blockIdx.y;
  const int64_t hw0 = (int64_t)blockIdx.x * PX;
  const int px = tid % PX;       // pixel handled in the load phase
  const int cs = tid / PX;       // 0..3 channel sub-lane in the load phase
  const bool pvalid = (hw0 + px) < HW;
  if (tid == 0) { cnt_sh = 0; inexact_sh = 0; }
  uint32_t mybits = 0;
  unsigned int mycnt = 0;
  bool myinexact = false;
  const float* xn = x + n * C * HW + hw0 + px;
  __syncthreads();
  for (int64_t c0 = 0; c0 < Cp; c0 += CC) {
#pragma unroll
    for (int i = 0; i < CC / 4; ++i) {
      const int cl = cs + 4 * i;
      const int64_t c = c0 + cl;
      float v = 0.0f;
      if (pvalid && c < C) v = xn[c * HW];
      const _Float16 h = (_Float16)v;
      myinexact |= ((float)h != v);
      mycnt += (v != 0.0f) ? 1u : 0u;
      if (fabsf(v) > thr && c < C) mybits |= 1u << (unsigned)(c / gs);
      tile[cl][px] = h;
    }
    __syncthreads();
    if (xp) {
      // write phase: 4 threads per pixel, 8 channels (16 B) each
      const int wp = tid / 4, part = tid % 4;
      if (hw0 + wp < HW) {
        _Float16 o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = tile[part * 8 + j][wp];
        *reinterpret_cast<uint4*>(xp + ((n * HW + hw0 + wp) * Cp + c0 + part * 8)) =
            *reinterpret_cast<const uint4*>(o);
      }
    }
    __syncthreads();
  }
  if (act) {
    bits_sh[cs][px] = mybits;
    __syncthreads();
    if (tid < PX && pvalid)
      act[n * HW + hw0 + tid] = bits_sh[0][tid] | bits_sh[1][tid] | bits_sh[2][tid] | bits_sh[3][tid];
  }
  if (nnz) {
    // wave-level reduction, then one shared atomic per wave
    unsigned int c = mycnt;
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    if ((tid & 63) == 0) atomicAdd(&cnt_sh, c);
  }
  if (myinexact) atomicOr(&inexact_sh, 1u);
  __syncthreads();
  if (tid == 0) {
    if (nnz) cf_count_publish(nnz, cnt_sh, blockIdx.x + gridDim.x * blockIdx.y, gridDim.x * gridDim.y);
    if (status && inexact_sh) atomicOr(status, (uint32_t)CF_STATUS_INEXACT_FP16);
  }
}

// The same activity bits and nonzero count from an fp16 NHWC copy that a
// fused conv already wrote (xp[NPIX][Cp], channels >= C zero), so a
// SparseFlow layer whose input carries one needs no fp32 pass.  Sixteen
// lanes per pixel, each reading 16-byte chunks c8 = lane, lane + 16, ... (a
// pixel's channels are one contiguous run, so a 16-lane group reads 256
// contiguous bytes per load); group sizes are multiples of 8, so the 8
// channels of a chunk share one group, and the pixel's bits are OR-reduced
// over its 16 lanes.  Grid-stride over pixels; the count is published with
// one atomic per block.
// Activity bits and nonzero count of an fp16 NHWC copy.  LP lanes share a
// pixel (LP = Cp/8 capped at 16, a power of two: every lane of a wave busy),
// each reading 16-byte chunks of 8 channels; a thread takes two pixels per
// iteration (two loads in flight).  The tests work on the halves' bits: a
// half is nonzero iff its magnitude bits are (so -0 counts as zero, as
// v != 0.0f), and |v| > thr iff its magnitude bits exceed thr_mag (the bits
// of the largest fp16 magnitude <= thr; -1 when thr < 0) and are not a NaN
// (<= 0x7c00), the order of non-negative fp16 values being that of their
// bits.  Each chunk lies in one channel group (gs is a multiple of 8).
template <int LP>
__global__ __launch_bounds__(256) void scan_nhwc_kernel(
    const _Float16* __restrict__ xp, int64_t npix, int Cp, int C, uint32_t* __restrict__ act,
    int gs, int thr_mag, unsigned long long* __restrict__ nnz) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  constexpr int PPB = 256 / LP;   // pixels of a block per half-iteration
  __shared__ unsigned int cnt_sh;
  const int tid = threadIdx.x, sub = tid % LP;
  if (tid == 0) cnt_sh = 0;
  __syncthreads();
  unsigned int cnt = 0;
  const int nc8 = Cp / 8;
  for (int64_t p0 = (int64_t)blockIdx.x * 2 * PPB; p0 < npix; p0 += (int64_t)gridDim.x * 2 * PPB) {
    int64_t pp[2];
    uint32_t bits[2] = {0u, 0u};
#pragma unroll
    for (int u = 0; u < 2; ++u) pp[u] = p0 + u * PPB + tid / LP;
    for (int c8 = sub; c8 < nc8; c8 += LP) {
      u32x4 v[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
        v[u] = pp[u] < npix ? *reinterpret_cast<const u32x4*>(xp + pp[u] * Cp + c8 * 8)
                            : u32x4{0u, 0u, 0u, 0u};
      const int nreal = C - c8 * 8;   // real channels in the chunk (may be <= 0 or >= 8)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        bool any = false;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int lo = (int)(v[u][k] & 0x7fffu), hi = (int)((v[u][k] >> 16) & 0x7fffu);
          cnt += (lo != 0 ? 1u : 0u) + (hi != 0 ? 1u : 0u);
          any |= (lo > thr_mag && lo <= 0x7c00 && 2 * k < nreal) ||
                 (hi > thr_mag && hi <= 0x7c00 && 2 * k + 1 < nreal);
        }
        if (any) bits[u] |= 1u << (unsigned)((c8 * 8) / gs);
      }
    }
    // the LP lanes of a pixel share it, so this reduction stays in bounds
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int off = LP / 2; off > 0; off >>= 1) bits[u] |= __shfl_xor(bits[u], off, LP);
      if (act && pp[u] < npix && sub == 0) act[pp[u]] = bits[u];
    }
  }
  if (nnz) {
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    if ((tid & 63) == 0) atomicAdd(&cnt_sh, cnt);
    __syncthreads();
    if (tid == 0) cf_count_publish(nnz, cnt_sh, blockIdx.x, gridDim.x);
  }
}

// fp16 NHWC [NB][HW][cp] -> fp32 NCHW [NB][C][HW]: materialises the fp32
// view of a fused conv output that was kept only as its NHWC copy.  A block
// moves 64 pixels x 32 channels through LDS (reads: 64-byte runs per pixel;
// writes: 256-byte runs per channel).
// XT: the copy's element, fp16 or one byte per channel (uint8_t).
template <typename XT>
__global__ __launch_bounds__(256) void nhwc_to_nchw_kernel(
    const XT* __restrict__ xp, float* __restrict__ out, int64_t C, int64_t HW, int64_t cp) {
  __shared__ float tile[CC][PX + 1];
  const int tid = threadIdx.x;
  const int64_t n = blockIdx.z;
  const int64_t hw0 = (int64_t)blockIdx.x * PX;
  const int64_t c0 = (int64_t)blockIdx.y * CC;
  {
    // read: 4 threads per pixel, 8 channels (16 or 8 bytes) each
    const int px = tid / 4, part = tid % 4;
    typedef XT x8 __attribute__((ext_vector_type(8)));
    x8 v = {};
    if (hw0 + px < HW && c0 + part * 8 < cp)
      v = *reinterpret_cast<const x8*>(xp + ((n * HW + hw0 + px) * cp + c0 + part * 8));
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[part * 8 + j][px] = (float)v[j];
  }
  __syncthreads();
  // write: 64 consecutive pixels of one channel per 64 threads
  const int px = tid % PX;
#pragma unroll
  for (int i = 0; i < CC / 4; ++i) {
    const int cl = tid / PX + 4 * i;
    const int64_t c = c0 + cl;
    if (c < C && hw0 + px < HW) out[(n * C + c) * HW + hw0 + px] = tile[cl][px];
  }
}

// Global average pool of an fp16 NHWC copy xp [NB][HW][cp]: out[n][c] =
// (sum over the HW pixels of xp[n][p][c]) * factor, factor = float(1)/HW --
// torch's mean on the GPU (an fp32 sum, then a multiply by float(1)/count).
// The copies this reads hold integers (spikes, SEW sums), whose fp32 sum is
// exact in any order.  Block (n, 512-channel slice); a thread sums two
// adjacent channels (one 4-byte load per pixel, 1 KB per pixel per block).
template <typename XT>
__global__ __launch_bounds__(256) void global_avgpool_nhwc_kernel(
    const XT* __restrict__ xp, const CfOutDesc* desc, float* __restrict__ out, int64_t HW,
    int C, int cp, float factor) {
  // Workgroup: image n, 64 channels; thread (g, j) sums channels c, c + 1
  // (c = 64 * blockIdx.y + 2 j) over pixels g, g + 8, ...; the eight
  // partial sums meet in LDS.  The copy's values are small integers, so
  // every partial sum is exact and the order of the additions does not
  // change the result.
  typedef XT h2 __attribute__((ext_vector_type(2)));
  __shared__ float red[8][64];
  const int64_t n = blockIdx.x;
  const int g = (int)threadIdx.x >> 5, j = (int)threadIdx.x & 31;
  const int c = (int)blockIdx.y * 64 + 2 * j;
  const XT* base = cf_copy_source(desc, xp);   // nullptr: all zero
  float s0 = 0.0f, s1 = 0.0f;
  if (base != nullptr && c < C) {
    const XT* src = base + n * HW * cp + c;
#pragma unroll 4
    for (int64_t p = g; p < HW; p += 8) {
      const h2 v = *reinterpret_cast<const h2*>(src + p * cp);
      s0 += (float)v[0];
      s1 += (float)v[1];
    }
  }
  red[g][2 * j] = s0;
  red[g][2 * j + 1] = s1;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int cc = (int)blockIdx.y * 64 + (int)threadIdx.x;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) s += red[k][threadIdx.x];
    if (cc < C) out[n * C + cc] = s * factor;
  }
}

// Token-major fp32 [NB][P][C] (a transformer's [T, B, N, C] activations)
// -> its fp16 copy [NB][P][cp] (channels C..cp-1 zero), the nonzero count
// (published in a count block) and the exactness status: the staging of a
// fused linear's input, which the matrix-core kernels read as an NHWC image
// of P pixels.  One 8-channel chunk per thread and pass (grid-stride).
__global__ __launch_bounds__(256) void pack_tokens_kernel(
    const float* __restrict__ x, int64_t rows, int C, int cp, _Float16* __restrict__ xp,
    unsigned long long* __restrict__ nnz, uint32_t* __restrict__ status) {
  __shared__ unsigned int cnt_sh;
  __shared__ unsigned int inexact_sh;
  if (threadIdx.x == 0) { cnt_sh = 0; inexact_sh = 0; }
  __syncthreads();
  const int nc8 = cp / 8;
  unsigned int cnt = 0;
  bool inexact = false;
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < rows * nc8;
       u += (int64_t)gridDim.x * 256) {
    const int64_t r = u / nc8;
    const int c0 = (int)(u % nc8) * 8;
    _Float16 o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = (c0 + j < C) ? x[r * C + c0 + j] : 0.0f;
      const _Float16 hv = (_Float16)v;
      inexact |= ((float)hv != v);
      cnt += (v != 0.0f) ? 1u : 0u;
      o[j] = hv;
    }
    *reinterpret_cast<uint4*>(xp + r * cp + c0) = *reinterpret_cast<const uint4*>(o);
  }
  if (nnz) {
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    if ((threadIdx.x & 63) == 0) atomicAdd(&cnt_sh, cnt);
  }
  if (inexact) atomicOr(&inexact_sh, 1u);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (nnz) cf_count_publish(nnz, cnt_sh, blockIdx.x, gridDim.x);
    if (status && inexact_sh) atomicOr(status, (uint32_t)CF_STATUS_INEXACT_FP16);
  }
}

// fp16 [NB][P][cp] -> fp32 [NB][P][C]: the fp32 form of a token-major fused
// output kept only as its fp16 copy.
__global__ __launch_bounds__(256) void tokens_to_f32_kernel(
    const _Float16* __restrict__ xp, float* __restrict__ out, int64_t rows, int C, int cp) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < rows * C;
       e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / C;
    const int c = (int)(e % C);
    out[e] = (float)xp[r * cp + c];
  }
}

// A plain Linear (no neuron) over a token-major fused output kept only as
// its fp16 copy (a network's last classifier layer after a fused
// Linear-LIF): out[m][o] = bias[o] + sum_k x[m][k] * w[o][k] in fp32, x read
// through the copy's output descriptor (an all-zero copy gives the bias).
// One workgroup per row: its 256 threads take every 256th k (coalesced
// weight rows), LT_OB outputs a pass; the partial sums are reduced in a
// fixed tree (lanes, then waves in order), so the result is deterministic.
// Spike values are small integers; a zero skips its products (exact).
constexpr int LT_OB = 16;
__global__ __launch_bounds__(256) void linear_tokens_kernel(
    const _Float16* __restrict__ xp, const CfOutDesc* __restrict__ desc,
    const float* __restrict__ w, const float* __restrict__ bias, float* __restrict__ out,
    int K, int cp, int O) {
  __shared__ float red[4][LT_OB];
  const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const _Float16* xs = cf_copy_source(desc, xp);
  const _Float16* xr = xs != nullptr ? xs + (size_t)m * cp : nullptr;
  for (int o0 = 0; o0 < O; o0 += LT_OB) {
    float acc[LT_OB];
#pragma unroll
    for (int j = 0; j < LT_OB; ++j) acc[j] = 0.0f;
    if (xr != nullptr) {
      for (int k = tid; k < K; k += 256) {
        const float xv = (float)xr[k];
        if (xv != 0.0f) {
#pragma unroll
          for (int j = 0; j < LT_OB; ++j)
            if (o0 + j < O) acc[j] = fmaf(xv, w[(size_t)(o0 + j) * K + k], acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < LT_OB; ++j)
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) acc[j] += __shfl_xor(acc[j], off, 64);
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < LT_OB; ++j) red[wave][j] = acc[j];
    }
    __syncthreads();
    if (tid < LT_OB && o0 + tid < O) {
      const float s = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
      out[(size_t)m * O + o0 + tid] = bias != nullptr ? bias[o0 + tid] + s : s;
    }
    __syncthreads();   // red is rewritten by the next pass
  }
}

// Max pooling of an fp16 NHWC copy (the spikes a fused conv wrote):
// out[n][oh][ow][c] = max over the k x k window (stride s, padding p; padded
// positions ignored, as torch's max_pool2d) of xp[n][ih][iw][c].  The max of
// spike values is exact in fp16.  One 8-channel chunk of one output pixel
// per thread; the nonzero count of the output is published (count block).
__global__ __launch_bounds__(256) void maxpool_nhwc_kernel(
    const _Float16* __restrict__ xp_own, const CfOutDesc* __restrict__ in_desc,
    _Float16* __restrict__ out, CfOutDesc* __restrict__ out_desc, int64_t NB, int H, int W,
    int Ho, int Wo, int cp, int k, int s, int p, unsigned long long* __restrict__ nnz) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  __shared__ unsigned any_sh[4];
  // the input where its producer left it; an all-zero input pools to an
  // all-zero output, which is then recorded in out_desc instead of written
  const _Float16* const xp = cf_copy_source(in_desc, xp_own);
  if (xp == nullptr && out_desc != nullptr) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      if (nnz) nnz[1] = 0ull;
      out_desc->copy = CF_COPY_ZERO;
      out_desc->vstate = 0u;
      out_desc->alias = nullptr;
    }
    return;
  }
  if (out_desc != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    out_desc->copy = CF_COPY_WRITTEN;
    out_desc->vstate = 0u;
    out_desc->alias = nullptr;
  }
  const int nc8 = cp / 8;
  const int64_t units = NB * Ho * Wo * nc8;
  // unit decode in 32-bit arithmetic (the host keeps units below 2^31):
  // 64-bit divisions by run-time values cost far more than the pool itself
  const uint32_t HoWo = (uint32_t)(Ho * Wo);
  uint32_t anyw = 0u;
  for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u < (uint32_t)units; u += gridDim.x * 256u) {
    const uint32_t pix = u / (uint32_t)nc8;
    const int c8 = (int)(u - pix * (uint32_t)nc8);
    const uint32_t n32 = pix / HoWo, r = pix - n32 * HoWo;
    const int oh = (int)(r / (uint32_t)Wo), ow = (int)(r - (uint32_t)oh * (uint32_t)Wo);
    const int64_t n = n32;
    h8 m;
    bool first = true;
    for (int dy = 0; dy < k; ++dy) {
      const int ih = oh * s - p + dy;
      if (ih < 0 || ih >= H) continue;
      for (int dx = 0; dx < k; ++dx) {
        const int iw = ow * s - p + dx;
        if (iw < 0 || iw >= W) continue;
        const h8 v = xp != nullptr
                         ? *reinterpret_cast<const h8*>(xp + ((n * H + ih) * W + iw) * cp + c8 * 8)
                         : h8{};
        if (first) {
          m = v;
          first = false;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) m[j] = v[j] > m[j] ? v[j] : m[j];
        }
      }
    }
    const uint4 w = __builtin_bit_cast(uint4, m);
    anyw |= (w.x | w.y | w.z | w.w) & 0x7fff7fffu;
    *reinterpret_cast<h8*>(out + (size_t)pix * cp + c8 * 8) = m;
  }
  if (nnz) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (threadIdx.x == 0) cf_count_publish(nnz, any ? 1ull : 0ull, blockIdx.x, gridDim.x);
  }
}

__global__ void route_kernel(const unsigned long long* __restrict__ nnz, int64_t numel,
                             double sparse_threshold, int32_t* __restrict__ route) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const unsigned long long k = cf_count_read(nnz);
    int r;
    if (k == 0) r = CF_ROUTE_ZERO;
    else if (1.0 - (double)k / (double)numel > sparse_threshold) r = CF_ROUTE_SPARSE;
    else r = CF_ROUTE_DENSE;
    *route = r;
  }
}

__global__ void zero_u64(unsigned long long* p) { *p = 0ull; }

}  // namespace

CF_API int cf_pack_input(const float* x, int64_t NB, int64_t C, int64_t H, int64_t W,
                         int64_t Cp, void* xp, uint32_t* act, int group_size, float threshold,
                         unsigned long long* nnz, uint32_t* status, void* stream) {
  if (!x || NB < 0 || C <= 0 || H <= 0 || W <= 0) return (int)hipErrorInvalidValue;
  if (xp && (Cp < C || Cp % CC != 0)) return (int)hipErrorInvalidValue;
  if (!xp) Cp = ((C + CC - 1) / CC) * CC;
  if (act && (group_size <= 0 || (C + group_size - 1) / group_size > 32)) return (int)hipErrorInvalidValue;
  if (group_size <= 0) group_size = 32;
  if (NB == 0) return 0;
  if (NB > 65535) return (int)hipErrorInvalidValue;
  const int64_t HW = H * W;
  dim3 grid(cf_blocks(HW, PX), (unsigned)NB);
  if (nnz && (unsigned long long)grid.x * grid.y >= CF_MAX_COUNT_WG) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, (hipStream_t)stream, x, C, HW, Cp,
                     (_Float16*)xp, act, group_size, threshold, nnz, status);
  return (int)hipGetLastError();
}

CF_API int cf_scan_nhwc(const void* xp, int64_t NB, int64_t H, int64_t W, int64_t Cp, int64_t C,
                        uint32_t* act, int group_size, float threshold, unsigned long long* nnz,
                        void* stream) {
  if (!xp || NB < 0 || H <= 0 || W <= 0 || C <= 0 || Cp < C || Cp % 8 != 0)
    return (int)hipErrorInvalidValue;
  if (act && (group_size <= 0 || group_size % 8 != 0 || (C + group_size - 1) / group_size > 32))
    return (int)hipErrorInvalidValue;
  if (group_size <= 0) group_size = 32;
  if (threshold != threshold) return (int)hipErrorInvalidValue;   // NaN
  const int64_t npix = NB * H * W;
  if (npix == 0) return 0;
  // bits of the largest fp16 magnitude <= threshold (-1: every value exceeds it)
  int thr_mag = -1;
  if (threshold > 65504.0f) {
    thr_mag = 0x7c00;   // only a larger infinity would exceed it: none
    if (threshold < __builtin_huge_valf()) thr_mag = 0x7bff;
  } else if (threshold == 65504.0f) {
    thr_mag = 0x7bff;
  } else if (threshold >= 0.0f) {
    const _Float16 h = (_Float16)threshold;
    unsigned short b;
    __builtin_memcpy(&b, &h, 2);
    thr_mag = (int)(b & 0x7fffu);
    if ((float)h > threshold) --thr_mag;   // rounded up: the next smaller magnitude
  }
  const int nc8 = (int)(Cp / 8);
  const int lp = nc8 >= 16 ? 16 : (nc8 >= 8 ? 8 : (nc8 >= 4 ? 4 : (nc8 >= 2 ? 2 : 1)));
  const int64_t per_blk = 2 * (256 / lp);
  const int64_t nblk = (npix + per_blk - 1) / per_blk;
  const dim3 grid((unsigned)(nblk < 2048 ? nblk : 2048)), block(256);
  hipStream_t st = (hipStream_t)stream;
  const _Float16* x = (const _Float16*)xp;
  if (lp == 16)
    hipLaunchKernelGGL(scan_nhwc_kernel<16>, grid, block, 0, st, x, npix, (int)Cp, (int)C, act,
                       group_size, thr_mag, nnz);
  else if (lp == 8)
    hipLaunchKernelGGL(scan_nhwc_kernel<8>, grid, block, 0, st, x, npix, (int)Cp, (int)C, act,
                       group_size, thr_mag, nnz);
  else if (lp == 4)
    hipLaunchKernelGGL(scan_nhwc_kernel<4>, grid, block, 0, st, x, npix, (int)Cp, (int)C, act,
                       group_size, thr_mag, nnz);
  else if (lp == 2)
    hipLaunchKernelGGL(scan_nhwc_kernel<2>, grid, block, 0, st, x, npix, (int)Cp, (int)C, act,
                       group_size, thr_mag, nnz);
  else
    hipLaunchKernelGGL(scan_nhwc_kernel<1>, grid, block, 0, st, x, npix, (int)Cp, (int)C, act,
                       group_size, thr_mag, nnz);
  return (int)hipGetLastError();
}

template <typename XT>
static int nhwc_to_nchw(const void* xp, float* out, int64_t NB, int64_t C, int64_t H, int64_t W,
                        int64_t cp, void* stream) {
  if (!xp || !out || NB < 0 || C <= 0 || H <= 0 || W <= 0 || cp < C || cp % 8 != 0 || NB > 65535)
    return (int)hipErrorInvalidValue;
  if (NB == 0) return 0;
  const int64_t HW = H * W;
  dim3 grid(cf_blocks(HW, PX), (unsigned)((C + CC - 1) / CC), (unsigned)NB);
  hipLaunchKernelGGL(nhwc_to_nchw_kernel<XT>, grid, dim3(256), 0, (hipStream_t)stream,
                     (const XT*)xp, out, C, HW, cp);
  return (int)hipGetLastError();
}

CF_API int cf_nhwc_to_nchw(const void* xp, float* out, int64_t NB, int64_t C, int64_t H,
                           int64_t W, int64_t cp, void* stream) {
  return nhwc_to_nchw<_Float16>(xp, out, NB, C, H, W, cp, stream);
}

CF_API int cf_nhwc_to_nchw_u8(const void* xp, float* out, int64_t NB, int64_t C, int64_t H,
                              int64_t W, int64_t cp, void* stream) {
  return nhwc_to_nchw<uint8_t>(xp, out, NB, C, H, W, cp, stream);
}

template <typename XT>
static int global_avgpool_nhwc(const void* xp, const void* desc, float* out, int64_t NB,
                               int64_t HW, int64_t C, int64_t cp, void* stream) {
  if (!xp || !out || NB < 0 || HW <= 0 || C <= 0 || cp < C || cp % 8 != 0 || NB > INT32_MAX ||
      NB * HW * cp > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  if (NB == 0) return 0;
  const float factor = 1.0f / (float)HW;
  hipLaunchKernelGGL(global_avgpool_nhwc_kernel<XT>,
                     dim3((unsigned)NB, (unsigned)((C + 63) / 64)), dim3(256), 0,
                     (hipStream_t)stream, (const XT*)xp, (const CfOutDesc*)desc, out, HW, (int)C,
                     (int)cp, factor);
  return (int)hipGetLastError();
}

CF_API int cf_global_avgpool_nhwc(const void* xp, const void* desc, float* out, int64_t NB,
                                  int64_t HW, int64_t C, int64_t cp, void* stream) {
  return global_avgpool_nhwc<_Float16>(xp, desc, out, NB, HW, C, cp, stream);
}

CF_API int cf_global_avgpool_nhwc_u8(const void* xp, const void* desc, float* out, int64_t NB,
                                     int64_t HW, int64_t C, int64_t cp, void* stream) {
  return global_avgpool_nhwc<uint8_t>(xp, desc, out, NB, HW, C, cp, stream);
}

// One-byte copy -> fp16 copy of the same layout (n elements, a multiple of
// 8): for the readers that take fp16 copies only.  Every byte value is exact
// in fp16.
__global__ __launch_bounds__(256) void copy_u8_to_f16_kernel(const uint8_t* __restrict__ src,
                                                             _Float16* __restrict__ dst,
                                                             int64_t n8) {
  typedef uint8_t u8v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 h8v __attribute__((ext_vector_type(8)));
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * 256) {
    const u8v8 v = *reinterpret_cast<const u8v8*>(src + 8 * i);
    h8v h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = (_Float16)(float)v[j];
    *reinterpret_cast<h8v*>(dst + 8 * i) = h;
  }
}

CF_API int cf_copy_u8_to_f16(const void* src, void* dst, int64_t n, void* stream) {
  if (!src || !dst || n < 0 || n % 8 != 0) return (int)hipErrorInvalidValue;
  if (n == 0) return 0;
  const int64_t n8 = n / 8;
  const unsigned grid = (unsigned)((n8 + 255) / 256 < 8192 ? (n8 + 255) / 256 : 8192);
  hipLaunchKernelGGL(copy_u8_to_f16_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)src, (_Float16*)dst, n8);
  return (int)hipGetLastError();
}

CF_API int cf_pack_tokens(const float* x, int64_t rows, int64_t C, int64_t cp, void* xp,
                          unsigned long long* nnz, uint32_t* status, void* stream) {
  if (!x || !xp || rows < 0 || C <= 0 || cp < C || cp % 8 != 0 || rows * cp > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  const int64_t units = rows * (cp / 8);
  const unsigned grid = (unsigned)((units + 255) / 256 < 2048 ? (units + 255) / 256 : 2048);
  hipLaunchKernelGGL(pack_tokens_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, x, rows,
                     (int)C, (int)cp, (_Float16*)xp, nnz, status);
  return (int)hipGetLastError();
}

CF_API int cf_tokens_to_f32(const void* xp, float* out, int64_t rows, int64_t C, int64_t cp,
                            void* stream) {
  if (!xp || !out || rows < 0 || C <= 0 || cp < C || rows * cp > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  const int64_t n = rows * C;
  const unsigned grid = (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(tokens_to_f32_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const _Float16*)xp, out, rows, (int)C, (int)cp);
  return (int)hipGetLastError();
}

CF_API int cf_linear_tokens(const void* xp, const void* desc, const float* w, const float* bias,
                            float* out, int64_t M, int64_t K, int64_t cp, int64_t O,
                            void* stream) {
  if (!xp || !w || !out || M < 0 || M > INT32_MAX || K <= 0 || cp < K || O <= 0 ||
      O > 4096 || K * O > INT32_MAX || (int64_t)M * cp > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  if (M == 0) return 0;
  hipLaunchKernelGGL(linear_tokens_kernel, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream,
                     (const _Float16*)xp, (const CfOutDesc*)desc, w, bias, out, (int)K, (int)cp,
                     (int)O);
  return (int)hipGetLastError();
}

CF_API int cf_maxpool_nhwc(const void* xp, const void* in_desc, void* out, void* out_desc,
                           int64_t NB, int64_t H, int64_t W,
                           int64_t cp, int64_t kernel_size, int64_t stride, int64_t padding,
                           unsigned long long* nz_out, void* stream) {
  if (!xp || !out || NB < 0 || H <= 0 || W <= 0 || cp <= 0 || cp % 8 != 0 || kernel_size <= 0 ||
      stride <= 0 || padding < 0 || 2 * padding > kernel_size || NB * H * W * cp > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  const int64_t Ho = (H + 2 * padding - kernel_size) / stride + 1;
  const int64_t Wo = (W + 2 * padding - kernel_size) / stride + 1;
  if (Ho <= 0 || Wo <= 0) return (int)hipErrorInvalidValue;
  if (NB == 0) return 0;
  const int64_t units = NB * Ho * Wo * (cp / 8);
  if (units >= ((int64_t)1 << 31)) return (int)hipErrorInvalidValue;   // 32-bit unit indices
  // about one unit a thread (more loads in flight than a grid-stride loop)
  const unsigned grid = (unsigned)((units + 255) / 256 < 65536 ? (units + 255) / 256 : 65536);
  hipLaunchKernelGGL(maxpool_nhwc_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (const _Float16*)xp, (const CfOutDesc*)in_desc, (_Float16*)out,
                     (CfOutDesc*)out_desc, NB, (int)H, (int)W, (int)Ho, (int)Wo,
                     (int)cp, (int)kernel_size, (int)stride, (int)padding, nz_out);
  return (int)hipGetLastError();
}

// Route word from the nonzero count, exactly the host formula of
// catfuse/sparseflow/ops/st_fusion_conv_bn_lif.py:510-524 evaluated in double.
CF_API int cf_route_from_nnz(const unsigned long long* nnz, int64_t numel,
                             double sparse_threshold, int32_t* route, void* stream) {
  if (!nnz || !route || numel <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(route_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, nnz, numel,
                     sparse_threshold, route);
  return (int)hipGetLastError();
}

// Clears a 64-bit device counter with a kernel (graph-capture safe: no memset node).
CF_API int cf_zero_counter(unsigned long long* p, void* stream) {
  if (!p) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(zero_u64, dim3(1), dim3(1), 0, (hipStream_t)stream, p);
  return (int)hipGetLastError();
}

namespace {

// Fills a copy buffer its producer did not write (descriptor ZERO: zeros;
// ALIAS: the aliased copy's bytes); a written copy is left alone.  16-byte
// units, grid-stride.
__global__ __launch_bounds__(256) void resolve_copy_kernel(uint4* __restrict__ buf, int64_t n16,
                                                           const CfOutDesc* desc) {
  const uint32_t st = desc->copy;
  if (st != CF_COPY_ZERO && st != CF_COPY_ALIAS) return;
  const uint4* src = reinterpret_cast<const uint4*>(desc->alias);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * 256)
    buf[i] = st == CF_COPY_ALIAS ? src[i] : make_uint4(0u, 0u, 0u, 0u);
}

// v [B][C][HW] from the per-channel potentials when the descriptor says the
// producer kept the state per channel (vstate 1); otherwise v is left alone.
__global__ __launch_bounds__(256) void expand_state_kernel(float* __restrict__ v,
                                                           const float* __restrict__ v_chan,
                                                           const CfOutDesc* desc, int64_t n,
                                                           int C, int64_t HW) {
  if (desc->vstate != 1u) return;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    v[i] = v_chan[(int)((i / HW) % C)];
}

}  // namespace

CF_API int cf_resolve_copy(void* buf, int64_t bytes, const void* desc, void* stream) {
  if (!buf || !desc || bytes < 0 || bytes % 16 != 0 || ((uintptr_t)buf & 15) != 0)
    return (int)hipErrorInvalidValue;
  if (bytes == 0) return 0;
  const int64_t n16 = bytes / 16;
  const unsigned nb = cf_blocks(n16, 256), grid = nb < 2048u ? nb : 2048u;
  hipLaunchKernelGGL(resolve_copy_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream,
                     (uint4*)buf, n16, (const CfOutDesc*)desc);
  return (int)hipGetLastError();
}

CF_API int cf_expand_state(float* v, const float* v_chan, const void* desc, int64_t B, int64_t C,
                           int64_t HW, void* stream) {
  if (!v || !v_chan || !desc || B < 0 || C <= 0 || HW <= 0 || C > INT32_MAX)
    return (int)hipErrorInvalidValue;
  const int64_t n = B * C * HW;
  if (n == 0) return 0;
  const unsigned nb = cf_blocks(n, 256), grid = nb < 2048u ? nb : 2048u;
  hipLaunchKernelGGL(expand_state_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, v,
                     v_chan, (const CfOutDesc*)desc, n, (int)C, HW);
  return (int)hipGetLastError();
}
