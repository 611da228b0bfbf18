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
      const float z = fmaf(acc[j], a.alpha[co], a.beta[co]);
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

// ---------------------------------------------------------------------------
// Conv(3 x 3, stride 1) -> BN -> LIF -> MaxPool2d(3, 2, 1) in one launch, for
// the analog first stage of a spiking patch splitter (Spikformer SPS conv0,
// models/spikformer_github.py:181-254: proj_conv -> proj_bn -> proj_lif ->
// maxpool), which otherwise writes the full-resolution spike map and reads it
// back for the pool.
//
// Workgroup: one PH x PW tile of pooled pixels of one image and COB output
// channels.  Its pooling windows cover (2 PH + 1) x (2 PW + 1) = 255 conv
// outputs, one per thread (the border row and column are recomputed by the
// neighbouring tile).  The staged input tile sits in LDS; the weights are
// read transposed ([Cin*9][Cout]) so each filter tap is one wave-uniform
// read of COB consecutive floats.  z is the same fp32 fused multiply-add
// chain as conv_direct_kernel's, so the spikes are bit-identical to
// conv_direct_kernel followed by the pool.  Per step each thread stores the
// COB spike bits of its conv output as one 64-bit word; a pooled output is
// the OR of the nine words of its window (the max of {0, 1} values; the
// pool's -inf padding never wins because every window holds a conv output).
// v_out keeps the final membrane of the conv outputs the tile owns (local
// rows and columns >= 1).
constexpr int DP_PH = 7, DP_PW = 8;                  // pooled tile
constexpr int DP_RH = 2 * DP_PH + 1, DP_RW = 2 * DP_PW + 1;   // 15 x 17 conv outputs
constexpr int DP_NPIX = DP_RH * DP_RW;               // 255
constexpr int DP_XH = DP_RH + 2, DP_XW = DP_RW + 2;  // staged input (3 x 3, stride 1)
constexpr int DP_MAXCIN = 4;

struct DirectPoolArgs {
  const float* x;      // [img][Cin][H][W], img = t*x_img_tstride + b
  const float* wt;     // [Cin*9][Cout]
  const float* alpha;
  const float* beta;
  const float* v_in;   // [B][Cout][Ho][Wo] or null
  float* v_out;        // [B][Cout][Ho][Wo] or null
  _Float16* out_nhwc;  // [T*B][Hp][Wp][cp_out]
  unsigned long long* nz_out;
  int cp_out;
  int T, B, Cin, Cout, H, W, Ho, Wo, pad, Hp, Wp, tiles_w, x_img_tstride;
  LifParams lif;
};

template <int COB, int LM>
__global__ __launch_bounds__(256) void conv_direct_pool_kernel(DirectPoolArgs a) {
  static_assert(COB % 8 == 0 && COB <= 64, "COB spike bits per 64-bit word");
  __shared__ float xs[DP_MAXCIN][DP_XH][DP_XW];
  __shared__ __attribute__((aligned(16))) float wsm[DP_MAXCIN * 9][COB];   // [tap][channel]
  __shared__ unsigned long long spk[2][256];
  __shared__ unsigned any_sh[4];
  const int tid = threadIdx.x;
  const int b = blockIdx.y, co0 = blockIdx.z * COB;
  const int ph0 = (blockIdx.x / a.tiles_w) * DP_PH, pw0 = (blockIdx.x % a.tiles_w) * DP_PW;
  const int cr0 = 2 * ph0 - 1, cc0 = 2 * pw0 - 1;    // conv output at local (0, 0)
  // thread 255 has no conv output; it computes a clamped duplicate, so the
  // conv loop has no divergent branch
  const int lr = min(tid / DP_RW, DP_RH - 1), lc = tid % DP_RW;
  const int cr = cr0 + lr, cc = cc0 + lc;
  const bool valid = tid < DP_NPIX && cr >= 0 && cr < a.Ho && cc >= 0 && cc < a.Wo;
  const bool dedupe = a.x_img_tstride == 0;
  const size_t HoWo = (size_t)a.Ho * a.Wo;
  const int nch = (co0 + COB == a.Cout ? a.cp_out - co0 : COB) / 8;   // 16-byte chunks written
  // membrane of this conv output, channel j at vbase + j * HoWo
  const size_t vbase = ((size_t)b * a.Cout + co0) * HoWo + (valid ? (size_t)cr * a.Wo + cc : 0);
  float z[COB], v[COB];
  if (a.v_in && valid) {
    const float* vin = a.v_in + vbase;
#pragma unroll
    for (int j = 0; j < COB; ++j) v[j] = vin[(size_t)j * HoWo];
  } else {
#pragma unroll
    for (int j = 0; j < COB; ++j) v[j] = lif_initial_v(a.lif);
  }
  uint32_t anyw = 0u;
  // this workgroup's filter slice; every lane reads the same weights, so
  // the conv reads them as LDS broadcasts (16 bytes, four channels, a read)
  for (int u = tid; u < a.Cin * 9 * COB; u += 256)
    wsm[u / COB][u % COB] = a.wt[(size_t)(u / COB) * a.Cout + co0 + u % COB];
  for (int t = 0; t < a.T; ++t) {
    if (t == 0 || !dedupe) {
      const int img = t * a.x_img_tstride + b;
      if (t > 0) __syncthreads();   // the previous step's reads of xs are complete
      const float* xb = a.x + (size_t)img * a.Cin * a.H * a.W;
      for (int u = tid; u < a.Cin * DP_XH * DP_XW; u += 256) {
        const int ci = u / (DP_XH * DP_XW), rr = (u / DP_XW) % DP_XH, c = u % DP_XW;
        const int ih = cr0 - a.pad + rr, iw = cc0 - a.pad + c;
        xs[ci][rr][c] = (ih >= 0 && ih < a.H && iw >= 0 && iw < a.W)
                            ? xb[((size_t)ci * a.H + ih) * a.W + iw] : 0.0f;
      }
      __syncthreads();
      float acc[COB];
#pragma unroll
      for (int j = 0; j < COB; ++j) acc[j] = 0.0f;
      for (int ci = 0; ci < a.Cin; ++ci) {
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
#pragma unroll
          for (int kw = 0; kw < 3; ++kw) {
            const float xv = xs[ci][lr + kh][lc + kw];
            const float4* wk = reinterpret_cast<const float4*>(wsm[(ci * 3 + kh) * 3 + kw]);
#pragma unroll
            for (int j = 0; j < COB; j += 4) {
              const float4 w4 = wk[j / 4];
              acc[j] = fmaf(xv, w4.x, acc[j]);
              acc[j + 1] = fmaf(xv, w4.y, acc[j + 1]);
              acc[j + 2] = fmaf(xv, w4.z, acc[j + 2]);
              acc[j + 3] = fmaf(xv, w4.w, acc[j + 3]);
            }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < COB; ++j) z[j] = fmaf(acc[j], a.alpha[co0 + j], a.beta[co0 + j]);
    }
    unsigned long long m = 0ull;
#pragma unroll
    for (int j = 0; j < COB; ++j) {
      float vv = lif_charge_m<LM>(v[j], z[j], a.lif);
      const bool f = lif_fire_reset_bit<LM>(vv, a.lif);
      v[j] = vv;
      m |= (f ? 1ull : 0ull) << j;
    }
    spk[t & 1][tid] = valid ? m : 0ull;
    __syncthreads();
    // pooled outputs: unit = (pooled pixel of the tile, 16-byte chunk)
    for (int u = tid; u < DP_PH * DP_PW * nch; u += 256) {
      const int pp = u / nch, ch = u % nch;
      const int py = pp / DP_PW, px = pp % DP_PW;
      const int gy = ph0 + py, gx = pw0 + px;
      if (gy >= a.Hp || gx >= a.Wp) continue;
      uint32_t bits = 0u;
      if (ch * 8 < COB) {
        unsigned long long w = 0ull;
#pragma unroll
        for (int dy = 0; dy < 3; ++dy)
#pragma unroll
          for (int dx = 0; dx < 3; ++dx) w |= spk[t & 1][(2 * py + dy) * DP_RW + 2 * px + dx];
        bits = (uint32_t)(w >> (ch * 8)) & 0xffu;
      }
      anyw |= bits;
      uint4 o;
      o.x = ((bits & 1u) ? 0x3c00u : 0u) | ((bits & 2u) ? 0x3c000000u : 0u);
      o.y = ((bits & 4u) ? 0x3c00u : 0u) | ((bits & 8u) ? 0x3c000000u : 0u);
      o.z = ((bits & 16u) ? 0x3c00u : 0u) | ((bits & 32u) ? 0x3c000000u : 0u);
      o.w = ((bits & 64u) ? 0x3c00u : 0u) | ((bits & 128u) ? 0x3c000000u : 0u);
      *reinterpret_cast<uint4*>(a.out_nhwc + (((size_t)t * a.B + b) * a.Hp + gy) * a.Wp * a.cp_out +
                                (size_t)gx * a.cp_out + co0 + ch * 8) = o;
    }
  }
  if (a.v_out && valid && lr >= 1 && lc >= 1) {
    float* vout = a.v_out + vbase;
#pragma unroll
    for (int j = 0; j < COB; ++j) vout[(size_t)j * HoWo] = v[j];
  }
  if (a.nz_out) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (tid == 0) {
      const unsigned nwg = gridDim.x * gridDim.y * gridDim.z;
      const unsigned wg = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
      cf_count_publish(a.nz_out, any ? 1ull : 0ull, wg, nwg);
    }
  }
}

// ---------------------------------------------------------------------------
// Conv(3 x 3, stride 1) -> BN -> AvgPool2d(2, 2) -> LIF in one launch, for
// an analog input (the first layer of a spiking VGG, whose conv is followed
// by a pool): the conv output is never written, the pooled spikes go out as
// the fp16 NHWC copy the next fused conv reads.
//
// Workgroup: one DA_P x DA_P tile of pooled pixels of one image and COB
// output channels, one pooled pixel a thread.  A thread computes the four
// conv outputs of its window with the fp32 fused multiply-add chain of
// conv_direct_kernel (taps in the order ci, kh, kw; then alpha, beta), sums
// them as ((z00 + z01) + z10) + z11 and scales by 0.25, the order of
// cf_avgpool2x2_lif, and runs the pooled neuron's LIF: the spikes equal
// cf_conv_direct (EPI_Z) followed by cf_avgpool2x2_lif bit for bit.  With a
// stride-0 time axis (direct encoding) the pooled input is computed once and
// feeds every step.  Input tile and filter slice sit in LDS (the filter
// transposed, [Cin*9][Cout]: one broadcast read per tap and four channels).
constexpr int DA_P = 16;                  // pooled tile
constexpr int DA_X = 2 * DA_P + 2;        // staged input rows / columns (34)

struct DirectAvgArgs {
  const float* x;      // [img][Cin][H][W], img = t*x_img_tstride + b
  const float* wt;     // [Cin*9][Cout]
  const float* alpha;
  const float* beta;
  const float* v_in;   // [B][Cout][Hp][Wp] or null
  float* v_out;        // [B][Cout][Hp][Wp] or null
  _Float16* out_nhwc;  // [T*B][Hp][Wp][cp_out]
  unsigned long long* nz_out;
  int cp_out;
  int T, B, Cin, Cout, H, W, pad, Hp, Wp, tiles_w, x_img_tstride;
  LifParams lif;
};

template <int COB, int LM>
__global__ __launch_bounds__(256) void conv_direct_avgpool_kernel(DirectAvgArgs a) {
  static_assert(COB % 8 == 0, "whole 16-byte chunks of spikes");
  __shared__ float xs[DP_MAXCIN][DA_X][DA_X];
  __shared__ __attribute__((aligned(16))) float wsm[DP_MAXCIN * 9][COB];   // [tap][channel]
  __shared__ unsigned any_sh[4];
  const int tid = threadIdx.x;
  const int b = blockIdx.y, co0 = blockIdx.z * COB;
  const int ph0 = (blockIdx.x / a.tiles_w) * DA_P, pw0 = (blockIdx.x % a.tiles_w) * DA_P;
  const int py = tid / DA_P, px = tid % DA_P;
  const int gy = ph0 + py, gx = pw0 + px;
  const bool valid = gy < a.Hp && gx < a.Wp;
  const bool dedupe = a.x_img_tstride == 0;
  const size_t HpWp = (size_t)a.Hp * a.Wp;
  // pooled membrane of this thread, channel j at vbase + j * HpWp
  const size_t vbase = ((size_t)b * a.Cout + co0) * HpWp + (valid ? (size_t)gy * a.Wp + gx : 0);
  float zp[COB], v[COB];
  if (a.v_in && valid) {
    const float* vin = a.v_in + vbase;
#pragma unroll
    for (int j = 0; j < COB; ++j) v[j] = vin[(size_t)j * HpWp];
  } else {
#pragma unroll
    for (int j = 0; j < COB; ++j) v[j] = lif_initial_v(a.lif);
  }
  // the copy's padding channels (Cout .. cp_out - 1) are written by the
  // workgroups of the last channel block
  const int nch = (co0 + COB == a.Cout ? a.cp_out - co0 : COB) / 8;
  uint32_t anyw = 0u;
  // this workgroup's filter slice (published by the staging barrier below)
  for (int u = tid; u < a.Cin * 9 * COB; u += 256)
    wsm[u / COB][u % COB] = a.wt[(size_t)(u / COB) * a.Cout + co0 + u % COB];
  const int r0 = 2 * ph0 - a.pad, c0 = 2 * pw0 - a.pad;   // input pixel at staged (0, 0)
  for (int t = 0; t < a.T; ++t) {
    if (t == 0 || !dedupe) {
      const int img = t * a.x_img_tstride + b;
      if (t > 0) __syncthreads();   // the previous step's reads of xs are complete
      const float* xb = a.x + (size_t)img * a.Cin * a.H * a.W;
      // every load of the tile in flight at once, then the LDS writes
      constexpr int NU = (DP_MAXCIN * DA_X * DA_X + 255) / 256;
      const int nst = a.Cin * DA_X * DA_X;
      float xv[NU];
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = tid + 256 * i;
        const int ci = u / (DA_X * DA_X), rr = (u / DA_X) % DA_X, c = u % DA_X;
        const int ih = r0 + rr, iw = c0 + c;
        xv[i] = (u < nst && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W)
                    ? xb[((size_t)ci * a.H + ih) * a.W + iw] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < NU; ++i) {
        const int u = tid + 256 * i;
        if (u < nst) (&xs[0][0][0])[u] = xv[i];
      }
      __syncthreads();
      // the four conv outputs of the window together: the 4 x 4 input patch
      // of each channel in registers, each tap's COB weights read once (LDS
      // broadcasts) for all four; every output keeps its own chain
      // (ci, kh, kw)
      float acc[4][COB];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < COB; ++j) acc[q][j] = 0.0f;
      for (int ci = 0; ci < a.Cin; ++ci) {
        // the channel's patch and all nine taps' weights requested together,
        // before the first product (one wait instead of one per tap)
        float pt[4][4];
        float4 wr[9][COB / 4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) pt[r][c] = xs[ci][2 * py + r][2 * px + c];
#pragma unroll
        for (int k = 0; k < 9; ++k)
#pragma unroll
          for (int j = 0; j < COB / 4; ++j)
            wr[k][j] = reinterpret_cast<const float4*>(wsm[ci * 9 + k])[j];
#pragma unroll
        for (int kh = 0; kh < 3; ++kh) {
#pragma unroll
          for (int kw = 0; kw < 3; ++kw) {
            float wv[COB];
#pragma unroll
            for (int j = 0; j < COB; j += 4) {
              const float4 w4 = wr[kh * 3 + kw][j / 4];
              wv[j] = w4.x;
              wv[j + 1] = w4.y;
              wv[j + 2] = w4.z;
              wv[j + 3] = w4.w;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float xv = pt[(q >> 1) + kh][(q & 1) + kw];
#pragma unroll
              for (int j = 0; j < COB; ++j) acc[q][j] = fmaf(xv, wv[j], acc[q][j]);
            }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < COB; ++j) {
        const float al = a.alpha[co0 + j], be = a.beta[co0 + j];
        zp[j] = fmaf(acc[0][j], al, be);
#pragma unroll
        for (int q = 1; q < 4; ++q) zp[j] = zp[j] + fmaf(acc[q][j], al, be);
      }
#pragma unroll
      for (int j = 0; j < COB; ++j) zp[j] = zp[j] * 0.25f;
    }
    uint32_t o[COB / 2];
#pragma unroll
    for (int j = 0; j < COB; ++j) {
      float vv = lif_charge_m<LM>(v[j], zp[j], a.lif);
      const bool f = lif_fire_reset_bit<LM>(vv, a.lif);
      v[j] = vv;
      const uint32_t h = f ? 0x3c00u : 0u;   // fp16 1.0
      if (j & 1) o[j / 2] |= h << 16;
      else o[j / 2] = h;
      anyw |= valid ? h : 0u;
    }
    if (valid) {
      _Float16* dst = a.out_nhwc + ((((size_t)t * a.B + b) * a.Hp + gy) * a.Wp + gx) * a.cp_out + co0;
      for (int ch = 0; ch < nch; ++ch) {
        uint4 w4 = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int k = 0; k < COB / 8; ++k)
          if (ch == k) w4 = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
        *reinterpret_cast<uint4*>(dst + ch * 8) = w4;
      }
    }
  }
  if (a.v_out && valid) {
    float* vout = a.v_out + vbase;
#pragma unroll
    for (int j = 0; j < COB; ++j) vout[(size_t)j * HpWp] = v[j];
  }
  if (a.nz_out) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (tid == 0) {
      const unsigned nwg = gridDim.x * gridDim.y * gridDim.z;
      const unsigned wg = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
      cf_count_publish(a.nz_out, any ? 1ull : 0ull, wg, nwg);
    }
  }
}

template <int LM>
hipError_t launch_direct_pool(const DirectPoolArgs& a, int cob, dim3 grid, hipStream_t st) {
  switch (cob) {
    case 64: hipLaunchKernelGGL((conv_direct_pool_kernel<64, LM>), grid, dim3(256), 0, st, a); break;
    case 48: hipLaunchKernelGGL((conv_direct_pool_kernel<48, LM>), grid, dim3(256), 0, st, a); break;
    case 32: hipLaunchKernelGGL((conv_direct_pool_kernel<32, LM>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((conv_direct_pool_kernel<16, LM>), grid, dim3(256), 0, st, a); break;
  }
  return hipGetLastError();
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

// Conv(3 x 3, stride 1, Cin <= 4) -> BN -> LIF -> MaxPool2d(3, 2, 1) of an
// analog input; writes only the pooled fp16 NHWC copy (channels Cout ..
// cp_out - 1 zero) and publishes its count block.
CF_API int cf_conv_direct_lif_maxpool(const float* x, const float* wt, const float* alpha,
                                      const float* beta, const float* v_in, float* v_out,
                                      void* out_nhwc, int64_t cp_out,
                                      unsigned long long* nz_out, int64_t T, int64_t B,
                                      int64_t Cin, int64_t Cout, int64_t H, int64_t W,
                                      int64_t pad, int64_t x_img_tstride, double tau,
                                      double v_th, double v_reset, int hard_reset,
                                      int decay_input, void* stream) {
  if (!x || !wt || !alpha || !beta || !out_nhwc || T <= 0 || B <= 0 || B > 65535 || Cin <= 0 ||
      Cin > DP_MAXCIN || Cout <= 0 || H <= 0 || W <= 0 || pad < 0 || pad > 2 ||
      x_img_tstride < 0 || cp_out < Cout || cp_out % 8 != 0)
    return (int)hipErrorInvalidValue;
  const int64_t Ho = H + 2 * pad - 2, Wo = W + 2 * pad - 2;
  if (Ho <= 0 || Wo <= 0) return (int)hipErrorInvalidValue;
  const int64_t Hp = (Ho - 1) / 2 + 1, Wp = (Wo - 1) / 2 + 1;
  const int64_t tiles_h = (Hp + DP_PH - 1) / DP_PH, tiles_w = (Wp + DP_PW - 1) / DP_PW;
  // 16 channels a workgroup: 87 VGPRs, five waves a SIMD to hide the
  // per-step barriers (wider groups hold z and v for more channels and run
  // two waves a SIMD)
  const int cob = Cout % 16 == 0 ? 16 : 0;
  if (cob == 0 || tiles_h * tiles_w > 0x7fffffff) return (int)hipErrorInvalidValue;
  const int64_t nwg = tiles_h * tiles_w * B * (Cout / cob);
  if (nz_out && nwg >= (int64_t)CF_MAX_COUNT_WG) return (int)hipErrorInvalidValue;
  DirectPoolArgs a;
  a.x = x; a.wt = wt; a.alpha = alpha; a.beta = beta; a.v_in = v_in; a.v_out = v_out;
  a.out_nhwc = (_Float16*)out_nhwc; a.nz_out = nz_out; a.cp_out = (int)cp_out;
  a.T = (int)T; a.B = (int)B; a.Cin = (int)Cin; a.Cout = (int)Cout; a.H = (int)H; a.W = (int)W;
  a.Ho = (int)Ho; a.Wo = (int)Wo; a.pad = (int)pad; a.Hp = (int)Hp; a.Wp = (int)Wp;
  a.tiles_w = (int)tiles_w; a.x_img_tstride = (int)x_img_tstride;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  const dim3 grid((unsigned)(tiles_h * tiles_w), (unsigned)B, (unsigned)(Cout / cob));
  const int lm = cf_lif_mode(a.lif);
  hipStream_t st = (hipStream_t)stream;
  if (lm == LM_HARD0_DECAY_P2) return (int)launch_direct_pool<LM_HARD0_DECAY_P2>(a, cob, grid, st);
  if (lm == LM_HARD_DECAY_P2) return (int)launch_direct_pool<LM_HARD_DECAY_P2>(a, cob, grid, st);
  return (int)launch_direct_pool<LM_GENERIC>(a, cob, grid, st);
}

// Conv(3 x 3, stride 1, Cin <= 4) -> BN -> AvgPool2d(2, 2) -> LIF of an
// analog input; writes the pooled fp16 NHWC copy (channels Cout .. cp_out - 1
// zero) and the pooled membrane, and publishes the output's count block.
CF_API int cf_conv_direct_avgpool_lif(const float* x, const float* wt, const float* alpha,
                                      const float* beta, const float* v_in, float* v_out,
                                      void* out_nhwc, int64_t cp_out,
                                      unsigned long long* nz_out, int64_t T, int64_t B,
                                      int64_t Cin, int64_t Cout, int64_t H, int64_t W,
                                      int64_t pad, int64_t x_img_tstride, double tau,
                                      double v_th, double v_reset, int hard_reset,
                                      int decay_input, void* stream) {
  if (!x || !wt || !alpha || !beta || !out_nhwc || T <= 0 || B <= 0 || B > 65535 || Cin <= 0 ||
      Cin > DP_MAXCIN || Cout <= 0 || Cout % 16 != 0 || H <= 0 || W <= 0 || pad < 0 ||
      pad > 2 || x_img_tstride < 0 || cp_out < Cout || cp_out % 8 != 0)
    return (int)hipErrorInvalidValue;
  const int64_t Ho = H + 2 * pad - 2, Wo = W + 2 * pad - 2;
  const int64_t Hp = Ho / 2, Wp = Wo / 2;
  if (Hp <= 0 || Wp <= 0) return (int)hipErrorInvalidValue;
  const int64_t tiles_h = (Hp + DA_P - 1) / DA_P, tiles_w = (Wp + DA_P - 1) / DA_P;
  // eight channels a workgroup: two waves a SIMD on a 32 x 32 image batch
  constexpr int cob = 8;
  if (tiles_h * tiles_w > 0x7fffffff) return (int)hipErrorInvalidValue;
  const int64_t nwg = tiles_h * tiles_w * B * (Cout / cob);
  if (nz_out && nwg >= (int64_t)CF_MAX_COUNT_WG) return (int)hipErrorInvalidValue;
  // 32-bit spatial indices; the copy's element offsets are 64-bit
  if (T * B * Cout * Hp * Wp > ((int64_t)1 << 40) || (int64_t)Cin * H * W > INT32_MAX)
    return (int)hipErrorInvalidValue;
  DirectAvgArgs a;
  a.x = x; a.wt = wt; a.alpha = alpha; a.beta = beta; a.v_in = v_in; a.v_out = v_out;
  a.out_nhwc = (_Float16*)out_nhwc; a.nz_out = nz_out; a.cp_out = (int)cp_out;
  a.T = (int)T; a.B = (int)B; a.Cin = (int)Cin; a.Cout = (int)Cout; a.H = (int)H; a.W = (int)W;
  a.pad = (int)pad; a.Hp = (int)Hp; a.Wp = (int)Wp;
  a.tiles_w = (int)tiles_w; a.x_img_tstride = (int)x_img_tstride;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  const dim3 grid((unsigned)(tiles_h * tiles_w), (unsigned)B, (unsigned)(Cout / cob));
  const int lm = cf_lif_mode(a.lif);
  hipStream_t st = (hipStream_t)stream;
  if (lm == LM_HARD0_DECAY_P2)
    hipLaunchKernelGGL((conv_direct_avgpool_kernel<cob, LM_HARD0_DECAY_P2>), grid, dim3(256), 0, st, a);
  else if (lm == LM_HARD_DECAY_P2)
    hipLaunchKernelGGL((conv_direct_avgpool_kernel<cob, LM_HARD_DECAY_P2>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((conv_direct_avgpool_kernel<cob, LM_GENERIC>), grid, dim3(256), 0, st, a);
  return (int)hipGetLastError();
}
