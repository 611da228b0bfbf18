// Fused Conv -> BN -> LIF (and Conv -> BN -> z) as an implicit GEMM on the
// gfx950 matrix cores.
//
//   D[cout][pixel] = sum_k W[cout][k] * X[k][pixel],  k = (kh, kw, cin)
//
// * A operand (weights): fp32 weights split into two fp16 limbs
//   w*s_c = hi + lo (s_c a per-output-channel power of two that keeps
//   |w*s_c| < 2^14), packed fragment-major (cf_wfrag_index).  Both limbs are
//   multiplied into the same fp32 accumulator, so the contraction carries
//   ~22 significant weight bits (fp32-faithful up to accumulation order).
// * B operand (activations): fp16 NHWC [img][H][W][Cp] from pack.hip.  Spikes
//   (and SEW sums, avgpool quarters) are exact in fp16, so x*hi and x*lo are
//   exact fp32 products.
// * Tile: BM output channels x BN output pixels per 256-thread workgroup
//   (4 waves in a 2x2 grid, each wave BM/2 x BN/2 via
//   v_mfma_f32_32x32x16_f16); one K step = one filter tap x 32 channels,
//   staged through LDS with a two-stage register->LDS pipeline.
// * Time: the workgroup loops t = 0..T-1; the membrane potential of every
//   output element it owns stays in VGPRs across t (TimeBlock(T) +
//   StreamFuse(Conv, LIF) + StateCarry(LIF)), z never touches HBM.
// * Routing on the device: when a nonzero count is supplied, nnz == 0 runs
//   no K loop at all (StaticZero: z = beta), and in RECT mode a SparseFlow
//   route skips every 32-channel K chunk whose prescan group bits are clear
//   for the tile.  Skipped chunks contribute exact zeros, so every route
//   yields bit-identical results.
//
// Reference behaviour replaced: catfuse/implementations/dense_keep.py:97-155
// (BN-folded conv + lif_sequential), catfuse/sparseflow/streamfuse_kernel.py
// :32-187 (sparse fused conv+BN+LIF over all T),
// catfuse/sparseflow/fused_conv_bn_lif_kernel.py:63-335 (bitmask-gated
// conv+BN+LIF), catfuse/implementations/base.py:250-308 (StaticZero).
#include "cf_common.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int KC = 32;        // channels per K step
constexpr int LDK = KC + 8;   // padded LDS row (halves)

enum { EPI_LIF = 0, EPI_Z = 1, EPI_POOL = 2 };
// identity_mode: where a non-NULL identity tensor enters the epilogue.
//   ID_ADD_SPIKE: out = identity + spike   (SEW ADD after the LIF)
//   ID_ADD_Z    : z = BN(conv) + identity  (spiking ResNet: BN -> Add -> LIF)
enum { ID_ADD_SPIKE = 1, ID_ADD_Z = 2 };

struct ConvArgs {
  const _Float16* x;
  const _Float16* w;
  const float* alpha;
  const float* beta;
  const float* v_in;
  float* v_out;
  float* out;
  _Float16* out_nhwc;
  int cp_out;
  const float* identity;
  const _Float16* identity_nhwc;  // spike-valued identity as fp16 NHWC, or null
  int cp_id;
  int identity_mode;
  const int32_t* ag_mask;
  const unsigned long long* nnz;  // count block of the input (cf_count_read), or null
  unsigned long long* nz_out;     // count block of the output: workgroups that wrote a
                                  // nonzero value (cf_count_publish), or null
  const CfOutDesc* x_desc;        // descriptors of the input's and the identity's copies
  const CfOutDesc* id_desc;       // (nullable); the output's is set to "written" (this
  CfOutDesc* out_desc;            // kernel always writes its outputs)
  int64_t numel;
  double sparse_thr;
  int T, B, Cp, Cout, Coutp, H, W, Ho, Wo, KH, KW, stride, pad;
  int x_img_tstride;
  int GH, GW, TBH, TBW;
  int gs;
  int n_ptiles;
  LifParams lif;
};

__device__ __forceinline__ int device_route(const unsigned long long* nnz, int64_t numel,
                                            double thr) {
  if (!nnz) return CF_ROUTE_DENSE;
  const unsigned long long k = cf_count_read(nnz);
  if (k == 0) return CF_ROUTE_ZERO;
  return (1.0 - (double)k / (double)numel > thr) ? CF_ROUTE_SPARSE : CF_ROUTE_DENSE;
}

// Largest LIF tile keeps 64 accumulator + 64 membrane registers per lane;
// it gets the full 512-register budget (accumulators move to AGPRs).
template <int BM, int BN, int EPI>
constexpr int conv_min_blocks() { return (BM * BN >= 128 * 128 && EPI == 0) ? 1 : 2; }

template <int BM, int BN, bool RECT, int EPI>
__global__ __launch_bounds__(256, (conv_min_blocks<BM, BN, EPI>())) void conv_mfma_kernel(ConvArgs a) {
  constexpr int WM = BM / 2, WN = BN / 2, MB = WM / 32, NB = WN / 32;
  constexpr int AU = BM / 32;  // 16-byte A units per thread per K step
  constexpr int BU = BN / 64;  // 16-byte B units per thread per K step
  static_assert(MB >= 1 && NB >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) _Float16 As[2][2][BM][LDK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN][LDK];
  __shared__ uint8_t actlist[64];
  __shared__ int nact_sh;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int ptile = blockIdx.x;
  const int cout0 = blockIdx.y * BM;
  const int HoWo = a.Ho * a.Wo;
  const int KHW = a.KH * a.KW;
  const int nch = a.Cp / KC;

  // Output pixel p of this tile -> (image, oh, ow); false if outside.
  auto pixel_of = [&](int p, int& img, int& oh, int& ow) -> bool {
    if (RECT) {
      const int gw = ptile % a.GW;
      const int gh = (ptile / a.GW) % a.GH;
      img = ptile / (a.GW * a.GH);
      oh = gh * a.TBH + p / a.TBW;
      ow = gw * a.TBW + p % a.TBW;
      return oh < a.Ho && ow < a.Wo;
    } else {
      const int64_t g = (int64_t)ptile * BN + p;
      if (g >= (int64_t)a.B * HoWo) { img = 0; oh = 0; ow = 0; return false; }
      img = (int)(g / HoWo);
      const int rem = (int)(g % HoWo);
      oh = rem / a.Wo;
      ow = rem % a.Wo;
      return true;
    }
  };

  // B-load pixels owned by this thread.
  int b_img[BU], b_ih[BU], b_iw[BU];
#pragma unroll
  for (int i = 0; i < BU; ++i) {
    const int u = tid + 256 * i;
    int img, oh, ow;
    const bool ok = pixel_of(u >> 2, img, oh, ow);
    b_img[i] = ok ? img : -1;
    b_ih[i] = oh * a.stride - a.pad;
    b_iw[i] = ow * a.stride - a.pad;
  }
  // Epilogue pixels owned by this lane.
  int e_img[NB], e_off[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int img, oh, ow;
    const bool ok = pixel_of(wn * WN + nb * 32 + (lane & 31), img, oh, ow);
    e_img[nb] = ok ? img : -1;
    e_off[nb] = oh * a.Wo + ow;
  }

  // the input where its producer left the values (nullptr: all zero)
  const _Float16* const xsrc = cf_copy_source(a.x_desc, a.x);
  auto gload = [&](int t, int tap, int chunk, u32x4 (&ar)[AU], u32x4 (&br)[BU]) {
    const int kh = tap / a.KW, kw = tap - (tap / a.KW) * a.KW;
    const int c0 = chunk * KC;
#pragma unroll
    for (int i = 0; i < AU; ++i) {
      const int u = tid + 256 * i;
      const int limb = u / (BM * 4), row = (u >> 2) % BM, part = u & 3;
      ar[i] = *reinterpret_cast<const u32x4*>(
          a.w + cf_wfrag_index(limb, cout0 + row, tap, c0 + part * 8, a.Coutp, KHW, a.Cp));
    }
    const int img_base = t * a.x_img_tstride;
#pragma unroll
    for (int i = 0; i < BU; ++i) {
      const int part = (tid + 256 * i) & 3;
      const int ih = b_ih[i] + kh, iw = b_iw[i] + kw;
      const bool ok = b_img[i] >= 0 && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
      const size_t off =
          ok ? ((((size_t)(img_base + b_img[i]) * a.H + ih) * a.W + iw) * a.Cp + c0 + part * 8) : 0;
      const u32x4 val = *reinterpret_cast<const u32x4*>(xsrc + off);
      br[i] = ok ? val : (u32x4)(0u);
    }
  };
  auto lstore = [&](int stage, const u32x4 (&ar)[AU], const u32x4 (&br)[BU]) {
#pragma unroll
    for (int i = 0; i < AU; ++i) {
      const int u = tid + 256 * i;
      const int limb = u / (BM * 4), row = (u >> 2) % BM, part = u & 3;
      *reinterpret_cast<u32x4*>(&As[stage][limb][row][part * 8]) = ar[i];
    }
#pragma unroll
    for (int i = 0; i < BU; ++i) {
      const int u = tid + 256 * i;
      *reinterpret_cast<u32x4*>(&Bs[stage][u >> 2][(u & 3) * 8]) = br[i];
    }
  };

  f16v acc[MB][NB];
  auto compute = [&](int stage) {
#pragma unroll
    for (int ks = 0; ks < KC / 16; ++ks) {
      h8 ah[MB], al[MB], bb[NB];
      const int kof = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int row = wm * WM + mb * 32 + (lane & 31);
        ah[mb] = *reinterpret_cast<const h8*>(&As[stage][0][row][kof]);
        al[mb] = *reinterpret_cast<const h8*>(&As[stage][1][row][kof]);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        bb[nb] = *reinterpret_cast<const h8*>(&Bs[stage][wn * WN + nb * 32 + (lane & 31)][kof]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[mb], bb[nb], acc[mb][nb], 0, 0, 0);
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[mb], bb[nb], acc[mb][nb], 0, 0, 0);
        }
    }
  };

  float v[MB][NB][16];
  if (EPI == EPI_LIF) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int co = cout0 + wm * WM + mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          float v0 = lif_initial_v(a.lif);
          if (a.v_in && co < a.Cout && e_img[nb] >= 0)
            v0 = a.v_in[((size_t)e_img[nb] * a.Cout + co) * HoWo + e_off[nb]];
          v[mb][nb][r] = v0;
        }
  }

  const int route = xsrc == nullptr ? CF_ROUTE_ZERO : device_route(a.nnz, a.numel, a.sparse_thr);
  const _Float16* const id_nhwc =
      a.identity_nhwc != nullptr ? cf_copy_source(a.id_desc, a.identity_nhwc) : nullptr;
  if (a.out_desc && tid == 0 && blockIdx.x == 0 && blockIdx.y == 0) {
    a.out_desc->copy = CF_COPY_WRITTEN;
    a.out_desc->vstate = 0u;
    a.out_desc->alias = nullptr;
  }
  const int ntiles_t = a.n_ptiles;
  uint32_t anyw = 0u;  // OR of the bits of every output value this thread writes

  for (int t = 0; t < a.T; ++t) {
    int nact;
    if (RECT) {
      __syncthreads();
      if (tid == 0) {
        uint32_t m;
        if (route == CF_ROUTE_ZERO) m = 0u;
        else if (route == CF_ROUTE_DENSE) m = 0xffffffffu;
        else m = (uint32_t)a.ag_mask[(size_t)t * ntiles_t + ptile];
        int n = 0;
        for (int c = 0; c < nch; ++c) {
          const int g0 = (c * KC) / a.gs, g1 = (c * KC + KC - 1) / a.gs;
          bool on = false;
          for (int g = g0; g <= g1 && g < 32; ++g) on |= ((m >> g) & 1u) != 0u;
          if (on) actlist[n++] = (uint8_t)c;
        }
        nact_sh = n;
      }
      __syncthreads();
      nact = nact_sh;
    } else {
      nact = (route == CF_ROUTE_ZERO) ? 0 : nch;
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

    const int S = KHW * nact;
    if (S > 0) {
      int tap = 0, j = 0;
      u32x4 ar[AU], br[BU];
      gload(t, 0, RECT ? (int)actlist[0] : 0, ar, br);
      lstore(0, ar, br);
      __syncthreads();
      for (int s = 0; s < S; ++s) {
        int ntap = tap, nj = j + 1;
        if (nj == nact) { nj = 0; ++ntap; }
        const bool more = (s + 1) < S;
        if (more) gload(t, ntap, RECT ? (int)actlist[nj] : nj, ar, br);
        compute(s & 1);
        if (more) lstore((s + 1) & 1, ar, br);
        __syncthreads();
        tap = ntap;
        j = nj;
      }
    }

    // Epilogue: BN affine, then LIF (or z) per output element.
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int co = cout0 + wm * WM + mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (co >= a.Cout) {
          if (a.out_nhwc && co < a.cp_out)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              if (e_img[nb] >= 0)
                store_nhwc(a.out_nhwc, a.cp_out, (size_t)t * a.B + e_img[nb], HoWo, e_off[nb], co, 0.0f);
          continue;
        }
        const float al = a.alpha[co], be = a.beta[co];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          if (e_img[nb] < 0) continue;
          const size_t o = ((size_t)(t * a.B + e_img[nb]) * a.Cout + co) * HoWo + e_off[nb];
          float z = __builtin_fmaf(acc[mb][nb][r], al, be);  // BN (one rounding, as the halo kernel)
          if (a.identity && a.identity_mode == ID_ADD_Z) z = z + a.identity[o];
          float ov;
          if (EPI == EPI_Z) {
            ov = z;
          } else {
            float vv = lif_charge(v[mb][nb][r], z, a.lif);
            float sp = lif_fire_reset(vv, a.lif);
            v[mb][nb][r] = vv;
            if (id_nhwc)
              ov = (float)id_nhwc[((size_t)t * a.B + e_img[nb]) * HoWo * a.cp_id +
                                  (size_t)e_off[nb] * a.cp_id + co] + sp;
            else if (a.identity_nhwc)
              ov = sp;   // elided identity: all zero
            else
              ov = (a.identity && a.identity_mode == ID_ADD_SPIKE) ? a.identity[o] + sp : sp;
          }
          anyw |= __float_as_uint(ov);
          if (a.out) a.out[o] = ov;
          if (a.out_nhwc)
            store_nhwc(a.out_nhwc, a.cp_out, (size_t)t * a.B + e_img[nb], HoWo, e_off[nb], co, ov);
        }
      }
  }

  if (EPI == EPI_LIF && a.v_out) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int co = cout0 + wm * WM + mb * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (co < a.Cout && e_img[nb] >= 0)
            a.v_out[((size_t)e_img[nb] * a.Cout + co) * HoWo + e_off[nb]] = v[mb][nb][r];
        }
  }
  if (a.nz_out) {
    // magnitude bits only: -0.0 counts as zero
    __shared__ unsigned any_sh[4];
    const bool any = cf_wg_any((anyw & 0x7fffffffu) != 0u, any_sh);
    if (tid == 0) cf_count_publish(a.nz_out, any ? 1ull : 0ull, blockIdx.x + gridDim.x * blockIdx.y,
                                  gridDim.x * gridDim.y);
  }
}

// ---------------------------------------------------------------------------
// Weight packing: fp32 [Cout][Cin][KH][KW] -> fp16 hi/lo limbs (cf_wfrag_index)
// with per-channel power-of-two prescale, and the folded epilogue affine
//   alpha = bn_scale / s_c,   beta = bn_shift + bias * bn_scale.
// With w_packed == nullptr only alpha/beta are produced (s_c = 1).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_weights_kernel(
    const float* __restrict__ w, int Cout, int Cin, int KHW, int Cp,
    const float* __restrict__ bn_scale, const float* __restrict__ bn_shift,
    const float* __restrict__ bias, _Float16* __restrict__ wp, int Coutp,
    float* __restrict__ alpha, float* __restrict__ beta) {
  __shared__ float red[256];
  const int co = blockIdx.x, tid = threadIdx.x;
  const int K = Cin * KHW;
  const bool real = co < Cout;
  float m = 0.0f;
  if (real && wp)
    for (int k = tid; k < K; k += 256) m = fmaxf(m, fabsf(w[(size_t)co * K + k]));
  red[tid] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  m = red[0];
  float sc = 1.0f, inv = 1.0f;
  if (wp && m > 0.0f) {
    int e;
    frexpf(m, &e);                   // m < 2^e
    int sh = 14 - e;
    if (sh > 100) sh = 100;
    if (sh < -100) sh = -100;
    sc = ldexpf(1.0f, sh);
    inv = ldexpf(1.0f, -sh);
  }
  if (wp) {
    // fragment-major layout (cf_wfrag_index)
    for (int i = tid; i < KHW * Cp; i += 256) {
      const int tap = i / Cp, c = i % Cp;
      float ws = 0.0f;
      if (real && c < Cin) ws = w[((size_t)co * Cin + c) * KHW + tap] * sc;
      const _Float16 hi = (_Float16)ws;
      const _Float16 lo = (_Float16)(ws - (float)hi);
      wp[cf_wfrag_index(0, co, tap, c, Coutp, KHW, Cp)] = hi;
      wp[cf_wfrag_index(1, co, tap, c, Coutp, KHW, Cp)] = lo;
    }
  }
  if (tid == 0) {
    const float bs = (real && bn_scale) ? bn_scale[co] : 1.0f;
    const float bh = (real && bn_shift) ? bn_shift[co] : 0.0f;
    const float bi = (real && bias) ? bias[co] : 0.0f;
    alpha[co] = real ? bs * inv : 0.0f;
    beta[co] = real ? (bias ? bh + bi * bs : bh) : 0.0f;
  }
}

template <int BM, int BN, bool RECT, int EPI>
hipError_t launch_conv(const ConvArgs& a, int n_ptiles, hipStream_t st) {
  dim3 grid((unsigned)n_ptiles, (unsigned)(a.Coutp / BM));
  hipLaunchKernelGGL((conv_mfma_kernel<BM, BN, RECT, EPI>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <bool RECT, int EPI>
hipError_t pick_tiles(const ConvArgs& a, int BMsel, int BNsel, int n_ptiles, hipStream_t st) {
  if (BMsel == 128 && BNsel == 128) return launch_conv<128, 128, RECT, EPI>(a, n_ptiles, st);
  if (BMsel == 128 && BNsel == 64) return launch_conv<128, 64, RECT, EPI>(a, n_ptiles, st);
  if (BMsel == 64 && BNsel == 128) return launch_conv<64, 128, RECT, EPI>(a, n_ptiles, st);
  if (BMsel == 64 && BNsel == 64) return launch_conv<64, 64, RECT, EPI>(a, n_ptiles, st);
  return hipErrorInvalidValue;
}

}  // namespace

CF_API int cf_pack_conv_weights(const float* w, int64_t Cout, int64_t Cin, int64_t KH,
                                int64_t KW, int64_t Coutp, int64_t Cp, const float* bn_scale,
                                const float* bn_shift, const float* bias, void* w_packed,
                                float* alpha, float* beta, void* stream) {
  if (!w || !alpha || !beta || Cout <= 0 || Cin <= 0 || KH <= 0 || KW <= 0 || Coutp < Cout ||
      (w_packed && Cp < Cin))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_weights_kernel, dim3((unsigned)Coutp), dim3(256), 0,
                     (hipStream_t)stream, w, (int)Cout, (int)Cin, (int)(KH * KW), (int)Cp,
                     bn_scale, bn_shift, bias, (_Float16*)w_packed, (int)Coutp, alpha, beta);
  return (int)hipGetLastError();
}

CF_API int cf_conv_halo(const void* x, const void* w_packed, const float* alpha,
                        const float* beta, const float* v_in, float* v_out, float* out,
                        void* out_nhwc, int64_t cp_out,
                        const float* identity, const void* identity_nhwc, int64_t cp_id,
                        int identity_mode, const int32_t* ag_mask, const int32_t* tile_order,
                        const unsigned long long* nnz, unsigned long long* nz_out,
                        const void* x_desc, const void* id_desc, void* out_desc,
                        int bias_info, const unsigned long long* id_nnz,
                        int64_t numel, double sparse_threshold,
                        int64_t T, int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp, int64_t H,
                        int64_t W, int64_t Ho, int64_t Wo, int64_t ksize, int64_t stride,
                        int64_t pad, int64_t tile_h, int64_t tile_w, int64_t group_size,
                        int epilogue, double tau, double v_th, double v_reset, int hard_reset,
                        int decay_input, void* stream);

CF_API int cf_conv_mfma(const void* x, const void* w_packed, const float* alpha,
                        const float* beta, const float* v_in, float* v_out, float* out,
                        void* out_nhwc, int64_t cp_out,
                        const float* identity, const void* identity_nhwc, int64_t cp_id,
                        int identity_mode, const int32_t* ag_mask, const int32_t* tile_order,
                        const unsigned long long* nnz, unsigned long long* nz_out,
                        const void* x_desc, const void* id_desc, void* out_desc,
                        int bias_info, const unsigned long long* id_nnz,
                        int64_t numel, double sparse_threshold,
                        int64_t T, int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp, int64_t H,
                        int64_t W, int64_t Ho, int64_t Wo, int64_t KH, int64_t KW, int64_t stride,
                        int64_t pad, int64_t x_img_tstride, int64_t tile_h, int64_t tile_w,
                        int64_t group_size, int epilogue, double tau, double v_th,
                        double v_reset, int hard_reset, int decay_input, void* stream) {
  if (!x || !w_packed || !alpha || !beta || (!out && !out_nhwc)) return (int)hipErrorInvalidValue;
  if (T <= 0 || B <= 0 || Cp <= 0 || Cp % KC != 0 || Cout <= 0 || Coutp < Cout ||
      Coutp % 64 != 0 || H <= 0 || W <= 0 || Ho <= 0 || Wo <= 0 || KH <= 0 || KW <= 0 ||
      stride <= 0 || pad < 0 || x_img_tstride < 0)
    return (int)hipErrorInvalidValue;
  // EPI_POOL (BN -> AvgPool2d(2, 2) -> LIF) runs in the halo kernel only
  if (epilogue != EPI_LIF && epilogue != EPI_Z && epilogue != EPI_POOL)
    return (int)hipErrorInvalidValue;
  if (identity && identity_mode != ID_ADD_SPIKE && identity_mode != ID_ADD_Z)
    return (int)hipErrorInvalidValue;
  if (identity_nhwc && (identity_mode != ID_ADD_SPIKE || cp_id < Cout || cp_id % 4 != 0))
    return (int)hipErrorInvalidValue;
  if (out_nhwc && (cp_out < Cout || cp_out > Coutp)) return (int)hipErrorInvalidValue;
  if (Ho != (H + 2 * pad - KH) / stride + 1 || Wo != (W + 2 * pad - KW) / stride + 1)
    return (int)hipErrorInvalidValue;
  if ((bias_info & ~(CF_BIAS_SILENT | CF_BIAS_VCHAN)) != 0 || (bias_info && !out_desc))
    return (int)hipErrorInvalidValue;
  const bool rect = tile_h > 0 && tile_w > 0;
  // 3x3 convolutions and 1x1 convolutions over feature maps of at least
  // 4x4 (stride 1/2, pad <= 2, one time-major input) always take the
  // halo-staged kernel, whatever the route or epilogue, so every
  // implementation of a layer accumulates in the same order.  The choice
  // depends on the layer shape only.
  const bool k_ok = (KH == 3 && KW == 3) || (KH == 1 && KW == 1 && Ho >= 4 && Wo >= 4);
  const bool halo_ok = k_ok && (stride == 1 || stride == 2) && pad <= 2 &&
                       x_img_tstride == B && T * B * Cout * Ho * Wo <= INT32_MAX &&
                       (!rect || (tile_h == 8 && (tile_w == 8 ||
                                                  (tile_w == 16 && stride == 1 && KH == 3))));
  if (epilogue == EPI_POOL && !halo_ok) return (int)hipErrorInvalidValue;
  if (halo_ok) {
    const int64_t th = 8, tw = rect ? tile_w : 8;
    return cf_conv_halo(x, w_packed, alpha, beta, v_in, v_out, out, out_nhwc, cp_out, identity,
                        identity_nhwc, cp_id, identity_mode,
                        rect ? ag_mask : nullptr, rect ? tile_order : nullptr, nnz, nz_out,
                        x_desc, id_desc, out_desc, bias_info, id_nnz, numel, sparse_threshold, T, B, Cp, Cout,
                        Coutp, H, W, Ho, Wo, KH, stride, pad, th, tw, rect ? group_size : 0,
                        epilogue, tau, v_th, v_reset, hard_reset, decay_input, stream);
  }
  if (rect) {
    if (!(tile_h * tile_w == 64 || tile_h * tile_w == 128)) return (int)hipErrorInvalidValue;
    if (Cp / KC > 64 || group_size <= 0 || (Cp + group_size - 1) / group_size > 32)
      return (int)hipErrorInvalidValue;
    if (nnz && !ag_mask) return (int)hipErrorInvalidValue;
  }
  if (tile_order && !(rect && ag_mask)) return (int)hipErrorInvalidValue;
  // 32-bit index ranges used inside the kernel
  if (B * Ho * Wo > INT32_MAX || T * B > INT32_MAX || (T * x_img_tstride + B) * H * W > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  ConvArgs a;
  a.x = (const _Float16*)x;
  a.w = (const _Float16*)w_packed;
  a.alpha = alpha; a.beta = beta; a.v_in = v_in; a.v_out = v_out; a.out = out;
  a.out_nhwc = (_Float16*)out_nhwc; a.cp_out = (int)cp_out;
  a.identity = identity; a.identity_mode = identity_mode; a.ag_mask = ag_mask; a.nnz = nnz; a.nz_out = nz_out; a.numel = numel;
  a.x_desc = (const CfOutDesc*)x_desc; a.id_desc = (const CfOutDesc*)id_desc;
  a.out_desc = (CfOutDesc*)out_desc;
  a.identity_nhwc = (const _Float16*)identity_nhwc; a.cp_id = (int)cp_id;
  a.sparse_thr = sparse_threshold;
  a.T = (int)T; a.B = (int)B; a.Cp = (int)Cp; a.Cout = (int)Cout; a.Coutp = (int)Coutp;
  a.H = (int)H; a.W = (int)W; a.Ho = (int)Ho; a.Wo = (int)Wo; a.KH = (int)KH; a.KW = (int)KW;
  a.stride = (int)stride; a.pad = (int)pad; a.x_img_tstride = (int)x_img_tstride;
  a.gs = group_size > 0 ? (int)group_size : 32;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  const int BMsel = (Coutp % 128 == 0) ? 128 : 64;
  int BNsel, n_ptiles;
  if (rect) {
    a.TBH = (int)tile_h; a.TBW = (int)tile_w;
    a.GH = (int)((Ho + tile_h - 1) / tile_h);
    a.GW = (int)((Wo + tile_w - 1) / tile_w);
    BNsel = (int)(tile_h * tile_w);
    n_ptiles = (int)(B * a.GH * a.GW);
  } else {
    a.TBH = a.TBW = 0; a.GH = a.GW = 1;
    BNsel = 128;
    n_ptiles = (int)((B * Ho * Wo + BNsel - 1) / BNsel);
  }
  if (nz_out && (unsigned long long)n_ptiles * (Coutp / 64) >= CF_MAX_COUNT_WG)
    return (int)hipErrorInvalidValue;
  a.n_ptiles = n_ptiles;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (rect) e = epilogue == EPI_Z ? pick_tiles<true, EPI_Z>(a, BMsel, BNsel, n_ptiles, st)
                                  : pick_tiles<true, EPI_LIF>(a, BMsel, BNsel, n_ptiles, st);
  else e = epilogue == EPI_Z ? pick_tiles<false, EPI_Z>(a, BMsel, BNsel, n_ptiles, st)
                             : pick_tiles<false, EPI_LIF>(a, BMsel, BNsel, n_ptiles, st);
  return (int)e;
}
