// Fused network stem: Conv(KH x KW, stride 2 or 1) -> BN -> LIF ->
// MaxPool(3, 2, 1) on the matrix cores, for an analog image that is repeated
// over T (direct encoding: the convolution is evaluated once per image and
// its z feeds all T LIF steps, which is exact because z is the same at every
// step).  Stride 2: the SEW/Spiking-ResNet 7x7 stem; stride 1: the first
// stage of a Spikformer patch splitter (3x3 conv, then the pool).
//
// Replaces, for the SEW/Spiking-ResNet stem, the reference's DenseKeep
// conv1 -> bn1 -> sn1 (catfuse/implementations/dense_keep.py:97-155 through
// catfuse/patterns.py:237-387) followed by SpikingJelly's MaxPool2d, which
// the reference leaves unfused.  The maxpool of spikes is a bitwise OR of
// the spike trains in the window, so it is exact.
//
// Precision: the image is split into fp16 limbs x = xh + xl (xl = x - xh
// rounded to fp16) and the weights into w*s = wh + wl (s a power of two per
// channel, undone in alpha).  Each output accumulates, in fp32 on the
// MFMA, wh*xh + wl*xh + wh*xl over the filter rows; the dropped wl*xl term
// is below 2^-22 |w x| per product.
//
// Workgroup: one 8 x 7 tile of pooled pixels of one image and 64 output
// channels; the filter rows' weight fragments stream from L2 two rows ahead
// (141 VGPRs: three workgroups per CU).  It computes the 17 x 15 conv outputs under the tile's pooling
// windows (the border row/column is recomputed by the neighbouring tile),
// runs the LIF over T for each, keeps the spike train of each conv output as
// a T-bit word in LDS, ORs the words over each 3 x 3 window and writes the
// pooled spikes (fp32 NCHW and/or the fp16 NHWC copy the next fused conv
// reads), and publishes the output's count block when asked.  v_out holds
// the final membrane of the conv outputs each tile owns.  For the patch
// splitter's first stage it replaces models/spikformer_github.py:181-254
// (proj_conv, proj_bn, proj_lif, maxpool: four passes there).
//
// K layout: for filter row kh the 32 k-values are kw * 4 + c (kw < 8,
// c < 4), so one 16-byte LDS read gives a lane two neighbouring input pixels
// of all channels.  Staged input: [limb][row][col][4] fp16.
#include "cf_common.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Pooled tile 8 x 7: its pooling windows cover 17 x 15 = 255 conv outputs,
// eight MFMA column tiles with a single idle lane.
constexpr int PTH = 8, PTW = 7;            // pooled tile
constexpr int PRH = 2 * PTH + 1;           // conv output rows under the tile (17)
constexpr int PRW = 2 * PTW + 1;           // conv output columns (15)
constexpr int NPIX = PRH * PRW;            // 255
constexpr int NTILE = (NPIX + 31) / 32;    // 8 MFMA column tiles
constexpr int MAXKH = 7;
constexpr int KROW = 32;                   // k-values per filter row
// Staged input rows / columns under a tile for conv stride S (1 or 2):
// 23 x 22 or 39 x 36.
template <int S> constexpr int stem_rh() { return (PRH - 1) * S + MAXKH; }
template <int S> constexpr int stem_rw() { return (PRW - 1) * S + 8; }
constexpr int BMS = 64;                    // output channels per workgroup

// Spike-word row stride (in words) per conv output: an odd number of dwords,
// so the 32 pixels of a column tile land in distinct LDS banks.
template <typename SW>
constexpr int spike_ld() {
  return sizeof(SW) == 1 ? BMS + 4 : (sizeof(SW) == 2 ? BMS + 2 : BMS + 1);
}

struct StemArgs {
  const float* x;        // [B][Cin][H][W]
  const _Float16* w;     // [2][Coutp][KH][32]
  const float* alpha;
  const float* beta;
  const float* v_in;     // [B][Hc][Wc][Cout] (channels-last) or null
  float* v_out;          // [B][Hc][Wc][Cout] (channels-last) or null
  float* out;            // [T][B][Cout][Hp][Wp] or null
  _Float16* out_nhwc;    // [T*B][Hp][Wp][cp_out] or null
  int cp_out;
  int u8;                // out_nhwc holds one byte per channel
  uint32_t* status;
  unsigned long long* nz_out;   // count block of the pooled output, or null
  int T, B, Cin, Cout, Coutp, H, W, KH, pad, Hc, Wc, Hp, Wp, GHp, GWp;
  LifParams lif;
};

// Raw buffer resource over [base, base + bytes): loads beyond the range
// return zeros (gfx9 word 3).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t stem_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
constexpr uint32_t STEM_OOB = 0x80000000u;  // beyond every range used here

// LEAN: the SEW / Spiking-ResNet stem as the fused network runs it: a hard
// reset neuron from its initial state (no v_in) over T = 4 steps, a 7-row
// filter, every output channel real (Cout = Coutp), the NHWC copy as the
// only output (no fp32 spikes); the same operations on the same values as
// the general instantiation, without its run-time branches.
template <typename SW, int LM, int S, bool LEAN = false>
__global__ __launch_bounds__(256, sizeof(SW) <= 2 ? 3 : 1) void conv_stem_kernel(StemArgs a) {
  static_assert(!LEAN || (sizeof(SW) == 1 && (LM == LM_HARD0_DECAY_P2 || LM == LM_HARD_DECAY_P2)),
                "lean stem: one-byte spike words, hard reset");
  constexpr int SLD = spike_ld<SW>();
  constexpr int RH = stem_rh<S>(), RW = stem_rw<S>();
  __shared__ __attribute__((aligned(16))) _Float16 xs[2][RH * RW * 4];
  __shared__ unsigned any_sh[4];
  __shared__ __attribute__((aligned(16))) SW spk[NPIX * SLD];
  __shared__ __attribute__((aligned(16))) SW pooled[PTH * PTW * SLD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int mt = wave >> 1, nsel = wave & 1;
  // XCD-aware work order (workgroup L runs on XCD L % 8; each XCD takes a
  // contiguous range of work items, tile-major with the 64-channel blocks
  // adjacent): horizontally neighbouring tiles, whose 56-byte segments of
  // the fp32 state rows share cache lines and whose input patches overlap,
  // run on the same XCD and meet in its L2.
  const int ncb = a.Coutp / BMS;
  const int nwork = a.B * a.GHp * a.GWp * ncb;
  const int L = blockIdx.x, xcd = L & 7;
  const int work = xcd * (nwork >> 3) + min(xcd, nwork & 7) + (L >> 3);
  const int tile = work / ncb;
  const int gw = tile % a.GWp, gh = (tile / a.GWp) % a.GHp, b = tile / (a.GWp * a.GHp);
  const int ph0 = gh * PTH, pw0 = gw * PTW;
  const int y0 = 2 * ph0 - 1, x0 = 2 * pw0 - 1;  // conv output at local (0, 0)
  const int cout0 = (work - tile * ncb) * BMS;

  // Weight fragments of this wave's 32 output channels, one filter row at a
  // time from L2 (the next row's loaded while the current row's MFMAs run).
  const int wco = cout0 + mt * 32 + (lane & 31);
  const _Float16* wp0 = a.w + (size_t)wco * a.KH * KROW + 8 * (lane >> 5);
  const size_t wlimb = (size_t)a.Coutp * a.KH * KROW;
  auto load_w = [&](int kh, h8* dh, h8* dl) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      dh[ks] = *reinterpret_cast<const h8*>(wp0 + kh * KROW + ks * 16);
      dl[ks] = *reinterpret_cast<const h8*>(wp0 + wlimb + kh * KROW + ks * 16);
    }
  };

  // Stage the input rows/columns under the tile, split into fp16 limbs.
  // All loads of the thread are issued before the first conversion.
  {
    constexpr int NP = (RH * RW + 255) / 256;  // positions per thread
    const int ih0 = y0 * S - a.pad, iw0 = x0 * S - a.pad;
    const size_t plane = (size_t)a.H * a.W;
    const float* xb = a.x + (size_t)b * a.Cin * plane;
    float xv[NP][4];
    if constexpr (LEAN) {
      // buffer loads over the image's planes: positions outside the image
      // and channels >= Cin read zeros (the host bounds the image's bytes
      // below 2^31)
      const __amdgpu_buffer_rsrc_t xr = stem_rsrc(xb, (uint32_t)(a.Cin * plane * 4));
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int p = tid + 256 * i;
        const int ry = p / RW, rx = p % RW;
        const int ih = ih0 + ry, iw = iw0 + rx;
        const bool in = p < RH * RW && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
        const uint32_t o = in ? (uint32_t)((ih * a.W + iw) * 4) : STEM_OOB;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          xv[i][c] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
              xr, c < a.Cin ? o + (uint32_t)(c * plane * 4) : STEM_OOB, 0, 0));
      }
    } else {
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int p = tid + 256 * i;
        const int ry = p / RW, rx = p % RW;
        const int ih = ih0 + ry, iw = iw0 + rx;
        const bool in = p < RH * RW && ih >= 0 && ih < a.H && iw >= 0 && iw < a.W;
        const float* src = xb + (size_t)ih * a.W + iw;
#pragma unroll
        for (int c = 0; c < 4; ++c) xv[i][c] = (in && c < a.Cin) ? src[c * plane] : 0.0f;
      }
    }
    bool overflow = false;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int p = tid + 256 * i;
      h4 hi, lo;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float v = xv[i][c];
        overflow |= !(fabsf(v) <= 65504.0f);
        const _Float16 h = (_Float16)v;
        hi[c] = h;
        lo[c] = (_Float16)(v - (float)h);
      }
      if (p < RH * RW) {
        *reinterpret_cast<h4*>(&xs[0][p * 4]) = hi;
        *reinterpret_cast<h4*>(&xs[1][p * 4]) = lo;
      }
    }
    if (overflow && a.status) atomicOr(a.status, (uint32_t)CF_STATUS_FP16_RANGE);
  }
  __syncthreads();

  // Conv outputs: 10 column tiles x 2 channel tiles over 4 waves; wave
  // (mt, nsel) takes channel tile mt and column tiles nsel, nsel + 2, ...
  const int kof2 = 2 * (lane >> 5);  // first kw of this lane's 8 k-values (+4 per ks)
  const int cl0 = mt * 32 + 4 * (lane >> 5);  // channel of register r: cl0 + 8 * (r / 4) + r % 4
  const size_t vplane = (size_t)a.Hc * a.Wc;

  // BN coefficients of this lane's 16 channels (registers 4*q .. 4*q+3 hold
  // channels cl0 + 8q .. + 3), loaded once.
  float alr[16], ber[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int co = cout0 + cl0 + 8 * (r >> 2) + (r & 3);  // < Coutp: alpha/beta are padded
    alr[r] = a.alpha[co];
    ber[r] = a.beta[co];
  }
  // Membrane state of this image, channels-last ([Hc][Wc][Cout]: a conv
  // output's channels are contiguous, so a lane's four consecutive channels
  // are one 16-byte access): a uniform 64-bit base and 32-bit offsets.
  const float* vin_b = (!LEAN && a.v_in) ? a.v_in + (size_t)b * a.Cout * vplane : nullptr;
  float* vout_b = a.v_out ? a.v_out + (size_t)b * a.Cout * vplane : nullptr;
  const bool full_c = LEAN || cout0 + BMS <= a.Cout;
  const bool vec_v = LEAN || (full_c && a.Cout % 4 == 0);   // 16-byte state accesses

  // Epilogue of one column tile: BN, then the LIF over T with a constant z,
  // the 16 elements of the lane stepped together; spike trains -> LDS (four
  // consecutive channels' words per store).
  auto epilogue = [&](int nt, const f16v& acc) {
    const int n = nt * 32 + (lane & 31);
    const int nc = n < NPIX ? n : NPIX - 1;
    const int ly = nc / PRW, lx = nc % PRW;
    const int y = y0 + ly, x = x0 + lx;
    const bool valid = n < NPIX && y >= 0 && y < a.Hc && x >= 0 && x < a.Wc;
    const bool own = valid && ly >= 1 && lx >= 1;
    const unsigned vo = (unsigned)((y * a.Wc + x) * a.Cout + cout0 + cl0);
    float zr[16], vr[16];
    uint32_t bits[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      zr[r] = __builtin_fmaf(acc[r], alr[r], ber[r]);
      vr[r] = lif_initial_v(a.lif);
      bits[r] = 0u;
    }
    if (!LEAN && vin_b && valid) {
      if (vec_v) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 f = *reinterpret_cast<const float4*>(vin_b + vo + 8 * q);
          vr[4 * q] = f.x; vr[4 * q + 1] = f.y; vr[4 * q + 2] = f.z; vr[4 * q + 3] = f.w;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = 8 * (r >> 2) + (r & 3);
          if (cout0 + cl0 + dc < a.Cout) vr[r] = vin_b[vo + dc];
        }
      }
    }
    constexpr bool HARD = LM == LM_HARD0_DECAY_P2 || LM == LM_HARD_DECAY_P2;
    if (LEAN || (HARD && !vin_b && a.T == 4)) {
      // Hard reset from the initial state with a constant z: a reset puts v
      // back to the initial value bit for bit (+0 or v_reset; no state is
      // ever -0), so the trajectory restarts, and the spike train follows
      // from the reset-free charges u_1 .. u_4 (the same operations on the
      // same values as the stepped form): with k the first step where
      // u_k >= v_th, the neuron fires at steps k, 2k, ... and ends at
      // u_(4 mod k) (the initial value when that is 0).
      const float v0 = lif_initial_v(a.lif);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float u1 = lif_charge_m<LM>(v0, zr[r], a.lif);
        const float u2 = lif_charge_m<LM>(u1, zr[r], a.lif);
        const float u3 = lif_charge_m<LM>(u2, zr[r], a.lif);
        const float u4 = lif_charge_m<LM>(u3, zr[r], a.lif);
        const bool f1 = u1 >= a.lif.v_th, f2 = u2 >= a.lif.v_th, f3 = u3 >= a.lif.v_th,
                   f4 = u4 >= a.lif.v_th;
        bits[r] = f1 ? 15u : f2 ? 10u : f3 ? 4u : f4 ? 8u : 0u;
        vr[r] = (f1 || f2) ? v0 : f3 ? u1 : f4 ? v0 : u4;
        // the selects are made here, each element's compare masks dead
        // right after (left to the uses, sixteen elements' masks would be
        // live together and spill from the scalar registers)
        asm volatile("" : "+v"(bits[r]), "+v"(vr[r]));
      }
    } else {
      for (int t = 0; t < a.T; ++t) {
        const uint32_t tbit = 1u << t;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          vr[r] = lif_charge_m<LM>(vr[r], zr[r], a.lif);
          bits[r] |= lif_fire_reset_bit<LM>(vr[r], a.lif) ? tbit : 0u;
        }
      }
    }
    if (vout_b && own) {
      if (vec_v) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<float4*>(vout_b + vo + 8 * q) =
              make_float4(vr[4 * q], vr[4 * q + 1], vr[4 * q + 2], vr[4 * q + 3]);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = 8 * (r >> 2) + (r & 3);
          if (cout0 + cl0 + dc < a.Cout) vout_b[vo + dc] = vr[r];
        }
      }
    }
    if constexpr (LEAN) {
      // four channels' words (bytes) per 32-bit LDS store, all channels
      // real; invalid outputs hold zero words
      if (n < NPIX) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t w = bits[4 * q] | (bits[4 * q + 1] << 8) | (bits[4 * q + 2] << 16) |
                             (bits[4 * q + 3] << 24);
          *reinterpret_cast<uint32_t*>(&spk[n * SLD + cl0 + 8 * q]) = valid ? w : 0u;
        }
      }
    } else if (n < NPIX) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // channels cl0 + 8q .. + 3; channels >= Cout and invalid outputs
        // hold zero words
        SW w4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int dc = 8 * q + j;
          const bool ok = valid && (full_c || cout0 + cl0 + dc < a.Cout);
          w4[j] = ok ? (SW)bits[4 * q + j] : (SW)0;
        }
        SW* dst = &spk[n * SLD + cl0 + 8 * q];
        if constexpr (sizeof(SW) == 1) {
          *reinterpret_cast<uint32_t*>(dst) = (uint32_t)w4[0] | ((uint32_t)w4[1] << 8) |
                                              ((uint32_t)w4[2] << 16) | ((uint32_t)w4[3] << 24);
        } else if constexpr (sizeof(SW) == 2) {
          *reinterpret_cast<uint32_t*>(dst) = (uint32_t)w4[0] | ((uint32_t)w4[1] << 16);
          *reinterpret_cast<uint32_t*>(dst + 2) = (uint32_t)w4[2] | ((uint32_t)w4[3] << 16);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[j] = w4[j];
        }
      }
    }
  };
  auto tile_base = [&](int nt) {
    const int n = nt * 32 + (lane & 31);
    const int nc = n < NPIX ? n : NPIX - 1;  // keeps dead lanes' reads inside the tile
    return ((S * (nc / PRW)) * RW + S * (nc % PRW) + kof2) * 4;
  };

  // Column tiles nsel, nsel + 2, ... of this wave, two at a time so that two
  // independent accumulation chains share the matrix core.  Accumulation
  // order per output: filter row, 16-k half, then wh*xh, wl*xh, wh*xl.
  for (int nt = nsel; nt < NTILE; nt += 4) {
    const bool two = nt + 2 < NTILE;
    const int base0 = tile_base(nt), base1 = tile_base(two ? nt + 2 : nt);
    f16v acc0, acc1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      acc0[r] = 0.0f;
      acc1[r] = 0.0f;
    }
    // filter row kh's fragments in buffer kh % 3, loaded two rows ahead
    h8 wh[3][2], wl[3][2];   // [row % 3][ks]
    load_w(0, wh[0], wl[0]);
    if (LEAN || a.KH > 1) load_w(1, wh[1], wl[1]);
#pragma unroll
    for (int kh = 0; kh < MAXKH; ++kh) {
      if (!LEAN && kh >= a.KH) break;
      const int cb = kh % 3;
      if (kh + 2 < (LEAN ? MAXKH : a.KH)) load_w(kh + 2, wh[(kh + 2) % 3], wl[(kh + 2) % 3]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int o = (kh * RW + 4 * ks) * 4;
        const h8 xh0 = *reinterpret_cast<const h8*>(&xs[0][base0 + o]);
        const h8 xl0 = *reinterpret_cast<const h8*>(&xs[1][base0 + o]);
        const h8 xh1 = *reinterpret_cast<const h8*>(&xs[0][base1 + o]);
        const h8 xl1 = *reinterpret_cast<const h8*>(&xs[1][base1 + o]);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wh[cb][ks], xh0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wh[cb][ks], xh1, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wl[cb][ks], xh0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wl[cb][ks], xh1, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wh[cb][ks], xl0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wh[cb][ks], xl1, acc1, 0, 0, 0);
      }
    }
    epilogue(nt, acc0);
    if (two) epilogue(nt + 2, acc1);
  }
  __syncthreads();

  // MaxPool(3, 2, 1) of spikes = OR of the spike words in the window (rows
  // and columns outside the conv output hold zero words, and every window
  // has a valid position).
  constexpr int NPOOL = PTH * PTW;
  if constexpr (sizeof(SW) <= 2) {
    // four (uint8) or two (uint16) channels' words per 32-bit LDS access
    constexpr int CPW = 4 / sizeof(SW);  // channels per word access
    for (int i = tid; i < NPOOL * (BMS / CPW); i += 256) {
      const int cg = i % (BMS / CPW), pp = i / (BMS / CPW);
      const int py = pp / PTW, px = pp % PTW;
      uint32_t o = 0u;
#pragma unroll
      for (int dy = 0; dy < 3; ++dy)
#pragma unroll
        for (int dx = 0; dx < 3; ++dx)
          o |= *reinterpret_cast<const uint32_t*>(
              &spk[((2 * py + dy) * PRW + 2 * px + dx) * SLD + cg * CPW]);
      *reinterpret_cast<uint32_t*>(&pooled[pp * SLD + cg * CPW]) = o;
    }
  } else {
    for (int i = tid; i < NPOOL * BMS; i += 256) {
      const int cl = i % BMS, pp = i / BMS;
      const int py = pp / PTW, px = pp % PTW;
      SW o = 0;
#pragma unroll
      for (int dy = 0; dy < 3; ++dy)
#pragma unroll
        for (int dx = 0; dx < 3; ++dx) o |= spk[((2 * py + dy) * PRW + 2 * px + dx) * SLD + cl];
      pooled[pp * SLD + cl] = o;
    }
  }
  __syncthreads();

  const int HpWp = a.Hp * a.Wp;
  uint32_t anyw = 0u;   // OR of the spike words this thread writes out
  if (!LEAN && a.out) {
    // fp32 NCHW: consecutive threads write consecutive pooled pixels of a row.
    for (int i = tid; i < BMS * NPOOL; i += 256) {
      const int pp = i % NPOOL, cl = i / NPOOL;
      const int py = pp / PTW, px = pp % PTW;
      const int co = cout0 + cl, oh = ph0 + py, ow = pw0 + px;
      if (co >= a.Cout || oh >= a.Hp || ow >= a.Wp) continue;
      const uint32_t wd = pooled[pp * SLD + cl];
      anyw |= wd;
      float* dst = a.out + ((size_t)b * a.Cout + co) * HpWp + (size_t)oh * a.Wp + ow;
      const size_t tstep = (size_t)a.B * a.Cout * HpWp;
      for (int t = 0; t < a.T; ++t) dst[t * tstep] = (float)((wd >> t) & 1u);
    }
  }
  if constexpr (LEAN) {
    // NHWC copy, 8 channels of one pooled pixel per store: the pixel's two
    // words of four channels' spike bytes; at step t, m = (w >> t) &
    // 0x01010101 holds the four spikes as bytes (the one-byte copy as it
    // is), and each pair of them spread to the low bytes of two halves
    // (v_perm) times 0x3c00 is the pair of fp16 spikes.
    for (int i = tid; i < NPOOL * (BMS / 8); i += 256) {
      const int c8 = i % (BMS / 8), pp = i / (BMS / 8);
      const int py = pp / PTW, px = pp % PTW;
      const int oh = ph0 + py, ow = pw0 + px, co8 = cout0 + 8 * c8;
      if (oh >= a.Hp || ow >= a.Wp || co8 >= a.cp_out) continue;
      const uint32_t w0 = *reinterpret_cast<const uint32_t*>(&pooled[pp * SLD + 8 * c8]);
      const uint32_t w1 = *reinterpret_cast<const uint32_t*>(&pooled[pp * SLD + 8 * c8 + 4]);
      anyw |= w0 | w1;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const size_t e = (((size_t)t * a.B + b) * HpWp + (size_t)oh * a.Wp + ow) * a.cp_out + co8;
        const uint32_t m0 = (w0 >> t) & 0x01010101u, m1 = (w1 >> t) & 0x01010101u;
        if (a.u8) {
          *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(a.out_nhwc) + e) = make_uint2(m0, m1);
        } else {
          uint4 hv;
          hv.x = __builtin_amdgcn_perm(0u, m0, 0x0c010c00u) * 0x3c00u;
          hv.y = __builtin_amdgcn_perm(0u, m0, 0x0c030c02u) * 0x3c00u;
          hv.z = __builtin_amdgcn_perm(0u, m1, 0x0c010c00u) * 0x3c00u;
          hv.w = __builtin_amdgcn_perm(0u, m1, 0x0c030c02u) * 0x3c00u;
          *reinterpret_cast<uint4*>(a.out_nhwc + e) = hv;
        }
      }
    }
  } else if (a.out_nhwc) {
    // fp16 NHWC: 16 bytes = 8 channels of one pooled pixel per store.
    for (int i = tid; i < NPOOL * (BMS / 8); i += 256) {
      const int c8 = i % (BMS / 8), pp = i / (BMS / 8);
      const int py = pp / PTW, px = pp % PTW;
      const int oh = ph0 + py, ow = pw0 + px, co8 = cout0 + 8 * c8;
      if (oh >= a.Hp || ow >= a.Wp || co8 >= a.cp_out) continue;
      uint32_t wd[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        wd[j] = pooled[pp * SLD + 8 * c8 + j];
        anyw |= wd[j];   // channels >= Cout hold zero words
      }
      for (int t = 0; t < a.T; ++t) {
        const size_t e = (((size_t)t * a.B + b) * HpWp + (size_t)oh * a.Wp + ow) * a.cp_out + co8;
        if (a.u8) {
          // one byte per channel: 8 bytes
          uint32_t lo = 0u, hi = 0u;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            lo |= ((wd[j] >> t) & 1u) << (8 * j);
            hi |= ((wd[4 + j] >> t) & 1u) << (8 * j);
          }
          *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(a.out_nhwc) + e) = make_uint2(lo, hi);
        } else {
          h8 hv;
#pragma unroll
          for (int j = 0; j < 8; ++j) hv[j] = ((wd[j] >> t) & 1u) ? (_Float16)1.0f : (_Float16)0.0f;
          *reinterpret_cast<h8*>(a.out_nhwc + e) = hv;
        }
      }
    }
  }
  // the output's count block: workgroups that wrote a spike
  if (a.nz_out) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (tid == 0) cf_count_publish(a.nz_out, any ? 1ull : 0ull, (unsigned)L, gridDim.x);
  }
}

// Stem weight packing: fp32 [Cout][Cin][KH][KW] -> fp16 hi/lo
// [2][Coutp][KH][32] with k = kw * 4 + c (zero beyond KW, Cin), the
// per-channel power-of-two prescale s_c that keeps |w s| < 2^14, and
//   alpha = bn_scale / s_c,  beta = bn_shift + bias * bn_scale.
__global__ __launch_bounds__(256) void pack_stem_weights_kernel(
    const float* __restrict__ w, int Cout, int Cin, int KH, int KW,
    const float* __restrict__ bn_scale, const float* __restrict__ bn_shift,
    const float* __restrict__ bias, _Float16* __restrict__ wp, int Coutp,
    float* __restrict__ alpha, float* __restrict__ beta) {
  __shared__ float red[256];
  const int co = blockIdx.x, tid = threadIdx.x;
  const int K = Cin * KH * KW;
  const bool real = co < Cout;
  float m = 0.0f;
  if (real)
    for (int k = tid; k < K; k += 256) m = fmaxf(m, fabsf(w[(size_t)co * K + k]));
  red[tid] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
    __syncthreads();
  }
  m = red[0];
  float sc = 1.0f, inv = 1.0f;
  if (m > 0.0f) {
    int e;
    frexpf(m, &e);  // m < 2^e
    int sh = 14 - e;
    if (sh > 100) sh = 100;
    if (sh < -100) sh = -100;
    sc = ldexpf(1.0f, sh);
    inv = ldexpf(1.0f, -sh);
  }
  for (int i = tid; i < KH * KROW; i += 256) {
    const int kh = i / KROW, k = i % KROW, kw = k / 4, c = k % 4;
    float ws = 0.0f;
    if (real && kw < KW && c < Cin) ws = w[(((size_t)co * Cin + c) * KH + kh) * KW + kw] * sc;
    const _Float16 hi = (_Float16)ws;
    const _Float16 lo = (_Float16)(ws - (float)hi);
    wp[((size_t)co * KH + kh) * KROW + k] = hi;
    wp[(((size_t)Coutp + co) * KH + kh) * KROW + k] = lo;
  }
  if (tid == 0) {
    const float bs = (real && bn_scale) ? bn_scale[co] : 1.0f;
    const float bh = (real && bn_shift) ? bn_shift[co] : 0.0f;
    const float bi = (real && bias) ? bias[co] : 0.0f;
    alpha[co] = real ? bs * inv : 0.0f;
    beta[co] = real ? (bias ? bh + bi * bs : bh) : 0.0f;
  }
}

template <typename SW, int S>
void launch_stem(const StemArgs& a, int lm, dim3 grid, hipStream_t st) {
  if constexpr (sizeof(SW) == 1) {
    const bool lean = !a.v_in && !a.out && a.out_nhwc && a.Cout == a.Coutp && a.T == 4 &&
                      a.KH == MAXKH && (lm == LM_HARD0_DECAY_P2 || lm == LM_HARD_DECAY_P2) &&
                      (int64_t)a.Cin * a.H * a.W * 4 <= INT32_MAX;
    if (lean) {
      if (lm == LM_HARD0_DECAY_P2)
        hipLaunchKernelGGL((conv_stem_kernel<SW, LM_HARD0_DECAY_P2, S, true>), grid, dim3(256), 0,
                           st, a);
      else
        hipLaunchKernelGGL((conv_stem_kernel<SW, LM_HARD_DECAY_P2, S, true>), grid, dim3(256), 0,
                           st, a);
      return;
    }
  }
  if (lm == LM_HARD0_DECAY_P2)
    hipLaunchKernelGGL((conv_stem_kernel<SW, LM_HARD0_DECAY_P2, S>), grid, dim3(256), 0, st, a);
  else if (lm == LM_HARD_DECAY_P2)
    hipLaunchKernelGGL((conv_stem_kernel<SW, LM_HARD_DECAY_P2, S>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((conv_stem_kernel<SW, LM_GENERIC, S>), grid, dim3(256), 0, st, a);
}

template <int S>
void launch_stem_s(const StemArgs& a, int lm, dim3 grid, hipStream_t st) {
  if (a.T <= 8) launch_stem<uint8_t, S>(a, lm, grid, st);
  else if (a.T <= 16) launch_stem<uint16_t, S>(a, lm, grid, st);
  else launch_stem<uint32_t, S>(a, lm, grid, st);
}

}  // namespace

CF_API int cf_pack_stem_weights(const float* w, int64_t Cout, int64_t Cin, int64_t KH, int64_t KW,
                                int64_t Coutp, const float* bn_scale, const float* bn_shift,
                                const float* bias, void* w_stem, float* alpha, float* beta,
                                void* stream) {
  if (!w || !w_stem || !alpha || !beta || Cout <= 0 || Cin <= 0 || Cin > 4 || KH <= 0 ||
      KH > MAXKH || KW <= 0 || KW > 8 || Coutp < Cout || Coutp % BMS != 0)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(pack_stem_weights_kernel, dim3((unsigned)Coutp), dim3(256), 0,
                     (hipStream_t)stream, w, (int)Cout, (int)Cin, (int)KH, (int)KW, bn_scale,
                     bn_shift, bias, (_Float16*)w_stem, (int)Coutp, alpha, beta);
  return (int)hipGetLastError();
}

static int conv_stem(const float* x, const void* w_stem, const float* alpha,
                     const float* beta, const float* v_in, float* v_out,
                     float* out, void* out_nhwc, int64_t cp_out, uint32_t* status,
                     unsigned long long* nz_out,
                     int64_t T, int64_t B, int64_t Cin, int64_t Cout, int64_t Coutp,
                     int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t stride,
                     int64_t pad, int64_t pool_k, int64_t pool_stride,
                     int64_t pool_pad, double tau, double v_th, double v_reset,
                     int hard_reset, int decay_input, int u8, void* stream) {
  if (!x || !w_stem || !alpha || !beta || (!out && !out_nhwc)) return (int)hipErrorInvalidValue;
  if (T <= 0 || T > 32 || B <= 0 || Cin <= 0 || Cin > 4 || Cout <= 0 || Coutp < Cout ||
      Coutp % BMS != 0 || H <= 0 || W <= 0 || KH <= 0 || KH > MAXKH || KW <= 0 || KW > 8 ||
      (stride != 1 && stride != 2) || pad < 0)
    return (int)hipErrorInvalidValue;
  if (pool_k != 3 || pool_stride != 2 || pool_pad != 1) return (int)hipErrorInvalidValue;
  if (out_nhwc && (cp_out < Cout || cp_out > Coutp || cp_out % 8 != 0))
    return (int)hipErrorInvalidValue;
  const int64_t Hc = (H + 2 * pad - KH) / stride + 1, Wc = (W + 2 * pad - KW) / stride + 1;
  if (Hc <= 0 || Wc <= 0) return (int)hipErrorInvalidValue;
  const int64_t Hp = (Hc + 2 - 3) / 2 + 1, Wp = (Wc + 2 - 3) / 2 + 1;
  const int64_t GHp = (Hp + PTH - 1) / PTH, GWp = (Wp + PTW - 1) / PTW;
  if (B * GHp * GWp > INT32_MAX || T * B * Cout * Hp * Wp > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  if (nz_out && B * GHp * GWp * (Coutp / BMS) >= (int64_t)CF_MAX_COUNT_WG)
    return (int)hipErrorInvalidValue;
  StemArgs a;
  a.x = x; a.w = (const _Float16*)w_stem; a.alpha = alpha; a.beta = beta;
  a.v_in = v_in; a.v_out = v_out; a.out = out; a.out_nhwc = (_Float16*)out_nhwc;
  a.cp_out = (int)cp_out; a.status = status; a.nz_out = nz_out; a.u8 = u8 ? 1 : 0;
  a.T = (int)T; a.B = (int)B; a.Cin = (int)Cin; a.Cout = (int)Cout; a.Coutp = (int)Coutp;
  a.H = (int)H; a.W = (int)W; a.KH = (int)KH; a.pad = (int)pad;
  a.Hc = (int)Hc; a.Wc = (int)Wc; a.Hp = (int)Hp; a.Wp = (int)Wp;
  a.GHp = (int)GHp; a.GWp = (int)GWp;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  dim3 grid((unsigned)(B * GHp * GWp * (Coutp / BMS)));
  hipStream_t st = (hipStream_t)stream;
  const int lm = cf_lif_mode(a.lif);
  if (stride == 2) launch_stem_s<2>(a, lm, grid, st);
  else launch_stem_s<1>(a, lm, grid, st);
  return (int)hipGetLastError();
}

CF_API int cf_conv_stem_lif_maxpool(const float* x, const void* w_stem, const float* alpha,
                                    const float* beta, const float* v_in, float* v_out,
                                    float* out, void* out_nhwc, int64_t cp_out, uint32_t* status,
                                    unsigned long long* nz_out,
                                    int64_t T, int64_t B, int64_t Cin, int64_t Cout, int64_t Coutp,
                                    int64_t H, int64_t W, int64_t KH, int64_t KW, int64_t stride,
                                    int64_t pad, int64_t pool_k, int64_t pool_stride,
                                    int64_t pool_pad, double tau, double v_th, double v_reset,
                                    int hard_reset, int decay_input, void* stream) {
  return conv_stem(x, w_stem, alpha, beta, v_in, v_out, out, out_nhwc, cp_out, status, nz_out, T,
                   B, Cin, Cout, Coutp, H, W, KH, KW, stride, pad, pool_k, pool_stride, pool_pad,
                   tau, v_th, v_reset, hard_reset, decay_input, 0, stream);
}

CF_API int cf_conv_stem_lif_maxpool_u8(const float* x, const void* w_stem, const float* alpha,
                                       const float* beta, const float* v_in, float* v_out,
                                       float* out, void* out_copy, int64_t cp_out,
                                       uint32_t* status, unsigned long long* nz_out, int64_t T,
                                       int64_t B, int64_t Cin, int64_t Cout, int64_t Coutp,
                                       int64_t H, int64_t W, int64_t KH, int64_t KW,
                                       int64_t stride, int64_t pad, int64_t pool_k,
                                       int64_t pool_stride, int64_t pool_pad, double tau,
                                       double v_th, double v_reset, int hard_reset,
                                       int decay_input, void* stream) {
  return conv_stem(x, w_stem, alpha, beta, v_in, v_out, out, out_copy, cp_out, status, nz_out, T,
                   B, Cin, Cout, Coutp, H, W, KH, KW, stride, pad, pool_k, pool_stride, pool_pad,
                   tau, v_th, v_reset, hard_reset, decay_input, 1, stream);
}
