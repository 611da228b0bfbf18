// Fused 3x3 Conv -> BN -> LIF on the matrix cores with the input halo staged
// in LDS and the time axis inside the tile.
//
// Workgroup tile: BM output channels x (TH x TW) output pixels of one image,
// for a block of up to TB = 4 time steps at once (2 for stride-2 3x3).  For every 32-channel
// chunk the workgroup stages the input halo of its tile for all time steps
// of the block in LDS ([t][RH][RW][32 ch], fp16, RH = (TH-1)*S + 3), then
// runs the 9 taps from LDS: each weight fragment (fp16 hi/lo limbs, loaded
// once per tap from L2 as one coalesced 1 KB access, one tap ahead) feeds
// the MFMAs of every time step.
// Activations are therefore read from L2 once per chunk instead of once per
// tap, and weights once per tap instead of once per tap and time step.
// When the K loop of a time block is complete the epilogue applies BN and
// the LIF for t = 0..TB-1 in order, with v in VGPRs across time blocks.
//
// Tiles are the SparseFlow prescan tiles (8x8 / 8x16), so the same kernel
// serves the SparseFlow route: a chunk is skipped for time step t when the
// tile's group bits for t are clear, and a chunk inactive at every step of
// the block is not even staged.  Routes are decided on the device from the
// nonzero count and are bit-identical (skipped chunks contribute zeros,
// and the accumulation order of the remaining ones is unchanged).
//
// Accumulation order per output element: chunk-major, then tap, then the
// two 16-channel halves, hi limb then lo limb.
#include "cf_common.h"

#include <stdlib.h>

#include <type_traits>

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Sixteen zero bytes in device memory: out-of-range halo units load from
// here, so a loaded register never needs a select that would force the
// wave to wait for the load before the taps run.
__device__ __attribute__((aligned(16))) u32x4 g_halo_zero;

// Returns x unchanged, hidden from the optimiser: per-element addresses
// derived from it are recomputed where they are used instead of being kept
// live (in registers or scratch) across the K loop.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <typename P>
__device__ __forceinline__ P* opaque_ptr(P* p) {
  asm volatile("" : "+s"(p));
  return p;
}

constexpr int KC = 32;       // channels per chunk
#ifndef CF_HALO_LDK
#define CF_HALO_LDK (KC + 8)
#endif
constexpr int LDK = CF_HALO_LDK;  // padded halo pixel (halves)
// Time steps per block: 4, or 2 for stride-2 3x3 tiles, whose 17 x 17 input
// halo would otherwise hold a workgroup per CU on LDS alone.
template <int S, int K>
constexpr int halo_tb() {
  return (S == 2 && K == 3) ? 2 : 4;
}

enum { EPI_LIF = 0, EPI_Z = 1 };
enum { ID_ADD_SPIKE = 1, ID_ADD_Z = 2 };

struct HaloArgs {
  const _Float16* x;        // [T*B][H][W][Cp]
  const _Float16* w;        // fragment-major limbs (cf_wfrag_index)
  const float* alpha;
  const float* beta;
  const float* v_in;
  float* v_out;
  float* out;               // [T][B][Cout][Ho][Wo]
  _Float16* out_nhwc;       // [T*B][Ho][Wo][cp_out] or null
  int cp_out;
  const float* identity;
  const _Float16* identity_nhwc;  // [T*B][Ho][Wo][cp_id] spike-valued identity, or null
  int cp_id;
  int identity_mode;
  const int32_t* ag_mask;   // [T][B*GH*GW]
  const unsigned long long* nnz;
  int64_t numel;
  double sparse_thr;
  int T, B, Cp, Cout, Coutp, H, W, Ho, Wo, pad;
  int GH, GW;
  int gs;
  LifParams lif;
};

__device__ __forceinline__ int halo_route(const unsigned long long* nnz, int64_t numel,
                                          double thr) {
  if (!nnz) return CF_ROUTE_DENSE;
  const unsigned long long k = *nnz;
  if (k == 0) return CF_ROUTE_ZERO;
  return (1.0 - (double)k / (double)numel > thr) ? CF_ROUTE_SPARSE : CF_ROUTE_DENSE;
}

// Workgroups per CU the register budget is sized for.  128-channel or
// 128-pixel tiles keep 4 x 32 accumulator registers per time block and get
// the full 512-register budget; 64 x 64 tiles fit in 168 registers, three
// workgroups per CU.
template <int BM, int TH, int TW, int S, int K>
constexpr int halo_min_blocks() {
  return (BM >= 128 || TH * TW >= 128) ? 1 : 3;
}

// K: filter size (3, or 1 for pointwise convolutions, whose strided input
// samples are staged densely: RH = TH, RW = TW).
// LM: LIF specialisation (cf_lif_mode) of the EPI_LIF epilogue.
template <int BM, int TH, int TW, int S, int K, int EPI, int LM>
__global__ __launch_bounds__(256, (halo_min_blocks<BM, TH, TW, S, K>()))
void conv_halo_kernel(HaloArgs a) {
  constexpr int BN = TH * TW;
  constexpr int WM = BM / 2, WN = BN / 2, MT = WM / 32, NT = WN / 32;
  constexpr int RH = K == 1 ? TH : (TH - 1) * S + K, RW = K == 1 ? TW : (TW - 1) * S + K;
  constexpr int SS = K == 1 ? S : 1;  // input step between staged pixels
  constexpr int KK = K * K;
  constexpr int HALO_PIX = RH * RW;
  constexpr int TB = halo_tb<S, K>();
  constexpr int UNITS = TB * HALO_PIX * 4;  // 16-byte units per chunk
  constexpr int PER = (UNITS + 255) / 256;  // staging units per thread
  static_assert(MT >= 1 && NT >= 1, "tile too small");
  constexpr int HBUF = TB * HALO_PIX * LDK;  // halo buffer (halves)
  // Output staging of the epilogue (in the halo buffer): one step's tile as
  // BN pixels x (BM + 8) halves; two buffers when they fit, so one barrier
  // per step separates a step's LDS writes from its copy-out.
  constexpr int OLD = BM + 8;
  constexpr int OSTEP = BN * OLD;
  constexpr int NOBUF = 2 * OSTEP <= HBUF ? 2 : 1;
  static_assert(OSTEP <= HBUF, "output staging exceeds the halo buffer");
  auto halo_idx = [](int P, int part) { return P * LDK + (part << 3); };
  __shared__ __attribute__((aligned(16))) _Float16 halo[HBUF];
  __shared__ __attribute__((aligned(16))) float bn_s[2][BM];  // alpha, beta of the tile

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tile = blockIdx.x;
  const int gw = tile % a.GW, gh = (tile / a.GW) % a.GH, b = tile / (a.GW * a.GH);
  const int oh0 = gh * TH, ow0 = gw * TW;
  const int ih0 = oh0 * S - a.pad, iw0 = ow0 * S - a.pad;
  const int cout0 = blockIdx.y * BM;
  const int HoWo = a.Ho * a.Wo;
  const int nch = a.Cp / KC;
  const int ntiles = a.B * a.GH * a.GW;
  if (tid < BM) {  // alpha/beta hold Coutp entries
    bn_s[0][tid] = a.alpha[cout0 + tid];
    bn_s[1][tid] = a.beta[cout0 + tid];
  }

  // Pixels this lane owns in the accumulator layout (column lane%32 of each N tile).
  int n_base[NT], e_off[NT];
  bool n_ok[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = wn * WN + nt * 32 + (lane & 31);
    const int py = n / TW, px = n % TW;
    n_base[nt] = K == 1 ? py * RW + px : (py * S) * RW + px * S;
    n_ok[nt] = (oh0 + py) < a.Ho && (ow0 + px) < a.Wo;
    e_off[nt] = (oh0 + py) * a.Wo + (ow0 + px);
  }

  // Output channel of accumulator register r in M tile mt is
  // co_lane + mt * 32 + 8 * (r / 4) + r % 4.  Element indices are 32-bit
  // (the host checks that every output tensor has fewer than 2^31 elements).
  const int co_lane = cout0 + wm * WM + 4 * (lane >> 5);
  const bool full_c = cout0 + BM <= a.Cout;  // every channel of the tile is real
  float v[MT][NT][16];
  if (EPI == EPI_LIF) {
    const int col = opaque(co_lane);
    const int vb = (b * a.Cout + col) * HoWo;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dc = mt * 32 + 8 * (r >> 2) + (r & 3);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float v0 = lif_initial_v(a.lif);
          if (a.v_in && col + dc < a.Cout && n_ok[nt]) v0 = a.v_in[vb + dc * HoWo + e_off[nt]];
          v[mt][nt][r] = v0;
        }
      }
  }

  const int route = halo_route(a.nnz, a.numel, a.sparse_thr);

  // Weight fragments (fragment-major packing): this lane's 16 bytes of the
  // fragment (M tile mt, tap, 16-channel step k16) are at
  // wbase[mt] + (tap * Cp/16 + k16) * 512 halves; the lo limb follows the hi
  // limb at limb_stride.
  const int k16s = a.Cp / 16;
  const _Float16* wbase[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    wbase[mt] = a.w + (size_t)((cout0 + wm * WM + mt * 32) / 32) * KK * k16s * 512 + lane * 8;
  const size_t limb_stride = (size_t)a.Coutp * KK * a.Cp;

  for (int tb0 = 0; tb0 < a.T; tb0 += TB) {
    const int nsteps = min(TB, a.T - tb0);
    uint32_t mask[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      uint32_t m = 0u;
      if (t < nsteps) {
        if (route == CF_ROUTE_DENSE) m = 0xffffffffu;
        else if (route == CF_ROUTE_SPARSE)
          m = (uint32_t)a.ag_mask[(size_t)(tb0 + t) * ntiles + tile];
      }
      mask[t] = m;
    }
    f16v acc[TB][MT][NT];
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[t][mt][nt][r] = 0.0f;

    // Chunks active at some step of the block, in order (uniform across the
    // workgroup: every thread evaluates the same masks).
    auto chunk_act = [&](int ch, bool (&act)[TB]) -> bool {
      const int g0 = (ch * KC) / a.gs, g1 = (ch * KC + KC - 1) / a.gs;
      uint32_t gbits = 0u;
      for (int g = g0; g <= g1 && g < 32; ++g) gbits |= 1u << g;
      bool any = false;
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        act[t] = (mask[t] & gbits) != 0u;
        any |= act[t];
      }
      return any;
    };
    // act[t] for a lane-dependent t (no dynamic register indexing).
    auto act_at = [](const bool (&act)[TB], int t) {
      bool r = false;
#pragma unroll
      for (int i = 0; i < TB; ++i) r = r || (t == i && act[i]);
      return r;
    };
    auto next_chunk = [&](int ch) -> int {
      bool tmp[TB];
      for (int c = ch + 1; c < nch; ++c)
        if (chunk_act(c, tmp)) return c;
      return nch;
    };
    // Halo staging through registers in groups of NSTG 16-byte units: all
    // loads of a group are issued before its LDS stores.  (No register
    // prefetch of the next chunk during the taps: vector memory loads retire
    // in order, so the taps' weight loads would wait for it anyway.)
    constexpr int NSTG = PER < 8 ? PER : 8;
    u32x4 stg[NSTG];
    auto halo_load = [&](int ch, int i0, u32x4 (&st)[NSTG]) {
      const int c0 = ch * KC;
      bool act[TB];
      chunk_act(ch, act);
#pragma unroll
      for (int i = 0; i < NSTG; ++i) {
        const int u = opaque(tid) + 256 * (i0 + i);
        const int part = u & 3;
        const int pix = (u >> 2) % HALO_PIX;
        const int t = (u >> 2) / HALO_PIX;
        const int ry = pix / RW, rx = pix % RW;
        const int ih = ih0 + ry * SS, iw = iw0 + rx * SS;
        const bool ok = u < UNITS && t < nsteps && act_at(act, t) && ih >= 0 && ih < a.H &&
                        iw >= 0 && iw < a.W;
        const u32x4* src =
            ok ? reinterpret_cast<const u32x4*>(
                     a.x + ((((size_t)(tb0 + t) * a.B + b) * a.H + ih) * a.W + iw) * a.Cp + c0 + part * 8)
               : &g_halo_zero;
        st[i] = *src;
      }
    };
    auto halo_store = [&](int i0, const u32x4 (&st)[NSTG]) {
#pragma unroll
      for (int i = 0; i < NSTG; ++i) {
        const int u = opaque(tid) + 256 * (i0 + i);
        if (u < UNITS) {
          const int part = u & 3;
          const int pix = (u >> 2) % HALO_PIX;
          const int t = (u >> 2) / HALO_PIX;
          *reinterpret_cast<u32x4*>(&halo[(t * HALO_PIX + pix) * LDK + part * 8]) = st[i];
        }
      }
    };
    auto halo_stage = [&](int ch) {
      for (int i0 = 0; i0 < PER; i0 += NSTG) {
        halo_load(ch, i0, stg);
        halo_store(i0, stg);
      }
    };
    // Weight fragments: [buffer][mt][ks], hi and lo limbs.  Tap 0 of a chunk
    // is loaded into buffer 0 before the chunk's halo is staged (loads
    // retire in order, so it is ready when the taps start).
    h8 ah[2][MT][2], al[2][MT][2];
    auto load_tap0 = [&](int chunk) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const _Float16* p = wbase[mt] + (size_t)(chunk * 2 + ks) * 512;
          ah[0][mt][ks] = *reinterpret_cast<const h8*>(p);
          al[0][mt][ks] = *reinterpret_cast<const h8*>(p + limb_stride);
        }
    };
    // The K loop of one chunk: no per-step branches.  A step the chunk is
    // inactive at (SparseFlow) was staged as zeros, and adding the exact
    // zero products leaves the accumulator's bits unchanged (it starts at
    // +0 and is never -0), so this equals skipping the step.
    auto run_taps = [&](int ch) {
#pragma unroll
      for (int tap = 0; tap < KK; ++tap) {
        const int cur = tap & 1;
        const int tap_off = (tap / K) * RW + (tap % K);
        // B fragments of all TB steps are read before the tap's MFMAs,
        // unconditionally (reads for steps this chunk skips are harmless and
        // keep the reads free of branches, which would serialise them).
        h8 bb[TB][2][NT];
#pragma unroll
        for (int t = 0; t < TB; ++t)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
              bb[t][ks][nt] = *reinterpret_cast<const h8*>(
                  &halo[halo_idx(t * HALO_PIX + n_base[nt] + tap_off, 2 * ks + (lane >> 5))]);
        if (tap + 1 < KK) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              const _Float16* p = wbase[mt] + (size_t)((tap + 1) * k16s + ch * 2 + ks) * 512;
              ah[cur ^ 1][mt][ks] = *reinterpret_cast<const h8*>(p);
              al[cur ^ 1][mt][ks] = *reinterpret_cast<const h8*>(p + limb_stride);
            }
          // Issue the next tap's weight loads before this tap's MFMAs.
          __builtin_amdgcn_sched_barrier(0);
        }
        // Consecutive MFMAs go to different accumulators (time steps, tiles)
        // so none waits for the previous one's result; each accumulator
        // still sums ks 0 hi, ks 0 lo, ks 1 hi, ks 1 lo in that order.
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int limb = 0; limb < 2; ++limb)
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                  acc[t][mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                      limb ? al[cur][mt][ks] : ah[cur][mt][ks], bb[t][ks][nt], acc[t][mt][nt],
                      0, 0, 0);
        // Later taps' reads stay below this tap's MFMAs (register budget).
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    int ch = next_chunk(-1);
    if (ch < nch) {
      load_tap0(ch);
      __syncthreads();  // previous time block's LDS reads are complete
      halo_stage(ch);
      __syncthreads();
    }
    while (ch < nch) {
      const int nx = next_chunk(ch);
      run_taps(ch);
      if (nx < nch) {
        load_tap0(nx);
        __syncthreads();  // all taps of this chunk have read the halo
        halo_stage(nx);
        __syncthreads();
      }
      ch = nx;
    }

    // Epilogue over the time block: BN, (identity), LIF, then the fp16 NHWC
    // copy of the step's output tile, staged in LDS (the halo buffer is free
    // here) and written as 16-byte chunks, one 2*BM-byte run per pixel.  A
    // spike-valued identity (SEW ADD) is read from its fp16 NHWC copy when
    // there is one: four consecutive channels of a pixel per 8-byte load,
    // exact for the integer values it holds.  The lean path (no fp32 output,
    // no fp32 identity, every channel real) has no per-element branches:
    // out-of-range pixels are computed from zero halo and never stored.
    __syncthreads();  // the last chunk's halo reads are complete
    const bool lean = EPI == EPI_LIF && !a.out && !a.identity && full_c;
    auto epi_step = [&](auto lean_c, int t) {
      constexpr bool LEAN = decltype(lean_c)::value;
      const int tt = tb0 + t;
      _Float16* ostage = halo + (t % NOBUF) * OSTEP;
      const int col = opaque(co_lane);
      const int ob = ((tt * a.B + b) * a.Cout + col) * HoWo;
      const _Float16* idn = a.identity_nhwc;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          // Registers 4*r4 .. 4*r4+3 hold four consecutive output channels.
          const int colb = wm * WM + mt * 32 + 8 * r4 + 4 * (lane >> 5);
          const float4 al4 = *reinterpret_cast<const float4*>(&bn_s[0][colb]);
          const float4 be4 = *reinterpret_cast<const float4*>(&bn_s[1][colb]);
          const float alv[4] = {al4.x, al4.y, al4.z, al4.w};
          const float bev[4] = {be4.x, be4.y, be4.z, be4.w};
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            h4 idh = {};
            if (idn) {
              const int pix = n_ok[nt] ? e_off[nt] : 0;
              idh = *reinterpret_cast<const h4*>(
                  idn + ((size_t)(tt * a.B + b) * HoWo + pix) * a.cp_id + col + mt * 32 + 8 * r4);
            }
            h4 pk;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * r4 + j;
              float z = acc[t][mt][nt][r] * alv[j] + bev[j];
              float ov;
              if constexpr (LEAN) {
                float vv = lif_charge_m<LM>(v[mt][nt][r], z, a.lif);
                const float sp = lif_fire_reset_bit<LM>(vv, a.lif) ? 1.0f : 0.0f;
                v[mt][nt][r] = vv;
                ov = idn ? (float)idh[j] + sp : sp;
              } else {
                const int dc = mt * 32 + 8 * r4 + j;
                const bool ok = col + dc < a.Cout && n_ok[nt];
                const int o = ob + dc * HoWo + e_off[nt];
                if (ok && a.identity && a.identity_mode == ID_ADD_Z) z = z + a.identity[o];
                if (EPI == EPI_Z) {
                  ov = z;
                } else {
                  float vv = lif_charge_m<LM>(v[mt][nt][r], z, a.lif);
                  const float sp = lif_fire_reset_bit<LM>(vv, a.lif) ? 1.0f : 0.0f;
                  v[mt][nt][r] = vv;
                  if (idn) ov = (float)idh[j] + sp;
                  else if (ok && a.identity && a.identity_mode == ID_ADD_SPIKE) ov = a.identity[o] + sp;
                  else ov = sp;
                }
                if (ok && a.out) a.out[o] = ov;
              }
              pk[j] = (_Float16)ov;
            }
            *reinterpret_cast<h4*>(&ostage[(wn * WN + nt * 32 + (lane & 31)) * OLD + colb]) = pk;
          }
        }
    };
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      if (t >= nsteps) break;
      if (NOBUF == 1 && t > 0) __syncthreads();  // the previous step's copy-out is complete
      if (lean) epi_step(std::true_type{}, t);
      else epi_step(std::false_type{}, t);
      if (a.out_nhwc) {
        __syncthreads();  // the step's tile is staged
        const _Float16* ostage = halo + (t % NOBUF) * OSTEP;
        constexpr int CH8 = BM / 8;  // 16-byte chunks per pixel
        for (int c = tid; c < BN * CH8; c += 256) {
          const int px = c / CH8, part = c % CH8;
          const int py = px / TW, pxx = px % TW;
          const int co8 = cout0 + part * 8;
          if (oh0 + py < a.Ho && ow0 + pxx < a.Wo && co8 < a.cp_out) {
            const size_t pix = (size_t)(oh0 + py) * a.Wo + (ow0 + pxx);
            *reinterpret_cast<u32x4*>(a.out_nhwc + (((size_t)(tb0 + t) * a.B + b) * HoWo + pix) * a.cp_out + co8) =
                *reinterpret_cast<const u32x4*>(&ostage[px * OLD + part * 8]);
          }
        }
      }
    }
  }

  if (EPI == EPI_LIF && a.v_out) {
    const int col = opaque(co_lane);
    const int vb = (b * a.Cout + col) * HoWo;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (!n_ok[nt]) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = mt * 32 + 8 * (r >> 2) + (r & 3);
          if (full_c || col + dc < a.Cout) a.v_out[vb + dc * HoWo + e_off[nt]] = v[mt][nt][r];
        }
    }
  }
}

template <int BM, int TH, int TW, int S, int K = 3>
hipError_t launch_halo(const HaloArgs& a, int epi, hipStream_t st) {
  dim3 grid((unsigned)(a.B * a.GH * a.GW), (unsigned)(a.Coutp / BM));
  const dim3 block(256);
  if (epi == EPI_Z) {
    hipLaunchKernelGGL((conv_halo_kernel<BM, TH, TW, S, K, EPI_Z, LM_GENERIC>), grid, block, 0, st, a);
  } else {
    switch (cf_lif_mode(a.lif)) {
      case LM_HARD0_DECAY_P2:
        hipLaunchKernelGGL((conv_halo_kernel<BM, TH, TW, S, K, EPI_LIF, LM_HARD0_DECAY_P2>), grid,
                           block, 0, st, a);
        break;
      case LM_HARD_DECAY_P2:
        hipLaunchKernelGGL((conv_halo_kernel<BM, TH, TW, S, K, EPI_LIF, LM_HARD_DECAY_P2>), grid,
                           block, 0, st, a);
        break;
      default:
        hipLaunchKernelGGL((conv_halo_kernel<BM, TH, TW, S, K, EPI_LIF, LM_GENERIC>), grid, block,
                           0, st, a);
    }
  }
  return hipGetLastError();
}

}  // namespace

// 3x3 convolutions (stride 1 or 2, any padding) with halo staging; the
// caller picks the tile (tile_h x tile_w in {8x8, 8x16}; 8x16 only with
// stride 1).  Arguments as cf_conv_mfma.
CF_API int cf_conv_halo(const void* x, const void* w_packed, const float* alpha,
                        const float* beta, const float* v_in, float* v_out, float* out,
                        void* out_nhwc, int64_t cp_out,
                        const float* identity, const void* identity_nhwc, int64_t cp_id,
                        int identity_mode, const int32_t* ag_mask,
                        const unsigned long long* nnz, int64_t numel, double sparse_threshold,
                        int64_t T, int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp, int64_t H,
                        int64_t W, int64_t Ho, int64_t Wo, int64_t ksize, int64_t stride,
                        int64_t pad, int64_t tile_h, int64_t tile_w, int64_t group_size,
                        int epilogue, double tau, double v_th, double v_reset, int hard_reset,
                        int decay_input, void* stream) {
  if (!x || !w_packed || !alpha || !beta || (!out && !out_nhwc)) return (int)hipErrorInvalidValue;
  if (ksize != 1 && ksize != 3) return (int)hipErrorInvalidValue;
  if (out_nhwc && (cp_out < Cout || cp_out > Coutp)) return (int)hipErrorInvalidValue;
  if (T <= 0 || B <= 0 || Cp <= 0 || Cp % KC != 0 || Cp / KC > 64 || Cout <= 0 ||
      Coutp < Cout || Coutp % 64 != 0 || H <= 0 || W <= 0 || pad < 0 || pad > 2)
    return (int)hipErrorInvalidValue;
  if (stride != 1 && stride != 2) return (int)hipErrorInvalidValue;
  if (Ho != (H + 2 * pad - ksize) / stride + 1 || Wo != (W + 2 * pad - ksize) / stride + 1 || Ho <= 0 ||
      Wo <= 0)
    return (int)hipErrorInvalidValue;
  if (epilogue != EPI_LIF && epilogue != EPI_Z) return (int)hipErrorInvalidValue;
  if (identity && identity_mode != ID_ADD_SPIKE && identity_mode != ID_ADD_Z)
    return (int)hipErrorInvalidValue;
  if (identity_nhwc && (identity_mode != ID_ADD_SPIKE || cp_id < Cout || cp_id % 4 != 0))
    return (int)hipErrorInvalidValue;
  if (!((tile_h == 8 && tile_w == 8) || (tile_h == 8 && tile_w == 16 && stride == 1 && ksize == 3)))
    return (int)hipErrorInvalidValue;
  if (ag_mask && (group_size <= 0 || (Cp + group_size - 1) / group_size > 32))
    return (int)hipErrorInvalidValue;
  if (T * B * Cout * Ho * Wo > INT32_MAX || T * B * H * W > ((int64_t)1 << 40))
    return (int)hipErrorInvalidValue;
  HaloArgs a;
  a.x = (const _Float16*)x; a.w = (const _Float16*)w_packed; a.alpha = alpha; a.beta = beta;
  a.v_in = v_in; a.v_out = v_out; a.out = out; a.identity = identity;
  a.identity_nhwc = (const _Float16*)identity_nhwc; a.cp_id = (int)cp_id;
  a.out_nhwc = (_Float16*)out_nhwc; a.cp_out = (int)cp_out;
  a.identity_mode = identity_mode; a.ag_mask = ag_mask;
  // Without masks the SparseFlow route cannot be taken: pass the count only
  // when masks exist (StaticZero is still detected through nnz == 0 below).
  a.nnz = nnz; a.numel = numel;
  a.sparse_thr = ag_mask ? sparse_threshold : 2.0;  // 2.0: sparsity never exceeds it
  a.T = (int)T; a.B = (int)B; a.Cp = (int)Cp; a.Cout = (int)Cout; a.Coutp = (int)Coutp;
  a.H = (int)H; a.W = (int)W; a.Ho = (int)Ho; a.Wo = (int)Wo; a.pad = (int)pad;
  a.GH = (int)((Ho + tile_h - 1) / tile_h);
  a.GW = (int)((Wo + tile_w - 1) / tile_w);
  a.gs = group_size > 0 ? (int)group_size : 32;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  hipStream_t st = (hipStream_t)stream;
  // 64-channel tiles: measured faster on every SEW-ResNet18 layer than
  // 128-channel ones (which hold one workgroup per CU slot).
  // CATFUSE_HALO_BM=128 selects 128-channel tiles (tuning).
  bool bm128 = false;
  if (const char* e = getenv("CATFUSE_HALO_BM")) {
    if (atoi(e) == 128) bm128 = (Coutp % 128 == 0);
    else if (atoi(e) == 64) bm128 = false;
  }
  hipError_t e;
  if (ksize == 1)
    e = stride == 1 ? launch_halo<64, 8, 8, 1, 1>(a, epilogue, st)
                    : launch_halo<64, 8, 8, 2, 1>(a, epilogue, st);
  else if (stride == 1 && tile_w == 16)
    e = launch_halo<64, 8, 16, 1>(a, epilogue, st);  // 64-channel tiles (register budget)
  else if (stride == 1)
    e = bm128 ? launch_halo<128, 8, 8, 1>(a, epilogue, st) : launch_halo<64, 8, 8, 1>(a, epilogue, st);
  else
    e = bm128 ? launch_halo<128, 8, 8, 2>(a, epilogue, st) : launch_halo<64, 8, 8, 2>(a, epilogue, st);
  return (int)e;
}
