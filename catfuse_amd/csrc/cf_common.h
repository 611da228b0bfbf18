// Shared device helpers for the catfuse_amd gfx950 kernels.
//
// Numerics contract (all kernels): built with -ffp-contract=off and
// correctly-rounded fp32 division, so the LIF recurrence below rounds every
// operation exactly as SpikingJelly's eval-mode multi-step torch path does
// on the CPU (see lif_charge / lif_fire_reset).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define CF_API extern "C" __attribute__((visibility("default")))

// Route words written on the device by the pack/route kernels and read by
// the conv kernels.  Values mirror catfuse's SpatialBackend decision:
//   ZERO   <=> count_nonzero(x) == 0                      (StaticZero)
//   SPARSE <=> 1 - nnz/numel > 0.7 (evaluated in double)  (SparseFlow)
//   DENSE  otherwise                                       (DenseKeep)
enum { CF_ROUTE_ZERO = 0, CF_ROUTE_SPARSE = 1, CF_ROUTE_DENSE = 2 };

// Status word bits (sticky, device side; read by catfuse_amd.runtime).
enum {
  CF_STATUS_INEXACT_FP16 = 1u,   // an input assumed fp16-exact was not
  CF_STATUS_FP16_RANGE = 2u,     // an analog input split into fp16 limbs was
                                 // outside the fp16 range (or not finite)
};

// Packed conv weights (cf_pack_conv_weights) are stored fragment-major: for
// each limb, 32-row output-channel tile, tap and 16-channel K step, the
// 32 x 16 A operand of one v_mfma_f32_32x32x16_f16 as 64 lanes x 8 halves
// (lane l holds row l % 32, channels 8 * (l / 32) .. + 7), so a wave loads a
// fragment with one fully coalesced 1 KB access.  Element (limb, co, tap, c):
__host__ __device__ inline size_t cf_wfrag_index(int limb, int co, int tap, int c, int Coutp,
                                                 int KHW, int Cp) {
  const size_t frag = (((size_t)limb * (Coutp / 32) + co / 32) * KHW + tap) * (Cp / 16) + c / 16;
  return (frag * 64 + (co % 32) + 32 * ((c % 16) / 8)) * 8 + (c % 8);
}

// LIF parameters passed by value to every kernel with a LIF epilogue.
struct LifParams {
  float tau;
  float v_th;
  float v_reset;     // ignored when hard == 0 (soft reset)
  float decay_coef;  // (float)(1 - 1/tau) computed in double on the host;
                     // used only by the soft-reset, no-decay-input charge
  float inv_tau;     // 1/tau, exact when tau_pow2 is set
  int tau_pow2;      // tau = +-2^k with 1/tau a normal float: x / tau and
                     // x * inv_tau round the same real number, so the
                     // multiply gives the division's bits
  int hard;          // 1: hard reset to v_reset; 0: soft reset v -= v_th
  int decay_input;   // 1: v += (x - (v - v_reset)) / tau
};

// x / tau, IEEE-rounded (the multiply form only where it is bit-identical).
__device__ __forceinline__ float lif_div_tau(float x, const LifParams& p) {
  return p.tau_pow2 ? x * p.inv_tau : x / p.tau;
}

// Charge step, SpikingJelly eval-mode op order.
//   hard, decay_input    : v = v + (x - (v - v_reset)) / tau
//   hard, no decay_input : v = v - (v - v_reset) / tau + x
//   soft, decay_input    : v = v + (x - v) / tau
//   soft, no decay_input : v = v * (1 - 1/tau) + x
__device__ __forceinline__ float lif_charge(float v, float x, const LifParams& p) {
  if (p.hard) {
    if (p.decay_input) return v + lif_div_tau(x - (v - p.v_reset), p);
    return (v - lif_div_tau(v - p.v_reset, p)) + x;
  }
  if (p.decay_input) return v + lif_div_tau(x - v, p);
  return v * p.decay_coef + x;
}

// Fire + reset.  Returns the spike (0/1) and updates v in place.
//   hard: v = v_reset * s + (1 - s) * v
//   soft: v = v - s * v_th
__device__ __forceinline__ float lif_fire_reset(float& v, const LifParams& p) {
  const float s = (v >= p.v_th) ? 1.0f : 0.0f;
  if (p.hard) v = p.v_reset * s + (1.0f - s) * v;
  else v = v - s * p.v_th;
  return s;
}

// LIF specialisations picked on the host.  LM_GENERIC takes the parameter
// branches above at run time; LM_HARD_DECAY_P2 is SpikingJelly's default
// LIFNode (hard reset, decay_input, tau a power of two) with the same
// operations in the same order and no branches.
// LM_HARD0_DECAY_P2 is the same with v_reset == +0.0 (SpikingJelly's
// default), where v - v_reset == v exactly.
enum { LM_GENERIC = 0, LM_HARD_DECAY_P2 = 1, LM_HARD0_DECAY_P2 = 2 };

__host__ __device__ inline int cf_lif_mode(const LifParams& p) {
  if (!(p.hard && p.decay_input && p.tau_pow2)) return LM_GENERIC;
  // +0.0 exactly (not -0.0): v - (+0) == v for every v, signed zeros included
  return __builtin_bit_cast(uint32_t, p.v_reset) == 0u ? LM_HARD0_DECAY_P2 : LM_HARD_DECAY_P2;
}

// In the P2 forms the product d * inv_tau is exact (a power of two; unless
// it falls below the normal range, where |v| would be below 2^-125 too), so
// one fused multiply-add rounds exactly as the separate multiply and add.
template <int LM>
__device__ __forceinline__ float lif_charge_m(float v, float x, const LifParams& p) {
  if constexpr (LM == LM_HARD0_DECAY_P2) return __builtin_fmaf(x - v, p.inv_tau, v);
  else if constexpr (LM == LM_HARD_DECAY_P2)
    return __builtin_fmaf(x - (v - p.v_reset), p.inv_tau, v);
  else return lif_charge(v, x, p);
}

// Fire + reset returning the spike as a bool.  The hard reset
// v_reset * s + (1 - s) * v is evaluated as fma(m, v, c) with m = 1 - s and
// c = v_reset * s selected from {v_reset, 0 * v_reset}: both products are
// exact (s, m are 0 or 1), so the fma's single rounding is the add's.
template <int LM>
__device__ __forceinline__ bool lif_fire_reset_bit(float& v, const LifParams& p) {
  if constexpr (LM == LM_HARD0_DECAY_P2 || LM == LM_HARD_DECAY_P2) {
    const bool f = v >= p.v_th;
    const float m = f ? 0.0f : 1.0f;
    const float c = LM == LM_HARD0_DECAY_P2 ? 0.0f : (f ? p.v_reset : 0.0f * p.v_reset);
    v = __builtin_fmaf(m, v, c);
    return f;
  } else {
    return lif_fire_reset(v, p) != 0.0f;
  }
}

__device__ __forceinline__ float lif_initial_v(const LifParams& p) {
  return p.hard ? p.v_reset : 0.0f;
}

// Cache-policy operand of the raw buffer store builtins: the non-temporal
// (streaming) hint.
constexpr int CF_CPOL_NT = 2;

// Count block of a producer pass (cf_pack_input, cf_scan_nhwc, a fused conv
// writing its output): CF_COUNT_BLOCK_WORDS u64,
//   [0] the pass accumulator, (sum of counts) << CF_TALLY_BITS | completed
//       groups; zero between passes;
//   [1] the count of the last completed pass, read by the kernels that
//       consume the pass's output (later in stream order);
//   [16 * (g + 1)] the accumulator of workgroup group g (workgroups whose
//       linear index is g modulo CF_COUNT_GROUPS), same packing, zero
//       between passes; each on a 128-byte line of its own.
// A workgroup adds its count and its completion to its group word with one
// atomic; the workgroup that completes its group adds the group's total and
// one group completion to [0] and clears the group word; the one that
// completes [0] stores the pass total in [1] and clears [0].  So the next
// pass starts from zero with no clearing launch, one atomic carries each
// count together with its completion (nothing orders two updates, so no
// fence is needed; an agent-scope release fence would write back the L2 of
// the workgroup's XCD), and the same-address atomics of a pass are spread
// over CF_COUNT_GROUPS words (at ~10 ns per same-address atomic, a single
// word costs ~10 us for a thousand workgroups finishing together).  A pass
// has fewer than 2^24 workgroups (the launchers check) and counts below 2^40.
constexpr int CF_TALLY_BITS = 24;
constexpr unsigned long long CF_MAX_COUNT_WG = 1ull << CF_TALLY_BITS;
constexpr unsigned CF_COUNT_GROUPS = 16;
constexpr unsigned CF_COUNT_BLOCK_WORDS = 16 * (CF_COUNT_GROUPS + 1);

// Called by one thread of every workgroup of the pass, once its count is
// final; wg is the workgroup's linear index, nwg the pass's workgroup count.
__device__ __forceinline__ void cf_count_publish(unsigned long long* blk, unsigned long long cnt,
                                                 unsigned wg, unsigned nwg) {
  constexpr unsigned long long TALLY = CF_MAX_COUNT_WG - 1ull;
  const unsigned g = wg % CF_COUNT_GROUPS;
  const unsigned ngroups = nwg < CF_COUNT_GROUPS ? nwg : CF_COUNT_GROUPS;
  const unsigned in_group = (nwg - g + CF_COUNT_GROUPS - 1) / CF_COUNT_GROUPS;
  unsigned long long* gw = blk + 16 * (g + 1);
  const unsigned long long prev = atomicAdd(gw, (cnt << CF_TALLY_BITS) | 1ull);
  if ((prev & TALLY) != (unsigned long long)in_group - 1ull) return;
  const unsigned long long gtot = (prev >> CF_TALLY_BITS) + cnt;
  *gw = 0ull;
  const unsigned long long prev0 = atomicAdd(&blk[0], (gtot << CF_TALLY_BITS) | 1ull);
  if ((prev0 & TALLY) == (unsigned long long)ngroups - 1ull) {
    blk[1] = (prev0 >> CF_TALLY_BITS) + gtot;
    blk[0] = 0ull;
  }
}

// Workgroup "any" of a per-thread predicate (256-thread workgroups): one
// wave vote per wave, combined through four LDS words after a barrier.
__device__ __forceinline__ bool cf_wg_any(bool pred, unsigned* sh4) {
  const bool w = __any(pred ? 1 : 0) != 0;
  if ((threadIdx.x & 63) == 0) sh4[threadIdx.x >> 6] = w ? 1u : 0u;
  __syncthreads();
  return (sh4[0] | sh4[1] | sh4[2] | sh4[3]) != 0u;
}

// The published count of a block (a pass of an earlier kernel).
__device__ __forceinline__ unsigned long long cf_count_read(const unsigned long long* blk) {
  return blk[1];
}

// Descriptor of a fused conv's output (16 bytes of device memory, written by
// the launch that is given one, read by later launches in stream order):
//   copy:   CF_COPY_WRITTEN  the fp16 NHWC copy buffer holds the values;
//           CF_COPY_ZERO     every value is zero and the buffer was not
//                            written;
//           CF_COPY_ALIAS    the values are those of the copy at `alias` (the
//                            layer's identity, same shape and pitch) and the
//                            buffer was not written;
//   vstate: 0 v_out holds the membrane state; 1 every pixel of channel c
//           holds v_chan[c] (the launch's per-channel buffer) and v_out was
//           not written.
enum { CF_COPY_WRITTEN = 0, CF_COPY_ZERO = 1, CF_COPY_ALIAS = 2 };
struct CfOutDesc {
  uint32_t copy;
  uint32_t vstate;
  const void* alias;
};
static_assert(sizeof(CfOutDesc) == 16, "descriptor layout");

// What a caller knows of a layer's response to its BN bias alone (the
// StaticZero drive: z = 0 * alpha + beta at every pixel, from the initial
// state), from cf_bias_response: CF_BIAS_SILENT no channel fires at any of
// the T steps; CF_BIAS_VCHAN the caller holds the per-channel final
// potentials (so a StaticZero launch need not write v_out).
enum { CF_BIAS_SILENT = 1, CF_BIAS_VCHAN = 2 };

// Where a copy's values are, given its descriptor (nullable): the buffer
// itself, the aliased copy, or nullptr for an all-zero copy.
template <typename T>
__device__ __forceinline__ const T* cf_copy_source(const CfOutDesc* d, const T* own) {
  if (d == nullptr) return own;
  const uint32_t st = d->copy;
  if (st == CF_COPY_ZERO) return nullptr;
  if (st == CF_COPY_ALIAS) return reinterpret_cast<const T*>(d->alias);
  return own;
}

// Host: LIF parameter block from SpikingJelly-level (double) parameters.
LifParams cf_make_lif_params(double tau, double v_th, double v_reset, int hard, int decay_input);

// fp16 NHWC copy of a boundary output element, read by the next fused conv
// instead of re-packing the fp32 tensor: nhwc[(img*HoWo + pix)*cp + co].
__device__ __forceinline__ void store_nhwc(_Float16* nhwc, int cp, size_t img, int HoWo, int pix,
                                           int co, float val) {
  nhwc[((size_t)img * HoWo + pix) * cp + co] = (_Float16)val;
}

// Number of dispatches one grid dimension may hold.
static inline unsigned cf_blocks(int64_t n, int per_block) {
  return (unsigned)((n + per_block - 1) / per_block);
}
