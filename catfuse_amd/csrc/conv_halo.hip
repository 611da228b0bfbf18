// Fused 3x3 (and 1x1) Conv -> BN -> LIF on the matrix cores with the input
// halo staged in LDS and the time axis inside the tile.
//
// Workgroup tile: BM = 64 output channels x (TH x TW) output pixels of one
// image, for a block of up to TB = 4 time steps at once (2 for stride-2 3x3).
// One K step = one 32-channel chunk of one time block: the input halo of the
// tile for the block's steps is copied to LDS ([t][row][col][32 ch], fp16)
// by direct global->LDS loads, then the KK taps run from LDS: each weight
// fragment (fp16 hi/lo limbs, one coalesced 1 KB load per fragment from L2,
// one tap ahead) feeds the MFMAs of every time step.  Two halo buffers: the
// loads of the next K step are spread over the current step's taps, so the
// matrix cores do not wait for the staging.  When the K loop of a time block
// is complete the epilogue applies BN and the LIF for its steps in order,
// with v in VGPRs across time blocks.
//
// Tiles are the SparseFlow prescan tiles (8x8 / 8x16), so the same kernel
// serves the SparseFlow route: a chunk inactive at every step of a block is
// skipped, and a step a chunk is inactive at is staged as zeros.  Routes are
// decided on the device from the nonzero count and are bit-identical
// (skipped or zero chunks add exact zeros, and the accumulation order of the
// remaining ones is unchanged).
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
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// One-byte spike copies.  A spike value n (0/1, a SEW sum, any integer
// 0..255) becomes the fp16 value n exactly: v_perm places the byte under a
// 0x64 high byte, i.e. the half 1024 + n (fp16 holds every integer below
// 2048), and subtracting 1024 is exact.  The reverse adds 1024 to a half
// holding an integer 0..255 and keeps its low byte.
__device__ __forceinline__ h8 u8x8_to_h8(u32x2 r) {
  u32x4 w;
  w[0] = __builtin_amdgcn_perm(0x64646464u, r[0], 0x04010400u);   // b0, b1
  w[1] = __builtin_amdgcn_perm(0x64646464u, r[0], 0x04030402u);   // b2, b3
  w[2] = __builtin_amdgcn_perm(0x64646464u, r[1], 0x04010400u);
  w[3] = __builtin_amdgcn_perm(0x64646464u, r[1], 0x04030402u);
  return __builtin_bit_cast(h8, w) - (h8)(_Float16)1024.0f;
}
__device__ __forceinline__ h4 u8x4_to_h4(uint32_t r) {
  u32x2 w;
  w[0] = __builtin_amdgcn_perm(0x64646464u, r, 0x04010400u);
  w[1] = __builtin_amdgcn_perm(0x64646464u, r, 0x04030402u);
  return __builtin_bit_cast(h4, w) - (h4)(_Float16)1024.0f;
}
__device__ __forceinline__ u32x2 h8_to_u8x8(h8 h) {
  const u32x4 w = __builtin_bit_cast(u32x4, h + (h8)(_Float16)1024.0f);
  u32x2 r;
  r[0] = __builtin_amdgcn_perm(w[1], w[0], 0x06040200u);   // low bytes of halves 0..3
  r[1] = __builtin_amdgcn_perm(w[3], w[2], 0x06040200u);
  return r;
}

// Raw buffer resource over [base, base + bytes) (gfx9 word 3).  Buffer
// loads outside the range return zeros and buffer stores outside it are
// dropped by the hardware, so the lean epilogue issues every load and store
// unconditionally (a fixed count per step, which lets the compiler wait for
// exactly the loads it needs instead of draining earlier stores).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t halo_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
constexpr uint32_t HALO_OOB = 0x80000000u;  // an offset beyond every range used here

// Sixteen zero bytes in device memory: absent route words (counts,
// descriptors) are read from here.
__device__ __attribute__((aligned(16))) u32x4 g_halo_zero;

// Returns x unchanged, hidden from the optimiser: per-element addresses
// derived from it are recomputed where they are used instead of being kept
// live (in registers or scratch) across the K loop.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

constexpr int KC = 32;  // channels per chunk: four 16-byte parts per staged pixel

// One direct global -> LDS load (buffer_load_dwordx4 ... lds): lane l
// copies the 16 bytes at byte offset voff of the buffer rsrc (zeros when
// voff is beyond its range) to LDS byte address lds + 16 l (lds
// wave-uniform); the buffer's base is in scalar registers, so a copy takes
// no vector address arithmetic.
// Issued through inline assembly so that the compiler does not track it:
// its own load counting then never waits for these copies (it only waits
// for loads it issued, which in-order completion makes safe: a copy issued
// after a load never delays the wait for that load).  The kernel waits for
// the copies itself (s_waitcnt vmcnt(0) and a barrier) before reading them.
typedef int cf_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void lds_buf_copy16(cf_v4i rsrc, unsigned voff, unsigned lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(lds)
      : "memory", "m0");
}
// Raw buffer resource words (as halo_rsrc) in scalar registers, for inline
// assembly.
__device__ __forceinline__ cf_v4i halo_rsrc_v4(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)(uintptr_t)base;
  cf_v4i r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xffffu));
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Time steps per block: 4.
template <int S, int K>
constexpr int halo_tb() {
  return 4;
}

// Halo buffers: two (the next K step is staged while the current one is
// computed), or one for stride-2 3x3 tiles, whose 17 x 17 input halo of
// four steps (74 KB) would not fit twice next to a second workgroup: their
// K steps stage after the taps, and the CU's other workgroup fills the gap.
template <int S, int K>
constexpr int halo_nbuf() {
  return (S == 2 && K == 3) ? 1 : 2;
}

// Staged halo geometry and LDS layout: [t][RH][RW] pixels of 64 bytes (32
// channels), the pixel's four 16-byte parts stored in the order
// part ^ swz(row, col).  The taps' B-fragment reads (ds_read_b128) are served
// 16 lanes at a time from 64 four-byte banks (16 sixteen-byte slots): lanes
// 0-7 read one part of 8 consecutive output pixels, lanes 8-15 the same
// pixels one output row down.  The XOR spreads these 16 reads over 16
// distinct slots for every tap and time step (checked exhaustively for each
// configuration used).  Stride-2 3x3 halos store their columns
// de-interleaved (even columns, then odd ones), so that consecutive output
// pixels read consecutive staged pixels at every tap.
template <int S, int K, int TH, int TW>
struct HaloGeom {
  static constexpr int RH = K == 1 ? TH : (TH - 1) * S + K;
  static constexpr int RW = K == 1 ? TW : (TW - 1) * S + K;
  static constexpr int SS = K == 1 ? S : 1;  // input step between staged pixels
  static constexpr bool DEINT = K == 3 && S == 2;
  static constexpr int HALF = (RW + 1) / 2;
  // staged column of halo column rx
  __device__ static constexpr int col(int rx) {
    return DEINT ? ((rx & 1) ? HALF + (rx >> 1) : (rx >> 1)) : rx;
  }
  // halo column of staged column c
  __device__ static constexpr int inv_col(int c) {
    return DEINT ? (c < HALF ? 2 * c : 2 * (c - HALF) + 1) : c;
  }
  __device__ static constexpr int swz(int ry, int c) {
    return K == 1 ? (((c >> 2) ^ (2 * ry)) & 3) : (TW == 16 ? ((c >> 2) & 3) : ((c >> 1) & 3));
  }
};

// EPI_POOL: BN -> AvgPool2d(2, 2) -> LIF, the pooled spikes as the fp16
// NHWC copy, the pooled membrane state (8x8 tiles of stride-1 3x3 convs).
enum { EPI_LIF = 0, EPI_Z = 1, EPI_POOL = 2 };
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
  int cin_real;             // real input channels (<= Cp): K halves beyond are zero padding
  int identity_mode;
  const int32_t* ag_mask;   // [T][B*GH*GW]
  const int32_t* order;     // [1 + B*GH*GW]: active tile count, then every tile, the
                            // active ones first (cf_compact_tiles), or null
  const unsigned long long* nnz;  // count block of the input (cf_count_read), or null
  unsigned long long* nz_out;     // count block of the output: workgroups that wrote a
                                  // nonzero value (cf_count_publish), or null
  // Descriptors (CfOutDesc, nullable) of the input's and the identity's
  // copies as their producers left them, and of this launch's output; what
  // the caller knows of the layer's response to its bias alone (bias_info:
  // CF_BIAS_SILENT, CF_BIAS_VCHAN; needs out_desc); the identity's count
  // block (for an output that aliases it), nullable.
  const CfOutDesc* x_desc;
  const CfOutDesc* id_desc;
  CfOutDesc* out_desc;
  int bias_info;
  const unsigned long long* id_nnz;
  int64_t numel;
  double sparse_thr;
  int T, B, Cp, Cout, Coutp, H, W, Ho, Wo, pad;
  int GH, GW;
  int gs;
  int gs_shift;             // log2(gs) when gs is a power of two, else -1
  int u8;                   // the input, identity and output copies hold one byte per
                            // channel (the U8 instantiations), else fp16
  LifParams lif;
};

// Workgroups per CU the kernel is sized for: 64 x 64 tiles fit in 168
// registers (three per CU); 64 x 128 tiles keep twice the accumulators and
// get the full register budget; stride-2 3x3 tiles, whose halo buffer
// leaves room for two workgroups per CU, get two workgroups' budget.
template <int TH, int TW, int S = 1, int K = 3>
constexpr int halo_min_blocks() {
  return TH * TW >= 128 ? 1 : ((S == 2 && K == 3) ? 2 : 3);
}

// K: filter size (3, or 1 for pointwise convolutions, whose strided input
// samples are staged densely: RH = TH, RW = TW).
// LM: LIF specialisation (cf_lif_mode) of the EPI_LIF epilogue.
// LEAN: the EPI_LIF epilogue without fp32 output or fp32 identity, every
// output channel real (Cout a multiple of 64): no per-element branches.
// ONEB: T fits one time block (T <= TB): the block loop runs once, so the
// K-loop state is dead in the epilogue (fewer live registers).
// HS: the SparseFlow route skips the MFMAs of a silent 16-channel chunk half
// (prescan groups narrower than a chunk); off, the K loop has no per-half
// branches (the instantiations a dense-only launch uses).
// DEEP: launches of at most one workgroup per CU (one wave per SIMD, nothing
// else to switch to while a wave waits): the register budget of one
// workgroup per CU, and stride-1 3x3 K loops load each tap's weight
// fragments two taps ahead (three register buffers) instead of one.
// One halo buffer (halves) of a configuration: whole 64-unit blocks of the
// staged halo of a time block (16-byte units of TB steps x RH x RW pixels).
template <int TH, int TW, int S, int K>
constexpr int halo_buf_halves() {
  using G = HaloGeom<S, K, TH, TW>;
  return ((halo_tb<S, K>() * G::RH * G::RW * 4 + 63) / 64) * 64 * 8;
}

// The work of workgroup L of the nL that compute one conv: a device
// function, so that one grid can run two convs of the same input side by
// side (conv_halo_pair_kernel).  halo: halo_nbuf() * halo_buf_halves() halves of LDS;
// bn_s: the tile's BN coefficients; any_sh: the workgroup's vote words.
template <int TH, int TW, int S, int K, int EPI, int LM, bool LEAN, bool ONEB, bool HS, bool U8,
          bool DEEP = false>
__device__ __forceinline__ void halo_body(const HaloArgs a, const int L, const int nL,
                                          _Float16* __restrict__ halo, float (*bn_s)[64],
                                          unsigned* any_sh) {
  static_assert(!U8 || (LEAN && EPI == EPI_LIF), "one-byte copies: the lean LIF epilogue only");
  // Element of the input, identity and output copies: one byte (U8) or one
  // half per channel.  Element offsets are the same in both layouts
  // ([T*B][H][W][cp]); the halo in LDS is fp16 either way (a U8 K step's
  // bytes are widened on their way into it), so the K loop is the same.
  using XT = std::conditional_t<U8, uint8_t, _Float16>;
  constexpr int XB = (int)sizeof(XT);
  using G = HaloGeom<S, K, TH, TW>;
  constexpr int BM = 64;
  constexpr int BN = TH * TW;
  constexpr int WM = BM / 2, WN = BN / 2, NT = WN / 32;
  constexpr int RH = G::RH, RW = G::RW, SS = G::SS;
  constexpr int KK = K * K;
  constexpr int TB = halo_tb<S, K>();
  constexpr int NBUF = halo_nbuf<S, K>();
  constexpr int TSTR = RH * RW * KC;           // staged time step (halves)
  constexpr int NU = TB * RH * RW * 4;         // 16-byte units per staged chunk
  constexpr int NB = (NU + 63) / 64;           // 64-unit blocks (one direct load each)
  constexpr int HB = NB * 64 * 8;              // one halo buffer (halves), whole blocks
  constexpr int NPF = (NB + 3) / 4;            // direct loads per thread per chunk
  constexpr int TBR = TB > 2 ? 2 : TB;         // time steps per batch of B-fragment reads
  // Output staging of the epilogue (in the halo buffer consumed last): one
  // step's tile as BN pixels x (BM + 8) halves; two of them when they fit, so
  // one barrier per step separates a step's LDS writes from its copy-out.
  constexpr int OLD = BM + 8;
  constexpr int OSTEP = BN * OLD;
  constexpr int NOBUF = 2 * OSTEP <= HB ? 2 : 1;
  static_assert(OSTEP <= HB, "output staging exceeds a halo buffer");
  static_assert(NT >= 1, "tile too small");
  static_assert(HB == halo_buf_halves<TH, TW, S, K>(), "halo buffer size");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
  const int wm = wave >> 1, wn = wave & 1;
  const int hi = lane >> 5;
  // XCD-aware work order: workgroup L runs on XCD L % 8 (dispatch is
  // round-robin over the 8 XCDs), and the XCD's workgroups take a contiguous
  // range of work items, tile-major with the tile's 64-channel output blocks
  // adjacent.  The blocks of a tile (which stage the same input halo) and
  // neighbouring tiles (whose halos overlap) then run together on one XCD and
  // share its L2.
  //
  // On the SparseFlow route with a compacted tile order, the XCD's range
  // holds its equal share of the active work items (tiles active at some
  // step, in the order's sequence) first, then its share of the inactive
  // ones (epilogue only): the long workgroups start first on every XCD.
  // A tile order whose count is negative (cf_compact_tiles' dispatch score
  // rejected SparseFlow) turns the sparse route into the dense one.
  // The words that decide the route and where the input and identity are
  // (the input's count, the copies' descriptors, the identity's count),
  // loaded together: an absent one reads the zero page instead (a written
  // copy, a zero count), its absence kept apart.
  const unsigned long long* const zp = reinterpret_cast<const unsigned long long*>(&g_halo_zero);
  const CfOutDesc* const zdesc = reinterpret_cast<const CfOutDesc*>(&g_halo_zero);
  const unsigned long long in_count = *(a.nnz != nullptr ? a.nnz + 1 : zp);
  const unsigned long long id_count = *(a.id_nnz != nullptr ? a.id_nnz + 1 : zp);
  const CfOutDesc xd = *(a.x_desc != nullptr ? a.x_desc : zdesc);
  const CfOutDesc idd = *(a.id_desc != nullptr ? a.id_desc : zdesc);
  int route = a.nnz == nullptr ? CF_ROUTE_DENSE
              : in_count == 0ull ? CF_ROUTE_ZERO
              : ((1.0 - (double)in_count / (double)a.numel > a.sparse_thr) ? CF_ROUTE_SPARSE
                                                                          : CF_ROUTE_DENSE);
  if (route == CF_ROUTE_SPARSE && a.order != nullptr && a.order[0] < 0) route = CF_ROUTE_DENSE;
  // The input and identity copies where their producers left the values:
  // an all-zero input takes StaticZero (its buffer is not read), an
  // all-zero identity is read as zeros, aliased ones where they point.
  const XT* const xsrc = xd.copy == CF_COPY_ZERO    ? nullptr
                         : xd.copy == CF_COPY_ALIAS ? (const XT*)xd.alias
                                                    : (const XT*)(const void*)a.x;
  if (xsrc == nullptr) route = CF_ROUTE_ZERO;
  const XT* const id_nhwc = a.identity_nhwc == nullptr   ? nullptr
                            : idd.copy == CF_COPY_ZERO  ? nullptr
                            : idd.copy == CF_COPY_ALIAS ? (const XT*)idd.alias
                                                        : (const XT*)(const void*)a.identity_nhwc;
  XT* const out_copy = (XT*)(void*)a.out_nhwc;
  auto set_out_desc = [&](uint32_t copy, const void* alias, bool vchan) {
    if (a.out_desc != nullptr && tid == 0 && L == 0) {
      a.out_desc->copy = copy;
      a.out_desc->vstate = vchan ? 1u : 0u;
      a.out_desc->alias = alias;
    }
  };
  // StaticZero with no initial state and the layer's bias response known
  // to the caller (cf_bias_response, computed once per layer with the lean
  // path's operations): when no channel fires on its bias alone the output
  // is the identity (all zero without one), and its copy is not written:
  // the descriptor marks it all zero, or an alias of the identity's copy
  // when that is a fused layer's copy of the same pitch (identity + 0 is
  // the identity, bit for bit: spike counts hold no -0).  When the caller
  // also holds the per-channel final potentials, v_out is not written
  // either; then workgroup 0 alone records the descriptor and the count,
  // and every workgroup returns here, before any other memory access.
  // The pooled epilogue likewise, when the pooled bias response
  // (cf_bias_response with pool = 1) is silent: the copy is recorded as all
  // zero and not written, v_out left to the caller's per-channel potentials
  // (or not asked for); otherwise a pooled StaticZero launch runs the
  // epilogue on z = beta below.
  if constexpr (EPI == EPI_POOL) {
    if (route == CF_ROUTE_ZERO && a.v_in == nullptr && a.out_desc != nullptr &&
        (a.bias_info & CF_BIAS_SILENT) != 0 &&
        ((a.bias_info & CF_BIAS_VCHAN) != 0 || a.v_out == nullptr)) {
      if (L == 0 && tid == 0) {
        if (a.nz_out != nullptr) a.nz_out[1] = 0ull;
        a.out_desc->copy = CF_COPY_ZERO;
        a.out_desc->vstate = (a.bias_info & CF_BIAS_VCHAN) != 0 ? 1u : 0u;
        a.out_desc->alias = nullptr;
      }
      return;
    }
  }
  const bool zlean = LEAN && EPI == EPI_LIF && route == CF_ROUTE_ZERO && a.v_in == nullptr &&
                     (a.T + 2) * BM <= NBUF * HB;   // [T][BM] spike rows + BM floats
  const bool zvchan = zlean && a.out_desc != nullptr && (a.bias_info & CF_BIAS_VCHAN) != 0;
  uint32_t zcopy = CF_COPY_WRITTEN;
  const void* zalias = nullptr;
  bool id_live = false;   // an aliased identity has a nonzero value
  if (zlean && a.out_desc != nullptr && (a.bias_info & CF_BIAS_SILENT) != 0) {
    if (id_nhwc == nullptr) {
      zcopy = CF_COPY_ZERO;
    } else if (a.id_desc != nullptr && a.cp_id == a.cp_out) {
      zcopy = CF_COPY_ALIAS;
      zalias = id_nhwc;
      id_live = a.id_nnz == nullptr || id_count != 0ull;   // unknown: nonzero
    }
    if (zcopy != CF_COPY_WRITTEN && (zvchan || a.v_out == nullptr)) {
      if (L == 0 && tid == 0) {
        if (a.nz_out != nullptr) a.nz_out[1] = id_live ? 1ull : 0ull;
        a.out_desc->copy = zcopy;
        a.out_desc->vstate = zvchan ? 1u : 0u;
        a.out_desc->alias = zalias;
      }
      return;
    }
  }
  const int ncb = a.Coutp / BM;
  const int ntiles = a.B * a.GH * a.GW;
  const int nwork = ntiles * ncb;
  const int xcd = L & 7, j = L >> 3;
  const int xstart = xcd * (nwork >> 3) + min(xcd, nwork & 7);   // the XCD's first work item
  int tile, cb;
  if (a.order != nullptr && route == CF_ROUTE_SPARSE) {
    const int na = min(a.order[0], ntiles) * ncb;                    // active work items
    const int ax = (na >> 3) + (xcd < (na & 7) ? 1 : 0);             // the XCD's share of them
    const int sa = xcd * (na >> 3) + min(xcd, na & 7);
    const int pos = j < ax ? sa + j : na + (xstart - sa) + (j - ax);
    tile = min(max(a.order[1 + pos / ncb], 0), ntiles - 1);
    cb = pos % ncb;
  } else {
    const int work = xstart + j;
    tile = work / ncb;
    cb = work - tile * ncb;
  }
  const int gw = tile % a.GW, gh = (tile / a.GW) % a.GH, b = tile / (a.GW * a.GH);
  const int oh0 = gh * TH, ow0 = gw * TW;
  const int ih0 = oh0 * S - a.pad, iw0 = ow0 * S - a.pad;
  const int cout0 = cb * BM;
  const int HoWo = a.Ho * a.Wo;
  const int nch = a.Cp / KC;
  if (tid < BM) {  // alpha/beta hold Coutp entries
    bn_s[0][tid] = a.alpha[cout0 + tid];
    bn_s[1][tid] = a.beta[cout0 + tid];
  }

  // Pixels this lane owns in the accumulator layout (column lane%32 of each
  // N tile).  Its B fragment reads: staged pixel of tap (0, 0) (rd_pix,
  // halves within a staged step) and the part swizzle of each kw (2 bits per
  // kw in rd_swz); the kh rows and time steps are constant offsets.
  int e_off[NT];
  bool n_ok[NT];
  int rd_pix[NT], rd_swz[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = wn * WN + nt * 32 + (lane & 31);
    const int py = n / TW, px = n % TW;
    n_ok[nt] = (oh0 + py) < a.Ho && (ow0 + px) < a.Wo;
    e_off[nt] = (oh0 + py) * a.Wo + (ow0 + px);
    const int ry = K == 1 ? py : py * S, rx = K == 1 ? px : px * S;
    rd_pix[nt] = (ry * RW + G::col(rx)) * KC;
    int sw = 0;
#pragma unroll
    for (int kw = 0; kw < K; ++kw) sw |= G::swz(ry, G::col(rx + kw)) << (2 * kw);
    rd_swz[nt] = sw;
  }
  auto rd_addr = [&](int nt, int kw, int ks) {
    const int sw = (rd_swz[nt] >> (2 * kw)) & 3;
    return rd_pix[nt] + (G::col(kw) - G::col(0)) * KC + (((2 * ks + hi) ^ sw) << 3);
  };

  // Output channel of accumulator register r is co_lane + 8 * (r / 4) + r % 4.
  // Element indices are 32-bit (the host checks that every output tensor has
  // fewer than 2^31 elements).
  const int co_lane = cout0 + wm * WM + 4 * hi;
  const bool full_c = cout0 + BM <= a.Cout;  // every channel of the tile is real

  uint32_t anyw = 0u;  // OR of the bits of the output values this thread stores
  // The output's count block: workgroups that stored a nonzero value.
  auto publish_count = [&]() {
    if (a.nz_out) {
      // magnitude bits only (-0.0 counts as zero): two halves per word on the
      // lean path, one fp32 value otherwise
      const uint32_t mag = LEAN ? 0x7fff7fffu : 0x7fffffffu;
      const bool any = cf_wg_any((anyw & mag) != 0u, any_sh);
      if (threadIdx.x == 0) cf_count_publish(a.nz_out, any ? 1ull : 0ull, (unsigned)L, (unsigned)nL);
    }
  };

  // StaticZero from the initial membrane state (no v_in): z is the BN bias
  // of the channel at every pixel, so all pixels of a channel follow one
  // membrane trajectory.  The lean path runs the LIF once per channel over
  // all T steps (the operations of the per-element epilogue below, on the
  // same values, so the same bits), keeps each step's spikes as a row of BM
  // halves in LDS, and writes the tile from the rows: identity + spikes per
  // 16-byte chunk (packed fp16 adds, as below), then the final potential at
  // every pixel.  No K loop, no per-element LIF.
  //
  // The copy and state decisions were made above (zcopy, zvchan): a copy
  // recorded as all zero or as an alias is not written, nor is v_out when
  // the caller holds the per-channel potentials.
  if constexpr (LEAN && EPI == EPI_LIF) {
    if (zlean) {
      const uint32_t cst = zcopy;
      const void* alias = zalias;
      const bool vchan = zvchan;
      if (id_live) anyw = 1u;   // the published count is the identity's
      const bool elide = cst != CF_COPY_WRITTEN;
      _Float16* srow = halo;                                       // [T][BM] spikes
      float* vrow = reinterpret_cast<float*>(halo + a.T * BM);     // [BM] final v
      if (tid < BM) {  // the thread that loaded this channel's alpha/beta
        const float z = __builtin_fmaf(0.0f, bn_s[0][tid], bn_s[1][tid]);
        float v = lif_initial_v(a.lif);
        for (int t = 0; t < a.T; ++t) {
          float vv = lif_charge_m<LM>(v, z, a.lif);
          srow[t * BM + tid] = lif_fire_reset_bit<LM>(vv, a.lif) ? (_Float16)1.0f : (_Float16)0.0f;
          v = vv;
        }
        vrow[tid] = v;
      }
      __syncthreads();
      constexpr int CH8Z = BM / 8;                       // 16-byte chunks per pixel
      constexpr int CPIZ = BN * CH8Z / 256;              // chunks per thread per step
      static_assert(BN * CH8Z % 256 == 0, "whole copy-out passes");
      const bool have_id = id_nhwc != nullptr;
      for (int t = 0; t < (elide ? 0 : a.T); ++t) {
        const size_t img = (size_t)t * a.B + b;
        const __amdgpu_buffer_rsrc_t ro =
            halo_rsrc(out_copy + img * HoWo * a.cp_out, (uint32_t)(HoWo * a.cp_out * XB));
        const __amdgpu_buffer_rsrc_t ri =
            halo_rsrc(have_id ? id_nhwc + img * HoWo * a.cp_id : (const XT*)a.identity_nhwc,
                      have_id ? (uint32_t)(HoWo * a.cp_id * XB) : 0u);
#pragma unroll
        for (int i = 0; i < CPIZ; ++i) {
          const int c = tid + 256 * i;
          const int px = c / CH8Z, part = c % CH8Z;
          const int py = px / TW, pxx = px % TW;
          const bool ok = (oh0 + py < a.Ho) & (ow0 + pxx < a.Wo) & (cout0 + part * 8 < a.Cout);
          const int pix = (oh0 + py) * a.Wo + ow0 + pxx;
          const h8 sp = *reinterpret_cast<const h8*>(&srow[t * BM + part * 8]);
          const uint32_t ioff = ok ? (uint32_t)((pix * a.cp_id + cout0 + part * 8) * XB) : HALO_OOB;
          h8 idv;
          if constexpr (U8)
            idv = u8x8_to_h8(__builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(ri, ioff, 0, 0)));
          else
            idv = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(ri, ioff, 0, 0));
          const h8 sumh = idv + sp;
          const u32x4 sum = __builtin_bit_cast(u32x4, sumh);
          anyw |= ok ? (sum[0] | sum[1] | sum[2] | sum[3]) : 0u;
          const uint32_t ooff = ok ? (uint32_t)((pix * a.cp_out + cout0 + part * 8) * XB) : HALO_OOB;
          if constexpr (U8)
            __builtin_amdgcn_raw_buffer_store_b64(h8_to_u8x8(sumh), ro, ooff, 0, 0);
          else
            __builtin_amdgcn_raw_buffer_store_b128(sum, ro, ooff, 0, 0);
        }
      }
      if (a.v_out && !vchan) {
        // pixel p of the tile, channels cg * VPT .. + VPT - 1 of the block
        constexpr int VPT = BM * BN / 256;
        const int p = tid % BN, cg = tid / BN;
        const int py = p / TW, pxx = p % TW;
        const bool ok = (oh0 + py < a.Ho) & (ow0 + pxx < a.Wo);
        const int pix = (oh0 + py) * a.Wo + ow0 + pxx;
        const __amdgpu_buffer_rsrc_t rv =
            halo_rsrc(a.v_out + (size_t)b * a.Cout * HoWo, (uint32_t)(a.Cout * HoWo * 4));
#pragma unroll
        for (int k = 0; k < VPT; ++k) {
          const int c = cg * VPT + k;
          __builtin_amdgcn_raw_buffer_store_b32(
              __float_as_uint(vrow[c]), rv,
              (ok && cout0 + c < a.Cout) ? (uint32_t)(((cout0 + c) * HoWo + pix) * 4) : HALO_OOB, 0, 0);
        }
      }
      publish_count();
      set_out_desc(cst, alias, vchan);
      return;
    }
  }
  // Group bits active at time step tt (uniform across the workgroup).
  auto step_mask = [&](int tt) -> uint32_t {
    if (tt >= a.T || route == CF_ROUTE_ZERO) return 0u;
    if (route == CF_ROUTE_DENSE) return 0xffffffffu;
    return (uint32_t)a.ag_mask[(size_t)tt * ntiles + tile];
  };
  // Group bits of channels c0 .. c0 + n - 1: groups g0 .. g1 they fall in.
  auto range_bits = [&](int c0, int n) -> uint32_t {
    int g0, g1;
    if (a.gs_shift >= 0) {
      g0 = c0 >> a.gs_shift;
      g1 = (c0 + n - 1) >> a.gs_shift;
    } else {
      g0 = c0 / a.gs;
      g1 = (c0 + n - 1) / a.gs;
    }
    if (g0 > 31) return 0u;
    const uint32_t hi = g1 >= 31 ? 0xffffffffu : ((2u << g1) - 1u);
    return hi & ~((1u << g0) - 1u);
  };
  // Group bits of chunk ch (its 32 channels).
  auto chunk_bits = [&](int ch) -> uint32_t { return range_bits(ch * KC, KC); };
  // With groups narrower than a chunk, the 16-channel halves of a chunk can
  // be silent on their own: bit ks * TB + t of half_act is set when half ks
  // of chunk ch is active at step tbs + t.  The MFMAs of a half that is
  // silent at every step of a batch of B-fragment reads are skipped: its
  // products are exact zeros, so the accumulators' bits are those of the
  // dense evaluation.
  const bool half_skip = HS && route == CF_ROUTE_SPARSE && a.gs < KC;
  auto half_act = [&](int tbs, int ch) -> uint32_t {
    const uint32_t g0 = range_bits(ch * KC, KC / 2), g1 = range_bits(ch * KC + KC / 2, KC / 2);
    uint32_t m = 0u;
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const uint32_t sm = step_mask(tbs + t);
      m |= ((sm & g0) != 0u ? 1u : 0u) << t;
      m |= ((sm & g1) != 0u ? 1u : 0u) << (TB + t);
    }
    return m;
  };
  // Steps (bit t) of the block starting at tbs (< T) that chunk ch is
  // active at: every step on the dense route, none on the zero route.
  auto chunk_act = [&](int tbs, int ch) -> uint32_t {
    const int nst = min(TB, a.T - tbs);
    if (route == CF_ROUTE_DENSE) return (1u << nst) - 1u;
    if (route == CF_ROUTE_ZERO) return 0u;
    const uint32_t gb = chunk_bits(ch);
    uint32_t m = 0u;
#pragma unroll
    for (int t = 0; t < TB; ++t) m |= ((step_mask(tbs + t) & gb) != 0u ? 1u : 0u) << t;
    return m;
  };
  // The K step after (tbs, ch): the next active chunk of the block, else the
  // first active chunk of a later block (tbs' = T when there is none), and
  // its step activity.  On the dense route every chunk of every block is a
  // step, in order.
  auto next_step = [&](int tbs, int ch, int& ntb, int& nc, uint32_t& nact) {
    if (route == CF_ROUTE_DENSE) {
      if (ch + 1 < nch) {
        ntb = tbs;
        nc = ch + 1;
      } else {
        ntb = tbs + TB < a.T ? tbs + TB : a.T;
        nc = 0;
      }
      nact = ntb < a.T ? (1u << min(TB, a.T - ntb)) - 1u : 0u;
      return;
    }
    for (int tb = tbs; tb < a.T; tb += TB) {
      for (int c = (tb == tbs ? ch + 1 : 0); c < nch; ++c) {
        const uint32_t m = chunk_act(tb, c);
        if (m) {
          ntb = tb;
          nc = c;
          nact = m;
          return;
        }
      }
    }
    ntb = a.T;
    nc = 0;
    nact = 0u;
  };
  const size_t img_stride = (size_t)a.H * a.W * a.Cp;  // halves per staged image
  // This thread's unit of direct load i is the same for every K step of the
  // tile: its source offset (halves, from the tile's top-left input pixel of
  // time step 0 of the block; 32-bit, checked on the host), whether the
  // pixel lies inside the image (bit i of cp_inb) and its time step within
  // the block (bits 2i.. of cp_t).  Per K step only the block, the chunk and
  // the step activity change.
  const XT* xtile = xsrc + (ptrdiff_t)((ptrdiff_t)ih0 * a.W + iw0) * a.Cp;
  // Unit of direct load i of this thread: 64-unit block 4 i + w of wave w
  // (wrapped into 0 .. NB-1: a wrapped load repeats another one, writing
  // the same bytes), lane l unit 64 * block + l.  Its source offset (halves,
  // from the tile's top-left input pixel of time step 0 of the block;
  // 32-bit, checked on the host), whether the pixel lies inside the image,
  // and its time step within the block.
  // (Unsigned in-tile arithmetic: divisions by the constant halo sizes are
  // a multiply-high and a shift; the pixel offset is a 24-bit product, exact
  // since the host bounds 4 * B * H * W * Cp below 2^31; the time step's
  // stride is two selects of workgroup-uniform multiples.)
  const int tstr1 = a.B * (int)img_stride;
  auto unit_of = [&](int i, int& off, bool& inb, int& t) {
    int blk = 4 * i + wave;
    if (4 * NPF > NB && blk >= NB) blk -= NB;
    const unsigned l = (unsigned)opaque(lane);
    const unsigned U = (unsigned)blk * 64u + l;
    const unsigned slot = l & 3u, pix = (unsigned)blk * 16u + (l >> 2);
    const unsigned c = pix % (unsigned)RW, ry = (pix / (unsigned)RW) % (unsigned)RH;
    const unsigned tu = min(pix / (unsigned)(RW * RH), (unsigned)(TB - 1));
    t = (int)tu;
    const int rx = G::inv_col((int)c);
    const unsigned part = slot ^ (unsigned)G::swz((int)ry, (int)c);
    const int ih = ih0 + (int)ry * SS, iw = iw0 + rx * SS;
    inb = (U < (unsigned)NU) & (ih >= 0) & (ih < a.H) & (iw >= 0) & (iw < a.W);
    const unsigned sp = __umul24((unsigned)((int)ry * SS), (unsigned)a.W) + (unsigned)(rx * SS);
    off = (int)(__umul24(sp, (unsigned)a.Cp) + part * 8u) + ((tu & 1u) ? tstr1 : 0) +
          ((tu & 2u) ? 2 * tstr1 : 0);
    return blk;
  };
  // The units are the same for every K step of the tile; each time block
  // keeps them in registers for its taps (cp_off, bit i of cp_inb, bits
  // 2i.. of cp_t), so a K step's loads cost a few instructions each.
  int cp_off[NPF];
  // (two bits of cp_t per load: 64 of them once a thread has more than 16)
  using StepBits = std::conditional_t<(2 * NPF > 32), uint64_t, uint32_t>;
  static_assert(NPF <= 32, "one bit of cp_inb per direct load");
  uint32_t cp_inb = 0u;
  StepBits cp_t = 0u;
  auto units_precompute = [&]() {
    cp_inb = 0u;
    cp_t = 0u;
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      bool inb;
      int t;
      unit_of(i, cp_off[i], inb, t);
      cp_inb |= (inb ? 1u : 0u) << i;
      cp_t |= (StepBits)t << (2 * i);
    }
  };
  // Direct loads i0 .. i1-1 (of NPF) of this thread for K step (tbs, ch)
  // with step activity act into halo buffer hb.  Units of steps the chunk is
  // inactive at, of pixels outside the image, and past the last unit (the
  // buffer's tail) load zeros.  No branches.  PRE: from the precomputed
  // units (inside a block's K loop), else computed here.
  auto stage_loads = [&](auto pre_c, int tbs, int ch, uint32_t act, _Float16* hb, int i0, int i1) {
    constexpr bool PRE = decltype(pre_c)::value;
    const int nst = tbs < a.T ? min(TB, a.T - tbs) : 0;  // 0: every unit loads zeros
    const uint32_t live = act & ((1u << nst) - 1u);    // steps to load, bit t
    const XT* xb = xtile + (size_t)(tbs * a.B + b) * img_stride + ch * KC;
    // (offsets in bytes below 2^31, checked on the host; a unit not loaded
    // takes an offset beyond the range and copies zeros)
    const cf_v4i xr = halo_rsrc_v4(xb, 0x7fffffffu);
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      int off, t, blk;
      bool inb;
      if constexpr (PRE) {
        blk = 4 * i + wave;
        if (4 * NPF > NB && blk >= NB) blk -= NB;
        off = cp_off[i];
        inb = ((cp_inb >> i) & 1u) != 0u;
        t = (int)((cp_t >> (2 * i)) & 3u);
      } else {
        blk = unit_of(i, off, inb, t);
      }
      const bool ok = inb & (((live >> t) & 1u) != 0u);
      if constexpr (U8) {
        // eight channels (bytes) of the unit, widened to its 16 LDS bytes;
        // a buffer load (an out-of-range offset reads zeros)
        const u32x2 r = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(halo_rsrc(xb, 0x7fffffffu),
                                                        ok ? (uint32_t)off : HALO_OOB, 0, 0));
        *reinterpret_cast<h8*>(hb + blk * 512 + opaque(lane) * 8) = u8x8_to_h8(r);
      } else {
        lds_buf_copy16(xr, ok ? (uint32_t)off * 2u : HALO_OOB,
                       __builtin_amdgcn_readfirstlane(lds_addr(hb + blk * 512)));
      }
    }
  };
  // One-byte copies inside the K loop: a K step's loads are issued into
  // registers, spread over the taps of the step before (stage_defer), and
  // widened into their halo buffer once those taps are done
  // (stage_commit), so their latency is hidden as the direct loads' is.
  u32x2 raw[U8 ? NPF : 1];
  auto stage_defer = [&](int tbs, int ch, uint32_t act, int i0, int i1) {
    if constexpr (U8) {
      const int nst = tbs < a.T ? min(TB, a.T - tbs) : 0;
      const uint32_t live = act & ((1u << nst) - 1u);
      const XT* xb = xtile + (size_t)(tbs * a.B + b) * img_stride + ch * KC;
      // buffer loads from the K step's base (offsets below 2^31, checked
      // on the host; units outside the image or the live steps read zeros)
      const __amdgpu_buffer_rsrc_t rx = halo_rsrc(xb, 0x7fffffffu);
#pragma unroll
      for (int i = i0; i < i1; ++i) {
        const bool inb = ((cp_inb >> i) & 1u) != 0u;
        const int t = (int)((cp_t >> (2 * i)) & 3u);
        const bool ok = inb & (((live >> t) & 1u) != 0u);
        raw[i] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(rx, ok ? (uint32_t)cp_off[i] : HALO_OOB,
                                                        0, 0));
      }
    }
  };
  auto stage_commit = [&](_Float16* hb) {
    if constexpr (U8) {
#pragma unroll
      for (int i = 0; i < NPF; ++i) {
        int blk = 4 * i + wave;
        if (4 * NPF > NB && blk >= NB) blk -= NB;
        *reinterpret_cast<h8*>(hb + blk * 512 + opaque(lane) * 8) = u8x8_to_h8(raw[i]);
      }
    }
  };

  // Weight fragments (fragment-major packing): this lane's 16 bytes of the
  // fragment (tap, 16-channel step k16) of its 32-channel M tile are at
  // wbase + (tap * Cp/16 + k16) * 512 halves; the lo limb follows the hi limb
  // at limb_stride.  Two register buffers, alternating with a running tap
  // count that continues across K steps; three (W2: tap j in buffer j % 3,
  // loaded at tap j - 2) in the DEEP stride-1 3x3 K loop, whose nine taps
  // per K step keep that assignment the same in every K step.
  const int k16s = a.Cp / 16;
  // Buffer loads from the wave's first fragment: the lane's 16 bytes at a
  // constant per-lane offset, the fragment's offset (and the lo limb's) in a
  // scalar register, so a load takes no vector address arithmetic.  (The
  // host bounds both limbs' bytes below 2^31.)
  const _Float16* wbase = a.w + (size_t)((cout0 + wm * WM) / 32) * KK * k16s * 512;
  const __amdgpu_buffer_rsrc_t wrsrc = halo_rsrc(wbase, 0x7fffffffu);
  const uint32_t w_lane = (uint32_t)opaque(lane) * 16u;
  const uint32_t limb_bytes = (uint32_t)a.Coutp * KK * (uint32_t)a.Cp * 2u;
  constexpr bool W2 = DEEP && KK == 9 && NBUF == 2;
  constexpr int NWB = W2 ? 3 : 2;
  h8 ah[NWB][2], al[NWB][2];
  auto load_w = [&](int buf, int tap, int ch) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint32_t so = (uint32_t)((tap * k16s + ch * 2 + ks) * 1024);
      ah[buf][ks] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, so, 0));
      al[buf][ks] = __builtin_bit_cast(
          h8, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, w_lane, so + limb_bytes, 0));
    }
  };

  f16v acc[TB][NT];
  // The taps of K step ch from halo buffer hb: tap j uses weight buffer
  // j & 1 and loads the weights of the next tap (at the last tap: the next
  // K step's tap 0, moved to buffer 0 after the taps; W2: buffer j % 3, and
  // the weights of tap j + 2, the next K step's taps 0 and 1 at the last
  // two taps), then the direct loads
  // of the next K step (ntb, nc) into the other halo buffer hb_next, spread
  // over taps 0 .. KK-2.  Every load is issued unconditionally (a next step
  // in a later time block stages zeros here, its weights are reloaded
  // before the epilogue), and hb and hb_next are restrict-qualified: the
  // compiler's load counting then stays exact, and a tap waits for its own
  // weights only, not for every outstanding load.  No
  // per-step branches: a step the chunk is inactive at was staged as zeros,
  // and adding the exact zero products leaves the accumulator's bits
  // unchanged (it starts at +0 and is never -0), so this equals skipping it.
  // SKIP: skip the MFMAs of a silent chunk half (hm: half_act of the step).
  // 16-channel halves of chunk ch whose MFMAs run (bit ks): none for a
  // wave whose 32 output channels are all padding (Cout not a multiple of
  // 64), the lower one only where the upper 16 input channels are padding
  // (Cin not a multiple of 32).  The skipped products are exact zeros
  // (zero weights and zero input channels), so the accumulators' bits are
  // those of the full evaluation.
  const bool wave_idle = cout0 + wm * WM >= a.Cout;
  auto ks_run = [&](int ch) -> uint32_t {
    if (wave_idle) return 0u;
    return ch * KC + KC / 2 < a.cin_real ? 3u : 1u;
  };
  auto run_taps = [&](auto skip_c, const _Float16* __restrict__ hb,
                      _Float16* __restrict__ hb_next, int ch, int ntb, int nc, uint32_t nact,
                      int wblk, uint32_t hm) {
    const uint32_t kr = ks_run(ch);
    constexpr bool SKIP = decltype(skip_c)::value;
    const int stb = ntb == wblk ? ntb : a.T;  // a.T: stage zeros
    // Taps the next K step's staging loads are spread over: the first three
    // (at most all but the last, after which the barrier publishes them).
    // Issued early, they have landed before the later taps wait for their
    // weight fragments, a wait the in-order load counter would otherwise
    // extend to every staging load issued before them.
    constexpr int SPAN = KK - 1 < 3 ? KK - 1 : 3;
    // B fragments are read TBR steps at a time (a batch), unconditionally
    // (reads of steps this chunk skips hold zeros), one 16-channel half
    // (ks) at a time: half ks of the next batch (the next TBR steps, or the
    // next tap's first ones) is read as soon as the MFMAs of this batch's
    // half ks are issued, into the registers they read, so its LDS latency
    // passes under the other half's MFMAs.  The first batch of the K step is
    // read before its taps.
    h8 bb[TBR][2][NT];
    auto read_half = [&](int tap, int th, int ks) {
      const int kh = tap / K, kw = tap % K;
#pragma unroll
      for (int tr = 0; tr < TBR; ++tr)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          bb[tr][ks][nt] = *reinterpret_cast<const h8*>(
              &hb[(th + tr) * TSTR + kh * RW * KC + rd_addr(nt, kw, ks)]);
    };
    read_half(0, 0, 0);
    read_half(0, 0, 1);
    // Every 16-channel half runs (the common case: all channels real, no
    // half skip): the K loop without per-half branches.
    auto taps = [&](auto full_c) {
      constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
    for (int tap = 0; tap < KK; ++tap) {
      const int cur = W2 ? tap % 3 : (tap & 1);
#pragma unroll
      for (int th = 0; th < TB; th += TBR) {
        if (th == 0) {
          if constexpr (W2) {
            if (tap + 2 < KK) load_w((tap + 2) % 3, tap + 2, ch);
            else load_w((tap + 2) % 3, tap + 2 - KK, nc);
          } else {
            if (tap + 1 < KK) load_w(cur ^ 1, tap + 1, ch);
            else load_w(cur ^ 1, 0, nc);
          }
          if constexpr (U8) {
            // both buffer counts: loads now (on the first SPAN taps, as the
            // direct loads), widened after the taps
            if (KK == 1) {
              stage_defer(stb, nc, nact, 0, NPF);
            } else if (tap < SPAN) {
              const int i0 = (tap * NPF) / SPAN, i1 = ((tap + 1) * NPF) / SPAN;
              if (i1 > i0) stage_defer(stb, nc, nact, i0, i1);
            }
          } else if (NBUF == 1) {
            // one buffer: the next K step stages after the taps
          } else if (KK == 1) {
            stage_loads(std::true_type{}, stb, nc, nact, hb_next, 0, NPF);
          } else if (tap < SPAN) {
            const int i0 = (tap * NPF) / SPAN, i1 = ((tap + 1) * NPF) / SPAN;
            if (i1 > i0) stage_loads(std::true_type{}, stb, nc, nact, hb_next, i0, i1);
          }
        }
        // Issue the loads before these MFMAs.
        __builtin_amdgcn_sched_barrier(0);
        // The batch after this one within the K step (none after the last
        // tap's last batch: the next K step's halo is not published yet).
        const int ntap = th + TBR < TB ? tap : tap + 1;
        const int nth = th + TBR < TB ? th + TBR : 0;
        // Consecutive MFMAs go to different accumulators (time steps, tiles)
        // so none waits for the previous one's result; each accumulator
        // still sums ks 0 hi, ks 0 lo, ks 1 hi, ks 1 lo in that order.
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          bool run = true;
          if constexpr (!FULL) {
            run = ((kr >> ks) & 1u) != 0u;
            if constexpr (SKIP) run = run && ((hm >> (ks * TB + th)) & ((1u << TBR) - 1u)) != 0u;
          }
          if (run) {
#pragma unroll
            for (int limb = 0; limb < 2; ++limb)
#pragma unroll
              for (int tr = 0; tr < TBR; ++tr)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                  acc[th + tr][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                      limb ? al[cur][ks] : ah[cur][ks], bb[tr][ks][nt], acc[th + tr][nt], 0, 0,
                      0);
          }
          // The next batch's half ks into the registers these MFMAs read.
          __builtin_amdgcn_sched_barrier(0);
          if (ntap < KK) read_half(ntap, nth, ks);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    };
    taps(std::false_type{});
    if (!W2 && (KK & 1)) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        ah[0][ks] = ah[1][ks];
        al[0][ks] = al[1][ks];
      }
    }
  };

  // First K step: staged and its tap-0 (W2: and tap-1) weights loaded
  // before the loop.
  int s_tb, s_ch;
  uint32_t s_act;
  next_step(0, -1, s_tb, s_ch, s_act);
  int pf_tb = s_tb;  // block of the K step already staged into buffer 0
  // (A single time block computes its units once, here, and stages its
  // first K step from them.)
  if constexpr (ONEB) units_precompute();
  if (s_tb < a.T) {
    load_w(0, 0, s_ch);
    if constexpr (W2) load_w(1, 1, s_ch);
    stage_loads(std::integral_constant<bool, ONEB>{}, s_tb, s_ch, s_act, halo, 0, NPF);
  }

  for (int tb0 = 0; tb0 < (ONEB ? 1 : a.T); tb0 += TB) {
    const int nsteps = min(TB, a.T - tb0);
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][nt][r] = 0.0f;

    // The block's K steps alternate halo buffers, starting with buffer 0.
    // (The units are recomputed per block, unconditionally, so that they are
    // not live across the epilogue.)
    if constexpr (!ONEB) units_precompute();
    int buf = 0;
    while (s_tb == tb0) {
      int ntb, nc;
      uint32_t nact;
      next_step(s_tb, s_ch, ntb, nc, nact);
      // This step's halo has landed (each wave waits for its own direct
      // loads, the barrier for everyone's); every wave has finished reading
      // the other buffer, which the taps below refill.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      run_taps(std::integral_constant<bool, HS>{}, halo + buf * HB,
               halo + (NBUF == 2 ? (buf ^ 1) * HB : 0), s_ch, ntb, nc, nact, tb0,
               half_skip ? half_act(s_tb, s_ch) : 0xffffffffu);
      if constexpr (NBUF == 1) {
        // the next K step of this block into the buffer, once every wave
        // has finished reading it
        if (ntb == tb0) {
          __syncthreads();
          if constexpr (U8) stage_commit(halo);
          else stage_loads(std::true_type{}, ntb, nc, nact, halo, 0, NPF);
        }
      } else {
        if constexpr (U8) stage_commit(halo + (buf ^ 1) * HB);
        buf ^= 1;
      }
      s_tb = ntb;
      s_ch = nc;
      s_act = nact;
    }

    // Epilogue over the time block: BN, (identity), LIF, then the fp16 NHWC
    // copy of the step's output tile, staged in LDS (the halo buffer consumed
    // last; the next K step's loads go to the other one) and written as
    // 16-byte chunks, one 2*BM-byte run per pixel.  A spike-valued identity
    // (SEW ADD) is read from its fp16 NHWC copy when there is one: four
    // consecutive channels of a pixel per 8-byte load, exact for the integer
    // values it holds.  The lean path (no fp32 output, no fp32 identity,
    // every channel real) has no per-element branches: out-of-range pixels
    // are computed from zero halo and never stored.
    // The last taps' reads are complete, and so are the direct loads they
    // issued (zeros into the buffer the output is staged in below).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // The next block's first K step: tap-0 weights and halo (into buffer 0)
    // in flight during the epilogue, which stages its output in buffer 1.
    // (Two-step blocks, where a forward of 4 steps always has a next block,
    // reuse the units computed for this block: they are the same for every
    // block.  Four-step blocks compute them here, which keeps the units out of
    // the registers live across their K loop.)
    if (NBUF == 2 && s_tb < a.T && s_tb != pf_tb) {
      load_w(0, 0, s_ch);
      if constexpr (W2) load_w(1, 1, s_ch);
      stage_loads(std::integral_constant<bool, (TB == 2)>{}, s_tb, s_ch, s_act, halo, 0, NPF);
      pf_tb = s_tb;
    }
    // (with one halo buffer the output is staged in it, and the next block's
    // first K step is staged after the epilogue)
    _Float16* obuf = halo + (NBUF - 1) * HB;
    // Addresses below are a workgroup-uniform 64-bit base (scalar registers)
    // plus a 32-bit per-lane offset.  Lane-constant parts: its channel
    // column (col), its pixel (e_off, 0 for pixels outside the output).
    const int col = opaque(co_lane);
    int epix[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) epix[nt] = n_ok[nt] ? e_off[nt] : 0;
    // BN -> AvgPool2d(2, 2) -> LIF: a 2x2 window of the tile is lanes l,
    // l + 1, l + 8, l + 9 of a 32-lane half (pixel column l % 8 of row
    // l / 8); the lane of its top-left pixel sums the four BN outputs in the
    // order of cf_avgpool2x2_lif (((z00 + z01) + z10) + z11) * 0.25 and runs
    // the pooled neuron's LIF, whose potential it keeps across the steps.
    // Stores go through buffer descriptors: out-of-range offsets drop.
    if constexpr (EPI == EPI_POOL) {
      static_assert(NBUF == 2 && TH == 8 && TW == 8, "pooled epilogue: 8x8 tiles");
      const int Hp = a.Ho / 2, Wp = a.Wo / 2, HpWp = Hp * Wp;
      const int l = lane & 31;
      bool pok[NT];
      int pofs[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int p = wn * WN + nt * 32 + l;
        const int ppy = (oh0 + p / TW) / 2, ppx = (ow0 + p % TW) / 2;
        pok[nt] = (l & 9) == 0 && ppy < Hp && ppx < Wp;
        pofs[nt] = pok[nt] ? ppy * Wp + ppx : 0;
      }
      float vp[NT][16];
      const float* vsrc = tb0 == 0 ? a.v_in : a.v_out;
      const __amdgpu_buffer_rsrc_t rvin =
          halo_rsrc(vsrc ? vsrc + (size_t)b * a.Cout * HpWp : a.v_out,
                    vsrc ? (uint32_t)(a.Cout * HpWp * 4) : 0u);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = 8 * (r >> 2) + (r & 3);
          const uint32_t off = (pok[nt] && col + dc < a.Cout)
                                   ? (uint32_t)(((col + dc) * HpWp + pofs[nt]) * 4) : HALO_OOB;
          vp[nt][r] = vsrc ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rvin, off, 0, 0))
                           : lif_initial_v(a.lif);
        }
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if (t > 0 && t >= nsteps) break;  // (unrolled: acc stays in registers)
        const size_t img = (size_t)(tb0 + t) * a.B + b;
        const __amdgpu_buffer_rsrc_t ro =
            halo_rsrc(a.out_nhwc + img * HpWp * a.cp_out, (uint32_t)(HpWp * a.cp_out * 2));
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int colb = wm * WM + 8 * r4 + 4 * hi;
          const float4 al4 = *reinterpret_cast<const float4*>(&bn_s[0][colb]);
          const float4 be4 = *reinterpret_cast<const float4*>(&bn_s[1][colb]);
          const float alv[4] = {al4.x, al4.y, al4.z, al4.w};
          const float bev[4] = {be4.x, be4.y, be4.z, be4.w};
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            h4 sph;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * r4 + j;
              const float z = __builtin_fmaf(acc[t][nt][r], alv[j], bev[j]);
              const float z01 = __shfl_down(z, 1, 64);
              const float z10 = __shfl_down(z, 8, 64);
              const float z11 = __shfl_down(z, 9, 64);
              const float zp = (((z + z01) + z10) + z11) * 0.25f;
              float vv = lif_charge_m<LM>(vp[nt][r], zp, a.lif);
              sph[j] = lif_fire_reset_bit<LM>(vv, a.lif) ? (_Float16)1.0f : (_Float16)0.0f;
              vp[nt][r] = vv;
            }
            const bool ok = pok[nt] && col + 8 * r4 < a.Cout;
            const u32x2 pw = __builtin_bit_cast(u32x2, sph);
            anyw |= ok ? (pw[0] | pw[1]) : 0u;
            __builtin_amdgcn_raw_buffer_store_b64(
                pw, ro, ok ? (uint32_t)((pofs[nt] * a.cp_out + col + 8 * r4) * 2) : HALO_OOB, 0,
                0);
          }
        }
      }
      if (a.v_out) {
        const __amdgpu_buffer_rsrc_t rv =
            halo_rsrc(a.v_out + (size_t)b * a.Cout * HpWp, (uint32_t)(a.Cout * HpWp * 4));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dc = 8 * (r >> 2) + (r & 3);
            const uint32_t off = (pok[nt] && col + dc < a.Cout)
                                     ? (uint32_t)(((col + dc) * HpWp + pofs[nt]) * 4) : HALO_OOB;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(vp[nt][r]), rv, off, 0, 0);
          }
      }
      continue;
    }
    // Membrane potentials of this lane's elements live in registers during
    // the epilogue only: from v_in (or the initial value) for the first time
    // block, from v_out (written at the end of the previous block's epilogue
    // by this same lane) for later ones.
    float v[NT][16];
    if (EPI == EPI_LIF) {
      const float* vsrc = tb0 == 0 ? a.v_in : a.v_out;
      const float* vbase = vsrc ? vsrc + (size_t)b * a.Cout * HoWo : nullptr;
      const float v0 = lif_initial_v(a.lif);
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) v[nt][r] = v0;
      if (vbase) {  // (workgroup-uniform: no per-element branches without a state)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = 8 * (r >> 2) + (r & 3);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            if ((full_c || col + dc < a.Cout) && n_ok[nt])
              v[nt][r] = vbase[(unsigned)((col + dc) * HoWo + e_off[nt])];
        }
      }
    }
    // One-byte copies: the identity of step t is loaded into idr[t & 1]
    // while step t - 1 is computed, before that step's stores (zeros without
    // an identity or beyond the block: an empty range): the four channels'
    // bytes, widened when used.  (The lean fp16 path adds the identity to
    // the staged tile at copy-out instead, below.)
    uint32_t idr[U8 ? 2 : 1][NT][4];
    auto id_load = [&](int t) {
      const bool have = id_nhwc && t < nsteps;
      const XT* base = have ? id_nhwc + (size_t)((tb0 + t) * a.B + b) * HoWo * a.cp_id
                            : (const XT*)a.identity_nhwc;
      const __amdgpu_buffer_rsrc_t rid =
          halo_rsrc(base, have ? (uint32_t)(HoWo * a.cp_id * XB) : 0u);
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const unsigned off = (unsigned)((epix[nt] * a.cp_id + col + 8 * r4) * XB);
          idr[t & 1][nt][r4] = __builtin_amdgcn_raw_buffer_load_b32(rid, off, 0, 0);
        }
    };
    if constexpr (U8) id_load(0);
    auto epi_step = [&](int t) {
      const int tt = tb0 + t;
      const int img = tt * a.B + b;
      _Float16* ostage = obuf + (t % NOBUF) * OSTEP;
      const XT* idn = id_nhwc;
      const XT* idbase = idn ? idn + (size_t)img * HoWo * a.cp_id : nullptr;
      if constexpr (U8) {
        if (t + 1 < TB) id_load(t + 1);
      }
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        // Registers 4*r4 .. 4*r4+3 hold four consecutive output channels.
        const int colb = wm * WM + 8 * r4 + 4 * hi;
        const float4 al4 = *reinterpret_cast<const float4*>(&bn_s[0][colb]);
        const float4 be4 = *reinterpret_cast<const float4*>(&bn_s[1][colb]);
        const float alv[4] = {al4.x, al4.y, al4.z, al4.w};
        const float bev[4] = {be4.x, be4.y, be4.z, be4.w};
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          h4 idh = {};
          if constexpr (U8) {
            idh = u8x4_to_h4(idr[t & 1][nt][r4]);
          } else if constexpr (LEAN) {
            // (added at copy-out)
          } else {
            if (idbase)
              idh = *reinterpret_cast<const h4*>(idbase + (unsigned)(epix[nt] * a.cp_id + col + 8 * r4));
          }
          h4 pk;
          if constexpr (LEAN) {
            // Spikes as halves; identity + spike in packed fp16 (exact: both
            // are small integers).  idh is +0 without an identity.
            h4 sph;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * r4 + j;
              const float z = __builtin_fmaf(acc[t][nt][r], alv[j], bev[j]);
              float vv = lif_charge_m<LM>(v[nt][r], z, a.lif);
              sph[j] = lif_fire_reset_bit<LM>(vv, a.lif) ? (_Float16)1.0f : (_Float16)0.0f;
              v[nt][r] = vv;
            }
            pk = idh + sph;
            if (U8 && a.nz_out) {
              const u32x2 pw = __builtin_bit_cast(u32x2, pk);
              anyw |= (n_ok[nt] && col + 8 * r4 < a.Cout) ? (pw[0] | pw[1]) : 0u;
            }
          } else {
            const int ob = ((tt * a.B + b) * a.Cout + col) * HoWo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int r = 4 * r4 + j;
              float z = __builtin_fmaf(acc[t][nt][r], alv[j], bev[j]);
              float ov;
              const int dc = 8 * r4 + j;
              const bool ok = col + dc < a.Cout && n_ok[nt];
              const int o = ob + dc * HoWo + e_off[nt];
              if (ok && a.identity && a.identity_mode == ID_ADD_Z) z = z + a.identity[o];
              if (EPI == EPI_Z) {
                ov = z;
              } else {
                float vv = lif_charge_m<LM>(v[nt][r], z, a.lif);
                const float sp = lif_fire_reset_bit<LM>(vv, a.lif) ? 1.0f : 0.0f;
                v[nt][r] = vv;
                if (idn) ov = (float)idh[j] + sp;
                else if (ok && a.identity && a.identity_mode == ID_ADD_SPIKE) ov = a.identity[o] + sp;
                else ov = sp;
              }
              if (ok && a.nz_out) anyw |= __float_as_uint(ov);
              if (ok && a.out) a.out[o] = ov;
              pk[j] = (_Float16)ov;
            }
          }
          *reinterpret_cast<h4*>(&ostage[(wn * WN + nt * 32 + (lane & 31)) * OLD + colb]) = pk;
        }
      }
    };
    // Copy-out of a staged step: BN * BM/8 sixteen-byte chunks, CPI per thread.
    constexpr int CH8 = BM / 8;  // 16-byte chunks per pixel
    constexpr int CPI = (BN * CH8 + 255) / 256;
    // Lean path: this thread's chunks are the same at every step (their
    // store offsets within a step's image and their LDS staging offsets),
    // computed once per block.
    uint32_t lo_off[LEAN ? CPI : 1], lo_lds[LEAN ? CPI : 1], lo_id[LEAN && !U8 ? CPI : 1];
    if constexpr (LEAN) {
#pragma unroll
      for (int i = 0; i < CPI; ++i) {
        const int c = tid + 256 * i;
        const int px = c / CH8, part = c % CH8;
        const int py = px / TW, pxx = px % TW;
        const bool ok = (oh0 + py < a.Ho) & (ow0 + pxx < a.Wo) & (cout0 + part * 8 < a.Cout);
        const int pix = (oh0 + py) * a.Wo + ow0 + pxx;
        lo_off[i] = ok ? (uint32_t)((pix * a.cp_out + cout0 + part * 8) * XB) : HALO_OOB;
        lo_lds[i] = (uint32_t)(px * OLD + part * 8);
        if constexpr (!U8) lo_id[i] = ok ? (uint32_t)((pix * a.cp_id + cout0 + part * 8) * 2) : HALO_OOB;
      }
    }
    // Lean fp16 path: the SEW identity is added to the staged tile at
    // copy-out, one 16-byte chunk (8 channels of a pixel, the copy-out's own
    // chunk) per load, issued before the step's LIF so it lands under it;
    // packed fp16 adds of small integers are exact.  Zeros without an
    // identity (an empty range).
    u32x4 idc[LEAN && !U8 ? CPI : 1];
    auto idc_load = [&](int t) {
      if constexpr (LEAN && !U8) {
        const bool have = id_nhwc && t < nsteps;
        const __amdgpu_buffer_rsrc_t rid =
            halo_rsrc(have ? (const void*)(id_nhwc + (size_t)((tb0 + t) * a.B + b) * HoWo * a.cp_id)
                           : (const void*)a.identity_nhwc,
                      have ? (uint32_t)(HoWo * a.cp_id * 2) : 0u);
#pragma unroll
        for (int i = 0; i < CPI; ++i) idc[i] = __builtin_amdgcn_raw_buffer_load_b128(rid, lo_id[i], 0, 0);
      }
    };
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      if (t > 0 && t >= nsteps) break;  // every block has a first step
      if (NOBUF == 1 && t > 0) __syncthreads();  // the previous step's copy-out is complete
      idc_load(t);
      epi_step(t);
      if (a.out_nhwc) {
        __syncthreads();  // the step's tile is staged
        const _Float16* ostage = obuf + (t % NOBUF) * OSTEP;
        _Float16* obase = a.out_nhwc + (size_t)((tb0 + t) * a.B + b) * HoWo * a.cp_out;
        if constexpr (LEAN) {
          // every chunk index is below BN * CH8; the hardware drops pixels
          // outside the output and channels >= Cout
          static_assert(BN * CH8 % 256 == 0, "lean copy-out assumes whole passes");
          const __amdgpu_buffer_rsrc_t ro =
              halo_rsrc(out_copy + (size_t)((tb0 + t) * a.B + b) * HoWo * a.cp_out,
                        (uint32_t)(HoWo * a.cp_out * XB));
#pragma unroll
          for (int i = 0; i < CPI; ++i) {
            const uint32_t off = lo_off[i];
            // streaming (non-temporal) stores: the copy is read back by the
            // next layer only after the whole output is written
            u32x4 chunk = *reinterpret_cast<const u32x4*>(&ostage[lo_lds[i]]);
            if constexpr (!U8) {
              chunk = __builtin_bit_cast(u32x4, __builtin_bit_cast(h8, chunk) +
                                                    __builtin_bit_cast(h8, idc[i]));
              if (a.nz_out)
                anyw |= off != HALO_OOB ? (chunk[0] | chunk[1] | chunk[2] | chunk[3]) : 0u;
            }
            if constexpr (U8)
              __builtin_amdgcn_raw_buffer_store_b64(h8_to_u8x8(__builtin_bit_cast(h8, chunk)), ro,
                                                    off, 0, CF_CPOL_NT);
            else
              __builtin_amdgcn_raw_buffer_store_b128(chunk, ro, off, 0, CF_CPOL_NT);
          }
        } else {
#pragma unroll
          for (int i = 0; i < CPI; ++i) {
            const int c = opaque(tid) + 256 * i;
            const int px = c / CH8, part = c % CH8;
            const int py = px / TW, pxx = px % TW;
            const int co8 = cout0 + part * 8;
            if ((c < BN * CH8) & (oh0 + py < a.Ho) & (ow0 + pxx < a.Wo) & (co8 < a.cp_out))
              *reinterpret_cast<u32x4*>(obase + (unsigned)(((oh0 + py) * a.Wo + ow0 + pxx) * a.cp_out + co8)) =
                  *reinterpret_cast<const u32x4*>(&ostage[px * OLD + part * 8]);
          }
        }
      }
    }
    // The block's final membrane potentials (the layer's state after the last block).
    if (LEAN && a.v_out) {
      // pixels outside the output and channels >= Cout are dropped
      const __amdgpu_buffer_rsrc_t rv =
          halo_rsrc(a.v_out + (size_t)b * a.Cout * HoWo, (uint32_t)(a.Cout * HoWo * 4));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = 8 * (r >> 2) + (r & 3);
          const uint32_t off = (n_ok[nt] && col + dc < a.Cout)
                                   ? (uint32_t)(((col + dc) * HoWo + e_off[nt]) * 4) : HALO_OOB;
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[nt][r]), rv, off, 0, 0);
        }
    } else if (EPI == EPI_LIF && a.v_out) {
      float* vbase = a.v_out + (size_t)b * a.Cout * HoWo;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        if (!n_ok[nt]) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dc = 8 * (r >> 2) + (r & 3);
          if (full_c || col + dc < a.Cout) vbase[(unsigned)((col + dc) * HoWo + e_off[nt])] = v[nt][r];
        }
      }
    }
    // One halo buffer: the next block's first K step, once every wave has
    // copied its output out of the buffer.
    if constexpr (NBUF == 1) {
      if (s_tb < a.T && s_tb != pf_tb) {
        __syncthreads();
        load_w(0, 0, s_ch);
        stage_loads(std::false_type{}, s_tb, s_ch, s_act, halo, 0, NPF);
        pf_tb = s_tb;
      }
    }
  }
  publish_count();
  set_out_desc(CF_COPY_WRITTEN, nullptr, false);
}

// The one-byte stride-1 3x3 instantiations hold the next K step's staged
// bytes in registers across the taps: the register budget of two workgroups
// per CU (at three they spill).
template <int TH, int TW, int S, int K, bool U8, bool DEEP>
constexpr int halo_kernel_min_blocks() {
  return DEEP ? 1 : ((U8 && S == 1 && K == 3 && halo_min_blocks<TH, TW, S, K>() > 2)
                         ? 2 : halo_min_blocks<TH, TW, S, K>());
}

template <int TH, int TW, int S, int K, int EPI, int LM, bool LEAN, bool ONEB, bool HS = false,
          bool U8 = false, bool DEEP = false>
__global__ __launch_bounds__(256, (halo_kernel_min_blocks<TH, TW, S, K, U8, DEEP>()))
void conv_halo_kernel(HaloArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 halo[halo_nbuf<S, K>() * halo_buf_halves<TH, TW, S, K>()];
  __shared__ __attribute__((aligned(16))) float bn_s[2][64];  // alpha, beta of the tile
  __shared__ unsigned any_sh[4];  // per-wave votes of the output count
  halo_body<TH, TW, S, K, EPI, LM, LEAN, ONEB, HS, U8, DEEP>(a, (int)blockIdx.x, (int)gridDim.x,
                                                             halo, bn_s, any_sh);
}

// Compute units of the current device (cached per device), or 0 when the
// runtime does not say.
int halo_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    cache[dev] = n > 0 ? n : -1;
  }
  return cache[dev] > 0 ? cache[dev] : 0;
}

// A lean EPI_LIF launch: the DEEP instantiation when deep (stride-1 3x3 8x8
// tiles without the half skip), else the ordinary one.
template <int TH, int TW, int S, int K, int LM, bool OB, bool HS, bool U8>
void launch_lean(bool deep, dim3 grid, dim3 block, hipStream_t st, const HaloArgs& a) {
  if constexpr (TH == 8 && TW == 8 && S == 1 && K == 3 && !HS) {
    if (deep) {
      hipLaunchKernelGGL((conv_halo_kernel<TH, TW, S, K, EPI_LIF, LM, true, OB, HS, U8, true>), grid,
                         block, 0, st, a);
      return;
    }
  }
  hipLaunchKernelGGL((conv_halo_kernel<TH, TW, S, K, EPI_LIF, LM, true, OB, HS, U8>), grid, block, 0,
                     st, a);
}

template <int TH, int TW, int S, int K = 3>
hipError_t launch_halo(const HaloArgs& a, int epi, hipStream_t st) {
  dim3 grid((unsigned)(a.B * a.GH * a.GW * (a.Coutp / 64)));
  const dim3 block(256);
  // at most one workgroup per CU: the DEEP K loop (used where it exists)
  const int cus = halo_cu_count();
  const bool deep = cus > 0 && grid.x <= (unsigned)cus;
  // lean: no fp32 output, no fp32 identity, whole 32-channel groups (the
  // stores drop channels >= Cout of a partly real 64-channel tile)
  const bool lean = epi == EPI_LIF && !a.out && !a.identity && a.Cout % 32 == 0;
  const bool oneb = a.T <= halo_tb<S, K>();
  if (a.u8) {
    // one-byte copies: the lean LIF epilogue on 8x8 tiles only (the SparseFlow
    // route without the half skip: the skipped products are zeros either way)
    if constexpr (TH == 8 && TW == 8) {
      if (!lean) return hipErrorInvalidValue;
      const int lm = cf_lif_mode(a.lif);
#define CF_HALO_U8(LMV)                                                                  \
  do {                                                                                   \
    if (oneb)                                                                            \
      launch_lean<TH, TW, S, K, LMV, true, false, true>(deep, grid, block, st, a);       \
    else                                                                                 \
      launch_lean<TH, TW, S, K, LMV, false, false, true>(deep, grid, block, st, a);      \
  } while (0)
      if (lm == LM_HARD0_DECAY_P2) CF_HALO_U8(LM_HARD0_DECAY_P2);
      else if (lm == LM_HARD_DECAY_P2) CF_HALO_U8(LM_HARD_DECAY_P2);
      else CF_HALO_U8(LM_GENERIC);
#undef CF_HALO_U8
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  if (epi == EPI_POOL) {
    // (the host admits it for stride-1 3x3 convs on 8x8 tiles only)
    if constexpr (TH == 8 && TW == 8 && S == 1 && K == 3) {
      const int lm = cf_lif_mode(a.lif);
#define CF_HALO_POOL(LMV)                                                                         \
  do {                                                                                            \
    if (oneb)                                                                                     \
      hipLaunchKernelGGL((conv_halo_kernel<TH, TW, S, K, EPI_POOL, LMV, false, true>), grid,      \
                         block, 0, st, a);                                                        \
    else                                                                                          \
      hipLaunchKernelGGL((conv_halo_kernel<TH, TW, S, K, EPI_POOL, LMV, false, false>), grid,     \
                         block, 0, st, a);                                                        \
  } while (0)
      if (lm == LM_HARD0_DECAY_P2) CF_HALO_POOL(LM_HARD0_DECAY_P2);
      else if (lm == LM_HARD_DECAY_P2) CF_HALO_POOL(LM_HARD_DECAY_P2);
      else CF_HALO_POOL(LM_GENERIC);
#undef CF_HALO_POOL
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  if (epi == EPI_Z) {
    hipLaunchKernelGGL((conv_halo_kernel<TH, TW, S, K, EPI_Z, LM_GENERIC, false, false>), grid,
                       block, 0, st, a);
  } else if (!lean) {
    hipLaunchKernelGGL((conv_halo_kernel<TH, TW, S, K, EPI_LIF, LM_GENERIC, false, false>), grid,
                       block, 0, st, a);
  } else {
    const int lm = cf_lif_mode(a.lif);
    // SparseFlow-capable with groups narrower than a chunk: the K loop that
    // skips silent chunk halves
    const bool hs = a.ag_mask != nullptr && a.gs < KC;
#define CF_HALO_LEAN(LMV, OB)                                                            \
  do {                                                                                   \
    if (hs)                                                                              \
      launch_lean<TH, TW, S, K, LMV, OB, true, false>(false, grid, block, st, a);        \
    else                                                                                 \
      launch_lean<TH, TW, S, K, LMV, OB, false, false>(deep, grid, block, st, a);        \
  } while (0)
    if (lm == LM_HARD0_DECAY_P2) {
      if (oneb) CF_HALO_LEAN(LM_HARD0_DECAY_P2, true);
      else CF_HALO_LEAN(LM_HARD0_DECAY_P2, false);
    } else if (lm == LM_HARD_DECAY_P2) {
      if (oneb) CF_HALO_LEAN(LM_HARD_DECAY_P2, true);
      else CF_HALO_LEAN(LM_HARD_DECAY_P2, false);
    } else {
      CF_HALO_LEAN(LM_GENERIC, false);
    }
#undef CF_HALO_LEAN
  }
  return hipGetLastError();
}

}  // namespace

namespace {

// Checks the arguments of one halo conv and fills its HaloArgs; 0 or a
// hipError_t (as int).
int make_halo_args(HaloArgs& a, const void* x, const void* w_packed, const float* alpha,
                   const float* beta, const float* v_in, float* v_out, float* out,
                   void* out_nhwc, int64_t cp_out, const float* identity,
                   const void* identity_nhwc, int64_t cp_id, int identity_mode,
                   const int32_t* ag_mask, const int32_t* tile_order,
                   const unsigned long long* nnz, unsigned long long* nz_out,
                   const void* x_desc, const void* id_desc, void* out_desc, int bias_info,
                   const unsigned long long* id_nnz, int64_t numel, double sparse_threshold, int64_t T, int64_t B, int64_t Cp, int64_t Cout,
                   int64_t Coutp, int64_t H, int64_t W, int64_t Ho, int64_t Wo, int64_t ksize,
                   int64_t stride, int64_t pad, int64_t tile_h, int64_t tile_w,
                   int64_t group_size, int epilogue, double tau, double v_th, double v_reset,
                   int hard_reset, int decay_input) {
  if (!x || !w_packed || !alpha || !beta || (!out && !out_nhwc)) return (int)hipErrorInvalidValue;
  if (ksize != 1 && ksize != 3) return (int)hipErrorInvalidValue;
  if (out_nhwc && (cp_out < Cout || cp_out > Coutp)) return (int)hipErrorInvalidValue;
  if (T <= 0 || B <= 0 || Cp <= 0 || Cp % KC != 0 || Cout <= 0 ||
      Coutp < Cout || Coutp % 64 != 0 || H <= 0 || W <= 0 || pad < 0 || pad > 2)
    return (int)hipErrorInvalidValue;
  if (stride != 1 && stride != 2) return (int)hipErrorInvalidValue;
  if (Ho != (H + 2 * pad - ksize) / stride + 1 || Wo != (W + 2 * pad - ksize) / stride + 1 || Ho <= 0 ||
      Wo <= 0)
    return (int)hipErrorInvalidValue;
  if (epilogue != EPI_LIF && epilogue != EPI_Z && epilogue != EPI_POOL)
    return (int)hipErrorInvalidValue;
  if (identity && identity_mode != ID_ADD_SPIKE && identity_mode != ID_ADD_Z)
    return (int)hipErrorInvalidValue;
  if (identity_nhwc && (identity_mode != ID_ADD_SPIKE || cp_id < Cout || cp_id % 4 != 0))
    return (int)hipErrorInvalidValue;
  // BN -> AvgPool2d(2, 2) -> LIF: stride-1 3x3 convs on 8x8 tiles, the
  // pooled spikes as the fp16 NHWC copy only (pitch a multiple of 4), whole
  // 32-channel groups, no identity (bias_info: the pooled bias response)
  if (epilogue == EPI_POOL &&
      (ksize != 3 || stride != 1 || tile_w != 8 || out || !out_nhwc || cp_out % 4 != 0 ||
       Cout % 32 != 0 || identity || identity_nhwc || Ho < 2 || Wo < 2))
    return (int)hipErrorInvalidValue;
  if (!((tile_h == 8 && tile_w == 8) || (tile_h == 8 && tile_w == 16 && stride == 1 && ksize == 3)))
    return (int)hipErrorInvalidValue;
  if (ag_mask && (group_size <= 0 || (Cp + group_size - 1) / group_size > 32))
    return (int)hipErrorInvalidValue;
  if (tile_order && !ag_mask) return (int)hipErrorInvalidValue;
  if ((bias_info & ~(CF_BIAS_SILENT | CF_BIAS_VCHAN)) != 0 || (bias_info && !out_desc))
    return (int)hipErrorInvalidValue;
  // 32-bit element indices of the outputs, 32-bit offsets of a tile's
  // input within one time block (4 steps) and of the packed weights (both
  // limbs)
  if (T * B * Cout * Ho * Wo > INT32_MAX || T * B * H * W > ((int64_t)1 << 40) ||
      8 * B * H * W * Cp > INT32_MAX || 4 * Coutp * ksize * ksize * Cp > INT32_MAX ||
      B * ((Ho + tile_h - 1) / tile_h) * ((Wo + tile_w - 1) / tile_w) * (Coutp / 64) * 256 > INT32_MAX)
    return (int)hipErrorInvalidValue;
  // (the grid is below 2^23 workgroups, within a count block's tally)
  // The membrane state passes from one time block to the next through v_out.
  const int tb = (stride == 2 && ksize == 3) ? halo_tb<2, 3>() : halo_tb<1, 3>();
  if (epilogue != EPI_Z && !v_out && T > tb) return (int)hipErrorInvalidValue;
  a.x = (const _Float16*)x; a.w = (const _Float16*)w_packed; a.alpha = alpha; a.beta = beta;
  a.v_in = v_in; a.v_out = v_out; a.out = out; a.identity = identity;
  a.identity_nhwc = (const _Float16*)identity_nhwc; a.cp_id = (int)cp_id;
  a.out_nhwc = (_Float16*)out_nhwc; a.cp_out = (int)cp_out;
  a.identity_mode = identity_mode; a.ag_mask = ag_mask; a.order = tile_order;
  // Without masks the SparseFlow route cannot be taken: pass the count only
  // when masks exist (StaticZero is still detected through nnz == 0 below).
  a.nnz = nnz; a.nz_out = nz_out; a.numel = numel;
  a.x_desc = (const CfOutDesc*)x_desc; a.id_desc = (const CfOutDesc*)id_desc;
  a.out_desc = (CfOutDesc*)out_desc; a.bias_info = bias_info; a.id_nnz = id_nnz;
  a.sparse_thr = ag_mask ? sparse_threshold : 2.0;  // 2.0: sparsity never exceeds it
  // the input's real channel count, numel / (T*B*H*W) when that divides and
  // is at most Cp (else every chunk runs whole)
  a.cin_real = (int)Cp;
  if (numel > 0 && numel % (T * B * H * W) == 0 && numel / (T * B * H * W) <= Cp)
    a.cin_real = (int)(numel / (T * B * H * W));
  a.T = (int)T; a.B = (int)B; a.Cp = (int)Cp; a.Cout = (int)Cout; a.Coutp = (int)Coutp;
  a.H = (int)H; a.W = (int)W; a.Ho = (int)Ho; a.Wo = (int)Wo; a.pad = (int)pad;
  a.GH = (int)((Ho + tile_h - 1) / tile_h);
  a.GW = (int)((Wo + tile_w - 1) / tile_w);
  a.gs = group_size > 0 ? (int)group_size : 32;
  a.gs_shift = (a.gs & (a.gs - 1)) == 0 ? __builtin_ctz((unsigned)a.gs) : -1;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  a.u8 = 0;
  return 0;
}

// A stride-2 3x3 conv and a stride-2 1x1 conv of the same input (a
// ResNet block's conv1 and its downsample) in one grid: workgroups
// 0 .. nLa-1 run the 3x3 conv's tiles, the rest the 1x1 conv's (whose input
// pixels are the 3x3 conv's centre taps), each as its own launch would (same
// accumulation order, so the same bits), sharing the input through the L2.
// Lean LIF epilogues only (fp16 NHWC outputs, no identity).
template <int LM, bool OBA, bool OBB, bool U8 = false>
__global__ __launch_bounds__(256, (halo_min_blocks<8, 8, 2, 3>()))
void conv_halo_pair_kernel(HaloArgs a, HaloArgs b, int nLa) {
  constexpr int HA = halo_nbuf<2, 3>() * halo_buf_halves<8, 8, 2, 3>();
  constexpr int HBB = halo_nbuf<2, 1>() * halo_buf_halves<8, 8, 2, 1>();
  __shared__ __attribute__((aligned(16))) _Float16 halo[HA > HBB ? HA : HBB];
  __shared__ __attribute__((aligned(16))) float bn_s[2][64];
  __shared__ unsigned any_sh[4];
  const int L = (int)blockIdx.x;
  if (L < nLa)
    halo_body<8, 8, 2, 3, EPI_LIF, LM, true, OBA, false, U8>(a, L, nLa, halo, bn_s, any_sh);
  else
    halo_body<8, 8, 2, 1, EPI_LIF, LM, true, OBB, false, U8>(b, L - nLa, (int)gridDim.x - nLa, halo,
                                                         bn_s, any_sh);
}

// The StaticZero drive of each channel (z = 0 * alpha + beta, from the
// initial state, T steps; pool: the pooled epilogue's average of four equal
// z, summed in its order) with the epilogues' operations: its final
// potential and whether it fires at some step.
template <int LM>
__global__ __launch_bounds__(256) void bias_response_kernel(const float* __restrict__ alpha,
                                                            const float* __restrict__ beta,
                                                            int Cout, int T, int pool,
                                                            LifParams lif,
                                                            float* __restrict__ v_final,
                                                            uint32_t* __restrict__ fires) {
  const int c = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (c >= Cout) return;
  const float z1 = __builtin_fmaf(0.0f, alpha[c], beta[c]);
  const float z = pool ? (((z1 + z1) + z1) + z1) * 0.25f : z1;
  float v = lif_initial_v(lif);
  bool f = false;
  for (int t = 0; t < T; ++t) {
    float vv = lif_charge_m<LM>(v, z, lif);
    f |= lif_fire_reset_bit<LM>(vv, lif);
    v = vv;
  }
  v_final[c] = v;
  fires[c] = f ? 1u : 0u;
}

}  // namespace

CF_API int cf_bias_response(const float* alpha, const float* beta, int64_t Cout, int64_t T,
                            int pool, double tau, double v_th, double v_reset, int hard_reset,
                            int decay_input, float* v_final, uint32_t* fires, void* stream) {
  if (!alpha || !beta || !v_final || !fires || Cout <= 0 || Cout > INT32_MAX || T <= 0 ||
      T > INT32_MAX || (pool != 0 && pool != 1))
    return (int)hipErrorInvalidValue;
  const LifParams lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  const dim3 grid(cf_blocks(Cout, 256)), block(256);
  hipStream_t st = (hipStream_t)stream;
  switch (cf_lif_mode(lif)) {
    case LM_HARD0_DECAY_P2:
      hipLaunchKernelGGL(bias_response_kernel<LM_HARD0_DECAY_P2>, grid, block, 0, st, alpha, beta,
                         (int)Cout, (int)T, pool, lif, v_final, fires);
      break;
    case LM_HARD_DECAY_P2:
      hipLaunchKernelGGL(bias_response_kernel<LM_HARD_DECAY_P2>, grid, block, 0, st, alpha, beta,
                         (int)Cout, (int)T, pool, lif, v_final, fires);
      break;
    default:
      hipLaunchKernelGGL(bias_response_kernel<LM_GENERIC>, grid, block, 0, st, alpha, beta,
                         (int)Cout, (int)T, pool, lif, v_final, fires);
  }
  return (int)hipGetLastError();
}

// 3x3 convolutions (stride 1 or 2, any padding) with halo staging; the
// caller picks the tile (tile_h x tile_w in {8x8, 8x16}; 8x16 only with
// stride 1).  u8: the copies (x, identity_nhwc, out_nhwc) hold one byte per
// channel (8x8 tiles, lean LIF epilogue).
static int conv_halo(const void* x, const void* w_packed, const float* alpha,
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
                     int decay_input, int u8, void* stream) {
  HaloArgs a;
  const int rc = make_halo_args(a, x, w_packed, alpha, beta, v_in, v_out, out, out_nhwc, cp_out,
                                identity, identity_nhwc, cp_id, identity_mode, ag_mask,
                                tile_order, nnz, nz_out, x_desc, id_desc, out_desc, bias_info,
                                id_nnz, numel,
                                sparse_threshold, T, B, Cp, Cout,
                                Coutp, H, W, Ho, Wo, ksize, stride, pad, tile_h, tile_w,
                                group_size, epilogue, tau, v_th, v_reset, hard_reset,
                                decay_input);
  if (rc) return rc;
  if (u8 && (tile_w != 8 || epilogue != EPI_LIF || out || identity || !out_nhwc ||
             Cout % 32 != 0 || cp_out % 8 != 0 || Cp % 32 != 0))
    return (int)hipErrorInvalidValue;
  a.u8 = u8 ? 1 : 0;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (ksize == 1)
    e = stride == 1 ? launch_halo<8, 8, 1, 1>(a, epilogue, st) : launch_halo<8, 8, 2, 1>(a, epilogue, st);
  else if (stride == 1 && tile_w == 16)
    e = launch_halo<8, 16, 1>(a, epilogue, st);
  else if (stride == 1)
    e = launch_halo<8, 8, 1>(a, epilogue, st);
  else
    e = launch_halo<8, 8, 2>(a, epilogue, st);
  return (int)e;
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
                        int decay_input, void* stream) {
  return conv_halo(x, w_packed, alpha, beta, v_in, v_out, out, out_nhwc, cp_out, identity,
                   identity_nhwc, cp_id, identity_mode, ag_mask, tile_order, nnz, nz_out, x_desc,
                   id_desc, out_desc, bias_info, id_nnz, numel, sparse_threshold, T, B, Cp, Cout,
                   Coutp, H, W, Ho, Wo, ksize, stride, pad, tile_h, tile_w, group_size, epilogue,
                   tau, v_th, v_reset, hard_reset, decay_input, 0, stream);
}

CF_API int cf_conv_halo_u8(const void* x, const void* w_packed, const float* alpha,
                           const float* beta, const float* v_in, float* v_out,
                           void* out_copy, int64_t cp_out, const void* identity_copy,
                           int64_t cp_id, const int32_t* ag_mask, const int32_t* tile_order,
                           const unsigned long long* nnz, unsigned long long* nz_out,
                           const void* x_desc, const void* id_desc, void* out_desc,
                           int bias_info, const unsigned long long* id_nnz,
                           int64_t numel, double sparse_threshold,
                           int64_t T, int64_t B, int64_t Cp, int64_t Cout, int64_t Coutp,
                           int64_t H, int64_t W, int64_t Ho, int64_t Wo, int64_t ksize,
                           int64_t stride, int64_t pad, int64_t group_size, double tau,
                           double v_th, double v_reset, int hard_reset, int decay_input,
                           void* stream) {
  return conv_halo(x, w_packed, alpha, beta, v_in, v_out, nullptr, out_copy, cp_out, nullptr,
                   identity_copy, cp_id, identity_copy ? ID_ADD_SPIKE : 0, ag_mask, tile_order,
                   nnz, nz_out, x_desc, id_desc, out_desc, bias_info, id_nnz, numel,
                   sparse_threshold, T, B, Cp, Cout, Coutp, H, W, Ho, Wo, ksize, stride, pad, 8,
                   8, group_size, EPI_LIF, tau, v_th, v_reset, hard_reset, decay_input, 1,
                   stream);
}

static int conv_halo_pair(
    const void* x, const unsigned long long* nnz, const void* x_desc, int64_t numel,
    int64_t T, int64_t B, int64_t Cp, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
    const void* w_a, const float* alpha_a, const float* beta_a, const float* v_in_a,
    float* v_out_a, void* out_a, int64_t cp_out_a, unsigned long long* nz_a, void* desc_a, int bias_info_a,
    int64_t Cout_a, int64_t Coutp_a, int64_t pad_a,
    const void* w_b, const float* alpha_b, const float* beta_b, const float* v_in_b,
    float* v_out_b, void* out_b, int64_t cp_out_b, unsigned long long* nz_b, void* desc_b, int bias_info_b,
    int64_t Cout_b, int64_t Coutp_b, int64_t pad_b,
    double tau, double v_th, double v_reset, int hard_reset, int decay_input, int u8,
    void* stream) {
  if (!out_a || !out_b || Cout_a % 32 != 0 || Cout_b % 32 != 0) return (int)hipErrorInvalidValue;
  if (u8 && (cp_out_a % 8 != 0 || cp_out_b % 8 != 0 || Cp % 32 != 0))
    return (int)hipErrorInvalidValue;
  HaloArgs a, b;
  int rc = make_halo_args(a, x, w_a, alpha_a, beta_a, v_in_a, v_out_a, nullptr, out_a, cp_out_a,
                          nullptr, nullptr, 0, 0, nullptr, nullptr, nnz, nz_a, x_desc, nullptr,
                          desc_a, bias_info_a, nullptr, numel, 2.0, T, B,
                          Cp, Cout_a, Coutp_a, H, W, Ho, Wo, 3, 2, pad_a, 8, 8, 0, EPI_LIF, tau,
                          v_th, v_reset, hard_reset, decay_input);
  if (rc) return rc;
  rc = make_halo_args(b, x, w_b, alpha_b, beta_b, v_in_b, v_out_b, nullptr, out_b, cp_out_b,
                      nullptr, nullptr, 0, 0, nullptr, nullptr, nnz, nz_b, x_desc, nullptr,
                      desc_b, bias_info_b, nullptr, numel, 2.0, T, B, Cp,
                      Cout_b, Coutp_b, H, W, Ho, Wo, 1, 2, pad_b, 8, 8, 0, EPI_LIF, tau, v_th,
                      v_reset, hard_reset, decay_input);
  if (rc) return rc;
  a.u8 = b.u8 = u8 ? 1 : 0;
  // each part's workgroup count as its own launch (below 2^23 together)
  const int64_t nLa = B * a.GH * a.GW * (Coutp_a / 64), nLb = B * b.GH * b.GW * (Coutp_b / 64);
  if (nLa + nLb >= ((int64_t)1 << 23)) return (int)hipErrorInvalidValue;
  const dim3 grid((unsigned)(nLa + nLb)), block(256);
  hipStream_t st = (hipStream_t)stream;
  const int lm = cf_lif_mode(a.lif);
  const int ob = T <= halo_tb<2, 3>() ? 2 : (T <= halo_tb<2, 1>() ? 1 : 0);
#define CF_PAIR(LMV)                                                                          \
  do {                                                                                        \
    if (u8) {                                                                                 \
      if (ob == 2)                                                                            \
        hipLaunchKernelGGL((conv_halo_pair_kernel<LMV, true, true, true>), grid, block, 0, st, \
                           a, b, (int)nLa);                                                   \
      else if (ob == 1)                                                                       \
        hipLaunchKernelGGL((conv_halo_pair_kernel<LMV, false, true, true>), grid, block, 0, st, \
                           a, b, (int)nLa);                                                   \
      else                                                                                    \
        hipLaunchKernelGGL((conv_halo_pair_kernel<LMV, false, false, true>), grid, block, 0,  \
                           st, a, b, (int)nLa);                                               \
    } else if (ob == 2)                                                                       \
      hipLaunchKernelGGL((conv_halo_pair_kernel<LMV, true, true>), grid, block, 0, st, a, b,   \
                         (int)nLa);                                                           \
    else if (ob == 1)                                                                         \
      hipLaunchKernelGGL((conv_halo_pair_kernel<LMV, false, true>), grid, block, 0, st, a, b,  \
                         (int)nLa);                                                           \
    else                                                                                      \
      hipLaunchKernelGGL((conv_halo_pair_kernel<LMV, false, false>), grid, block, 0, st, a, b, \
                         (int)nLa);                                                           \
  } while (0)
  if (lm == LM_HARD0_DECAY_P2) CF_PAIR(LM_HARD0_DECAY_P2);
  else if (lm == LM_HARD_DECAY_P2) CF_PAIR(LM_HARD_DECAY_P2);
  else CF_PAIR(LM_GENERIC);
#undef CF_PAIR
  return (int)hipGetLastError();
}

CF_API int cf_conv_halo_pair(
    const void* x, const unsigned long long* nnz, const void* x_desc, int64_t numel,
    int64_t T, int64_t B, int64_t Cp, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
    const void* w_a, const float* alpha_a, const float* beta_a, const float* v_in_a,
    float* v_out_a, void* out_a, int64_t cp_out_a, unsigned long long* nz_a, void* desc_a,
    int bias_info_a, int64_t Cout_a, int64_t Coutp_a, int64_t pad_a,
    const void* w_b, const float* alpha_b, const float* beta_b, const float* v_in_b,
    float* v_out_b, void* out_b, int64_t cp_out_b, unsigned long long* nz_b, void* desc_b,
    int bias_info_b, int64_t Cout_b, int64_t Coutp_b, int64_t pad_b,
    double tau, double v_th, double v_reset, int hard_reset, int decay_input, void* stream) {
  return conv_halo_pair(x, nnz, x_desc, numel, T, B, Cp, H, W, Ho, Wo, w_a, alpha_a, beta_a,
                        v_in_a, v_out_a, out_a, cp_out_a, nz_a, desc_a, bias_info_a, Cout_a,
                        Coutp_a, pad_a, w_b, alpha_b, beta_b, v_in_b, v_out_b, out_b, cp_out_b,
                        nz_b, desc_b, bias_info_b, Cout_b, Coutp_b, pad_b, tau, v_th, v_reset,
                        hard_reset, decay_input, 0, stream);
}

CF_API int cf_conv_halo_pair_u8(
    const void* x, const unsigned long long* nnz, const void* x_desc, int64_t numel,
    int64_t T, int64_t B, int64_t Cp, int64_t H, int64_t W, int64_t Ho, int64_t Wo,
    const void* w_a, const float* alpha_a, const float* beta_a, const float* v_in_a,
    float* v_out_a, void* out_a, int64_t cp_out_a, unsigned long long* nz_a, void* desc_a,
    int bias_info_a, int64_t Cout_a, int64_t Coutp_a, int64_t pad_a,
    const void* w_b, const float* alpha_b, const float* beta_b, const float* v_in_b,
    float* v_out_b, void* out_b, int64_t cp_out_b, unsigned long long* nz_b, void* desc_b,
    int bias_info_b, int64_t Cout_b, int64_t Coutp_b, int64_t pad_b,
    double tau, double v_th, double v_reset, int hard_reset, int decay_input, void* stream) {
  return conv_halo_pair(x, nnz, x_desc, numel, T, B, Cp, H, W, Ho, Wo, w_a, alpha_a, beta_a,
                        v_in_a, v_out_a, out_a, cp_out_a, nz_a, desc_a, bias_info_a, Cout_a,
                        Coutp_a, pad_a, w_b, alpha_b, beta_b, v_in_b, v_out_b, out_b, cp_out_b,
                        nz_b, desc_b, bias_info_b, Cout_b, Coutp_b, pad_b, tau, v_th, v_reset,
                        hard_reset, decay_input, 1, stream);
}
