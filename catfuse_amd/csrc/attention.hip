// Spiking self-attention core with its LIF (Spikformer SSA: Q K^T V * scale,
// then attn_lif), on the matrix cores.
//
// Reference: models/spikformer_github.py:139-160 (SSA.forward: q, k, v are
// spike tensors [T, B, heads, N, dh]; attn = (q @ k^T) * scale; y = attn @ v;
// attn_lif over T).  There is no softmax, so for binary Q, K, V the product
// is evaluated as Q (K^T V):
//   KV = K^T V   dh x dh integers <= N: exact as fp32 sums, then as fp16
//                (N <= 2048) for the second product;
//   Y  = Q KV    N x dh integers <= N * dh: exact in the fp32 accumulators;
//   z  = Y * scale, one rounding; the LIF over T with v in registers.
// The reference's fp32 evaluation rounds attn and every partial sum of
// attn @ v; this one rounds once, so z differs from it by rounding only.
//
// Layouts (token-major, the fp16 NHWC copies of the fused linears): q, k, v
// are fp16 [T*B][N][pitch] with head h at channels off + h*dh .. + dh - 1
// (off = qoff, koff, voff; one concatenated QKV tensor or three tensors);
// out is fp16 [T*B][N][cp_out] with head h at channels h*dh ..; v_in / v_out
// fp32 [B][N][heads*dh].  One workgroup per (b, head), all T steps; dh = 32.
// An input whose count block (nnz) publishes zero takes the zero route: no
// operand reads and no MFMAs, z = 0 (the bits Q (K^T V) * scale has for zero
// operands) into the LIF.
#include "cf_common.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int DH = 32;          // head dim (one MFMA tile edge)
constexpr int NMAX = 256;       // tokens per image this kernel stages (LDS)

struct AttnArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  int qoff, koff, voff, pitch;
  _Float16* out;
  int cp_out;
  const float* v_in;
  float* v_out;
  const unsigned long long* nnz;   // count block of Q, K, V (one tensor), or null
  unsigned long long* nz_out;
  CfOutDesc* out_desc;             // output descriptor (CfOutDesc), or null
  int zero_info;                   // CF_BIAS_* for the LIF on z = 0 (needs out_desc)
  int T, B, N, heads;
  float scale;
  LifParams lif;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

template <int LM>
__global__ __launch_bounds__(256) void spike_attention_kernel(AttnArgs a) {
  // K and V of the current step, transposed ([d][n], n padded to a
  // multiple of 16 with zeros) so each MFMA operand is one 16-byte read.
  // Rows are NMAX + 8 halves apart (528 bytes, 132 dwords: 4 banks on from
  // the row above), so the 32 rows an operand read touches spread over all
  // banks instead of sharing four.
  constexpr int KLD = NMAX + 8;
  __shared__ __attribute__((aligned(16))) _Float16 kT[DH][KLD];
  __shared__ __attribute__((aligned(16))) _Float16 vT[DH][KLD];
  __shared__ __attribute__((aligned(16))) float kvp[4][DH][DH + 1];  // per-wave partial K^T V
  __shared__ __attribute__((aligned(16))) _Float16 kvT[DH][DH];      // (K^T V)^T as fp16
  __shared__ unsigned any_sh[4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5, col = lane & 31;
  const int b = blockIdx.x / a.heads, h = blockIdx.x % a.heads;
  const int N = a.N, C = a.heads * DH;
  const int NP = (N + 15) & ~15;            // K-dim of K^T V, padded
  const int nks = NP / 16;                  // its 16-deep MFMA steps
  const int ntile = (N + 31) / 32;          // 32-token row tiles of Y
  // row tiles of this wave: wave, wave + 4
  constexpr int MAXT = NMAX / 32 / 4;       // row tiles per wave at most
  float v[MAXT][16];
  uint32_t anyw = 0u;
  const bool zero_in = a.nnz != nullptr && cf_count_read(a.nnz) == 0ull;   // uniform
  // An all-zero Q/K/V from the initial state drives every neuron with z = 0:
  // when the caller knows that the LIF never fires on it and holds the
  // final potential, the output is all zero and the state uniform, so
  // workgroup 0 records that in the descriptor and the count, and no
  // workgroup stores anything else.
  if (zero_in && a.v_in == nullptr && a.out_desc != nullptr && (a.zero_info & CF_BIAS_SILENT) &&
      ((a.zero_info & CF_BIAS_VCHAN) || a.v_out == nullptr)) {
    if (blockIdx.x == 0 && tid == 0) {
      if (a.nz_out != nullptr) a.nz_out[1] = 0ull;
      a.out_desc->copy = CF_COPY_ZERO;
      a.out_desc->vstate = (a.zero_info & CF_BIAS_VCHAN) ? 1u : 0u;
      a.out_desc->alias = nullptr;
    }
    return;
  }
  if (a.out_desc != nullptr && blockIdx.x == 0 && tid == 0) {
    a.out_desc->copy = CF_COPY_WRITTEN;
    a.out_desc->vstate = 0u;
    a.out_desc->alias = nullptr;
  }

  // initial membrane potentials
#pragma unroll
  for (int i = 0; i < MAXT; ++i) {
    const int tile = wave + 4 * i;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int n = tile * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
      float v0 = lif_initial_v(a.lif);
      if (a.v_in && tile < ntile && n < N) v0 = a.v_in[((size_t)b * N + n) * C + h * DH + col];
      v[i][r] = v0;
    }
  }

  for (int t = 0; t < a.T; ++t) {
    const size_t img = (size_t)t * a.B + b;
    const _Float16* qb = a.q + img * N * a.pitch + a.qoff + h * DH;
    const _Float16* kb = a.k + img * N * a.pitch + a.koff + h * DH;
    const _Float16* vb = a.v + img * N * a.pitch + a.voff + h * DH;
    // this step's Q rows (A operand: row tile*32 + col, k 16 hi ..), issued
    // first so their latency overlaps the K^T V phase; rows beyond N read
    // zeros (out of the buffer's range)
    const __amdgpu_buffer_rsrc_t rq = attn_rsrc(qb, (uint32_t)(((size_t)(N - 1) * a.pitch + DH) * 2));
    h8 qr[MAXT][2];
    h8 kv0 = {}, kv1 = {};
    if (!zero_in) {
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int n = (wave + 4 * i) * 32 + col;
      const uint32_t qo = n < N ? (uint32_t)(((size_t)n * a.pitch) * 2) : 0x80000000u;
      qr[i][0] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 16 * hi, 0, 0));
      qr[i][1] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 32 + 16 * hi, 0, 0));
    }
    __syncthreads();  // the previous step's reads of kT / vT / kvT are complete
    // stage K, V transposed: unit u = tid + 256 i = (token u / 4, 8-channel
    // part u % 4); every load of the thread is issued before the first LDS
    // write, so the step waits for one load latency, not one per unit
    constexpr int SU = NMAX * 4 / 256;
    h8 kx[SU], vx[SU];
#pragma unroll
    for (int i = 0; i < SU; ++i) {
      const int u = tid + 256 * i, n = u >> 2, c = (u & 3) * 8;
      kx[i] = h8{};
      vx[i] = h8{};
      if (n < N) {
        kx[i] = *reinterpret_cast<const h8*>(kb + (size_t)n * a.pitch + c);
        vx[i] = *reinterpret_cast<const h8*>(vb + (size_t)n * a.pitch + c);
      }
    }
#pragma unroll
    for (int i = 0; i < SU; ++i) {
      const int u = tid + 256 * i, n = u >> 2, c = (u & 3) * 8;
      if (n < NP) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          kT[c + j][n] = kx[i][j];
          vT[c + j][n] = vx[i][j];
        }
      }
    }
    __syncthreads();
    // K^T V: wave w accumulates the K steps w, w + 4, ...
    {
      f32x16 acc = {};
      for (int s = wave; s < nks; s += 4) {
        const int n0 = s * 16 + 8 * hi;
        const h8 av = *reinterpret_cast<const h8*>(&kT[col][n0]);   // A[i = col][n]
        const h8 bv = *reinterpret_cast<const h8*>(&vT[col][n0]);   // B[n][j = col]
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) kvp[wave][8 * (r >> 2) + 4 * hi + (r & 3)][col] = acc[r];
    }
    __syncthreads();
    // sum the partials (integers: exact in any order) and keep (K^T V)^T in
    // fp16 (entries <= N, exact): kvT[j][i] = KV[i][j]
    for (int e = tid; e < DH * DH; e += 256) {
      const int i = e >> 5, j = e & 31;
      const float s = kvp[0][i][j] + kvp[1][i][j] + kvp[2][i][j] + kvp[3][i][j];
      kvT[j][i] = (_Float16)s;
    }
    __syncthreads();
    // Y = Q KV per 32-token row tile; B operand: KV[i][j = col] for i in the step
    kv0 = *reinterpret_cast<const h8*>(&kvT[col][8 * hi]);
    kv1 = *reinterpret_cast<const h8*>(&kvT[col][16 + 8 * hi]);
    }  // !zero_in
    _Float16* ob = a.out + img * N * a.cp_out + h * DH;
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int tile = wave + 4 * i;
      if (tile >= ntile) break;
      f32x16 y = {};
      if (!zero_in) {
        y = __builtin_amdgcn_mfma_f32_32x32x16_f16(qr[i][0], kv0, y, 0, 0, 0);
        y = __builtin_amdgcn_mfma_f32_32x32x16_f16(qr[i][1], kv1, y, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int nr = tile * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
        const float z = y[r] * a.scale;
        float vv = lif_charge_m<LM>(v[i][r], z, a.lif);
        const bool f = lif_fire_reset_bit<LM>(vv, a.lif);
        v[i][r] = vv;
        if (nr < N) {
          ob[(size_t)nr * a.cp_out + col] = f ? (_Float16)1.0f : (_Float16)0.0f;
          anyw |= f ? 1u : 0u;
        }
      }
    }
  }
  if (a.v_out) {
#pragma unroll
    for (int i = 0; i < MAXT; ++i) {
      const int tile = wave + 4 * i;
      if (tile >= ntile) break;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = tile * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (n < N) a.v_out[((size_t)b * N + n) * C + h * DH + col] = v[i][r];
      }
    }
  }
  if (a.nz_out) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (tid == 0) cf_count_publish(a.nz_out, any ? 1ull : 0ull, blockIdx.x, gridDim.x);
  }
}


// ---------------------------------------------------------------------------
// Two-pass form for any token count and head dims 32 or 64.
//
// Pass 1 (attn_kv_kernel): one workgroup per (step, image, head) reduces
// K^T V over all N tokens, 256 at a time: the chunk's K and V staged
// transposed in LDS (zero-padded to whole 16-token MFMA steps), the dh x dh
// result as 32 x 32 tiles (dh = 64: one tile per wave over every token;
// dh = 32: the four waves take every fourth 16-token step and their partial
// tiles are summed in LDS).  Every product is 0/1 and every partial sum an
// integer below 2^24, so the fp32 result is exact in any order.  Written to
// the workspace kv [T*B*heads][dh][dh] (row i of K^T, column j of V).
//
// Pass 2 (attn_y_lif_kernel): one workgroup per (image, head, 128-token
// block), all T steps: KV_t is split into two fp16 limbs that are exact
// (hi = KV & ~1023, lo = KV & 1023: integers below 2^16), Y = Q KV_hi +
// Q KV_lo on the matrix cores (every partial sum an integer below 2^24:
// exact), z = Y * scale (one rounding), the LIF with v in registers (wave w:
// tokens 32 w .. 32 w + 31 of the block, dh channels).  The values equal the
// single-pass kernel's (same exact Y, same rounding, same LIF).
constexpr int KV_CHUNK = 256;    // tokens per staged chunk of pass 1
constexpr int Y_TOKENS = 128;    // tokens per workgroup of pass 2

struct AttnKvArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  int qoff, koff, voff, pitch;
  _Float16* out;
  int cp_out;
  const float* v_in;
  float* v_out;
  float* kv;                       // workspace [T*B*heads][dh][dh]
  const unsigned long long* nnz;
  unsigned long long* nz_out;
  CfOutDesc* out_desc;
  int zero_info;
  int T, B, N, heads;
  float scale;
  LifParams lif;
};

// The zero route's elision (as the single-pass kernel): an all-zero Q/K/V
// from the initial state with a silent, caller-held LIF response to z = 0
// records the output as all zero and stores nothing else.
__device__ __forceinline__ bool attn_zero_elided(const AttnKvArgs& a, bool zero_in) {
  return zero_in && a.v_in == nullptr && a.out_desc != nullptr &&
         (a.zero_info & CF_BIAS_SILENT) && ((a.zero_info & CF_BIAS_VCHAN) || a.v_out == nullptr);
}

template <int DHV>
__global__ __launch_bounds__(256) void attn_kv_kernel(AttnKvArgs a) {
  constexpr int KLD = KV_CHUNK + 8;   // row pitch (halves): rows 4 banks apart
  __shared__ __attribute__((aligned(16))) _Float16 kT[DHV][KLD];
  __shared__ __attribute__((aligned(16))) _Float16 vT[DHV][KLD];
  __shared__ __attribute__((aligned(16))) float kvp[DHV == 32 ? 4 : 1][32][33];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5, col = lane & 31;
  const int img = blockIdx.x / a.heads, h = blockIdx.x % a.heads;   // img = t * B + b
  const int N = a.N;
  if (a.nnz != nullptr && cf_count_read(a.nnz) == 0ull) return;     // pass 2 takes z = 0
  const _Float16* kb = a.k + (size_t)img * N * a.pitch + a.koff + h * DHV;
  const _Float16* vb = a.v + (size_t)img * N * a.pitch + a.voff + h * DHV;
  // dh = 64: wave (wi, wj) computes the tile KV[32 wi ..][32 wj ..]
  const int wi = DHV == 64 ? (wave >> 1) : 0, wj = DHV == 64 ? (wave & 1) : 0;
  f32x16 acc = {};
  constexpr int PARTS = DHV / 8;                   // 8-channel parts per token
  constexpr int SU = KV_CHUNK * PARTS / 256;       // staged units per thread
  for (int n0 = 0; n0 < N; n0 += KV_CHUNK) {
    const int nc = min(KV_CHUNK, N - n0);
    const int ncp = (nc + 15) & ~15;
    h8 kx[SU], vx[SU];
#pragma unroll
    for (int i = 0; i < SU; ++i) {
      const int u = tid + 256 * i, n = u / PARTS, c = (u % PARTS) * 8;
      kx[i] = h8{};
      vx[i] = h8{};
      if (n < nc) {
        kx[i] = *reinterpret_cast<const h8*>(kb + (size_t)(n0 + n) * a.pitch + c);
        vx[i] = *reinterpret_cast<const h8*>(vb + (size_t)(n0 + n) * a.pitch + c);
      }
    }
    __syncthreads();   // the previous chunk's operand reads are complete
#pragma unroll
    for (int i = 0; i < SU; ++i) {
      const int u = tid + 256 * i, n = u / PARTS, c = (u % PARTS) * 8;
      if (n < ncp) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          kT[c + j][n] = kx[i][j];
          vT[c + j][n] = vx[i][j];
        }
      }
    }
    __syncthreads();
    const int nks = ncp / 16;
    for (int s = (DHV == 32 ? wave : 0); s < nks; s += (DHV == 32 ? 4 : 1)) {
      const int nn = s * 16 + 8 * hi;
      const h8 av = *reinterpret_cast<const h8*>(&kT[32 * wi + col][nn]);   // A[i][n]
      const h8 bv = *reinterpret_cast<const h8*>(&vT[32 * wj + col][nn]);   // B[n][j]
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc, 0, 0, 0);
    }
  }
  float* kvo = a.kv + (size_t)blockIdx.x * DHV * DHV;
  if constexpr (DHV == 64) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * wi + 8 * (r >> 2) + 4 * hi + (r & 3);
      kvo[i * DHV + 32 * wj + col] = acc[r];
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) kvp[wave][8 * (r >> 2) + 4 * hi + (r & 3)][col] = acc[r];
    __syncthreads();
    for (int e = tid; e < 32 * 32; e += 256) {
      const int i = e >> 5, j = e & 31;
      kvo[e] = kvp[0][i][j] + kvp[1][i][j] + kvp[2][i][j] + kvp[3][i][j];
    }
  }
}

template <int DHV, int LM>
__global__ __launch_bounds__(256) void attn_y_lif_kernel(AttnKvArgs a) {
  constexpr int NCT = DHV / 32;                       // 32-channel column tiles
  __shared__ __attribute__((aligned(16))) _Float16 kvT[2][DHV][DHV + 8];   // limbs, [j][i]
  __shared__ unsigned any_sh[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5, col = lane & 31;
  const int nblk = (a.N + Y_TOKENS - 1) / Y_TOKENS;
  const int bh = blockIdx.x / nblk, blk = blockIdx.x % nblk;
  const int b = bh / a.heads, h = bh % a.heads;
  const int N = a.N, C = a.heads * DHV;
  const int tile0 = blk * Y_TOKENS + 32 * wave;       // this wave's first token
  const bool zero_in = a.nnz != nullptr && cf_count_read(a.nnz) == 0ull;
  if (attn_zero_elided(a, zero_in)) {
    if (blockIdx.x == 0 && tid == 0) {
      if (a.nz_out != nullptr) a.nz_out[1] = 0ull;
      a.out_desc->copy = CF_COPY_ZERO;
      a.out_desc->vstate = (a.zero_info & CF_BIAS_VCHAN) ? 1u : 0u;
      a.out_desc->alias = nullptr;
    }
    return;
  }
  if (a.out_desc != nullptr && blockIdx.x == 0 && tid == 0) {
    a.out_desc->copy = CF_COPY_WRITTEN;
    a.out_desc->vstate = 0u;
    a.out_desc->alias = nullptr;
  }
  float v[NCT][16];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int n = tile0 + 8 * (r >> 2) + 4 * hi + (r & 3);
      float v0 = lif_initial_v(a.lif);
      if (a.v_in && n < N) v0 = a.v_in[((size_t)b * N + n) * C + h * DHV + 32 * ct + col];
      v[ct][r] = v0;
    }
  uint32_t anyw = 0u;
  for (int t = 0; t < a.T; ++t) {
    const size_t img = (size_t)t * a.B + b;
    f32x16 y[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) y[ct] = f32x16{};
    if (!zero_in) {
      // Q rows of this wave's 32 tokens (A operand: row col, k 8 hi ..);
      // rows beyond N read zeros
      const _Float16* qb = a.q + img * N * a.pitch + a.qoff + h * DHV;
      const __amdgpu_buffer_rsrc_t rq =
          attn_rsrc(qb, (uint32_t)(((size_t)(N - 1) * a.pitch + DHV) * 2));
      const int n = tile0 + col;
      const uint32_t qo = n < N ? (uint32_t)(((size_t)n * a.pitch) * 2) : 0x80000000u;
      h8 qr[DHV / 16];
#pragma unroll
      for (int ks = 0; ks < DHV / 16; ++ks)
        qr[ks] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(rq, qo + 32 * ks + 16 * hi, 0, 0));
      // KV_t as two exact fp16 limbs, transposed: kvT[limb][j][i] = KV[i][j]
      const float* kvi = a.kv + (img * a.heads + h) * DHV * DHV;
      __syncthreads();   // the previous step's reads of kvT are complete
      for (int e = tid; e < DHV * DHV; e += 256) {
        const int i = e / DHV, j = e % DHV;
        const uint32_t kvv = (uint32_t)kvi[e];          // an integer below 2^16
        kvT[0][j][i] = (_Float16)(float)(kvv & ~1023u);
        kvT[1][j][i] = (_Float16)(float)(kvv & 1023u);
      }
      __syncthreads();
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int limb = 0; limb < 2; ++limb)
#pragma unroll
          for (int ks = 0; ks < DHV / 16; ++ks) {
            const h8 bv = *reinterpret_cast<const h8*>(&kvT[limb][32 * ct + col][16 * ks + 8 * hi]);
            y[ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(qr[ks], bv, y[ct], 0, 0, 0);
          }
    }
    _Float16* ob = a.out + img * N * a.cp_out + h * DHV;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int nr = tile0 + 8 * (r >> 2) + 4 * hi + (r & 3);
        const float z = y[ct][r] * a.scale;
        float vv = lif_charge_m<LM>(v[ct][r], z, a.lif);
        const bool f = lif_fire_reset_bit<LM>(vv, a.lif);
        v[ct][r] = vv;
        if (nr < N) {
          ob[(size_t)nr * a.cp_out + 32 * ct + col] = f ? (_Float16)1.0f : (_Float16)0.0f;
          anyw |= f ? 1u : 0u;
        }
      }
  }
  if (a.v_out) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = tile0 + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (n < N) a.v_out[((size_t)b * N + n) * C + h * DHV + 32 * ct + col] = v[ct][r];
      }
  }
  if (a.nz_out) {
    const bool any = cf_wg_any(anyw != 0u, any_sh);
    if (tid == 0) cf_count_publish(a.nz_out, any ? 1ull : 0ull, blockIdx.x, gridDim.x);
  }
}

}  // namespace

CF_API int cf_spike_attention_lif(const void* q, const void* k, const void* v, int64_t qoff,
                                  int64_t koff, int64_t voff, int64_t pitch, void* out,
                                  int64_t cp_out, const float* v_in, float* v_out,
                                  const unsigned long long* nnz, unsigned long long* nz_out,
                                  void* out_desc, int zero_info,
                                  int64_t T, int64_t B, int64_t N,
                                  int64_t heads, int64_t head_dim, double scale, double tau,
                                  double v_th, double v_reset, int hard_reset, int decay_input,
                                  void* stream) {
  if (!q || !k || !v || !out || T <= 0 || B <= 0 || N <= 0 || heads <= 0) return (int)hipErrorInvalidValue;
  if (head_dim != DH || N > NMAX) return (int)hipErrorInvalidValue;
  const int64_t C = heads * head_dim;
  if (pitch % 8 != 0 || qoff % 8 != 0 || koff % 8 != 0 || voff % 8 != 0 || qoff < 0 ||
      koff < 0 || voff < 0 || qoff + C > pitch || koff + C > pitch || voff + C > pitch ||
      cp_out < C || T * B * N * pitch > ((int64_t)1 << 40) || B * heads >= (int64_t)CF_MAX_COUNT_WG ||
      (int64_t)(N - 1) * pitch * 2 + 64 > INT32_MAX)
    return (int)hipErrorInvalidValue;
  if ((zero_info & ~(CF_BIAS_SILENT | CF_BIAS_VCHAN)) != 0 || (zero_info && !out_desc))
    return (int)hipErrorInvalidValue;
  AttnArgs a;
  a.q = (const _Float16*)q; a.k = (const _Float16*)k; a.v = (const _Float16*)v;
  a.qoff = (int)qoff; a.koff = (int)koff; a.voff = (int)voff; a.pitch = (int)pitch;
  a.out = (_Float16*)out; a.cp_out = (int)cp_out; a.v_in = v_in; a.v_out = v_out;
  a.nnz = nnz; a.nz_out = nz_out; a.T = (int)T;
  a.out_desc = (CfOutDesc*)out_desc; a.zero_info = zero_info; a.B = (int)B; a.N = (int)N; a.heads = (int)heads;
  a.scale = (float)scale;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  const dim3 grid((unsigned)(B * heads)), block(256);
  const int lm = cf_lif_mode(a.lif);
  hipStream_t st = (hipStream_t)stream;
  if (lm == LM_HARD0_DECAY_P2)
    hipLaunchKernelGGL(spike_attention_kernel<LM_HARD0_DECAY_P2>, grid, block, 0, st, a);
  else if (lm == LM_HARD_DECAY_P2)
    hipLaunchKernelGGL(spike_attention_kernel<LM_HARD_DECAY_P2>, grid, block, 0, st, a);
  else
    hipLaunchKernelGGL(spike_attention_kernel<LM_GENERIC>, grid, block, 0, st, a);
  return (int)hipGetLastError();
}

CF_API int cf_spike_attention_kv_lif(const void* q, const void* k, const void* v, int64_t qoff,
                                     int64_t koff, int64_t voff, int64_t pitch, void* out,
                                     int64_t cp_out, const float* v_in, float* v_out,
                                     float* kv_ws, const unsigned long long* nnz,
                                     unsigned long long* nz_out, void* out_desc, int zero_info,
                                     int64_t T, int64_t B, int64_t N, int64_t heads,
                                     int64_t head_dim, double scale, double tau, double v_th,
                                     double v_reset, int hard_reset, int decay_input,
                                     void* stream) {
  if (!q || !k || !v || !out || !kv_ws || T <= 0 || B <= 0 || N <= 0 || heads <= 0)
    return (int)hipErrorInvalidValue;
  if (head_dim != 32 && head_dim != 64) return (int)hipErrorInvalidValue;
  const int64_t C = heads * head_dim;
  const int64_t nblk = (N + Y_TOKENS - 1) / Y_TOKENS;
  // K^T V entries <= N must stay below 2^16 (two exact fp16 limbs) and Y
  // below 2^24 (exact fp32 sums): N < 65536 / ... head_dim * N < 2^24
  if (N >= 65536 || head_dim * N >= (int64_t)1 << 24) return (int)hipErrorInvalidValue;
  if (pitch % 8 != 0 || qoff % 8 != 0 || koff % 8 != 0 || voff % 8 != 0 || qoff < 0 ||
      koff < 0 || voff < 0 || qoff + C > pitch || koff + C > pitch || voff + C > pitch ||
      cp_out < C || T * B * N * pitch > ((int64_t)1 << 40) ||
      B * heads * nblk >= (int64_t)CF_MAX_COUNT_WG || T * B * heads > INT32_MAX ||
      (int64_t)(N - 1) * pitch * 2 + 128 > INT32_MAX)
    return (int)hipErrorInvalidValue;
  if ((zero_info & ~(CF_BIAS_SILENT | CF_BIAS_VCHAN)) != 0 || (zero_info && !out_desc))
    return (int)hipErrorInvalidValue;
  AttnKvArgs a;
  a.q = (const _Float16*)q; a.k = (const _Float16*)k; a.v = (const _Float16*)v;
  a.qoff = (int)qoff; a.koff = (int)koff; a.voff = (int)voff; a.pitch = (int)pitch;
  a.out = (_Float16*)out; a.cp_out = (int)cp_out; a.v_in = v_in; a.v_out = v_out;
  a.kv = kv_ws; a.nnz = nnz; a.nz_out = nz_out; a.out_desc = (CfOutDesc*)out_desc;
  a.zero_info = zero_info; a.T = (int)T; a.B = (int)B; a.N = (int)N; a.heads = (int)heads;
  a.scale = (float)scale;
  a.lif = cf_make_lif_params(tau, v_th, v_reset, hard_reset, decay_input);
  hipStream_t st = (hipStream_t)stream;
  const dim3 g1((unsigned)(T * B * heads)), g2((unsigned)(B * heads * nblk)), block(256);
  if (head_dim == 64)
    hipLaunchKernelGGL(attn_kv_kernel<64>, g1, block, 0, st, a);
  else
    hipLaunchKernelGGL(attn_kv_kernel<32>, g1, block, 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  const int lm = cf_lif_mode(a.lif);
#define CF_ATTN_Y(DHV)                                                                         \
  do {                                                                                         \
    if (lm == LM_HARD0_DECAY_P2)                                                               \
      hipLaunchKernelGGL((attn_y_lif_kernel<DHV, LM_HARD0_DECAY_P2>), g2, block, 0, st, a);    \
    else if (lm == LM_HARD_DECAY_P2)                                                           \
      hipLaunchKernelGGL((attn_y_lif_kernel<DHV, LM_HARD_DECAY_P2>), g2, block, 0, st, a);     \
    else                                                                                       \
      hipLaunchKernelGGL((attn_y_lif_kernel<DHV, LM_GENERIC>), g2, block, 0, st, a);           \
  } while (0)
  if (head_dim == 64) CF_ATTN_Y(64);
  else CF_ATTN_Y(32);
#undef CF_ATTN_Y
  return (int)hipGetLastError();
}
