// The SparseFlow-routed fused conv without caller workspace, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// cf_conv_mfma's SparseFlow route needs four device buffers beside its
// inputs and outputs: the input's per-pixel channel-group activity bits
// (cf_scan_nhwc), its nonzero-count block, the prescan tile masks
// (cf_prescan_tiles) and the compacted tile order (cf_compact_tiles).  Here
// they live in one file-scope device array,
// `scratch`, of CF_NOALLOC_SCRATCH_BYTES per GPU: the runtime places a copy
// of it on every device the library runs on, and it stays until the process
// ends.  Its device address is looked up once per device with
// hipGetSymbolAddress (host code only ever passes that address, never the
// array's name, which on the host is a stand-in symbol).  Every call on one
// GPU shares that GPU's array: calls that overlap on one GPU (streams not
// ordered against each other) race.  The count block is cleared by a kernel
// at the start of every call; the activity bits, tile masks and tile order
// are fully rewritten by every call before they are read.
#include <mutex>

// cf_common.h first: the C-ABI header's constant macros must not rename its
// enumerators
#include "cf_common.h"
#include "catfuse_amd.h"

namespace {

constexpr size_t NA_COUNT_BYTES = 4096;   // count block (CF_COUNT_BLOCK_WORDS u64) + pad
constexpr size_t NA_ACT_BYTES = (size_t)CF_NOALLOC_MAX_PIXELS * 4;
constexpr size_t NA_TILE_BYTES = (size_t)CF_NOALLOC_MAX_TILES * 4;
constexpr size_t NA_ORDER_BYTES = (size_t)CF_NOALLOC_MAX_TILES * 4 + 256;   // count + tiles
static_assert(CF_COUNT_BLOCK_WORDS * 8 <= NA_COUNT_BYTES, "count block exceeds its slot");
static_assert(NA_COUNT_BYTES + NA_ACT_BYTES + 2 * NA_TILE_BYTES + NA_ORDER_BYTES ==
                  CF_NOALLOC_SCRATCH_BYTES,
              "scratch layout does not add up to CF_NOALLOC_SCRATCH_BYTES");

__device__ __align__(256) unsigned char scratch[CF_NOALLOC_SCRATCH_BYTES];

constexpr int NA_MAX_DEVICES = 64;
std::mutex na_mutex;
void* na_ptr[NA_MAX_DEVICES] = {};

// The current device's copy of `scratch` (looked up once per device).
int na_scratch(unsigned char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= NA_MAX_DEVICES) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(na_mutex);
  if (!na_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    na_ptr[dev] = p;
  }
  *out = (unsigned char*)na_ptr[dev];
  return 0;
}

__global__ void na_clear_block(unsigned long long* __restrict__ blk) {
  for (int i = threadIdx.x; i < CF_COUNT_BLOCK_WORDS; i += blockDim.x) blk[i] = 0ull;
}

}  // namespace

CF_API int cf_conv_sparse_noalloc(
    const void* x, int64_t Cin, const void* w_packed, const float* alpha, const float* beta,
    const float* v_in, float* v_out, float* out, void* out_nhwc, int64_t cp_out,
    const float* identity, const void* identity_nhwc, int64_t cp_id, int identity_mode,
    unsigned long long* nz_out, double sparse_threshold, int64_t T, int64_t B, int64_t Cp,
    int64_t Cout, int64_t Coutp, int64_t H, int64_t W, int64_t Ho, int64_t Wo, int64_t ksize,
    int64_t stride, int64_t pad, int64_t tile_h, int64_t tile_w, int64_t group_size,
    int epilogue, double tau, double v_th, double v_reset, int hard_reset, int decay_input,
    void* stream) {
  // Shape checks before anything touches the device.
  if (!x || T <= 0 || B <= 0 || Cin <= 0 || Cp < Cin || H <= 0 || W <= 0 || Ho <= 0 ||
      Wo <= 0 || ksize <= 0 || stride <= 0 || pad < 0 || tile_h <= 0 || tile_w <= 0 ||
      group_size <= 0 || group_size % 8 != 0 || (Cin + group_size - 1) / group_size > 32)
    return (int)hipErrorInvalidValue;
  const int64_t NB = T * B;
  const int64_t GH = (Ho + tile_h - 1) / tile_h, GW = (Wo + tile_w - 1) / tile_w;
  if (NB * H * W > (int64_t)CF_NOALLOC_MAX_PIXELS || NB * GH * GW > (int64_t)CF_NOALLOC_MAX_TILES)
    return CF_ERROR_NOALLOC_LIMIT;
  unsigned char* s = nullptr;
  int rc = na_scratch(&s);
  if (rc) return rc;
  unsigned long long* blk = (unsigned long long*)s;
  uint32_t* act = (uint32_t*)(s + NA_COUNT_BYTES);
  int32_t* ag = (int32_t*)(s + NA_COUNT_BYTES + NA_ACT_BYTES);
  int32_t* tc = (int32_t*)(s + NA_COUNT_BYTES + NA_ACT_BYTES + NA_TILE_BYTES);
  int32_t* order = (int32_t*)(s + NA_COUNT_BYTES + NA_ACT_BYTES + 2 * NA_TILE_BYTES);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(na_clear_block, dim3(1), dim3(256), 0, st, blk);
  rc = (int)hipGetLastError();
  if (rc) return rc;
  rc = cf_scan_nhwc(x, NB, H, W, Cp, Cin, act, (int)group_size, 1e-6f, blk, stream);
  if (rc) return rc;
  const int64_t groups = (Cin + group_size - 1) / group_size;
  rc = cf_prescan_tiles(act, NB, H, W, Ho, Wo, ksize, stride, pad, tile_h, tile_w, groups, ag,
                        tc, stream);
  if (rc) return rc;
  // tile masks are per (step, image, tile); the conv's tiles are (image, tile)
  rc = cf_compact_tiles(ag, T, B * GH * GW, groups, 0.0, -1.0, 0.0, order, stream);
  if (rc) return rc;
  return cf_conv_mfma(x, w_packed, alpha, beta, v_in, v_out, out, out_nhwc, cp_out, identity,
                      identity_nhwc, cp_id, identity_mode, ag, order, blk, nz_out,
                      nullptr, nullptr, nullptr, 0, nullptr, NB * Cin * H * W,
                      sparse_threshold, T, B, Cp, Cout, Coutp, H, W, Ho, Wo, ksize, ksize,
                      stride, pad, B, tile_h, tile_w, group_size, epilogue, tau, v_th, v_reset,
                      hard_reset, decay_input, stream);
}
