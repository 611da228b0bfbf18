// Library metadata, error strings and the matrix-core operand layout probe.
// cf_common.h first: the C-ABI header's constant macros must not rename its
// enumerators
#include "cf_common.h"
#include "catfuse_amd.h"

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

// One wave computes D(32x32) = A(32x16) * B(16x32) with the operand and
// accumulator lane mapping that conv_mfma.hip assumes:
//   A: lane l holds A[l%32][8*(l/32) .. +7]      B: lane l holds B[8*(l/32) .. +7][l%32]
//   D: lane l, register r holds D[8*(r/4) + 4*(l/32) + r%4][l%32]
__global__ void mfma_layout_probe(const _Float16* __restrict__ A, const _Float16* __restrict__ B,
                                  float* __restrict__ D) {
  const int l = threadIdx.x;
  h8 a, b;
  for (int j = 0; j < 8; ++j) {
    a[j] = A[(l % 32) * 16 + 8 * (l / 32) + j];
    b[j] = B[(8 * (l / 32) + j) * 32 + (l % 32)];
  }
  f16v c;
  for (int r = 0; r < 16; ++r) c[r] = 0.0f;
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  for (int r = 0; r < 16; ++r) D[(8 * (r / 4) + 4 * (l / 32) + (r % 4)) * 32 + (l % 32)] = c[r];
}

}  // namespace

CF_API int cf_version(void) { return 100; }

CF_API const char* cf_error_string(int code) {
  if (code == CF_ERROR_NOALLOC_LIMIT)
    return "input exceeds the no-allocation workspace (CF_NOALLOC_MAX_PIXELS / "
           "CF_NOALLOC_MAX_TILES)";
  return hipGetErrorString((hipError_t)code);
}

CF_API int cf_probe_mfma_layout(const void* A, const void* B, float* D, void* stream) {
  if (!A || !B || !D) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_layout_probe, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const _Float16*)A, (const _Float16*)B, D);
  return (int)hipGetLastError();
}
