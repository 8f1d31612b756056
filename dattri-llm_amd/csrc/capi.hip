// C-ABI plumbing: error reporting, version, and the MFMA lane-layout self test.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace da {

static thread_local char g_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DA_OK;
}

__global__ void zero_f32_2d_kernel(float* out, int64_t rows, int64_t cols, int64_t ld) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * cols) return;
  const int64_t r = idx / cols;
  out[r * ld + (idx - r * cols)] = 0.f;
}

int zero_f32_2d(float* out, int64_t rows, int64_t cols, int64_t ld, hipStream_t stream) {
  const int64_t n = rows * cols;
  if (n <= 0) return DA_OK;
  zero_f32_2d_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(out, rows, cols, ld);
  return check_launch("zero_f32_2d");
}

// One wave computes C = A . B^T for a single 32x32 block with the library's
// operand convention and dumps the accumulator registers verbatim.
template <int DT>
__global__ __launch_bounds__(64) void selftest_mfma_kernel(const char* a, const char* b, float* out) {
  const int lane = threadIdx.x;
  const int row = lane & 31, half = lane >> 5;
  // A and B are (32 x 2 chunks) of 16 bytes: row stride 32 bytes.
  const u32x4 va = ld16(a + row * 32 + half * 16);
  const u32x4 vb = ld16(b + row * 32 + half * 16);
  f32x16 acc = {};
  Mfma32<DT>::mma(acc, va, vb);
#pragma unroll
  for (int r = 0; r < 16; ++r) out[lane * 16 + r] = acc[r];
}

}  // namespace da

extern "C" {

int da_abi_version(void) { return 1; }

const char* da_last_error(void) { return da::g_error; }

int da_selftest_mfma(int dtype, const void* a, const void* b, float* out, void* stream) {
  if (!a || !b || !out) return da::set_error(DA_ERR_INVALID, "da_selftest_mfma: null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case DA_BF16:
      da::selftest_mfma_kernel<DA_BF16><<<1, 64, 0, s>>>((const char*)a, (const char*)b, out);
      break;
    case DA_F16:
      da::selftest_mfma_kernel<DA_F16><<<1, 64, 0, s>>>((const char*)a, (const char*)b, out);
      break;
    case DA_F32:
      da::selftest_mfma_kernel<DA_F32><<<1, 64, 0, s>>>((const char*)a, (const char*)b, out);
      break;
    default:
      return da::set_error(DA_ERR_INVALID, "da_selftest_mfma: bad dtype %d", dtype);
  }
  return da::check_launch("da_selftest_mfma");
}

}  // extern "C"
