// C-ABI plumbing: error reporting, version, and the MFMA lane-layout self test.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

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

int device_cu_count(int64_t* n) {
  // Written by whichever thread gets there first, always with the same value.
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(DA_ERR_HIP, "hipGetDevice failed");
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *n = c;
      return DA_OK;
    }
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return set_error(DA_ERR_HIP, "hipDeviceGetAttribute(multiProcessorCount) failed");
  if (dev >= 0 && dev < 64) cache[dev].store(cus, std::memory_order_relaxed);
  *n = cus;
  return DA_OK;
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

// One wave computes C = A . B^T for a single MFMA block with the library's
// operand convention and dumps the accumulator registers verbatim.
// shape 32: 32x32 block, A/B are 32 rows x 32 bytes (one chunk per lane half).
// shape 16: 16x16 block, A/B are 16 rows x 64 bytes (one chunk per lane quarter).
template <int DT>
__global__ __launch_bounds__(64) void selftest_mfma32_kernel(const char* a, const char* b, float* out) {
  const int lane = threadIdx.x;
  const int row = lane & 31, half = lane >> 5;
  const u32x4 va = ld16(a + row * 32 + half * 16);
  const u32x4 vb = ld16(b + row * 32 + half * 16);
  f32x16 acc = {};
  Mfma32<DT>::mma(acc, va, vb);
#pragma unroll
  for (int r = 0; r < 16; ++r) out[lane * 16 + r] = acc[r];
}

template <int DT>
__global__ __launch_bounds__(64) void selftest_mfma16_kernel(const char* a, const char* b, float* out) {
  const int lane = threadIdx.x;
  const int row = lane & 15, quarter = lane >> 4;
  const u32x4 va = ld16(a + row * 64 + quarter * 16);
  const u32x4 vb = ld16(b + row * 64 + quarter * 16);
  f32x4 acc = {};
  Mfma16<DT>::mma(acc, va, vb);
#pragma unroll
  for (int r = 0; r < 4; ++r) out[lane * 4 + r] = acc[r];
}

}  // namespace da

extern "C" {

int da_abi_version(void) { return 13; }

const char* da_last_error(void) { return da::g_error; }

int da_selftest_mfma(int dtype, int shape, const void* a, const void* b, float* out, void* stream) {
  if (!a || !b || !out) return da::set_error(DA_ERR_INVALID, "da_selftest_mfma: null pointer");
  if (shape != 16 && shape != 32) return da::set_error(DA_ERR_INVALID, "da_selftest_mfma: shape must be 16 or 32");
  if (!da::valid_dtype(dtype)) return da::set_error(DA_ERR_INVALID, "da_selftest_mfma: bad dtype %d", dtype);
  hipStream_t s = (hipStream_t)stream;
#define DA_ST(DT)                                                                                   \
  if (shape == 32)                                                                                  \
    da::selftest_mfma32_kernel<DT><<<1, 64, 0, s>>>((const char*)a, (const char*)b, out);          \
  else                                                                                              \
    da::selftest_mfma16_kernel<DT><<<1, 64, 0, s>>>((const char*)a, (const char*)b, out);
  switch (dtype) {
    case DA_BF16: DA_ST(DA_BF16) break;
    case DA_F16: DA_ST(DA_F16) break;
    default: DA_ST(DA_F32) break;
  }
#undef DA_ST
  return da::check_launch("da_selftest_mfma");
}

}  // extern "C"
