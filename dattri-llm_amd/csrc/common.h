// Shared device/host helpers for the gfx950 kernels of the gradient-scoring path.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, the gfx950 MFMA
// instructions (v_mfma_f32_32x32x16_{bf16,f16}, v_mfma_f32_32x32x2_f32) and
// 16-byte vector memory operations.  There is no other target.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "dattri_amd.h"

namespace da {

// ---------------------------------------------------------------------------
// Vector types.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: 8 accelerator complex dies, 32 CUs each

// ---------------------------------------------------------------------------
// Element traits.  Storage is raw bits; arithmetic is always fp32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}
// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN, quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}

template <int DT> struct Elem;
template <> struct Elem<DA_F32> {
  static constexpr int kBytes = 4;
  static constexpr int kVec = 4;  // elements per 16-byte chunk
  __device__ static float load(const void* p, int64_t i) { return ((const float*)p)[i]; }
  __device__ static void store(void* p, int64_t i, float v) { ((float*)p)[i] = v; }
  __device__ static float from_bits(uint32_t b) { return __uint_as_float(b); }
};
template <> struct Elem<DA_BF16> {
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  __device__ static float load(const void* p, int64_t i) {
    return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  }
  __device__ static void store(void* p, int64_t i, float v) {
    ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
  }
  __device__ static float from_bits(uint32_t b) { return bf16_bits_to_f32(b); }
};
template <> struct Elem<DA_F16> {
  static constexpr int kBytes = 2;
  static constexpr int kVec = 8;
  __device__ static float load(const void* p, int64_t i) {
    return f16_bits_to_f32(((const uint16_t*)p)[i]);
  }
  __device__ static void store(void* p, int64_t i, float v) {
    ((uint16_t*)p)[i] = f32_to_f16_bits(v);
  }
  __device__ static float from_bits(uint32_t b) { return f16_bits_to_f32(b); }
};

// Unpack one 16-byte chunk into fp32 lanes (kVec values).
template <int DT>
__device__ __forceinline__ void unpack16(u32x4 v, float* out) {
  if constexpr (DT == DA_F32) {
    out[0] = __uint_as_float(v[0]);
    out[1] = __uint_as_float(v[1]);
    out[2] = __uint_as_float(v[2]);
    out[3] = __uint_as_float(v[3]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      out[2 * q] = Elem<DT>::from_bits(v[q] & 0xffffu);
      out[2 * q + 1] = Elem<DT>::from_bits(v[q] >> 16);
    }
  }
}

// ---------------------------------------------------------------------------
// 32x32 MFMA on one 16-byte lane chunk per operand.
//
// Operand convention used by every kernel in this library: in a 32x32 block,
// lane l supplies row (l % 32) of A and column (l % 32) of B, and the lane's
// 16-byte chunk holds the k-elements [kb + kVec*(l/32), kb + kVec*(l/32) + kVec).
// Because the contraction is a plain sum, any k-permutation that is the same
// for A and B gives the same product; kernels exploit that to read long
// contiguous runs per lane.
//
// Accumulator layout (checked by da_selftest_mfma): acc[r] of lane l holds
// C[8*(r/4) + 4*(l/32) + (r%4)][l % 32].
// ---------------------------------------------------------------------------
template <int DT> struct Mfma32;
template <> struct Mfma32<DA_BF16> {
  __device__ static __forceinline__ void mma(f32x16& acc, u32x4 a, u32x4 b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma32<DA_F16> {
  __device__ static __forceinline__ void mma(f32x16& acc, u32x4 a, u32x4 b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma32<DA_F32> {
  __device__ static __forceinline__ void mma(f32x16& acc, u32x4 a, u32x4 b) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[s]), __uint_as_float(b[s]), acc,
                                                 0, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// 16x16 MFMA (v_mfma_f32_16x16x32_{bf16,f16}, v_mfma_f32_16x16x4_f32).
//
// Lane l supplies row (l % 16) of A / column (l % 16) of B; its 16-byte chunk
// holds the k-elements [kb + kVec*(l/16), ... + kVec) (fp32: four MFMAs, one
// element each).  Accumulator: acc[r] of lane l holds C[4*(l/16) + r][l % 16]
// (checked by da_selftest_mfma).
// ---------------------------------------------------------------------------
template <int DT> struct Mfma16;
template <> struct Mfma16<DA_BF16> {
  __device__ static __forceinline__ void mma(f32x4& acc, u32x4 a, u32x4 b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma16<DA_F16> {
  __device__ static __forceinline__ void mma(f32x4& acc, u32x4 a, u32x4 b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma16<DA_F32> {
  __device__ static __forceinline__ void mma(f32x4& acc, u32x4 a, u32x4 b) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[s]), __uint_as_float(b[s]), acc,
                                                 0, 0, 0);
  }
};
__device__ __forceinline__ int acc16_row(int r, int lane) { return 4 * (lane >> 4) + r; }
__device__ __forceinline__ int acc16_col(int lane) { return lane & 15; }

__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
__device__ __forceinline__ int acc_col(int lane) { return lane & 31; }

// ---------------------------------------------------------------------------
// Reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// ---------------------------------------------------------------------------
// Grid helpers.
// ---------------------------------------------------------------------------
// The dispatcher places workgroup w on XCD (w % 8).  Remap so each XCD owns a
// contiguous range of logical tile ids (so neighbouring tiles, which share
// operand rows, hit the same L2).  Bijective for any n.
__device__ __forceinline__ int64_t xcd_remap(int64_t w, int64_t n) {
  const int64_t q = n / kXcds, r = n % kXcds;
  const int64_t xcd = w % kXcds, local = w / kXcds;
  const int64_t start = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
  return start + local;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *(u32x4*)p = v; }

// ---------------------------------------------------------------------------
// Buffer loads straight into LDS (gfx950: 16 bytes per lane).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) char lds_char;

// One 16-byte-per-lane buffer load into LDS at lds_addr + 16 * lane (M0 holds
// the wave-uniform LDS byte address).  Inline assembly, so the compiler does
// not wait for every outstanding load before each LDS read (it cannot tell a
// ring's stages apart); callers wait with explicit vmcnt counts.  The LDS
// address is an operand bound to M0 ("{m0}"), so the compiler writes M0
// itself and knows the statement reads it: nothing it keeps in M0 (LDS
// bounds, other DMA addresses) is overwritten behind its back.  An offset at
// or past the resource's range reads zeros and touches no memory.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "{m0}"(lds_addr)
               : "memory");
}

// The same with the non-temporal hint: for data read once (streamed factor
// rows), so that it does not push data that is read again out of L2.
__device__ __forceinline__ void dma16_nt(u32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :
               : "v"(voff), "s"(rsrc), "{m0}"(lds_addr)
               : "memory");
}

// Raw buffer resource over [base, base + bytes) (stride 0: byte offsets).
__device__ __forceinline__ u32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, bytes, 0x00020000u};
}

// A wave-uniform 16-byte value, forced into scalar registers.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ u32x4 uniform4(u32x4 v) {
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane(v[0]), (uint32_t)__builtin_amdgcn_readfirstlane(v[1]),
               (uint32_t)__builtin_amdgcn_readfirstlane(v[2]), (uint32_t)__builtin_amdgcn_readfirstlane(v[3])};
}

}  // namespace da

// ---------------------------------------------------------------------------
// Host-side error plumbing (defined in capi.hip).
// ---------------------------------------------------------------------------
namespace da {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Zero a (rows x cols) fp32 matrix with leading dimension ld using a kernel
// (never a memset node, so callers may capture it in a HIP graph).
int zero_f32_2d(float* out, int64_t rows, int64_t cols, int64_t ld, hipStream_t stream);
// CUs of the current device (the workgroup slots of the stream-K and split
// launches), cached per device.
int device_cu_count(int64_t* n);
inline size_t elem_bytes(int dt) { return dt == DA_F32 ? 4 : 2; }
inline bool valid_dtype(int dt) { return dt == DA_F32 || dt == DA_BF16 || dt == DA_F16; }
}  // namespace da
