// Shared definitions for the libdsa HIP kernels (gfx950 / CDNA4 only).
//
// Every entry point reports failures through a negative status code and a
// thread-local message that dsa_last_error() returns.
#pragma once

#include <hip/hip_runtime.h>
#include "dsa.h"  // public C-ABI: definitions must match these declarations
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#define DSA_OK 0
#define DSA_EINVAL (-1)      // invalid argument (shape, pointer, alignment)
#define DSA_EUNSUPPORTED (-2) // valid but not implemented on this path
#define DSA_ELAUNCH (-3)     // HIP runtime reported an error

#define DSA_LDS __attribute__((address_space(3)))

typedef __bf16 dsa_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 dsa_bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 dsa_bf16x2 __attribute__((ext_vector_type(2)));
typedef float dsa_f32x16 __attribute__((ext_vector_type(16)));
typedef float dsa_f32x4 __attribute__((ext_vector_type(4)));
typedef float dsa_f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t dsa_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t dsa_u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 dsa_f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 dsa_f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 dsa_f16x2 __attribute__((ext_vector_type(2)));
typedef short dsa_i16x4 __attribute__((ext_vector_type(4)));

// Input element types (the dtype codes of dsa.h).
#define DSA_BF16 0
#define DSA_F16 1
#define DSA_F32 2

namespace dsa {

// The 16-bit input types share one MFMA shape (32x32x16, fp32 accumulate)
// and one LDS layout; Elem<T> names the vector types and the matrix op.
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  typedef dsa_bf16x8 x8;
  typedef dsa_bf16x4 x4;
  typedef dsa_bf16x2 x2;
  static __device__ __forceinline__ dsa_f32x16 mfma32(x8 a, x8 b, dsa_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<_Float16> {
  typedef dsa_f16x8 x8;
  typedef dsa_f16x4 x4;
  typedef dsa_f16x2 x2;
  static __device__ __forceinline__ dsa_f32x16 mfma32(x8 a, x8 b, dsa_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Records an error message for dsa_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Converts the status of the last launch on the calling thread.
int check_launch(const char* what);

// Number of XCDs the dispatcher round-robins workgroups over on MI355X.
constexpr int kNumXcd = 8;

// Remaps a dispatch index so that each XCD receives one contiguous range of
// the logical work order (consecutive workgroups on one XCD share L2 lines).
// Lanes l and l ^ 32 combine through v_permlane32_swap, a VALU op with no LDS
// round trip.  Both lanes of a pair get the same result (max is exact, and
// a + b == b + a in IEEE arithmetic).
__device__ __forceinline__ float pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 64 lanes in a fixed order, the same value in every lane: DPP
// butterflies inside each 16-lane row (quad xor 1, quad xor 2, half-row
// mirror, row mirror), then the four row sums read from lanes 0, 16, 32, 48.
// Every lane of the wave must be active.
__device__ __forceinline__ float wave_total(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ int xcd_remap(int wg, int total) {
  const int per = total / kNumXcd;
  const int rem = total % kNumXcd;
  const int xcd = wg % kNumXcd;
  const int slot = wg / kNumXcd;
  return xcd * per + (xcd < rem ? xcd : rem) + slot;
}

// Workgroup barrier after which every wave sees the LDS writes (and reads)
// that any wave issued before it.  __syncthreads alone orders LDS through the
// hardware LDS queue only, and a ds_write issued just before the barrier has
// been seen to land after another wave's ds_read issued just after it (under
// concurrent buffer->LDS traffic), so each wave first retires its own LDS
// operations (lgkmcnt(0)).  kWithVmem also retires vector memory operations
// (vmcnt(0)), which includes this wave's buffer->LDS loads.
template <bool kWithVmem = false>
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(kWithVmem ? 0x0070 : 0xC07F);  // [vmcnt(0)] lgkmcnt(0)
  __syncthreads();
}

}  // namespace dsa
