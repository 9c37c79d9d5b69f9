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

namespace dsa {

// Records an error message for dsa_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Converts the status of the last launch on the calling thread.
int check_launch(const char* what);

// Number of XCDs the dispatcher round-robins workgroups over on MI355X.
constexpr int kNumXcd = 8;

// Remaps a dispatch index so that each XCD receives one contiguous range of
// the logical work order (consecutive workgroups on one XCD share L2 lines).
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
