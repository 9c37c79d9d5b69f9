// Row arithmetic shared by the route kernels (gfx950): exact fixed-point row
// sums, a one-wave bitonic sort of up to 2048 keys and a workgroup-wide one
// in LDS for longer rows.
//
// A row value m >= 0 is represented as the integer floor(m * 2^(52 + s)), so
// row and prefix sums are exact and independent of summation order; a sum is
// rounded once to fp32 and scaled back by 2^-(52 + s).  The row exponent s
// (row_shift) is the largest integer with keys * max * 2^s < 2^10, so no sum
// of a row's images reaches 2^62 whatever the mass's magnitude; a power-of-two
// scale leaves the fp32 arithmetic on the sums unchanged.  The CPU oracle uses
// the same arithmetic, which makes routes bit-exact given the same fp32 inputs.
#pragma once

#include "dsa_common.h"

namespace dsa {

constexpr double kFixedScale = 4503599627370496.0;  // 2^52
constexpr float kInvFixed = 2.220446049250313e-16f; // 2^-52

__device__ __forceinline__ int64_t to_fixed(float v) {
  return (int64_t)__builtin_floor((double)v * kFixedScale);
}

__device__ __forceinline__ float fixed_to_f32(int64_t x) {
  return (float)x * kInvFixed;  // i64 -> f32 rounds to nearest even
}

// Row exponent s of a row of `keys` values whose largest is max_value (0 for
// an all-zero row).
__device__ __forceinline__ int row_shift(float max_value, int keys) {
  if (!(max_value > 0.f)) return 0;
  return 9 - ilogb((double)keys * (double)max_value);
}

__device__ __forceinline__ int64_t to_fixed(float v, int shift) {
  return (int64_t)__builtin_floor(ldexp((double)v, 52 + shift));
}

__device__ __forceinline__ float fixed_to_f32(int64_t x, int shift) {
  return ldexpf((float)x, -(52 + shift));  // i64 -> f32 rounds to nearest even
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
  return v;
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// Sorts the 64 * kPer keys of one wave (element e = lane * kPer + j in
// key[j]) into descending order, in place: a bitonic network, with partners
// kPer or more elements apart exchanged across lanes and closer ones inside a
// lane.
template <int kPer>
__device__ __forceinline__ void sort_desc(uint64_t key[kPer], int lane) {
  constexpr int kN = 64 * kPer;
#pragma unroll
  for (int size = 2; size <= kN; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= kPer) {
        const int lane_mask = stride / kPer;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int e = lane * kPer + j;
          const uint64_t other = __shfl_xor((unsigned long long)key[j], lane_mask);
          const bool desc = (e & size) == 0;
          const bool lower = (e & stride) == 0;
          const uint64_t hi = key[j] > other ? key[j] : other;
          const uint64_t lo = key[j] > other ? other : key[j];
          key[j] = (desc == lower) ? hi : lo;
        }
      } else {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          if (j & stride) continue;
          const int jp = j | stride;
          const int e = lane * kPer + j;
          const bool desc = (e & size) == 0;
          const uint64_t a = key[j], b = key[jp];
          const uint64_t hi = a > b ? a : b;
          const uint64_t lo = a > b ? b : a;
          key[j] = desc ? hi : lo;
          key[jp] = desc ? lo : hi;
        }
      }
    }
  }
}

// Reductions over a 256-thread workgroup (four waves); red holds four
// entries.  Every thread returns the result.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max_f32(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  lds_barrier();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  lds_barrier();
  return r;
}

__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* red) {
  v = wave_sum_i64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  lds_barrier();
  const int64_t r = (red[0] + red[1]) + (red[2] + red[3]);
  lds_barrier();
  return r;
}

// Sorts kN (a power of two) keys in LDS into descending order with a bitonic
// network run by a 256-thread workgroup.  Keys written before the call are
// covered by its first barrier; the sorted keys are visible to every thread
// when it returns.
template <int kN>
__device__ __forceinline__ void sort_desc_lds(uint64_t* keys) {
  const int tid = threadIdx.x;
  for (int size = 2; size <= kN; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      lds_barrier();
      for (int i = tid; i < kN / 2; i += 256) {
        const int lo = 2 * stride * (i / stride) + (i % stride);
        const int hi = lo + stride;
        const bool descending = (lo & size) == 0;
        const uint64_t a = keys[lo], b = keys[hi];
        if ((a < b) == descending) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
    }
  }
  lds_barrier();
}

}  // namespace dsa
