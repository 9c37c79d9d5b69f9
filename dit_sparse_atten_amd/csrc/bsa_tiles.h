// K-tile staging shared by the attention forward and the exact block-mass
// kernels (gfx950): 64-key half-tiles of K loaded straight into LDS.
#pragma once

#include "dsa_common.h"

namespace dsa {

constexpr int kHeadDim = 128;
constexpr int kRowBytes = kHeadDim * 2;        // one K row: 256 bytes
constexpr int kHalfKeys = 64;                  // keys per pipelined half-tile
constexpr int kKStage = kHalfKeys * kRowBytes; // 16 KB LDS stage (K or V^T)

typedef const __attribute__((address_space(4))) int32_t* const_i32;
typedef const __attribute__((address_space(4))) float* const_f32;

// K stage [64 keys][128 dims]: 16-byte chunk XOR (row & 15), so the 32 rows a
// fragment load reads at one chunk hit distinct banks.
__device__ __forceinline__ int k2_swz(int r, int c) { return c ^ (r & 15); }

// Raw buffer resources for the direct-to-LDS loads.  The MUBUF form
// (buffer_load ... lds) is used rather than global_load_lds because the
// compiler counts the latter as an LGKM event of unknown order and then waits
// for every outstanding LDS read (lgkmcnt(0)) before each fragment use; MUBUF
// LDS loads only count on vmcnt.  Dword 3 is the gfx9 raw-buffer format word.
// A raw buffer (stride 0) returns zeros for offsets at or past num_records
// (the vector offset is checked, the scalar offset is not).
constexpr int kBufferDword3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferDword3);
}

// 16 bytes per lane into LDS at lds + 16 * lane.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* lds,
                                           uint32_t voffset, uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (DSA_LDS void*)lds, 16, voffset, soffset, 0, 0);
}

// Resource covering the 64 K rows (16-bit elements, token stride k_st) of a
// half-tile starting at key0; rows at or past kv_tokens read as zeros (a
// half-tile wholly past the end has no records), and the last row ends at its
// head_dim-th element.  The host keeps 64 rows of K within 2^31 bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t k_tile_rsrc(const void* kbase, int64_t k_st,
                                                             int key0, int kv_tokens,
                                                             int head_dim) {
  const int rows = min(kHalfKeys, kv_tokens - key0);
  const uint32_t bytes = rows > 0 ? (uint32_t)((rows - 1) * k_st * 2 + head_dim * 2) : 0u;
  return make_rsrc(static_cast<const unsigned char*>(kbase) + (int64_t)key0 * k_st * 2, bytes);
}

// A chunk of 8 dims at or past head_dim stages from this offset: past every
// buffer's range (the hosts keep K and V within 2^31 bytes), so it reads as
// zeros and a head_dim below 128 runs as 128 with zero dims.
constexpr uint32_t kDeadChunk = 0x80000000u;

__device__ __forceinline__ uint32_t dead_bits(int chunk, int head_dim) {
  return chunk * 8 < head_dim ? 0u : kDeadChunk;
}

// Per-lane byte offsets of one 256-thread workgroup's share of a K half-tile:
// thread (wave, lane) loads 16-byte chunks j = 0..3 of the [64][128] tile in
// the k2_swz layout.  `k_st` is the token stride in elements.
__device__ __forceinline__ void k_tile_offsets(int wave, int lane, int64_t k_st, int head_dim,
                                               uint32_t koff[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = (wave * 4 + j) * 64 + lane;
    const int row = idx >> 4;
    const int c = k2_swz(row, idx & 15);
    koff[j] = (uint32_t)((row * (int)k_st + c * 8) * 2) | dead_bits(c, head_dim);
  }
}

// Tile-local coordinate of index i on a tile axis of `length` tokens, mapped
// to [-1, 1] in fp32 as the reference's spatial offsets are
// (attention_backends/sparse.py:141-146): (i - c) / max(c, 1/2), c = (length - 1) / 2.
__device__ __forceinline__ float tile_axis(int i, int length) {
  const float center = (float)(length - 1) / 2.0f;
  const float scale = fmaxf((float)(length - 1) / 2.0f, 0.5f);
  return ((float)i - center) / scale;
}

// Q fragments of one query row for the S^T = K Q^T products: qf[dc] holds
// dims 16 dc + 8 g .. + 7, zeros at or past head_dim.
template <typename X8, typename T>
__device__ __forceinline__ void load_q_fragments(const T* qrow, int g, int head_dim, X8 qf[8]) {
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) {
    if (dc * 16 + g * 8 < head_dim) {
      qf[dc] = *reinterpret_cast<const X8*>(qrow + dc * 16 + g * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[dc][e] = (T)0.0f;
    }
  }
}

}  // namespace dsa
