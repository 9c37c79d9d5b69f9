// Spatial-tile attention statistics for gfx950 (MI355X).
//
// Replaces the statistics of the reference's matrix-sparse backend
// (attention_backends/sparse.py): the exact dense route of `_dense_route`
// (sparse.py:184-233) and the per-step statistics of `sparse_chunk`
// (sparse.py:718-750), with the normalisations of `_sparse_attention`
// (sparse.py:859-864, 908-922).  For query tile qt and key tile kt of one head,
// with p = exp(scale * <q_t, k_s> - lse_t) over the keys the softmax saw:
//   mass = sum p, q_y = sum p * y(t), q_x = sum p * x(t),
//   k_y = sum p * y(s), k_x = sum p * x(s),
// where y, x are the tile-local coordinates of sparse.py:141-157 (each axis
// mapped to [-1, 1]).  Outputs: mass / tokens (fp32 and fp16) and the
// centroids moment / max(mass, 1e-12) (fp16), as the reference stores them.
// Tokens are in tile-major order (each tile contiguous); the CSR, when given,
// lists the key tiles of each (head, query tile) row, and cells it does not
// list are written as zeros.
//
// Design: the block-mass kernel's structure (one 4-wave workgroup per (head,
// query tile), K half-tiles through LDS by buffer->LDS loads, S^T on
// v_mfma_f32_32x32x16_bf16 so each lane owns one query row, fixed-order
// reductions through LDS), plus key-offset lookups from two per-tile LDS
// tables read as 16-byte vectors.
#include "bsa_tiles.h"

#include <hip/hip_fp16.h>

#include <cmath>
#include <type_traits>

namespace {

using dsa::kHalfKeys;
using dsa::kKStage;
using dsa::kRowBytes;

constexpr int kStats = 5;  // mass, q_y, q_x, k_y, k_x
constexpr int kMaxTiles = 2048;
constexpr float kLog2e = 1.4426950408889634f;

struct TileStatsParams {
  const __bf16* q;
  const __bf16* k;
  const float* lse;
  const int32_t* row_ptr;  // null: every key tile
  const int32_t* col_idx;
  float* mass32;   // [H, nt, nt] mass / tokens
  __half* mass16;  // optional, the same in fp16
  __half* cqy;     // optional centroids (fp16)
  __half* cqx;
  __half* cky;
  __half* ckx;
  int64_t q_st, q_sh, k_st, k_sh, lse_sh;
  int32_t tokens, heads, tiles, tile, tile_h, tile_w;
  float scale_log2;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// (i - center) / scale for one tile axis, as sparse.py:141-146 computes it in fp32.
__device__ __forceinline__ float axis_offset(int i, int length) {
  const float center = (float)(length - 1) / 2.0f;
  const float scale = fmaxf((float)(length - 1) / 2.0f, 0.5f);
  return ((float)i - center) / scale;
}

template <bool kRouted, int kNh>
__global__ void __launch_bounds__(256, 2) tile_stats_kernel(TileStatsParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k1[kKStage];
  __shared__ __attribute__((aligned(16))) float off_y[128];
  __shared__ __attribute__((aligned(16))) float off_x[128];
  __shared__ float part[2][4][kStats];
  __shared__ uint32_t listed[kMaxTiles / 32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % p.tiles;
  const int h = work / p.tiles;

  if (tid < 128) {
    // Local token index -> (row, column) inside the tile, row-major.
    const int r = tid / p.tile_w, c = tid % p.tile_w;
    off_y[tid] = tid < p.tile ? axis_offset(r, p.tile_h) : 0.f;
    off_x[tid] = tid < p.tile ? axis_offset(c, p.tile_w) : 0.f;
  }
  if (tid < kMaxTiles / 32) listed[tid] = 0u;

  const int local_row = wave * 32 + qi;
  const int tq = qt * p.tile + local_row;
  const bool row_ok = local_row < p.tile && tq < p.tokens;
  const bool wave_active = wave * 32 < p.tile;
  const int tq_c = tq < p.tokens ? tq : p.tokens - 1;
  const __bf16* qrow = p.q + h * p.q_sh + (int64_t)tq_c * p.q_st;
  dsa_bf16x8 qf[8];
#pragma unroll
  for (int dc = 0; dc < 8; ++dc)
    qf[dc] = *reinterpret_cast<const dsa_bf16x8*>(qrow + dc * 16 + g * 8);
  const float lse2 = row_ok ? p.lse[h * p.lse_sh + tq] * kLog2e : INFINITY;

  int start = 0, end = p.tiles;
  if (kRouted) {
    const dsa::const_i32 rp = (dsa::const_i32)p.row_ptr;
    start = rp[(int64_t)h * p.tiles + qt];
    end = rp[(int64_t)h * p.tiles + qt + 1];
  }
  const dsa::const_i32 cidx = (dsa::const_i32)p.col_idx;
  auto tile_of = [&](int j) -> int {
    const int kt = kRouted ? cidx[start + j] : j;
    return (unsigned)kt < (unsigned)p.tiles ? kt : -1;
  };
  const int ntile = end - start;

  const __bf16* kbase = p.k + h * p.k_sh;
  int koff[4];
  dsa::k_tile_offsets(wave, lane, p.k_st, koff);
  auto issue = [&](int kt, int half, unsigned char* dst) __attribute__((always_inline)) {
    const int key0 = (kt < 0 ? 0 : kt) * p.tile + half * kHalfKeys;
    const __amdgpu_buffer_rsrc_t rsrc = dsa::k_tile_rsrc(kbase, p.k_st, key0, p.tokens);
#pragma unroll
    for (int j = 0; j < 4; ++j) dsa::lds_load16(rsrc, dst + (wave * 4 + j) * 1024, koff[j], 0);
  };

  const int64_t cell0 = ((int64_t)h * p.tiles + qt) * p.tiles;
  // Writes the cell of key tile kt, the j-th of this row (its partials sit in
  // part[j & 1]).
  auto flush = [&](int j, int kt) __attribute__((always_inline)) {
    if (wave == 0 && lane == 0 && kt >= 0) {
      float v[kStats];
      const float(*pr)[kStats] = part[j & 1];
#pragma unroll
      for (int s = 0; s < kStats; ++s) v[s] = (pr[0][s] + pr[1][s]) + (pr[2][s] + pr[3][s]);
      const int64_t cell = cell0 + kt;
      const float normalized = v[0] / (float)p.tokens;
      p.mass32[cell] = normalized;
      if (p.mass16) p.mass16[cell] = __float2half(normalized);
      const float den = fmaxf(v[0], 1e-12f);
      if (p.cqy) p.cqy[cell] = __float2half(v[1] / den);
      if (p.cqx) p.cqx[cell] = __float2half(v[2] / den);
      if (p.cky) p.cky[cell] = __float2half(v[3] / den);
      if (p.ckx) p.ckx[cell] = __float2half(v[4] / den);
      if (kRouted) listed[kt >> 5] |= 1u << (kt & 31);
    }
  };

  dsa::lds_barrier();  // offset tables and the listed bitmap are ready
  const float oyq = off_y[local_row < p.tile ? local_row : 0];
  const float oxq = off_x[local_row < p.tile ? local_row : 0];

  float am = 0.f, aky = 0.f, akx = 0.f;
  // Accumulates one staged half-tile of key tile kt into the lane sums.
  // NKK: 32-key sub-tiles holding valid keys (1 when at most 32 are valid);
  // kFull: all 64 keys valid (no per-key mask).
  auto compute = [&](const unsigned char* cur, int half, int valid, auto nkk_c, auto full_c)
                     __attribute__((always_inline)) {
    constexpr int NKK = decltype(nkk_c)::value;
    constexpr bool kFull = decltype(full_c)::value;
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      dsa_f32x16 sacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
      const int row = kk * 32 + qi;
#pragma unroll
      for (int dc = 0; dc < 8; ++dc) {
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            cur + row * kRowBytes + dsa::k2_swz(row, dc * 2 + g) * 16);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[dc], sacc, 0, 0, 0);
      }
#pragma unroll
      for (int quad = 0; quad < 4; ++quad) {
        // Keys half * 64 + kk * 32 + 8 * quad + 4 * g + (0..3) of the tile.
        const int key_local = half * kHalfKeys + kk * 32 + 8 * quad + 4 * g;
        const int kl = key_local < 128 ? key_local : 124;
        const dsa_f32x4 ky = *reinterpret_cast<const dsa_f32x4*>(&off_y[kl]);
        const dsa_f32x4 kx = *reinterpret_cast<const dsa_f32x4*>(&off_x[kl]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key_in_half = kk * 32 + 8 * quad + 4 * g + e;
          float pv = __builtin_amdgcn_exp2f(fmaf(sacc[quad * 4 + e], p.scale_log2, -lse2));
          if (!kFull) pv = key_in_half < valid ? pv : 0.f;
          am += pv;
          aky = fmaf(pv, ky[e], aky);
          akx = fmaf(pv, kx[e], akx);
        }
      }
    }
  };

  auto end_tile = [&](int j) __attribute__((always_inline)) {
    const float m = wave_sum(am);
    const float qy = wave_sum(am * oyq);
    const float qx = wave_sum(am * oxq);
    const float ky = wave_sum(aky);
    const float kx = wave_sum(akx);
    if (lane == 0) {
      float* dst = part[j & 1][wave];
      dst[0] = m;
      dst[1] = qy;
      dst[2] = qx;
      dst[3] = ky;
      dst[4] = kx;
    }
    am = aky = akx = 0.f;
  };

  // Steps walk (tile j, half i); every step waits for its stage, flushes the
  // previous tile once all partials are in LDS, prefetches, then computes.
  const int nsteps = ntile * kNh;
  if (nsteps > 0) issue(tile_of(0), 0, lds_k0);
  int prev_kt = -1;
  for (int sidx = 0; sidx < nsteps; ++sidx) {
    const int j = sidx / kNh;
    const int half = sidx % kNh;
    const int kt = tile_of(j);
    dsa::lds_barrier<true>();
    if (half == 0 && j > 0) flush(j - 1, prev_kt);
    if (sidx + 1 < nsteps) {
      const int nj = (sidx + 1) / kNh, nhalf = (sidx + 1) % kNh;
      issue(tile_of(nj), nhalf, (sidx & 1) ? lds_k0 : lds_k1);
    }
    if (wave_active) {
      int valid = 0;
      if (kt >= 0) {
        valid = min(kHalfKeys, p.tile - half * kHalfKeys);
        valid = min(valid, p.tokens - (kt * p.tile + half * kHalfKeys));
      }
      const unsigned char* cur = (sidx & 1) ? lds_k1 : lds_k0;
      using one = std::integral_constant<int, 1>;
      using two = std::integral_constant<int, 2>;
      if (valid == kHalfKeys) compute(cur, half, valid, two{}, std::true_type{});
      else if (valid > 32) compute(cur, half, valid, two{}, std::false_type{});
      else compute(cur, half, valid, one{}, std::false_type{});
    }
    if (half == kNh - 1) {
      end_tile(j);
      prev_kt = kt;
    }
  }
  dsa::lds_barrier();
  if (nsteps > 0) flush(ntile - 1, prev_kt);
  if (kRouted) {
    dsa::lds_barrier();
    // Cells this row does not list hold zero mass and zero centroids.
    const __half zero = __float2half(0.f);
    for (int kt = tid; kt < p.tiles; kt += 256) {
      if (listed[kt >> 5] & (1u << (kt & 31))) continue;
      const int64_t cell = cell0 + kt;
      p.mass32[cell] = 0.f;
      if (p.mass16) p.mass16[cell] = zero;
      if (p.cqy) p.cqy[cell] = zero;
      if (p.cqx) p.cqx[cell] = zero;
      if (p.cky) p.cky[cell] = zero;
      if (p.ckx) p.ckx[cell] = zero;
    }
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" int dsa_tile_stats(const void* q, const void* k, const int64_t* strides,
                              int32_t tokens, int32_t heads, int32_t head_dim, int32_t tile_h,
                              int32_t tile_w, const float* lse, int64_t lse_head_stride,
                              const int32_t* row_ptr, const int32_t* col_idx, float scale,
                              float* mass, void* mass_f16, void* centroid_q_y,
                              void* centroid_q_x, void* centroid_k_y, void* centroid_k_x,
                              hipStream_t stream) {
  dsa::clear_error();
  if (!q || !k || !strides || !lse || !mass)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: null pointer argument");
  if ((row_ptr == nullptr) != (col_idx == nullptr))
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: row_ptr and col_idx must both be set");
  if (tokens <= 0 || heads <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: tokens and heads must be positive");
  if (head_dim != dsa::kHeadDim)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_tile_stats: head_dim %d unsupported (128)",
                          head_dim);
  if (tile_h <= 0 || tile_w <= 0 || tile_h * tile_w > 128)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_tile_stats: tile %dx%d unsupported (<= 128)",
                          tile_h, tile_w);
  const int32_t tile = tile_h * tile_w;
  if (tokens % tile != 0)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: %d tokens are not whole %d-token tiles",
                          tokens, tile);
  const int32_t tiles = tokens / tile;
  if (tiles > kMaxTiles)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_tile_stats: %d tiles (at most %d)", tiles,
                          kMaxTiles);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: scale must be positive and finite");
  if (!aligned16(q) || !aligned16(k))
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: q and k must be 16-byte aligned");
  for (int i = 0; i < 4; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: stride %d is not a non-negative "
                                        "multiple of 8 elements", i);
  if (strides[2] * (int64_t)(2 * 64) > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_tile_stats: key token stride too large");
  if (lse_head_stride < tokens)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: lse head stride < tokens");
  const int64_t grid = (int64_t)heads * tiles;
  if (grid > 0x7fffffff)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: grid too large");

  TileStatsParams p;
  p.q = static_cast<const __bf16*>(q);
  p.k = static_cast<const __bf16*>(k);
  p.lse = lse;
  p.row_ptr = row_ptr;
  p.col_idx = col_idx;
  p.mass32 = mass;
  p.mass16 = static_cast<__half*>(mass_f16);
  p.cqy = static_cast<__half*>(centroid_q_y);
  p.cqx = static_cast<__half*>(centroid_q_x);
  p.cky = static_cast<__half*>(centroid_k_y);
  p.ckx = static_cast<__half*>(centroid_k_x);
  p.q_st = strides[0]; p.q_sh = strides[1];
  p.k_st = strides[2]; p.k_sh = strides[3];
  p.lse_sh = lse_head_stride;
  p.tokens = tokens;
  p.heads = heads;
  p.tiles = tiles;
  p.tile = tile;
  p.tile_h = tile_h;
  p.tile_w = tile_w;
  p.scale_log2 = scale * kLog2e;
  const dim3 blocks((unsigned)grid), threads(256);
  const bool routed = row_ptr != nullptr;
  if (tile > kHalfKeys) {
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<true, 2>), blocks, threads, 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<false, 2>), blocks, threads, 0, stream, p);
  } else {
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<true, 1>), blocks, threads, 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<false, 1>), blocks, threads, 0, stream, p);
  }
  return dsa::check_launch("dsa_tile_stats");
}
