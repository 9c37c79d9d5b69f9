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
//
// Tiles of 65..127 tokens whose 8-rounded size is below the half-tile slots
// (64 + 32 up to 96 tokens, else 128) take the gathered key stream instead:
// the row's key tiles are concatenated, each padded to tile_pad (the tile
// rounded up to 8), and staged as 64-key chunks, so a 72-token tile costs 72
// key slots rather than 96.  A chunk spans at most two tiles, and the tile
// boundary (a multiple of 8 positions into the chunk) falls between the
// lanes' 4-key runs, so each run accumulates into one tile and the earlier
// tile is reduced at the boundary.  Every kernel runs one wave per 32 query
// rows of the tile (at least two), so no wave idles above 32 tokens.
#include "bsa_tiles.h"

#include <hip/hip_fp16.h>

#include <cmath>
#include <type_traits>

namespace {

using dsa::kHalfKeys;
using dsa::kKStage;
using dsa::kRowBytes;

constexpr int kStats = 5;  // mass, q_y, q_x, k_y, k_x
constexpr int kMaxTiles = 16384;  // key tiles a row's `listed` bitmap covers (2 KB)
constexpr float kLog2e = 1.4426950408889634f;

struct TileStatsParams {
  const void* q;  // element type T of the kernel instance
  const void* k;
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
  int32_t tile_pad;  // gathered stream: key slots per tile (tile rounded up to 8)
  int32_t head_dim;  // 8..128, a multiple of 8
  float scale_log2;
};

// (i - center) / scale for one tile axis, as sparse.py:141-146 computes it in fp32.
__device__ __forceinline__ float axis_offset(int i, int length) {
  const float center = (float)(length - 1) / 2.0f;
  const float scale = fmaxf((float)(length - 1) / 2.0f, 0.5f);
  return ((float)i - center) / scale;
}

// kWaves: waves per workgroup, one per 32 query rows of the tile (2..4).
template <typename T, bool kRouted, int kNh, bool kGather = false, int kWaves = 4>
__global__ void __launch_bounds__(kWaves * 64, 2) tile_stats_kernel(TileStatsParams p) {
  typedef dsa::Elem<T> E;
  constexpr int kThreads = kWaves * 64;
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k1[kKStage];
  __shared__ __attribute__((aligned(16))) float off_y[128];
  __shared__ __attribute__((aligned(16))) float off_x[128];
  __shared__ float part[2][kWaves][kStats];
  __shared__ uint32_t listed[kMaxTiles / 32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % p.tiles;
  const int h = work / p.tiles;

  for (int i = tid; i < 128; i += kThreads) {
    // Local token index -> (row, column) inside the tile, row-major.
    const int r = i / p.tile_w, c = i % p.tile_w;
    off_y[i] = i < p.tile ? axis_offset(r, p.tile_h) : 0.f;
    off_x[i] = i < p.tile ? axis_offset(c, p.tile_w) : 0.f;
  }
  if (kRouted)
    for (int i = tid; i < kMaxTiles / 32; i += kThreads) listed[i] = 0u;

  const int local_row = wave * 32 + qi;
  const int tq = qt * p.tile + local_row;
  const bool row_ok = local_row < p.tile && tq < p.tokens;
  const bool wave_active = wave * 32 < p.tile;
  const int tq_c = tq < p.tokens ? tq : p.tokens - 1;
  const T* qrow = static_cast<const T*>(p.q) + h * p.q_sh + (int64_t)tq_c * p.q_st;
  typename E::x8 qf[8];
  dsa::load_q_fragments(qrow, g, p.head_dim, qf);
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

  const T* kbase = static_cast<const T*>(p.k) + h * p.k_sh;
  uint32_t koff[4];
  dsa::k_tile_offsets(wave, lane, p.k_st, p.head_dim, koff);
  auto issue = [&](int kt, int half, unsigned char* dst) __attribute__((always_inline)) {
    const int key0 = (kt < 0 ? 0 : kt) * p.tile + half * kHalfKeys;
    const __amdgpu_buffer_rsrc_t rsrc = dsa::k_tile_rsrc(kbase, p.k_st, key0, p.tokens);
    if constexpr (kWaves == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) dsa::lds_load16(rsrc, dst + (wave * 4 + j) * 1024, koff[j], 0);
    } else {
      // The stage's 16 1-KB slices, dealt round-robin over the waves.
      for (int i = wave; i < kKStage / 1024; i += kWaves) {
        const int row = i * 4 + (lane >> 4);
        const int c = dsa::k2_swz(row, lane & 15);
        dsa::lds_load16(rsrc, dst + i * 1024,
                        (uint32_t)((row * (int)p.k_st + c * 8) * 2) | dsa::dead_bits(c, p.head_dim),
                        0);
      }
    }
  };

  const int64_t cell0 = ((int64_t)h * p.tiles + qt) * p.tiles;
  // Writes the cell of key tile kt, the j-th of this row (its partials sit in
  // part[j & 1]).
  // Lane s < 5 of wave 0 sums statistic s over the waves and writes it.
  auto flush = [&](int j, int kt) __attribute__((always_inline)) {
    if (wave == 0 && lane < kStats && kt >= 0) {
      const float(*pr)[kStats] = part[j & 1];
      auto total = [&](int s) {  // (w0 + w1) + (w2 + w3) over the waves present
        if constexpr (kWaves == 1) return pr[0][s];
        else if constexpr (kWaves == 2) return pr[0][s] + pr[1][s];
        else if constexpr (kWaves == 3) return (pr[0][s] + pr[1][s]) + pr[2][s];
        else return (pr[0][s] + pr[1][s]) + (pr[2][s] + pr[3][s]);
      };
      const float mass = total(0);
      const int64_t cell = cell0 + kt;
      if (lane == 0) {
        const float normalized = mass / (float)p.tokens;
        p.mass32[cell] = normalized;
        if (p.mass16) p.mass16[cell] = __float2half(normalized);
        if (kRouted) listed[kt >> 5] |= 1u << (kt & 31);
      } else {
        __half* dst = lane == 1 ? p.cqy : lane == 2 ? p.cqx : lane == 3 ? p.cky : p.ckx;
        if (dst) dst[cell] = __float2half(total(lane) / fmaxf(mass, 1e-12f));
      }
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
        const typename E::x8 a = *reinterpret_cast<const typename E::x8*>(
            cur + row * kRowBytes + dsa::k2_swz(row, dc * 2 + g) * 16);
        sacc = E::mfma32(a, qf[dc], sacc);
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
    const float m = dsa::wave_total(am);
    const float qy = dsa::wave_total(am * oyq);
    const float qx = dsa::wave_total(am * oxq);
    const float ky = dsa::wave_total(aky);
    const float kx = dsa::wave_total(akx);
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

  if constexpr (kGather) {
    const int bp = p.tile_pad;
    const __amdgpu_buffer_rsrc_t k_all = dsa::make_rsrc(
        kbase, (uint32_t)((int64_t)(p.tokens - 1) * p.k_st * 2 + kRowBytes));
    const uint32_t kst2 = (uint32_t)(p.k_st * 2);
    // Stages the chunk that starts `o0` slots into tile kta and runs on into
    // tile ktb (both in range): stream position r lands in K stage row r;
    // pad slots load whatever they address and are masked.
    auto issue_gather = [&](int kta, int ktb, int o0, unsigned char* dst)
        __attribute__((always_inline)) {
      for (int i = wave; i < kKStage / 1024; i += kWaves) {
        const int row = i * 4 + (lane >> 4);
        const int o = o0 + row;
        const bool first = o < bp;
        const int token = (first ? kta : ktb) * p.tile + (first ? o : o - bp);
        const int c = dsa::k2_swz(row, lane & 15);
        dsa::lds_load16(k_all, dst + i * 1024,
                        ((uint32_t)token * kst2 + (uint32_t)(c * 16)) | dsa::dead_bits(c, p.head_dim),
                        0);
      }
    };
    // Accumulates chunk positions [0, 32 NKK): those before `second` belong
    // to tile ja (at tile-local offset o0 + position), the rest to the next
    // tile (offset position - second).  At position `split` tile ja ends and
    // is reduced.  masked: pad slots, positions >= left and out-of-range
    // tiles (ok_a / ok_b false) count zero.
    auto compute_gather = [&](const unsigned char* cur, int o0, int second, int split, int ja,
                              bool masked, int left, bool ok_a, bool ok_b, auto nkk_c)
        __attribute__((always_inline)) {
      constexpr int NKK = decltype(nkk_c)::value;
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        dsa_f32x16 sacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
        const int row = kk * 32 + qi;
#pragma unroll
        for (int dc = 0; dc < 8; ++dc) {
          const typename E::x8 a = *reinterpret_cast<const typename E::x8*>(
              cur + row * kRowBytes + dsa::k2_swz(row, dc * 2 + g) * 16);
          sacc = E::mfma32(a, qf[dc], sacc);
        }
#pragma unroll
        for (int quad = 0; quad < 4; ++quad) {
          // This lane's keys: positions 8 unit + 4 g + (0..3); a tile
          // boundary (a multiple of 8) never splits them.
          const int unit = kk * 4 + quad;
          if (8 * unit == split) end_tile(ja);
          const bool in_a = 8 * unit < second;
          const int base = (in_a ? o0 : -second) + 8 * unit + 4 * g;
          const dsa_f32x4 ky = *reinterpret_cast<const dsa_f32x4*>(&off_y[base]);
          const dsa_f32x4 kx = *reinterpret_cast<const dsa_f32x4*>(&off_x[base]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float pv = __builtin_amdgcn_exp2f(fmaf(sacc[quad * 4 + e], p.scale_log2, -lse2));
            if (masked) {
              const bool ok = (in_a ? ok_a : ok_b) && base + e < p.tile &&
                              8 * unit + 4 * g + e < left;
              pv = ok ? pv : 0.f;
            }
            am += pv;
            aky = fmaf(pv, ky[e], aky);
            akx = fmaf(pv, kx[e], akx);
          }
        }
      }
    };

    const int n = ntile;
    if (n > 0) {
      const int total = (n - 1) * bp + p.tile;  // slots up to the row's last key
      const int chunks = (total + 63) >> 6;
      auto tile_at = [&](int j) { return tile_of(j < n ? j : n - 1); };
      int j0 = 0, o0 = 0;
      int ka = tile_at(0), kb = tile_at(1);
      issue_gather(ka < 0 ? 0 : ka, kb < 0 ? 0 : kb, 0, lds_k0);
      int pend_j = -1, pend_kt = -1;
      for (int c = 0; c < chunks; ++c) {
        dsa::lds_barrier<true>();
        if (pend_j >= 0) flush(pend_j, pend_kt);
        pend_j = -1;
        int j1 = j0, o1 = o0 + 64;
        if (o1 >= bp) { o1 -= bp; ++j1; }
        const int ka1 = tile_at(j1), kb1 = tile_at(j1 + 1);
        if (c + 1 < chunks)
          issue_gather(ka1 < 0 ? 0 : ka1, kb1 < 0 ? 0 : kb1, o1, (c & 1) ? lds_k0 : lds_k1);
        const int second = bp - o0;
        const bool has_next = j0 + 1 < n;
        const int split = has_next && second < 64 ? second : -1;
        const int left = total - c * 64;
        const bool masked = bp > p.tile || left < 64 || ka < 0 || kb < 0;
        const unsigned char* cur = (c & 1) ? lds_k1 : lds_k0;
        using one = std::integral_constant<int, 1>;
        using two = std::integral_constant<int, 2>;
        if (left <= 32)
          compute_gather(cur, o0, second, split, j0, masked, left, ka >= 0, kb >= 0, one{});
        else
          compute_gather(cur, o0, second, split, j0, masked, left, ka >= 0, kb >= 0, two{});
        if (has_next && second <= 64) {
          if (second == 64) end_tile(j0);
          pend_j = j0;
          pend_kt = ka;
        }
        j0 = j1; o0 = o1; ka = ka1; kb = kb1;
      }
      end_tile(n - 1);
      dsa::lds_barrier();
      if (pend_j >= 0) flush(pend_j, pend_kt);
      flush(n - 1, tile_at(n - 1));
    }
  } else {
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
  }
  if (kRouted) {
    dsa::lds_barrier();
    // Cells this row does not list hold zero mass and zero centroids.
    const __half zero = __float2half(0.f);
    for (int kt = tid; kt < p.tiles; kt += kThreads) {
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

template <typename T>
void launch_tile_stats(const TileStatsParams& p, bool routed, bool gather, hipStream_t stream) {
  const int32_t tile = p.tile;
  const dim3 blocks((unsigned)((int64_t)p.heads * p.tiles)), threads(256);
  if (gather && tile <= 96) {
    const dim3 three(192);
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<T, true, 2, true, 3>), blocks, three, 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<T, false, 2, true, 3>), blocks, three, 0, stream, p);
  } else if (gather) {
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<T, true, 2, true, 4>), blocks, threads, 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<T, false, 2, true, 4>), blocks, threads, 0, stream, p);
  } else if (tile > 96) {
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<T, true, 2>), blocks, threads, 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<T, false, 2>), blocks, threads, 0, stream, p);
  } else if (tile > kHalfKeys) {
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<T, true, 2, false, 3>), blocks, dim3(192), 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<T, false, 2, false, 3>), blocks, dim3(192), 0, stream, p);
  } else {
    // Two waves even for tiles of at most 32 tokens (one of them then only
    // stages K): one-wave workgroups, four per CU, leave too few waves to
    // hide the dense pass's latency.
    if (routed)
      hipLaunchKernelGGL((tile_stats_kernel<T, true, 1, false, 2>), blocks, dim3(128), 0, stream, p);
    else
      hipLaunchKernelGGL((tile_stats_kernel<T, false, 1, false, 2>), blocks, dim3(128), 0, stream, p);
  }
}

}  // namespace

extern "C" int dsa_tile_stats(const void* q, const void* k, int32_t dtype, const int64_t* strides,
                              int32_t tokens, int32_t heads, int32_t head_dim, int32_t tile_h,
                              int32_t tile_w, const float* lse, int64_t lse_head_stride,
                              const int32_t* row_ptr, const int32_t* col_idx, float scale,
                              float* mass, void* mass_f16, void* centroid_q_y,
                              void* centroid_q_x, void* centroid_k_y, void* centroid_k_x,
                              hipStream_t stream) {
  dsa::clear_error();
  if (!q || !k || !strides || !lse || !mass)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: null pointer argument");
  if (dtype != DSA_BF16 && dtype != DSA_F16)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_tile_stats: dtype %d unsupported (bf16 or fp16)",
                          dtype);
  if ((row_ptr == nullptr) != (col_idx == nullptr))
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: row_ptr and col_idx must both be set");
  if (tokens <= 0 || heads <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_tile_stats: tokens and heads must be positive");
  if (head_dim <= 0 || head_dim > dsa::kHeadDim || head_dim % 8 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_tile_stats: head_dim %d unsupported (a multiple of 8 up to 128)",
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
  p.q = q;
  p.k = k;
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
  p.tile_pad = (tile + 7) & ~7;
  p.head_dim = head_dim;
  p.scale_log2 = scale * kLog2e;
  const bool routed = row_ptr != nullptr;
  const int32_t plain_slots = tile - kHalfKeys <= 32 ? kHalfKeys + 32 : 2 * kHalfKeys;
  const bool gather = tile > kHalfKeys && tile < 2 * kHalfKeys && p.tile_pad < plain_slots &&
                      ((int64_t)tokens + 8) * strides[2] * 2 + kRowBytes <= 0x7fffffff;
  if (dtype == DSA_F16)
    launch_tile_stats<_Float16>(p, routed, gather, stream);
  else
    launch_tile_stats<__bf16>(p, routed, gather, stream);
  return dsa::check_launch("dsa_tile_stats");
}
