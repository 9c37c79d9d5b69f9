// Route updates of the matrix-sparse backend for gfx950: low-mass drop and
// the next-step expansion policies.
//
// Replaces attention_backends/sparse.py:
//   _drop_low_mass + _preserve_one_per_row  339-348, 327-336  -> head stats + drop_kernel
//   first-frame sink of the next mask      883-884
//   _expand "all" / "directional"          350-373 (+ _spatial_neighbors 258-276,
//                                          _apply_directional_steps 285-324)
// Routes are [heads, tiles, tiles] bytes over tile-major tiles; a tile id is
// (frame, y, x) on the per-frame grid of blocks_h x blocks_w tiles.
//
// Arithmetic, shared with the CPU oracle (the reference's torch reductions
// round in a build-specific order):
//  * per-head selected-mass sums are exact fixed-point sums rounded once to
//    fp32 (then to fp16 for fp16 mass);
//  * fp16 mass (the reference's stored route mass): mean = fp16(float(sum16) /
//    count), ratio = fp16(float(m) / float(mean)), kept if ratio >=
//    fp16(drop_factor), as torch evaluates fp16 tensors against Python floats;
//  * fp32 mass: mean = sum / count, ratio = m / max(mean, 1e-12), kept if
//    ratio >= drop_factor;
//  * a row emptied by the drop keeps its first highest-mass original tile;
//  * directional: centroid direction = 0 if fp16 |c| < fp16(threshold), else
//    sign(c); huge blocks use fp32 ratios of the fp16 mass.
#include "route_common.h"

#include <hip/hip_fp16.h>

namespace {

using dsa::fixed_to_f32;
using dsa::to_fixed;

__device__ __forceinline__ float load_mass(const void* mass, int is_f16, int64_t i) {
  return is_f16 ? __half2float(static_cast<const __half*>(mass)[i])
                : static_cast<const float*>(mass)[i];
}

// Per head: exact fixed-point sum of the selected mass and the number of
// selected cells.  The head's cells split into chunks of kHeadChunk, one
// workgroup each; integer sums are exact, so the atomic adds of the
// workgroup partials give the same total in any order.  Readers round the
// total once to fp32 (fixed_to_f32).  `acc` / `cnt` start at zero
// (head_zero_kernel).
constexpr int kHeadChunk = 16384;

__global__ void __launch_bounds__(256) head_zero_kernel(unsigned long long* acc, int32_t* cnt,
                                                       int32_t heads) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < heads) {
    acc[i] = 0ull;
    cnt[i] = 0;
  }
}

__global__ void __launch_bounds__(256) head_partial_kernel(const uint8_t* mask, const void* mass,
                                                          int is_f16, int32_t cells,
                                                          unsigned long long* acc, int32_t* cnt) {
  __shared__ int64_t wsum[4];
  __shared__ int32_t wcnt[4];
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int c0 = blockIdx.x * kHeadChunk;
  const int c1 = min(c0 + kHeadChunk, cells);
  const int64_t base = (int64_t)h * cells;
  int64_t s = 0;
  int32_t c = 0;
  for (int i = c0 + tid; i < c1; i += 256) {
    if (mask[base + i]) {
      const float v = load_mass(mass, is_f16, base + i);
      s += to_fixed(v > 0.f ? v : 0.f);
      ++c;
    }
  }
  s = dsa::wave_sum_i64(s);
  c = dsa::wave_sum_i32(c);
  if ((tid & 63) == 0) {
    wsum[tid >> 6] = s;
    wcnt[tid >> 6] = c;
  }
  dsa::lds_barrier();
  if (tid == 0) {
    const int64_t total = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const int32_t count = (wcnt[0] + wcnt[1]) + (wcnt[2] + wcnt[3]);
    if (total) atomicAdd(&acc[h], (unsigned long long)total);
    if (count) atomicAdd(&cnt[h], count);
  }
}

// head_scratch (float[4 * heads], 8-byte aligned) holds the per-head int64
// fixed-point sums, then the int32 counts.
struct HeadStats {
  unsigned long long* acc;
  int32_t* cnt;
};

HeadStats head_stats_of(float* head_scratch, int32_t heads) {
  return {reinterpret_cast<unsigned long long*>(head_scratch),
          reinterpret_cast<int32_t*>(head_scratch + 2 * heads)};
}

void launch_head_stats(const uint8_t* mask, const void* mass, int is_f16, int32_t heads,
                       int32_t cells, HeadStats hs, hipStream_t stream) {
  hipLaunchKernelGGL(head_zero_kernel, dim3((unsigned)((heads + 255) / 256)), dim3(256), 0,
                     stream, hs.acc, hs.cnt, heads);
  const dim3 grid((unsigned)((cells + kHeadChunk - 1) / kHeadChunk), (unsigned)heads);
  hipLaunchKernelGGL(head_partial_kernel, grid, dim3(256), 0, stream, mask, mass, is_f16, cells,
                     hs.acc, hs.cnt);
}

struct DropParams {
  const uint8_t* mask;
  const void* mass;
  const unsigned long long* head_acc;  // exact fixed-point selected-mass sums
  const int32_t* head_count;
  uint8_t* out;
  int32_t* counts;
  int32_t heads, tiles, sink, is_f16;
  float drop;
};

// One wave per (head, query tile) row.
__global__ void __launch_bounds__(256) drop_kernel(DropParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.heads * p.tiles) return;  // whole wave exits together
  const int h = row / p.tiles;
  const int K = p.tiles;
  const int64_t base = (int64_t)row * K;
  const int count = max(p.head_count[h], 1);
  const float head_sum = fixed_to_f32((int64_t)p.head_acc[h]);
  float mean;
  float drop = p.drop;
  if (p.is_f16) {
    const float sum16 = __half2float(__float2half(head_sum));
    mean = __half2float(__float2half(sum16 / (float)count));
    drop = __half2float(__float2half(p.drop));
  } else {
    mean = fmaxf(head_sum / (float)count, 1e-12f);
  }
  auto kept_at = [&](int k, float& m) -> bool {
    m = load_mass(p.mass, p.is_f16, base + k);
    float ratio = m / mean;
    if (p.is_f16) ratio = __half2float(__float2half(ratio));
    return ratio >= drop;  // NaN (0 / 0) compares false
  };
  // Pass 1: does the row keep anything, did it select anything, and its
  // first maximal original tile.
  int kept_any = 0, orig_any = 0;
  float best = -INFINITY;
  int best_k = 0x7fffffff;
  for (int k = lane; k < K; k += 64) {
    if (p.mask[base + k] == 0) continue;
    float m;
    kept_any |= kept_at(k, m) ? 1 : 0;
    orig_any = 1;
    if (m > best || (m == best && k < best_k)) {
      best = m;
      best_k = k;
    }
  }
  kept_any = __any(kept_any) ? 1 : 0;
  orig_any = __any(orig_any) ? 1 : 0;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ob = __shfl_xor(best, m);
    const int ok = __shfl_xor(best_k, m);
    if (ob > best || (ob == best && ok < best_k)) {
      best = ob;
      best_k = ok;
    }
  }
  // A row the drop emptied keeps its first highest-mass original tile; the
  // sink columns are set afterwards and take no part in that test.
  const int restore_k = (orig_any && !kept_any) ? best_k : -1;
  // Pass 2: write the row once.
  int selected = 0;
  for (int k = lane; k < K; k += 64) {
    float m;
    const bool set = (p.mask[base + k] != 0 && kept_at(k, m)) || k < p.sink || k == restore_k;
    p.out[base + k] = set ? 1 : 0;
    selected += set;
  }
  selected = dsa::wave_sum_i32(selected);
  if (lane == 0) p.counts[row] = selected;
}

// --- expansion ------------------------------------------------------------

constexpr int kPolicyAll = 1;
constexpr int kPolicyDirectional = 2;

struct ExpandParams {
  const uint8_t* mask;
  const __half* mass;
  const __half* cqy;
  const __half* cqx;
  const __half* cky;
  const __half* ckx;
  const unsigned long long* head_acc;  // exact fixed-point sums (directional only)
  const int32_t* head_count;
  uint8_t* out;
  int32_t heads, tiles, frames, blocks_h, blocks_w, policy;
  float threshold, huge;
};

__global__ void __launch_bounds__(256) copy_bytes_kernel(const uint8_t* src, uint8_t* dst,
                                                        int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

__device__ __forceinline__ int direction_of(__half c, __half threshold) {
  const float v = __half2float(c);
  if (fabsf(v) < __half2float(threshold)) return 0;
  return v > 0.f ? 1 : (v < 0.f ? -1 : 0);
}

// One thread per cell: selected cells mark their targets in `out` (which
// already holds the mask; every write stores 1).
__global__ void __launch_bounds__(256) expand_kernel(ExpandParams p) {
  const int64_t cells = (int64_t)p.tiles * p.tiles;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= cells * p.heads) return;
  if (!p.mask[idx]) return;
  const int h = (int)(idx / cells);
  const int64_t cell = idx % cells;
  const int qt = (int)(cell / p.tiles), kt = (int)(cell % p.tiles);
  const int per_frame = p.blocks_h * p.blocks_w;
  const int qf = qt / per_frame, qy = (qt % per_frame) / p.blocks_w, qx = qt % p.blocks_w;
  const int kf = kt / per_frame, ky = (kt % per_frame) / p.blocks_w, kx = kt % p.blocks_w;
  uint8_t* hout = p.out + (int64_t)h * cells;
  auto mark = [&](int y1, int x1, int y2, int x2) {
    if (y1 < 0 || y1 >= p.blocks_h || x1 < 0 || x1 >= p.blocks_w) return;
    if (y2 < 0 || y2 >= p.blocks_h || x2 < 0 || x2 >= p.blocks_w) return;
    const int t1 = qf * per_frame + y1 * p.blocks_w + x1;
    const int t2 = kf * per_frame + y2 * p.blocks_w + x2;
    hout[(int64_t)t1 * p.tiles + t2] = 1;
  };
  bool huge = p.policy == kPolicyAll;
  if (p.policy == kPolicyDirectional) {
    const float count = (float)max(p.head_count[h], 1);
    const float mean = fmaxf(fixed_to_f32((int64_t)p.head_acc[h]) / count, 1e-12f);
    huge = __half2float(p.mass[idx]) / mean >= p.huge;
  }
  if (huge) {
    // Eight coupled neighbours: the same (dy, dx) on the query and key tiles.
    for (int dy = -1; dy <= 1; ++dy)
      for (int dx = -1; dx <= 1; ++dx)
        if (dy || dx) mark(qy + dy, qx + dx, ky + dy, kx + dx);
    return;
  }
  const __half thr = __float2half(p.threshold);
  const int dqy = direction_of(p.cqy[idx], thr), dqx = direction_of(p.cqx[idx], thr);
  const int dky = direction_of(p.cky[idx], thr), dkx = direction_of(p.ckx[idx], thr);
  if (dqy || dqx) mark(qy + dqy, qx + dqx, ky, kx);                 // move Q only
  if (dky || dkx) mark(qy, qx, ky + dky, kx + dkx);                 // move K only
  if (dqy || dqx || dky || dkx) mark(qy + dqy, qx + dqx, ky + dky, kx + dkx);  // both
}

int check_tiles(const char* what, int32_t heads, int32_t tiles) {
  if (heads <= 0 || tiles <= 0)
    return dsa::set_error(DSA_EINVAL, "%s: heads and tiles must be positive", what);
  if ((int64_t)heads * tiles * tiles > 0x7fffffffLL)
    return dsa::set_error(DSA_EINVAL, "%s: route too large", what);
  return DSA_OK;
}

}  // namespace

extern "C" int dsa_drop_low_mass(const uint8_t* mask, const void* mass, int32_t mass_is_f16,
                                 int32_t heads, int32_t tiles, float drop_factor,
                                 int32_t sink_tiles, float* head_scratch, uint8_t* out,
                                 int32_t* counts, hipStream_t stream) {
  dsa::clear_error();
  if (!mask || !mass || !head_scratch || !out || !counts)
    return dsa::set_error(DSA_EINVAL, "dsa_drop_low_mass: null pointer");
  const int status = check_tiles("dsa_drop_low_mass", heads, tiles);
  if (status) return status;
  if (!(drop_factor > 0.f))
    return dsa::set_error(DSA_EINVAL, "dsa_drop_low_mass: drop_factor must be positive "
                                      "(a non-positive factor keeps the mask unchanged)");
  if (reinterpret_cast<uintptr_t>(head_scratch) % 8 != 0)
    return dsa::set_error(DSA_EINVAL, "dsa_drop_low_mass: head_scratch must be 8-byte aligned");
  const HeadStats hs = head_stats_of(head_scratch, heads);
  launch_head_stats(mask, mass, mass_is_f16 ? 1 : 0, heads, tiles * tiles, hs, stream);
  DropParams p{mask, mass, hs.acc, hs.cnt, out, counts, heads, tiles,
               sink_tiles < 0 ? 0 : sink_tiles, mass_is_f16 ? 1 : 0, drop_factor};
  hipLaunchKernelGGL(drop_kernel, dim3((unsigned)(((int64_t)heads * tiles + 3) / 4)), dim3(256),
                     0, stream, p);
  return dsa::check_launch("dsa_drop_low_mass");
}

extern "C" int dsa_expand_route(const uint8_t* mask, const void* mass_f16,
                                const void* centroid_q_y, const void* centroid_q_x,
                                const void* centroid_k_y, const void* centroid_k_x,
                                int32_t heads, int32_t frames, int32_t blocks_h,
                                int32_t blocks_w, int32_t policy, float centroid_threshold,
                                float huge_factor, float* head_scratch, uint8_t* out,
                                hipStream_t stream) {
  dsa::clear_error();
  if (!mask || !out) return dsa::set_error(DSA_EINVAL, "dsa_expand_route: null route");
  if (policy != kPolicyAll && policy != kPolicyDirectional)
    return dsa::set_error(DSA_EINVAL, "dsa_expand_route: policy must be 1 (all) or 2 (directional)");
  if (frames <= 0 || blocks_h <= 0 || blocks_w <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_expand_route: empty tile grid");
  const int64_t tiles64 = (int64_t)frames * blocks_h * blocks_w;
  if (tiles64 > 0x7fffffff) return dsa::set_error(DSA_EINVAL, "dsa_expand_route: too many tiles");
  const int32_t tiles = (int32_t)tiles64;
  const int status = check_tiles("dsa_expand_route", heads, tiles);
  if (status) return status;
  if (policy == kPolicyDirectional &&
      (!mass_f16 || !centroid_q_y || !centroid_q_x || !centroid_k_y || !centroid_k_x ||
       !head_scratch))
    return dsa::set_error(DSA_EINVAL,
                          "dsa_expand_route: directional needs mass, centroids and scratch");
  const int64_t n = (int64_t)heads * tiles * tiles;
  hipLaunchKernelGGL(copy_bytes_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     mask, out, n);
  if (head_scratch && reinterpret_cast<uintptr_t>(head_scratch) % 8 != 0)
    return dsa::set_error(DSA_EINVAL, "dsa_expand_route: head_scratch must be 8-byte aligned");
  const HeadStats hs = head_scratch ? head_stats_of(head_scratch, heads) : HeadStats{nullptr, nullptr};
  if (policy == kPolicyDirectional)
    launch_head_stats(mask, mass_f16, 1, heads, tiles * tiles, hs, stream);
  ExpandParams p;
  p.mask = mask;
  p.mass = static_cast<const __half*>(mass_f16);
  p.cqy = static_cast<const __half*>(centroid_q_y);
  p.cqx = static_cast<const __half*>(centroid_q_x);
  p.cky = static_cast<const __half*>(centroid_k_y);
  p.ckx = static_cast<const __half*>(centroid_k_x);
  p.head_acc = hs.acc;
  p.head_count = hs.cnt;
  p.out = out;
  p.heads = heads;
  p.tiles = tiles;
  p.frames = frames;
  p.blocks_h = blocks_h;
  p.blocks_w = blocks_w;
  p.policy = policy;
  p.threshold = centroid_threshold;
  p.huge = huge_factor;
  hipLaunchKernelGGL(expand_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_expand_route");
}
