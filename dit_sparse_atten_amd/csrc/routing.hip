// Frontier mask and frontier-aware directional route update for gfx950.
//
// Replaces attention_backends/routing.py:
//   frontier_mask               10-41  -> frontier_kernel
//   directional_budget_update   92-168 -> fill (candidates) + dir_expand_kernel
//   (_sparse_best_targets 53-80,          + dir_select_kernel
//    _select_fixed_budget 83-89)
// Routes are [heads, blocks, blocks] bytes (query block rows, key block
// columns); neighbors is the layout's [blocks, 4] int32 table (-1 = none;
// any entry outside [0, blocks) counts as none).
//
// Arithmetic shared bit-for-bit with the CPU oracle: row mean = fp32(exact
// row sum / K); score = fp32(fp32(m + fp32(persistence * mean) [previous])
// + fp32(bonus * mean) [candidate]); budget = clamp(ceil(fp32(|previous| *
// budget_scale)), 1, cap); every ordering is value descending, then key index
// ascending; the best neighbour is the first direction holding the maximum.
#include "route_common.h"

namespace {

using dsa::fixed_to_f32;
using dsa::to_fixed;
using dsa::wave_sum_i32;
using dsa::wave_sum_i64;

// ---------------------------------------------------------------------------
// Frontier: selected cells with an unselected valid neighbour along the query
// axis (rows) or the key axis (columns).  One wave per (head, query block).
// ---------------------------------------------------------------------------

struct FrontierParams {
  const uint8_t* route;
  const int32_t* nb;
  uint8_t* frontier;
  unsigned long long* count;  // optional total of set cells
  int32_t heads, blocks;
};

__global__ void __launch_bounds__(256) zero_u64_kernel(unsigned long long* value) { *value = 0ull; }

__global__ void __launch_bounds__(256) frontier_kernel(FrontierParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);  // h * blocks + q
  if (row >= p.heads * p.blocks) return;                // whole wave exits together
  const int B = p.blocks;
  const int q = row % B;
  const uint8_t* hroute = p.route + (int64_t)(row / B) * B * B;
  const uint8_t* rrow = hroute + (int64_t)q * B;
  int nq[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) nq[d] = p.nb[q * 4 + d];
  int c = 0;
  for (int k = lane; k < B; k += 64) {
    const bool on = rrow[k] != 0;
    bool open = false;
    if (on) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int t = nq[d];
        open |= (unsigned)t < (unsigned)B && hroute[(int64_t)t * B + k] == 0;
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int t = p.nb[k * 4 + d];
        open |= (unsigned)t < (unsigned)B && rrow[t] == 0;
      }
    }
    const uint8_t f = (on && open) ? 1 : 0;
    p.frontier[(int64_t)row * B + k] = f;
    c += f;
  }
  if (p.count) {
    c = wave_sum_i32(c);
    if (lane == 0 && c) atomicAdd(p.count, (unsigned long long)c);
  }
}

// ---------------------------------------------------------------------------
// Directional budget update.
// ---------------------------------------------------------------------------

constexpr int kExpandQ = 1;
constexpr int kExpandK = 2;
constexpr int kExpandJoint = 4;

struct DirParams {
  const float* mass;            // [H, B, B], non-negative
  const uint8_t* previous;      // [H, B, B]
  const uint8_t* prev_frontier; // [H, B, B] or null (computed from previous)
  const int32_t* nb;            // [B, 4]
  uint8_t* candidates;          // [H, B, B]; zero before dir_expand_kernel
  uint8_t* exploration;         // [H, B, B] or null
  uint8_t* route;               // [H, B, B]
  int32_t* counts;              // [H, B] (selected + sink per row)
  uint8_t* dropped;             // optional
  uint8_t* added;               // optional
  int32_t heads, blocks, cap, explore, sink, flags;
  float persistence, min_ratio, bonus, budget_scale;
};

__global__ void __launch_bounds__(256) fill_zero_kernel(uint8_t* out, int64_t bytes) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
  if (i + 16 <= bytes) {
    const dsa_u32x4 z = {0u, 0u, 0u, 0u};
    *reinterpret_cast<dsa_u32x4*>(out + i) = z;
  } else {
    for (int64_t j = i; j < bytes; ++j) out[j] = 0;
  }
}

// One wave per (head, query block): for every source-frontier cell, the best
// unselected query-axis and key-axis neighbours; eligible targets are marked
// in `candidates` (several cells may mark one target: every write stores 1).
__global__ void __launch_bounds__(256) dir_expand_kernel(DirParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.heads * p.blocks) return;
  const int B = p.blocks;
  const int q = row % B;
  const int64_t hbase = (int64_t)(row / B) * B * B;
  const uint8_t* hprev = p.previous + hbase;
  const float* hmass = p.mass + hbase;
  uint8_t* hcand = p.candidates + hbase;
  const uint8_t* prow = hprev + (int64_t)q * B;
  const float* mrow = hmass + (int64_t)q * B;
  int nq[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) nq[d] = p.nb[q * 4 + d];
  for (int k = lane; k < B; k += 64) {
    // Query-axis neighbours (rows nq[d], same key block).
    float best_q = -INFINITY;
    int tq = 0;
    bool open = false;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int t = nq[d];
      if ((unsigned)t < (unsigned)B && hprev[(int64_t)t * B + k] == 0) {
        open = true;
        const float value = hmass[(int64_t)t * B + k];
        if (value > best_q) { best_q = value; tq = t; }
      }
    }
    // Key-axis neighbours (same row, key blocks nb[k][d]).
    float best_k = -INFINITY;
    int tk = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int t = p.nb[k * 4 + d];
      if ((unsigned)t < (unsigned)B && prow[t] == 0) {
        open = true;
        const float value = mrow[t];
        if (value > best_k) { best_k = value; tk = t; }
      }
    }
    const bool source = p.prev_frontier ? p.prev_frontier[hbase + (int64_t)q * B + k] != 0
                                        : (prow[k] != 0 && open);
    if (!source) continue;
    const float floor_value = mrow[k] * p.min_ratio;
    const bool eq = best_q != -INFINITY && best_q >= floor_value;
    const bool ek = best_k != -INFINITY && best_k >= floor_value;
    if ((p.flags & kExpandQ) && eq) hcand[(int64_t)tq * B + k] = 1;
    if ((p.flags & kExpandK) && ek) hcand[(int64_t)q * B + tk] = 1;
    if ((p.flags & kExpandJoint) && eq && ek) hcand[(int64_t)tq * B + tk] = 1;
  }
}

// Order-preserving image of a float (-0.0 taken as +0.0), key index below
// (kN - 1 - e in the low bits, so equal values order by ascending index).
template <int kN>
__device__ __forceinline__ uint64_t order_key(bool flag, float value, int e) {
  uint32_t bits = __float_as_uint(value == 0.f ? 0.f : value);
  bits = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return ((uint64_t)flag << 63) | ((uint64_t)bits << 31) | (uint32_t)(kN - 1 - e);
}

template <int kN>
__device__ __forceinline__ int key_index(uint64_t key) {
  return kN - 1 - (int)(key & (uint64_t)(kN - 1));
}

// Scatters the first `count` sorted keys as flags into f[0..kN) (LDS) and
// returns this lane's kPer flags e = lane * kPer + j.
template <int kPer>
__device__ __forceinline__ void sorted_prefix_flags(const uint64_t key[kPer], int lane, int count,
                                                    bool need_flag_bit, uint8_t* f,
                                                    bool out[kPer]) {
  constexpr int kN = 64 * kPer;
#pragma unroll
  for (int j = 0; j < kPer; ++j) f[lane * kPer + j] = 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int pos = lane * kPer + j;
    if (pos < count && (!need_flag_bit || (key[j] >> 63))) f[key_index<kN>(key[j])] = 1;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < kPer; ++j) out[j] = f[lane * kPer + j] != 0;
  __builtin_amdgcn_wave_barrier();
}

// One wave per (head, query block): final candidates, exploration, scores
// and the fixed-budget selection, then the sink columns.  K <= 64 * kPer.
template <int kPer>
__global__ void __launch_bounds__(256) dir_select_kernel(DirParams p) {
  constexpr int kN = 64 * kPer;
  __shared__ uint8_t flags[4][kN];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  if (row >= p.heads * p.blocks) return;  // whole wave exits together; no barriers below
  const int K = p.blocks;
  const int64_t base = (int64_t)row * K;
  uint8_t* f = flags[wave];

  float m[kPer];
  bool prev[kPer], cand[kPer], pool[kPer];
  int prev_count = 0, pool_count = 0;
  int64_t fixed_sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    const bool in = e < K;
    m[j] = in ? p.mass[base + e] : 0.f;
    prev[j] = in && p.previous[base + e] != 0;
    cand[j] = in && !prev[j] && p.candidates[base + e] != 0;
    pool[j] = prev[j] || cand[j];
    prev_count += prev[j];
  }
  // Exact row sum (scaled fixed point, route_common.h) for the row mean.
  float row_max = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) row_max = fmaxf(row_max, m[j] > 0.f ? m[j] : 0.f);
  const int shift = dsa::row_shift(dsa::wave_max_f32(row_max), K);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    fixed_sum += e < K ? to_fixed(m[j] > 0.f ? m[j] : 0.f, shift) : 0;
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    if (e < K) p.candidates[base + e] = cand[j];
  }

  uint64_t key[kPer];
  if (p.explore > 0) {
    // Highest-mass blocks outside the pool (pool blocks rank last, by index).
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * kPer + j;
      key[j] = e < K ? order_key<kN>(!pool[j], pool[j] ? 0.f : m[j], e) : 0ull;
    }
    dsa::sort_desc<kPer>(key, lane);
    bool ex[kPer];
    sorted_prefix_flags<kPer>(key, lane, p.explore < K ? p.explore : K, false, f, ex);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * kPer + j;
      if (e < K) {
        if (p.exploration) p.exploration[base + e] = ex[j];
        pool[j] = pool[j] || ex[j];
      }
    }
  } else if (p.exploration) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * kPer + j;
      if (e < K) p.exploration[base + e] = 0;
    }
  }

#pragma unroll
  for (int j = 0; j < kPer; ++j) pool_count += pool[j];
  pool_count = wave_sum_i32(pool_count);
  prev_count = wave_sum_i32(prev_count);
  fixed_sum = wave_sum_i64(fixed_sum);
  const float mean = fixed_to_f32(fixed_sum, shift) / (float)K;
  const float prior = p.persistence * mean;
  const float bonus = p.bonus * mean;
  int budget = (int)ceilf((float)prev_count * p.budget_scale);
  budget = budget < 1 ? 1 : (budget > p.cap ? p.cap : budget);
  int count = budget < pool_count ? budget : pool_count;
  count = count < 1 ? 1 : count;

#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    float score = m[j];
    if (prev[j]) score = score + prior;
    if (p.bonus != 0.f && cand[j]) score = score + bonus;
    key[j] = e < K ? order_key<kN>(pool[j], pool[j] ? score : 0.f, e) : 0ull;
  }
  dsa::sort_desc<kPer>(key, lane);
  bool sel[kPer];
  sorted_prefix_flags<kPer>(key, lane, count, true, f, sel);

  int selected = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    if (e < K) {
      const uint8_t on = (sel[j] || e < p.sink) ? 1 : 0;
      p.route[base + e] = on;
      selected += on;
      if (p.dropped) p.dropped[base + e] = prev[j] && !sel[j];
      if (p.added) p.added[base + e] = sel[j] && !prev[j];
    }
  }
  selected = wave_sum_i32(selected);
  if (lane == 0) p.counts[row] = selected;
}

// Rows of 2049..16384 blocks: one 256-thread workgroup per (head, query
// block), the arithmetic of dir_select_kernel with element e = tid + 256 j in
// registers and both sorts over LDS keys.  Keys order by flag, value, then
// ascending index whatever kN is, so the selection equals the one-wave
// kernel's.
constexpr int kWideBlocks = 16384;

template <int kPer>
__global__ void __launch_bounds__(256) dir_select_wide_kernel(DirParams p) {
  constexpr int kN = 256 * kPer;
  __shared__ uint64_t keys[kN];  // 128 KB at 16384 blocks (LDS: 160 KB per CU)
  __shared__ uint8_t flags[kN];
  __shared__ int64_t red64[4];
  __shared__ float red32[4];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int K = p.blocks;
  const int64_t base = (int64_t)row * K;

  float m[kPer];
  bool prev[kPer], cand[kPer], pool[kPer];
  int prev_count = 0;
  float row_max = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + 256 * j;
    const bool in = e < K;
    m[j] = in ? p.mass[base + e] : 0.f;
    prev[j] = in && p.previous[base + e] != 0;
    cand[j] = in && !prev[j] && p.candidates[base + e] != 0;
    pool[j] = prev[j] || cand[j];
    prev_count += prev[j];
    row_max = fmaxf(row_max, m[j] > 0.f ? m[j] : 0.f);
    if (in) p.candidates[base + e] = cand[j];
  }
  const int shift = dsa::row_shift(dsa::block_max(row_max, red32), K);
  int64_t fixed_sum = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + 256 * j;
    fixed_sum += e < K ? to_fixed(m[j] > 0.f ? m[j] : 0.f, shift) : 0;
  }

  // The first `count` sorted keys (with the flag bit, if need_flag) as flags
  // of their elements; out[j] for this thread's elements.
  auto prefix_flags = [&](int count, bool need_flag, bool out[kPer]) {
    for (int e = tid; e < kN; e += 256) flags[e] = 0;
    dsa::lds_barrier();
    for (int pos = tid; pos < count; pos += 256)
      if (!need_flag || (keys[pos] >> 63)) flags[key_index<kN>(keys[pos])] = 1;
    dsa::lds_barrier();
#pragma unroll
    for (int j = 0; j < kPer; ++j) out[j] = flags[tid + 256 * j] != 0;
    dsa::lds_barrier();  // keys and flags are free again
  };

  if (p.explore > 0) {
    // Highest-mass blocks outside the pool (pool blocks rank last, by index).
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 256 * j;
      keys[e] = e < K ? order_key<kN>(!pool[j], pool[j] ? 0.f : m[j], e) : 0ull;
    }
    dsa::sort_desc_lds<kN>(keys);
    bool ex[kPer];
    prefix_flags(p.explore < K ? p.explore : K, false, ex);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 256 * j;
      if (e < K) {
        if (p.exploration) p.exploration[base + e] = ex[j];
        pool[j] = pool[j] || ex[j];
      }
    }
  } else if (p.exploration) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 256 * j;
      if (e < K) p.exploration[base + e] = 0;
    }
  }

  int pool_count = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) pool_count += pool[j];
  pool_count = (int)dsa::block_sum_i64(pool_count, red64);
  prev_count = (int)dsa::block_sum_i64(prev_count, red64);
  fixed_sum = dsa::block_sum_i64(fixed_sum, red64);
  const float mean = fixed_to_f32(fixed_sum, shift) / (float)K;
  const float prior = p.persistence * mean;
  const float bonus = p.bonus * mean;
  int budget = (int)ceilf((float)prev_count * p.budget_scale);
  budget = budget < 1 ? 1 : (budget > p.cap ? p.cap : budget);
  int count = budget < pool_count ? budget : pool_count;
  count = count < 1 ? 1 : count;

#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + 256 * j;
    float score = m[j];
    if (prev[j]) score = score + prior;
    if (p.bonus != 0.f && cand[j]) score = score + bonus;
    keys[e] = e < K ? order_key<kN>(pool[j], pool[j] ? score : 0.f, e) : 0ull;
  }
  dsa::sort_desc_lds<kN>(keys);
  bool sel[kPer];
  prefix_flags(count, true, sel);

  int selected = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + 256 * j;
    if (e < K) {
      const uint8_t on = (sel[j] || e < p.sink) ? 1 : 0;
      p.route[base + e] = on;
      selected += on;
      if (p.dropped) p.dropped[base + e] = prev[j] && !sel[j];
      if (p.added) p.added[base + e] = sel[j] && !prev[j];
    }
  }
  selected = (int)dsa::block_sum_i64(selected, red64);
  if (tid == 0) p.counts[row] = selected;
}

unsigned row_groups(int64_t rows) { return (unsigned)((rows + 3) / 4); }

int check_route_shape(const char* what, int32_t heads, int32_t blocks, const int32_t* nb) {
  if (heads <= 0 || blocks <= 0)
    return dsa::set_error(DSA_EINVAL, "%s: heads and blocks must be positive", what);
  if (blocks > kWideBlocks)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: %d blocks (at most %d)", what, blocks,
                          kWideBlocks);
  if (!nb) return dsa::set_error(DSA_EINVAL, "%s: neighbors must be given", what);
  if ((int64_t)heads * blocks > 0x7fffffffLL)
    return dsa::set_error(DSA_EINVAL, "%s: route too large", what);
  return DSA_OK;
}

}  // namespace

extern "C" int dsa_frontier_mask(const uint8_t* route, int32_t heads, int32_t blocks,
                                 const int32_t* neighbors, uint8_t* frontier,
                                 unsigned long long* count, hipStream_t stream) {
  dsa::clear_error();
  if (!route || !frontier) return dsa::set_error(DSA_EINVAL, "dsa_frontier_mask: null route");
  const int status = check_route_shape("dsa_frontier_mask", heads, blocks, neighbors);
  if (status) return status;
  FrontierParams p{route, neighbors, frontier, count, heads, blocks};
  if (count) hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(1), 0, stream, count);
  hipLaunchKernelGGL(frontier_kernel, dim3(row_groups((int64_t)heads * blocks)), dim3(256), 0,
                     stream, p);
  return dsa::check_launch("dsa_frontier_mask");
}

extern "C" int dsa_directional_update(
    const float* mass, const uint8_t* previous, const uint8_t* previous_frontier,
    const int32_t* neighbors, int32_t heads, int32_t blocks, int32_t cap, float persistence,
    float min_ratio, float candidate_bonus, float budget_scale, int32_t explore_count,
    int32_t expand_flags, int32_t sink_blocks, uint8_t* route, int32_t* counts,
    uint8_t* candidates, uint8_t* exploration, uint8_t* dropped, uint8_t* added,
    hipStream_t stream) {
  dsa::clear_error();
  if (!mass || !previous || !route || !counts || !candidates)
    return dsa::set_error(DSA_EINVAL, "dsa_directional_update: null required pointer");
  const int status = check_route_shape("dsa_directional_update", heads, blocks, neighbors);
  if (status) return status;
  if (cap < 1 || cap > blocks)
    return dsa::set_error(DSA_EINVAL, "dsa_directional_update: cap %d outside [1, %d]", cap,
                          blocks);
  if (!(budget_scale > 0.f))
    return dsa::set_error(DSA_EINVAL, "dsa_directional_update: budget_scale must be positive");
  if (explore_count < 0 || sink_blocks < 0 || (expand_flags & ~7))
    return dsa::set_error(DSA_EINVAL, "dsa_directional_update: invalid explore/sink/flags");
  if ((reinterpret_cast<uintptr_t>(candidates) & 15u) != 0)
    return dsa::set_error(DSA_EINVAL, "dsa_directional_update: candidates must be 16-byte aligned");
  if (!(persistence >= 0.f) || !(min_ratio >= 0.f) || !(candidate_bonus >= 0.f))
    return dsa::set_error(DSA_EINVAL,
                          "dsa_directional_update: persistence, min_ratio and bonus must be >= 0");
  DirParams p;
  p.mass = mass;
  p.previous = previous;
  p.prev_frontier = previous_frontier;
  p.nb = neighbors;
  p.candidates = candidates;
  p.exploration = exploration;
  p.route = route;
  p.counts = counts;
  p.dropped = dropped;
  p.added = added;
  p.heads = heads;
  p.blocks = blocks;
  p.cap = cap;
  p.explore = explore_count;
  p.sink = sink_blocks;
  p.flags = expand_flags;
  p.persistence = persistence;
  p.min_ratio = min_ratio;
  p.bonus = candidate_bonus;
  p.budget_scale = budget_scale;
  const int64_t cells = (int64_t)heads * blocks * blocks;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((cells + 4095) / 4096)), dim3(256), 0,
                     stream, candidates, cells);
  const unsigned rows = (unsigned)((int64_t)heads * blocks);
  const unsigned groups = row_groups(rows);
  hipLaunchKernelGGL(dir_expand_kernel, dim3(groups), dim3(256), 0, stream, p);
  if (blocks <= 512)
    hipLaunchKernelGGL(dir_select_kernel<8>, dim3(groups), dim3(256), 0, stream, p);
  else if (blocks <= 1024)
    hipLaunchKernelGGL(dir_select_kernel<16>, dim3(groups), dim3(256), 0, stream, p);
  else if (blocks <= 2048)
    hipLaunchKernelGGL(dir_select_kernel<32>, dim3(groups), dim3(256), 0, stream, p);
  else if (blocks <= 4096)
    hipLaunchKernelGGL(dir_select_wide_kernel<16>, dim3(rows), dim3(256), 0, stream, p);
  else if (blocks <= 8192)
    hipLaunchKernelGGL(dir_select_wide_kernel<32>, dim3(rows), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(dir_select_wide_kernel<64>, dim3(rows), dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_directional_update");
}
