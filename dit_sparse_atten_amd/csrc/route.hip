// Sampled route update for gfx950: persistence prior, top-mass selection,
// first-frame sink and CSR construction.
//
// Replaces attention_backends/flex.py (the sampled mass itself,
// _sampled_block_mass 205-251, is sampled_mass.hip):
//   prior + _top_mass_route + _add_first_frame_sink
//                         83-94, 535-548, 550-566 -> route_select_kernel
//   _pack_route / _build_block_mask (KV direction)
//                         275-355, layout_ops.py:128-151 -> counts/scan/compact,
//                                                          pack_rows_kernel
//
// Selection arithmetic (shared bit-for-bit with the CPU oracle): a row value
// m >= 0 is represented as the integer floor(m * 2^52); row sums and prefix
// sums are exact integer sums rounded once to fp32; threshold =
// fp32(fp32(sum) * fp32(target)); prior m' = fp32(m + fp32(rho * fp32(sum/K)));
// order = value descending, key index ascending; count = #{prefix < threshold}
// + 1, clamped to the cap; then the sink columns are OR-ed in.
#include "bsa_tiles.h"
#include "route_common.h"

namespace {

using dsa::fixed_to_f32;
using dsa::to_fixed;
using dsa::wave_sum_i32;
using dsa::wave_sum_i64;

constexpr int kHeadDim = 128;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Top-mass selection: one wave per (head, query-block) row, K <= 64 * kPer
// (512, 1024 or 2048).
// ---------------------------------------------------------------------------

struct SelectParams {
  const float* mass;       // [rows, K]
  const uint8_t* previous; // [rows, K] or null
  uint8_t* route;          // [rows, K]
  int32_t* counts;         // [rows]
  int32_t rows, keys, cap, sink;
  float rho, target;
};

template <int kPer>
__global__ void __launch_bounds__(256) route_select_kernel(SelectParams p) {
  constexpr int kN = 64 * kPer;
  __shared__ uint8_t flags[4][kN];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  if (row >= p.rows) return;  // whole wave exits together; no barriers below
  const int K = p.keys;
  const float* mrow = p.mass + (int64_t)row * K;

  // Element e = lane * kPer + j.
  float v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    float x = e < K ? mrow[e] : 0.f;
    v[j] = x > 0.f ? x : 0.f;  // rows are probabilities: clamp -0.0 and noise
  }
  auto row_max = [&]() {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) mx = fmaxf(mx, v[j]);
    return dsa::wave_max_f32(mx);
  };
  if (p.previous) {
    const int s0 = dsa::row_shift(row_max(), K);
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) s += to_fixed(v[j], s0);
    s = wave_sum_i64(s);
    const float mean = fixed_to_f32(s, s0) / (float)K;
    const float prior = p.rho * mean;
    const uint8_t* prow = p.previous + (int64_t)row * K;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * kPer + j;
      if (e < K && prow[e]) v[j] = v[j] + prior;
    }
  }
  const int shift = dsa::row_shift(row_max(), K);
  int64_t total = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) total += to_fixed(v[j], shift);
  total = wave_sum_i64(total);
  const float threshold = fixed_to_f32(total, shift) * p.target;

  // Descending sort of key = value bits << 32 | (kN - 1 - index).
  uint64_t key[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    key[j] = e < K ? ((uint64_t)__float_as_uint(v[j]) << 32) | (uint32_t)(kN - 1 - e) : 0ull;
  }
  dsa::sort_desc<kPer>(key, lane);

  // Exact prefix sums in sorted order.
  int64_t pre[kPer];
  int64_t run = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    run += to_fixed(__uint_as_float((uint32_t)(key[j] >> 32)), shift);
    pre[j] = run;
  }
  int64_t scan = run;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const int64_t up = __shfl_up((long long)scan, m);
    if (lane >= m) scan += up;
  }
  const int64_t offset = scan - run;
  int below = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    if (e < K && fixed_to_f32(pre[j] + offset, shift) < threshold) ++below;
  }
  int count = wave_sum_i32(below) + 1;
  count = count < p.cap ? count : p.cap;

  uint8_t* f = flags[wave];
#pragma unroll
  for (int j = 0; j < kPer; ++j) f[lane * kPer + j] = 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int pos = lane * kPer + j;
    if (pos < count) f[kN - 1 - (int)(key[j] & 0xffffffffu)] = 1;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  int selected = 0;
  uint8_t* rout = p.route + (int64_t)row * K;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = lane * kPer + j;
    if (e < K) {
      const uint8_t on = (f[e] || e < p.sink) ? 1 : 0;
      rout[e] = on;
      selected += on;
    }
  }
  selected = wave_sum_i32(selected);
  if (lane == 0) p.counts[row] = selected;
}

// Rows of 2049..16384 keys: one 256-thread workgroup per row, the same
// arithmetic as route_select_kernel, values in registers (kPer per thread,
// element e = tid + 256 j) and a bitonic sort of the 64-bit keys in LDS.
constexpr int kWideKeys = 16384;

template <int kPer>
__global__ void __launch_bounds__(256) route_select_wide_kernel(SelectParams p) {
  constexpr int kN = 256 * kPer;
  __shared__ uint64_t keys[kN];  // 128 KB at 16384 keys (LDS: 160 KB per CU)
  __shared__ uint8_t flags[kN];
  __shared__ int64_t scan[256];
  __shared__ int64_t red64[4];
  __shared__ float red32[4];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int K = p.keys;
  const float* mrow = p.mass + (int64_t)row * K;

  float v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + 256 * j;
    const float x = e < K ? mrow[e] : 0.f;
    v[j] = x > 0.f ? x : 0.f;
  }
  auto row_max = [&]() {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) mx = fmaxf(mx, v[j]);
    return dsa::block_max(mx, red32);
  };
  if (p.previous) {
    const int s0 = dsa::row_shift(row_max(), K);
    int64_t sum = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) sum += to_fixed(v[j], s0);
    sum = dsa::block_sum_i64(sum, red64);
    const float mean = fixed_to_f32(sum, s0) / (float)K;
    const float prior = p.rho * mean;
    const uint8_t* prow = p.previous + (int64_t)row * K;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid + 256 * j;
      if (e < K && prow[e]) v[j] = v[j] + prior;
    }
  }
  const int shift = dsa::row_shift(row_max(), K);
  int64_t total = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) total += to_fixed(v[j], shift);
  total = dsa::block_sum_i64(total, red64);
  const float threshold = fixed_to_f32(total, shift) * p.target;

  // Descending bitonic sort of value bits << 32 | (kN - 1 - index).
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = tid + 256 * j;
    keys[e] = e < K ? ((uint64_t)__float_as_uint(v[j]) << 32) | (uint32_t)(kN - 1 - e) : 0ull;
  }
  dsa::sort_desc_lds<kN>(keys);

  // Exact prefix sums in sorted order: each thread a contiguous segment.
  const int seg0 = tid * kPer;
  int64_t local = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) local += to_fixed(__uint_as_float((uint32_t)(keys[seg0 + j] >> 32)), shift);
  scan[tid] = local;
  dsa::lds_barrier();
  for (int offset = 1; offset < 256; offset <<= 1) {
    const int64_t add = tid >= offset ? scan[tid - offset] : 0;
    dsa::lds_barrier();
    scan[tid] += add;
    dsa::lds_barrier();
  }
  int64_t run = scan[tid] - local;
  int below = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    run += to_fixed(__uint_as_float((uint32_t)(keys[seg0 + j] >> 32)), shift);
    if (seg0 + j < K && fixed_to_f32(run, shift) < threshold) ++below;
  }
  below = (int)dsa::block_sum_i64(below, red64);
  int count = below + 1;
  count = count < p.cap ? count : p.cap;

  // Selected flags: the first `count` sorted positions.
  for (int e = tid; e < kN; e += 256) flags[e] = 0;
  dsa::lds_barrier();
  for (int pos = tid; pos < count; pos += 256)
    flags[kN - 1 - (int)(keys[pos] & 0xffffffffu)] = 1;
  dsa::lds_barrier();
  int selected = 0;
  uint8_t* rout = p.route + (int64_t)row * K;
  for (int e = tid; e < K; e += 256) {
    const uint8_t on = (flags[e] || e < p.sink) ? 1 : 0;
    rout[e] = on;
    selected += on;
  }
  selected = (int)dsa::block_sum_i64(selected, red64);
  if (tid == 0) p.counts[row] = selected;
}

// ---------------------------------------------------------------------------
// Route rows -> counts -> row_ptr -> col_idx; stable packing.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256) route_counts_kernel(const uint8_t* route, int32_t rows,
                                                          int32_t keys, int32_t* counts) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint8_t* r = route + (int64_t)row * keys;
  int c = 0;
  for (int e = lane; e < keys; e += 64) c += r[e] != 0;
  c = wave_sum_i32(c);
  if (lane == 0) counts[row] = c;
}

// Single-workgroup exclusive scan: row_ptr[0..rows], nnz = row_ptr[rows].
__global__ void __launch_bounds__(1024) scan_counts_kernel(const int32_t* counts, int32_t rows,
                                                          int32_t* row_ptr, int64_t* nnz) {
  __shared__ int64_t partial[1024];
  const int t = threadIdx.x;
  const int per = (rows + 1023) / 1024;
  const int begin = t * per;
  const int end = begin + per < rows ? begin + per : rows;
  int64_t local = 0;
  for (int i = begin; i < end; ++i) local += counts[i];
  partial[t] = local;
  dsa::lds_barrier();
  for (int offset = 1; offset < 1024; offset <<= 1) {
    const int64_t add = t >= offset ? partial[t - offset] : 0;
    dsa::lds_barrier();
    partial[t] += add;
    dsa::lds_barrier();
  }
  int64_t run = partial[t] - local;
  for (int i = begin; i < end; ++i) {
    row_ptr[i] = (int32_t)run;
    run += counts[i];
  }
  if (t == 1023) {
    row_ptr[rows] = (int32_t)partial[1023];
    if (nnz) *nnz = partial[1023];
  }
}

// Ascending selected column ids of each row at row_ptr[row].
__global__ void __launch_bounds__(256) route_compact_kernel(const uint8_t* route, int32_t rows,
                                                           int32_t keys, const int32_t* row_ptr,
                                                           int32_t* col_idx) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint8_t* r = route + (int64_t)row * keys;
  int base = row_ptr[row];
  for (int e0 = 0; e0 < keys; e0 += 64) {
    const int e = e0 + lane;
    const bool on = e < keys && r[e] != 0;
    const uint64_t mask = __ballot(on);
    if (on) col_idx[base + __popcll(mask & ((1ull << lane) - 1))] = e;
    base += __popcll(mask);
  }
}

// Stable partition: selected ids ascending, then unselected ids ascending.
__global__ void __launch_bounds__(256) pack_rows_kernel(const uint8_t* route, int32_t rows,
                                                       int32_t keys, int32_t* counts,
                                                       int32_t* indices) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint8_t* r = route + (int64_t)row * keys;
  int32_t* out = indices + (int64_t)row * keys;
  int total = 0;
  for (int e = lane; e < keys; e += 64) total += r[e] != 0;
  total = wave_sum_i32(total);
  int sel = 0, unsel = total;
  for (int e0 = 0; e0 < keys; e0 += 64) {
    const int e = e0 + lane;
    const bool valid = e < keys;
    const bool on = valid && r[e] != 0;
    const uint64_t below = (1ull << lane) - 1;
    const uint64_t on_mask = __ballot(on);
    const uint64_t off_mask = __ballot(valid && !on);
    if (on) out[sel + __popcll(on_mask & below)] = e;
    else if (valid) out[unsel + __popcll(off_mask & below)] = e;
    sel += __popcll(on_mask);
    unsel += __popcll(off_mask);
  }
  if (lane == 0) counts[row] = total;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" int dsa_route_select(const float* mass, const uint8_t* previous, int32_t rows,
                                int32_t keys, float rho, float target, int32_t cap,
                                int32_t sink_blocks, uint8_t* route, int32_t* counts,
                                hipStream_t stream) {
  dsa::clear_error();
  if (!mass || !route || !counts) return dsa::set_error(DSA_EINVAL, "dsa_route_select: null pointer");
  if (rows <= 0 || keys <= 0) return dsa::set_error(DSA_EINVAL, "dsa_route_select: empty route");
  if (keys > kWideKeys)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_route_select: at most %d key blocks (got %d)",
                          kWideKeys, keys);
  if (!(target > 0.f && target <= 1.f))
    return dsa::set_error(DSA_EINVAL, "mass_target must be in (0, 1]");
  if (cap < 1) return dsa::set_error(DSA_EINVAL, "dsa_route_select: cap must be >= 1");
  if (!(rho >= 0.f)) return dsa::set_error(DSA_EINVAL, "route_persistence must be non-negative");
  SelectParams p;
  p.mass = mass;
  p.previous = previous;
  p.route = route;
  p.counts = counts;
  p.rows = rows;
  p.keys = keys;
  p.cap = cap;
  p.sink = sink_blocks < 0 ? 0 : sink_blocks;
  p.rho = rho;
  p.target = target;
  const dim3 groups((unsigned)((rows + 3) / 4)), threads(256);
  if (keys <= 512)
    hipLaunchKernelGGL(route_select_kernel<8>, groups, threads, 0, stream, p);
  else if (keys <= 1024)
    hipLaunchKernelGGL(route_select_kernel<16>, groups, threads, 0, stream, p);
  else if (keys <= 2048)
    hipLaunchKernelGGL(route_select_kernel<32>, groups, threads, 0, stream, p);
  else if (keys <= 4096)
    hipLaunchKernelGGL(route_select_wide_kernel<16>, dim3((unsigned)rows), threads, 0, stream, p);
  else if (keys <= 8192)
    hipLaunchKernelGGL(route_select_wide_kernel<32>, dim3((unsigned)rows), threads, 0, stream, p);
  else
    hipLaunchKernelGGL(route_select_wide_kernel<64>, dim3((unsigned)rows), threads, 0, stream, p);
  return dsa::check_launch("dsa_route_select");
}

extern "C" int dsa_route_to_csr(const uint8_t* route, int32_t rows, int32_t keys,
                                const int32_t* counts_or_null, int32_t* counts_out,
                                int32_t* row_ptr, int32_t* col_idx, int64_t* nnz,
                                hipStream_t stream) {
  dsa::clear_error();
  if (!route || !row_ptr || !col_idx)
    return dsa::set_error(DSA_EINVAL, "dsa_route_to_csr: null pointer");
  if (rows <= 0 || keys <= 0) return dsa::set_error(DSA_EINVAL, "dsa_route_to_csr: empty route");
  if ((int64_t)rows * keys > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_route_to_csr: route too large for int32 CSR");
  const int32_t* counts = counts_or_null;
  if (!counts) {
    if (!counts_out)
      return dsa::set_error(DSA_EINVAL, "dsa_route_to_csr: counts_out needed when counts is null");
    hipLaunchKernelGGL(route_counts_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       stream, route, rows, keys, counts_out);
    counts = counts_out;
  }
  hipLaunchKernelGGL(scan_counts_kernel, dim3(1), dim3(1024), 0, stream, counts, rows, row_ptr,
                     nnz);
  hipLaunchKernelGGL(route_compact_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream,
                     route, rows, keys, row_ptr, col_idx);
  return dsa::check_launch("dsa_route_to_csr");
}

extern "C" int dsa_pack_rows(const uint8_t* route, int32_t rows, int32_t keys, int32_t* counts,
                             int32_t* indices, hipStream_t stream) {
  dsa::clear_error();
  if (!route || !counts || !indices) return dsa::set_error(DSA_EINVAL, "dsa_pack_rows: null pointer");
  if (rows <= 0 || keys <= 0) return dsa::set_error(DSA_EINVAL, "dsa_pack_rows: empty route");
  hipLaunchKernelGGL(pack_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream,
                     route, rows, keys, counts, indices);
  return dsa::check_launch("dsa_pack_rows");
}
