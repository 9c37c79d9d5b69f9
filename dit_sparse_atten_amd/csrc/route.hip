// Sampled route update for gfx950: block-mass estimate, persistence prior,
// top-mass selection, first-frame sink and CSR construction.
//
// Replaces attention_backends/flex.py:
//   _sampled_block_mass   205-251  -> sampled_mass_kernel (one fused launch)
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
// Sampled block mass
// ---------------------------------------------------------------------------

struct MassParams {
  const __bf16* q;
  const __bf16* k;
  float* mass;  // [heads, blocks, blocks]
  int64_t q_st, q_sh, k_st, k_sh;
  int32_t tokens, heads, blocks, block_size;
  float scale;        // score scale (d^-1/2 unless given)
  float logw_full;    // log(block_size / samples)
  float logw_last;    // log(size of the last block / samples)
};

// Token index of sampled slot j (block j / S, sample j % S), flex.py:224-231.
template <int S>
__device__ __forceinline__ int sampled_token(int j, int tokens, int block_size) {
  const int blk = j / S;
  const int s = j % S;
  int size = tokens - blk * block_size;
  size = size < block_size ? size : block_size;
  int local = ((2 * s + 1) * size) / (2 * S);
  local = local < size - 1 ? local : size - 1;
  return blk * block_size + local;
}

// bf16 rounding (round to nearest even) of two fp32 values, returned as fp32.
__device__ __forceinline__ void round_bf16_pair(float a, float b, float& ra, float& rb) {
  const dsa_f32x2 two = {a, b};
  const dsa_bf16x2 h = __builtin_convertvector(two, dsa_bf16x2);
  const uint32_t bits = __builtin_bit_cast(uint32_t, h);
  ra = __builtin_bit_cast(float, bits << 16);
  rb = __builtin_bit_cast(float, bits & 0xFFFF0000u);
}

// One workgroup (4 waves x 32 sampled queries) scans every sampled key twice:
// sweep 1 builds each query's log-sum-exp, sweep 2 sums the normalised
// probabilities per (query block, key block).  The sampled score matrix is
// never written to memory.  The scan is VALU-bound (the per-score rounding
// and softmax work outweighs the 32x32x16 MFMAs several times), so scores
// are rounded in pairs, the log2(e) scale and log-weight fold into one fma,
// the max runs over the rounded scores, and only the tile holding the
// sequence's last sampled keys pays the per-score tail checks.  Sampled key
// rows are gathered straight into LDS (buffer loads with a per-lane row
// offset), double-buffered one 64-key tile ahead of the compute.
template <int S>
__global__ void __launch_bounds__(256) sampled_mass_kernel(MassParams p) {
  constexpr int kTileKeys = 64;
  constexpr int KBS = 32 / S;  // key blocks covered by one 32-key sub-tile
  __shared__ __attribute__((aligned(1024))) unsigned char st0[kTileKeys * 256];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[kTileKeys * 256];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;
  const int h = blockIdx.y;
  const int ns = p.blocks * S;
  const int tiles = (ns + kTileKeys - 1) / kTileKeys;
  const int q0 = blockIdx.x * 128 + wave * 32;  // first sampled query of this wave

  int qs = q0 + qi;
  qs = qs < ns ? qs : ns - 1;
  const __bf16* qrow =
      p.q + h * p.q_sh + (int64_t)sampled_token<S>(qs, p.tokens, p.block_size) * p.q_st;
  dsa_bf16x8 qf[8];
#pragma unroll
  for (int dc = 0; dc < 8; ++dc)
    qf[dc] = *reinterpret_cast<const dsa_bf16x8*>(qrow + dc * 16 + g * 8);

  // The head's K rows as one raw buffer (the host keeps them within 2^31 bytes).
  const __bf16* kbase = p.k + h * p.k_sh;
  const __amdgpu_buffer_rsrc_t k_rsrc =
      dsa::make_rsrc(kbase, (uint32_t)(((int64_t)(p.tokens - 1) * p.k_st + kHeadDim) * 2));
  // This lane's 4 chunks of tile t: LDS slot idx = (wave * 4 + j) * 64 + lane
  // holds chunk (idx & 15) ^ (row & 15) of tile row idx >> 4.
  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    const int kt0 = t * kTileKeys;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = (wave * 4 + j) * 64 + lane;
      const int row = idx >> 4;
      const int c = (idx & 15) ^ (row & 15);
      int key = kt0 + row;
      key = key < ns ? key : ns - 1;
      const uint32_t off = (uint32_t)(
          ((int64_t)sampled_token<S>(key, p.tokens, p.block_size) * p.k_st + c * 8) * 2);
      dsa::lds_load16(k_rsrc, dst + (wave * 4 + j) * 1024, off, 0);
    }
  };

  const int last_block = p.blocks - 1;
  const float c_full = p.logw_full * kLog2e;
  const float c_last = p.logw_last * kLog2e;
  // Tiles before this one hold only full, in-range key blocks.
  const int first_tail_tile = (last_block * S) / kTileKeys;
  float m2 = -INFINITY, l2 = 0.f, lse2 = 0.f;

  auto compute = [&](const unsigned char* lds_k, int t, int sweep) __attribute__((always_inline)) {
    const int kt0 = t * kTileKeys;
    const bool tail = t >= first_tail_tile;
#pragma unroll
    for (int sub = 0; sub < kTileKeys / 32; ++sub) {
      dsa_f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int dc = 0; dc < 8; ++dc) {
        const int key = sub * 32 + qi;
        const int c = dc * 2 + g;
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            lds_k + key * 256 + ((c ^ (key & 15)) << 4));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[dc], acc, 0, 0, 0);
      }
      // Score = bf16(bf16(q.k) * scale), as a bf16 matmul and a bf16 scale
      // multiply; the softmax input in log2 units is score * log2e + c with
      // c = log(block size / S) * log2e.
      float sc[16], cw[16];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float a0, a1;
        round_bf16_pair(acc[r], acc[r + 1], a0, a1);
        round_bf16_pair(a0 * p.scale, a1 * p.scale, sc[r], sc[r + 1]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) cw[r] = c_full;
      if (tail) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = kt0 + sub * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          cw[r] = j / S == last_block ? c_last : c_full;
          if (j >= ns) sc[r] = -INFINITY;
        }
      }
      if (sweep == 0) {
        // Running max of x = score * log2e + c (log2e > 0: c_last differs
        // from c_full only in the tail).
        float mx = m2;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaf(sc[r], kLog2e, cw[r]));
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sum += __builtin_amdgcn_exp2f(fmaf(sc[r], kLog2e, cw[r] - mx));
        l2 = l2 * __builtin_amdgcn_exp2f(m2 - mx) + sum;
        m2 = mx;
      } else {
        float pk[KBS];
#pragma unroll
        for (int b = 0; b < KBS; ++b) pk[b] = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int local = 8 * (r >> 2) + 4 * g + (r & 3);
          pk[local / S] += __builtin_amdgcn_exp2f(fmaf(sc[r], kLog2e, cw[r] - lse2));
        }
        // Sum over the S query lanes of each query block and both halves.
#pragma unroll
        for (int b = 0; b < KBS; ++b) {
#pragma unroll
          for (int m = 1; m < S; m <<= 1) pk[b] += __shfl_xor(pk[b], m);
          pk[b] += __shfl_xor(pk[b], 32);
        }
        if (g == 0 && (qi % S) == 0) {
          const int qs_first = q0 + qi;
          if (qs_first < ns) {
            const int qb = qs_first / S;
            float* out = p.mass + ((int64_t)h * p.blocks + qb) * p.blocks;
#pragma unroll
            for (int b = 0; b < KBS; ++b) {
              const int kb = (kt0 + sub * 32) / S + b;
              if (kb < p.blocks) out[kb] = pk[b] * (1.0f / S);
            }
          }
        }
      }
    }
  };

  // Step: wait for the current tile (and every older memory operation),
  // barrier (all waves' loads landed; every wave done with the other stage),
  // prefetch the next tile into the other stage, compute the current one.
  auto step = [&](int t, int sweep, int next_t, const unsigned char* cur,
                  unsigned char* nxt) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (next_t >= 0) issue(next_t, nxt);
    compute(cur, t, sweep);
  };

  for (int sweep = 0; sweep < 2; ++sweep) {
    issue(0, st0);
    for (int t = 0; t < tiles; t += 2) {
      step(t, sweep, t + 1 < tiles ? t + 1 : -1, st0, st1);
      if (t + 1 >= tiles) break;
      step(t + 1, sweep, t + 2 < tiles ? t + 2 : -1, st1, st0);
    }
    if (sweep == 0) {  // each query's log-sum-exp (log2 units)
      // Lanes l and l ^ 32 hold the two halves of one query's keys; both get
      // the same total (the pair's two terms in one fixed order, so a
      // contracted fma rounds alike in both lanes).
      const auto ms = __builtin_amdgcn_permlane32_swap(__float_as_uint(m2), __float_as_uint(m2),
                                                       false, false);
      const auto ls = __builtin_amdgcn_permlane32_swap(__float_as_uint(l2), __float_as_uint(l2),
                                                       false, false);
      const float ma = __uint_as_float(ms[0]), mb = __uint_as_float(ms[1]);
      const float mx = fmaxf(ma, mb);
      const float tot = __uint_as_float(ls[0]) * __builtin_amdgcn_exp2f(ma - mx) +
                        __uint_as_float(ls[1]) * __builtin_amdgcn_exp2f(mb - mx);
      lse2 = mx + __builtin_log2f(tot);
      __syncthreads();  // every wave done with st0/st1 before sweep 2 refills st0
    }
  }
}

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
  if (p.previous) {
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) s += to_fixed(v[j]);
    s = wave_sum_i64(s);
    const float mean = fixed_to_f32(s) / (float)K;
    const float prior = p.rho * mean;
    const uint8_t* prow = p.previous + (int64_t)row * K;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = lane * kPer + j;
      if (e < K && prow[e]) v[j] = v[j] + prior;
    }
  }
  int64_t total = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) total += to_fixed(v[j]);
  total = wave_sum_i64(total);
  const float threshold = fixed_to_f32(total) * p.target;

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
    run += to_fixed(__uint_as_float((uint32_t)(key[j] >> 32)));
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
    if (e < K && fixed_to_f32(pre[j] + offset) < threshold) ++below;
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

extern "C" int dsa_sampled_mass(const void* q, const void* k, const int64_t* strides,
                                int32_t tokens, int32_t heads, int32_t head_dim,
                                int32_t block_size, int32_t samples, float scale, float* mass,
                                hipStream_t stream) {
  dsa::clear_error();
  if (!q || !k || !mass || !strides)
    return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: null pointer");
  if (tokens <= 0 || heads <= 0 || block_size <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: tokens/heads/block must be positive");
  if (head_dim != kHeadDim)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_sampled_mass: head_dim %d unsupported (128)",
                          head_dim);
  if (samples <= 0 || samples > block_size)
    return dsa::set_error(DSA_EINVAL, "route_samples must be in [1, block_size]");
  if (samples > 32 || (samples & (samples - 1)) != 0)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_sampled_mass: samples must be a power of two <= 32 (got %d)",
                          samples);
  if (!(scale > 0.f)) return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: scale must be > 0");
  if (!aligned16(q) || !aligned16(k))
    return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: q/k must be 16-byte aligned");
  for (int i = 0; i < 4; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return dsa::set_error(DSA_EINVAL,
                            "dsa_sampled_mass: stride %d not a non-negative multiple of 8", i);
  if (((int64_t)(tokens - 1) * strides[2] + kHeadDim) * 2 > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_sampled_mass: one head's K rows must span < 2 GiB");
  MassParams p;
  p.q = static_cast<const __bf16*>(q);
  p.k = static_cast<const __bf16*>(k);
  p.mass = mass;
  p.q_st = strides[0]; p.q_sh = strides[1]; p.k_st = strides[2]; p.k_sh = strides[3];
  p.tokens = tokens;
  p.heads = heads;
  p.block_size = block_size;
  p.blocks = (tokens + block_size - 1) / block_size;
  p.scale = scale;
  // fp32 log of an fp32 quotient, as torch's (sizes.float() / samples).log().
  const int last = tokens - (p.blocks - 1) * block_size;
  p.logw_full = logf((float)block_size / (float)samples);
  p.logw_last = logf((float)last / (float)samples);
  const int ns = p.blocks * samples;
  const dim3 grid((unsigned)((ns + 127) / 128), (unsigned)heads);
  switch (samples) {
    case 1: hipLaunchKernelGGL(sampled_mass_kernel<1>, grid, dim3(256), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(sampled_mass_kernel<2>, grid, dim3(256), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(sampled_mass_kernel<4>, grid, dim3(256), 0, stream, p); break;
    case 8: hipLaunchKernelGGL(sampled_mass_kernel<8>, grid, dim3(256), 0, stream, p); break;
    case 16: hipLaunchKernelGGL(sampled_mass_kernel<16>, grid, dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL(sampled_mass_kernel<32>, grid, dim3(256), 0, stream, p); break;
  }
  return dsa::check_launch("dsa_sampled_mass");
}

extern "C" int dsa_route_select(const float* mass, const uint8_t* previous, int32_t rows,
                                int32_t keys, float rho, float target, int32_t cap,
                                int32_t sink_blocks, uint8_t* route, int32_t* counts,
                                hipStream_t stream) {
  dsa::clear_error();
  if (!mass || !route || !counts) return dsa::set_error(DSA_EINVAL, "dsa_route_select: null pointer");
  if (rows <= 0 || keys <= 0) return dsa::set_error(DSA_EINVAL, "dsa_route_select: empty route");
  if (keys > 2048)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_route_select: at most 2048 key blocks (got %d)",
                          keys);
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
  else
    hipLaunchKernelGGL(route_select_kernel<32>, groups, threads, 0, stream, p);
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
