// Block-sparse attention forward for gfx950 (MI355X), bf16 in/out, fp32 softmax.
//
// Replaces the FlexAttention call of the reference backend
// (attention_backends/flex.py:379-399 `_flex_output`, kernel options
// flex.py:360-364) and its dense SDPA fallback (attention_backends/dense.py:14-48).
//
// Semantics per (batch b, head h, query row t):
//   O[b,t,h,:] = softmax_k( scale * <Q[b,t,h,:], K[b,k,h,:]> ) @ V[b,k,h,:]
// where k ranges over the tokens of every key block listed in the CSR row of
// (route batch, h, t / BLOCK).  Without a CSR every key block is listed (dense
// fallback).  Keys past `kv_tokens` in a partial last block are masked.
//
// Work decomposition: one workgroup (4 wave64s) per (b, h, query block of 128
// rows); wave w owns query rows 32w..32w+31, one row per lane pair (l, l^32).
// S^T = K Q^T is computed with v_mfma_f32_32x32x16_bf16 so that each lane's
// accumulators belong to a single query row: the online-softmax max/sum stay
// in registers and need one cross-half exchange.  P^T leaves the accumulators
// already in the B-operand layout of O^T = V^T P^T; the V tile is transposed
// into LDS with its keys stored in the matching order.
#include "dsa_common.h"

#include <stdlib.h>

namespace {

struct BsaParams {
  const __bf16* q;
  const __bf16* k;
  const __bf16* v;
  __bf16* o;
  float* lse;
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int64_t o_sb, o_st, o_sh;
  const int32_t* row_ptr;  // null: every key block (dense)
  const int32_t* col_idx;
  int32_t batch, heads, q_tokens, kv_tokens, q_blocks, kv_blocks, route_batches;
  float scale;       // softmax scale applied to <q, k>
  float scale_log2;  // scale * log2(e)
};

constexpr int kHeadDim = 128;
constexpr int kRowBytes = kHeadDim * 2;  // one K row / one V^T row: 256 bytes

// LDS position (16-byte units within a 256-byte row) of K chunk `c` of key row
// `r`.  Rows are XOR-swizzled so 16 consecutive rows read at one chunk hit 16
// distinct bank groups.
__device__ __forceinline__ int k_swz(int r, int c) { return c ^ (r & 15); }

// LDS position of logical key chunk `c` (8 keys) of V^T row `d`.  The second
// term makes the transposing writes (rows 8 apart) conflict-free as well.
__device__ __forceinline__ int v_swz(int d, int c) {
  return c ^ (d & 15) ^ ((d >> 3) & 15);
}

template <int BLOCK>
__global__ void __launch_bounds__(256, 2) bsa_fwd_kernel(BsaParams p) {
  static_assert(BLOCK == 128, "this kernel tiles 128-token blocks");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k[BLOCK * kRowBytes];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v[kHeadDim * BLOCK * 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;   // half-wave: selects the 8-element K-slice
  const int qi = lane & 31;  // MFMA row/column owned by this lane

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;

  int start = 0, end = p.kv_blocks;
  if (p.row_ptr) {
    const int rb = p.route_batches == 1 ? 0 : b;
    const int64_t row = ((int64_t)rb * p.heads + h) * p.q_blocks + qb;
    start = p.row_ptr[row];
    end = p.row_ptr[row + 1];
  }

  // Q^T fragments (B operand of S^T = K Q^T): lane holds 8 consecutive head
  // dims of its query row for each of the 8 K-steps of 16.
  const int tq = qb * BLOCK + wave * 32 + qi;
  const int tq_c = tq < p.q_tokens ? tq : p.q_tokens - 1;
  const __bf16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)tq_c * p.q_st;
  dsa_bf16x8 qf[8];
#pragma unroll
  for (int dc = 0; dc < 8; ++dc)
    qf[dc] = *reinterpret_cast<const dsa_bf16x8*>(qrow + dc * 16 + g * 8);

  const __bf16* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + h * p.v_sh;

  float m_run = -INFINITY;  // running max of raw scores <q,k>
  float l_run = 0.f;        // running sum of this half-wave's probabilities
  dsa_f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;

  for (int it = start; it < end; ++it) {
    const int kb = p.row_ptr ? p.col_idx[it] : it;
    if ((unsigned)kb >= (unsigned)p.kv_blocks) continue;  // malformed index: skip
    const int key0 = kb * BLOCK;

    __syncthreads();  // previous tile fully consumed

    // K tile -> LDS, direct from global (16 B per lane); the source chunk is
    // chosen so that the linear LDS image is the swizzled layout.
#pragma unroll
    for (int j = 0; j < BLOCK * 16 / 256; ++j) {
      const int chunk_base = (wave * (BLOCK * 16 / 256) + j) * 64;
      const int idx = chunk_base + lane;
      const int row = idx >> 4;
      const int c = (idx & 15) ^ (row & 15);
      int key = key0 + row;
      key = key < p.kv_tokens ? key : p.kv_tokens - 1;
      const __bf16* src = kbase + (int64_t)key * p.k_st + c * 8;
      __builtin_amdgcn_global_load_lds(
          src, (DSA_LDS void*)(lds_k + chunk_base * 16), 16, 0, 0);
    }

    // V tile -> registers -> transposed V^T in LDS.  Thread (kg, c) owns head
    // dims 8c..8c+7 of the 8 keys that form logical key chunk kg.
    {
      const int kg = tid >> 4;
      const int c = tid & 15;
      const int grp = kg >> 1, half = kg & 1;
      dsa_u32x4 vr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int key = key0 + grp * 16 + 4 * half + (i & 3) + 8 * (i >> 2);
        key = key < p.kv_tokens ? key : p.kv_tokens - 1;
        vr[i] = *reinterpret_cast<const dsa_u32x4*>(vbase + (int64_t)key * p.v_st + c * 8);
      }
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) {
        dsa_u32x4 out;
        const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int w = 0; w < 4; ++w)
          out[w] = __builtin_amdgcn_perm(vr[2 * w + 1][dd >> 1], vr[2 * w][dd >> 1], sel);
        const int d = c * 8 + dd;
        *reinterpret_cast<dsa_u32x4*>(lds_v + d * (BLOCK * 2) + v_swz(d, kg) * 16) = out;
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // S^T = K Q^T: 4 sub-tiles of 32 keys x 32 query rows.
    dsa_f32x16 sacc[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int key = kt * 32 + qi;
        const int c = dc * 2 + g;
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            lds_k + key * kRowBytes + k_swz(key, c) * 16);
        sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[dc], sacc[kt], 0, 0, 0);
      }
    }

    // Accumulator (kt, r) holds key kt*32 + 8*(r/4) + 4*g + r%4.
    if (key0 + BLOCK > p.kv_tokens) {
      const int valid = p.kv_tokens - key0;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= valid) sacc[kt][r] = -INFINITY;
        }
    }

    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * p.scale_log2);
    const float mb = m_use * p.scale_log2;

    float rs = 0.f;
    dsa_bf16x8 pf[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kt = j >> 1, hf = j & 1;
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t], p.scale_log2, -mb));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t + 1], p.scale_log2, -mb));
        rs += p0 + p1;
        const dsa_f32x2 two = {p0, p1};
        const dsa_bf16x2 pb = __builtin_convertvector(two, dsa_bf16x2);
        pf[j][t] = pb[0];
        pf[j][t + 1] = pb[1];
      }
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;

    // O^T += V^T P^T over 8 K-steps of 16 keys.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int d = dt * 32 + qi;
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            lds_v + d * (BLOCK * 2) + v_swz(d, 2 * j + g) * 16);
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[j], oacc[dt], 0, 0, 0);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (tq < p.q_tokens) {
    __bf16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const dsa_f32x2 lo = {oacc[dt][rr * 4 + 0] * inv, oacc[dt][rr * 4 + 1] * inv};
        const dsa_f32x2 hi = {oacc[dt][rr * 4 + 2] * inv, oacc[dt][rr * 4 + 3] * inv};
        const dsa_bf16x2 blo = __builtin_convertvector(lo, dsa_bf16x2);
        const dsa_bf16x2 bhi = __builtin_convertvector(hi, dsa_bf16x2);
        const dsa_bf16x4 v4 = {blo[0], blo[1], bhi[0], bhi[1]};
        *reinterpret_cast<dsa_bf16x4*>(orow + dt * 32 + rr * 8 + g * 4) = v4;
      }
    if (p.lse && g == 0) {
      p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
          l_tot > 0.f ? m_run * p.scale + logf(l_tot) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined variant: 4 waves x 32 query rows per 128-row block (2 blocks per
// CU), keys streamed as 64-key half-tiles one step ahead of the compute: K by
// direct global->LDS loads into a double buffer, V through registers into a
// double-buffered transposed V^T.  One barrier per half-tile; lazy softmax
// rescaling; row sums from the bf16 probabilities with dot2.
// ---------------------------------------------------------------------------

constexpr int kHalfKeys = 64;
constexpr int kKStage = kHalfKeys * kRowBytes;    // 16 KB: [64 keys][128 dims]
constexpr int kVtRow = kHalfKeys * 2;             // 128 B: one head dim, 64 keys
constexpr int kVStage = kHeadDim * kVtRow;        // 16 KB: [128 dims][64 keys]
constexpr float kRescaleLog2 = 8.0f;              // rescale once p could exceed 2^8

// V^T half-tile: row = head dim (128 B, 8 chunks of 8 logical keys).  Even and
// odd rows sit in different bank halves; XOR ((d >> 1) ^ (d >> 4)) & 7 makes
// the 16 rows of a fragment read distinct and halves transposing-write clashes.
__device__ __forceinline__ int vt_swz(int d, int c) { return c ^ (((d >> 1) ^ (d >> 4)) & 7); }

__global__ void __launch_bounds__(256, 2) bsa_fwd3_kernel(BsaParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k[2 * kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v[2 * kVStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 5;
  const int qi = lane & 31;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;

  int start = 0, end = p.kv_blocks;
  if (p.row_ptr) {
    const int rb = p.route_batches == 1 ? 0 : b;
    const int64_t row = ((int64_t)rb * p.heads + h) * p.q_blocks + qb;
    start = p.row_ptr[row];
    end = p.row_ptr[row + 1];
  }
  const int nsub = 2 * (end - start);

  const int tq = qb * 128 + wave * 32 + qi;
  const int tq_c = tq < p.q_tokens ? tq : p.q_tokens - 1;
  const __bf16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)tq_c * p.q_st;
  dsa_bf16x8 qf[8];
#pragma unroll
  for (int dc = 0; dc < 8; ++dc)
    qf[dc] = *reinterpret_cast<const dsa_bf16x8*>(qrow + dc * 16 + g * 8);

  const __bf16* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + h * p.v_sh;

  // Key block of half-tile `sub`, or -1 when the CSR entry is out of range.
  auto block_of = [&](int sub) -> int {
    const int it = start + (sub >> 1);
    const int kb = p.row_ptr ? p.col_idx[it] : it;
    return (unsigned)kb < (unsigned)p.kv_blocks ? kb : -1;
  };
  auto first_key = [&](int sub) -> int {
    const int kb = block_of(sub);
    return (kb < 0 ? 0 : kb) * 128 + (sub & 1) * kHalfKeys;
  };

  // V transposition duty: keys 4*vq..4*vq+3 of the half-tile, head dims 8*vc..8*vc+7.
  const int vq = tid >> 4;
  const int vc = tid & 15;
  dsa_u32x4 vr[4];

  auto issue = [&](int sub, int stage) {
    const int key0 = first_key(sub);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int chunk_base = (wave * 4 + j) * 64;
      const int idx = chunk_base + lane;
      const int row = idx >> 4;
      int key = key0 + row;
      key = key < p.kv_tokens ? key : p.kv_tokens - 1;
      const __bf16* src = kbase + (int64_t)key * p.k_st + k_swz(row, idx & 15) * 8;
      __builtin_amdgcn_global_load_lds(
          src, (DSA_LDS void*)(lds_k + stage * kKStage + chunk_base * 16), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int key = key0 + vq * 4 + i;
      key = key < p.kv_tokens ? key : p.kv_tokens - 1;
      vr[i] = *reinterpret_cast<const dsa_u32x4*>(vbase + (int64_t)key * p.v_st + vc * 8);
    }
  };

  // Logical key order inside each 16-key group swaps the two middle quads, so
  // that V^T chunk (2j + g) holds exactly the keys of the P^T B-operand slots.
  const int quad = vq & 3;
  const int lkey = (vq >> 2) * 16 + (((quad & 1) << 1) | (quad >> 1)) * 4;
  auto store_vt = [&](int stage) {
    unsigned char* base = lds_v + stage * kVStage;
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
      dsa_u32x2 out;
      out[0] = __builtin_amdgcn_perm(vr[1][dd >> 1], vr[0][dd >> 1], sel);
      out[1] = __builtin_amdgcn_perm(vr[3][dd >> 1], vr[2][dd >> 1], sel);
      const int d = vc * 8 + dd;
      *reinterpret_cast<dsa_u32x2*>(base + d * kVtRow + vt_swz(d, lkey >> 3) * 16 +
                                    (lkey & 7) * 2) = out;
    }
  };

  float m_run = -INFINITY;  // reference max, log2-scaled units
  float l_run = 0.f;        // this half-wave's partial row sum
  dsa_f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  const dsa_bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

  if (nsub > 0) issue(0, 0);
  for (int sub = 0; sub < nsub; ++sub) {
    const int stage = sub & 1;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K stage and V registers landed
    store_vt(stage);
    __syncthreads();  // stage visible to all waves; the other stage is free
    if (sub + 1 < nsub) issue(sub + 1, stage ^ 1);

    const unsigned char* kt_lds = lds_k + stage * kKStage;
    const unsigned char* vt_lds = lds_v + stage * kVStage;
    const int kb = block_of(sub);
    const int key0 = first_key(sub);
    int valid = kb < 0 ? 0 : p.kv_tokens - key0;
    valid = valid < kHalfKeys ? valid : kHalfKeys;

    dsa_f32x16 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int row = kt * 32 + qi;
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            kt_lds + row * kRowBytes + k_swz(row, dc * 2 + g) * 16);
        sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[dc], sacc[kt], 0, 0, 0);
      }
    }
    if (valid < kHalfKeys) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= valid) sacc[kt][r] = -INFINITY;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mx2 = mx * p.scale_log2;
    const bool up = mx2 > m_run + kRescaleLog2;
    if (__any(up)) {
      const float alpha = up ? __builtin_amdgcn_exp2f(m_run - mx2) : 1.0f;
      m_run = up ? mx2 : m_run;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;

    dsa_bf16x8 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kt = j >> 1, hf = j & 1;
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const float p0 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t], p.scale_log2, -m_use));
        const float p1 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t + 1], p.scale_log2, -m_use));
        const dsa_f32x2 two = {p0, p1};
        const dsa_bf16x2 pb = __builtin_convertvector(two, dsa_bf16x2);
        l_run = __builtin_amdgcn_fdot2_f32_bf16(pb, ones, l_run, false);
        pf[j][t] = pb[0];
        pf[j][t + 1] = pb[1];
      }
    }

#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int d = dt * 32 + qi;
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            vt_lds + d * kVtRow + vt_swz(d, 2 * j + g) * 16);
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[j], oacc[dt], 0, 0, 0);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (tq < p.q_tokens) {
    __bf16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const dsa_f32x2 lo = {oacc[dt][rr * 4 + 0] * inv, oacc[dt][rr * 4 + 1] * inv};
        const dsa_f32x2 hi = {oacc[dt][rr * 4 + 2] * inv, oacc[dt][rr * 4 + 3] * inv};
        const dsa_bf16x2 blo = __builtin_convertvector(lo, dsa_bf16x2);
        const dsa_bf16x2 bhi = __builtin_convertvector(hi, dsa_bf16x2);
        const dsa_bf16x4 v4 = {blo[0], blo[1], bhi[0], bhi[1]};
        *reinterpret_cast<dsa_bf16x4*>(orow + dt * 32 + rr * 8 + g * 4) = v4;
      }
    if (p.lse && g == 0) {
      // m_run is in log2 units of scaled scores: lse = ln2 * m + ln(l).
      p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
          l_tot > 0.f ? m_run * 0.6931471805599453f + logf(l_tot) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// v4: the v3 pipeline with uniform block indices read through scalar loads
// (so waiting on them never drains the prefetch), per-lane load offsets
// computed once, operand fragments staged in double-buffered groups of four,
// and V^T rows placed so that the transposing writes use both bank halves.
// ---------------------------------------------------------------------------

typedef const __attribute__((address_space(4))) int32_t* dsa_const_i32;

// Physical V^T row of head dim d: rows d and d^1 swap when bit 3 of d is set,
// so the 16 rows (8 apart) written by one transposing store straddle both
// 128-byte bank halves.
__device__ __forceinline__ int vt_row(int d) { return d ^ ((d >> 3) & 1); }

__global__ void __launch_bounds__(256, 2) bsa_fwd4_kernel(BsaParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k[2 * kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v[2 * kVStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;

  int start = 0, end = p.kv_blocks;
  if (p.row_ptr) {
    const dsa_const_i32 rp = (dsa_const_i32)p.row_ptr;
    const int rb = p.route_batches == 1 ? 0 : b;
    const int64_t row = ((int64_t)rb * p.heads + h) * p.q_blocks + qb;
    start = rp[row];
    end = rp[row + 1];
  }
  const dsa_const_i32 cidx = (dsa_const_i32)p.col_idx;
  const int nsub = 2 * (end - start);

  const int tq = qb * 128 + wave * 32 + qi;
  const int tq_c = tq < p.q_tokens ? tq : p.q_tokens - 1;
  const __bf16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)tq_c * p.q_st;
  dsa_bf16x8 qf[8];
#pragma unroll
  for (int dc = 0; dc < 8; ++dc)
    qf[dc] = *reinterpret_cast<const dsa_bf16x8*>(qrow + dc * 16 + g * 8);

  const __bf16* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + h * p.v_sh;

  // Per-lane element offsets inside one half-tile (rows relative to its first key).
  int krow[4], koff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = (wave * 4 + j) * 64 + lane;
    krow[j] = idx >> 4;
    koff[j] = krow[j] * (int)p.k_st + k_swz(krow[j], idx & 15) * 8;
  }
  const int vq = tid >> 4;
  const int vc = tid & 15;
  int voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) voff[i] = (vq * 4 + i) * (int)p.v_st + vc * 8;

  auto block_of = [&](int sub) -> int {
    const int it = start + (sub >> 1);
    const int kb = p.row_ptr ? cidx[it] : it;
    return (unsigned)kb < (unsigned)p.kv_blocks ? kb : -1;
  };

  dsa_u32x4 vr[4];
  auto issue = [&](int key0, int stage) {
    const __bf16* ktile = kbase + (int64_t)key0 * p.k_st;
    const __bf16* vtile = vbase + (int64_t)key0 * p.v_st;
    unsigned char* kdst = lds_k + stage * kKStage + wave * 4 * 1024;
    if (key0 + kHalfKeys <= p.kv_tokens) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_global_load_lds(ktile + koff[j], (DSA_LDS void*)(kdst + j * 1024), 16,
                                         0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vr[i] = *reinterpret_cast<const dsa_u32x4*>(vtile + voff[i]);
    } else {
      // Partial last block: clamp rows to the last token.
      const int last = p.kv_tokens - 1 - key0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int idx = (wave * 4 + j) * 64 + lane;
        const int r = krow[j] < last ? krow[j] : last;
        __builtin_amdgcn_global_load_lds(ktile + (int64_t)r * p.k_st + k_swz(krow[j], idx & 15) * 8,
                                         (DSA_LDS void*)(kdst + j * 1024), 16, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = vq * 4 + i < last ? vq * 4 + i : last;
        vr[i] = *reinterpret_cast<const dsa_u32x4*>(vtile + (int64_t)r * p.v_st + vc * 8);
      }
    }
  };

  const int quad = vq & 3;
  const int lkey = (vq >> 2) * 16 + (((quad & 1) << 1) | (quad >> 1)) * 4;
  auto store_vt = [&](int stage) {
    unsigned char* base = lds_v + stage * kVStage;
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
      dsa_u32x2 out;
      out[0] = __builtin_amdgcn_perm(vr[1][dd >> 1], vr[0][dd >> 1], sel);
      out[1] = __builtin_amdgcn_perm(vr[3][dd >> 1], vr[2][dd >> 1], sel);
      const int d = vc * 8 + dd;
      *reinterpret_cast<dsa_u32x2*>(base + vt_row(d) * kVtRow + vt_swz(d, lkey >> 3) * 16 +
                                    (lkey & 7) * 2) = out;
    }
  };

  float m_run = -INFINITY;
  float l_run = 0.f;
  dsa_f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  const dsa_bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

  int kb_cur = nsub > 0 ? block_of(0) : -1;
  if (nsub > 0) issue((kb_cur < 0 ? 0 : kb_cur) * 128, 0);
  for (int sub = 0; sub < nsub; ++sub) {
    const int stage = sub & 1;
    const int kb_next = (sub + 1 < nsub) ? ((sub & 1) ? block_of(sub + 1) : kb_cur) : -1;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this half-tile's K stage and V registers
    store_vt(stage);
    __syncthreads();
    if (sub + 1 < nsub)
      issue((kb_next < 0 ? 0 : kb_next) * 128 + ((sub + 1) & 1) * kHalfKeys, stage ^ 1);

    const unsigned char* kt_lds = lds_k + stage * kKStage;
    const unsigned char* vt_lds = lds_v + stage * kVStage;
    const int key0 = (kb_cur < 0 ? 0 : kb_cur) * 128 + (sub & 1) * kHalfKeys;
    int valid = kb_cur < 0 ? 0 : p.kv_tokens - key0;
    valid = valid < kHalfKeys ? valid : kHalfKeys;

    // S^T = K Q^T: 16 MFMAs, fragments staged four at a time.
    dsa_f32x16 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
    {
      dsa_bf16x8 fa[4], fb[4];
      auto load_k = [&](dsa_bf16x8* dst, int grp) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int step = grp * 4 + u;  // step = dc * 2 + kt
          const int kt = step & 1, dc = step >> 1;
          const int row = kt * 32 + qi;
          dst[u] = *reinterpret_cast<const dsa_bf16x8*>(
              kt_lds + row * kRowBytes + k_swz(row, dc * 2 + g) * 16);
        }
      };
      auto mfma_k = [&](const dsa_bf16x8* src, int grp) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int step = grp * 4 + u;
          const int kt = step & 1, dc = step >> 1;
          sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(src[u], qf[dc], sacc[kt], 0, 0, 0);
        }
      };
      load_k(fa, 0);
      load_k(fb, 1);
      mfma_k(fa, 0);
      load_k(fa, 2);
      mfma_k(fb, 1);
      load_k(fb, 3);
      mfma_k(fa, 2);
      mfma_k(fb, 3);
    }
    if (valid < kHalfKeys) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= valid) sacc[kt][r] = -INFINITY;
    }

    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mx2 = mx * p.scale_log2;
    const bool up = mx2 > m_run + kRescaleLog2;
    if (__any(up)) {
      const float alpha = up ? __builtin_amdgcn_exp2f(m_run - mx2) : 1.0f;
      m_run = up ? mx2 : m_run;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;

    dsa_bf16x8 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kt = j >> 1, hf = j & 1;
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const float p0 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t], p.scale_log2, -m_use));
        const float p1 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t + 1], p.scale_log2, -m_use));
        const dsa_f32x2 two = {p0, p1};
        const dsa_bf16x2 pb = __builtin_convertvector(two, dsa_bf16x2);
        l_run = __builtin_amdgcn_fdot2_f32_bf16(pb, ones, l_run, false);
        pf[j][t] = pb[0];
        pf[j][t + 1] = pb[1];
      }
    }

    // O^T += V^T P^T: 16 MFMAs, fragments staged four at a time.
    {
      dsa_bf16x8 fa[4], fb[4];
      auto load_v = [&](dsa_bf16x8* dst, int grp) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int step = grp * 4 + u;  // step = j * 4 + dt
          const int j = step >> 2, dt = step & 3;
          const int d = dt * 32 + qi;
          dst[u] = *reinterpret_cast<const dsa_bf16x8*>(
              vt_lds + vt_row(d) * kVtRow + vt_swz(d, 2 * j + g) * 16);
        }
      };
      auto mfma_v = [&](const dsa_bf16x8* src, int grp) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int step = grp * 4 + u;
          const int j = step >> 2, dt = step & 3;
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(src[u], pf[j], oacc[dt], 0, 0, 0);
        }
      };
      load_v(fa, 0);
      load_v(fb, 1);
      mfma_v(fa, 0);
      load_v(fa, 2);
      mfma_v(fb, 1);
      load_v(fb, 3);
      mfma_v(fa, 2);
      mfma_v(fb, 3);
    }
    if (sub & 1) kb_cur = kb_next;
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (tq < p.q_tokens) {
    __bf16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const dsa_f32x2 lo = {oacc[dt][rr * 4 + 0] * inv, oacc[dt][rr * 4 + 1] * inv};
        const dsa_f32x2 hi = {oacc[dt][rr * 4 + 2] * inv, oacc[dt][rr * 4 + 3] * inv};
        const dsa_bf16x2 blo = __builtin_convertvector(lo, dsa_bf16x2);
        const dsa_bf16x2 bhi = __builtin_convertvector(hi, dsa_bf16x2);
        const dsa_bf16x4 v4 = {blo[0], blo[1], bhi[0], bhi[1]};
        *reinterpret_cast<dsa_bf16x4*>(orow + dt * 32 + rr * 8 + g * 4) = v4;
      }
    if (p.lse && g == 0) {
      p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
          l_tot > 0.f ? m_run * 0.6931471805599453f + logf(l_tot) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// v5: K and V half-tiles both staged by direct global->LDS loads into
// double buffers that are distinct LDS objects (the loop is unrolled by two so
// each stage is a compile-time buffer and reads of one stage carry no wait on
// the DMA into the other); V^T fragments come from the transposing LDS load.
// ---------------------------------------------------------------------------

// K stage [64 keys][128 dims]: 16-byte chunk XOR (row & 15), so the 32 rows a
// b128 fragment load reads at one chunk hit distinct banks.
__device__ __forceinline__ int k2_swz(int r, int c) { return c ^ (r & 15); }
// V stage [64 keys][128 dims]: chunk XOR ((row & 3) << 2); a transposing load
// reads 4 consecutive rows x 32 bytes per 16 lanes, which this spreads over
// all banks.
__device__ __forceinline__ int v2_swz(int r, int c) { return c ^ ((r & 3) << 2); }

typedef short dsa_s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, lane i returns element (i % 4)
// of the 64-bit rows read by lanes i/4 + 4*jj, jj = 0..3.
__device__ __forceinline__ dsa_u32x2 lds_read_tr16(const unsigned char* addr) {
  const dsa_s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((DSA_LDS dsa_s16x4*)(addr));
  return __builtin_bit_cast(dsa_u32x2, v);
}

__device__ __forceinline__ dsa_bf16x8 read_vt_fragment(const unsigned char* vt, int j, int dt,
                                                       int g, int grp, int gi) {
  // Lane i of 16-lane group grp reads 4 consecutive head dims of one key row;
  // the transposing load hands each lane 4 keys of one head dim.
  const int d0 = dt * 32 + 16 * (grp & 1) + 4 * (gi & 3);
  const int chunk = d0 >> 3;
  const int within = (d0 & 7) * 2;
  dsa_u32x4 a32;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = 16 * j + 8 * t + 4 * g + (gi >> 2);
    const dsa_u32x2 part = lds_read_tr16(vt + row * kRowBytes + v2_swz(row, chunk) * 16 + within);
    a32[2 * t] = part[0];
    a32[2 * t + 1] = part[1];
  }
  return __builtin_bit_cast(dsa_bf16x8, a32);
}

__global__ void __launch_bounds__(256, 2) bsa_fwd5_kernel(BsaParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k1[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v1[kKStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;
  const int grp = lane >> 4;
  const int gi = lane & 15;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;

  int start = 0, end = p.kv_blocks;
  if (p.row_ptr) {
    const dsa_const_i32 rp = (dsa_const_i32)p.row_ptr;
    const int rb = p.route_batches == 1 ? 0 : b;
    const int64_t row = ((int64_t)rb * p.heads + h) * p.q_blocks + qb;
    start = rp[row];
    end = rp[row + 1];
  }
  const dsa_const_i32 cidx = (dsa_const_i32)p.col_idx;
  const int nsub = 2 * (end - start);

  const int tq = qb * 128 + wave * 32 + qi;
  const int tq_c = tq < p.q_tokens ? tq : p.q_tokens - 1;
  const __bf16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)tq_c * p.q_st;
  dsa_bf16x8 qf[8];
#pragma unroll
  for (int dc = 0; dc < 8; ++dc)
    qf[dc] = *reinterpret_cast<const dsa_bf16x8*>(qrow + dc * 16 + g * 8);

  const __bf16* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const __bf16* vbase = p.v + b * p.v_sb + h * p.v_sh;

  // Rows (relative to the half-tile's first key) and 16-byte source chunks
  // this lane stages; the linear LDS image is the swizzled layout.
  int lrow[4], kchunk[4], vchunk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int idx = (wave * 4 + j) * 64 + lane;
    lrow[j] = idx >> 4;
    kchunk[j] = k2_swz(lrow[j], idx & 15);
    vchunk[j] = v2_swz(lrow[j], idx & 15);
  }

  auto block_of = [&](int sub) -> int {
    const int it = start + (sub >> 1);
    const int kb = p.row_ptr ? cidx[it] : it;
    return (unsigned)kb < (unsigned)p.kv_blocks ? kb : -1;
  };

  auto issue = [&](int key0, unsigned char* kdst, unsigned char* vdst) {
    int last = p.kv_tokens - 1 - key0;  // rows past the sequence end are clamped
    last = last < kHalfKeys - 1 ? last : kHalfKeys - 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = lrow[j] < last ? lrow[j] : last;
      const int64_t key = key0 + r;
      __builtin_amdgcn_global_load_lds(kbase + key * p.k_st + kchunk[j] * 8,
                                       (DSA_LDS void*)(kdst + (wave * 4 + j) * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vbase + key * p.v_st + vchunk[j] * 8,
                                       (DSA_LDS void*)(vdst + (wave * 4 + j) * 1024), 16, 0, 0);
    }
  };

  float m_run = -INFINITY;
  float l_run = 0.f;
  dsa_f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  const dsa_bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

  auto compute = [&](const unsigned char* kt_lds, const unsigned char* vt_lds, int valid) {
    dsa_f32x16 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int row = kt * 32 + qi;
        const dsa_bf16x8 a = *reinterpret_cast<const dsa_bf16x8*>(
            kt_lds + row * kRowBytes + k2_swz(row, dc * 2 + g) * 16);
        sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[dc], sacc[kt], 0, 0, 0);
      }
    }
    if (valid < kHalfKeys) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= valid) sacc[kt][r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mx2 = mx * p.scale_log2;
    const bool up = mx2 > m_run + kRescaleLog2;
    if (__any(up)) {
      const float alpha = up ? __builtin_amdgcn_exp2f(m_run - mx2) : 1.0f;
      m_run = up ? mx2 : m_run;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    dsa_bf16x8 pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kt = j >> 1, hf = j & 1;
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const float p0 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t], p.scale_log2, -m_use));
        const float p1 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t + 1], p.scale_log2, -m_use));
        const dsa_f32x2 two = {p0, p1};
        const dsa_bf16x2 pb = __builtin_convertvector(two, dsa_bf16x2);
        l_run = __builtin_amdgcn_fdot2_f32_bf16(pb, ones, l_run, false);
        pf[j][t] = pb[0];
        pf[j][t + 1] = pb[1];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const dsa_bf16x8 a = read_vt_fragment(vt_lds, j, dt, g, grp, gi);
        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[j], oacc[dt], 0, 0, 0);
      }
    }
  };

  // One half-tile step: wait for this stage, release the other one, prefetch
  // the next half-tile into it, compute this one.
  auto step = [&](int sub, int kb, int kb_next, const unsigned char* kc, const unsigned char* vc,
                  unsigned char* kn, unsigned char* vn) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (sub + 1 < nsub)
      issue((kb_next < 0 ? 0 : kb_next) * 128 + ((sub + 1) & 1) * kHalfKeys, kn, vn);
    const int key0 = (kb < 0 ? 0 : kb) * 128 + (sub & 1) * kHalfKeys;
    int valid = kb < 0 ? 0 : p.kv_tokens - key0;
    valid = valid < kHalfKeys ? valid : kHalfKeys;
    compute(kc, vc, valid);
  };

  if (nsub > 0) {
    int kb = block_of(0);
    issue((kb < 0 ? 0 : kb) * 128, lds_k0, lds_v0);
    for (int sub = 0; sub < nsub; sub += 2) {
      // Even half-tile (stage 0) and odd half-tile (stage 1) of key block kb.
      const int kb_after = (sub + 2 < nsub) ? block_of(sub + 2) : -1;
      step(sub, kb, kb, lds_k0, lds_v0, lds_k1, lds_v1);
      step(sub + 1, kb, kb_after, lds_k1, lds_v1, lds_k0, lds_v0);
      kb = kb_after;
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (tq < p.q_tokens) {
    __bf16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const dsa_f32x2 lo = {oacc[dt][rr * 4 + 0] * inv, oacc[dt][rr * 4 + 1] * inv};
        const dsa_f32x2 hi = {oacc[dt][rr * 4 + 2] * inv, oacc[dt][rr * 4 + 3] * inv};
        const dsa_bf16x2 blo = __builtin_convertvector(lo, dsa_bf16x2);
        const dsa_bf16x2 bhi = __builtin_convertvector(hi, dsa_bf16x2);
        const dsa_bf16x4 v4 = {blo[0], blo[1], bhi[0], bhi[1]};
        *reinterpret_cast<dsa_bf16x4*>(orow + dt * 32 + rr * 8 + g * 4) = v4;
      }
    if (p.lse && g == 0) {
      p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
          l_tot > 0.f ? m_run * 0.6931471805599453f + logf(l_tot) : -INFINITY;
    }
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" int dsa_bsa_fwd(const void* q, const void* k, const void* v, void* o,
                           const int64_t* strides, int32_t batch, int32_t q_tokens,
                           int32_t kv_tokens, int32_t heads, int32_t head_dim,
                           int32_t block_size, const int32_t* row_ptr,
                           const int32_t* col_idx, int32_t route_batches, float scale,
                           float* lse, hipStream_t stream) {
  dsa::clear_error();
  if (!q || !k || !v || !o || !strides)
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: null tensor or stride pointer");
  if (batch <= 0 || heads <= 0 || q_tokens <= 0 || kv_tokens <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: batch/heads/tokens must be positive");
  if (head_dim != kHeadDim)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_bsa_fwd: head_dim %d unsupported (128 only)",
                          head_dim);
  if (block_size != 128)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_bsa_fwd: block_size %d unsupported (128)",
                          block_size);
  if ((row_ptr == nullptr) != (col_idx == nullptr))
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: row_ptr and col_idx must both be set or null");
  if (row_ptr && route_batches != 1 && route_batches != batch)
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: route_batches must be 1 or batch");
  if (row_ptr && q_tokens != kv_tokens)
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: a block route needs q_tokens == kv_tokens");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: scale must be positive and finite");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: tensors must be 16-byte aligned");
  for (int i = 0; i < 12; ++i)
    if (strides[i] % 8 != 0)
      return dsa::set_error(DSA_EINVAL,
                            "dsa_bsa_fwd: stride %d (=%lld) is not a multiple of 8 elements", i,
                            (long long)strides[i]);
  const int32_t q_blocks = (q_tokens + block_size - 1) / block_size;
  const int32_t kv_blocks = (kv_tokens + block_size - 1) / block_size;
  const int64_t grid = (int64_t)batch * heads * q_blocks;
  if (grid > 0x7fffffff) return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: grid too large");

  BsaParams p;
  p.q = static_cast<const __bf16*>(q);
  p.k = static_cast<const __bf16*>(k);
  p.v = static_cast<const __bf16*>(v);
  p.o = static_cast<__bf16*>(o);
  p.lse = lse;
  p.q_sb = strides[0]; p.q_st = strides[1]; p.q_sh = strides[2];
  p.k_sb = strides[3]; p.k_st = strides[4]; p.k_sh = strides[5];
  p.v_sb = strides[6]; p.v_st = strides[7]; p.v_sh = strides[8];
  p.o_sb = strides[9]; p.o_st = strides[10]; p.o_sh = strides[11];
  p.row_ptr = row_ptr;
  p.col_idx = col_idx;
  p.batch = batch; p.heads = heads; p.q_tokens = q_tokens; p.kv_tokens = kv_tokens;
  p.q_blocks = q_blocks; p.kv_blocks = kv_blocks;
  p.route_batches = row_ptr ? route_batches : 1;
  p.scale = scale;
  p.scale_log2 = scale * 1.4426950408889634f;
  static const int variant = [] {
    const char* env = getenv("DSA_BSA_VARIANT");
    return env ? atoi(env) : 5;
  }();
  if (variant == 1)
    hipLaunchKernelGGL(bsa_fwd_kernel<128>, dim3((unsigned)grid), dim3(256), 0, stream, p);
  else if (variant == 4)
    hipLaunchKernelGGL(bsa_fwd4_kernel, dim3((unsigned)grid), dim3(256), 0, stream, p);
  else if (variant == 3)
    hipLaunchKernelGGL(bsa_fwd3_kernel, dim3((unsigned)grid), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(bsa_fwd5_kernel, dim3((unsigned)grid), dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_bsa_fwd");
}
