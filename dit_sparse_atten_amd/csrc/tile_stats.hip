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
// Design: the block-mass kernel's structure (one workgroup per (head, query
// tile), K half-tiles through LDS by buffer->LDS loads, S^T on the 32x32x16
// MFMA so each lane owns one query row, fixed-order reductions through LDS).
// The sums over keys run on the matrix cores too: each lane rounds its
// 2^15-scaled probabilities to fp16 (relative error <= 2^-11 per term), and
// C += W * P^T accumulates, per query, the row's mass and its key-offset
// moments, with W a table of weight rows (1, and hi/lo fp16 halves of each
// key offset) so the offsets enter at fp32 accuracy.  That leaves one FMA,
// one exp2 and half a conversion of VALU work per score (against four VALU
// ops and the exp2 for fp32 sums), which bounds this pass; the query-side
// moments are one multiply per row at the end of each tile.
//
// Tiles of 65..127 tokens whose 8-rounded size is below the half-tile slots
// (64 + 32 up to 96 tokens, else 128) take the gathered key stream instead:
// the row's key tiles are concatenated, each padded to tile_pad (the tile
// rounded up to 8), and staged as 64-key chunks, so a 72-token tile costs 72
// key slots rather than 96.  A chunk spans at most two tiles, and the tile
// boundary (a multiple of 8 positions into the chunk) falls between the
// lanes' 4-key runs.  The weight table sends the keys of even and odd tiles
// to different accumulator rows, so both tiles of a chunk accumulate in one
// pass and the earlier one is reduced after it.  Every kernel runs one wave per 32 query
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
// The sums run on the matrix cores: C += P * W with P (queries x keys) the
// probabilities in fp16, scaled by 2^15 so that values down to 2^-29 stay
// normal, and W (keys x columns) a table of weights.  Columns 8 par + s hold
// the sums of the key tiles of parity par (tile index mod 2): s = 0 mass,
// 1 / 2 the fp16 high parts of the key offsets y / x, 3 / 4 their low parts
// (v - fp16(v)), and 5 / 6 the mass again, to be weighed by the query offsets
// y / x when the tile ends.  W lives in dynamic LDS: kWRows rows (row 5 par +
// s for s <= 4) of wcols entries, the positions of each 16-key group stored
// in the order 0-3, 8-11, 4-7, 12-15 so that the eight weights one lane
// supplies to an MFMA are one 16-byte read; wcols = 8 mod 128 puts the ten
// rows on distinct LDS banks.
constexpr int kSlots = 7;
constexpr int kWRows = 10;
constexpr float kPShift = 15.f;
constexpr float kPUnscale = 1.f / 32768.f;
constexpr int kMaxTiles = 16384;  // tiles per row, as the route selection over them
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
  int32_t wcols;     // weight-table row length (>= 2 tile_pad + 64 gathered, else 128)
  int32_t xcd_slots; // workgroups of this launch resident at once on one XCD
  float scale_log2;
};

using dsa::tile_axis;

// Eight fp32 values as an fp16 MFMA operand (round to nearest even).
__device__ __forceinline__ dsa_f16x8 pack_f16x8(const float* v) {
  dsa_f16x8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const dsa_f32x2 two = {v[2 * i], v[2 * i + 1]};
    const dsa_f16x2 h = __builtin_convertvector(two, dsa_f16x2);
    r[2 * i] = h[0];
    r[2 * i + 1] = h[1];
  }
  return r;
}

// kWaves: waves per workgroup, one per 32 query rows of the tile (2..4).
template <typename T, bool kRouted, int kNh, bool kGather = false, int kWaves = 4>
__global__ void __launch_bounds__(kWaves * 64, 3) tile_stats_kernel(TileStatsParams p) {
  typedef dsa::Elem<T> E;
  constexpr int kThreads = kWaves * 64;
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k1[kKStage];
  __shared__ float part[2][kWaves][kSlots];
  __shared__ __attribute__((aligned(16))) float uq[3][128];  // 1, y, x of each query row
  extern __shared__ __attribute__((aligned(16))) _Float16 wtab[];  // [kWRows][p.wcols]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % p.tiles;
  const int h = work / p.tiles;

  // Weights: a key at position pos of the staged stream belongs to a tile of
  // parity par at tile-local offset off (the aligned path stages one tile at
  // a time: par 0, off = pos); pad slots weigh 0.
  for (int i = tid; i < kWRows * p.wcols; i += kThreads) {
    const int r = i / p.wcols, si = i % p.wcols;
    const int pos = (si & ~12) | ((si & 4) << 1) | ((si & 8) >> 1);  // bits 2, 3 swapped
    int par = 0, off = pos;
    if (kGather) {
      const int q = pos % (2 * p.tile_pad);
      par = q / p.tile_pad;
      off = q % p.tile_pad;
    }
    float w = 0.f;
    if (r / 5 == par && off < p.tile) {
      // Local token index -> (row, column) inside the tile, row-major.
      const float y = tile_axis(off / p.tile_w, p.tile_h);
      const float x = tile_axis(off % p.tile_w, p.tile_w);
      const int kind = r % 5;
      w = kind == 0 ? 1.f
        : kind == 1 ? (float)(_Float16)y
        : kind == 2 ? (float)(_Float16)x
        : kind == 3 ? y - (float)(_Float16)y
                    : x - (float)(_Float16)x;
    }
    wtab[i] = (_Float16)w;
  }
  for (int i = tid; i < 128; i += kThreads) {
    const bool in = i < p.tile;
    uq[0][i] = 1.f;
    uq[1][i] = in ? tile_axis(i / p.tile_w, p.tile_h) : 0.f;
    uq[2][i] = in ? tile_axis(i % p.tile_w, p.tile_w) : 0.f;
  }
  const int64_t cell0 = ((int64_t)h * p.tiles + qt) * p.tiles;
  if (kRouted) {
    // Cells this row does not list hold zero mass and zero centroids: clear
    // the row first; the listed cells are written after the first
    // vmcnt(0) barrier, so they land after these stores.
    const __half zero = __float2half(0.f);
    for (int kt = tid; kt < p.tiles; kt += kThreads) {
      const int64_t cell = cell0 + kt;
      p.mass32[cell] = 0.f;
      if (p.mass16) p.mass16[cell] = zero;
      if (p.cqy) p.cqy[cell] = zero;
      if (p.cqx) p.cqx[cell] = zero;
      if (p.cky) p.cky[cell] = zero;
      if (p.ckx) p.ckx[cell] = zero;
    }
  }

  const int local_row = wave * 32 + qi;
  const int tq = qt * p.tile + local_row;
  const bool row_ok = local_row < p.tile && tq < p.tokens;
  const bool wave_active = wave * 32 < p.tile;
  const int tq_c = tq < p.tokens ? tq : p.tokens - 1;
  const T* qrow = static_cast<const T*>(p.q) + h * p.q_sh + (int64_t)tq_c * p.q_st;
  typename E::x8 qf[8];
  dsa::load_q_fragments(qrow, g, p.head_dim, qf);
  // p * 2^15 = exp2(scale_log2 s - (lse log2 e - 15)).
  const float lse2 = row_ok ? p.lse[h * p.lse_sh + tq] * kLog2e - kPShift : INFINITY;

  int start = 0, end = p.tiles;
  if (kRouted) {
    const dsa::const_i32 rp = (dsa::const_i32)p.row_ptr;
    start = rp[(int64_t)h * p.tiles + qt];
    end = rp[(int64_t)h * p.tiles + qt + 1];
  }
  const dsa::const_i32 cidx = (dsa::const_i32)p.col_idx;
  const int ntile = end - start;
  // The row's tiles are walked cyclically from index rot.  Workgroup slot s
  // of an XCD (blockIdx.x / 8: the XCD's dispatch order) starts s / xcd_slots
  // of the way along, so that a workgroup starting when slot s - xcd_slots
  // ends picks up about where the resident ones are: the XCD's workgroups
  // then read the same key tiles at about the same time, from its L2.  Each
  // cell's sums are independent of the walk (up to fp32 rounding, fixed by
  // the launch shape and the device's CU count).
  const int rot = ntile > 0 && p.xcd_slots > 0
                      ? (int)((int64_t)(blockIdx.x / dsa::kNumXcd) * ntile / p.xcd_slots % ntile)
                      : 0;
  auto tile_of = [&](int j) -> int {
    const int jj = j + rot < ntile ? j + rot : j + rot - ntile;
    const int kt = kRouted ? cidx[start + jj] : jj;
    return (unsigned)kt < (unsigned)p.tiles ? kt : -1;
  };

  const T* kbase = static_cast<const T*>(p.k) + h * p.k_sh;
  uint32_t koff[4];
  dsa::k_tile_offsets(wave, lane, p.k_st, p.head_dim, koff);
  auto issue = [&](int kt, int half, unsigned char* dst) __attribute__((always_inline)) {
    const int key0 = (kt < 0 ? 0 : kt) * p.tile + half * kHalfKeys;
    const __amdgpu_buffer_rsrc_t rsrc = dsa::k_tile_rsrc(kbase, p.k_st, key0, p.tokens, p.head_dim);
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

  // Writes the cell of key tile kt, the j-th of this row (its partials sit in
  // part[j & 1]).  Lane s < 5 of wave 0 sums statistic s over the waves.
  auto flush = [&](int j, int kt) __attribute__((always_inline)) {
    if (wave == 0 && lane < kStats && kt >= 0) {
      const float(*pr)[kSlots] = part[j & 1];
      // mass, q_y, q_x from one slot; k_y, k_x as high + low parts.
      const int s0 = lane == 0 ? 0 : lane == 1 ? 5 : lane == 2 ? 6 : lane - 2;
      const int s1 = lane >= 3 ? lane : -1;
      auto waves = [&](auto slot) {  // (w0 + w1) + (w2 + w3) over the waves present
        if constexpr (kWaves == 1) return slot(0);
        else if constexpr (kWaves == 2) return slot(0) + slot(1);
        else if constexpr (kWaves == 3) return (slot(0) + slot(1)) + slot(2);
        else return (slot(0) + slot(1)) + (slot(2) + slot(3));
      };
      const float total =
          waves([&](int w) { return s1 >= 0 ? pr[w][s0] + pr[w][s1] : pr[w][s0]; });
      const float mass = waves([&](int w) { return pr[w][0]; });
      const int64_t cell = cell0 + kt;
      if (lane == 0) {
        const float normalized = mass / (float)p.tokens;
        p.mass32[cell] = normalized;
        if (p.mass16) p.mass16[cell] = __float2half(normalized);
      } else {
        __half* dst = lane == 1 ? p.cqy : lane == 2 ? p.cqx : lane == 3 ? p.cky : p.ckx;
        if (dst) dst[cell] = __float2half(total / fmaxf(mass, 1e-12f));
      }
    }
  };

  dsa::lds_barrier();  // the tables are ready

  // This lane's column of the sums (C column qi) and its weight row; the
  // unused columns (7, 15, 16..31) read row 0 too, and are never reduced.
  const int col = qi & 7, cpar = qi >> 3;
  const _Float16* wrow =
      wtab + (qi < 16 && col <= 4 ? 5 * cpar + col : (qi < 16 && col <= 6 ? 5 * cpar : 0)) *
                 p.wcols;
  // Its query weights at the end of a tile: 1, or the query offset y / x.
  const float* urow = uq[col == 5 ? 1 : col == 6 ? 2 : 0] + wave * 32 + 4 * g;
  dsa_f32x16 racc;
#pragma unroll
  for (int r = 0; r < 16; ++r) racc[r] = 0.f;
  // P of one 32-key sub-tile (pvs[4 quad + e]: key 8 quad + 4 g + e of this
  // lane's query) into the sums: two MFMAs of 16 keys each, with the weights
  // of the same keys (positions 16 h + 4 g + {0..3, 8..11} from the stream
  // position wbase of the sub-tile, stored at wbase + 16 h + 8 g + 0..7).
  auto reduce = [&](const float* pvs, int wbase) __attribute__((always_inline)) {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const dsa_f16x8 b = *reinterpret_cast<const dsa_f16x8*>(wrow + wbase + 16 * h2 + 8 * g);
      racc = dsa::Elem<_Float16>::mfma32(pack_f16x8(pvs + 8 * h2), b, racc);
    }
  };
  // Tile j (parity par) has ended: the lanes of its columns weigh their 16
  // query rows (8 i + 4 g + e: racc[4 i + e]), add the other half's, write
  // part[j & 1][wave] and clear their accumulators.
  auto end_tile = [&](int j, int par) __attribute__((always_inline)) {
    const bool mine = cpar == par && col < kSlots;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const dsa_f32x4 u = *reinterpret_cast<const dsa_f32x4*>(urow + 8 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum = fmaf(u[e], racc[4 * i + e], sum);
    }
    sum = dsa::pair32_sum(sum);
    if (mine && g == 0) part[j & 1][wave][col] = sum * kPUnscale;
#pragma unroll
    for (int r = 0; r < 16; ++r) racc[r] = mine ? 0.f : racc[r];
  };

  // Accumulates one staged half-tile of key tile kt.
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
      float pvs[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key_in_half = kk * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
        float pv = __builtin_amdgcn_exp2f(fmaf(sacc[i], p.scale_log2, -lse2));
        if (!kFull) pv = key_in_half < valid ? pv : 0.f;
        pvs[i] = pv;
      }
      reduce(pvs, half * kHalfKeys + kk * 32);
    }
  };


  if constexpr (kGather) {
    const int bp = p.tile_pad;
    const __amdgpu_buffer_rsrc_t k_all = dsa::make_rsrc(
        kbase, (uint32_t)((int64_t)(p.tokens - 1) * p.k_st * 2 + p.head_dim * 2));
    const uint32_t kst2 = (uint32_t)(p.k_st * 2);
    // Per-lane part of a slice's offsets: slice i stages stream rows 4 i +
    // (lane >> 4) at 16-byte column k2_swz(row, lane & 15), which depends on
    // i only through i mod 4; kDeadChunk (added: the rest stays below 2^31)
    // marks columns past head_dim.
    uint32_t lanepart[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int c = dsa::k2_swz(m * 4 + (lane >> 4), lane & 15);
      lanepart[m] = (uint32_t)(lane >> 4) * kst2 + (uint32_t)(c * 16) + dsa::dead_bits(c, p.head_dim);
    }
    // Stages the chunk that starts `o0` slots into tile kta and runs on into
    // tile ktb (both in range): stream row r is token kta tile + o0 + r
    // before the boundary (r < bp - o0), else ktb tile + o0 + r - bp (the
    // unsigned sums wrap back into range); pad slots load whatever they
    // address and are masked.
    auto issue_gather = [&](int kta, int ktb, int o0, unsigned char* dst)
        __attribute__((always_inline)) {
      const uint32_t base_a = (uint32_t)(kta * p.tile + o0) * kst2;
      const uint32_t base_b = (uint32_t)(ktb * p.tile + o0 - bp) * kst2;
      const int second = bp - o0;
#pragma unroll
      for (int i = 0; i < kKStage / 1024; ++i) {
        if (i % kWaves != wave) continue;
        const bool first = i * 4 + (lane >> 4) < second;
        dsa::lds_load16(k_all, dst + i * 1024,
                        (first ? base_a : base_b) + (uint32_t)(i * 4) * kst2 + lanepart[i & 3], 0);
      }
    };
    // Accumulates chunk positions [0, 32 NKK): those before `second` belong
    // to the chunk's first tile (at tile-local offset o0 + position), the
    // rest to the next tile (offset position - second); the weight table
    // sends each to the rows of its tile's parity.  wpos0: the chunk's
    // start in the table (its stream position mod 2 tile_pad).  masked: pad
    // slots, positions >= left and out-of-range tiles (ok_a / ok_b false)
    // count zero.
    auto compute_gather = [&](const unsigned char* cur, int o0, int second, int wpos0,
                              int left, bool ok_a, bool ok_b, auto nkk_c, auto masked_c)
        __attribute__((always_inline)) {
      constexpr int NKK = decltype(nkk_c)::value;
      constexpr bool masked = decltype(masked_c)::value;
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
        // Positions counted: [0, lim_a) of the first tile and [second,
        // second + span_b) of the next (pad slots, the row's end and
        // out-of-range tiles excluded).
        const int lim_a = ok_a ? min(min(second, p.tile - o0), left) : 0;
        const int span_b = ok_b ? max(min(p.tile, left - second), 0) : 0;
        float pvs[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // This lane's keys: positions 8 quad + 4 g + (0..3) of the
          // sub-tile; a tile boundary (a multiple of 8) never splits them.
          const int pos = kk * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
          float pv = __builtin_amdgcn_exp2f(fmaf(sacc[i], p.scale_log2, -lse2));
          if constexpr (masked) {
            const bool ok = pos < lim_a || (unsigned)(pos - second) < (unsigned)span_b;
            pv = ok ? pv : 0.f;
          }
          pvs[i] = pv;
        }
        reduce(pvs, wpos0 + kk * 32);
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
      int wpos0 = 0;  // the chunk's stream position mod 2 tile_pad
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
        const int left = total - c * 64;
        const bool masked = bp > p.tile || left < 64 || ka < 0 || kb < 0;
        const unsigned char* cur = (c & 1) ? lds_k1 : lds_k0;
        using one = std::integral_constant<int, 1>;
        using two = std::integral_constant<int, 2>;
        // Only chunks with pad slots, the row's end or an out-of-range tile
        // pay for the per-key mask (left <= 32 implies masked).
        if (left <= 32)
          compute_gather(cur, o0, second, wpos0, left, ka >= 0, kb >= 0, one{}, std::true_type{});
        else if (masked)
          compute_gather(cur, o0, second, wpos0, left, ka >= 0, kb >= 0, two{}, std::true_type{});
        else
          compute_gather(cur, o0, second, wpos0, left, ka >= 0, kb >= 0, two{}, std::false_type{});
        if (has_next && second <= 64) {
          // Tile j0 ended in this chunk.
          end_tile(j0, j0 & 1);
          pend_j = j0;
          pend_kt = ka;
        }
        j0 = j1; o0 = o1; ka = ka1; kb = kb1;
        wpos0 += 64;
        if (wpos0 >= 2 * bp) wpos0 -= 2 * bp;
      }
      end_tile(n - 1, (n - 1) & 1);
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
      end_tile(j, 0);
      prev_kt = kt;
    }
  }
  dsa::lds_barrier();
  if (nsteps > 0) flush(ntile - 1, prev_kt);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Compute units of the stream's device (cached per device; 0 if unknown).
int device_cus(hipStream_t stream) {
  constexpr int kMaxDevices = 64;
  static int cus[kMaxDevices] = {0};
  int device = -1;
  if (stream == nullptr || hipStreamGetDevice(stream, &device) != hipSuccess)
    if (hipGetDevice(&device) != hipSuccess) return 0;
  if (device < 0 || device >= kMaxDevices) return 0;
  if (cus[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return 0;
    cus[device] = n;
  }
  return cus[device];
}

template <typename T>
void launch_tile_stats(TileStatsParams p, bool routed, bool gather, hipStream_t stream) {
  const int32_t tile = p.tile;
  const int32_t need = gather ? 2 * p.tile_pad + 64 : 128;
  p.wcols = (need + 119) / 128 * 128 + 8;  // the least >= need that is 8 mod 128
  const size_t lds = (size_t)kWRows * p.wcols * sizeof(_Float16);
  const dim3 blocks((unsigned)((int64_t)p.heads * p.tiles));
  const int cus = device_cus(stream);
  auto go = [&](auto kernel, int waves) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, waves * 64, lds) !=
        hipSuccess)
      per_cu = 0;
    p.xcd_slots = per_cu * cus / dsa::kNumXcd;  // 0: natural walk order
    hipLaunchKernelGGL(kernel, blocks, dim3(waves * 64), lds, stream, p);
  };
  if (gather && tile <= 96) {
    routed ? go(tile_stats_kernel<T, true, 2, true, 3>, 3)
           : go(tile_stats_kernel<T, false, 2, true, 3>, 3);
  } else if (gather) {
    routed ? go(tile_stats_kernel<T, true, 2, true, 4>, 4)
           : go(tile_stats_kernel<T, false, 2, true, 4>, 4);
  } else if (tile > 96) {
    routed ? go(tile_stats_kernel<T, true, 2>, 4) : go(tile_stats_kernel<T, false, 2>, 4);
  } else if (tile > kHalfKeys) {
    routed ? go(tile_stats_kernel<T, true, 2, false, 3>, 3)
           : go(tile_stats_kernel<T, false, 2, false, 3>, 3);
  } else {
    // Two waves even for tiles of at most 32 tokens (one of them then only
    // stages K): one-wave workgroups, four per CU, leave too few waves to
    // hide the dense pass's latency.
    routed ? go(tile_stats_kernel<T, true, 1, false, 2>, 2)
           : go(tile_stats_kernel<T, false, 1, false, 2>, 2);
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
