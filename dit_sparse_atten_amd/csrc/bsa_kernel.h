// Block-sparse attention forward for gfx950 (MI355X): bf16 or fp16 in/out,
// fp32 softmax.  The kernel templates shared by bsa_fwd.hip (bf16 instances
// and the C-ABI entry points) and bsa_fwd_f16.hip (fp16 instances).
//
// Replaces the FlexAttention call of the reference backend
// (attention_backends/flex.py:379-399 `_flex_output`, kernel options
// flex.py:360-364) and its dense SDPA fallback (attention_backends/dense.py:14-48).
//
// Semantics per (batch b, head h, query row t):
//   O[b,t,h,:] = softmax_k( scale * <Q[b,t,h,:], K[b,k,h,:]> ) @ V[b,k,h,:]
// where k ranges over the tokens of every key block listed in the CSR row of
// (route batch, h, t / 128).  Without a CSR every key block is listed (dense
// fallback).  Keys past `kv_tokens` in a partial last block are masked.
//
// Design (per 128-row query block, one 4-wave workgroup, two per CU):
//  * wave w owns query rows 32w..32w+31; S^T = K Q^T uses
//    v_mfma_f32_32x32x16_bf16 (or _f16) so each lane's accumulators belong to one query
//    row (row max / sum stay in registers, one cross-half exchange) and P^T
//    leaves the accumulators already in the B-operand layout of O^T = V^T P^T;
//  * keys stream as 64-key half-tiles of K and V, double-buffered in LDS by
//    direct buffer->LDS loads issued one half-tile ahead; the two stages are
//    distinct LDS objects so reads of one never wait on the DMA into the
//    other, and rows past the sequence end read as zeros (buffer range check);
//  * V is staged row-major like K, straight from the caller's tensor; the
//    V^T A-operand fragments of O^T = V^T P^T come out of that stage through
//    gfx950's transposing LDS read (ds_read_b64_tr_b16: in each 16-lane
//    group, lane j receives element j % 4 of the 8 bytes that lane
//    4 r + j / 4 addresses, r = 0..3), so no transposed copy of V exists;
//    each lane addresses the 4-key quads in the order 0, 2, 1, 3 (the key
//    order of the P^T slots);
//  * online softmax with a lazily moved reference max (rescale only when a
//    score exceeds it by 2^8); with key norms from key_norm_kernel, a row
//    takes its max only while the Cauchy-Schwarz bound |q| max|k| could put a
//    score more than 2^32 (bf16; fp16: 2^15) above the reference (in practice
//    on its first half-tile only); row sums add the fp32 P in plain VALU adds
//    (v_dot2 would contend with the matrix core for issue); the row max and
//    the final row sum pair lanes l and l ^ 32 with v_permlane32_swap;
//  * query / key blocks of 1..128 tokens (the matrix-sparse backend's spatial
//    tiles): routed whole blocks of 65..127 keys stream the row's kept blocks
//    as one gathered key sequence (kGather), and routed blocks of at most 64
//    tokens run 2-wave workgroups (kWaves);
//  * the last, partial round of query blocks may run as 2..8 key ranges each
//    (choose_split), whose fp32 partials bsa_merge_kernel combines;
//  * routed calls may walk each row's key blocks from a rotated start (the
//    aligned walk, walk_start): the workgroups resident on one XCD then read
//    the same key blocks at about the same time, from its L2.
#pragma once

#include <algorithm>
#include <type_traits>

#include "bsa_tiles.h"

namespace bsa {

struct BsaParams {
  const void* q;  // element type T of the kernel instance
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t q_sb, q_st, q_sh;
  int64_t k_sb, k_st, k_sh;
  int64_t v_sb, v_st, v_sh;
  int64_t o_sb, o_st, o_sh;
  const int32_t* row_ptr;  // null: every key block (dense)
  const int32_t* col_idx;
  const int32_t* order;    // routed: work item of each launch slot (null: identity)
  int32_t* queue;          // work-queue counter, zero at launch (null: slot = blockIdx.x)
  uint64_t* walk;          // routed: aligned-walk position table (null: plain walk)
  // Per (batch, head): kNormParts maxima of the key norms over consecutive
  // token ranges, from key_norm_kernel (null: every half-tile takes its row
  // max).
  const float* kv_norm;
  int32_t batch, heads, q_tokens, kv_tokens, q_blocks, kv_blocks, route_batches;
  int32_t block;     // tokens per query block and per key block (1..128)
  int32_t head_dim;  // 8..128, a multiple of 8; dims past it are zero in the stages
  int32_t causal;    // dense only: query t attends keys k <= t
  int32_t deterministic;  // host side: 1 = plain walk (results reproducible bit for bit)
  int32_t block_pad; // gathered stream: key slots per block (block rounded up to 8)
  float scale;       // softmax scale applied to <q, k>
  float scale_log2;  // scale * log2(e)
  // Split tail: workgroups from split_from on each compute one of `parts` key
  // ranges of query block split_from + (wg - split_from) / parts and leave
  // their unnormalised partial in `part` for bsa_merge_kernel.
  int32_t split_from;
  int32_t parts;
  float* part;
  // Fused tile statistics (the kStats instances), per query row and key tile
  // of stat_tile = tile_h * tile_w tokens: rs_logm = log2 of the row's
  // unnormalised probability mass on the key tile, sum 2^(scale_log2 s), and
  // rs_mean = its mass-weighted mean key offsets (y, x) as two fp16 (null:
  // not written, the exact block mass needs only the mass).  Routed:
  // at e * block + r for CSR entry e and query row r of the tile, entries at
  // or past rs_entries not written.  Dense: at (h * tiles + key tile) *
  // q_tokens + query token.
  float* rs_logm;
  uint32_t* rs_mean;
  int64_t rs_entries;
  int32_t tile_h, tile_w;
  int32_t stat_tile;  // tokens per statistics tile (1..128)
  // Stream slots per statistics tile: gathered stream block_pad, plain
  // stream 64 kNh (a tile per key block), dense token stream stat_tile.
  int32_t stat_pad;
  // Attention dropout (dense calls, the fp32-compute kernel): a probability
  // is kept when its Philox uniform is >= drop_thresh (0: no dropout), then
  // scaled by drop_scale = 1 / (1 - dropout_p).
  uint32_t drop_thresh;
  float drop_scale;
  uint32_t drop_seed_lo, drop_seed_hi, drop_offset;
};

// One split partial: O [128 rows][128 dims] relative to the row's reference
// max, then m (log2 units of the scaled scores) and l per row, in fp32.
constexpr int kPartFloats = 128 * 128 + 2 * 128;
constexpr int kMaxPartGroups = 1024;  // split workgroups per call (two rounds of 512 slots)

using dsa::kHeadDim;
using dsa::kRowBytes;
using dsa::kHalfKeys;
using dsa::kKStage;
using dsa::k2_swz;
using dsa::k_tile_rsrc;
using dsa::lds_load16;
using dsa::make_rsrc;
typedef dsa::const_i32 dsa_const_i32;

constexpr float kRescaleLog2 = 8.0f;  // move the max once p could exceed 2^8
// Half-tiles whose scores provably stay within 2^bound_log2 of the reference
// max (key-norm bound) skip the row max.  The P operand carries p in the
// input type: bf16 (fp32's exponent range) takes p <= 2^32, which leaves fp32
// sums and O accumulators of up to 2^20 keys finite for |v| < 2^76; fp16
// overflows at 65,504, so it takes p <= 2^15.  raise_log2: how far below its
// largest p a row's first half-tile may be scaled to meet the bound (fp16
// keeps that p a normal number).
template <typename T>
constexpr float bound_log2() { return std::is_same<T, _Float16>::value ? 15.0f : 32.0f; }
template <typename T>
constexpr float raise_log2() { return std::is_same<T, _Float16>::value ? 4.0f : 16.0f; }
constexpr int kNormParts = 64;        // key-norm maxima per (batch, head), one per lane
constexpr int64_t kMaxNormPairs = 4096;  // (batch, head) pairs with norms (1 MiB)

// V stage [64 keys][128 dims], row-major like K: the 16-byte chunk c of key
// row r sits at chunk position c ^ v_swz_mask(r), masks 0, 6, 10, 12 for
// r & 3 = 0..3.  One transposed read of a 16-lane group touches 4 consecutive
// key rows x 32 bytes (two chunks); these masks give the 4 rows' segments
// distinct bank groups, for 32 as for 64 four-byte banks per clock.
__device__ __forceinline__ int v_swz_mask(int r) { return (0xCA60 >> (4 * (r & 3))) & 15; }
__device__ __forceinline__ int v_swz(int r, int c) { return c ^ v_swz_mask(r); }

// ds_read_b64_tr_b16 at an LDS address, as four 16-bit elements of type T.
template <typename T>
__device__ __forceinline__ typename dsa::Elem<T>::x4 lds_read_tr(const unsigned char* lds) {
  const dsa_i16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) dsa_i16x4*)(lds));
  return __builtin_bit_cast(typename dsa::Elem<T>::x4, raw);
}

// Aligned key walk.  The accumulation order of a row's key blocks does not
// change its result beyond fp32 rounding, so a routed workgroup may start its
// walk anywhere in its row and wrap around.  Workgroups that each walk their
// own route from the first key block drift apart within a few rows (their
// rows differ in length and their clocks in speed), and an XCD's resident
// workgroups then read key blocks spread over most of a head, far more than
// its 4 MB L2 holds.  With a walk table, every workgroup publishes (time,
// batch-head, key block) in its XCD's row of the table once per key block,
// and a starting workgroup starts at the first of its key blocks at or past
// the circular mean of the fresh positions of the same batch-head, so the
// XCD's workgroups of one head move as a pack.  The start then depends on
// timing: results can differ in the last bits from run to run, which is why
// a deterministic call passes no table.
constexpr int kWalkSlots = 64;                             // entries per XCD
constexpr size_t kWalkBytes = (size_t)dsa::kNumXcd * kWalkSlots * sizeof(uint64_t);
constexpr uint32_t kWalkFreshTicks = 100;                  // 16 us in 0.16 us ticks
constexpr int kWalkMaxBlocks = 65535;                      // key blocks a position encodes

// XCD of the calling wave (HW_REG_XCC_ID, bits 3:0).
__device__ __forceinline__ int xcc_id() {
  return (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & (dsa::kNumXcd - 1));
}

// The 100 MHz real-time counter in 0.16 us ticks, truncated to 32 bits.
__device__ __forceinline__ uint32_t walk_now() {
  return (uint32_t)(__builtin_amdgcn_s_memrealtime() >> 4);
}

__device__ __forceinline__ uint64_t walk_entry(int bh, int kb) {
  return ((uint64_t)walk_now() << 32) | ((uint64_t)(bh & 0xffff) << 16) | (uint64_t)kb;
}

// Index into the row's key list at which a workgroup of batch-head bh starts
// (one full wave calls it; every lane gets the result): 0 without fresh
// entries, else the first entry at or past the entries' circular mean key
// block (the list is ascending; for any other order the start is still a
// valid rotation).
__device__ __forceinline__ int walk_start(const uint64_t* tab, int lane, int bh, int kv_blocks,
                                          dsa::const_i32 cidx, int start, int nblk) {
  const uint64_t e = __hip_atomic_load(tab + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool fresh = e != 0 && (int)((e >> 16) & 0xffff) == (bh & 0xffff) &&
                     walk_now() - (uint32_t)(e >> 32) < kWalkFreshTicks;
  const float turn = 6.2831853f / (float)kv_blocks;
  const float angle = fresh ? (float)(int)(e & 0xffff) * turn : 0.f;
  const float c = dsa::wave_total(fresh ? __cosf(angle) : 0.f);
  const float sn = dsa::wave_total(fresh ? __sinf(angle) : 0.f);
  if (c * c + sn * sn < 1e-6f) return 0;
  float mean = atan2f(sn, c);
  if (mean < 0.f) mean += 6.2831853f;
  const int pos = min(kv_blocks - 1, max(0, (int)(mean / turn)));
  // 64 evenly spaced probes bracket the answer; a second probe of the
  // bracketing segment (at most 64 entries up to 4,096 blocks) finds it.
  const int below = (int)__popcll(__ballot(cidx[start + (int)(((int64_t)lane * nblk) >> 6)] < pos));
  const int lo = below == 0 ? 0 : (int)(((int64_t)(below - 1) * nblk) >> 6);
  const int hi = below == 64 ? nblk : (int)(((int64_t)below * nblk) >> 6);
  if (hi - lo > 64) return lo < nblk ? lo : 0;
  const int i = lo + lane;
  const int in_seg = (int)__popcll(__ballot(i < hi && cidx[start + i] < pos));
  const int r = lo + in_seg;
  return r < nblk ? r : 0;
}

// kRouted: key blocks from the CSR row (false: every key block, dense).
// kNh: 64-key half-tiles per key block (2 for blocks of 65..128 keys, else 1).
// kSkip: some half-tile of every block holds at most 32 valid keys (block
// sizes 65..96, or at most 32), so those steps run one 32-key sub-tile.
// kGather (routed, whole blocks of 65..127 keys): the row's kept blocks are
// concatenated, each padded to block_pad keys, and streamed as 64-key chunks,
// so a 72-key block costs 72 key slots instead of 64 + 32.  Row r of a
// chunk's K and V stages holds stream position r, so the S^T, P^T and V^T
// lane layouts are those of the plain stream.
//
// kWaves: waves per workgroup, 32 query rows each (4; 2 for routed blocks of
// at most 64 tokens, whose rows two waves cover: smaller workgroups spread
// over the four SIMDs instead of leaving two waves per workgroup idle).
//
// kStats: the workgroup also writes the per-row tile statistics (rs_logm,
// rs_mean) from the probabilities of its own softmax.  Either every key block
// is one statistics tile (stat_tile == block: routed calls in either stream,
// and dense calls of tile-sized blocks), or a dense call runs 128-token
// blocks over tiles of 64..128 tokens, a multiple of 8 (the token stream).
// The key-side sums run on the matrix cores beside O^T = V^T P^T: with the
// same P^T operand, C += W^T P^T where W^T (kStatRows x keys, an LDS table)
// holds, for the key tiles of each parity (stream tile index mod 2), the
// rows 1, y_hi, x_hi, y_lo, x_lo of each key's tile-local offsets split into
// an input-type high part and the remainder.  The rows sit at C rows 0-3, 8
// (even tiles) and 4-7, 12 (odd tiles), so each lane's accumulators 0..4
// are its query row's five sums for the key tiles of its own half's parity.
// Tiles span two chunks at most (65..128 keys against 64-key chunks) and two
// tiles of one parity never share a chunk, so each lane carries the five sums
// of one open tile across chunks and closes it in the chunk where it ends.
// In the plain stream a key block is staged as kNh half-tiles from its first
// key, so tile j's half-tile `half` reads the table from position
// (j & 1) stat_pad + 64 half with stat_pad = 64 kNh, and the tile closes
// after its last half-tile.  A dense token stream is the token sequence
// itself, 64 keys per step, so the table serves with tiles of stat_tile
// slots (every step 16-aligned in its period, at most one tile end each).
constexpr int kStatRows = 11;    // 2 parities x 5 kinds, then a zero row
constexpr int kStatCols = 392;   // >= 2 * 120 + 64 positions; = 8 mod 128 spreads the rows' banks

//
// kMassOnly (with kStats, tile blocks, no rs_mean: the exact block mass):
// a tile is a key block, so its mass is the part of the row sum its own
// half-tiles add; each lane keeps its half of that sum and the close adds
// the two halves.  No weight table, no key-side MFMAs.
template <typename T, bool kRouted, int kNh, bool kSkip, bool kGather = false, int kWaves = 4,
          bool kStats = false, bool kMassOnly = false>
__global__ void __launch_bounds__(kWaves * 64, 2)
    bsa_fwd_kernel(BsaParams p) {
  typedef dsa::Elem<T> E;
  typedef typename E::x8 x8;
  static_assert(!kGather || kRouted, "the gathered stream takes a block route");
  // Only the dense 128-token instance may run the token stream; every other
  // statistics instance has one tile per key block.
  constexpr bool kTokenStream = kStats && !kRouted && kNh == 2 && !kSkip;
  // The key-norm bound (compute), except in the plain-stream instances that
  // skip empty sub-tiles (65..96-key blocks, blocks of at most 32): there it
  // ran slower (same-box A/B: 9 x 10 tiles 66.9 -> 70.9 ms, 3 x 8 tiles
  // 382 -> 411 ms).
  constexpr bool kNormBound = kGather || !kSkip;
  // Wave priority (s_setprio) over one phase of each step, so that the two
  // waves sharing a SIMD fall into opposite phases and one's VALU work runs
  // beside the other's MFMAs: the gathered stream raises it for the softmax,
  // the dense 128-token kernel for the PV products.  Same-box A/B, kernel
  // time: 720p tiles 58.6 -> 58.2 ms, dense config-2 shape 56.5 -> 55.2 ms.
  // The routed 128-token kernel and the statistics instances (720p tiles
  // with statistics 74.4 -> 75.2 ms with it) ran slower and set none.
  constexpr bool kPrioSoftmax = kGather && !kStats;
  constexpr bool kPrioPv = !kRouted && !kStats && !kSkip && kNh == 2;
  // 2-wave workgroups (blocks of at most 64 keys) stage one block at a time:
  // 32 KB of LDS lets four of them share a CU (two waves per SIMD) where the
  // double-buffered 64 KB allowed two; the next block's loads start after
  // every wave has finished with the current one, and the other workgroups
  // of the CU cover their latency.
  constexpr bool kSingleStage = kWaves == 2;
  static_assert(!kSingleStage || kNh == 1, "2-wave workgroups take blocks of at most 64 keys");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k1[kSingleStage ? 16 : kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v0[kKStage];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_v1[kSingleStage ? 16 : kKStage];
  static_assert(!kMassOnly || (kStats && !kGather), "mass-only statistics are tile blocks");
  // Blocks of at most 64 keys read table positions below 2 * 64 only, and a
  // narrower table keeps four 2-wave workgroups within a CU's LDS.
  constexpr int kCols = kNh == 1 ? 136 : kStatCols;
  __shared__ __attribute__((aligned(16))) T wtab[kStats && !kMassOnly ? kStatRows * kCols : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;

  // Dense: each XCD takes a contiguous range of (b, h) rows, whose workgroups
  // stream the same keys in lock step through that XCD's L2.  Routed: slots
  // are dealt round-robin over the XCDs, so every XCD gets an eighth of every
  // head (routes whose keep differs from head to head, 0.2 to 0.65 per head
  // under spatially local attention, would otherwise leave the XCDs holding
  // the dense heads working alone), and `order` (launch_order_kernel) puts
  // each head's rows longest first, so the workgroups resident side by side
  // run rows of similar length and stay in step through the L2.
  //
  // With a work queue, each workgroup takes the next launch slot from a
  // counter when it starts, rather than the slot of its dispatch index: the
  // dispatcher deals workgroups to the XCDs round-robin, and the XCDs do not
  // run equally fast (on one box the odd ones took 5% longer over the same
  // work), so fixed slots leave the fast XCDs idle at the end.  Slots are then
  // taken in start order across the whole chip (dense calls walk them in
  // order: all XCDs read one head's keys at a time).  A row's result does not
  // depend on which workgroup computes it.
  int wg = (int)blockIdx.x;
  if (p.queue != nullptr) {
    __shared__ int wg_lds;
    if (tid == 0)
      wg_lds = __hip_atomic_fetch_add(p.queue, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    wg = __builtin_amdgcn_readfirstlane(wg_lds);
  }
  const bool split = wg >= p.split_from;
  int slot = wg, part = 0;
  if (split) {
    const int t = wg - p.split_from;
    slot = p.split_from + t / p.parts;
    part = t % p.parts;
  }
  int work = slot;
  if (kRouted && p.order) work = ((dsa_const_i32)p.order)[slot];
  else if (!kRouted && !split && !p.queue) work = dsa::xcd_remap(wg, p.split_from);
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;

  int start = 0, end = p.kv_blocks;
  if (!kRouted && p.causal) {
    // Keys up to the block's last query row (query t sees keys k <= t).
    const int last_row = min(qb * p.block + p.block, p.q_tokens) - 1;
    end = min(p.kv_blocks, last_row / p.block + 1);
  }
  if (kRouted) {
    const dsa_const_i32 rp = (dsa_const_i32)p.row_ptr;
    const int rb = p.route_batches == 1 ? 0 : b;
    const int64_t row = ((int64_t)rb * p.heads + h) * p.q_blocks + qb;
    start = rp[row];
    end = rp[row + 1];
  }
  if (split) {  // key part `part` of the row's blocks
    const int n = end - start;
    end = start + (int)((int64_t)n * (part + 1) / p.parts);
    start = start + (int)((int64_t)n * part / p.parts);
  }
  const dsa_const_i32 cidx = (dsa_const_i32)p.col_idx;
  const int nblk = end - start;

  // Aligned walk (split workgroups keep their plain key range): wave 0 picks
  // the start, the others read it from LDS; thread 0 publishes positions.
  int rot = 0;
  uint64_t* walk_at = nullptr;
  if (kRouted && !split && p.walk != nullptr) {
    uint64_t* const tab = p.walk + xcc_id() * kWalkSlots;
    if (nblk > 1) {
      __shared__ int rot_lds;
      if (wave == 0) {
        const int r = walk_start(tab, lane, bh, p.kv_blocks, cidx, start, nblk);
        if (lane == 0) rot_lds = r;
      }
      __syncthreads();
      rot = __builtin_amdgcn_readfirstlane(rot_lds);
    }
    if (tid == 0) walk_at = tab + (wg / dsa::kNumXcd) % kWalkSlots;
  }
  // List index of the j-th key block walked.
  auto walked = [&](int j) -> int { return start + (j + rot < nblk ? j + rot : j + rot - nblk); };

  // Rows past the block (blocks shorter than 128) or the sequence are
  // computed on a clamped row and never stored; waves wholly past the block
  // only stage their share of K/V.
  const int local_row = wave * 32 + qi;
  const int tq = qb * p.block + local_row;
  const bool row_ok = local_row < p.block && tq < p.q_tokens;
  const bool wave_active = wave * 32 < p.block;
  const int tq_c = tq < p.q_tokens ? tq : p.q_tokens - 1;
  const T* qrow = static_cast<const T*>(p.q) + b * p.q_sb + h * p.q_sh + (int64_t)tq_c * p.q_st;
  x8 qf[8];
  dsa::load_q_fragments(qrow, g, p.head_dim, qf);
  // Key-norm bound of the lane's row: |scale_log2 s| <= |scale_log2| |q| kmax
  // (Cauchy-Schwarz) over every key of the (batch, head), with kmax the
  // largest key norm (from its kNormParts partial maxima, one per lane) and
  // |q| from the row's fragments (lanes l and l ^ 32 hold its two halves),
  // rounded up.  thr = bound - bound_log2 (+inf without norms): while the
  // reference max m_run >= thr, no p of the row can exceed 2^bound_log2.
  float thr = INFINITY;
  if (kNormBound && p.kv_norm != nullptr) {
    float kmax = p.kv_norm[(int64_t)bh * kNormParts + lane];
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) kmax = fmaxf(kmax, __shfl_xor(kmax, m));
    float qq = 0.f;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc)
#pragma unroll
      for (int e = 0; e < 8; ++e) qq = fmaf((float)qf[dc][e], (float)qf[dc][e], qq);
    const float qn = sqrtf(dsa::pair32_sum(qq)) * fabsf(p.scale_log2) * 1.0001f;
    thr = fmaf(qn, kmax, -bound_log2<T>());
  }

  const T* kbase = static_cast<const T*>(p.k) + b * p.k_sb + h * p.k_sh;
  const T* vbase = static_cast<const T*>(p.v) + b * p.v_sb + h * p.v_sh;
  // Each wave stages kSlices of the 16 1-KB slices of a K or V stage.
  static_assert(kWaves == 4 || (kWaves == 2 && !kGather), "2-wave groups: plain stream only");
  constexpr int kSlices = 16 / kWaves;
  // Per-lane source byte offsets relative to the half-tile's first key (a
  // chunk of dims at or past head_dim loads zeros, dsa::dead_bits).
  uint32_t koff[kSlices], voff[kSlices];
#pragma unroll
  for (int j = 0; j < kSlices; ++j) {
    const int idx = (wave * kSlices + j) * 64 + lane;
    const int row = idx >> 4;
    const int kc = k2_swz(row, idx & 15), vc = v_swz(row, idx & 15);
    koff[j] = (uint32_t)((row * (int)p.k_st + kc * 8) * 2) | dsa::dead_bits(kc, p.head_dim);
    voff[j] = (uint32_t)((row * (int)p.v_st + vc * 8) * 2) | dsa::dead_bits(vc, p.head_dim);
  }

  // V^T fragment reads: lane (g, i = lane % 32) of the PV product needs dims
  // 32 dt + i of the 16-key group's quads (2 g) and (2 g + 1) in slot order,
  // i.e. key rows 4 g + r and 8 + 4 g + r (r = 0..3; the quad order 0, 2, 1, 3
  // of the P^T slots).  In its 16-lane group, lane 4 r + c addresses key row
  // 4 g + r, dims 32 dt + 16 ((lane >> 4) & 1) + 4 c .. + 3; the transposed
  // read hands every lane its own dim of the 4 rows.  Byte offsets per dt.
  int vfrag[4];
  {
    const int lam = lane & 15, r = lam >> 2, c = lam & 3;
    const int row = 4 * g + r;
    const int sub = 2 * ((lane >> 4) & 1) + (c >> 1);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      vfrag[dt] = row * kRowBytes + v_swz(row, 4 * dt + sub) * 16 + (c & 1) * 8;
  }
  // K fragment of chunk dc (row kt 32 + qi): the chunk index 2 dc + g XOR
  // (qi & 15) times 16 is (dc << 5) ^ ((g ^ (qi & 15)) << 4), and the row's
  // 256 bytes leave the low 8 address bits to it, so every offset is
  // kt 8192 + (kfrag ^ (dc << 5)); likewise vfrag[dt] = vfrag[0] ^ (dt << 6).
  // kLeanAddr instances rebuild the offsets from these two registers each
  // step (an empty asm keeps the compiler from hoisting them back out): the
  // 4-wave statistics instances, which otherwise spill the eight K offsets to
  // scratch and reload them inside the QK chain (720p 9 x 8 tiles 85.2 ->
  // 84.0 ms).  kDeferSums: the plain-stream 4-wave statistics instances add
  // a chunk's key-side sums in the next chunk's softmax (see wprev): dense
  // 9 x 8 tiles 81.6 -> 80.1 ms, routed 9 x 10 75.2 -> 73.5 ms.  Same-box A/B;
  // the gathered stream and the 2-wave instances ran 0-5% slower with it.
  constexpr bool kLeanAddr = kStats && kNh == 2;
  constexpr bool kDeferSums = kStats && kNh == 2 && !kGather && !kMassOnly;
  const int kfrag = qi * kRowBytes + ((g ^ (qi & 15)) << 4);

  auto block_of = [&](int j) -> int {
    const int kb = kRouted ? cidx[walked(j)] : start + j;
    return (unsigned)kb < (unsigned)p.kv_blocks ? kb : -1;
  };

  // Stages half-tile `half` of key block kb (an invalid block stages block 0,
  // which is then fully masked).
  auto issue = [&](int kb, int half, unsigned char* kdst, unsigned char* vdst) {
    const int kbc = kb < 0 ? 0 : kb;
    const int key0 = kbc * p.block + half * kHalfKeys;
    const __amdgpu_buffer_rsrc_t k_rsrc = k_tile_rsrc(kbase, p.k_st, key0, p.kv_tokens, p.head_dim);
    const __amdgpu_buffer_rsrc_t v_rsrc = k_tile_rsrc(vbase, p.v_st, key0, p.kv_tokens, p.head_dim);
#pragma unroll
    for (int j = 0; j < kSlices; ++j)
      lds_load16(k_rsrc, kdst + (wave * kSlices + j) * 1024, koff[j], 0);
#pragma unroll
    for (int j = 0; j < kSlices; ++j)
      lds_load16(v_rsrc, vdst + (wave * kSlices + j) * 1024, voff[j], 0);
  };
  // Stages the 64-key chunk that starts `o0` slots into stream block kb0 and
  // runs on into kb1 (the blocks are in range; pad and tail slots load
  // whatever they address, or zeros past the end, and are masked).
  const __amdgpu_buffer_rsrc_t k_all_rsrc = make_rsrc(
      kbase, (uint32_t)((int64_t)(p.kv_tokens - 1) * p.k_st * 2 + p.head_dim * 2));
  const __amdgpu_buffer_rsrc_t v_all_rsrc = make_rsrc(
      vbase, (uint32_t)((int64_t)(p.kv_tokens - 1) * p.v_st * 2 + p.head_dim * 2));
  // Lane (wave, lane) stages the 16-byte chunk (lane & 15) of the chunk's
  // stream rows g_r0 + 4 j, j = 0..3.  Row r holds token base0 + r while
  // o0 + r < block_pad (block kb0) and base1 + r after (block kb1), with
  // base0 = kb0 block + o0 and base1 = kb1 block + o0 - block_pad, so its
  // byte offset is a per-lane constant (gk / gv: row stride plus chunk, with
  // the dead-dims bit added, as no valid offset on this path reaches 2^31)
  // plus base0 or base1 times the stride, uniform per block.
  const int g_r0 = wave * 16 + (lane >> 4);
  uint32_t gk[4] = {0u, 0u, 0u, 0u}, gv[4] = {0u, 0u, 0u, 0u};
  if constexpr (kGather) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = g_r0 + 4 * j;
      const int kc = k2_swz(row, lane & 15), vc = v_swz(row, lane & 15);
      gk[j] = (uint32_t)row * (uint32_t)(p.k_st * 2) + (uint32_t)(kc * 16) +
              dsa::dead_bits(kc, p.head_dim);
      gv[j] = (uint32_t)row * (uint32_t)(p.v_st * 2) + (uint32_t)(vc * 16) +
              dsa::dead_bits(vc, p.head_dim);
    }
  }
  auto issue_gather = [&](int kb0, int kb1, int o0, unsigned char* kdst, unsigned char* vdst)
      __attribute__((always_inline)) {
    const int base0 = kb0 * p.block + o0, base1 = kb1 * p.block + o0 - p.block_pad;
    const uint32_t ks = (uint32_t)(p.k_st * 2), vs = (uint32_t)(p.v_st * 2);
    const uint32_t k0 = (uint32_t)base0 * ks, kd = (uint32_t)(base1 - base0) * ks;
    const uint32_t v0 = (uint32_t)base0 * vs, vd = (uint32_t)(base1 - base0) * vs;
    const int first_end = p.block_pad - o0;  // rows below it are in block kb0
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool first = g_r0 + 4 * j < first_end;
      lds_load16(k_all_rsrc, kdst + (wave * 4 + j) * 1024, gk[j] + k0 + (first ? 0u : kd), 0);
      lds_load16(v_all_rsrc, vdst + (wave * 4 + j) * 1024, gv[j] + v0 + (first ? 0u : vd), 0);
    }
  };
  // Valid keys of half-tile `half` of block kb (0 for an invalid block).
  auto valid_of = [&](int kb, int half) -> int {
    if (kb < 0) return 0;
    const int key0 = kb * p.block + half * kHalfKeys;
    int valid = min(kHalfKeys, p.block - half * kHalfKeys);
    return min(valid, p.kv_tokens - key0);
  };

  // Statistics weights: stream position pos (mod 2 block_pad) is tile-local
  // offset off of a tile of parity par; pad slots weigh 0.  Within each
  // 16-position group the positions are stored in the order 0-3, 8-11, 4-7,
  // 12-15, so the eight keys a lane half supplies (P^T slot order) are one
  // 16-byte read.
  const T* wrow = wtab;
  // carry: the lane's five sums of its parity's open tile, up to the chunk
  // before the current one; wprev: the last chunk's sums, which its MFMAs
  // leave for the next chunk's softmax to add (reading them in the same step
  // would hold the wave until the whole PV chain has drained).  A tile that
  // ends in a chunk is therefore closed one step later (pend_par, pend_idx),
  // or after the walk.
  float carry[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  float wprev[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  int pend_par = -1, pend_idx = 0;
  if constexpr (kStats && !kMassOnly) {
    const int bp = p.stat_pad;
    for (int i = tid; i < kStatRows * kCols; i += kWaves * 64) {
      const int r = i / kCols, si = i % kCols;
      const int pos = (si & ~12) | ((si & 4) << 1) | ((si & 8) >> 1);
      const int q2 = pos % (2 * bp);
      const int par = q2 / bp, off = q2 % bp;
      float w = 0.f;
      if (r < 10 && r / 5 == par && off < p.stat_tile) {
        const float y = dsa::tile_axis(off / p.tile_w, p.tile_h);
        const float x = dsa::tile_axis(off % p.tile_w, p.tile_w);
        const float yh = (float)(T)y, xh = (float)(T)x;
        const int kind = r % 5;
        w = kind == 0 ? 1.f : kind == 1 ? yh : kind == 2 ? xh : kind == 3 ? y - yh : x - xh;
      }
      wtab[i] = (T)w;
    }
    dsa::lds_barrier();
    // C row of lane qi's A row: 0-3 and 8 even kinds, 4-7 and 12 odd, else zero.
    wrow = wtab + (qi < 4 ? qi : qi < 8 ? qi + 1 : qi == 8 ? 4 : qi == 12 ? 9 : 10) * kCols;
  }

  float m_run = -INFINITY;
  float l_run = 0.f;
  dsa_f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;

  // NKT: 32-key sub-tiles of the half-tile that hold valid keys (2, or 1 when
  // at most 32 are valid: the last half of a 65..96-key block, or a block of
  // at most 32 keys), so empty sub-tiles cost neither MFMAs nor softmax work.
  // Gathered stream: `invalid` has bit p set when stream position p of the
  // chunk is a pad slot, past the row's last key or in an out-of-range block;
  // accumulator r of lane half g holds position 32 kt + 8 (r >> 2) + 4 g + (r & 3).
  // lim: causal bound of this lane's row, keys at or past `lim` in the
  // half-tile are masked (at least 64 when nothing is).
  auto compute = [&](const unsigned char* kt_lds, const unsigned char* v_lds, int valid,
                     int lim, uint64_t invalid, int wbase, auto nkt_c)
      __attribute__((always_inline)) {
    constexpr int NKT = decltype(nkt_c)::value;
    dsa_f32x16 sacc[NKT];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
    [[maybe_unused]] int kf = kfrag, vf = vfrag[0];
    if constexpr (kLeanAddr) asm volatile("" : "+v"(kf), "+v"(vf));
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        const int row = kt * 32 + qi;
        const unsigned char* at =
            kLeanAddr ? kt_lds + kt * 32 * kRowBytes + (kf ^ (dc << 5))
                      : kt_lds + row * kRowBytes + k2_swz(row, dc * 2 + g) * 16;
        const x8 a = *reinterpret_cast<const x8*>(at);
        sacc[kt] = E::mfma32(a, qf[dc], sacc[kt]);
      }
    }
    if constexpr (NKT == 2) {
      // Keep four K reads in flight ahead of the MFMA chain (the default
      // schedule issues two, and each MFMA then waits on LDS latency).
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
      for (int i = 0; i < 12; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    if constexpr (kPrioSoftmax) __builtin_amdgcn_s_setprio(1);
    if constexpr (kStats && kDeferSums) {
#pragma unroll
      for (int i = 0; i < 5; ++i) carry[i] += wprev[i];
    }
    if constexpr (kGather) {
      if (invalid != 0) {
        const uint64_t mine = invalid >> (4 * g);
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
          const uint32_t bits = (uint32_t)(mine >> (32 * kt));
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (bits & (1u << (8 * (r >> 2) + (r & 3)))) sacc[kt][r] = -INFINITY;
        }
      }
    } else if (valid < NKT * 32 || lim < NKT * 32) {
      // Position 32 kt + 8 (r >> 2) + 4 g + (r & 3) against the bound, with
      // the lane's 4 g moved to the bound so each test is against a literal.
      const int bound = min(valid, lim) - 4 * g;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + 8 * (r >> 2) + (r & 3) >= bound) sacc[kt][r] = -INFINITY;
    }
    // The row max only matters when the reference max may have to move: while
    // m_run >= thr in every lane, no p of the half-tile exceeds 2^bound_log2
    // and the max is not taken (a row's first half-tile, with m_run = -inf,
    // always takes it).
    const bool take_max = !kNormBound || __any(!(m_run >= thr));
    if (take_max) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
      mx = dsa::pair32_max(mx);
      const float mx2 = mx * p.scale_log2;
      float m_new = mx2 > m_run + kRescaleLog2 ? mx2 : m_run;
      bool up = mx2 > m_run + kRescaleLog2;
      if constexpr (kNormBound) {
        // Raise the reference to thr when that costs this half-tile at most
        // 2^-raise_log2 of its largest p: the bound test then holds for the
        // rest of the row.
        if (thr > m_new && thr <= mx2 + raise_log2<T>()) m_new = thr;
        up = m_new != m_run;
      }
      if (__any(up)) {
        const float alpha = up ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        if constexpr (kStats) {
#pragma unroll
          for (int i = 0; i < 5; ++i) carry[i] *= alpha;
        }
      }
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    x8 pf[2 * NKT];
    float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
    for (int j = 0; j < 2 * NKT; ++j) {
      const int kt = j >> 1, hf = j & 1;
#pragma unroll
      for (int t = 0; t < 8; t += 2) {
        const float p0 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t], p.scale_log2, -m_use));
        const float p1 =
            __builtin_amdgcn_exp2f(fmaf(sacc[kt][hf * 8 + t + 1], p.scale_log2, -m_use));
        const dsa_f32x2 two = {p0, p1};
        const typename E::x2 pb = __builtin_convertvector(two, typename E::x2);
        sum0 += p0;
        sum1 += p1;
        pf[j][t] = pb[0];
        pf[j][t + 1] = pb[1];
      }
    }
    l_run += sum0 + sum1;
    if constexpr (kMassOnly) carry[0] += sum0 + sum1;
    if constexpr (kPrioSoftmax) __builtin_amdgcn_s_setprio(0);
    if constexpr (kPrioPv) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int j = 0; j < 2 * NKT; ++j) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        // Key rows 16 j + 4 g + r (slots 0..3) and 16 j + 8 + 4 g + r (4..7).
        const unsigned char* at =
            v_lds + (kLeanAddr ? vf ^ (dt << 6) : vfrag[dt]) + j * 16 * kRowBytes;
        const typename E::x4 lo = lds_read_tr<T>(at);
        const typename E::x4 hi = lds_read_tr<T>(at + 8 * kRowBytes);
        const x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        oacc[dt] = E::mfma32(a, pf[j], oacc[dt]);
      }
    }
    if constexpr (kPrioPv) __builtin_amdgcn_s_setprio(0);
    if constexpr (kGather && NKT == 2) {
      // Gathered stream: V^T reads two per MFMA, four ahead.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
      for (int i = 0; i < 14; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
    }
    if constexpr (kStats && !kMassOnly) {
      // The key-side sums of this chunk (weights from stream position wbase).
      dsa_f32x16 wacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) wacc[r] = 0.f;
#pragma unroll
      for (int j = 0; j < 2 * NKT; ++j) {
        const x8 a = *reinterpret_cast<const x8*>(wrow + wbase + 16 * j + 8 * g);
        wacc = E::mfma32(a, pf[j], wacc);
      }
#pragma unroll
      for (int i = 0; i < 5; ++i) {
        if constexpr (kDeferSums) wprev[i] = wacc[i];
        else carry[i] += wacc[i];
      }
    }
  };

  // Fused statistics: a tile of parity par has ended; the lanes of that parity
  // write their query row's entry at `at` (when `ok`) and start the next tile
  // of that parity from zero.
  // The lane's part of an entry's index (its query row: local_row for
  // routed entries e * block + local_row, tq for dense ones) is folded into
  // per-lane pointers once; a close adds the uniform part `at`.
  float* const logm_lane = kStats ? p.rs_logm + (kRouted ? local_row : tq) : nullptr;
  uint32_t* const mean_lane =
      kStats && p.rs_mean != nullptr ? p.rs_mean + (kRouted ? local_row : tq) : nullptr;
  auto close_tile = [&](int par, int64_t at, bool ok) __attribute__((always_inline)) {
    if constexpr (kMassOnly) {
      // Both lane halves hold part of the tile's mass (their keys of each
      // half-tile): the sum of the two, written by one half.
      const float mass = dsa::pair32_sum(carry[0]);
      if (g == par && ok) logm_lane[at] = mass > 0.f ? __log2f(mass) + m_run : -INFINITY;
      carry[0] = 0.f;
      return;
    }
    if (g == par) {
      if (ok) {
        const float mass = carry[0];
        logm_lane[at] = mass > 0.f ? __log2f(mass) + m_run : -INFINITY;
        if (mean_lane != nullptr) {
          // The means are stored in fp16: the hardware reciprocal (1 ulp in
          // fp32) is exact enough.
          const float inv = mass > 0.f ? __builtin_amdgcn_rcpf(mass) : 0.f;
          const dsa_f32x2 mean = {(carry[1] + carry[3]) * inv, (carry[2] + carry[4]) * inv};
          const dsa_f16x2 hm = __builtin_convertvector(mean, dsa_f16x2);
          mean_lane[at] = __builtin_bit_cast(uint32_t, hm);
        }
      }
#pragma unroll
      for (int i = 0; i < 5; ++i) carry[i] = 0.f;
    }
  };
  // The pending close, once the sums of the chunk it ended in are in carry:
  // pend_idx is the walk index j (routed), the key block (dense tile blocks)
  // or the tile index (dense token stream).  Chunks of 64 keys end at most
  // one tile each (tiles hold 64 or more stream slots).
  auto close_pending = [&]() __attribute__((always_inline)) {
    if (pend_par < 0) return;
    if constexpr (kRouted) {
      const int64_t e = walked(pend_idx);
      close_tile(pend_par, e * p.block, row_ok && e < p.rs_entries);
    } else {
      const bool tokens = kTokenStream && p.stat_tile != p.block;
      const int64_t per_head = tokens ? p.kv_tokens / p.stat_tile : p.kv_blocks;
      close_tile(pend_par, ((int64_t)h * per_head + pend_idx) * p.q_tokens, row_ok);
    }
    pend_par = -1;
  };
  // One pipelined step: wait for the current stage, prefetch the next
  // half-tile (next_kb == -2: none), then compute on the current one
  // (skip_c: this step may hold at most 32 valid keys).
  // (j: the walk index of block kb, for the statistics of tile blocks.)
  auto step = [&](int kb, int half, int next_kb, int next_half, const unsigned char* kc,
                  const unsigned char* vc, unsigned char* kn, unsigned char* vn,
                  auto skip_c, int j) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (!kSingleStage && next_kb != -2) issue(next_kb, next_half, kn, vn);
    if (walk_at != nullptr && half == 0 && kb >= 0)
      __hip_atomic_store(walk_at, walk_entry(bh, kb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wave_active) {
      const int valid = valid_of(kb, half);
      // Causal (dense): keys past this lane's query row are masked.
      const int lim = !kRouted && p.causal ? tq - (kb * p.block + half * kHalfKeys) + 1 : kHalfKeys;
      // Statistics: tile blocks read the table from the tile's parity and
      // this half-tile's offset in it; the token stream from its first token
      // pos (keys pos .. pos + 63).
      const int pos = kb * p.block + half * kHalfKeys;
      const bool tile_blocks = !kTokenStream || p.stat_tile == p.block;
      int wbase = 0;
      if constexpr (kStats)
        wbase = tile_blocks ? (j & 1) * p.stat_pad + half * kHalfKeys : pos % (2 * p.stat_pad);
      // A skip step holds at most 32 valid keys: the kSkip instances run
      // blocks whose last half-tile has 1..32 keys (65..96-key blocks, or
      // blocks of at most 32), and only that half-tile is a skip step.  One
      // compute instance per call site keeps the O accumulators in place
      // (two, chosen at run time, made the register allocator copy them
      // on every step).
      if constexpr (decltype(skip_c)::value)
        compute(kc, vc, valid, lim, 0ull, wbase, std::integral_constant<int, 1>{});
      else
        compute(kc, vc, valid, lim, 0ull, wbase, std::integral_constant<int, 2>{});
      if constexpr (kStats) {
        if constexpr (kDeferSums) close_pending();
        if (tile_blocks) {
          // Block kb is tile j of the walk: it ends with its last half-tile.
          if (half == kNh - 1) {
            pend_par = j & 1;
            pend_idx = kRouted ? j : kb;
          }
        } else {
          // The tile ending in (pos, pos + 64] (the sequence end included), if any.
          const int m = min(pos + kHalfKeys, p.kv_tokens) / p.stat_tile;
          if (m >= 1 && m * p.stat_tile > pos) {
            pend_par = (m - 1) & 1;
            pend_idx = m - 1;
          }
        }
        if constexpr (!kDeferSums) close_pending();
      }
    }
    if constexpr (kSingleStage) {
      __syncthreads();  // every wave is done with the stage
      if (next_kb != -2) issue(next_kb, next_half, kn, vn);
    }
  };
  // Gathered stream step: chunk at slot o0 of stream block j0 (whose block
  // index is kb0; kb0 < 0 or kb1 < 0: out of range), `left` valid stream
  // slots from the chunk start to the row's last key; next_kb0 == -2: no
  // next chunk.
  // Gathered stream: stream tile j closes into its CSR entry.
  auto close_stream_tile = [&](int j) __attribute__((always_inline)) {
    const int64_t e = walked(j);
    close_tile(j & 1, e * p.block, row_ok && e < p.rs_entries);
  };
  auto step_gather = [&](int kb0, int kb1, int o0, int left, int next_kb0, int next_kb1,
                         int next_o0, const unsigned char* kc, const unsigned char* vc,
                         unsigned char* kn, unsigned char* vn, int j0, int wbase)
      __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (next_kb0 != -2)
      issue_gather(next_kb0 < 0 ? 0 : next_kb0, next_kb1 < 0 ? 0 : next_kb1, next_o0, kn, vn);
    if (walk_at != nullptr && kb0 >= 0)
      __hip_atomic_store(walk_at, walk_entry(bh, kb0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wave_active) {
      const int second = p.block_pad - o0;  // first slot of block kb1
      uint64_t invalid = 0;
      if (left < 64) invalid = ~0ull << left;
      if (p.block_pad > p.block) {
        const int lo = max(p.block - o0, 0);
        const int hi = min(second, 64);
        if (lo < hi)
          invalid |= (hi == 64 ? ~0ull : (1ull << hi) - 1) & ~((1ull << lo) - 1);
      }
      if (kb0 < 0) invalid |= second >= 64 ? ~0ull : (1ull << second) - 1;
      if (kb1 < 0 && second < 64) invalid |= ~0ull << second;
      // One compute instance only: a second, 32-key one (for a row's last
      // chunk) made the register allocator copy the O accumulators on every
      // step; the masked slots of that rare chunk cost less.
      compute(kc, vc, 0, kHalfKeys, invalid, wbase, std::integral_constant<int, 2>{});
      // Block j0 ends in this chunk (the row's last block closes after the walk).
      if constexpr (kStats) {
        if constexpr (kDeferSums) close_pending();
        if (second <= 64 && j0 + 1 < nblk) {
          pend_par = j0 & 1;
          pend_idx = j0;
        }
        if constexpr (!kDeferSums) close_pending();
      }
    }
  };
  const std::bool_constant<false> no_skip;
  const std::bool_constant<kSkip> may_skip;

  if (kGather && nblk > 0) {
    // Stream block j: CSR entry j clamped to the row (slots past the row's
    // last key are masked), -1 when out of range.
    auto gblock = [&](int j) -> int {
      const int kb = cidx[walked(j < nblk ? j : nblk - 1)];
      return (unsigned)kb < (unsigned)p.kv_blocks ? kb : -1;
    };
    const int bp = p.block_pad;
    const int total = (nblk - 1) * bp + p.block;  // slots up to the row's last key
    const int chunks = (total + 63) >> 6;
    int j0 = 0, o0 = 0;
    int w0 = 0;  // the chunk's stream position mod 2 bp (statistics weights)
    auto next_w = [&](int w) { return w + 64 >= 2 * bp ? w + 64 - 2 * bp : w + 64; };
    int kb0 = gblock(0), kb1 = gblock(1);
    issue_gather(kb0 < 0 ? 0 : kb0, kb1 < 0 ? 0 : kb1, 0, lds_k0, lds_v0);
    for (int c = 0; c < chunks; c += 2) {
      int j1 = j0, o1 = o0 + 64;
      if (o1 >= bp) { o1 -= bp; ++j1; }
      const bool more1 = c + 1 < chunks;
      const int kb0n = more1 ? gblock(j1) : -2, kb1n = more1 ? gblock(j1 + 1) : -2;
      const int w1 = next_w(w0);
      step_gather(kb0, kb1, o0, total - c * 64, kb0n, kb1n, o1, lds_k0, lds_v0, lds_k1,
                  lds_v1, j0, w0);
      if (!more1) break;
      int j2 = j1, o2 = o1 + 64;
      if (o2 >= bp) { o2 -= bp; ++j2; }
      const bool more2 = c + 2 < chunks;
      const int kb0m = more2 ? gblock(j2) : -2, kb1m = more2 ? gblock(j2 + 1) : -2;
      step_gather(kb0n, kb1n, o1, total - (c + 1) * 64, kb0m, kb1m, o2, lds_k1, lds_v1,
                  lds_k0, lds_v0, j1, w1);
      j0 = j2; o0 = o2; kb0 = kb0m; kb1 = kb1m;
      w0 = next_w(w1);
    }
  } else if (!kGather && nblk > 0) {
    int kb = block_of(0);
    issue(kb, 0, lds_k0, lds_v0);
    if (kNh == 2) {
      // The first half of a 65..128-key block always holds 64 keys (short
      // only at the sequence end, which the masked two-sub-tile path covers).
      for (int j = 0; j < nblk; ++j) {
        const int kb_after = j + 1 < nblk ? block_of(j + 1) : -2;
        step(kb, 0, kb, 1, lds_k0, lds_v0, lds_k1, lds_v1, no_skip, j);
        step(kb, 1, kb_after, 0, lds_k1, lds_v1, lds_k0, lds_v0, may_skip, j);
        kb = kb_after;
      }
    } else {
      for (int j = 0; j < nblk; j += 2) {
        const int kb1 = j + 1 < nblk ? block_of(j + 1) : -2;
        step(kb, 0, kb1, 0, lds_k0, lds_v0, kSingleStage ? lds_k0 : lds_k1,
             kSingleStage ? lds_v0 : lds_v1, may_skip, j);
        if (kb1 == -2) break;
        const int kb2 = j + 2 < nblk ? block_of(j + 2) : -2;
        step(kb1, 0, kb2, 0, kSingleStage ? lds_k0 : lds_k1, kSingleStage ? lds_v0 : lds_v1,
             lds_k0, lds_v0, may_skip, j + 1);
        kb = kb2;
      }
    }
  }
  if constexpr (kStats) {
    // The last chunk's sums, the pending close, and the gathered stream's
    // last tile (closed after the walk).
    if (wave_active && nblk > 0) {
      if constexpr (kDeferSums) {
#pragma unroll
        for (int i = 0; i < 5; ++i) carry[i] += wprev[i];
      }
      close_pending();
      if constexpr (kGather) close_stream_tile(nblk - 1);
    }
  }

  const float l_tot = dsa::pair32_sum(l_run);
  if (split) {
    if (row_ok) {
      float* po = p.part + (int64_t)(wg - p.split_from) * kPartFloats;
      float* prow = po + local_row * kHeadDim;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const dsa_f32x4 v4 = {oacc[dt][rr * 4 + 0], oacc[dt][rr * 4 + 1],
                                oacc[dt][rr * 4 + 2], oacc[dt][rr * 4 + 3]};
          *reinterpret_cast<dsa_f32x4*>(prow + dt * 32 + rr * 8 + g * 4) = v4;
        }
      if (g == 0) {
        po[128 * 128 + local_row] = m_run;
        po[128 * 128 + 128 + local_row] = l_tot;
      }
    }
    return;
  }
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok) {
    T* orow = static_cast<T*>(p.o) + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const dsa_f32x2 lo = {oacc[dt][rr * 4 + 0] * inv, oacc[dt][rr * 4 + 1] * inv};
        const dsa_f32x2 hi = {oacc[dt][rr * 4 + 2] * inv, oacc[dt][rr * 4 + 3] * inv};
        const typename E::x2 blo = __builtin_convertvector(lo, typename E::x2);
        const typename E::x2 bhi = __builtin_convertvector(hi, typename E::x2);
        const typename E::x4 v4 = {blo[0], blo[1], bhi[0], bhi[1]};
        if (dt * 32 + rr * 8 + g * 4 < p.head_dim)
          *reinterpret_cast<typename E::x4*>(orow + dt * 32 + rr * 8 + g * 4) = v4;
      }
    if (p.lse && g == 0) {
      p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
          l_tot > 0.f ? m_run * 0.6931471805599453f + logf(l_tot) : -INFINITY;
    }
  }
}

// Launch order of a routed call: within each (batch, head) group its query
// blocks by key-block count descending, ties by index ascending (a stable
// sort), so the workgroups that run side by side walk rows of similar length
// and stay in step through the L2 (a same-box A/B at config 2: 40.54 against
// 41.50 ms).  One workgroup per group: a bitonic sort of (count + 1) << 32 |
// ~index keys in LDS, padding keys 0 last.
constexpr int kMaxOrderBlocks = 8192;     // query blocks per (batch, head) group
constexpr int64_t kMaxOrderItems = 262144;  // work items per call (1 MiB of order)

// Internal linkage: each translation unit that launches it has its own copy.
// Workgroup 0 also clears the work-queue counter (when there is one).
static __global__ void __launch_bounds__(256) launch_order_kernel(const int32_t* row_ptr,
                                                           int32_t* order, int32_t heads,
                                                           int32_t q_blocks,
                                                           int32_t route_batches, int32_t n,
                                                           int32_t* queue) {
  __shared__ uint64_t keys[kMaxOrderBlocks];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  if (queue != nullptr && bh == 0 && tid == 0) queue[0] = 0;
  const int rb = route_batches == 1 ? 0 : bh / heads;
  const int32_t* rp = row_ptr + ((int64_t)rb * heads + bh % heads) * q_blocks;
  for (int i = tid; i < n; i += 256) {
    uint64_t key = 0;
    if (i < q_blocks)
      key = ((uint64_t)(uint32_t)(rp[i + 1] - rp[i] + 1) << 32) | (uint32_t)~(uint32_t)i;
    keys[i] = key;
  }
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      dsa::lds_barrier();
      for (int i = tid; i < n / 2; i += 256) {
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
  dsa::lds_barrier();
  const int32_t base = bh * q_blocks;
  for (int i = tid; i < q_blocks; i += 256)
    order[base + i] = base + (int32_t)~(uint32_t)keys[i];
}

constexpr size_t kQueueBytes = 256;

// Clears the work-queue counter of a call that has no launch order kernel.
static __global__ void __launch_bounds__(64) queue_reset_kernel(int32_t* queue) {
  if (threadIdx.x == 0) queue[0] = 0;
}

// Bytes at the front of a call's scratch: the work-queue counter (256), the
// launch order of `items` work items rounded up to 256, the aligned-walk
// table, and the key-norm maxima of `pairs` (batch, head) pairs (none above
// kMaxNormPairs: every half-tile then takes its row max); 0 when the call has
// too many items to order (it then runs in dispatch order without a queue,
// and without norms).
inline size_t round256(size_t bytes) { return (bytes + 255) & ~(size_t)255; }
inline size_t norm_bytes(int64_t pairs) {
  return pairs > kMaxNormPairs ? 0 : round256((size_t)pairs * kNormParts * sizeof(float));
}
inline size_t order_bytes(int64_t items, int32_t q_blocks, int64_t pairs) {
  if (items > kMaxOrderItems || q_blocks > kMaxOrderBlocks) return 0;
  return kQueueBytes + round256((size_t)items * sizeof(int32_t)) + kWalkBytes + norm_bytes(pairs);
}

// Key-norm maxima per (batch, head): workgroup (s, bh) takes the s-th of
// kNormParts consecutive token ranges of the head's keys, 16 lanes per key row
// (one 16-byte chunk of 8 dims each, dims past head_dim not read), and writes
// the largest norm of its range.  The attention kernels bound a half-tile's
// scores by it (compute); the bound only decides whether the row max is
// taken, so it may exceed the true largest norm but never fall below it.

template <typename T>
__global__ void __launch_bounds__(256) key_norm_kernel(BsaParams p, float* out) {
  const int part = blockIdx.x, bh = blockIdx.y;
  const int h = bh % p.heads, b = bh / p.heads;
  const int tid = threadIdx.x, c = tid & 15;
  const int per = (p.kv_tokens + kNormParts - 1) / kNormParts;
  const int t0 = part * per, t1 = min(t0 + per, p.kv_tokens);
  const T* kb = static_cast<const T*>(p.k) + b * p.k_sb + h * p.k_sh + c * 8;
  const bool live = c * 8 < p.head_dim;
  float best = 0.f;
  for (int t = t0 + (tid >> 4); t < t1; t += 16) {
    float ss = 0.f;
    if (live) {
      const typename dsa::Elem<T>::x8 x =
          *reinterpret_cast<const typename dsa::Elem<T>::x8*>(kb + (int64_t)t * p.k_st);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf((float)x[e], (float)x[e], ss);
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m);
    best = fmaxf(best, ss);
  }
  best = fmaxf(best, __shfl_xor(best, 16));
  best = fmaxf(best, __shfl_xor(best, 32));
  __shared__ float wave_max[4];
  if ((tid & 63) == 0) wave_max[tid >> 6] = best;
  __syncthreads();
  if (tid == 0)
    out[(int64_t)bh * kNormParts + part] =
        sqrtf(fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3])));
}

// Combines the `parts` partials of each split query block: with M the largest
// row max, O = sum_i O_i 2^(m_i - M) / sum_i l_i 2^(m_i - M) and
// LSE = M ln 2 + ln(sum_i l_i 2^(m_i - M)).  Two threads per row, 64 dims each.
template <typename T>
__global__ void __launch_bounds__(256) bsa_merge_kernel(BsaParams p) {
  const int item = blockIdx.x;
  const int work = p.order ? p.order[p.split_from + item] : p.split_from + item;
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;
  const int r = threadIdx.x >> 1, half = threadIdx.x & 1;
  const int tq = qb * p.block + r;
  if (r >= p.block || tq >= p.q_tokens) return;
  const float* base = p.part + (int64_t)item * p.parts * kPartFloats;
  float m_max = -INFINITY;
  for (int i = 0; i < p.parts; ++i) m_max = fmaxf(m_max, base[i * kPartFloats + 128 * 128 + r]);
  float w[8];
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w[i] = 0.f;
    if (i < p.parts) {
      const float m_i = base[i * kPartFloats + 128 * 128 + r];
      w[i] = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - m_max);
      l = fmaf(w[i], base[i * kPartFloats + 128 * 128 + 128 + r], l);
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = static_cast<T*>(p.o) + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
  for (int c = half * 8; c < half * 8 + 8; ++c) {  // 8-dim chunks of this thread's 64
    if (c * 8 >= p.head_dim) break;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i >= p.parts) break;
      const float* src = base + i * kPartFloats + r * kHeadDim + c * 8;
      const dsa_f32x4 a = *reinterpret_cast<const dsa_f32x4*>(src);
      const dsa_f32x4 bq = *reinterpret_cast<const dsa_f32x4*>(src + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] = fmaf(w[i], a[e], acc[e]);
        acc[4 + e] = fmaf(w[i], bq[e], acc[4 + e]);
      }
    }
    typename dsa::Elem<T>::x8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (T)(acc[e] * inv);
    *reinterpret_cast<typename dsa::Elem<T>::x8*>(orow + c * 8) = out;
  }
  if (p.lse && half == 0)
    p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
        l > 0.f ? m_max * 0.6931471805599453f + logf(l) : -INFINITY;
}

inline bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

constexpr int kMaxDevices = 64;

// The device `stream` belongs to (the current device for the null stream), or
// -1 when it cannot be told.
inline int stream_device(hipStream_t stream) {
  int device = -1;
  if (stream == nullptr || hipStreamGetDevice(stream, &device) != hipSuccess) {
    if (hipGetDevice(&device) != hipSuccess) return -1;
  }
  return device >= 0 && device < kMaxDevices ? device : -1;
}

// Workgroup slots (two attention workgroups per CU) of the stream's device,
// cached per device.
inline int device_slots(hipStream_t stream) {
  static int slots[kMaxDevices] = {0};
  const int device = stream_device(stream);
  if (device < 0) return 0;
  if (slots[device] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return 0;
    slots[device] = 2 * cus;
  }
  return slots[device];
}

// Split of the last round: the last k of n query blocks each run as `parts`
// key ranges, chosen to minimise the predicted time in rounds of one
// workgroup's time, (n - k) / slots + ceil(parts k / slots) / parts, over k =
// n mod slots (or that plus one round) and 2..max_parts parts, at most
// max_groups split workgroups.  Returns k (0: no split).
inline int choose_split(int64_t n, int slots, int max_parts, int64_t max_groups, int* parts) {
  *parts = 1;
  if (slots <= 0 || n <= 0 || max_parts < 2) return 0;
  const int64_t rem = n % slots;
  if (rem == 0) return 0;
  double best = (double)((n + slots - 1) / slots) - 0.05;  // split only for a clear gain
  int best_k = 0;
  for (int extra = 0; extra <= 1; ++extra) {
    const int64_t k = rem + (int64_t)extra * slots;
    if (k > n) break;
    for (int pp = 2; pp <= max_parts; ++pp) {
      if (k * pp > max_groups) break;
      const double t = (double)((n - k) / slots) +
                       (double)((k * pp + slots - 1) / slots) / (double)pp;
      if (t < best) {
        best = t;
        best_k = (int)k;
        *parts = pp;
      }
    }
  }
  if (best_k == 0) *parts = 1;
  return best_k;
}

// Parts a split query block may take: at least 8 key blocks per part of the
// whole key range (short ranges, such as 512 text tokens, gain less than the
// merge costs), at most 8.
inline int max_parts_for(int32_t kv_blocks) { return std::min(8, kv_blocks / 8); }

constexpr size_t kPartBytes = sizeof(float) * kPartFloats;

// Routed calls take the gathered key stream when every key block is whole and
// holds 65..127 keys and its 8-rounded size is below the plain layout's slots
// per block (64 + 32 up to 96 keys, else 128), and the whole K and V
// sequences of one head each span < 2 GiB (one buffer resource addresses each).
inline bool gather_blocks(int32_t block, int32_t kv_tokens) {
  if (block <= kHalfKeys || block >= 2 * kHalfKeys || kv_tokens % block != 0) return false;
  const int32_t pad = (block + 7) & ~7;
  const int32_t plain = block - kHalfKeys <= 32 ? kHalfKeys + 32 : 2 * kHalfKeys;
  return pad < plain;
}

inline bool use_gather(int32_t block, int32_t kv_tokens, int64_t k_token_stride,
                int64_t v_token_stride) {
  if (!gather_blocks(block, kv_tokens)) return false;
  const int64_t stride = std::max(k_token_stride, v_token_stride);
  return ((int64_t)kv_tokens + 8) * stride * 2 + kRowBytes <= 0x7fffffff;
}

// Launches a prepared call.  `scratch` (null when `scratch_bytes` is 0)
// holds, when there is room for them (order_bytes), the work-queue counter
// and, for a routed call, the launch order and the aligned-walk table; then
// the split partials of the last round.
template <typename T>
int launch_typed(BsaParams p, void* scratch, size_t scratch_bytes, hipStream_t stream,
                 const char* who) {
  const int64_t grid = (int64_t)p.batch * p.heads * p.q_blocks;
  size_t used = 0;
  p.order = nullptr;
  p.walk = nullptr;
  p.queue = nullptr;
  p.kv_norm = nullptr;
  const int64_t norms = (int64_t)p.batch * p.heads;
  const size_t lead = order_bytes(grid, p.q_blocks, norms);
  const int32_t nh = p.block > kHalfKeys ? 2 : 1;
  // Blocks whose last half-tile holds 1..32 keys run it as one sub-tile.
  const int rem = p.block % kHalfKeys;
  const bool skip = rem != 0 && rem <= 32;
  const bool gather = p.row_ptr && use_gather(p.block, p.kv_tokens, p.k_st, p.v_st);
  // Resident workgroups: two per CU, four for the single-stage 2-wave ones
  // (routed blocks, or dense statistics, of at most 64 keys).
  const bool two_wave = nh == 1 && (p.row_ptr || p.rs_logm);
  const int slots = device_slots(stream) * (two_wave ? 2 : 1);
  if (lead > 0 && scratch_bytes >= lead) {
    unsigned char* base = static_cast<unsigned char*>(scratch);
    used = lead;
    unsigned char* const walk_end = base + lead - norm_bytes(norms);
    if (norm_bytes(norms) > 0 && (gather || !skip)) {
      float* kv_norm = reinterpret_cast<float*>(walk_end);
      hipLaunchKernelGGL(key_norm_kernel<T>, dim3(kNormParts, (unsigned)norms), dim3(256), 0,
                         stream, p, kv_norm);
      p.kv_norm = kv_norm;
    }
    // Calls of more than one round of workgroups take their slots from the
    // work queue.
    if (grid > slots) p.queue = reinterpret_cast<int32_t*>(base);
    if (p.row_ptr) {
      int32_t* order = reinterpret_cast<int32_t*>(base + kQueueBytes);
      p.order = order;
      // The walk table needs no clearing: stale entries are too old to count
      // and any entry only moves where a row's walk starts.
      if (!p.deterministic && p.kv_blocks <= kWalkMaxBlocks)
        p.walk = reinterpret_cast<uint64_t*>(walk_end - kWalkBytes);
      int n = 2;
      while (n < p.q_blocks) n <<= 1;
      hipLaunchKernelGGL(launch_order_kernel, dim3((unsigned)(p.batch * p.heads)), dim3(256), 0,
                         stream, p.row_ptr, order, p.heads, p.q_blocks, p.route_batches, n,
                         p.queue);
    } else if (p.queue) {
      hipLaunchKernelGGL(queue_reset_kernel, dim3(1), dim3(64), 0, stream, p.queue);
    }
  }
  float* part = reinterpret_cast<float*>(static_cast<unsigned char*>(scratch) + used);
  // Statistics of tile blocks: the tile's slots in the stream.
  if (p.rs_logm && p.stat_tile == p.block) p.stat_pad = gather ? p.block_pad : nh * kHalfKeys;
  // The tiles of a dense token stream need not align with the split's key
  // ranges: such calls run unsplit (tile blocks always align).
  const int64_t part_groups = p.rs_logm && !p.row_ptr && p.stat_tile != p.block
                                  ? 0
                                  : (int64_t)((scratch_bytes - used) / kPartBytes);
  int parts = 1;
  const int split = choose_split(grid, slots, max_parts_for(p.kv_blocks),
                                 std::min<int64_t>(part_groups, kMaxPartGroups), &parts);
  p.split_from = (int32_t)(grid - split);
  p.parts = parts;
  p.part = part;
  const dim3 blocks((unsigned)(grid - split + (int64_t)split * parts)), threads(256),
      two_waves(128);
  auto four = [&](auto kernel) { hipLaunchKernelGGL(kernel, blocks, threads, 0, stream, p); };
  auto two = [&](auto kernel) { hipLaunchKernelGGL(kernel, blocks, two_waves, 0, stream, p); };
  if (gather) {
    if (p.rs_logm) four(bsa_fwd_kernel<T, true, 2, true, true, 4, true>);
    else four(bsa_fwd_kernel<T, true, 2, true, true>);
  } else if (p.row_ptr && p.rs_logm) {
    if (nh == 2)
      skip ? four(bsa_fwd_kernel<T, true, 2, true, false, 4, true>)
           : four(bsa_fwd_kernel<T, true, 2, false, false, 4, true>);
    else skip ? two(bsa_fwd_kernel<T, true, 1, true, false, 2, true>)
              : two(bsa_fwd_kernel<T, true, 1, false, false, 2, true>);
  } else if (p.row_ptr) {
    if (nh == 2) skip ? four(bsa_fwd_kernel<T, true, 2, true>) : four(bsa_fwd_kernel<T, true, 2, false>);
    else skip ? two(bsa_fwd_kernel<T, true, 1, true, false, 2>)
              : two(bsa_fwd_kernel<T, true, 1, false, false, 2>);
  } else if (p.rs_logm) {
    // Dense statistics: 128-token blocks (the token stream, or tiles of 128),
    // or blocks of one tile each, in 2-wave workgroups up to 64 tokens.
    if (nh == 2 && !skip && p.rs_mean == nullptr && p.stat_tile == p.block)
      four(bsa_fwd_kernel<T, false, 2, false, false, 4, true, true>);
    else if (nh == 2)
      skip ? four(bsa_fwd_kernel<T, false, 2, true, false, 4, true>)
           : four(bsa_fwd_kernel<T, false, 2, false, false, 4, true>);
    else skip ? two(bsa_fwd_kernel<T, false, 1, true, false, 2, true>)
              : two(bsa_fwd_kernel<T, false, 1, false, false, 2, true>);
  } else {
    if (nh == 2) skip ? four(bsa_fwd_kernel<T, false, 2, true>) : four(bsa_fwd_kernel<T, false, 2, false>);
    else skip ? four(bsa_fwd_kernel<T, false, 1, true>) : four(bsa_fwd_kernel<T, false, 1, false>);
  }
  if (split > 0)
    hipLaunchKernelGGL(bsa_merge_kernel<T>, dim3((unsigned)split), dim3(256), 0, stream, p);
  return dsa::check_launch(who);
}

}  // namespace bsa

// fp16 instances (bsa_fwd_f16.hip).
int bsa_launch_f16(bsa::BsaParams p, void* scratch, size_t scratch_bytes, hipStream_t stream,
                   const char* who);
// fp32-compute kernel (bsa_fwd_f32.hip): fp32 inputs (dtype DSA_F32), dense
// calls with dropout, and head dims 136..256, of any input type.
int bsa_launch_f32(bsa::BsaParams p, int32_t dtype, hipStream_t stream, const char* who);
