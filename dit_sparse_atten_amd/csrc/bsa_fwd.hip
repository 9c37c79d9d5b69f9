// C-ABI entry points of the block-sparse attention forward (gfx950), and the
// bf16 kernel instances; the kernels are in bsa_kernel.h, the fp16 instances
// in bsa_fwd_f16.hip.
//
// Replaces the FlexAttention call of the reference backend
// (attention_backends/flex.py:379-399 `_flex_output`, kernel options
// flex.py:360-364) and its dense SDPA fallback (attention_backends/dense.py:14-48).
#include <cmath>
#include <hip/hip_fp16.h>
#include <mutex>

#include "bsa_kernel.h"

using namespace bsa;

namespace {

int prepare(const void* q, const void* k, const void* v, void* o, int32_t dtype,
            const int64_t* strides,
            int32_t batch, int32_t q_tokens, int32_t kv_tokens, int32_t heads,
            int32_t head_dim, int32_t block_size, const int32_t* row_ptr,
            const int32_t* col_idx, int32_t route_batches, float scale, int32_t causal,
            int32_t deterministic, float* lse, const char* who, BsaParams* p) {
  if (!q || !k || !v || !o || !strides)
    return dsa::set_error(DSA_EINVAL, "%s: null tensor or stride pointer", who);
  if (dtype != DSA_BF16 && dtype != DSA_F16 && dtype != DSA_F32)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: dtype %d unsupported (bf16, fp16 or fp32)", who,
                          dtype);
  if (batch <= 0 || heads <= 0 || q_tokens <= 0 || kv_tokens <= 0)
    return dsa::set_error(DSA_EINVAL, "%s: batch/heads/tokens must be positive", who);
  if (head_dim <= 0 || head_dim > 2 * kHeadDim || head_dim % 8 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "%s: head_dim %d unsupported (a multiple of 8 up to 256)", who, head_dim);
  if (causal != 0 && causal != 1)
    return dsa::set_error(DSA_EINVAL, "%s: causal must be 0 or 1", who);
  if (deterministic != 0 && deterministic != 1)
    return dsa::set_error(DSA_EINVAL, "%s: deterministic must be 0 or 1", who);
  if (causal && row_ptr)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: causal attention takes no block route", who);
  if (block_size <= 0 || block_size > 128)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: block_size %d unsupported (1..128)", who,
                          block_size);
  if ((row_ptr == nullptr) != (col_idx == nullptr))
    return dsa::set_error(DSA_EINVAL, "%s: row_ptr and col_idx must both be set or null", who);
  if (row_ptr && route_batches != 1 && route_batches != batch)
    return dsa::set_error(DSA_EINVAL, "%s: route_batches must be 1 or batch", who);
  if (row_ptr && q_tokens != kv_tokens)
    return dsa::set_error(DSA_EINVAL, "%s: a block route needs q_tokens == kv_tokens", who);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return dsa::set_error(DSA_EINVAL, "%s: scale must be positive and finite", who);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return dsa::set_error(DSA_EINVAL, "%s: tensors must be 16-byte aligned", who);
  for (int i = 0; i < 12; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return dsa::set_error(DSA_EINVAL,
                            "%s: stride %d (=%lld) is not a non-negative multiple of 8 "
                            "elements", who, i, (long long)strides[i]);
  if (strides[4] * (int64_t)(2 * 64) > 0x7fffffff || strides[7] * (int64_t)(2 * 64) > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "%s: key/value token stride too large (64 rows must span < 2 GiB)", who);
  const int32_t q_blocks = (q_tokens + block_size - 1) / block_size;
  const int32_t kv_blocks = (kv_tokens + block_size - 1) / block_size;
  const int64_t grid = (int64_t)batch * heads * q_blocks;
  if (grid > 0x3fffffff || (int64_t)batch * heads > 65535)
    return dsa::set_error(DSA_EINVAL, "%s: grid too large", who);
  p->q = q;
  p->k = k;
  p->v = v;
  p->o = o;
  p->lse = lse;
  p->q_sb = strides[0]; p->q_st = strides[1]; p->q_sh = strides[2];
  p->k_sb = strides[3]; p->k_st = strides[4]; p->k_sh = strides[5];
  p->v_sb = strides[6]; p->v_st = strides[7]; p->v_sh = strides[8];
  p->o_sb = strides[9]; p->o_st = strides[10]; p->o_sh = strides[11];
  p->row_ptr = row_ptr;
  p->col_idx = col_idx;
  p->batch = batch; p->heads = heads; p->q_tokens = q_tokens; p->kv_tokens = kv_tokens;
  p->q_blocks = q_blocks; p->kv_blocks = kv_blocks;
  p->route_batches = row_ptr ? route_batches : 1;
  p->block = block_size;
  p->block_pad = (block_size + 7) & ~7;
  p->head_dim = head_dim;
  p->causal = causal;
  p->deterministic = deterministic;
  p->rs_logm = nullptr;
  p->rs_mean = nullptr;
  p->rs_entries = 0;
  p->tile_h = p->tile_w = 0;
  p->stat_tile = p->stat_pad = 0;
  p->drop_thresh = 0;
  p->drop_scale = 1.f;
  p->drop_seed_lo = p->drop_seed_hi = p->drop_offset = 0;
  p->scale = scale;
  p->scale_log2 = scale * 1.4426950408889634f;
  return DSA_OK;
}

// Launches the attention of a prepared call on `scratch_bytes` of scratch
// (launch order, then split partials; see launch_typed).
int launch(int32_t dtype, BsaParams p, void* scratch, size_t scratch_bytes, hipStream_t stream,
           const char* who) {
  // fp32 inputs, dropout and head dims above 128 run the fp32-compute kernel
  // (no scratch).
  if (dtype == DSA_F32 || p.drop_thresh != 0 || p.head_dim > kHeadDim)
    return bsa_launch_f32(p, dtype, stream, who);
  return dtype == DSA_F16 ? bsa_launch_f16(p, scratch, scratch_bytes, stream, who)
                          : launch_typed<__bf16>(p, scratch, scratch_bytes, stream, who);
}

}  // namespace

// Scratch of dsa_bsa_fwd_noalloc: the work-queue counter (256 bytes), the
// launch order of up to kMaxOrderItems work items (1 MiB), the aligned-walk
// table (4 KiB) and the key-norm maxima of up to kMaxNormPairs (batch, head)
// pairs (1 MiB), then kMaxPartGroups split partials (68,157,440 bytes).
// Every device the library runs on holds its own copy until the process
// ends; host code reaches it only through the address hipGetSymbolAddress
// returns on that device (scratch_on).
constexpr size_t kScratchBytes = kQueueBytes + (size_t)kMaxOrderItems * sizeof(int32_t) +
                                 kWalkBytes + (size_t)kMaxNormPairs * kNormParts * sizeof(float) +
                                 (size_t)kMaxPartGroups * kPartBytes;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

std::mutex g_scratch_lock;
void* g_scratch[kMaxDevices] = {};

// Device address of `device`'s scratch array, resolved once per device with
// that device current.
int scratch_on(int device, void** out, const char* who) {
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch[device] == nullptr) {
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess)
      return dsa::set_error(DSA_ELAUNCH, "%s: no current HIP device", who);
    if (current != device && hipSetDevice(device) != hipSuccess)
      return dsa::set_error(DSA_ELAUNCH, "%s: cannot select device %d", who, device);
    void* address = nullptr;
    const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (current != device) (void)hipSetDevice(current);
    if (err != hipSuccess || address == nullptr)
      return dsa::set_error(DSA_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s",
                            who, device, hipGetErrorString(err));
    g_scratch[device] = address;
  }
  *out = g_scratch[device];
  return DSA_OK;
}

}  // namespace

namespace {

// Cells of the fused statistics: one workgroup per (head, query tile) row.
// For each key tile the row lists (every tile when dense), query row r of the tile contributes
// w_r = 2^(rs_logm - lse_r log2 e), its probability mass on that key tile:
//   mass = sum w_r, q_y = sum w_r y(r), q_x = sum w_r x(r),
//   k_y = sum w_r mean_y, k_x = sum w_r mean_x,
// each summed in a fixed order (eight lanes per listed tile, then a
// three-step exchange).  Outputs as dsa_tile_stats writes them: mass / tokens (fp32,
// fp16) and the centroids moment / max(mass, 1e-12) (fp16); cells the row
// does not list are zero.
struct ReduceParams {
  const float* rs_logm;
  const uint32_t* rs_mean;
  int64_t entries;
  const float* lse;  // [heads, tokens]
  const int32_t* row_ptr;
  const int32_t* col_idx;
  float* mass32;
  __half* mass16;
  __half* cqy;
  __half* cqx;
  __half* cky;
  __half* ckx;
  int32_t tokens, tiles, tile, tile_h, tile_w;
  int32_t dense;  // 1: every key tile, rows at (h * tiles + kt) * tokens + token
  int32_t raw;    // 1: mass32 holds the plain sum (the exact block mass), not sum / tokens,
                  // and rs_mean is absent
};

__global__ void __launch_bounds__(256) tile_stats_reduce_kernel(ReduceParams p) {
  __shared__ float lse2[128], uy[128], ux[128];
  const int tid = threadIdx.x, lane = tid & 63;
  const int row = blockIdx.x;
  const int h = row / p.tiles, qt = row % p.tiles;
  // Rows past the tile read zeros (their log-masses are -inf).
  for (int i = tid; i < 128; i += 256) {
    const bool in = i < p.tile;
    lse2[i] = in ? p.lse[(int64_t)h * p.tokens + (int64_t)qt * p.tile + i] * 1.4426950408889634f
                 : 0.f;
    uy[i] = in ? dsa::tile_axis(i / p.tile_w, p.tile_h) : 0.f;
    ux[i] = in ? dsa::tile_axis(i % p.tile_w, p.tile_w) : 0.f;
  }
  const int64_t cell0 = (int64_t)row * p.tiles;
  if (p.dense) {
    // Every cell of the row is listed and written below.
    dsa::lds_barrier();
  } else {
    const __half zero = __float2half(0.f);
    for (int kt = tid; kt < p.tiles; kt += 256) {
      p.mass32[cell0 + kt] = 0.f;
      if (p.mass16) p.mass16[cell0 + kt] = zero;
      if (p.cqy) p.cqy[cell0 + kt] = zero;
      if (p.cqx) p.cqx[cell0 + kt] = zero;
      if (p.cky) p.cky[cell0 + kt] = zero;
      if (p.ckx) p.ckx[cell0 + kt] = zero;
    }
    // The zeros land before the listed cells are written (vmcnt(0) barrier).
    dsa::lds_barrier<true>();
  }
  const int start = p.dense ? 0 : p.row_ptr[row];
  const int end = p.dense ? p.tiles : (int)min((int64_t)p.row_ptr[row + 1], p.entries);
  // kGroup lanes reduce one listed cell (lane j of the group takes the rows
  // j, j + kGroup, ...), so a wave has 64 / kGroup cells' row loads in flight
  // at once and combines each cell's five sums in log2(kGroup) exchange
  // steps.  The summation order is fixed: per lane in row order, then the
  // exchange tree.
  constexpr int kGroup = 8;
  constexpr int kRowsPerLane = 128 / kGroup;
  const int sub = lane % kGroup;
  const int groups = 256 / kGroup;
  for (int e = start + tid / kGroup; e - (int)(tid / kGroup) < end; e += groups) {
    const int kt = e < end ? (p.dense ? e : p.col_idx[e]) : -1;
    const bool ok = (unsigned)kt < (unsigned)p.tiles;
    const int64_t at0 = p.dense ? ((int64_t)h * p.tiles + kt) * p.tokens + (int64_t)qt * p.tile
                                : (int64_t)e * p.tile;
    // Every row load of the lane is issued before the first is used.
    float lg[kRowsPerLane];
    uint32_t mn[kRowsPerLane];
#pragma unroll
    for (int i = 0; i < kRowsPerLane; ++i) {
      const int r = sub + i * kGroup;
      const bool in = ok && r < p.tile;
      lg[i] = in ? p.rs_logm[at0 + r] : -INFINITY;
      mn[i] = in && !p.raw ? p.rs_mean[at0 + r] : 0u;
    }
    float m = 0.f, qy = 0.f, qx = 0.f, ky = 0.f, kx = 0.f;
#pragma unroll
    for (int i = 0; i < kRowsPerLane; ++i) {
      const int r = sub + i * kGroup;
      const float w = __builtin_amdgcn_exp2f(lg[i] - lse2[r]);
      const dsa_f16x2 mean = __builtin_bit_cast(dsa_f16x2, mn[i]);
      m += w;
      qy = fmaf(w, uy[r], qy);
      qx = fmaf(w, ux[r], qx);
      ky = fmaf(w, (float)mean[0], ky);
      kx = fmaf(w, (float)mean[1], kx);
    }
#pragma unroll
    for (int off = 1; off < kGroup; off <<= 1) {
      m += __shfl_xor(m, off);
      qy += __shfl_xor(qy, off);
      qx += __shfl_xor(qx, off);
      ky += __shfl_xor(ky, off);
      kx += __shfl_xor(kx, off);
    }
    if (ok && sub == 0) {
      const int64_t cell = cell0 + kt;
      const float normalized = p.raw ? m : m / (float)p.tokens;
      const float den = fmaxf(m, 1e-12f);
      p.mass32[cell] = normalized;
      if (p.mass16) p.mass16[cell] = __float2half(normalized);
      if (p.cqy) p.cqy[cell] = __float2half(qy / den);
      if (p.cqx) p.cqx[cell] = __float2half(qx / den);
      if (p.cky) p.cky[cell] = __float2half(ky / den);
      if (p.ckx) p.ckx[cell] = __float2half(kx / den);
    }
  }
}

// Bytes of the fused per-row statistics of `entries` CSR entries of `tile`
// query rows (fp32 log-mass and two fp16 means each), rounded up to 256.
size_t row_stats_bytes(int64_t entries, int32_t tile) {
  return ((size_t)entries * tile * 2 * sizeof(float) + 255) & ~(size_t)255;
}

// The same with the log-masses only (the exact block mass).
size_t row_mass_bytes(int64_t entries, int32_t tile) {
  return ((size_t)entries * tile * sizeof(float) + 255) & ~(size_t)255;
}

// Dense statistics calls of 64..128-token tiles that are a multiple of 8 run
// the attention on 128-token blocks: each 64-key step then holds at most one
// tile end and starts 16-aligned in the weight table's period of two tiles.
// Other dense calls, and routed ones, run blocks of one tile each.
bool token_stream(int32_t tile) { return tile >= kHalfKeys && tile % 8 == 0; }


}  // namespace

extern "C" size_t dsa_bsa_workspace_bytes_block(int32_t batch, int32_t heads,
                                                int32_t kv_tokens, int32_t head_dim,
                                                int32_t block_size) {
  if (batch <= 0 || heads <= 0 || kv_tokens <= 0 || head_dim <= 0) return 0;
  if (block_size <= 0 || block_size > 128) return 0;
  const int32_t kv_blocks = (kv_tokens + block_size - 1) / block_size;
  // Routed calls are self-attention (q_tokens == kv_tokens): batch x heads x
  // kv_blocks work items to order.
  const size_t order =
      order_bytes((int64_t)batch * heads * kv_blocks, kv_blocks, (int64_t)batch * heads);
  return order + (max_parts_for(kv_blocks) >= 2 ? (size_t)kMaxPartGroups * kPartBytes : 0);
}

extern "C" size_t dsa_bsa_workspace_bytes(int32_t batch, int32_t heads, int32_t kv_tokens,
                                          int32_t head_dim) {
  return dsa_bsa_workspace_bytes_block(batch, heads, kv_tokens, head_dim, 128);
}

extern "C" int dsa_bsa_fwd(const void* q, const void* k, const void* v, void* o,
                           int32_t dtype, const int64_t* strides, int32_t batch, int32_t q_tokens,
                           int32_t kv_tokens, int32_t heads, int32_t head_dim,
                           int32_t block_size, const int32_t* row_ptr,
                           const int32_t* col_idx, int32_t route_batches, float scale,
                           int32_t causal, int32_t deterministic, float* lse, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  dsa::clear_error();
  BsaParams p;
  const int status = prepare(q, k, v, o, dtype, strides, batch, q_tokens, kv_tokens, heads, head_dim,
                             block_size, row_ptr, col_idx, route_batches, scale, causal,
                             deterministic, lse, "dsa_bsa_fwd", &p);
  if (status != DSA_OK) return status;
  if (workspace_bytes > 0 && (!workspace || !aligned16(workspace)))
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd: workspace must be 16-byte aligned");
  return launch(dtype, p, workspace, workspace ? workspace_bytes : 0, stream, "dsa_bsa_fwd");
}

extern "C" int dsa_bsa_fwd_noalloc(const void* q, const void* k, const void* v, void* o,
                                   int32_t dtype, const int64_t* strides, int32_t batch, int32_t q_tokens,
                                   int32_t kv_tokens, int32_t heads, int32_t head_dim,
                                   int32_t block_size, const int32_t* row_ptr,
                                   const int32_t* col_idx, int32_t route_batches, float scale,
                                   int32_t causal, int32_t deterministic, float* lse,
                                   hipStream_t stream) {
  dsa::clear_error();
  BsaParams p;
  const int status = prepare(q, k, v, o, dtype, strides, batch, q_tokens, kv_tokens, heads, head_dim,
                             block_size, row_ptr, col_idx, route_batches, scale, causal,
                             deterministic, lse, "dsa_bsa_fwd_noalloc", &p);
  if (status != DSA_OK) return status;
  const int device = stream_device(stream);
  if (device < 0)
    return dsa::set_error(DSA_EINVAL, "dsa_bsa_fwd_noalloc: cannot tell the stream's device");
  void* area = nullptr;
  const int found = scratch_on(device, &area, "dsa_bsa_fwd_noalloc");
  if (found != DSA_OK) return found;
  // Calls of more work items than the order region holds run in launch
  // order, as dsa_bsa_fwd does; the split never takes more partials than the
  // array holds.  So no call size needs more scratch than this.
  return launch(dtype, p, area, kScratchBytes, stream, "dsa_bsa_fwd_noalloc");
}

extern "C" int dsa_bsa_fwd_dropout(const void* q, const void* k, const void* v, void* o,
                                   int32_t dtype, const int64_t* strides, int32_t batch,
                                   int32_t q_tokens, int32_t kv_tokens, int32_t heads,
                                   int32_t head_dim, float scale, int32_t causal, float dropout_p,
                                   uint64_t seed, uint32_t offset, float* lse,
                                   hipStream_t stream) {
  const char* who = "dsa_bsa_fwd_dropout";
  dsa::clear_error();
  if (!(dropout_p > 0.f && dropout_p < 1.f))
    return dsa::set_error(DSA_EINVAL, "%s: dropout_p must be in (0, 1), got %g", who,
                          (double)dropout_p);
  BsaParams p;
  const int status = prepare(q, k, v, o, dtype, strides, batch, q_tokens, kv_tokens, heads,
                             head_dim, 128, nullptr, nullptr, 1, scale, causal, 1, lse, who, &p);
  if (status != DSA_OK) return status;
  // keep = (u >= round(dropout_p 2^32)), at least 1 (no uniform is below 0).
  const double thresh = std::nearbyint((double)dropout_p * 4294967296.0);
  p.drop_thresh = (uint32_t)std::min(std::max(thresh, 1.0), 4294967295.0);
  p.drop_scale = 1.f / (1.f - dropout_p);
  p.drop_seed_lo = (uint32_t)(seed & 0xffffffffu);
  p.drop_seed_hi = (uint32_t)(seed >> 32);
  p.drop_offset = offset;
  return launch(dtype, p, nullptr, 0, stream, who);
}

extern "C" size_t dsa_bsa_fwd_tile_stats_workspace_bytes(int32_t heads, int32_t tokens,
                                                         int32_t head_dim, int32_t tile_h,
                                                         int32_t tile_w, int64_t entries) {
  if (heads <= 0 || tokens <= 0 || head_dim <= 0 || tile_h <= 0 || tile_w <= 0 || entries < 0)
    return 0;
  if ((int64_t)tile_h * tile_w > 128) return 0;
  const int32_t tile = tile_h * tile_w;
  if (tokens % tile != 0) return 0;
  // The attention runs on blocks of one tile, or (dense, token_stream) on
  // 128-token blocks; every call writes the per-row statistics.
  size_t attention = dsa_bsa_workspace_bytes_block(1, heads, tokens, head_dim, tile);
  if (token_stream(tile))
    attention = std::max(attention, dsa_bsa_workspace_bytes_block(1, heads, tokens, head_dim, 128));
  return attention + row_stats_bytes(entries, tile);
}

extern "C" int dsa_bsa_fwd_tile_stats(const void* q, const void* k, const void* v, void* o,
                                      int32_t dtype, const int64_t* strides, int32_t tokens,
                                      int32_t heads, int32_t head_dim, int32_t tile_h,
                                      int32_t tile_w, const int32_t* row_ptr,
                                      const int32_t* col_idx, int64_t entries, float scale,
                                      int32_t deterministic, float* lse, float* mass,
                                      void* mass_f16, void* centroid_q_y, void* centroid_q_x,
                                      void* centroid_k_y, void* centroid_k_x, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream) {
  const char* who = "dsa_bsa_fwd_tile_stats";
  dsa::clear_error();
  if (!lse || !mass || !strides)
    return dsa::set_error(DSA_EINVAL, "%s: lse, mass and strides are required", who);
  if ((row_ptr == nullptr) != (col_idx == nullptr))
    return dsa::set_error(DSA_EINVAL, "%s: row_ptr and col_idx must both be set or null", who);
  if (tile_h <= 0 || tile_w <= 0 || (int64_t)tile_h * tile_w > 128)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: tile %dx%d unsupported (1..128 tokens)", who,
                          tile_h, tile_w);
  const int32_t tile = tile_h * tile_w;
  if (tokens <= 0 || tokens % tile != 0)
    return dsa::set_error(DSA_EINVAL, "%s: %d tokens are not whole %d-token tiles", who, tokens,
                          tile);
  if (entries < 0) return dsa::set_error(DSA_EINVAL, "%s: entries must be >= 0", who);
  const int32_t tiles = tokens / tile;
  const bool dense = row_ptr == nullptr;
  if (dense && entries < (int64_t)heads * tiles * tiles)
    return dsa::set_error(DSA_EINVAL, "%s: dense statistics need entries >= heads * tiles^2",
                          who);
  // (The fp32-compute kernel, which also runs head dims above 128, always
  // runs blocks of one tile.)
  const bool blocks128 = dense && dtype != DSA_F32 && head_dim <= kHeadDim && token_stream(tile);
  BsaParams p;
  int status = prepare(q, k, v, o, dtype, strides, 1, tokens, tokens, heads, head_dim,
                       blocks128 ? 128 : tile, row_ptr, col_idx, 1, scale, 0, deterministic, lse, who,
                       &p);
  if (status != DSA_OK) return status;
  if (workspace_bytes > 0 && (!workspace || !aligned16(workspace)))
    return dsa::set_error(DSA_EINVAL, "%s: workspace must be 16-byte aligned", who);
  const size_t need = dsa_bsa_fwd_tile_stats_workspace_bytes(heads, tokens, head_dim, tile_h,
                                                             tile_w, entries);
  if (workspace_bytes < need)
    return dsa::set_error(DSA_EINVAL, "%s: workspace of %zu bytes, %zu needed", who,
                          workspace_bytes, need);
  const size_t rs = row_stats_bytes(entries, tile);
  unsigned char* base = static_cast<unsigned char*>(workspace);
  p.rs_logm = reinterpret_cast<float*>(base);
  p.rs_mean = reinterpret_cast<uint32_t*>(base + (size_t)entries * tile * sizeof(float));
  p.rs_entries = entries;
  p.tile_h = tile_h;
  p.tile_w = tile_w;
  p.stat_tile = tile;
  p.stat_pad = tile;  // the token stream's; launch_typed sets that of tile blocks
  status = launch(dtype, p, base + rs, workspace_bytes - rs, stream, who);
  if (status != DSA_OK) return status;
  ReduceParams r;
  r.rs_logm = p.rs_logm;
  r.rs_mean = p.rs_mean;
  r.entries = entries;
  r.lse = lse;
  r.row_ptr = row_ptr;
  r.col_idx = col_idx;
  r.mass32 = mass;
  r.mass16 = static_cast<__half*>(mass_f16);
  r.cqy = static_cast<__half*>(centroid_q_y);
  r.cqx = static_cast<__half*>(centroid_q_x);
  r.cky = static_cast<__half*>(centroid_k_y);
  r.ckx = static_cast<__half*>(centroid_k_x);
  r.tokens = tokens;
  r.tiles = tiles;
  r.tile = tile;
  r.tile_h = tile_h;
  r.tile_w = tile_w;
  r.dense = dense ? 1 : 0;
  r.raw = 0;
  hipLaunchKernelGGL(tile_stats_reduce_kernel, dim3((unsigned)(heads * tiles)), dim3(256), 0,
                     stream, r);
  return dsa::check_launch(who);
}

extern "C" size_t dsa_bsa_fwd_block_mass_workspace_bytes(int32_t heads, int32_t tokens,
                                                         int32_t head_dim) {
  if (heads <= 0 || tokens <= 0 || head_dim <= 0) return 0;
  const size_t attention = dsa_bsa_workspace_bytes_block(1, heads, tokens, head_dim, 128);
  if (tokens % 128 != 0) return attention;
  const int64_t blocks = tokens / 128;
  return attention + row_mass_bytes((int64_t)heads * blocks * blocks, 128);
}

extern "C" int dsa_bsa_fwd_block_mass(const void* q, const void* k, const void* v, void* o,
                                      int32_t dtype, const int64_t* strides, int32_t tokens,
                                      int32_t heads, int32_t head_dim, float scale, float* lse,
                                      float* mass, void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
  const char* who = "dsa_bsa_fwd_block_mass";
  dsa::clear_error();
  if (!lse || !mass || !strides)
    return dsa::set_error(DSA_EINVAL, "%s: lse, mass and strides are required", who);
  // fp32 inputs: the fp32-compute kernel takes the mass from its own
  // probabilities, on whole 128-token blocks.
  if (dtype == DSA_F32 && tokens % 128 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: fp32 needs tokens a multiple of 128, got %d", who,
                          tokens);
  BsaParams p;
  int status = prepare(q, k, v, o, dtype, strides, 1, tokens, tokens, heads, head_dim, 128,
                       nullptr, nullptr, 1, scale, 0, 1, lse, who, &p);
  if (status != DSA_OK) return status;
  if (workspace_bytes > 0 && (!workspace || !aligned16(workspace)))
    return dsa::set_error(DSA_EINVAL, "%s: workspace must be 16-byte aligned", who);
  const size_t need = dsa_bsa_fwd_block_mass_workspace_bytes(heads, tokens, head_dim);
  if (workspace_bytes < need)
    return dsa::set_error(DSA_EINVAL, "%s: workspace of %zu bytes, %zu needed", who,
                          workspace_bytes, need);
  unsigned char* base = static_cast<unsigned char*>(workspace);
  if (tokens % 128 != 0) {
    // A partial last block: the dense attention, then the block-mass pass.
    // (Heads wider than 128 take the mass from the fp32-compute kernel's
    // statistics below.)
    status = launch(dtype, p, base, workspace_bytes, stream, who);
    if (status != DSA_OK) return status;
    const int64_t mass_strides[4] = {strides[1], strides[2], strides[4], strides[5]};
    return dsa_block_mass(q, k, dtype, mass_strides, tokens, heads, head_dim, 128, lse, tokens,
                          scale, mass, stream);
  }
  const int32_t blocks = tokens / 128;
  const int64_t entries = (int64_t)heads * blocks * blocks;
  const size_t rs = row_mass_bytes(entries, 128);
  p.rs_logm = reinterpret_cast<float*>(base);
  p.rs_mean = nullptr;  // the mean key offsets are not needed
  p.rs_entries = entries;
  p.tile_h = 1;
  p.tile_w = 128;
  p.stat_tile = 128;
  p.stat_pad = 128;
  status = launch(dtype, p, base + rs, workspace_bytes - rs, stream, who);
  if (status != DSA_OK) return status;
  ReduceParams r;
  r.rs_logm = p.rs_logm;
  r.rs_mean = p.rs_mean;
  r.entries = entries;
  r.lse = lse;
  r.row_ptr = nullptr;
  r.col_idx = nullptr;
  r.mass32 = mass;
  r.mass16 = r.cqy = r.cqx = r.cky = r.ckx = nullptr;
  r.tokens = tokens;
  r.tiles = blocks;
  r.tile = 128;
  r.tile_h = 1;
  r.tile_w = 128;
  r.dense = 1;
  r.raw = 1;
  hipLaunchKernelGGL(tile_stats_reduce_kernel, dim3((unsigned)(heads * blocks)), dim3(256), 0,
                     stream, r);
  return dsa::check_launch(who);
}
