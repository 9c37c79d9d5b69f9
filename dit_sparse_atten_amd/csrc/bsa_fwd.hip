// C-ABI entry points of the block-sparse attention forward (gfx950), and the
// bf16 kernel instances; the kernels are in bsa_kernel.h, the fp16 instances
// in bsa_fwd_f16.hip.
//
// Replaces the FlexAttention call of the reference backend
// (attention_backends/flex.py:379-399 `_flex_output`, kernel options
// flex.py:360-364) and its dense SDPA fallback (attention_backends/dense.py:14-48).
#include <cmath>
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
  if (dtype != DSA_BF16 && dtype != DSA_F16)
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: dtype %d unsupported (bf16 or fp16)", who, dtype);
  if (batch <= 0 || heads <= 0 || q_tokens <= 0 || kv_tokens <= 0)
    return dsa::set_error(DSA_EINVAL, "%s: batch/heads/tokens must be positive", who);
  if (head_dim <= 0 || head_dim > kHeadDim || head_dim % 8 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "%s: head_dim %d unsupported (a multiple of 8 up to 128)", who, head_dim);
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
  p->scale = scale;
  p->scale_log2 = scale * 1.4426950408889634f;
  return DSA_OK;
}

// Launches the attention of a prepared call on `scratch_bytes` of scratch
// (launch order, then split partials; see launch_typed).
int launch(int32_t dtype, BsaParams p, void* scratch, size_t scratch_bytes, hipStream_t stream,
           const char* who) {
  return dtype == DSA_F16 ? bsa_launch_f16(p, scratch, scratch_bytes, stream, who)
                          : launch_typed<__bf16>(p, scratch, scratch_bytes, stream, who);
}

}  // namespace

// Scratch of dsa_bsa_fwd_noalloc: the launch order of up to kMaxOrderItems
// work items (1 MiB) and the aligned-walk table (4 KiB), then kMaxPartGroups
// split partials (68,157,440 bytes).
// Every device the library runs on holds its own copy until the process
// ends; host code reaches it only through the address hipGetSymbolAddress
// returns on that device (scratch_on).
constexpr size_t kScratchBytes = (size_t)kMaxOrderItems * sizeof(int32_t) + kWalkBytes +
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

extern "C" size_t dsa_bsa_workspace_bytes_block(int32_t batch, int32_t heads,
                                                int32_t kv_tokens, int32_t head_dim,
                                                int32_t block_size) {
  if (batch <= 0 || heads <= 0 || kv_tokens <= 0 || head_dim <= 0) return 0;
  if (block_size <= 0 || block_size > 128) return 0;
  const int32_t kv_blocks = (kv_tokens + block_size - 1) / block_size;
  // Routed calls are self-attention (q_tokens == kv_tokens): batch x heads x
  // kv_blocks work items to order.
  const size_t order = order_bytes((int64_t)batch * heads * kv_blocks, kv_blocks);
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
