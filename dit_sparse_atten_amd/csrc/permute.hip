// Token-permutation gather for gfx950: dst[b, t, h, :] = src[b, perm[t], h, :].
//
// Replaces the Morton micro-tile reorder and restore of the reference:
//   SpatialTokenLayout.reorder_qkv -> layout_ops.reorder_qkv  (spatial.py:86-89,
//       layout_ops.py:86-125, its three index_select fallback 100-101)
//   SpatialTokenLayout.restore     -> index_select(1, inverse) (spatial.py:91-93)
// Up to three tensors move in one launch.  Each (b, t, h) row is a contiguous
// run of head_dim elements; it is copied as 16-byte chunks so that the lanes
// covering one row read and write one contiguous segment, whatever the
// token / head strides of source and destination are.  Bit-exact data movement.
// The bound is the device copy rate: at 57,600 tokens x 40 heads x 128 bf16
// a head-major reorder of three tensors moves 5.4 TB/s, a plain copy 5.3.
#include "dsa_common.h"

namespace {

constexpr int kMaxTensors = 3;

struct PermuteParams {
  const unsigned char* src[kMaxTensors];
  unsigned char* dst[kMaxTensors];
  int64_t src_sb[kMaxTensors], src_st[kMaxTensors], src_sh[kMaxTensors];  // bytes
  int64_t dst_sb[kMaxTensors], dst_st[kMaxTensors], dst_sh[kMaxTensors];
  const int32_t* perm;
  int32_t tensors, batch, tokens, heads, chunks_per_row;
};

// Head-major destination tokens per workgroup.  Measured at 57,600 tokens x 40
// heads: 2 is fastest; 4, 8 and 16 lose up to 7% (the larger groups leave a
// single-tensor launch too few workgroups to fill the chip evenly).
constexpr int kGroupTokens = 2;
constexpr int kUnroll = 4;  // 16-byte chunks in flight per thread

// Grid: x = group of kGroup destination tokens, y = tensor * batch + b.  The
// group's chunks are numbered so that consecutive threads cover consecutive
// destination bytes.  A head-major destination (kGroup = kGroupTokens) is
// walked head-outer: each head contributes kGroup consecutive 256-byte rows.
// A token-major one (kGroup = 1) is walked as the token's contiguous
// heads * row_bytes.  Each thread issues kUnroll loads before its stores.
template <int kGroup>
__global__ void __launch_bounds__(256) permute_rows_kernel(PermuteParams p) {
  __shared__ int32_t source[kGroup];
  const int t0 = blockIdx.x * kGroup;
  const int rows = min(kGroup, p.tokens - t0);
  const int n = blockIdx.y / p.batch;
  const int b = blockIdx.y % p.batch;
  if constexpr (kGroup > 1) {
    if (threadIdx.x < rows) source[threadIdx.x] = p.perm[t0 + threadIdx.x];
    __syncthreads();
  } else {
    if ((unsigned)p.perm[t0] >= (unsigned)p.tokens) return;  // invalid index: row left untouched
  }
  const unsigned char* src = p.src[n] + b * p.src_sb[n];
  unsigned char* dst = p.dst[n] + b * p.dst_sb[n] + (int64_t)t0 * p.dst_st[n];
  const int64_t src_st = p.src_st[n], src_sh = p.src_sh[n];
  const int64_t dst_st = p.dst_st[n], dst_sh = p.dst_sh[n];
  const int cpr = p.chunks_per_row;
  const int total = rows * p.heads * cpr;
  for (int base = 0; base < total; base += 256 * kUnroll) {
    dsa_u32x4 value[kUnroll];
    unsigned char* out[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = base + u * 256 + (int)threadIdx.x;
      out[u] = nullptr;
      if (i < total) {
        const int row = i / cpr;
        const int c = i - row * cpr;
        const int h = kGroup > 1 ? row / rows : row;
        const int t = kGroup > 1 ? row - h * rows : 0;
        const int s = kGroup > 1 ? source[t] : p.perm[t0];
        if ((unsigned)s < (unsigned)p.tokens) {  // invalid index: row left untouched
          value[u] = *reinterpret_cast<const dsa_u32x4*>(src + s * src_st + h * src_sh + c * 16);
          out[u] = dst + t * dst_st + h * dst_sh + c * 16;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (out[u] != nullptr) *reinterpret_cast<dsa_u32x4*>(out[u]) = value[u];
  }
}

}  // namespace

extern "C" int dsa_permute_rows(int32_t tensors, const void* const* src, void* const* dst,
                                const int64_t* src_strides, const int64_t* dst_strides,
                                const int32_t* perm, int32_t batch, int32_t tokens,
                                int32_t heads, int32_t row_bytes, hipStream_t stream) {
  dsa::clear_error();
  if (tensors < 1 || tensors > kMaxTensors)
    return dsa::set_error(DSA_EINVAL, "dsa_permute_rows: 1 to 3 tensors per call");
  if (!src || !dst || !src_strides || !dst_strides || !perm)
    return dsa::set_error(DSA_EINVAL, "dsa_permute_rows: null pointer");
  if (batch <= 0 || tokens <= 0 || heads <= 0 || row_bytes <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_permute_rows: sizes must be positive");
  if (row_bytes % 16 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_permute_rows: row bytes %d not a multiple of 16",
                          row_bytes);
  PermuteParams p;
  for (int n = 0; n < tensors; ++n) {
    if (!src[n] || !dst[n]) return dsa::set_error(DSA_EINVAL, "dsa_permute_rows: null tensor");
    if ((reinterpret_cast<uintptr_t>(src[n]) | reinterpret_cast<uintptr_t>(dst[n])) & 15u)
      return dsa::set_error(DSA_EINVAL, "dsa_permute_rows: tensors must be 16-byte aligned");
    for (int i = 0; i < 3; ++i)
      if ((src_strides[n * 3 + i] | dst_strides[n * 3 + i]) & 15)
        return dsa::set_error(DSA_EINVAL, "dsa_permute_rows: byte strides must be multiples of 16");
    p.src[n] = static_cast<const unsigned char*>(src[n]);
    p.dst[n] = static_cast<unsigned char*>(dst[n]);
    p.src_sb[n] = src_strides[n * 3 + 0];
    p.src_st[n] = src_strides[n * 3 + 1];
    p.src_sh[n] = src_strides[n * 3 + 2];
    p.dst_sb[n] = dst_strides[n * 3 + 0];
    p.dst_st[n] = dst_strides[n * 3 + 1];
    p.dst_sh[n] = dst_strides[n * 3 + 2];
  }
  p.perm = perm;
  p.tensors = tensors;
  p.batch = batch;
  p.tokens = tokens;
  p.heads = heads;
  p.chunks_per_row = row_bytes / 16;
  if ((int64_t)tensors * batch > 65535)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_permute_rows: batch too large");
  if ((int64_t)kGroupTokens * heads * p.chunks_per_row > (1 << 30))
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_permute_rows: rows too wide");
  bool head_major = true;  // every destination has its token stride below its head stride
  for (int n = 0; n < tensors; ++n) head_major = head_major && p.dst_st[n] < p.dst_sh[n];
  if (head_major) {
    const unsigned groups = (unsigned)((tokens + kGroupTokens - 1) / kGroupTokens);
    hipLaunchKernelGGL(permute_rows_kernel<kGroupTokens>,
                       dim3(groups, (unsigned)(tensors * batch)), dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL(permute_rows_kernel<1>, dim3((unsigned)tokens, (unsigned)(tensors * batch)),
                       dim3(256), 0, stream, p);
  }
  return dsa::check_launch("dsa_permute_rows");
}
