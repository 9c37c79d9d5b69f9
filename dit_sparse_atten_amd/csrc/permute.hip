// Token-permutation gather for gfx950: dst[b, t, h, :] = src[b, perm[t], h, :].
//
// Replaces the Morton micro-tile reorder and restore of the reference:
//   SpatialTokenLayout.reorder_qkv -> layout_ops.reorder_qkv  (spatial.py:86-89,
//       layout_ops.py:86-125, its three index_select fallback 100-101)
//   SpatialTokenLayout.restore     -> index_select(1, inverse) (spatial.py:91-93)
// Up to three tensors move in one launch.  Each (b, t, h) row is a contiguous
// run of head_dim elements; it is copied as 16-byte chunks so that the 16
// lanes covering one row read and write one contiguous segment, whatever the
// token / head strides of source and destination are.  Bit-exact data movement.
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

// Grid: x = destination token, y = tensor * batch + b.  The 256 threads of a
// workgroup stride over the heads * chunks_per_row chunks of that token.
__global__ void __launch_bounds__(256) permute_rows_kernel(PermuteParams p) {
  const int t = blockIdx.x;
  const int n = blockIdx.y / p.batch;
  const int b = blockIdx.y % p.batch;
  const int s = p.perm[t];
  if ((unsigned)s >= (unsigned)p.tokens) return;  // invalid index: row left untouched
  const unsigned char* src = p.src[n] + b * p.src_sb[n] + (int64_t)s * p.src_st[n];
  unsigned char* dst = p.dst[n] + b * p.dst_sb[n] + (int64_t)t * p.dst_st[n];
  const int per_token = p.heads * p.chunks_per_row;
  for (int i = threadIdx.x; i < per_token; i += 256) {
    const int h = i / p.chunks_per_row;
    const int c = i - h * p.chunks_per_row;
    const dsa_u32x4 value =
        *reinterpret_cast<const dsa_u32x4*>(src + h * p.src_sh[n] + c * 16);
    *reinterpret_cast<dsa_u32x4*>(dst + h * p.dst_sh[n] + c * 16) = value;
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
  if ((int64_t)heads * p.chunks_per_row > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_permute_rows: rows too wide");
  hipLaunchKernelGGL(permute_rows_kernel, dim3((unsigned)tokens, (unsigned)(tensors * batch)),
                     dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_permute_rows");
}
