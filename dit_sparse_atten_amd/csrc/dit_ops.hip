// Elementwise / row-normalisation kernels of the Wan DiT block around the
// attention path (gfx950): the end-to-end denoising loop's non-GEMM work.
//
// Replaces, for the Wan2.1 transformer block the reference drives through
// Diffusers (wan_diffusers.py:75-191; diffusers WanTransformerBlock):
//   norm1/norm3 + modulate   LayerNorm (no affine) then x * (1 + scale) + shift
//   norm2                    LayerNorm with weight and bias (cross_attn_norm)
//   norm_q / norm_k + RoPE   RMSNorm over the projected q/k rows (weight), then
//                            the 3D rotary embedding of each head's (even,
//                            odd) pairs (svg_ops.py:22-202 holds the
//                            reference's own fused RoPE variant)
//   gated residual           x + gate * y (gate = 1 for the cross-attention)
// Rows are bf16 [rows, dim] with a contiguous last axis; statistics and
// arithmetic are fp32; outputs are rounded once to bf16.  One 256-thread
// workgroup per row, 8 consecutive elements per thread and pass.
#include "dsa_common.h"

namespace {

__device__ __forceinline__ float block_sum(float v, float* scratch) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  dsa::lds_barrier();
  const float total = (scratch[0] + scratch[1]) + (scratch[2] + scratch[3]);
  dsa::lds_barrier();  // scratch may be reused by the next reduction
  return total;
}

__device__ __forceinline__ void load8(const __bf16* src, float out[8]) {
  const dsa_bf16x8 v = *reinterpret_cast<const dsa_bf16x8*>(src);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}

__device__ __forceinline__ void store8(__bf16* dst, const float in[8]) {
  dsa_bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const dsa_f32x2 two = {in[e], in[e + 1]};
    const dsa_bf16x2 b = __builtin_convertvector(two, dsa_bf16x2);
    v[e] = b[0];
    v[e + 1] = b[1];
  }
  *reinterpret_cast<dsa_bf16x8*>(dst) = v;
}

constexpr int kMaxPer = 4;  // 8-element chunks per thread: dim <= 256 * 8 * 4 = 8192

struct LnParams {
  const __bf16* x;
  __bf16* out;
  const float* weight;  // [dim] or null
  const float* bias;    // [dim] or null
  const float* shift;   // [groups, dim] or null
  const float* scale;   // [groups, dim] or null
  int64_t x_stride, out_stride;
  int32_t rows, dim, rows_per_group;
  float eps;
};

// out = ((x - mean) / sqrt(var + eps)) [* weight + bias] [* (1 + scale) + shift]
__global__ void __launch_bounds__(256) layernorm_modulate_kernel(LnParams p) {
  __shared__ float scratch[4];
  const int row = blockIdx.x;
  const __bf16* x = p.x + (int64_t)row * p.x_stride;
  float v[kMaxPer][8];
  const int chunks = p.dim / 8;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < chunks) {
      load8(x + c * 8, v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[i][e];
    }
  }
  const float mean = block_sum(s, scratch) / (float)p.dim;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[i][e] - mean;
        q = fmaf(d, d, q);
      }
    }
  }
  const float rstd = rsqrtf(block_sum(q, scratch) / (float)p.dim + p.eps);
  const int group = row / p.rows_per_group;
  __bf16* out = p.out + (int64_t)row * p.out_stride;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c >= chunks) continue;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = c * 8 + e;
      float t = (v[i][e] - mean) * rstd;
      if (p.weight) t = fmaf(t, p.weight[j], p.bias ? p.bias[j] : 0.f);
      if (p.scale) t = fmaf(t, 1.f + p.scale[(int64_t)group * p.dim + j],
                            p.shift ? p.shift[(int64_t)group * p.dim + j] : 0.f);
      y[e] = t;
    }
    store8(out + c * 8, y);
  }
}

struct RmsRopeParams {
  const __bf16* x;
  __bf16* out;
  const float* weight;  // [dim]
  const float* cos_sin;  // [tokens, head_dim / 2, 2] (cos, sin) or null (no rotation)
  int64_t x_stride, out_stride;
  int32_t rows, dim, head_dim, tokens;
  float eps;
};

// out = rope(x / sqrt(mean(x^2) + eps) * weight), the rotation acting on each
// head's consecutive (even, odd) pairs with the precomputed (cos, sin) of the
// row's token (row % tokens) and pair.
__global__ void __launch_bounds__(256) rmsnorm_rope_kernel(RmsRopeParams p) {
  __shared__ float scratch[4];
  const int row = blockIdx.x;
  const __bf16* x = p.x + (int64_t)row * p.x_stride;
  float v[kMaxPer][8];
  const int chunks = p.dim / 8;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < chunks) {
      load8(x + c * 8, v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) q = fmaf(v[i][e], v[i][e], q);
    }
  }
  const float rstd = rsqrtf(block_sum(q, scratch) / (float)p.dim + p.eps);
  const int token = row % p.tokens;
  const float* cs_row = p.cos_sin ? p.cos_sin + (int64_t)token * p.head_dim : nullptr;
  __bf16* out = p.out + (int64_t)row * p.out_stride;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c >= chunks) continue;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = v[i][e] * rstd * p.weight[c * 8 + e];
    if (cs_row) {
      // The 8 elements are 4 consecutive pairs of one head: (cos, sin) x 4.
      const int pair0 = ((c * 8) % p.head_dim) / 2;
      const dsa_f32x4 t0 = *reinterpret_cast<const dsa_f32x4*>(cs_row + pair0 * 2);
      const dsa_f32x4 t1 = *reinterpret_cast<const dsa_f32x4*>(cs_row + pair0 * 2 + 4);
      const float cs[4] = {t0[0], t0[2], t1[0], t1[2]};
      const float sn[4] = {t0[1], t0[3], t1[1], t1[3]};
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float a = y[e], b = y[e + 1];
        y[e] = a * cs[e / 2] - b * sn[e / 2];
        y[e + 1] = a * sn[e / 2] + b * cs[e / 2];
      }
    }
    store8(out + c * 8, y);
  }
}

struct ResidualParams {
  const __bf16* x;
  const __bf16* y;
  __bf16* out;
  const float* gate;  // [groups, dim] or null (gate 1)
  int64_t x_stride, y_stride, out_stride;
  int32_t rows, dim, rows_per_group;
};

__global__ void __launch_bounds__(256) gated_residual_kernel(ResidualParams p) {
  const int row = blockIdx.x;
  const int chunks = p.dim / 8;
  const int group = row / p.rows_per_group;
  for (int c = threadIdx.x; c < chunks; c += 256) {
    float a[8], b[8], r[8];
    load8(p.x + (int64_t)row * p.x_stride + c * 8, a);
    load8(p.y + (int64_t)row * p.y_stride + c * 8, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = p.gate ? p.gate[(int64_t)group * p.dim + c * 8 + e] : 1.f;
      r[e] = fmaf(g, b[e], a[e]);
    }
    store8(p.out + (int64_t)row * p.out_stride + c * 8, r);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int check_rows(const char* what, const void* x, const void* out, int64_t xs, int64_t os,
               int32_t rows, int32_t dim) {
  if (!x || !out) return dsa::set_error(DSA_EINVAL, "%s: null tensor", what);
  if (rows <= 0 || dim <= 0 || dim % 8 != 0 || dim > 256 * 8 * kMaxPer)
    return dsa::set_error(DSA_EINVAL, "%s: dim %d must be a positive multiple of 8 <= %d", what,
                          dim, 256 * 8 * kMaxPer);
  if (!aligned16(x) || !aligned16(out) || xs % 8 != 0 || os % 8 != 0 || xs < dim || os < dim)
    return dsa::set_error(DSA_EINVAL, "%s: rows must be 16-byte aligned with strides >= dim", what);
  return DSA_OK;
}

}  // namespace

extern "C" int dsa_layernorm_modulate(const void* x, int64_t x_stride, int32_t rows, int32_t dim,
                                      const float* weight, const float* bias,
                                      const float* shift, const float* scale,
                                      int32_t rows_per_group, float eps, void* out,
                                      int64_t out_stride, hipStream_t stream) {
  dsa::clear_error();
  const int status = check_rows("dsa_layernorm_modulate", x, out, x_stride, out_stride, rows, dim);
  if (status) return status;
  if ((bias && !weight) || (shift && !scale))
    return dsa::set_error(DSA_EINVAL, "dsa_layernorm_modulate: bias needs weight, shift needs scale");
  if ((scale && rows_per_group <= 0) || !(eps > 0.f))
    return dsa::set_error(DSA_EINVAL, "dsa_layernorm_modulate: rows_per_group and eps must be positive");
  LnParams p{static_cast<const __bf16*>(x), static_cast<__bf16*>(out), weight, bias, shift,
             scale, x_stride, out_stride, rows, dim, rows_per_group > 0 ? rows_per_group : rows,
             eps};
  hipLaunchKernelGGL(layernorm_modulate_kernel, dim3((unsigned)rows), dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_layernorm_modulate");
}

extern "C" int dsa_rmsnorm_rope(const void* x, int64_t x_stride, int32_t rows, int32_t dim,
                                int32_t head_dim, const float* weight, const float* cos_sin,
                                int32_t tokens, float eps, void* out, int64_t out_stride,
                                hipStream_t stream) {
  dsa::clear_error();
  const int status = check_rows("dsa_rmsnorm_rope", x, out, x_stride, out_stride, rows, dim);
  if (status) return status;
  if (!weight) return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: weight required");
  if (head_dim <= 0 || head_dim % 8 != 0 || dim % head_dim != 0)
    return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: head_dim must divide dim (multiple of 8)");
  if (cos_sin && (tokens <= 0 || rows % tokens != 0 || !aligned16(cos_sin)))
    return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: rows must be whole sequences and "
                                      "cos_sin 16-byte aligned");
  if (!(eps > 0.f)) return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: eps must be positive");
  RmsRopeParams p{static_cast<const __bf16*>(x), static_cast<__bf16*>(out), weight, cos_sin,
                  x_stride, out_stride, rows, dim, head_dim, tokens > 0 ? tokens : rows, eps};
  hipLaunchKernelGGL(rmsnorm_rope_kernel, dim3((unsigned)rows), dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_rmsnorm_rope");
}

extern "C" int dsa_gated_residual(const void* x, int64_t x_stride, const void* y,
                                  int64_t y_stride, const float* gate, int32_t rows, int32_t dim,
                                  int32_t rows_per_group, void* out, int64_t out_stride,
                                  hipStream_t stream) {
  dsa::clear_error();
  int status = check_rows("dsa_gated_residual", x, out, x_stride, out_stride, rows, dim);
  if (status) return status;
  status = check_rows("dsa_gated_residual", y, out, y_stride, out_stride, rows, dim);
  if (status) return status;
  if (gate && rows_per_group <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_gated_residual: rows_per_group must be positive");
  ResidualParams p{static_cast<const __bf16*>(x), static_cast<const __bf16*>(y),
                   static_cast<__bf16*>(out), gate, x_stride, y_stride, out_stride, rows, dim,
                   rows_per_group > 0 ? rows_per_group : rows};
  hipLaunchKernelGGL(gated_residual_kernel, dim3((unsigned)rows), dim3(256), 0, stream, p);
  return dsa::check_launch("dsa_gated_residual");
}
