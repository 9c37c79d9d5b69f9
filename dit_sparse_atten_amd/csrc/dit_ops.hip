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
// arithmetic are fp32; outputs are rounded once to bf16.  Per-column
// parameters are fp32 and 16-byte aligned.
#include <initializer_list>
#include <type_traits>

#include "dsa_common.h"

namespace {

// One wave per row: each lane holds kC chunks of 8 consecutive elements
// (chunk c = lane + 64 i), so a row needs no workgroup barrier.  A workgroup
// is kWaves waves, one row each.  At 57,600 rows of 1536 that is 14,400
// workgroups, several rounds of the chip's slots; walking 2 or 4 rows per
// wave with the next row prefetched measured 4-16% slower (fewer workgroups,
// and a last round left partly empty).
// Per-column parameters (weight, bias, shift, scale, gate) are read with
// 16-byte loads per row; the rows of a workgroup share them through L1/L2.
constexpr int kWaves = 4;
constexpr int kMaxChunks = 16;  // dim <= 64 * 8 * 16 = 8192

__device__ __forceinline__ void load8(const __bf16* src, float out[8]) {
  const dsa_bf16x8 v = *reinterpret_cast<const dsa_bf16x8*>(src);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}

__device__ __forceinline__ void load8f(const float* src, float out[8]) {
  const dsa_f32x4 a = *reinterpret_cast<const dsa_f32x4*>(src);
  const dsa_f32x4 b = *reinterpret_cast<const dsa_f32x4*>(src + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    out[e] = a[e];
    out[e + 4] = b[e];
  }
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

template <int kC>
__device__ __forceinline__ void load_row(const __bf16* row, int lane, int chunks, float v[kC][8]) {
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) load8(row + c * 8, v[i]);
  }
}

// Row of this wave.
__device__ __forceinline__ int wave_row() { return blockIdx.x * kWaves + (threadIdx.x >> 6); }

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
template <int kC>
__global__ void __launch_bounds__(256) layernorm_modulate_kernel(LnParams p) {
  const int lane = threadIdx.x & 63;
  const int chunks = p.dim / 8;
  const int row = wave_row();
  if (row >= p.rows) return;
  float v[kC][8];
  load_row<kC>(p.x + (int64_t)row * p.x_stride, lane, chunks, v);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kC; ++i)
    if (lane + 64 * i < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[i][e];
    }
  const float mean = dsa::wave_total(s) / (float)p.dim;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kC; ++i)
    if (lane + 64 * i < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[i][e] - mean;
        q = fmaf(d, d, q);
      }
    }
  const float rstd = rsqrtf(dsa::wave_total(q) / (float)p.dim + p.eps);
  const int64_t group_off = (int64_t)(row / p.rows_per_group) * p.dim;
  __bf16* out = p.out + (int64_t)row * p.out_stride;
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const int c = lane + 64 * i;
    if (c >= chunks) continue;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (v[i][e] - mean) * rstd;
    if (p.weight) {
      float w[8], b[8];
      load8f(p.weight + c * 8, w);
      if (p.bias) {
        load8f(p.bias + c * 8, b);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = fmaf(y[e], w[e], b[e]);
    }
    if (p.scale) {
      float sc[8], sh[8];
      load8f(p.scale + group_off + c * 8, sc);
      if (p.shift) {
        load8f(p.shift + group_off + c * 8, sh);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) sh[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = fmaf(y[e], 1.f + sc[e], sh[e]);
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
template <int kC>
__global__ void __launch_bounds__(256) rmsnorm_rope_kernel(RmsRopeParams p) {
  const int lane = threadIdx.x & 63;
  const int chunks = p.dim / 8;
  const int row = wave_row();
  if (row >= p.rows) return;
  float v[kC][8];
  load_row<kC>(p.x + (int64_t)row * p.x_stride, lane, chunks, v);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < kC; ++i)
    if (lane + 64 * i < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) q = fmaf(v[i][e], v[i][e], q);
    }
  const float rstd = rsqrtf(dsa::wave_total(q) / (float)p.dim + p.eps);
  const float* cs_row =
      p.cos_sin ? p.cos_sin + (int64_t)(row % p.tokens) * p.head_dim : nullptr;
  __bf16* out = p.out + (int64_t)row * p.out_stride;
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const int c = lane + 64 * i;
    if (c >= chunks) continue;
    float w[8], y[8];
    load8f(p.weight + c * 8, w);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = v[i][e] * rstd * w[e];
    if (cs_row) {
      // The 8 elements are 4 consecutive pairs of one head: (cos, sin) x 4.
      float t[8];
      load8f(cs_row + ((c * 8) % p.head_dim), t);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float a = y[e], b = y[e + 1];
        y[e] = a * t[e] - b * t[e + 1];
        y[e + 1] = a * t[e + 1] + b * t[e];
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

// out = x + gate * y (a pure stream: no reduction).
template <int kC>
__global__ void __launch_bounds__(256) gated_residual_kernel(ResidualParams p) {
  const int lane = threadIdx.x & 63;
  const int chunks = p.dim / 8;
  const int row = wave_row();
  if (row >= p.rows) return;
  const int64_t group_off = (int64_t)(row / p.rows_per_group) * p.dim;
  float a[kC][8], b[kC][8];
  load_row<kC>(p.x + (int64_t)row * p.x_stride, lane, chunks, a);
  load_row<kC>(p.y + (int64_t)row * p.y_stride, lane, chunks, b);
#pragma unroll
  for (int i = 0; i < kC; ++i) {
    const int c = lane + 64 * i;
    if (c >= chunks) continue;
    float g[8], r[8];
    if (p.gate) {
      load8f(p.gate + group_off + c * 8, g);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) g[e] = 1.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = fmaf(g[e], b[i][e], a[i][e]);
    store8(p.out + (int64_t)row * p.out_stride + c * 8, r);
  }
}

// Calls f(std::integral_constant<int, kC>) with the smallest instantiated
// chunk count covering dim / 8 chunks per 64-lane row.
template <typename F>
void with_chunks(int dim, F&& f) {
  const int c = (dim / 8 + 63) / 64;
  if (c <= 1) f(std::integral_constant<int, 1>{});
  else if (c <= 2) f(std::integral_constant<int, 2>{});
  else if (c <= 3) f(std::integral_constant<int, 3>{});
  else if (c <= 4) f(std::integral_constant<int, 4>{});
  else if (c <= 8) f(std::integral_constant<int, 8>{});
  else f(std::integral_constant<int, 16>{});
}

dim3 row_grid(int32_t rows) { return dim3((unsigned)((rows + kWaves - 1) / kWaves)); }

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int check_rows(const char* what, const void* x, const void* out, int64_t xs, int64_t os,
               int32_t rows, int32_t dim) {
  if (!x || !out) return dsa::set_error(DSA_EINVAL, "%s: null tensor", what);
  if (rows <= 0 || dim <= 0 || dim % 8 != 0 || dim > 64 * 8 * kMaxChunks)
    return dsa::set_error(DSA_EINVAL, "%s: dim %d must be a positive multiple of 8 <= %d", what,
                          dim, 64 * 8 * kMaxChunks);
  if (!aligned16(x) || !aligned16(out) || xs % 8 != 0 || os % 8 != 0 || xs < dim || os < dim)
    return dsa::set_error(DSA_EINVAL, "%s: rows must be 16-byte aligned with strides >= dim", what);
  return DSA_OK;
}

int check_params(const char* what, std::initializer_list<const float*> params) {
  for (const float* param : params)
    if (param && !aligned16(param))
      return dsa::set_error(DSA_EINVAL, "%s: fp32 parameter vectors must be 16-byte aligned", what);
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
  if (check_params("dsa_layernorm_modulate", {weight, bias, shift, scale})) return DSA_EINVAL;
  LnParams p{static_cast<const __bf16*>(x), static_cast<__bf16*>(out), weight, bias, shift,
             scale, x_stride, out_stride, rows, dim, rows_per_group > 0 ? rows_per_group : rows,
             eps};
  with_chunks(dim, [&](auto kc) {
    hipLaunchKernelGGL(layernorm_modulate_kernel<decltype(kc)::value>, row_grid(rows), dim3(256),
                       0, stream, p);
  });
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
  if (check_params("dsa_rmsnorm_rope", {weight})) return DSA_EINVAL;
  if (head_dim <= 0 || head_dim % 8 != 0 || dim % head_dim != 0)
    return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: head_dim must divide dim (multiple of 8)");
  if (cos_sin && (tokens <= 0 || rows % tokens != 0 || !aligned16(cos_sin)))
    return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: rows must be whole sequences and "
                                      "cos_sin 16-byte aligned");
  if (!(eps > 0.f)) return dsa::set_error(DSA_EINVAL, "dsa_rmsnorm_rope: eps must be positive");
  RmsRopeParams p{static_cast<const __bf16*>(x), static_cast<__bf16*>(out), weight, cos_sin,
                  x_stride, out_stride, rows, dim, head_dim, tokens > 0 ? tokens : rows, eps};
  with_chunks(dim, [&](auto kc) {
    hipLaunchKernelGGL(rmsnorm_rope_kernel<decltype(kc)::value>, row_grid(rows), dim3(256), 0,
                       stream, p);
  });
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
  if (check_params("dsa_gated_residual", {gate})) return DSA_EINVAL;
  ResidualParams p{static_cast<const __bf16*>(x), static_cast<const __bf16*>(y),
                   static_cast<__bf16*>(out), gate, x_stride, y_stride, out_stride, rows, dim,
                   rows_per_group > 0 ? rows_per_group : rows};
  with_chunks(dim, [&](auto kc) {
    hipLaunchKernelGGL(gated_residual_kernel<decltype(kc)::value>, row_grid(rows), dim3(256), 0,
                       stream, p);
  });
  return dsa::check_launch("dsa_gated_residual");
}
