// Exact block attention mass for gfx950 (MI355X), bf16 or fp16 Q/K.
//
// Replaces `_block_attention_mass` / `_exact_block_mass_kernel` of the
// reference (attention_backends/flex.py:96-202):
//   mass[h, qb, kb] = sum_{t in qb, s in kb} exp(scale * <q_t, k_s> - lse[h, t])
// over valid tokens, where lse is the natural-log softmax normaliser that the
// dense forward (dsa_bsa_fwd with an lse output) returned for the same Q/K and
// scale.  Row qb sums to the number of valid queries in the block.
//
// Design: one 4-wave workgroup per (head, 128-query block) walks every key
// block once.  K streams through LDS in 64-key half-tiles (the same
// buffer->LDS staging as the forward kernel); S^T = K Q^T on
// v_mfma_f32_32x32x16_bf16 (or _f16) leaves each lane with one query row, so
// p = exp2(s * scale * log2(e) - lse * log2(e)) needs no max and no exchange.
// Each lane sums its probabilities per key block; a wave reduction and a
// fixed-order sum of the four wave partials (through LDS, double-buffered by
// block parity and ordered by the staging barrier) give one value per
// (qb, kb), written once: no atomics, run-to-run deterministic.
#include "bsa_tiles.h"

#include <cmath>

namespace {

using dsa::kHalfKeys;
using dsa::kKStage;
using dsa::kRowBytes;

struct BlockMassParams {
  const void* q;  // element type T of the kernel instance
  const void* k;
  const float* lse;  // [heads, tokens] (token stride 1, head stride lse_sh)
  float* mass;       // [heads, blocks, blocks]
  int64_t q_st, q_sh, k_st, k_sh, lse_sh;
  int32_t tokens, heads, blocks;
  int32_t head_dim;  // 8..256, a multiple of 8
  float scale_log2;  // scale * log2(e)
};

constexpr float kLog2e = 1.4426950408889634f;


// kHalves: head dims up to 128 * kHalves; above 128 each half-tile is staged
// as two 128-dim halves whose products add into one fp32 accumulator.
template <typename T, int kHalves = 1>
__global__ void __launch_bounds__(256, 2) block_mass_kernel(BlockMassParams p) {
  typedef dsa::Elem<T> E;
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[kKStage * kHalves];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k1[kKStage * kHalves];
  __shared__ float part[2][4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;

  const int work = dsa::xcd_remap(blockIdx.x, gridDim.x);
  const int qb = work % p.blocks;
  const int h = work / p.blocks;

  const int tq = qb * 128 + wave * 32 + qi;
  const bool row_ok = tq < p.tokens;
  const int tq_c = row_ok ? tq : p.tokens - 1;
  const T* qrow = static_cast<const T*>(p.q) + h * p.q_sh + (int64_t)tq_c * p.q_st;
  typename E::x8 qf[8 * kHalves];
#pragma unroll
  for (int hf = 0; hf < kHalves; ++hf)
    dsa::load_q_fragments(qrow + 128 * hf, g, p.head_dim - 128 * hf, qf + 8 * hf);
  // Rows past the sequence end get lse = +inf, so every p of theirs is 0.
  const float lse2 = row_ok ? p.lse[h * p.lse_sh + tq] * kLog2e : INFINITY;

  const T* kbase = static_cast<const T*>(p.k) + h * p.k_sh;
  uint32_t koff[kHalves][4];
#pragma unroll
  for (int hf = 0; hf < kHalves; ++hf)
    dsa::k_tile_offsets(wave, lane, p.k_st, p.head_dim - 128 * hf, koff[hf]);
  auto issue = [&](int key0, unsigned char* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int hf = 0; hf < kHalves; ++hf) {
      const __amdgpu_buffer_rsrc_t rsrc =
          dsa::k_tile_rsrc(kbase + 128 * hf, p.k_st, key0, p.tokens, p.head_dim - 128 * hf);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        dsa::lds_load16(rsrc, dst + hf * kKStage + (wave * 4 + j) * 1024, koff[hf][j], 0);
    }
  };

  float* mrow = p.mass + ((int64_t)h * p.blocks + qb) * p.blocks;
  auto flush = [&](int kb) __attribute__((always_inline)) {
    if (wave == 0 && lane == 0) {
      const float* pr = part[kb & 1];
      mrow[kb] = (pr[0] + pr[1]) + (pr[2] + pr[3]);
    }
  };

  float acc0 = 0.f, acc1 = 0.f;
  auto step = [&](int sub, const unsigned char* cur, unsigned char* nxt)
                  __attribute__((always_inline)) {
    // This stage has landed, and every wave's partial of the previous block
    // is in LDS.
    dsa::lds_barrier<true>();
    // Partials of the previous key block were stored before this barrier.
    if (sub >= 2 && (sub & 1) == 0) flush((sub >> 1) - 1);
    if (sub + 1 < 2 * p.blocks) issue((sub + 1) * kHalfKeys, nxt);
    const int valid = p.tokens - sub * kHalfKeys;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      dsa_f32x16 sacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
      const int row = kt * 32 + qi;
#pragma unroll
      for (int hf = 0; hf < kHalves; ++hf)
#pragma unroll
        for (int dc = 0; dc < 8; ++dc) {
          const typename E::x8 a = *reinterpret_cast<const typename E::x8*>(
              cur + hf * kKStage + row * kRowBytes + dsa::k2_swz(row, dc * 2 + g) * 16);
          sacc = E::mfma32(a, qf[8 * hf + dc], sacc);
        }
      if (valid < kHalfKeys) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3) >= valid) sacc[r] = -INFINITY;
      }
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        acc0 += __builtin_amdgcn_exp2f(fmaf(sacc[r], p.scale_log2, -lse2));
        acc1 += __builtin_amdgcn_exp2f(fmaf(sacc[r + 1], p.scale_log2, -lse2));
      }
    }
    if (sub & 1) {
      const float total = dsa::wave_total(acc0 + acc1);
      if (lane == 0) part[(sub >> 1) & 1][wave] = total;
      acc0 = 0.f;
      acc1 = 0.f;
    }
  };

  const int nsub = 2 * p.blocks;
  issue(0, lds_k0);
  for (int sub = 0; sub < nsub; sub += 2) {
    step(sub, lds_k0, lds_k1);
    step(sub + 1, lds_k1, lds_k0);
  }
  dsa::lds_barrier();
  flush(p.blocks - 1);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" int dsa_block_mass(const void* q, const void* k, int32_t dtype, const int64_t* strides,
                              int32_t tokens, int32_t heads, int32_t head_dim,
                              int32_t block_size, const float* lse, int64_t lse_head_stride,
                              float scale, float* mass, hipStream_t stream) {
  dsa::clear_error();
  if (!q || !k || !strides || !lse || !mass)
    return dsa::set_error(DSA_EINVAL, "dsa_block_mass: null pointer argument");
  if (dtype != DSA_BF16 && dtype != DSA_F16)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_block_mass: dtype %d unsupported (bf16 or fp16)",
                          dtype);
  if (tokens <= 0 || heads <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_block_mass: tokens and heads must be positive");
  if (head_dim <= 0 || head_dim > 2 * dsa::kHeadDim || head_dim % 8 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_block_mass: head_dim %d unsupported (a multiple of 8 up to 256)",
                          head_dim);
  if (block_size != 128)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_block_mass: block_size %d unsupported (128 only)", block_size);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return dsa::set_error(DSA_EINVAL, "dsa_block_mass: scale must be positive and finite");
  if (!aligned16(q) || !aligned16(k))
    return dsa::set_error(DSA_EINVAL, "dsa_block_mass: q and k must be 16-byte aligned");
  for (int i = 0; i < 4; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return dsa::set_error(DSA_EINVAL,
                            "dsa_block_mass: stride %d (=%lld) is not a non-negative multiple "
                            "of 8 elements", i, (long long)strides[i]);
  if (strides[2] * (int64_t)(2 * 64) > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_block_mass: key token stride %lld too large",
                          (long long)strides[2]);
  if (lse_head_stride < tokens)
    return dsa::set_error(DSA_EINVAL, "dsa_block_mass: lse head stride %lld < tokens %d",
                          (long long)lse_head_stride, tokens);
  const int32_t blocks = (tokens + block_size - 1) / block_size;
  const int64_t grid = (int64_t)heads * blocks;
  if (grid > 0x7fffffff)
    return dsa::set_error(DSA_EINVAL, "dsa_block_mass: grid too large");

  BlockMassParams p;
  p.q = q;
  p.k = k;
  p.lse = lse;
  p.mass = mass;
  p.q_st = strides[0]; p.q_sh = strides[1];
  p.k_st = strides[2]; p.k_sh = strides[3];
  p.lse_sh = lse_head_stride;
  p.tokens = tokens;
  p.heads = heads;
  p.blocks = blocks;
  p.head_dim = head_dim;
  p.scale_log2 = scale * kLog2e;
  const bool wide = head_dim > dsa::kHeadDim;
  const dim3 blocks_dim((unsigned)grid), threads(256);
  if (dtype == DSA_F16 && wide)
    hipLaunchKernelGGL((block_mass_kernel<_Float16, 2>), blocks_dim, threads, 0, stream, p);
  else if (dtype == DSA_F16)
    hipLaunchKernelGGL((block_mass_kernel<_Float16, 1>), blocks_dim, threads, 0, stream, p);
  else if (wide)
    hipLaunchKernelGGL((block_mass_kernel<__bf16, 2>), blocks_dim, threads, 0, stream, p);
  else
    hipLaunchKernelGGL((block_mass_kernel<__bf16, 1>), blocks_dim, threads, 0, stream, p);
  return dsa::check_launch("dsa_block_mass");
}
