// Sampled block-mass estimate for gfx950 (bf16 or fp16 Q/K).
//
// Replaces `_sampled_block_mass` (attention_backends/flex.py:205-251): per
// block b of size_b = min(T - block * b, block) tokens, S samples at local
// offsets floor((2 s + 1) size_b / (2 S)); scores of every sampled query
// against every sampled key, computed by a matmul in the input type and
// multiplied by the scale in the input type (so rounded twice to bf16 or
// fp16), plus log(size_b / S) per key sample; an fp32 softmax over all
// sampled keys; mass[h, qb, kb] = mean over the query samples of block qb of
// the sum over the key samples of block kb.
//
// Any S in 1..block (<= 128) runs on a power-of-two sample stride SP >= S:
// sample slots s >= S of every block are padding, masked out of the
// softmax (keys) and out of the mean (queries).  SP <= 32: a 32-key sub-tile
// covers 32 / SP key blocks and a wave's 32 query lanes 32 / SP query blocks,
// so block sums are lane shuffles.  SP = 64 or 128: a key block spans one or
// two whole 64-key tiles and a query block two or four waves; each wave's
// block sum goes through LDS and the workgroup adds them in a fixed order
// after the next barrier (no atomics: the mass, the input of the bit-exact
// route selection, is run-to-run deterministic).
#include <type_traits>

#include "bsa_tiles.h"

namespace {

constexpr int kHeadDim = 128;
constexpr float kLog2e = 1.4426950408889634f;

struct MassParams {
  const void* q;  // element type T of the kernel instance
  const void* k;
  float* mass;  // [heads, blocks, blocks]
  int64_t q_st, q_sh, k_st, k_sh;
  int32_t tokens, heads, blocks, block_size, samples;  // samples: S (real)
  int32_t head_dim;  // 8..256, a multiple of 8
  float scale;      // score scale (d^-1/2 unless given)
  float logw_full;  // log(block_size / S)
  float logw_last;  // log(size of the last block / S)
};

// Token of padded sample slot j (block j / SP, sample j % SP) for S real
// samples per block (flex.py:224-231); a padding slot repeats the block's
// last sample (it is masked).
template <int SP>
__device__ __forceinline__ int sampled_token(int j, int tokens, int block_size, int S) {
  const int blk = j / SP;
  int s = j % SP;
  s = s < S ? s : S - 1;
  int size = tokens - blk * block_size;
  size = size < block_size ? size : block_size;
  int local = ((2 * s + 1) * size) / (2 * S);
  local = local < size - 1 ? local : size - 1;
  return blk * block_size + local;
}

// Rounding of two fp32 values to T (round to nearest even; fp16 overflows to
// inf as torch's fp16 matmul does), returned as fp32.
template <typename T>
__device__ __forceinline__ void round_pair(float a, float b, float& ra, float& rb) {
  const dsa_f32x2 two = {a, b};
  const typename dsa::Elem<T>::x2 h = __builtin_convertvector(two, typename dsa::Elem<T>::x2);
  if constexpr (std::is_same<T, __bf16>::value) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, h);
    ra = __builtin_bit_cast(float, bits << 16);
    rb = __builtin_bit_cast(float, bits & 0xFFFF0000u);
  } else {
    ra = (float)h[0];
    rb = (float)h[1];
  }
}

// One workgroup (4 waves x 32 sampled queries) scans every sampled key twice:
// sweep 1 builds each query's log-sum-exp, sweep 2 sums the normalised
// probabilities per (query block, key block).  The sampled score matrix is
// never written to memory.  The scan is VALU-bound (the per-score rounding
// and softmax work outweighs the 32x32x16 MFMAs several times), so scores
// are rounded in pairs, the log2(e) scale and log-weight fold into one fma,
// the max runs over the rounded scores, and only the tile holding the
// sequence's last sampled keys (every tile with padding slots) pays the
// per-score checks.  Sampled key rows are gathered straight into LDS (buffer
// loads with a per-lane row offset), double-buffered one 64-key tile ahead.
//
// kHalves: head dims up to 128 * kHalves.  Head dims above 128 stage each
// tile as two 128-dim halves (dims 0..127, then 128..) and add both halves'
// products into one fp32 accumulator before the score is rounded, as one
// matmul over all dims does.
template <typename T, int SP, bool kPad, int kHalves = 1>
__global__ void __launch_bounds__(256) sampled_mass_kernel(MassParams p) {
  typedef dsa::Elem<T> E;
  constexpr int kTileKeys = 64;
  constexpr int kHalfBytes = kTileKeys * 256;  // one 128-dim half of a tile
  constexpr bool kWide = SP >= 64;
  constexpr int KBS = kWide ? 1 : 32 / SP;  // key blocks of one 32-key sub-tile
  __shared__ __attribute__((aligned(1024))) unsigned char st0[kHalfBytes * kHalves];
  __shared__ __attribute__((aligned(1024))) unsigned char st1[kHalfBytes * kHalves];
  __shared__ float wide_part[2][4];  // kWide: per-wave block sums, by block parity

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;
  const int h = blockIdx.y;
  const int S = kPad ? p.samples : SP;
  const int ns = p.blocks * SP;
  const int tiles = (ns + kTileKeys - 1) / kTileKeys;
  const int q0 = blockIdx.x * 128 + wave * 32;  // first sampled query of this wave

  int qs = q0 + qi;
  const bool q_real = qs < ns && (qs % SP) < S;
  qs = qs < ns ? qs : ns - 1;
  const T* qrow = static_cast<const T*>(p.q) + h * p.q_sh +
                  (int64_t)sampled_token<SP>(qs, p.tokens, p.block_size, S) * p.q_st;
  typename E::x8 qf[8 * kHalves];
#pragma unroll
  for (int hf = 0; hf < kHalves; ++hf)
    dsa::load_q_fragments(qrow + 128 * hf, g, p.head_dim - 128 * hf, qf + 8 * hf);

  // The head's K rows as one raw buffer (the host keeps them within 2^31 bytes).
  const T* kbase = static_cast<const T*>(p.k) + h * p.k_sh;
  __amdgpu_buffer_rsrc_t k_rsrc[kHalves];
#pragma unroll
  for (int hf = 0; hf < kHalves; ++hf)
    k_rsrc[hf] = dsa::make_rsrc(kbase + 128 * hf,
                                (uint32_t)(((int64_t)(p.tokens - 1) * p.k_st + kHeadDim) * 2));
  // This lane's 4 chunks of tile t: LDS slot idx = (wave * 4 + j) * 64 + lane
  // holds chunk (idx & 15) ^ (row & 15) of tile row idx >> 4.
  auto issue = [&](int t, unsigned char* dst) __attribute__((always_inline)) {
    const int kt0 = t * kTileKeys;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int idx = (wave * 4 + j) * 64 + lane;
      const int row = idx >> 4;
      const int c = (idx & 15) ^ (row & 15);
      int key = kt0 + row;
      key = key < ns ? key : ns - 1;
      const uint32_t base = (uint32_t)(
          ((int64_t)sampled_token<SP>(key, p.tokens, p.block_size, S) * p.k_st + c * 8) * 2);
#pragma unroll
      for (int hf = 0; hf < kHalves; ++hf)
        dsa::lds_load16(k_rsrc[hf], dst + hf * kHalfBytes + (wave * 4 + j) * 1024,
                        base | dsa::dead_bits(c, p.head_dim - 128 * hf), 0);
    }
  };

  const int last_block = p.blocks - 1;
  const float c_full = p.logw_full * kLog2e;
  const float c_last = p.logw_last * kLog2e;
  // Tiles before this one hold only full, in-range key blocks.
  const int first_tail_tile = kPad ? 0 : (last_block * SP) / kTileKeys;
  float m2 = -INFINITY, l2 = 0.f, lse2 = 0.f;
  float wide_acc = 0.f;  // kWide: this lane's sum over the current key block

  auto compute = [&](const unsigned char* lds_k, int t, int sweep) __attribute__((always_inline)) {
    const int kt0 = t * kTileKeys;
    const bool tail = t >= first_tail_tile;
#pragma unroll
    for (int sub = 0; sub < kTileKeys / 32; ++sub) {
      dsa_f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int hf = 0; hf < kHalves; ++hf)
#pragma unroll
        for (int dc = 0; dc < 8; ++dc) {
          const int key = sub * 32 + qi;
          const int c = dc * 2 + g;
          const typename E::x8 a = *reinterpret_cast<const typename E::x8*>(
              lds_k + hf * kHalfBytes + key * 256 + ((c ^ (key & 15)) << 4));
          acc = E::mfma32(a, qf[8 * hf + dc], acc);
        }
      // Score = T(T(q.k) * scale), as a matmul and a scale multiply in T;
      // the softmax input in log2 units is score * log2e + c with
      // c = log(block size / S) * log2e.
      float sc[16], cw[16];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float a0, a1;
        round_pair<T>(acc[r], acc[r + 1], a0, a1);
        round_pair<T>(a0 * p.scale, a1 * p.scale, sc[r], sc[r + 1]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) cw[r] = c_full;
      if (tail) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = kt0 + sub * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          cw[r] = j / SP == last_block ? c_last : c_full;
          if (j >= ns || (kPad && (j % SP) >= S)) sc[r] = -INFINITY;
        }
      }
      if (sweep == 0) {
        // Running max of x = score * log2e + c (log2e > 0: c_last differs
        // from c_full only in the tail).
        float mx = m2;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaf(sc[r], kLog2e, cw[r]));
        // While every key this lane has seen is masked (mx = -inf, as for
        // the lanes past the last sampled key when blocks * S <= 4), the
        // terms and the rescale take a finite reference and are exactly
        // zero, where -inf - (-inf) would make them NaN.
        const float mref = mx == -INFINITY ? 0.f : mx;
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sum += __builtin_amdgcn_exp2f(fmaf(sc[r], kLog2e, cw[r] - mref));
        l2 = l2 * __builtin_amdgcn_exp2f(m2 - mref) + sum;
        m2 = mx;
      } else if constexpr (kWide) {
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          sum += __builtin_amdgcn_exp2f(fmaf(sc[r], kLog2e, cw[r] - lse2));
        wide_acc += q_real ? sum : 0.f;
      } else {
        float pk[KBS];
#pragma unroll
        for (int b = 0; b < KBS; ++b) pk[b] = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int local = 8 * (r >> 2) + 4 * g + (r & 3);
          pk[local / SP] += __builtin_amdgcn_exp2f(fmaf(sc[r], kLog2e, cw[r] - lse2));
        }
        // Sum over the SP query lanes of each query block (padding lanes
        // add zero) and both halves.
#pragma unroll
        for (int b = 0; b < KBS; ++b) {
          if (kPad && !q_real) pk[b] = 0.f;
#pragma unroll
          for (int m = 1; m < SP; m <<= 1) pk[b] += __shfl_xor(pk[b], m);
          pk[b] += __shfl_xor(pk[b], 32);
        }
        if (g == 0 && (qi % SP) == 0) {
          const int qs_first = q0 + qi;
          if (qs_first < ns) {
            const int qb = qs_first / SP;
            float* out = p.mass + ((int64_t)h * p.blocks + qb) * p.blocks;
#pragma unroll
            for (int b = 0; b < KBS; ++b) {
              const int kb = (kt0 + sub * 32) / SP + b;
              if (kb < p.blocks) out[kb] = pk[b] / (float)S;
            }
          }
        }
      }
    }
    if constexpr (kWide) {
      // Key block (kt0 / SP) complete after this tile: publish this wave's sum.
      if (sweep == 1 && ((t + 1) * kTileKeys) % SP == 0) {
        const float total = dsa::wave_total(wide_acc);
        if (lane == 0) wide_part[(kt0 / SP) & 1][wave] = total;
        wide_acc = 0.f;
      }
    }
  };

  // kWide: writes the mass of key block kb from the wave sums published for
  // it (after a barrier); the waves of one query block are added in order.
  auto flush_wide = [&](int kb) __attribute__((always_inline)) {
    if constexpr (kWide) {
      constexpr int kWavesPerBlock = SP / 32;
      if (tid < 4 / kWavesPerBlock) {
        const int qb = (blockIdx.x * 128) / SP + tid;
        if (qb < p.blocks && kb < p.blocks) {
          float total = 0.f;
#pragma unroll
          for (int w = 0; w < kWavesPerBlock; ++w) total += wide_part[kb & 1][tid * kWavesPerBlock + w];
          p.mass[((int64_t)h * p.blocks + qb) * p.blocks + kb] = total / (float)S;
        }
      }
    }
  };

  // Step: wait for the current tile (and every older memory and LDS
  // operation), barrier (all waves' loads landed, every wave done with the
  // other stage, wave sums published), prefetch the next tile into the other
  // stage, write the key block finished by the previous tile (kWide), compute
  // the current one.
  auto step = [&](int t, int sweep, int next_t, const unsigned char* cur,
                  unsigned char* nxt) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWide ? 0x0070 : 0x0F70);  // vmcnt(0) [lgkmcnt(0)]
    __syncthreads();
    if (next_t >= 0) issue(next_t, nxt);
    if (kWide && sweep == 1 && t > 0 && (t * kTileKeys) % SP == 0) flush_wide(t * kTileKeys / SP - 1);
    compute(cur, t, sweep);
  };

  for (int sweep = 0; sweep < 2; ++sweep) {
    issue(0, st0);
    for (int t = 0; t < tiles; t += 2) {
      step(t, sweep, t + 1 < tiles ? t + 1 : -1, st0, st1);
      if (t + 1 >= tiles) break;
      step(t + 1, sweep, t + 2 < tiles ? t + 2 : -1, st1, st0);
    }
    if (sweep == 0) {  // each query's log-sum-exp (log2 units)
      // Lanes l and l ^ 32 hold the two halves of one query's keys; both get
      // the same total (the pair's two terms in one fixed order, so a
      // contracted fma rounds alike in both lanes).
      const auto ms = __builtin_amdgcn_permlane32_swap(__float_as_uint(m2), __float_as_uint(m2),
                                                       false, false);
      const auto ls = __builtin_amdgcn_permlane32_swap(__float_as_uint(l2), __float_as_uint(l2),
                                                       false, false);
      const float ma = __uint_as_float(ms[0]), mb = __uint_as_float(ms[1]);
      const float mx = fmaxf(ma, mb);
      const float tot = __uint_as_float(ls[0]) * __builtin_amdgcn_exp2f(ma - mx) +
                        __uint_as_float(ls[1]) * __builtin_amdgcn_exp2f(mb - mx);
      lse2 = mx + __builtin_log2f(tot);
      __syncthreads();  // every wave done with st0/st1 before sweep 2 refills st0
    }
  }
  if constexpr (kWide) {  // the last key block
    dsa::lds_barrier();
    flush_wide(p.blocks - 1);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

template <typename T, int kHalves>
void launch_mass(const MassParams& p, int sp, bool pad, dim3 grid, hipStream_t stream) {
#define DSA_MASS(SPV, PADV) \
  hipLaunchKernelGGL((sampled_mass_kernel<T, SPV, PADV, kHalves>), grid, dim3(256), 0, stream, p)
  if (!pad) {
    switch (sp) {
      case 1: DSA_MASS(1, false); break;
      case 2: DSA_MASS(2, false); break;
      case 4: DSA_MASS(4, false); break;
      case 8: DSA_MASS(8, false); break;
      case 16: DSA_MASS(16, false); break;
      default: DSA_MASS(32, false); break;
    }
  } else {
    switch (sp) {
      case 4: DSA_MASS(4, true); break;
      case 8: DSA_MASS(8, true); break;
      case 16: DSA_MASS(16, true); break;
      case 32: DSA_MASS(32, true); break;
      case 64: DSA_MASS(64, true); break;
      default: DSA_MASS(128, true); break;
    }
  }
#undef DSA_MASS
}

}  // namespace

extern "C" int dsa_sampled_mass(const void* q, const void* k, int32_t dtype,
                                const int64_t* strides, int32_t tokens, int32_t heads,
                                int32_t head_dim, int32_t block_size, int32_t samples,
                                float scale, float* mass, hipStream_t stream) {
  dsa::clear_error();
  if (!q || !k || !mass || !strides)
    return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: null pointer");
  if (dtype != DSA_BF16 && dtype != DSA_F16)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_sampled_mass: dtype %d unsupported (bf16 or fp16)",
                          dtype);
  if (tokens <= 0 || heads <= 0 || block_size <= 0)
    return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: tokens/heads/block must be positive");
  if (head_dim <= 0 || head_dim > 2 * kHeadDim || head_dim % 8 != 0)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_sampled_mass: head_dim %d unsupported (a multiple of 8 up to 256)",
                          head_dim);
  if (block_size > 128)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_sampled_mass: block_size %d unsupported (<= 128)",
                          block_size);
  if (samples <= 0 || samples > block_size)
    return dsa::set_error(DSA_EINVAL, "route_samples must be in [1, block_size]");
  if (!(scale > 0.f)) return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: scale must be > 0");
  if (!aligned16(q) || !aligned16(k))
    return dsa::set_error(DSA_EINVAL, "dsa_sampled_mass: q/k must be 16-byte aligned");
  for (int i = 0; i < 4; ++i)
    if (strides[i] % 8 != 0 || strides[i] < 0)
      return dsa::set_error(DSA_EINVAL,
                            "dsa_sampled_mass: stride %d not a non-negative multiple of 8", i);
  if (((int64_t)(tokens - 1) * strides[2] + kHeadDim) * 2 > 0x7fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED,
                          "dsa_sampled_mass: one head's K rows must span < 2 GiB");
  int sp = 1;
  while (sp < samples) sp <<= 1;  // power-of-two sample stride
  MassParams p;
  p.q = q;
  p.k = k;
  p.mass = mass;
  p.q_st = strides[0]; p.q_sh = strides[1]; p.k_st = strides[2]; p.k_sh = strides[3];
  p.tokens = tokens;
  p.heads = heads;
  p.block_size = block_size;
  p.samples = samples;
  p.head_dim = head_dim;
  p.blocks = (tokens + block_size - 1) / block_size;
  if ((int64_t)p.blocks * sp > 0x3fffffff)
    return dsa::set_error(DSA_EUNSUPPORTED, "dsa_sampled_mass: too many sampled tokens");
  p.scale = scale;
  // fp32 log of an fp32 quotient, as torch's (sizes.float() / samples).log().
  const int last = tokens - (p.blocks - 1) * block_size;
  p.logw_full = logf((float)block_size / (float)samples);
  p.logw_last = logf((float)last / (float)samples);
  const int ns = p.blocks * sp;
  const dim3 grid((unsigned)((ns + 127) / 128), (unsigned)heads);
  // Padded instances for sample counts that are not a power of two, and for
  // 64 and 128 samples (key and query blocks wider than a sub-tile or wave).
  const bool pad = sp != samples || sp > 32;
  const bool wide = head_dim > kHeadDim;
  if (dtype == DSA_F16)
    wide ? launch_mass<_Float16, 2>(p, sp, pad, grid, stream)
         : launch_mass<_Float16, 1>(p, sp, pad, grid, stream);
  else
    wide ? launch_mass<__bf16, 2>(p, sp, pad, grid, stream)
         : launch_mass<__bf16, 1>(p, sp, pad, grid, stream);
  return dsa::check_launch("dsa_sampled_mass");
}
