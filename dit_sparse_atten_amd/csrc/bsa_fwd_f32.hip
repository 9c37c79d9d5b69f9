// Attention forward in fp32 arithmetic on the matrix cores (gfx950): the
// float32 calls (fp32 in and out), dense calls with attention dropout, and
// calls of head dims 136..256, for every input type.
//
// Replaces, for those calls, the SDPA of the reference's DenseBackend
// (attention_backends/dense.py:34-47, which computes in the `dtype` it is
// given and hands dropout_p to SDPA) and the float32 `sparse_chunk` /
// `_dense_route` of MatrixSparseBackend (attention_backends/sparse.py:184-233,
// 670-751; it computes in q's own dtype, sparse.py:700-708).
//
// Design (per block of up to 128 query rows, one 4-wave workgroup, two per
// CU; wave w owns query rows 32 w .. 32 w + 31):
//  * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x2_f32.  The wave's
//    query rows are the B operand's columns, so each lane's 16 accumulators
//    belong to one query row, as in the 16-bit kernels (lane (g, i) holds
//    key 8 (r >> 2) + 4 g + (r & 3) of accumulator r, for row i).  In step s
//    of S^T, lane half g supplies dim (kD / 2) g + s: its row's Q from kD / 2
//    registers, key row i's K from LDS.  In O^T, step r takes each lane
//    half's own probability of accumulator r as B, and as A the four dims
//    4 i .. 4 i + 3 of that key's V row (one LDS read, one element per output
//    tile), so output tile dt holds dims 4 m + dt of accumulator row m;
//  * keys are staged as 32-key sub-tiles of K and V converted to fp32 (16 KB
//    each), double-buffered through registers; K's 16-byte chunks are XORed
//    with the key row & 15 so that the 16 lanes of a fragment read hit
//    distinct banks; V rows are plain (32 lanes read one 512-byte row);
//  * fp32 online softmax (exact running max, exp2), and the fp32
//    probabilities enter P V unrounded;
//  * kStats: per query row and key tile (one tile per key block), the row's
//    unnormalised mass log2 sum 2^(scale_log2 s) and its mass-weighted mean
//    key offsets, in the format the 16-bit kernels write (rs_logm, rs_mean)
//    for tile_stats_reduce_kernel; at kD = 256 the first of the two
//    launches writes them;
//  * kD = 256 (head dims 136..256): S^T runs over all 256 dims (128 Q
//    registers per lane), and O is computed in two launches of 128 output
//    dims each (`dim0` = 0, 128), each staging only its half of V, so the O
//    accumulators stay at 64 registers; the second launch recomputes S;
//  * kDropout (dense only): each probability enters P V as keep * p /
//    (1 - dropout_p); the normaliser counts every key, as dropout applied
//    after the softmax does.  keep = (u >= drop_thresh) for a uniform 32-bit
//    u from Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random
//    numbers: as easy as 1, 2, 3", SC 2011) with key (seed_lo, seed_hi) and
//    counter (key index / 4, query token, batch * heads + head, offset); its
//    four outputs are the uniforms of keys 4 c .. 4 c + 3.
#include <cmath>

#include "bsa_kernel.h"

namespace bsa {
namespace {

constexpr int kSubKeys = 32;  // keys per staged sub-tile (16 KB of V in fp32, 16 or 32 KB of K)
constexpr int kMaxHeadDim = 256;

template <typename T>
__device__ __forceinline__ dsa_f32x4 load4(const T* ptr) {
  if constexpr (std::is_same<T, float>::value) {
    return *reinterpret_cast<const dsa_f32x4*>(ptr);
  } else {
    const typename dsa::Elem<T>::x4 x = *reinterpret_cast<const typename dsa::Elem<T>::x4*>(ptr);
    return __builtin_convertvector(x, dsa_f32x4);
  }
}

template <typename T>
__device__ __forceinline__ void store4(T* ptr, dsa_f32x4 x) {
  if constexpr (std::is_same<T, float>::value) {
    *reinterpret_cast<dsa_f32x4*>(ptr) = x;
  } else {
    *reinterpret_cast<typename dsa::Elem<T>::x4*>(ptr) =
        __builtin_convertvector(x, typename dsa::Elem<T>::x4);
  }
}

__device__ __forceinline__ dsa_f32x16 mfma_f32(float a, float b, dsa_f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

}  // namespace

// Philox4x32-10: ten rounds of (hi, lo) = M x; out = {hi1 ^ c1 ^ k0, lo1,
// hi0 ^ c3 ^ k1, lo0} with M0 = 0xD2511F53 on c0 and M1 = 0xCD9E8D57 on c2,
// the key bumped by (0x9E3779B9, 0xBB67AE85) before every round but the
// first (Salmon et al., SC 2011).
__device__ __forceinline__ dsa_u32x4 philox4x32_10(dsa_u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int round = 0; round < 10; ++round) {
    if (round > 0) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
    c = dsa_u32x4{hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0};
  }
  return c;
}

// kD: the dims S^T runs over (128, or 256 for head dims 136..256); dim0: the
// first of the 128 output dims this launch computes.
template <typename T, int kD, bool kRouted, bool kStats, bool kDropout>
__global__ void __launch_bounds__(256, kD == 128 ? 2 : 1) bsa_fwd_f32_kernel(BsaParams p,
                                                                            int dim0) {
  static_assert(!(kDropout && (kRouted || kStats)), "dropout: dense attention only");
  constexpr int kHalfD = kD / 2;      // dims per lane half in S^T
  constexpr int kRowChunks = kD / 4;  // 16-byte chunks of a staged K row
  __shared__ __attribute__((aligned(16))) float ks[2][kSubKeys * kD];
  __shared__ __attribute__((aligned(16))) float vs[2][kSubKeys * kHeadDim];
  __shared__ dsa_f32x2 offs[kStats ? 128 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int qi = lane & 31;
  const int work = (int)blockIdx.x;
  const int qb = work % p.q_blocks;
  const int bh = work / p.q_blocks;
  const int h = bh % p.heads;
  const int b = bh / p.heads;

  int start = 0, end = p.kv_blocks;
  if (!kRouted && p.causal) {
    const int last_row = min(qb * p.block + p.block, p.q_tokens) - 1;
    end = min(p.kv_blocks, last_row / p.block + 1);
  }
  if (kRouted) {
    const dsa::const_i32 rp = (dsa::const_i32)p.row_ptr;
    const int rb = p.route_batches == 1 ? 0 : b;
    const int64_t row = ((int64_t)rb * p.heads + h) * p.q_blocks + qb;
    start = rp[row];
    end = rp[row + 1];
  }
  const dsa::const_i32 cidx = (dsa::const_i32)p.col_idx;
  const int nblk = end - start;

  const int local_row = wave * 32 + qi;
  const int tq = qb * p.block + local_row;
  const bool row_ok = local_row < p.block && tq < p.q_tokens;
  const bool wave_active = wave * 32 < p.block;
  const int tq_c = tq < p.q_tokens ? tq : p.q_tokens - 1;

  // Dims kHalfD g .. kHalfD g + kHalfD - 1 of the lane's query row (zeros
  // past head_dim).
  float qreg[kHalfD];
  {
    const T* qrow = static_cast<const T*>(p.q) + b * p.q_sb + h * p.q_sh +
                    (int64_t)tq_c * p.q_st + kHalfD * g;
#pragma unroll
    for (int u = 0; u < kHalfD / 4; ++u) {
      const dsa_f32x4 x =
          kHalfD * g + 4 * u < p.head_dim ? load4(qrow + 4 * u) : dsa_f32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[4 * u + e] = x[e];
    }
  }
  if constexpr (kStats) {
    // Tile-local (y, x) of each key offset in a block (zeros past it: the
    // masked keys of a partial sub-tile read them with p = 0).
    for (int i = tid; i < 128; i += 256) {
      const bool in = i < p.stat_tile;
      offs[i] = dsa_f32x2{in ? dsa::tile_axis(i / p.tile_w, p.tile_h) : 0.f,
                          in ? dsa::tile_axis(i % p.tile_w, p.tile_w) : 0.f};
    }
  }

  const T* kbase = static_cast<const T*>(p.k) + b * p.k_sb + h * p.k_sh;
  const T* vbase = static_cast<const T*>(p.v) + b * p.v_sb + h * p.v_sh;
  auto block_of = [&](int j) -> int {
    const int kb = kRouted ? cidx[start + j] : start + j;
    return (unsigned)kb < (unsigned)p.kv_blocks ? kb : -1;
  };
  // The first walk index at or past j whose key block is in range.
  auto next_valid = [&](int j) -> int {
    while (j < nblk && block_of(j) < 0) ++j;
    return j;
  };
  auto keys_of = [&](int kb) -> int { return min(p.block, p.kv_tokens - kb * p.block); };

  // Sub-tile staging: thread t moves elements 4 c .. 4 c + 3 of key rows
  // r = (256 u + t) / (row chunks), c = t % (row chunks): every dim of K, and
  // dims dim0 .. dim0 + 127 of V; rows past the sequence and dims past
  // head_dim stage zeros.
  constexpr int kKLoads = kSubKeys * kRowChunks / 256, kVLoads = kSubKeys * 32 / 256;
  dsa_f32x4 kreg[kKLoads], vreg[kVLoads];
  auto fetch = [&](int kb, int st) {
    const int key0 = kb * p.block + st * kSubKeys;
#pragma unroll
    for (int u = 0; u < kKLoads; ++u) {
      const int idx = u * 256 + tid, r = idx / kRowChunks, c = idx % kRowChunks;
      const int key = key0 + r;
      const bool ok = key < p.kv_tokens && 4 * c < p.head_dim;
      kreg[u] = ok ? load4(kbase + (int64_t)key * p.k_st + 4 * c) : dsa_f32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int idx = u * 256 + tid, r = idx >> 5, c = idx & 31;
      const int key = key0 + r;
      const bool ok = key < p.kv_tokens && dim0 + 4 * c < p.head_dim;
      vreg[u] = ok ? load4(vbase + (int64_t)key * p.v_st + dim0 + 4 * c) : dsa_f32x4{0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kKLoads; ++u) {
      const int idx = u * 256 + tid, r = idx / kRowChunks, c = idx % kRowChunks;
      *reinterpret_cast<dsa_f32x4*>(&ks[buf][r * kD + 4 * (c ^ (r & 15))]) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < kVLoads; ++u) {
      const int idx = u * 256 + tid, r = idx >> 5, c = idx & 31;
      *reinterpret_cast<dsa_f32x4*>(&vs[buf][r * kHeadDim + 4 * c]) = vreg[u];
    }
  };

  float m_run = -INFINITY;  // log2 units of the scaled scores
  float l_run = 0.f;
  dsa_f32x16 oacc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  float cm = 0.f, cy = 0.f, cx = 0.f;  // statistics of the open key tile

  auto compute = [&](int buf, int kb, int st) __attribute__((always_inline)) {
    const int key0 = kb * p.block + st * kSubKeys;
    const int valid = min(kSubKeys, min(p.block - st * kSubKeys, p.kv_tokens - key0));
    const int lim = !kRouted && p.causal ? tq - key0 + 1 : kSubKeys;
    dsa_f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    const float* krow = &ks[buf][qi * kD];
#pragma unroll
    for (int u = 0; u < kHalfD / 4; ++u) {
      const dsa_f32x4 kv = *reinterpret_cast<const dsa_f32x4*>(
          krow + 4 * (((kHalfD / 4) * g + u) ^ (qi & 15)));
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mfma_f32(kv[e], qreg[4 * u + e], s);
    }
    const int bound = min(valid, lim);
    if (bound < kSubKeys) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + 4 * g + (r & 3) >= bound) s[r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = dsa::pair32_max(mx) * p.scale_log2;
    const float m_new = fmaxf(m_run, mx);
    if (__any(m_new != m_run)) {
      const float alpha = m_new == m_run ? 1.f : exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
      if constexpr (kStats) {
        cm *= alpha;
        cy *= alpha;
        cx *= alpha;
      }
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float pr[16];
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      pr[r] = exp2f(fmaf(s[r], p.scale_log2, -m_use));
      sum += pr[r];
    }
    l_run += sum;
    if constexpr (kStats) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const dsa_f32x2 o = offs[st * kSubKeys + 8 * (r >> 2) + 4 * g + (r & 3)];
        cm += pr[r];
        cy = fmaf(pr[r], o[0], cy);
        cx = fmaf(pr[r], o[1], cx);
      }
    }
    if constexpr (kDropout) {
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const uint32_t key = (uint32_t)(key0 + 8 * grp + 4 * g);
        const dsa_u32x4 u = philox4x32_10(
            dsa_u32x4{key >> 2, (uint32_t)tq_c, (uint32_t)bh, p.drop_offset}, p.drop_seed_lo,
            p.drop_seed_hi);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          pr[4 * grp + e] = u[e] >= p.drop_thresh ? pr[4 * grp + e] * p.drop_scale : 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 8 * (r >> 2) + 4 * g + (r & 3);
      const dsa_f32x4 vv = *reinterpret_cast<const dsa_f32x4*>(&vs[buf][key * kHeadDim + 4 * qi]);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) oacc[dt] = mfma_f32(vv[dt], pr[r], oacc[dt]);
    }
  };

  // The statistics of walk index j (key block kb), after its last sub-tile.
  auto close_tile = [&](int j, int kb) {
    const float tm = dsa::pair32_sum(cm), ty = dsa::pair32_sum(cy), tx = dsa::pair32_sum(cx);
    if (g == 0 && row_ok) {
      int64_t at;
      bool ok = true;
      if (kRouted) {
        const int64_t e = start + j;
        at = e * p.block + local_row;
        ok = e < p.rs_entries;
      } else {
        at = ((int64_t)h * p.kv_blocks + kb) * p.q_tokens + tq;
      }
      if (ok) {
        p.rs_logm[at] = tm > 0.f ? log2f(tm) + m_run : -INFINITY;
        if (p.rs_mean != nullptr) {
          const float inv = tm > 0.f ? 1.f / tm : 0.f;
          const dsa_f16x2 mean =
              __builtin_convertvector(dsa_f32x2{ty * inv, tx * inv}, dsa_f16x2);
          p.rs_mean[at] = __builtin_bit_cast(uint32_t, mean);
        }
      }
    }
    cm = cy = cx = 0.f;
  };

  int j = next_valid(0), st = 0;
  int kb = j < nblk ? block_of(j) : -1;
  if (j < nblk) {
    fetch(kb, 0);
    store(0);
  }
  dsa::lds_barrier();
  int buf = 0;
  while (j < nblk) {
    int nj = j, nst = st + 1, nkb = kb;
    if (nst * kSubKeys >= keys_of(kb)) {
      nst = 0;
      nj = next_valid(j + 1);
      nkb = nj < nblk ? block_of(nj) : -1;
    }
    const bool more = nj < nblk;
    if (more) fetch(nkb, nst);
    if (wave_active) {
      compute(buf, kb, st);
      if constexpr (kStats) {
        if (nst == 0) close_tile(j, kb);
      }
    }
    if (more) store(buf ^ 1);
    dsa::lds_barrier();
    buf ^= 1;
    j = nj;
    st = nst;
    kb = nkb;
  }

  const float l_tot = dsa::pair32_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok) {
    T* orow = static_cast<T*>(p.o) + b * p.o_sb + h * p.o_sh + (int64_t)tq * p.o_st;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int m = 8 * (rr >> 2) + 4 * g + (rr & 3);
      if (dim0 + 4 * m < p.head_dim)
        store4(orow + dim0 + 4 * m, dsa_f32x4{oacc[0][rr] * inv, oacc[1][rr] * inv,
                                              oacc[2][rr] * inv, oacc[3][rr] * inv});
    }
    if (p.lse && g == 0 && dim0 == 0)
      p.lse[((int64_t)b * p.heads + h) * p.q_tokens + tq] =
          l_tot > 0.f ? m_run * 0.6931471805599453f + logf(l_tot) : -INFINITY;
  }
}

template <typename T>
int launch_f32_typed(const BsaParams& p, hipStream_t stream, const char* who) {
  const int64_t grid = (int64_t)p.batch * p.heads * p.q_blocks;
  const dim3 blocks((unsigned)grid), threads(256);
  auto run = [&](auto kernel, int dim0) {
    hipLaunchKernelGGL(kernel, blocks, threads, 0, stream, p, dim0);
  };
  if (p.head_dim > kHeadDim) {
    // Head dims 136..256: two launches of 128 output dims each; the first
    // also writes the statistics (both see the same probabilities).
    if (p.rs_logm && p.drop_thresh != 0)
      return dsa::set_error(DSA_EUNSUPPORTED, "%s: dropout takes dense attention only", who);
    for (int dim0 = 0; dim0 < p.head_dim; dim0 += kHeadDim) {
      const bool stats = p.rs_logm && dim0 == 0;
      if (p.drop_thresh != 0) {
        if (p.row_ptr)
          return dsa::set_error(DSA_EUNSUPPORTED, "%s: dropout takes dense attention only", who);
        run(bsa_fwd_f32_kernel<T, kMaxHeadDim, false, false, true>, dim0);
      } else if (p.row_ptr) {
        if (stats) run(bsa_fwd_f32_kernel<T, kMaxHeadDim, true, true, false>, dim0);
        else run(bsa_fwd_f32_kernel<T, kMaxHeadDim, true, false, false>, dim0);
      } else {
        if (stats) run(bsa_fwd_f32_kernel<T, kMaxHeadDim, false, true, false>, dim0);
        else run(bsa_fwd_f32_kernel<T, kMaxHeadDim, false, false, false>, dim0);
      }
    }
  } else if (p.drop_thresh != 0) {
    if (p.row_ptr || p.rs_logm)
      return dsa::set_error(DSA_EUNSUPPORTED, "%s: dropout takes dense attention only", who);
    run(bsa_fwd_f32_kernel<T, kHeadDim, false, false, true>, 0);
  } else if constexpr (std::is_same<T, float>::value) {
    if (p.row_ptr) {
      if (p.rs_logm) run(bsa_fwd_f32_kernel<float, kHeadDim, true, true, false>, 0);
      else run(bsa_fwd_f32_kernel<float, kHeadDim, true, false, false>, 0);
    } else {
      if (p.rs_logm) run(bsa_fwd_f32_kernel<float, kHeadDim, false, true, false>, 0);
      else run(bsa_fwd_f32_kernel<float, kHeadDim, false, false, false>, 0);
    }
  } else {
    return dsa::set_error(DSA_EUNSUPPORTED, "%s: 16-bit inputs run the 16-bit kernels", who);
  }
  return dsa::check_launch(who);
}

}  // namespace bsa

// fp32-compute launches: every call of fp32 inputs (dtype DSA_F32), dense
// calls with dropout, and calls of head dims 136..256 of any input type.
int bsa_launch_f32(bsa::BsaParams p, int32_t dtype, hipStream_t stream, const char* who) {
  if (dtype == DSA_F32) return bsa::launch_f32_typed<float>(p, stream, who);
  if (dtype == DSA_F16) return bsa::launch_f32_typed<_Float16>(p, stream, who);
  return bsa::launch_f32_typed<__bf16>(p, stream, who);
}
