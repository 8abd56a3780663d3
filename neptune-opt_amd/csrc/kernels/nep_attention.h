// nep_attention.h -- causal online-softmax attention fold on gfx950 MFMA (bf16 in, fp32 acc).
//
// O = softmax(scale * Q K^T + causal mask) V per (batch, head), evaluated as a fold over key
// tiles with the logsumexp repair: running max m, running sum l and accumulator O are moved to
// a new max by exp(m - m') (the logsumexp skeleton's slope exp(s - s2)), so no score matrix is
// materialised.  Scores live in the base-2 domain t = scale*log2(e) * q.k.
//
// Mapping (one workgroup = 4 wave64s = BLOCK_M = 128 queries, 32 per wave; key tiles of 64):
//  * S^T = K Q^T with v_mfma_f32_32x32x16_bf16: A = K rows (key = lane%32, 8 consecutive head
//    dims per lane from LDS), B = Q^T (query = lane%32, 8 head dims, held in registers).  The
//    32x32 result gives lane l the scores of query l%32 for keys 8*(r/4) + 4*(l/32) + r%4, so
//    the softmax of a query needs its own 32 registers plus one exchange with lane l^32.
//  * O^T += V^T P^T: B = P^T straight from the score registers, A = V^T read from an LDS copy
//    of the tile stored transposed ([dim][key]).  The MFMA contraction order over keys is
//    permuted identically in A and B, which is what lets P^T stay in its accumulator layout.
//  * P V runs in fp16 (unit roundoff 2^-11, 8x finer than bf16 for P): V is converted
//    bf16 -> fp16 while staged, exact for |v| < 65536.  If any staged V tile of a query block
//    holds a larger magnitude, the block is recomputed with P V in bf16 (a second instance of
//    the loop, so the two modes do not add up in registers).
//  * Lazy rescaling: the reference max only moves when the running max exceeds it by more than
//    8 (base 2), so P <= 256 (exact range of fp16) and O is rescaled on few tiles.
//  * The row sum l accumulates the fp16-rounded P with v_dot2 (the values the MFMA multiplies).
//  * Tiles above the causal diagonal are skipped per wave; workgroups run heaviest query block
//    first and a head's blocks share one XCD (workgroup id % 8 == head % 8), so its K/V stay in
//    that XCD's L2.
#pragma once

namespace nep {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kAttnBM = 128;           // queries per workgroup
constexpr int kAttnBN = 64;            // keys per tile
constexpr int kAttnWaves = 4;
constexpr float kRescaleSlack = 8.0f;  // base-2 headroom before the reference max moves

template <int D>
struct AttnLds {
  static constexpr int KSTRIDE = D + 8;         // bf16 per K row (16-byte pad)
  static constexpr int VSTRIDE = kAttnBN + 4;   // 16-bit words per V^T row (8-byte pad)
  __bf16 k[kAttnBN * KSTRIDE];
  u16 vt[D * VSTRIDE];
};

__device__ __forceinline__ u32 pack_bf16x2(float a, float b) {
  f32x2 f = {a, b};
  bf16x2 h = __builtin_convertvector(f, bf16x2);
  return __builtin_bit_cast(u32, h);
}
__device__ __forceinline__ u32 pack_f16x2(float a, float b) {
  f32x2 f = {a, b};
  half2_t h = __builtin_convertvector(f, half2_t);
  return half2_bits(h);
}

// Per-query-block state and the key-tile loop, in one P V precision.
template <int D, bool CAUSAL, bool F16V>
struct AttnBlock {
  static constexpr int KSTEPS = D / 16;          // MFMA k-steps of S^T
  static constexpr int DBLK = D / 32;            // 32-row blocks of O^T
  static constexpr int CHUNKS = D / 8;           // 16-byte chunks per row
  static constexpr int NT = 64 * kAttnWaves;
  static constexpr int KITEMS = kAttnBN * CHUNKS;           // 16-byte K pieces per tile
  static constexpr int VITEMS = (kAttnBN / 4) * CHUNKS;     // (key quad, dim chunk) V pieces
  static constexpr int KLOADS = (KITEMS + NT - 1) / NT;
  static constexpr int VLOADS = (VITEMS + NT - 1) / NT;

  // Runs the block; returns false (after a uniform early exit) if F16V meets an fp16 overflow.
  __device__ static bool run(AttnLds<D>& sm, const bf16x8* qreg, const __bf16* kp,
                             const __bf16* vp, i64 kss, i64 vss, int sk, int q0, int qw,
                             int my_q, float c, f32x16* oacc, float& m_out, float& l_out) {
    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hi = lane >> 5;
    int kv_end = sk;
    if constexpr (CAUSAL) kv_end = min(sk, q0 + kAttnBM);
    const int ntiles = (kv_end + kAttnBN - 1) / kAttnBN;
#pragma unroll
    for (int a = 0; a < DBLK; ++a) oacc[a] = f32x16{};
    float m_ref = -kInf;   // reference max (base 2) of this lane's query
    float l_run = 0.0f;

    u32x4 kbuf[KLOADS];
    u32x4 vbuf[VLOADS][4];
    auto fetch = [&](int tile) {
      const int k0 = tile * kAttnBN;
#pragma unroll
      for (int i = 0; i < KLOADS; ++i) {
        const int cc = tid + i * NT;
        const int key = k0 + cc / CHUNKS, ch = cc % CHUNKS;
        kbuf[i] = (cc < KITEMS && key < sk) ? load16_cached(kp + (i64)key * kss + ch * 8)
                                            : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < VLOADS; ++i) {
        const int cc = tid + i * NT;
        const int ch = cc % CHUNKS, quad = cc / CHUNKS;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + quad * 4 + r;
          vbuf[i][r] = (cc < VITEMS && key < sk) ? load16_cached(vp + (i64)key * vss + ch * 8)
                                                 : u32x4{0u, 0u, 0u, 0u};
        }
      }
    };
    // any |v| >= 65536 (bf16 magnitude bits >= 0x4780) does not fit fp16
    auto overflow = [&]() -> int {
      u32 mx = 0;
#pragma unroll
      for (int i = 0; i < VLOADS; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const u32 x = vbuf[i][r][w] & 0x7fff7fffu;
            mx = max(mx, max(x & 0xffffu, x >> 16));
          }
      return mx >= 0x4780u ? 1 : 0;
    };
    auto stash = [&]() {
#pragma unroll
      for (int i = 0; i < KLOADS; ++i) {
        const int cc = tid + i * NT;
        const int key = cc / CHUNKS, ch = cc % CHUNKS;
        if (cc < KITEMS) *(u32x4*)(sm.k + key * AttnLds<D>::KSTRIDE + ch * 8) = kbuf[i];
      }
#pragma unroll
      for (int i = 0; i < VLOADS; ++i) {
        const int cc = tid + i * NT;
        if (cc >= VITEMS) continue;
        const int ch = cc % CHUNKS, quad = cc / CHUNKS;
        // head dim ch*8 + j of the 4 keys of the quad -> V^T[dim][quad*4 .. +3]
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int word = j >> 1;
          u32 e[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) e[r] = vbuf[i][r][word];
          u32x2 w;
          if constexpr (F16V) {
            // bf16 -> fp32 is a shift / mask; two fp32 -> one packed fp16 pair (exact here)
            if (j & 1) {
              w.x = pack_f16x2(as_f32(e[0] & 0xffff0000u), as_f32(e[1] & 0xffff0000u));
              w.y = pack_f16x2(as_f32(e[2] & 0xffff0000u), as_f32(e[3] & 0xffff0000u));
            } else {
              w.x = pack_f16x2(as_f32(e[0] << 16), as_f32(e[1] << 16));
              w.y = pack_f16x2(as_f32(e[2] << 16), as_f32(e[3] << 16));
            }
          } else {
            if (j & 1) {
              w.x = (e[0] >> 16) | (e[1] & 0xffff0000u);
              w.y = (e[2] >> 16) | (e[3] & 0xffff0000u);
            } else {
              w.x = (e[0] & 0xffffu) | (e[1] << 16);
              w.y = (e[2] & 0xffffu) | (e[3] << 16);
            }
          }
          *(u32x2*)(sm.vt + (ch * 8 + j) * AttnLds<D>::VSTRIDE + quad * 4) = w;
        }
      }
    };

    if (ntiles > 0) fetch(0);
    for (int tile = 0; tile < ntiles; ++tile) {
      // barrier: every wave is done with the previous tile in LDS (and, in fp16 mode, the
      // workgroup agrees on whether this V tile fits fp16)
      if constexpr (F16V) {
        if (__syncthreads_or(overflow())) return false;
      } else {
        __syncthreads();
      }
      stash();
      __syncthreads();
      if (tile + 1 < ntiles) fetch(tile + 1);
      const int k0 = tile * kAttnBN;
      if (CAUSAL && k0 > qw + 31) continue;   // tile entirely above this wave's diagonal
      // ---- S^T = K Q^T for the two 32-key blocks of the tile
      f32x16 sacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = f32x16{};
        const __bf16* krow = sm.k + (kb * 32 + l32) * AttnLds<D>::KSTRIDE + 8 * hi;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const bf16x8 a = *(const bf16x8*)(krow + 16 * s);
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[s], sacc[kb], 0, 0, 0);
        }
      }
      // ---- masks only on the diagonal tile and the ragged last tile
      const bool need_mask = (CAUSAL && k0 + kAttnBN - 1 > qw) || (k0 + kAttnBN > sk);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
            if ((CAUSAL && key > my_q) || key >= sk) sacc[kb][r] = -kInf;
          }
      }
      float tmax = -kInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) tmax = __builtin_fmaxf(tmax, sacc[kb][r]);
      tmax = __builtin_fmaxf(tmax, partner<32>(tmax)) * c;
      // move the reference max only when P would exceed 2^8 (or on the first finite tile)
      const bool move = tmax > m_ref + kRescaleSlack;
      if (__builtin_amdgcn_ballot_w64(move) != 0) {
        const float m_new = move ? tmax : m_ref;
        const float alpha = (m_ref == -kInf) ? 0.0f : __builtin_amdgcn_exp2f(m_ref - m_new);
        l_run *= alpha;
#pragma unroll
        for (int a = 0; a < DBLK; ++a) oacc[a] *= alpha;
        m_ref = m_new;
      }
      const float shift = (m_ref == -kInf) ? 0.0f : m_ref;
      u32 pk[2][8];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r], c, -shift));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r + 1], c, -shift));
          if constexpr (F16V) {
            const u32 w = pack_f16x2(p0, p1);
            pk[kb][r >> 1] = w;
            l_run = __builtin_amdgcn_fdot2(as_half2(w), half2_t{(_Float16)1.0f, (_Float16)1.0f},
                                           l_run, false);
          } else {
            pk[kb][r >> 1] = pack_bf16x2(p0, p1);
            l_run += p0 + p1;
          }
        }
      // ---- O^T += V^T P^T over the 4 key steps (16 keys each) of the tile
#pragma unroll
      for (int cs = 0; cs < 4; ++cs) {
        const int kb = cs >> 1, half = cs & 1;
        u32x4 bw;
        bw.x = pk[kb][4 * half + 0];
        bw.y = pk[kb][4 * half + 1];
        bw.z = pk[kb][4 * half + 2];
        bw.w = pk[kb][4 * half + 3];
        const int kbase = kb * 32 + 16 * half + 4 * hi;
#pragma unroll
        for (int a = 0; a < DBLK; ++a) {
          const u16* vrow = sm.vt + (a * 32 + l32) * AttnLds<D>::VSTRIDE + kbase;
          const u32x2 lo = *(const u32x2*)(vrow);
          const u32x2 up = *(const u32x2*)(vrow + 8);
          const u32x4 av = {lo.x, lo.y, up.x, up.y};
          if constexpr (F16V) {
            oacc[a] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, av),
                                                             __builtin_bit_cast(f16x8, bw),
                                                             oacc[a], 0, 0, 0);
          } else {
            oacc[a] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av),
                                                              __builtin_bit_cast(bf16x8, bw),
                                                              oacc[a], 0, 0, 0);
          }
        }
      }
    }
    m_out = m_ref;
    l_out = l_run;
    return true;
  }
};

template <int D, bool CAUSAL>
__device__ __forceinline__ void attention_fwd(const __bf16* __restrict__ q,
                                              const __bf16* __restrict__ k,
                                              const __bf16* __restrict__ v,
                                              __bf16* __restrict__ o, float* __restrict__ lse,
                                              int heads, int sq, int sk, i64 qsb, i64 qsh,
                                              i64 qss, i64 ksb, i64 ksh, i64 kss, i64 vsb,
                                              i64 vsh, i64 vss, float scale_log2) {
  static_assert(D % 32 == 0 && D <= 256, "head dim must be a multiple of 32");
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  __shared__ AttnLds<D> sm;

  const int nqb = (sq + kAttnBM - 1) / kAttnBM;
  const int bh_count = gridDim.x / nqb;
  const int id = blockIdx.x;
  const int qb = nqb - 1 - id / bh_count;   // heaviest query block first
  const int bh = id % bh_count;
  const int b = bh / heads, h = bh % heads;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * kAttnBM, qw = q0 + wave * 32;
  const int my_q = qw + l32;
  const __bf16* qp = q + b * qsb + h * qsh;
  const __bf16* kp = k + b * ksb + h * ksh;
  const __bf16* vp = v + b * vsb + h * vsh;

  // Q^T operand: query my_q, head dims [16s + 8*hi, +8) for k-step s.
  bf16x8 qreg[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    if (my_q < sq) qreg[s] = *(const bf16x8*)(qp + (i64)my_q * qss + 16 * s + 8 * hi);
    else qreg[s] = bf16x8{};
  }
  f32x16 oacc[DBLK];
  float m_ref, l_run;
  if (!AttnBlock<D, CAUSAL, true>::run(sm, qreg, kp, vp, kss, vss, sk, q0, qw, my_q,
                                        scale_log2, oacc, m_ref, l_run)) {
    __syncthreads();
    AttnBlock<D, CAUSAL, false>::run(sm, qreg, kp, vp, kss, vss, sk, q0, qw, my_q,
                                     scale_log2, oacc, m_ref, l_run);
  }
  // ---- readout: O / l, and the natural-log LSE of the scaled scores
  const float l_tot = l_run + partner<32>(l_run);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (my_q < sq) {
    __bf16* orow = o + ((i64)bh * sq + my_q) * D;
#pragma unroll
    for (int a = 0; a < DBLK; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w.x = pack_bf16x2(oacc[a][4 * g + 0] * inv, oacc[a][4 * g + 1] * inv);
        w.y = pack_bf16x2(oacc[a][4 * g + 2] * inv, oacc[a][4 * g + 3] * inv);
        *(u32x2*)(orow + a * 32 + 8 * g + 4 * hi) = w;
      }
    }
    if (lse != nullptr && hi == 0)
      lse[(i64)bh * sq + my_q] = (m_ref + __builtin_log2f(l_tot)) * 0.6931471805599453f;
  }
}

}  // namespace nep
