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
//  * O^T += V^T P^T: B = P^T straight from the score registers (bf16), A = V^T read from an LDS
//    copy of the tile stored transposed ([dim][key]).  The MFMA contraction order over keys is
//    permuted identically in A and B, which is what lets P^T stay in its accumulator layout.
//  * P V runs in fp16 (unit roundoff 2^-11, 8x finer than bf16 for P in (0, 1]): V is
//    converted bf16 -> fp16 while it is staged, which is exact for |v| in fp16's normal range.
//    A key tile holding any |v| > 65504 is staged and multiplied in bf16 instead (a
//    workgroup-uniform decision taken at the staging barrier).
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

template <int D>
struct AttnLds {
  static constexpr int KSTRIDE = D + 8;         // bf16 per K row (16-byte pad)
  static constexpr int VSTRIDE = kAttnBN + 4;   // bf16 per V^T row (8-byte pad)
  __bf16 k[kAttnBN * KSTRIDE];
  __bf16 vt[D * VSTRIDE];
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

template <int D, bool CAUSAL>
__device__ __forceinline__ void attention_fwd(const __bf16* __restrict__ q,
                                              const __bf16* __restrict__ k,
                                              const __bf16* __restrict__ v,
                                              __bf16* __restrict__ o, float* __restrict__ lse,
                                              int heads, int sq, int sk, i64 qsb, i64 qsh,
                                              i64 qss, i64 ksb, i64 ksh, i64 kss, i64 vsb,
                                              i64 vsh, i64 vss, float scale_log2) {
  static_assert(D % 32 == 0 && D <= 256, "head dim must be a multiple of 32");
  constexpr int KSTEPS = D / 16;          // MFMA k-steps of S^T
  constexpr int DBLK = D / 32;            // 32-row blocks of O^T
  constexpr int CHUNKS = D / 8;           // 16-byte chunks per row
  __shared__ AttnLds<D> sm;

  const int nqb = (sq + kAttnBM - 1) / kAttnBM;
  const int bh_count = gridDim.x / nqb;
  const int id = blockIdx.x;
  const int qb = nqb - 1 - id / bh_count;   // heaviest query block first
  const int bh = id % bh_count;
  const int b = bh / heads, h = bh % heads;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
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
#pragma unroll
  for (int a = 0; a < DBLK; ++a) oacc[a] = f32x16{};
  float m_run = -kInf, l_run = 0.0f;

  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + kAttnBM);
  const int ntiles = (kv_end + kAttnBN - 1) / kAttnBN;

  // cooperative tile loads: K as [key][dim] rows, V as 4-key x 8-dim blocks for transposition
  constexpr int NT = 64 * kAttnWaves;
  constexpr int KITEMS = kAttnBN * CHUNKS;                  // 16-byte K pieces per tile
  constexpr int VITEMS = (kAttnBN / 4) * CHUNKS;            // (key quad, dim chunk) V pieces
  constexpr int KLOADS = (KITEMS + NT - 1) / NT;
  constexpr int VLOADS = (VITEMS + NT - 1) / NT;
  u32x4 kbuf[KLOADS];
  u32x4 vbuf[VLOADS][4];

  auto fetch = [&](int tile) {
    const int k0 = tile * kAttnBN;
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = tid + i * NT;
      const int key = k0 + c / CHUNKS, ch = c % CHUNKS;
      kbuf[i] = (c < KITEMS && key < sk) ? load16_cached(kp + (i64)key * kss + ch * 8)
                                         : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < VLOADS; ++i) {
      const int c = tid + i * NT;
      const int ch = c % CHUNKS, quad = c / CHUNKS;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + quad * 4 + r;
        vbuf[i][r] = (c < VITEMS && key < sk) ? load16_cached(vp + (i64)key * vss + ch * 8)
                                              : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  // fp16 staging of V is exact unless a value exceeds fp16's range (65504 after rounding)
  auto v_overflows = [&]() -> int {
    int bad = 0;
#pragma unroll
    for (int i = 0; i < VLOADS; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const u32 x = vbuf[i][r][w];
          // bf16 magnitude bits >= 0x477f (65280 + half ulp region) can round past 65504
          bad |= ((x & 0x7fffu) >= 0x4780u) | (((x >> 16) & 0x7fffu) >= 0x4780u);
        }
      }
    }
    return bad;
  };
  auto to_f16 = [](u32 bf) -> u32 {  // one bf16 (low 16 bits) -> fp16 bits
    return half2_bits(__builtin_convertvector(f32x2{as_f32(bf << 16), 0.0f}, half2_t)) & 0xffffu;
  };
  auto stash = [&](bool f16v) {
#pragma unroll
    for (int i = 0; i < KLOADS; ++i) {
      const int c = tid + i * NT;
      const int key = c / CHUNKS, ch = c % CHUNKS;
      if (c < KITEMS) *(u32x4*)(sm.k + key * AttnLds<D>::KSTRIDE + ch * 8) = kbuf[i];
    }
#pragma unroll
    for (int i = 0; i < VLOADS; ++i) {
      const int c = tid + i * NT;
      if (c >= VITEMS) continue;
      const int ch = c % CHUNKS, quad = c / CHUNKS;
      // element j of the chunk is head dim ch*8 + j; write the 4 keys of the quad for it
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int word = j >> 1, shift = (j & 1) * 16;
        u32 e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          e[r] = (vbuf[i][r][word] >> shift) & 0xffffu;
          if (f16v) e[r] = to_f16(e[r]);
        }
        u32x2 w;
        w.x = e[0] | (e[1] << 16);
        w.y = e[2] | (e[3] << 16);
        *(u32x2*)(sm.vt + (ch * 8 + j) * AttnLds<D>::VSTRIDE + quad * 4) = w;
      }
    }
  };

  if (ntiles > 0) fetch(0);
  for (int tile = 0; tile < ntiles; ++tile) {
    // barrier: every wave is done with the previous tile in LDS; also decides the V format
    const bool f16v = __syncthreads_or(v_overflows()) == 0;
    stash(f16v);
    __syncthreads();
    if (tile + 1 < ntiles) fetch(tile + 1);
    const int k0 = tile * kAttnBN;
    const bool active = !CAUSAL || k0 <= qw + 31;
    if (!active) continue;
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
    // ---- scale, mask and the running max of this lane's query
    const bool diag = CAUSAL && (k0 + kAttnBN - 1 > qw);
    float tmax = -kInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
        float t = sacc[kb][r] * scale_log2;
        if ((diag && key > my_q) || key >= sk) t = -kInf;
        sacc[kb][r] = t;
        tmax = __builtin_fmaxf(tmax, t);
      }
    }
    tmax = __builtin_fmaxf(tmax, partner<32>(tmax));
    const float m_new = __builtin_fmaxf(m_run, tmax);
    // a fully masked query row (only past the end of the sequence) keeps m = -inf
    const float alpha = (m_new == -kInf) ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    const float m_use = (m_new == -kInf) ? 0.0f : m_new;
    float psum = 0.0f;
    u32 pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(sacc[kb][r] - m_use);
        const float p1 = __builtin_amdgcn_exp2f(sacc[kb][r + 1] - m_use);
        psum += p0 + p1;
        pk[kb][r >> 1] = f16v ? pack_f16x2(p0, p1) : pack_bf16x2(p0, p1);
      }
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int a = 0; a < DBLK; ++a) oacc[a] *= alpha;
    // ---- O^T += V^T P^T over the 4 key steps (16 keys each) of the tile
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kb = c >> 1, half = c & 1;
      u32x4 bw;
      bw.x = pk[kb][4 * half + 0];
      bw.y = pk[kb][4 * half + 1];
      bw.z = pk[kb][4 * half + 2];
      bw.w = pk[kb][4 * half + 3];
      const int kbase = kb * 32 + 16 * half + 4 * hi;
      if (f16v) {
        const f16x8 bop = __builtin_bit_cast(f16x8, bw);
#pragma unroll
        for (int a = 0; a < DBLK; ++a) {
          const _Float16* vrow = (const _Float16*)sm.vt + (a * 32 + l32) * AttnLds<D>::VSTRIDE + kbase;
          const f16x4 lo = *(const f16x4*)(vrow);
          const f16x4 up = *(const f16x4*)(vrow + 8);
          const f16x8 aop = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
          oacc[a] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop, bop, oacc[a], 0, 0, 0);
        }
      } else {
        const bf16x8 bop = __builtin_bit_cast(bf16x8, bw);
#pragma unroll
        for (int a = 0; a < DBLK; ++a) {
          const __bf16* vrow = sm.vt + (a * 32 + l32) * AttnLds<D>::VSTRIDE + kbase;
          const bf16x4 lo = *(const bf16x4*)(vrow);
          const bf16x4 up = *(const bf16x4*)(vrow + 8);
          const bf16x8 aop = __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7);
          oacc[a] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aop, bop, oacc[a], 0, 0, 0);
        }
      }
    }
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
      lse[(i64)bh * sq + my_q] = (m_run + __builtin_log2f(l_tot)) * 0.6931471805599453f;
  }
}

}  // namespace nep
