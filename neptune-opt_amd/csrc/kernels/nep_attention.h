// nep_attention.h -- causal online-softmax attention fold on gfx950 MFMA (bf16 or fp16 in,
// fp32 accumulation).
//
// O = softmax(scale * Q K^T + causal mask) V per (batch, head), evaluated as a fold over key
// tiles with the logsumexp repair: running max m, running sum l and accumulator O are moved to
// a new max by exp(m - m') (the logsumexp skeleton's slope exp(s - s2)), so no score matrix is
// materialised.  Scores live in the base-2 domain t = scale*log2(e) * q.k.
//
// Two kernels per call:
//  * attention_vt_pack: V [key][dim] -> per key tile a V^T image in fp16 (the exact MFMA
//    operand order, XOR-swizzled for conflict-free LDS reads) plus one power-of-two exponent
//    per tile.  Tiles whose largest finite |v| reaches 2^15 are stored as v * 2^-e (exact: a
//    16-bit input keeps its significant bits in fp16 down to |v| >= 2^(e-14)); the fold feeds
//    such a tile P * 2^e instead of P and weights its row sum by 2^-e, both exact, so no
//    accumulator is rescaled.  A tile value below 2^(e-14) keeps an absolute precision of
//    2^(e-25) only, so the fold takes tiles with e <= e_max on this path.  The stored exponent
//    is the tile's own (kVtNonFinite for a tile holding inf or NaN).  The image is written
//    once per call and read by every query block of the head.
//  * attention_fwd: one workgroup = 8 wave64s = BLOCK_M = 256 queries (32 per wave), one
//    workgroup per CU (two waves per SIMD): each staged K / V^T tile serves 256 queries.
//    K (the caller's strided rows, bounds-checked buffer loads) and the V^T image go
//    straight from HBM into double-buffered LDS (buffer_load ... lds, no registers): tile t+1
//    is in flight while tile t is computed, with one barrier per tile.  A workgroup that read
//    a tile exponent above e_max (|v| >= 2^(e_max+15), inf or NaN in V) recomputes its
//    queries with attention_exact_rows instead: fp32 scores, fp32 P and the caller's V, so
//    every input has a defined result without a device-side trap or a host round trip.
//
// MFMA mapping (v_mfma_f32_32x32x16_{bf16,f16}):
//  * S^T = K Q^T: A = K rows (key = lane%32, 8 consecutive head dims per lane from LDS),
//    B = Q^T (query = lane%32, 8 head dims, registers).  Lane l holds the scores of query l%32
//    for keys 8*(r/4) + 4*(l/32) + r%4 (register r), so a query's softmax needs its own 32
//    registers plus one exchange with lane l^32.
//  * O^T += V^T P^T: B = P^T straight from the score registers (fp16), A = 8 fp16 of V^T row
//    `dim` for the same keys, which the V^T image stores contiguously.  The contraction order
//    over keys is permuted identically in A and B.
//  * P V in fp16 (unit roundoff 2^-11, 8x finer than bf16 for P).
//  * Lazy rescaling: the reference max only moves when the running max exceeds it by more than
//    8 (base 2), so P <= 256 (exact range of fp16) and O is rescaled on few tiles.
//  * The row sum l accumulates the fp32 P (before its fp16 rounding), so the logsumexp side
//    output carries fp32 accuracy; O is normalised by the same l.
//  * Tiles above the causal diagonal are skipped per wave; workgroups run heaviest query block
//    first and a head's blocks share one XCD (workgroup id % 8 == head % 8), so its K and V^T
//    stay in that XCD's L2.
#pragma once

namespace nep {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// wave64s per fold workgroup (32 queries each): two per SIMD up to head dim 128; at head dim
// 256 a wave's O^T and Q^T operands alone take 192 registers, so one wave per SIMD
template <int D>
constexpr int attn_waves() { return D <= 128 ? 8 : 4; }
constexpr int kAttnBN = 64;            // keys per tile
constexpr int kAttnThreads = 256;      // V^T pack workgroup: 4 wave64s
constexpr float kRescaleSlack = 8.0f;  // base-2 headroom before the reference max moves
constexpr u32 kRawBufferWord3 = 0x00020000u;   // gfx9 raw buffer descriptor, dword 3
constexpr u32 kVtScaleFrom = 142u;     // fp32 biased exponent of 2^15: tiles at or above scale
constexpr int kVtNonFinite = 255;      // tile exponent recorded for a tile holding inf or NaN
constexpr int kVtExpClamp = 24;        // largest exponent the fold's scaling arithmetic takes

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
// 2^k for |k| <= 126 (exact, built from the exponent field)
__device__ __forceinline__ float exp2_int(int k) { return as_f32((u32)(127 + k) << 23); }

// The 16-bit input types: widening of the low / high element of a packed pair, RNE packing of
// two fp32 values, the 8-element MFMA operand and the QK^T MFMA of that type.
template <typename T>
struct AttnIn;
template <>
struct AttnIn<__bf16> {
  typedef bf16x8 vec8;
  __device__ static __forceinline__ float lo(u32 w) { return as_f32(w << 16); }
  __device__ static __forceinline__ float hi(u32 w) { return as_f32(w & 0xffff0000u); }
  __device__ static __forceinline__ u32 pack2(float a, float b) { return pack_bf16x2(a, b); }
  __device__ static __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct AttnIn<_Float16> {
  typedef f16x8 vec8;
  __device__ static __forceinline__ float lo(u32 w) { return (float)as_half2(w)[0]; }
  __device__ static __forceinline__ float hi(u32 w) { return (float)as_half2(w)[1]; }
  __device__ static __forceinline__ u32 pack2(float a, float b) { return pack_f16x2(a, b); }
  __device__ static __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Position (0..63, before the row swizzle) of tile key `key` in a V^T image row: chunk
// j = 2*(key/16) + (key/4)%2 holds keys 16*(j/2) + 4*(j%2) + {0,1,2,3} and the same + 8, which
// is the key order of lane (j%2)*32 + .. in the P^T operand of k-step j/2.
__device__ __forceinline__ int vt_slot(int key) {
  const int w = key & 15;
  return ((key >> 4) * 2 + ((w >> 2) & 1)) * 8 + (w & 3) + ((w >> 3) << 2);
}

// LDS rows are read 16 bytes per lane, 16 consecutive rows per LDS cycle (64 banks of 4 bytes,
// 256 bytes per clock).  Row r keeps its 16-byte chunk c at position c ^ swizzle<CH>(r), so the
// 16 rows of one cycle hit 16 different bank groups: rows of 16 or 32 chunks XOR with r % 16,
// rows of 8 chunks (128 bytes: two rows per 256-byte bank sweep) XOR with (r / 2) % 8.
template <int CH>
__device__ __forceinline__ int swizzle(int row) {
  static_assert(CH == 8 || CH == 16 || CH == 32, "rows of 8, 16 or 32 chunks");
  if constexpr (CH >= 16) return row & 15;
  else return (row >> 1) & 7;
}

// V [keys, D] of one head -> fp16 V^T tile images [ntiles][D][64] (16-byte chunk j of row d
// stored at chunk j ^ swizzle<8>(d)) and one exponent per tile: 0 below 2^15, e for a largest
// finite |v| in [2^(14+e), 2^(15+e)), kVtNonFinite for a tile holding inf or NaN.  The image
// of a tile is scaled by 2^-min(e, kVtExpClamp).  Keys past sk are zero.
template <typename T, int D>
__device__ __forceinline__ void attention_vt_pack(const T* __restrict__ v, u16* __restrict__ vt,
                                                  int* __restrict__ exps, int heads, int sk,
                                                  i64 vsb, i64 vsh, i64 vss) {
  typedef AttnIn<T> In;
  constexpr int CH = D / 8;                         // 16-byte chunks per key row
  constexpr int UNITS = (kAttnBN / 2) * CH;         // (key pair, dim chunk) units
  constexpr int UPT = UNITS / kAttnThreads;
  static_assert(UNITS % kAttnThreads == 0, "head dim must be 64, 128 or 256");
  __shared__ __attribute__((aligned(16))) u16 img[D * kAttnBN];
  __shared__ u32 wave_max[kAttnThreads / 64];
  __shared__ int wave_bad[kAttnThreads / 64];
  const int ntiles = (sk + kAttnBN - 1) / kAttnBN;
  const int bh = blockIdx.x / ntiles, t = blockIdx.x % ntiles;
  const int b = bh / heads, h = bh % heads;
  const T* vp = v + b * vsb + h * vsh;
  const int k0 = t * kAttnBN, tid = threadIdx.x;

  u32x4 raw[UPT][2];
  u32 mx = 0;      // largest finite magnitude (fp32 bits: integer order = magnitude order)
  int bad = 0;     // a non-finite value in the tile
#pragma unroll
  for (int u = 0; u < UPT; ++u) {
    const int unit = tid + u * kAttnThreads, kp = unit / CH, ch = unit % CH;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int key = k0 + 2 * kp + r;
      raw[u][r] = key < sk ? load16_cached(vp + (i64)key * vss + ch * 8) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32 a = as_u32(In::lo(raw[u][r][w])) & 0x7fffffffu;
        const u32 c = as_u32(In::hi(raw[u][r][w])) & 0x7fffffffu;
        bad |= (a >= 0x7f800000u) | (c >= 0x7f800000u);
        mx = max(mx, max(a < 0x7f800000u ? a : 0u, c < 0x7f800000u ? c : 0u));
      }
    }
  }
  mx = max(mx, partner_u32<1>(mx));
  mx = max(mx, partner_u32<2>(mx));
  mx = max(mx, partner_u32<4>(mx));
  mx = max(mx, partner_u32<8>(mx));
  mx = max(mx, partner_u32<16>(mx));
  mx = max(mx, partner_u32<32>(mx));
  bad = group_or<64>(bad);
  if ((tid & 63) == 0) {
    wave_max[tid >> 6] = mx;
    wave_bad[tid >> 6] = bad;
  }
  __syncthreads();
  mx = max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3]));
  bad = wave_bad[0] | wave_bad[1] | wave_bad[2] | wave_bad[3];
  const u32 ebits = mx >> 23;
  const int e_tile = ebits >= kVtScaleFrom ? (int)(ebits - kVtScaleFrom + 1) : 0;
  const float down = exp2_int(-min(e_tile, kVtExpClamp));

#pragma unroll
  for (int u = 0; u < UPT; ++u) {
    const int unit = tid + u * kAttnThreads, kp = unit / CH, ch = unit % CH;
    const int slot = vt_slot(2 * kp);             // keys 2kp, 2kp+1 are adjacent slots
#pragma unroll
    for (int d2 = 0; d2 < 8; ++d2) {
      const int dim = ch * 8 + d2;
      const u32 w0 = raw[u][0][d2 >> 1], w1 = raw[u][1][d2 >> 1];
      const float f0 = (d2 & 1) ? In::hi(w0) : In::lo(w0);
      const float f1 = (d2 & 1) ? In::hi(w1) : In::lo(w1);
      const u32 word = pack_f16x2(f0 * down, f1 * down);
      const int pos = (((slot >> 3) ^ swizzle<8>(dim)) << 3) | (slot & 7);
      *(u32*)(img + dim * kAttnBN + pos) = word;
    }
  }
  __syncthreads();
  u16* dst = vt + ((i64)bh * ntiles + t) * (D * kAttnBN);
#pragma unroll
  for (int c = tid; c < D * kAttnBN / 8; c += kAttnThreads)
    store16(dst + c * 8, *(const u32x4*)(img + c * 8));
  if (tid == 0) exps[(i64)bh * ntiles + t] = bad ? kVtNonFinite : e_tile;
}

// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ u32 lds_address(const void* p) {
  return (u32)(unsigned long long)(const __attribute__((address_space(3))) void*)p;
}

// S^T = K Q^T of one 64-key tile at head dim 128 (both 32-key blocks, 16 MFMAs) as one
// instruction block.  The compiler, left to itself, waits for each LDS read right before its
// MFMA, which serialises the phase on LDS latency; here the K fragments are read ahead into
// v224-v255 (eight quads, reserved through the clobber list) and each MFMA waits only for its
// own read: LDS reads retire in order, so lgkmcnt counts down.  A quad is refilled one MFMA
// after the MFMA that read it.  The block starts with lgkmcnt(0), so no earlier scalar load
// (also counted by lgkmcnt, retiring out of order) can be outstanding, and ends with s_nops
// for the wait states before VALU reads the last MFMA's result.  addr[s] is the LDS address
// of the k-step s fragment of key block 0; block 1 is 32 rows (8192 bytes) further.
// OP names the MFMA input type (bf16 or f16).
#define NEP_ATTN_S_TILE_D128(OP) \
  asm volatile( \
      "s_waitcnt lgkmcnt(0)\n" \
      "ds_read_b128 v[224:227], %[a0]\n" \
      "ds_read_b128 v[228:231], %[a1]\n" \
      "ds_read_b128 v[232:235], %[a2]\n" \
      "ds_read_b128 v[236:239], %[a3]\n" \
      "ds_read_b128 v[240:243], %[a4]\n" \
      "ds_read_b128 v[244:247], %[a5]\n" \
      "ds_read_b128 v[248:251], %[a6]\n" \
      "ds_read_b128 v[252:255], %[a7]\n" \
      "s_waitcnt lgkmcnt(7)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[224:227], %[q0], 0\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[228:231], %[q1], %[s0]\n" \
      "ds_read_b128 v[224:227], %[a0] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[232:235], %[q2], %[s0]\n" \
      "ds_read_b128 v[228:231], %[a1] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[236:239], %[q3], %[s0]\n" \
      "ds_read_b128 v[232:235], %[a2] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[240:243], %[q4], %[s0]\n" \
      "ds_read_b128 v[236:239], %[a3] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[244:247], %[q5], %[s0]\n" \
      "ds_read_b128 v[240:243], %[a4] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[248:251], %[q6], %[s0]\n" \
      "ds_read_b128 v[244:247], %[a5] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s0], v[252:255], %[q7], %[s0]\n" \
      "ds_read_b128 v[248:251], %[a6] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[224:227], %[q0], 0\n" \
      "ds_read_b128 v[252:255], %[a7] offset:8192\n" \
      "s_waitcnt lgkmcnt(6)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[228:231], %[q1], %[s1]\n" \
      "s_waitcnt lgkmcnt(5)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[232:235], %[q2], %[s1]\n" \
      "s_waitcnt lgkmcnt(4)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[236:239], %[q3], %[s1]\n" \
      "s_waitcnt lgkmcnt(3)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[240:243], %[q4], %[s1]\n" \
      "s_waitcnt lgkmcnt(2)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[244:247], %[q5], %[s1]\n" \
      "s_waitcnt lgkmcnt(1)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[248:251], %[q6], %[s1]\n" \
      "s_waitcnt lgkmcnt(0)\n" \
      "v_mfma_f32_32x32x16_" OP " %[s1], v[252:255], %[q7], %[s1]\n" \
      "s_nop 7\n" \
      "s_nop 7\n" \
      "s_nop 7\n" \
      : [s0] "=&v"(s0), [s1] "=&v"(s1) \
      : [a0] "v"(addr[0]), [a1] "v"(addr[1]), [a2] "v"(addr[2]), [a3] "v"(addr[3]), \
        [a4] "v"(addr[4]), [a5] "v"(addr[5]), [a6] "v"(addr[6]), [a7] "v"(addr[7]), \
        [q0] "v"(q[0]), [q1] "v"(q[1]), [q2] "v"(q[2]), [q3] "v"(q[3]), [q4] "v"(q[4]), \
        [q5] "v"(q[5]), [q6] "v"(q[6]), [q7] "v"(q[7]) \
      : "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", \
        "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", \
        "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255", "memory");

template <typename T>
__device__ __forceinline__ void attention_s_tile_d128(const u32 (&addr)[8],
                                                      const typename AttnIn<T>::vec8 (&q)[8],
                                                      f32x16& s0, f32x16& s1) {
  if constexpr (__is_same(T, __bf16)) {
    NEP_ATTN_S_TILE_D128("bf16")
  } else {
    NEP_ATTN_S_TILE_D128("f16")
  }
}
#undef NEP_ATTN_S_TILE_D128

// LDS-DMA of one tile operand: 16 bytes per lane into 1 KB blocks; piece i of wave w fills
// block i*W + w (W waves per workgroup).  `dst` is the wave's block (wave-uniform, it becomes M0).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, void* dst, int voffset,
                                      int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)dst, 16, voffset, soffset, 0, 0);
}

// Exact fold of the queries [q0, q0 + kAttnBM) of one head, for a workgroup whose key range
// holds a V tile the MFMA path does not take (|v| >= 2^(e_max+15), inf or NaN).  fp32
// throughout: a query's row is held by 4 adjacent lanes (D/4 head dims each); per key the
// score is the group sum of their partial dot products, and (m, l, O) are moved to every new
// maximum exactly (not lazily).  Masked keys contribute nothing, so only the rows that see a
// non-finite V value turn non-finite, as IEEE arithmetic on the visible keys gives.
template <typename T, int D, bool CAUSAL, int W, int BM = 32 * W>
__device__ void attention_exact_rows(const T* __restrict__ qp, const T* __restrict__ kp,
                                     const T* __restrict__ vp, T* __restrict__ orow0,
                                     float* __restrict__ lse_row0, int sq, int sk, int q0,
                                     i64 qss, i64 kss, i64 vss, float scale_log2) {
  typedef AttnIn<T> In;
  constexpr int DQ = D / 4;                    // head dims per lane
  constexpr int ROWS = W * 64 / 4;             // queries per round
  const int tid = threadIdx.x, c = tid & 3;
  for (int r0 = q0; r0 < q0 + BM; r0 += ROWS) {
    const int my_q = r0 + (tid >> 2);
    const bool active = my_q < sq;
    float qv[DQ], ov[DQ];
#pragma unroll
    for (int d8 = 0; d8 < DQ; d8 += 8) {
      const u32x4 w = active ? load16_cached(qp + (i64)my_q * qss + c * DQ + d8)
                             : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        qv[d8 + 2 * i] = In::lo(w[i]) * scale_log2;
        qv[d8 + 2 * i + 1] = In::hi(w[i]) * scale_log2;
      }
    }
#pragma unroll
    for (int d = 0; d < DQ; ++d) ov[d] = 0.0f;
    float m = -kInf, l = 0.0f;
    const int kend = CAUSAL ? min(sk, r0 + ROWS) : sk;
    const int last = !active ? -1 : (CAUSAL ? min(my_q, sk - 1) : sk - 1);
#pragma unroll 2
    for (int j = 0; j < kend; ++j) {
      const T* kr = kp + (i64)j * kss + c * DQ;
      const T* vr = vp + (i64)j * vss + c * DQ;
      u32x4 kw[DQ / 8], vw[DQ / 8];
#pragma unroll
      for (int i = 0; i < DQ / 8; ++i) {
        kw[i] = load16_cached(kr + 8 * i);
        vw[i] = load16_cached(vr + 8 * i);
      }
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < DQ / 8; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          dot = __builtin_fmaf(qv[8 * i + 2 * w], In::lo(kw[i][w]), dot);
          dot = __builtin_fmaf(qv[8 * i + 2 * w + 1], In::hi(kw[i][w]), dot);
        }
      const float s = group_sum<4>(dot);   // every lane of the group: the whole score
      if (j <= last) {
        if (s > m) {
          const float alpha = m == -kInf ? 0.0f : __builtin_amdgcn_exp2f(m - s);
          l *= alpha;
#pragma unroll
          for (int d = 0; d < DQ; ++d) ov[d] *= alpha;
          m = s;
        }
        // m is still -inf only while every score seen is -inf: those add nothing
        const float p = m == -kInf ? 0.0f : __builtin_amdgcn_exp2f(s - m);
        l += p;
#pragma unroll
        for (int i = 0; i < DQ / 8; ++i)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            ov[8 * i + 2 * w] = __builtin_fmaf(p, In::lo(vw[i][w]), ov[8 * i + 2 * w]);
            ov[8 * i + 2 * w + 1] = __builtin_fmaf(p, In::hi(vw[i][w]), ov[8 * i + 2 * w + 1]);
          }
      }
    }
    if (active) {
      T* orow = orow0 + (i64)my_q * D + c * DQ;
#pragma unroll
      for (int d8 = 0; d8 < DQ; d8 += 8) {
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = In::pack2(ov[d8 + 2 * i] / l, ov[d8 + 2 * i + 1] / l);
        *(u32x4*)(orow + d8) = w;
      }
      if (lse_row0 != nullptr && c == 0)
        lse_row0[my_q] = (m + __builtin_log2f(l)) * 0.6931471805599453f;
    }
  }
}

template <typename T, int D, bool CAUSAL>
__device__ __forceinline__ void attention_fwd(const T* __restrict__ q, const T* __restrict__ k,
                                              const u16* __restrict__ vt,
                                              const int* __restrict__ exps,
                                              const T* __restrict__ v, T* __restrict__ o,
                                              float* __restrict__ lse, int heads, int sq, int sk,
                                              i64 qsb, i64 qsh, i64 qss, i64 ksb, i64 ksh,
                                              i64 kss, i64 vsb, i64 vsh, i64 vss, int e_max,
                                              float scale_log2) {
  static_assert(D == 64 || D == 128 || D == 256, "head dim must be 64, 128 or 256");
  typedef AttnIn<T> In;
  typedef typename In::vec8 vec8;
  constexpr int kAttnWaves = attn_waves<D>();
  constexpr int kAttnBM = 32 * kAttnWaves;           // queries per workgroup
  constexpr int CH = D / 8;                          // 16-byte chunks per K row
  constexpr int KSTEPS = D / 16;                     // MFMA k-steps of S^T
  constexpr int DBLK = D / 32;                       // 32-row blocks of O^T
  constexpr int TILE = kAttnBN * D * 2;              // bytes of one K tile (= one V^T tile)
  constexpr int PIECES = TILE / 1024 / kAttnWaves;   // 1 KB DMA blocks per wave and operand
  constexpr int KROWS = 1024 * kAttnWaves / (CH * 16);   // K rows per DMA round of all waves
  static_assert(PIECES >= 1 && KROWS >= 1, "DMA mapping");
  // Separate arrays per buffer: the compiler then proves that LDS reads of one buffer do not
  // depend on DMA into the other and does not wait for it.
  __shared__ __attribute__((aligned(1024))) unsigned char kbuf0[TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char kbuf1[TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char vbuf0[TILE];
  __shared__ __attribute__((aligned(1024))) unsigned char vbuf1[TILE];

  const int nqb = (sq + kAttnBM - 1) / kAttnBM;
  const int bh_count = gridDim.x / nqb;
  const int id = blockIdx.x;
  const int qb = nqb - 1 - id / bh_count;   // heaviest query block first
  const int bh = id % bh_count;
  const int b = bh / heads, h = bh % heads;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int ksw = swizzle<CH>(l32), vsw = swizzle<8>(l32);   // rows kb*32 + l32, a*32 + l32
  const int q0 = qb * kAttnBM, qw = q0 + wave * 32;
  const int my_q = qw + l32;
  const T* qp = q + b * qsb + h * qsh;
  const T* kp = k + b * ksb + h * ksh;
  const int ntiles_all = (sk + kAttnBN - 1) / kAttnBN;
  const u16* vth = vt + (i64)bh * ntiles_all * (D * kAttnBN);
  const int* eh = exps + (i64)bh * ntiles_all;

  // Q^T operand: query my_q, head dims [16s + 8*hi, +8) for k-step s.
  vec8 qreg[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    if (my_q < sq) qreg[s] = *(const vec8*)(qp + (i64)my_q * qss + 16 * s + 8 * hi);
    else qreg[s] = vec8{};
  }

  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + kAttnBM);
  const int ntiles = (kv_end + kAttnBN - 1) / kAttnBN;

  // DMA addressing.  LDS chunk L = (i*W + wave)*64 + lane (W waves) of a K tile is key L / CH, position
  // L % CH, and holds head-dim chunk (L % CH) ^ swizzle<CH>(key) of that key; piece i moves
  // KROWS keys further.  When KROWS is a multiple of 16 the swizzle does not depend on i and one
  // offset serves every piece; otherwise (head dim 256: 8 keys per round) each piece has its own.
  constexpr int KOFFS = KROWS % 16 == 0 ? 1 : PIECES;
  int koffs[KOFFS];
#pragma unroll
  for (int i = 0; i < KOFFS; ++i) {
    const int chunk = (i * kAttnWaves + wave) * 64 + lane, key = chunk / CH, p = chunk % CH;
    koffs[i] = (int)((i64)key * kss * 2) + ((p ^ swizzle<CH>(key)) << 4);
  }
  const int kstep = (int)((i64)KROWS * kss * 2);
  // K(tile) and V^T(tile) into LDS; keys at or past sk read as zero (buffer range check),
  // and are masked to -inf anyway.
  auto issue = [&](int tile, unsigned char* kdst, unsigned char* vdst) {
    const int k0 = tile * kAttnBN;
    const int rows = min(kAttnBN, sk - k0);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kp + (i64)k0 * kss), (short)0, (int)(((i64)(rows - 1) * kss + D) * 2),
        (int)kRawBufferWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(vth + (i64)tile * (D * kAttnBN)), (short)0, TILE, (int)kRawBufferWord3);
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      if constexpr (KOFFS == 1) dma16(rk, kdst + (i * kAttnWaves + wave) * 1024, koffs[0] + i * kstep, 0);
      else dma16(rk, kdst + (i * kAttnWaves + wave) * 1024, koffs[i], 0);
      dma16(rv, vdst + (i * kAttnWaves + wave) * 1024, lane * 16, (i * kAttnWaves + wave) * 1024);
    }
  };
  auto wait_dma = []() { __builtin_amdgcn_s_waitcnt(0x0F70); };   // vmcnt(0)

  f32x16 oacc[DBLK];
#pragma unroll
  for (int a = 0; a < DBLK; ++a) oacc[a] = f32x16{};
  float m_ref = -kInf;   // reference max (base 2) of this lane's query
  float l_even = 0.0f, l_odd = 0.0f;   // row sum of the fp32 P, in two chains

  auto body = [&](int tile, const unsigned char* kt, const unsigned char* vtt, int e_in) {
    const int k0 = tile * kAttnBN;
    if (CAUSAL && k0 > qw + 31) return;   // tile entirely above this wave's diagonal
    const int e = min(e_in, kVtExpClamp);
    // ---- S^T = K Q^T for the two 32-key blocks of the tile (head dim 128: one instruction
    // block with the K reads ahead of their MFMAs)
    f32x16 sacc[2];
    if constexpr (D == 128) {
      const u32 krow0 = lds_address(kt) + l32 * (CH * 16);
      u32 addr[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) addr[s] = krow0 + (((2 * s + hi) ^ ksw) << 4);
      attention_s_tile_d128<T>(addr, qreg, sacc[0], sacc[1]);
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = f32x16{};
        const unsigned char* krow = kt + (kb * 32 + l32) * (CH * 16);
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const vec8 a = *(const vec8*)(krow + (((2 * s + hi) ^ ksw) << 4));
          sacc[kb] = In::mfma(a, qreg[s], sacc[kb]);
        }
      }
    }
    // ---- masks only on the diagonal tile and the ragged last tile
    if ((CAUSAL && k0 + kAttnBN - 1 > qw) || (k0 + kAttnBN > sk)) {
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
    tmax = __builtin_fmaxf(tmax, partner<32>(tmax)) * scale_log2;
    // A V^T tile stored as v * 2^-e gets P' = P * 2^e (exact) and a row-sum weight of 2^-e;
    // P' <= 2^15 because the reference max is held max(0, e - 7) above its slack position.
    const float lift = (float)max(0, e - 7);
    // move the reference max only when P' would exceed 2^(8 + min(e, 7)), or on the first
    // finite tile
    const bool move = tmax + lift > m_ref + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(move) != 0) {
      const float m_new = move ? tmax + lift : m_ref;
      const float alpha = (m_ref == -kInf) ? 0.0f : __builtin_amdgcn_exp2f(m_ref - m_new);
      l_even *= alpha;
      l_odd *= alpha;
#pragma unroll
      for (int a = 0; a < DBLK; ++a) oacc[a] *= alpha;
      m_ref = m_new;
    }
    const float shift = ((m_ref == -kInf) ? 0.0f : m_ref) - (float)e;
    const float wl = exp2_int(-e);   // row-sum weight of this tile's P'
    u32 pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r], scale_log2, -shift));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r + 1], scale_log2, -shift));
        pk[kb][r >> 1] = pack_f16x2(p0, p1);
        l_even = __builtin_fmaf(p0, wl, l_even);
        l_odd = __builtin_fmaf(p1, wl, l_odd);
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
      const int chunk = ((2 * cs + hi) ^ vsw) << 4;
#pragma unroll
      for (int a = 0; a < DBLK; ++a) {
        const u32x4 av = *(const u32x4*)(vtt + (a * 32 + l32) * (kAttnBN * 2) + chunk);
        oacc[a] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, av),
                                                         __builtin_bit_cast(f16x8, bw),
                                                         oacc[a], 0, 0, 0);
      }
    }
  };

  // Tile t is computed from buffers t % 2 while the DMA of tile t+1 fills the others (last
  // read in iteration t-1, before this iteration's barrier).  Unrolled by two so every LDS
  // address names its array.
  // Every wave reads every exponent of the block's key range, so `exact` is workgroup-uniform.
  bool exact = false;
  // e_pending (per lane, the same in all) is loaded one iteration ahead and made uniform only
  // after the next wait_dma, which retires it with the DMA: the load's latency is never waited
  // for on its own.
  int e_pending = ntiles > 0 ? eh[0] : 0;
  if (ntiles > 0) issue(0, kbuf0, vbuf0);
  for (int tile = 0; tile < ntiles;) {
    wait_dma();
    __syncthreads();
    asm volatile("" : "+v"(e_pending));
    int e_cur = __builtin_amdgcn_readfirstlane(e_pending);
    e_pending = tile + 1 < ntiles ? eh[tile + 1] : 0;
    __builtin_amdgcn_sched_barrier(0);
    if (tile + 1 < ntiles) issue(tile + 1, kbuf1, vbuf1);
    exact |= e_cur > e_max;
    body(tile, kbuf0, vbuf0, e_cur);
    if (++tile >= ntiles) break;
    wait_dma();
    __syncthreads();
    asm volatile("" : "+v"(e_pending));
    e_cur = __builtin_amdgcn_readfirstlane(e_pending);
    e_pending = tile + 1 < ntiles ? eh[tile + 1] : 0;
    __builtin_amdgcn_sched_barrier(0);
    if (tile + 1 < ntiles) issue(tile + 1, kbuf0, vbuf0);
    exact |= e_cur > e_max;
    body(tile, kbuf1, vbuf1, e_cur);
    ++tile;
  }
  T* orow0 = o + (i64)bh * sq * D;
  float* lse_row0 = lse != nullptr ? lse + (i64)bh * sq : nullptr;
  if (exact) {
    attention_exact_rows<T, D, CAUSAL, kAttnWaves>(qp, kp, v + b * vsb + h * vsh, orow0,
                                                   lse_row0, sq, sk, q0, qss, kss, vss,
                                                   scale_log2);
    return;
  }
  // ---- readout: O / l, and the natural-log LSE of the scaled scores.  The wave's 32 output
  // rows go through its own 32 * D * 2 bytes of LDS (16-byte chunks XOR-swizzled by row) and
  // out as whole rows, 16 bytes per lane; the barrier first lets every wave finish its reads
  // of the last tile's buffers.
  const float l_lane = l_even + l_odd;
  const float l_tot = l_lane + partner<32>(l_lane);
  // l_tot is 0 only for a row whose visible scores are all -inf: 0 * inf = NaN, as softmax
  const float inv = 1.0f / l_tot;
  __syncthreads();
  // a tile buffer holds two waves' rows (TILE = 2 * 32 rows * D * 2 bytes)
  constexpr int CPR = D / 8;                 // 16-byte chunks per row
  constexpr int SW = CPR < 16 ? CPR - 1 : 15;
  unsigned char* const buf = wave < 2 ? kbuf0 : wave < 4 ? kbuf1 : wave < 6 ? vbuf0 : vbuf1;
  unsigned char* stage = buf + (wave & 1) * (32 * D * 2);
#pragma unroll
  for (int a = 0; a < DBLK; ++a) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w.x = In::pack2(oacc[a][4 * g + 0] * inv, oacc[a][4 * g + 1] * inv);
      w.y = In::pack2(oacc[a][4 * g + 2] * inv, oacc[a][4 * g + 3] * inv);
      *(u32x2*)(stage + l32 * (D * 2) + (((4 * a + g) ^ (l32 & SW)) << 4) + 8 * hi) = w;
    }
  }
  if (lse_row0 != nullptr && hi == 0 && my_q < sq)
    lse_row0[my_q] = (m_ref + __builtin_log2f(l_tot)) * 0.6931471805599453f;
  __builtin_amdgcn_wave_barrier();
  if constexpr (CPR <= 64) {
    constexpr int RPI = 64 / CPR;            // rows per wave-wide 16-byte-per-lane store
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int row = RPI * i + lane / CPR, c = lane % CPR;
      const u32x4 w = *(const u32x4*)(stage + row * (D * 2) + ((c ^ (row & SW)) << 4));
      if (qw + row < sq) store16(orow0 + (i64)(qw + row) * D + 8 * c, w);
    }
  }
}


#ifdef NEP_ATTN_W64_ASM
typedef u32 u32x8 __attribute__((ext_vector_type(8)));
typedef u32 u32x32 __attribute__((ext_vector_type(32)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x32 __attribute__((ext_vector_type(32)));

// Head dim 128: one workgroup = 4 wave64s (one per SIMD) x 64 queries (two 32-query blocks per
// wave) = 256 queries, so every K / V^T fragment read from LDS feeds two MFMAs.  The key-tile
// loop is the instruction-scheduled block NEP_ATTN_W64_ASM (generated, with its register map,
// by neptune_codegen/attention_asm.py): the softmax of tile t runs between the MFMAs of
// S(t+1) = K(t+1) Q^T, the row sums of t and the row max of t+1 between those of
// O^T += V^T(t) P^T(t).  Same arithmetic, operation for operation, as attention_fwd; same LDS
// layouts (K rows of 16 swizzled chunks, the V^T image) in NBUF buffers each (the next NBUF-2
// tiles in flight while t is computed), one barrier per tile.
// This function prepares the per-lane addresses, pins them to the block's registers (the block
// loads the Q^T operands itself, behind the first tile's DMA), and does the readout (or the
// exact fp32 path) afterwards.  Q rows must be less than 2^22 elements apart.
template <typename T, bool CAUSAL>
__device__ __forceinline__ void attention_fwd_w64(const T* __restrict__ q, const T* __restrict__ k,
                                                  const u16* __restrict__ vt,
                                                  const int* __restrict__ exps,
                                                  const T* __restrict__ v, T* __restrict__ o,
                                                  float* __restrict__ lse, int heads, int sq,
                                                  int sk, i64 qsb, i64 qsh, i64 qss, i64 ksb,
                                                  i64 ksh, i64 kss, i64 vsb, i64 vsh, i64 vss,
                                                  int e_max, float scale_log2) {
  typedef AttnIn<T> In;
  constexpr int D = 128, W = 4, BM = 256;
  constexpr int TILE = kAttnBN * D * 2;
  constexpr int NBUF = NEP_ATTN_W64_NBUF;   // K and V^T tile buffers
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * NBUF * TILE];   // K..., V...

  const int nqb = (sq + BM - 1) / BM;
  const int bh_count = gridDim.x / nqb;
  const int id = blockIdx.x;
  // Workgroups go to the XCDs round-robin (id % 8); each XCD takes its heads (head % 8 ==
  // id % 8) two at a time, heaviest query block first within the pair, so the query blocks
  // reading a head's K / V^T run together and share that XCD's L2.  Other head counts: the
  // heaviest query block of every head first.
  int qblk, bh;
  if (bh_count % 8 == 0) {
    const int x = id & 7, slot = id >> 3, hx_n = bh_count >> 3;
    const int pair = slot / (2 * nqb), r = slot - pair * 2 * nqb;
    int hx;
    if (2 * pair + 1 < hx_n) {
      qblk = nqb - 1 - (r >> 1);
      hx = 2 * pair + (r & 1);
    } else {
      qblk = nqb - 1 - r;
      hx = 2 * pair;
    }
    bh = hx * 8 + x;
  } else {
    qblk = nqb - 1 - id / bh_count;
    bh = id % bh_count;
  }
  const int b = bh / heads, h = bh % heads;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qblk * BM, qw = q0 + wave * 64;
  const T* qp = q + b * qsb + h * qsh;
  const T* kp = k + b * ksb + h * ksh;
  const int ntiles_all = (sk + kAttnBN - 1) / kAttnBN;
  const u16* vth = vt + (i64)bh * ntiles_all * (D * kAttnBN);
  const int* eh = exps + (i64)bh * ntiles_all;

  // Q rows of the workgroup: the loop loads its Q^T operands itself (rows past sq read 0)
  const int qss2 = (int)(qss * 2);
  const T* qbase = qp + (i64)q0 * qss;
  const int q_nr = (min(sq - q0, BM) - 1) * qss2 + 256;
  u32x2 qoff;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) qoff[blk] = (u32)((wave * 64 + 32 * blk + l32) * qss2 + 16 * hi);
  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + BM);
  const int ntiles = (kv_end + kAttnBN - 1) / kAttnBN;
  const int last_w = CAUSAL ? min(ntiles - 1, qw / kAttnBN) : ntiles - 1;
  const u32 lds_base = lds_address(lds);
  const int ksw = swizzle<16>(l32), vsw = swizzle<8>(l32);
  u32x8 kaddr;
#pragma unroll
  for (int s = 0; s < 8; ++s) kaddr[s] = lds_base + l32 * 256 + (((2 * s + hi) ^ ksw) << 4);
  u32x4 vaddr;
#pragma unroll
  for (int cs = 0; cs < 4; ++cs)
    vaddr[cs] = lds_base + NBUF * TILE + l32 * 128 + (((2 * cs + hi) ^ vsw) << 4);
  // K DMA: 16 rows per round of the 4 waves; lane -> key 4*wave + lane/16, chunk lane%16
  const int kss2 = (int)(kss * 2);
  const int key = 4 * wave + (lane >> 4), part = lane & 15;
  const int koff0 = key * kss2 + ((part ^ swizzle<16>(key)) << 4);
  u32x4 koff;
#pragma unroll
  for (int i = 0; i < 4; ++i) koff[i] = (u32)(koff0 + i * 16 * kss2);
  u32x2 lb;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int my_q = qw + 32 * blk + l32;
    lb[blk] = (u32)((CAUSAL ? min(my_q, sk - 1) : sk - 1) - 4 * hi);
  }
  const u32 voff = lane * 16;

  f32x32 oacc[4];
  f32x8 st;   // m_ref[2], (l_even, l_odd)[2], tile max[2] (unused)
  int exact;
  asm volatile(NEP_ATTN_W64_ASM
               : "={a[0:31]}"(oacc[0]), "={a[32:63]}"(oacc[1]), "={a[64:95]}"(oacc[2]),
                 "={a[96:127]}"(oacc[3]), "={v[220:227]}"(st), "={s74}"(exact)
               , "+{v[254:255]}"(qoff)
               : "{s[98:99]}"(qbase), "{s97}"(q_nr), "{v[208:215]}"(kaddr),
                 "{v[216:219]}"(vaddr), "{v[240:243]}"(koff), "{v[244:245]}"(lb), "{v246}"(voff),
                 "{s[48:49]}"(kp), "{s[50:51]}"(vth), "{s[52:53]}"(eh), "{s54}"(kss2),
                 "{s55}"(sk), "{s56}"(ntiles), "{s57}"(last_w), "{s58}"(scale_log2),
                 "{s59}"(e_max), "{s60}"(qw), "{s61}"(lds_base), "{s63}"(wave)
               : NEP_ATTN_W64_CLOBBERS);

  T* orow0 = o + (i64)bh * sq * D;
  float* lse_row0 = lse != nullptr ? lse + (i64)bh * sq : nullptr;
  if (exact) {
    attention_exact_rows<T, D, CAUSAL, W, BM>(qp, kp, v + b * vsb + h * vsh, orow0, lse_row0,
                                             sq, sk, q0, qss, kss, vss, scale_log2);
    return;
  }
  // ---- readout: O / l, and the natural-log LSE of the scaled scores.  The wave's 64 output
  // rows go through its own 16 KB of LDS (16-byte chunks XOR-swizzled by row, conflict-free;
  // every read of the loop is done: the loop ended with a barrier after its last reads), then
  // out as whole rows, 16 bytes per lane.
  unsigned char* stage = lds + wave * (64 * D * 2);
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const float l_lane = st[2 + 2 * blk] + st[3 + 2 * blk];
    const float l_tot = l_lane + partner<32>(l_lane);
    // l_tot is 0 only for a row whose visible scores are all -inf: 0 * inf = NaN, as softmax
    const float inv = 1.0f / l_tot;
    const int row = 32 * blk + l32;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = (a & 1) * 16 + 4 * g;
        const f32x32& acc = oacc[blk * 2 + (a >> 1)];
        u32x2 w;
        w.x = In::pack2(acc[r + 0] * inv, acc[r + 1] * inv);
        w.y = In::pack2(acc[r + 2] * inv, acc[r + 3] * inv);
        *(u32x2*)(stage + row * (D * 2) + (((4 * a + g) ^ (row & 15)) << 4) + 8 * hi) = w;
      }
    }
    const int my_q = qw + row;
    if (lse_row0 != nullptr && hi == 0 && my_q < sq)
      lse_row0[my_q] = (st[blk] + __builtin_log2f(l_tot)) * 0.6931471805599453f;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the wave's own LDS writes
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = 4 * i + (lane >> 4), c = lane & 15;
    const u32x4 w = *(const u32x4*)(stage + row * (D * 2) + ((c ^ (row & 15)) << 4));
    if (qw + row < sq) store16(orow0 + (i64)(qw + row) * D + 8 * c, w);
  }
}
#endif  // NEP_ATTN_W64_ASM

}  // namespace nep
