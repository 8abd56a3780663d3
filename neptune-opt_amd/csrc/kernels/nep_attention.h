// nep_attention.h -- causal online-softmax attention fold on gfx950 MFMA (bf16 in, fp32 acc).
//
// O = softmax(scale * Q K^T + causal mask) V per (batch, head), evaluated as a fold over key
// tiles with the logsumexp repair: running max m, running sum l and accumulator O are moved to
// a new max by exp(m - m') (the logsumexp skeleton's slope exp(s - s2)), so no score matrix is
// materialised.  Scores live in the base-2 domain t = scale*log2(e) * q.k.
//
// Two kernels per call:
//  * attention_vt_pack: V [key][dim] bf16 -> per key tile a V^T image in fp16 (the exact MFMA
//    operand order, XOR-swizzled for conflict-free LDS reads) plus one power-of-two exponent
//    per tile.  Tiles whose largest |v| reaches 2^15 are stored as v * 2^-e (exact: bf16
//    values keep their 8 significant bits in fp16 down to |v| >= 2^(e-17)); the fold feeds
//    such a tile P * 2^e instead of P and weights its row sum by 2^-e, both exact, so no
//    accumulator is rescaled.  A tile value below 2^(e-14) keeps an absolute precision of
//    2^(e-25) only, so the caller bounds e (e_max); a tile above it, or holding inf/NaN,
//    clears *status, which the caller turns into an error.  The image is written once per
//    call and read by every query block of the head.
//  * attention_fwd: one workgroup = 8 wave64s = BLOCK_M = 256 queries (32 per wave), one
//    workgroup per CU (two waves per SIMD): each staged K / V^T tile serves 256 queries.
//    K (bf16, the caller's strided rows, bounds-checked buffer loads) and the V^T image go
//    straight from HBM into double-buffered LDS (buffer_load ... lds, no registers): tile t+1
//    is in flight while tile t is computed, with one barrier per tile.
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
//  * The row sum l accumulates the fp16-rounded P with v_dot2 (the values the MFMA multiplies).
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

constexpr int kAttnWaves = 8;          // wave64s per fold workgroup (32 queries each)
constexpr int kAttnBM = 32 * kAttnWaves;   // queries per fold workgroup
constexpr int kAttnBN = 64;            // keys per tile
constexpr int kAttnThreads = 256;      // V^T pack workgroup: 4 wave64s
constexpr float kRescaleSlack = 8.0f;  // base-2 headroom before the reference max moves
constexpr u32 kRawBufferWord3 = 0x00020000u;   // gfx9 raw buffer descriptor, dword 3
constexpr u32 kVtScaleFrom = 142u;     // bf16 biased exponent of 2^15: tiles at or above scale

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

// Position (0..63, before the row swizzle) of tile key `key` in a V^T image row: chunk
// j = 2*(key/16) + (key/4)%2 holds keys 16*(j/2) + 4*(j%2) + {0,1,2,3} and the same + 8, which
// is the key order of lane (j%2)*32 + .. in the P^T operand of k-step j/2.
__device__ __forceinline__ int vt_slot(int key) {
  const int w = key & 15;
  return ((key >> 4) * 2 + ((w >> 2) & 1)) * 8 + (w & 3) + ((w >> 3) << 2);
}

// LDS rows are read 16 bytes per lane, 16 consecutive rows per LDS cycle (64 banks of 4 bytes,
// 256 bytes per clock).  Row r keeps its 16-byte chunk c at position c ^ swizzle<CH>(r), so the
// 16 rows of one cycle hit 16 different bank groups: rows of 16+ chunks XOR with r % 16, rows of
// 8 chunks (128 bytes: two rows per 256-byte bank sweep) XOR with (r / 2) % 8.
template <int CH>
__device__ __forceinline__ int swizzle(int row) {
  static_assert(CH == 8 || CH == 16, "rows of 8 or 16 chunks");
  if constexpr (CH == 16) return row & 15;
  else return (row >> 1) & 7;
}

// V bf16 [keys, D] of one head -> fp16 V^T tile images [ntiles][D][64] (16-byte chunk j of row
// d stored at chunk j ^ swizzle<8>(d)) and one exponent per tile.  Keys past sk are zero.
template <int D>
__device__ __forceinline__ void attention_vt_pack(const __bf16* __restrict__ v,
                                                  u16* __restrict__ vt, int* __restrict__ exps,
                                                  int* __restrict__ status, int e_max,
                                                  int heads, int sk, i64 vsb, i64 vsh, i64 vss) {
  constexpr int CH = D / 8;                         // 16-byte chunks per key row
  constexpr int UNITS = (kAttnBN / 2) * CH;         // (key pair, dim chunk) units
  constexpr int UPT = UNITS / kAttnThreads;
  static_assert(UNITS % kAttnThreads == 0, "head dim must be 64 or 128");
  __shared__ __attribute__((aligned(16))) u16 img[D * kAttnBN];
  __shared__ u32 wave_max[kAttnThreads / 64];
  const int ntiles = (sk + kAttnBN - 1) / kAttnBN;
  const int bh = blockIdx.x / ntiles, t = blockIdx.x % ntiles;
  const int b = bh / heads, h = bh % heads;
  const __bf16* vp = v + b * vsb + h * vsh;
  const int k0 = t * kAttnBN, tid = threadIdx.x;

  u32x4 raw[UPT][2];
  u32 mx = 0;
#pragma unroll
  for (int u = 0; u < UPT; ++u) {
    const int unit = tid + u * kAttnThreads, kp = unit / CH, ch = unit % CH;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int key = k0 + 2 * kp + r;
      raw[u][r] = key < sk ? load16_cached(vp + (i64)key * vss + ch * 8) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const u32 x = raw[u][r][w] & 0x7fff7fffu;
        mx = max(mx, max(x & 0xffffu, x >> 16));
      }
    }
  }
  // largest bf16 magnitude of the tile (integer order = magnitude order, NaN above inf)
  mx = max(mx, partner_u32<1>(mx));
  mx = max(mx, partner_u32<2>(mx));
  mx = max(mx, partner_u32<4>(mx));
  mx = max(mx, partner_u32<8>(mx));
  mx = max(mx, partner_u32<16>(mx));
  mx = max(mx, partner_u32<32>(mx));
  if ((tid & 63) == 0) wave_max[tid >> 6] = mx;
  __syncthreads();
  mx = max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3]));
  const u32 ebits = mx >> 7;                  // 255: the tile holds inf or NaN
  const int e_tile = ebits >= kVtScaleFrom ? (int)(ebits - kVtScaleFrom + 1) : 0;
  // the fold's scaling arithmetic covers e <= 24; a refused tile is clamped into it
  const int e = min(e_tile, 24);
  const float down = exp2_int(-e);

#pragma unroll
  for (int u = 0; u < UPT; ++u) {
    const int unit = tid + u * kAttnThreads, kp = unit / CH, ch = unit % CH;
    const int slot = vt_slot(2 * kp);             // keys 2kp, 2kp+1 are adjacent slots
#pragma unroll
    for (int d2 = 0; d2 < 8; ++d2) {
      const int dim = ch * 8 + d2;
      const u32 w0 = raw[u][0][d2 >> 1], w1 = raw[u][1][d2 >> 1];
      const u32 b0 = (d2 & 1) ? (w0 & 0xffff0000u) : (w0 << 16);
      const u32 b1 = (d2 & 1) ? (w1 & 0xffff0000u) : (w1 << 16);
      const u32 word = pack_f16x2(as_f32(b0) * down, as_f32(b1) * down);
      const int pos = (((slot >> 3) ^ swizzle<8>(dim)) << 3) | (slot & 7);
      *(u32*)(img + dim * kAttnBN + pos) = word;
    }
  }
  __syncthreads();
  u16* dst = vt + ((i64)bh * ntiles + t) * (D * kAttnBN);
#pragma unroll
  for (int c = tid; c < D * kAttnBN / 8; c += kAttnThreads)
    store16(dst + c * 8, *(const u32x4*)(img + c * 8));
  if (tid == 0) {
    exps[bh * ntiles + t] = e;
    if (e_tile > e_max) *status = 0;
  }
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
__device__ __forceinline__ void attention_s_tile_d128(const u32 (&addr)[8], const bf16x8 (&q)[8],
                                                      f32x16& s0, f32x16& s1) {
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n"
      "ds_read_b128 v[224:227], %[a0]\n"
      "ds_read_b128 v[228:231], %[a1]\n"
      "ds_read_b128 v[232:235], %[a2]\n"
      "ds_read_b128 v[236:239], %[a3]\n"
      "ds_read_b128 v[240:243], %[a4]\n"
      "ds_read_b128 v[244:247], %[a5]\n"
      "ds_read_b128 v[248:251], %[a6]\n"
      "ds_read_b128 v[252:255], %[a7]\n"
      "s_waitcnt lgkmcnt(7)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[224:227], %[q0], 0\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[228:231], %[q1], %[s0]\n"
      "ds_read_b128 v[224:227], %[a0] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[232:235], %[q2], %[s0]\n"
      "ds_read_b128 v[228:231], %[a1] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[236:239], %[q3], %[s0]\n"
      "ds_read_b128 v[232:235], %[a2] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[240:243], %[q4], %[s0]\n"
      "ds_read_b128 v[236:239], %[a3] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[244:247], %[q5], %[s0]\n"
      "ds_read_b128 v[240:243], %[a4] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[248:251], %[q6], %[s0]\n"
      "ds_read_b128 v[244:247], %[a5] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s0], v[252:255], %[q7], %[s0]\n"
      "ds_read_b128 v[248:251], %[a6] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[224:227], %[q0], 0\n"
      "ds_read_b128 v[252:255], %[a7] offset:8192\n"
      "s_waitcnt lgkmcnt(6)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[228:231], %[q1], %[s1]\n"
      "s_waitcnt lgkmcnt(5)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[232:235], %[q2], %[s1]\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[236:239], %[q3], %[s1]\n"
      "s_waitcnt lgkmcnt(3)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[240:243], %[q4], %[s1]\n"
      "s_waitcnt lgkmcnt(2)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[244:247], %[q5], %[s1]\n"
      "s_waitcnt lgkmcnt(1)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[248:251], %[q6], %[s1]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "v_mfma_f32_32x32x16_bf16 %[s1], v[252:255], %[q7], %[s1]\n"
      "s_nop 7\n"
      "s_nop 7\n"
      "s_nop 7\n"
      : [s0] "=&v"(s0), [s1] "=&v"(s1)
      : [a0] "v"(addr[0]), [a1] "v"(addr[1]), [a2] "v"(addr[2]), [a3] "v"(addr[3]),
        [a4] "v"(addr[4]), [a5] "v"(addr[5]), [a6] "v"(addr[6]), [a7] "v"(addr[7]),
        [q0] "v"(q[0]), [q1] "v"(q[1]), [q2] "v"(q[2]), [q3] "v"(q[3]), [q4] "v"(q[4]),
        [q5] "v"(q[5]), [q6] "v"(q[6]), [q7] "v"(q[7])
      : "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234",
        "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245",
        "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255", "memory");
}

// LDS-DMA of one tile operand: 16 bytes per lane into 1 KB blocks; piece i of wave w fills
// block i*W + w (W waves per workgroup).  `dst` is the wave's block (wave-uniform, it becomes M0).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, void* dst, int voffset,
                                      int soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)dst, 16, voffset, soffset, 0, 0);
}

template <int D, bool CAUSAL>
__device__ __forceinline__ void attention_fwd(const __bf16* __restrict__ q,
                                              const __bf16* __restrict__ k,
                                              const u16* __restrict__ vt,
                                              const int* __restrict__ exps,
                                              __bf16* __restrict__ o, float* __restrict__ lse,
                                              int heads, int sq, int sk, i64 qsb, i64 qsh,
                                              i64 qss, i64 ksb, i64 ksh, i64 kss,
                                              float scale_log2) {
  static_assert(D == 64 || D == 128, "head dim must be 64 or 128");
  constexpr int CH = D / 8;                          // 16-byte chunks per K row
  constexpr int KSTEPS = D / 16;                     // MFMA k-steps of S^T
  constexpr int DBLK = D / 32;                       // 32-row blocks of O^T
  constexpr int TILE = kAttnBN * D * 2;              // bytes of one K tile (= one V^T tile)
  constexpr int PIECES = TILE / 1024 / kAttnWaves;   // 1 KB DMA blocks per wave and operand
  constexpr int KROWS = 1024 * kAttnWaves / (CH * 16);   // K rows per DMA round of all waves
  static_assert(PIECES >= 1 && KROWS % 16 == 0, "DMA mapping");
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
  const __bf16* qp = q + b * qsb + h * qsh;
  const __bf16* kp = k + b * ksb + h * ksh;
  const int ntiles_all = (sk + kAttnBN - 1) / kAttnBN;
  const u16* vth = vt + (i64)bh * ntiles_all * (D * kAttnBN);
  const int* eh = exps + bh * ntiles_all;

  // Q^T operand: query my_q, head dims [16s + 8*hi, +8) for k-step s.
  bf16x8 qreg[KSTEPS];
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s) {
    if (my_q < sq) qreg[s] = *(const bf16x8*)(qp + (i64)my_q * qss + 16 * s + 8 * hi);
    else qreg[s] = bf16x8{};
  }

  int kv_end = sk;
  if constexpr (CAUSAL) kv_end = min(sk, q0 + kAttnBM);
  const int ntiles = (kv_end + kAttnBN - 1) / kAttnBN;

  // DMA addressing.  LDS chunk L = (i*W + wave)*64 + lane (W waves) of a K tile is key L / CH, position
  // L % CH, and holds head-dim chunk (L % CH) ^ swizzle<CH>(key) of that key; piece i moves
  // KROWS keys further (KROWS is a multiple of 16, so the swizzle does not depend on i).
  int koff0;
  {
    const int chunk = wave * 64 + lane, key = chunk / CH, p = chunk % CH;
    koff0 = (int)((i64)key * kss * 2) + ((p ^ swizzle<CH>(key)) << 4);
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
      dma16(rk, kdst + (i * kAttnWaves + wave) * 1024, koff0 + i * kstep, 0);
      dma16(rv, vdst + (i * kAttnWaves + wave) * 1024, lane * 16, (i * kAttnWaves + wave) * 1024);
    }
  };
  auto wait_dma = []() { __builtin_amdgcn_s_waitcnt(0x0F70); };   // vmcnt(0)

  f32x16 oacc[DBLK];
#pragma unroll
  for (int a = 0; a < DBLK; ++a) oacc[a] = f32x16{};
  float m_ref = -kInf;   // reference max (base 2) of this lane's query
  float l_run = 0.0f;

  auto body = [&](int tile, const unsigned char* kt, const unsigned char* vtt, int e) {
    const int k0 = tile * kAttnBN;
    if (CAUSAL && k0 > qw + 31) return;   // tile entirely above this wave's diagonal
    // ---- S^T = K Q^T for the two 32-key blocks of the tile (head dim 128: one instruction
    // block with the K reads ahead of their MFMAs)
    f32x16 sacc[2];
    if constexpr (D == 128) {
      const u32 krow0 = lds_address(kt) + l32 * (CH * 16);
      u32 addr[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) addr[s] = krow0 + (((2 * s + hi) ^ ksw) << 4);
      attention_s_tile_d128(addr, qreg, sacc[0], sacc[1]);
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = f32x16{};
        const unsigned char* krow = kt + (kb * 32 + l32) * (CH * 16);
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const bf16x8 a = *(const bf16x8*)(krow + (((2 * s + hi) ^ ksw) << 4));
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[s], sacc[kb], 0, 0, 0);
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
      l_run *= alpha;
#pragma unroll
      for (int a = 0; a < DBLK; ++a) oacc[a] *= alpha;
      m_ref = m_new;
    }
    const float shift = ((m_ref == -kInf) ? 0.0f : m_ref) - (float)e;
    const u32 h16 = e < 15 ? (u32)(15 - e) << 10 : 1u << (24 - e);   // fp16 2^-e, e <= 24
    const half2_t w2 = as_half2(h16 | (h16 << 16));
    u32 pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r], scale_log2, -shift));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][r + 1], scale_log2, -shift));
        const u32 w = pack_f16x2(p0, p1);
        pk[kb][r >> 1] = w;
        l_run = __builtin_amdgcn_fdot2(as_half2(w), w2, l_run, false);
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
  // The exponent of tile t+1 is loaded at the top of iteration t, ahead of that iteration's
  // DMA: vmcnt retires in order, so a later wait on it would also wait for the DMA.
  if (ntiles > 0) issue(0, kbuf0, vbuf0);
  int e_cur = ntiles > 0 ? eh[0] : 0;
  for (int tile = 0; tile < ntiles;) {
    wait_dma();
    __syncthreads();
    int e_next = tile + 1 < ntiles ? eh[tile + 1] : 0;
    __builtin_amdgcn_sched_barrier(0);
    if (tile + 1 < ntiles) issue(tile + 1, kbuf1, vbuf1);
    body(tile, kbuf0, vbuf0, e_cur);
    e_cur = e_next;
    if (++tile >= ntiles) break;
    wait_dma();
    __syncthreads();
    e_next = tile + 1 < ntiles ? eh[tile + 1] : 0;
    __builtin_amdgcn_sched_barrier(0);
    if (tile + 1 < ntiles) issue(tile + 1, kbuf0, vbuf0);
    body(tile, kbuf1, vbuf1, e_cur);
    e_cur = e_next;
    ++tile;
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
