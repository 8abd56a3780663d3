// nep_device.h -- device primitives shared by every neptune HIP kernel (gfx950, wave64).
//
// Compiled through hiprtc: the emitter pastes this text ahead of the generated code, so it
// must not include host headers.  Everything here is written for CDNA4: 64-wide wavefronts,
// DPP / ds_swizzle cross-lane exchange, 128-bit global loads.
#pragma once

namespace nep {

typedef unsigned int u32;
typedef unsigned short u16;
typedef long long i64;
typedef unsigned long long u64;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr float kInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float as_f32(u32 b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ u32 as_u32(float f) { return __builtin_bit_cast(u32, f); }
// Bit casts take their operand by value: __builtin_bit_cast applied directly to an
// ext_vector element expression (w.y) is compiled as a cast of element 0 by this clang.
__device__ __forceinline__ half2_t as_half2(u32 b) { return __builtin_bit_cast(half2_t, b); }
__device__ __forceinline__ u32 half2_bits(half2_t h) { return __builtin_bit_cast(u32, h); }
__device__ __forceinline__ bool is_nan(float v) { return v != v; }
__device__ __forceinline__ bool is_finite(float v) { return __builtin_isfinite(v); }

// exp(x) as 2^(x*log2 e) on the hardware exp2 (v_exp_f32): the textbook base change, used for
// the fold terms where the reference's Triton lowering also uses an approximate exponential.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// num / den for a denominator shared by many numerators (a fold term's per-tile producer
// value): one IEEE division 1/den that the compiler shares across the unrolled elements, then
// a multiply per element (<= 1.5 ulp from the quotient).  A denominator below 2^-64 is first
// scaled by the exact power of two 2^64 on both sides, so 1/den stays finite for denormals.
__device__ __forceinline__ float quot(float num, float den) {
  const float sc = __builtin_fabsf(den) < 0x1p-64f ? 0x1p64f : 1.0f;
  return (num * sc) * (1.0f / (den * sc));
}

// Repair slopes and biases (evaluated once per tile and once per merge, never per element) use
// the hardware square root, reciprocal square root and reciprocal (v_sqrt_f32, v_rsq_f32,
// v_rcp_f32: 1 ulp each), the precision class of the reference's Triton lowering, whose
// tl.sqrt and fp32 division are not correctly rounded either.  Arguments outside
// [2^-64, 2^64] are first scaled by an exact power of two, so the instructions never see a
// denormal input or produce a denormal result; 0, inf and NaN keep their IEEE results.
__device__ __forceinline__ float fsqrt(float x) {
  const bool small = x < 0x1p-64f;
  return __builtin_amdgcn_sqrtf(small ? x * 0x1p64f : x) * (small ? 0x1p-32f : 1.0f);
}
__device__ __forceinline__ float frsq(float x) {
  const float sc = x < 0x1p-64f ? 0x1p64f : (x > 0x1p64f ? 0x1p-64f : 1.0f);
  const float back = x < 0x1p-64f ? 0x1p32f : (x > 0x1p64f ? 0x1p-32f : 1.0f);
  return __builtin_amdgcn_rsqf(x * sc) * back;
}
__device__ __forceinline__ float fquot(float num, float den) {
  const float a = __builtin_fabsf(den);
  const float sc = a < 0x1p-64f ? 0x1p64f : (a > 0x1p64f ? 0x1p-64f : 1.0f);
  return (num * __builtin_amdgcn_rcpf(den * sc)) * sc;
}

// ---------------------------------------------------------------- storage dtypes
// bf16 -> fp32 is exact (the high half of an fp32 pattern).  fp32 -> bf16 rounds to nearest
// even.  f32_to_bf16_bits is the integer statement of that rounding (NaN -> the canonical
// quiet NaN 0x7fc0 with its sign, as torch's own conversion does).  The storage paths use the
// hardware conversion v_cvt_pk_bf16_f32 (two values per instruction), which a GPU test shows
// bit-identical to f32_to_bf16_bits for all 2^32 non-NaN fp32 inputs under this build's float
// modes (ties, denormals, overflow, infinities); a NaN stays a NaN, its payload may differ.
__device__ __forceinline__ float bf16_bits_to_f32(u32 b16) { return as_f32(b16 << 16); }
__device__ __forceinline__ u32 f32_to_bf16_bits(float f) {
  u32 b = as_u32(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return ((b >> 16) & 0x8000u) | 0x7fc0u;
  b += 0x7fffu + ((b >> 16) & 1u);
  return b >> 16;
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// (bf16(a) | bf16(b) << 16), round to nearest even, in one v_cvt_pk_bf16_f32
__device__ __forceinline__ u32 bf16x2_rne(float a, float b) {
  const f32x2_t f = {a, b};
  return __builtin_bit_cast(u32, __builtin_convertvector(f, bf16x2_t));
}

struct F32 {
  typedef float T;
  static constexpr int kVec = 4;  // elements per 16-byte load
  static constexpr u32 kNegInfWord = 0xff800000u;  // a 32-bit word of -inf elements
  __device__ static __forceinline__ float load(const T* p) { return *p; }
  __device__ static __forceinline__ void store(T* p, float v) { *p = v; }
  __device__ static __forceinline__ float round(float v) { return v; }
  __device__ static __forceinline__ void unpack(const u32x4& w, float* o) {
    o[0] = as_f32(w.x); o[1] = as_f32(w.y); o[2] = as_f32(w.z); o[3] = as_f32(w.w);
  }
  // unpack for a word unpacked again later: the values are not kept between the two (for
  // fp32 the word is the values, so this is unpack).
  __device__ static __forceinline__ void reunpack(const u32x4& w, float* o) { unpack(w, o); }
  __device__ static __forceinline__ u32x4 pack(const float* v) {
    u32x4 w; w.x = as_u32(v[0]); w.y = as_u32(v[1]); w.z = as_u32(v[2]); w.w = as_u32(v[3]);
    return w;
  }
};

struct BF16 {
  typedef u16 T;
  static constexpr int kVec = 8;
  static constexpr u32 kNegInfWord = 0xff80ff80u;
  __device__ static __forceinline__ float load(const T* p) { return bf16_bits_to_f32(*p); }
  __device__ static __forceinline__ void store(T* p, float v) { *p = (u16)bf16x2_rne(v, v); }
  __device__ static __forceinline__ float round(float v) { return as_f32(bf16x2_rne(v, v) << 16); }
  __device__ static __forceinline__ void unpack(const u32x4& w, float* o) {
    o[0] = as_f32(w.x << 16); o[1] = as_f32(w.x & 0xffff0000u);
    o[2] = as_f32(w.y << 16); o[3] = as_f32(w.y & 0xffff0000u);
    o[4] = as_f32(w.z << 16); o[5] = as_f32(w.z & 0xffff0000u);
    o[6] = as_f32(w.w << 16); o[7] = as_f32(w.w & 0xffff0000u);
  }
  // unpack whose results the compiler cannot share with another unpack of the same word
  // (through an opaque copy of the word), so a caller that unpacks a held row once per pass
  // holds 16-bit words, not fp32 values.
  __device__ static __forceinline__ void reunpack(const u32x4& w, float* o) {
    u32x4 c = w;
    asm volatile("" : "+v"(c));
    unpack(c, o);
  }
  __device__ static __forceinline__ u32x4 pack(const float* v) {
    u32x4 w;
    w.x = bf16x2_rne(v[0], v[1]);
    w.y = bf16x2_rne(v[2], v[3]);
    w.z = bf16x2_rne(v[4], v[5]);
    w.w = bf16x2_rne(v[6], v[7]);
    return w;
  }
};

// fp16 uses the hardware conversions: v_cvt_f32_f16 is exact and v_cvt_f16_f32 rounds to
// nearest even (the default round mode), with fp16 denormals kept.
struct F16 {
  typedef _Float16 T;
  static constexpr int kVec = 8;
  static constexpr u32 kNegInfWord = 0xfc00fc00u;
  __device__ static __forceinline__ float load(const T* p) { return (float)*p; }
  __device__ static __forceinline__ void store(T* p, float v) { *p = (_Float16)v; }
  __device__ static __forceinline__ float round(float v) { return (float)(_Float16)v; }
  __device__ static __forceinline__ void unpack(const u32x4& w, float* o) {
    const half2_t h0 = as_half2(w.x), h1 = as_half2(w.y), h2 = as_half2(w.z), h3 = as_half2(w.w);
    o[0] = (float)h0.x; o[1] = (float)h0.y; o[2] = (float)h1.x; o[3] = (float)h1.y;
    o[4] = (float)h2.x; o[5] = (float)h2.y; o[6] = (float)h3.x; o[7] = (float)h3.y;
  }
  __device__ static __forceinline__ void reunpack(const u32x4& w, float* o) {
    u32x4 c = w;
    asm volatile("" : "+v"(c));
    unpack(c, o);
  }
  __device__ static __forceinline__ u32x4 pack(const float* v) {
    half2_t h0, h1, h2, h3;
    h0.x = (_Float16)v[0]; h0.y = (_Float16)v[1]; h1.x = (_Float16)v[2]; h1.y = (_Float16)v[3];
    h2.x = (_Float16)v[4]; h2.y = (_Float16)v[5]; h3.x = (_Float16)v[6]; h3.y = (_Float16)v[7];
    u32x4 w;
    w.x = half2_bits(h0); w.y = half2_bits(h1); w.z = half2_bits(h2); w.w = half2_bits(h3);
    return w;
  }
};

// 128-bit global load/store (global_load_dwordx4).  Callers guarantee 16-byte alignment.
__device__ __forceinline__ u32x4 load16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load16_cached(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(void* p, const u32x4& w) {
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------- cross-lane exchange
// partner<S>(v) returns the value of a lane in the partner group of size S inside the
// wavefront.  Steps 1 and 2 are exact xor exchanges (DPP quad_perm); 4 and 8 use the DPP
// half-row / row mirrors, which pair every lane with a lane of the partner group -- valid for
// butterfly reductions because after the smaller steps every lane of a group holds the same
// value.  16 and 32 are exact xor exchanges through gfx950's v_permlane16_swap /
// v_permlane32_swap (VALU, no LDS round trip): swapping a value with itself leaves every lane
// holding the pair (lower, upper) of its 16- or 32-lane partner group, verified on the GPU:
// permlane16_swap(v, v) = {v[l & ~16], v[l | 16]}, permlane32_swap(v, v) = {v[l & 31],
// v[(l & 31) | 32]}.  All lanes of the wavefront must be active.
template <int S>
__device__ __forceinline__ u32 partner_u32(u32 v) {
  if constexpr (S == 1) return (u32)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
  else if constexpr (S == 2) return (u32)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
  else if constexpr (S == 4) return (u32)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
  else if constexpr (S == 8) return (u32)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
  else {
    static_assert(S == 16 || S == 32, "partner step must be 1..32");
    const u32 lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0));
    if constexpr (S == 16) {
      const auto p = __builtin_amdgcn_permlane16_swap(v, v, true, false);
      return (lane & 16u) ? p[0] : p[1];
    } else {
      const auto p = __builtin_amdgcn_permlane32_swap(v, v, true, false);
      return (lane & 32u) ? p[0] : p[1];
    }
  }
}

// Both members of the S-lane partner pair (lower group's value, upper group's value), the same
// in every lane of the pair: reductions combine them in one order, bit-identical across lanes.
template <int S>
__device__ __forceinline__ void pair_u32(u32 v, u32& lo, u32& hi) {
  static_assert(S == 16 || S == 32, "pair exchange is for steps 16 and 32");
  if constexpr (S == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, true, false);
    lo = p[0];
    hi = p[1];
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, true, false);
    lo = p[0];
    hi = p[1];
  }
}
template <int S>
__device__ __forceinline__ float partner(float v) { return as_f32(partner_u32<S>(as_u32(v))); }
template <int S>
__device__ __forceinline__ int partner(int v) { return (int)partner_u32<S>((u32)v); }

// Sum / max over aligned groups of G lanes (G a power of two <= 64); every lane of the group
// receives the result.
template <int S>
__device__ __forceinline__ float pair_sum(float v) {
  u32 lo, hi;
  pair_u32<S>(as_u32(v), lo, hi);
  return as_f32(lo) + as_f32(hi);
}
template <int S>
__device__ __forceinline__ float pair_max(float v) {
  u32 lo, hi;
  pair_u32<S>(as_u32(v), lo, hi);
  return __builtin_fmaxf(as_f32(lo), as_f32(hi));
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += partner<1>(v);
  if constexpr (G >= 4) v += partner<2>(v);
  if constexpr (G >= 8) v += partner<4>(v);
  if constexpr (G >= 16) v += partner<8>(v);
  if constexpr (G >= 32) v = pair_sum<16>(v);
  if constexpr (G >= 64) v = pair_sum<32>(v);
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (G >= 2) v = __builtin_fmaxf(v, partner<1>(v));
  if constexpr (G >= 4) v = __builtin_fmaxf(v, partner<2>(v));
  if constexpr (G >= 8) v = __builtin_fmaxf(v, partner<4>(v));
  if constexpr (G >= 16) v = __builtin_fmaxf(v, partner<8>(v));
  if constexpr (G >= 32) v = pair_max<16>(v);
  if constexpr (G >= 64) v = pair_max<32>(v);
  return v;
}
template <int G>
__device__ __forceinline__ int group_or(int v) {
  if constexpr (G >= 2) v |= partner<1>(v);
  if constexpr (G >= 4) v |= partner<2>(v);
  if constexpr (G >= 8) v |= partner<4>(v);
  if constexpr (G >= 16) v |= partner<8>(v);
  if constexpr (G >= 32) v |= partner<16>(v);
  if constexpr (G >= 64) v |= partner<32>(v);
  return v;
}

__device__ __forceinline__ int lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0));
}

// ---------------------------------------------------------------- correctly rounded fp32
// Division and square root: hiprtc compiles HIP with correctly rounded fp32 '/' and sqrtf
// (the -fhip-fp32-correctly-rounded-divide-sqrt default), so div_rn(a, b) is a / b.
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }
__device__ __forceinline__ float sqrt_rn(float a) { return sqrtf(a); }

// rsqrt_rn(x): 1/sqrt(x) correctly rounded to fp32 (round to nearest even).
// Method: r0 = fp32(1 / sqrt(double(x))) is within one fp32 ulp of the exact value.  The
// exact value 1/sqrt(x) lies above the midpoint h between two adjacent fp32 numbers iff
// h*h*x < 1.  With h exact in double (25 significant bits), p = h*h is exact (50 bits) and
// fma(p, x, -1) rounds p*x-1 once, which cannot change its sign.  So the two midpoints around
// r0 decide exactly whether r0 or a neighbour is the correctly rounded result.  Special cases
// follow IEEE rsqrt: +0 -> +inf, -0 -> -inf, x < 0 -> NaN, +inf -> +0, NaN -> NaN.
__device__ __forceinline__ float rsqrt_rn(float x) {
  if (!(x > 0.0f) || x == kInf) {
    if (x == 0.0f) return __builtin_copysignf(kInf, x);
    if (x == kInf) return 0.0f;
    return __builtin_nanf("");
  }
  const double xd = (double)x;
  // For x in (0, inf), 1/sqrt(x) lies in [5e-20, 3e22]: r is a positive normal number, so
  // its neighbours are the adjacent bit patterns.
  float r = (float)(1.0 / __builtin_sqrt(xd));
  const float r_dn = as_f32(as_u32(r) - 1u);
  const float r_up = as_f32(as_u32(r) + 1u);
  const double h_lo = 0.5 * ((double)r + (double)r_dn);
  const double h_hi = 0.5 * ((double)r + (double)r_up);
  const double lo_test = __builtin_fma(h_lo * h_lo, xd, -1.0);  // > 0  => exact < h_lo
  const double hi_test = __builtin_fma(h_hi * h_hi, xd, -1.0);  // < 0  => exact > h_hi
  if (lo_test > 0.0) return r_dn;
  if (hi_test < 0.0) return r_up;
  // On a midpoint exactly (test == 0) round to even.
  if (lo_test == 0.0) return (as_u32(r) & 1u) ? r_dn : r;
  if (hi_test == 0.0) return (as_u32(r) & 1u) ? r_up : r;
  return r;
}

}  // namespace nep
