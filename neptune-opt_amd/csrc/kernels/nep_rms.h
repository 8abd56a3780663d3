// nep_rms.h -- full-vector RMSNorm and L2-normalize over the last dimension (gfx950).
//
// Numeric stages follow the reference's structured RMS backend (neptune_codegen/
// emitters.py:549-627, contract skeleton.py:213-217), compiled without FMA contraction:
//   v = fp32(x); total = sum(v*v); count = #columns; mean = div_rn(total, count);
//   scale = rsqrt_rn(mean + eps); n = round_dtype(v * scale); y = n * fp32(gamma) -> dtype.
// L2-normalize (no reference function) uses the same statistics with the readout
//   y = round_dtype(div_rn(v, max(sqrt_rn(total), eps))), i.e. torch.nn.functional.normalize.
//
// Mapping: TPR lanes per row hold the whole row in registers (NV 16-byte slots per lane), so x
// is read once and y written once.  Workgroups loop over row blocks (uniform trip count), and
// gamma stays in registers across rows.
#pragma once

namespace nep {

template <int TPR>
__device__ __forceinline__ float row_sum(float v, float* lds) {
  constexpr int G = TPR < 64 ? TPR : 64;
  v = group_sum<G>(v);
  if constexpr (TPR > 64) {
    constexpr int WPR = TPR / 64;
    const int wave = threadIdx.x >> 6, first = (wave / WPR) * WPR;
    __syncthreads();
    if (lane_id() == 0) lds[wave] = v;
    __syncthreads();
    float r = lds[first];
#pragma unroll
    for (int w = 1; w < WPR; ++w) r += lds[first + w];
    v = r;
  }
  return v;
}

template <class St, bool VECTOR>
struct RowIO {
  typedef typename St::T T;
  static constexpr int VEC = VECTOR ? St::kVec : 1;
  __device__ static __forceinline__ bool load(const T* row, i64 stride_col, i64 e, i64 c1,
                                              float* v) {
    if (e >= c1) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = 0.0f;
      return false;
    }
    if constexpr (VECTOR) St::unpack(load16(row + e), v);
    else v[0] = St::load(row + e * stride_col);
    return true;
  }
  __device__ static __forceinline__ void load_gamma(const T* g, i64 stride_g, i64 e, i64 c1,
                                                    float* v) {
    if (e >= c1) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = 0.0f;
      return;
    }
    if constexpr (VECTOR) St::unpack(load16_cached(g + e), v);
    else v[0] = St::load(g + e * stride_g);
  }
  __device__ static __forceinline__ void store(T* o, i64 e, i64 c1, const float* v) {
    if (e >= c1) return;
    if constexpr (VECTOR) store16(o + e, St::pack(v));
    else St::store(o + e, v[0]);
  }
};

// Readout of one element given the row statistics.
template <class St, bool L2>
__device__ __forceinline__ float rms_readout(float v, float g, float scale) {
  if constexpr (L2) {
    return div_rn(v, scale);  // scale holds max(sqrt_rn(total), eps)
  } else {
    const float normalized = St::round(v * scale);
    return normalized * g;
  }
}

// v / s rounded correctly, with the row's reciprocal y = RN(1/s) shared by its elements:
// q0 = RN(v*y) is within one ulp of v/s, the remainder r = q0*s - v is exact in one FMA, and
// RN(q0 - r*y) is the correctly rounded quotient (Markstein's correction).  Holds for s and
// 1/s normal, v zero (either sign) or |v| >= 2^-100 (below that the remainder can underflow),
// and a normal or zero quotient; the caller sends every other element through div_rn.  Checked
// against IEEE division on the host (tests/csrc/div_by_row_check.c): 2.8e8 random pairs and
// every fp32 v in [2^-100, 2), both signs, for eight divisors, without a difference.
__device__ __forceinline__ float div_by_row(float v, float s, float y) {
  const float q0 = v * y;
  const float r = __builtin_fmaf(q0, s, -v);
  return __builtin_fmaf(-r, y, q0);
}

template <bool L2>
__device__ __forceinline__ float rms_scale(float total, float count, float eps) {
  if constexpr (L2) {
    return __builtin_fmaxf(sqrt_rn(total), eps);
  } else {
    const float mean = div_rn(total, count);
    return rsqrt_rn(mean + eps);
  }
}

// Serial plan: x [rows, ncols] strided -> out [rows, ncols] contiguous.
// Requires ncols <= TPR * NV * VEC (checked by the host).  The vector path keeps the row and
// gamma as packed 16-byte words (NV words each per lane) and unpacks on use, which halves the
// registers of holding them as fp32.
template <class St, int TPR, int NV, bool VECTOR, bool L2, int WG>
__device__ __forceinline__ void rms_serial(const typename St::T* __restrict__ x,
                                           const typename St::T* __restrict__ gamma,
                                           typename St::T* __restrict__ out, i64 rows,
                                           i64 ncols, i64 stride_row, i64 stride_col,
                                           i64 stride_gamma, float eps) {
  typedef RowIO<St, VECTOR> IO;
  constexpr int VEC = IO::VEC;
  constexpr int RPW = WG / TPR;
  __shared__ float lds[WG / 64];
  const int t = threadIdx.x % TPR;
  const float count = (float)ncols;
  if constexpr (VECTOR) {
    // gamma stays in registers as packed words (NV per lane) and is unpacked at its use: no LDS
    // staging and no barrier before the first row (84.1 -> 83.7 us at cfg3).
    u32x4 gr[L2 ? 1 : NV];
    if constexpr (!L2) {
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const i64 e = (i64)(u * TPR + t) * VEC;
        gr[u] = e < ncols ? load16_cached(gamma + e) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    // Rows are double-buffered in registers: the next row's loads are issued before this
    // row is reduced and written, so HBM reads stay in flight across the reduction, the
    // readout and the stores.
    const i64 step = (i64)gridDim.x * RPW;
    u32x4 xn[NV];
    auto fetch = [&](i64 base) {
      const i64 row = base + threadIdx.x / TPR;
      const i64 c1 = row < rows ? ncols : 0;
      const typename St::T* rp = x + (row < rows ? row : 0) * stride_row;
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const i64 e = (i64)(u * TPR + t) * VEC;
        xn[u] = e < c1 ? load16(rp + e) : u32x4{0u, 0u, 0u, 0u};
      }
    };
    if ((i64)blockIdx.x * RPW < rows) fetch((i64)blockIdx.x * RPW);
    for (i64 base = (i64)blockIdx.x * RPW; base < rows; base += step) {
      const i64 row = base + threadIdx.x / TPR;
      const bool live = row < rows;
      const i64 c1 = live ? ncols : 0;
      u32x4 xr[NV];
#pragma unroll
      for (int u = 0; u < NV; ++u) xr[u] = xn[u];
      if (base + step < rows) fetch(base + step);
      float total = 0.0f;
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        float v[VEC];
        St::unpack(xr[u], v);
#pragma unroll
        for (int j = 0; j < VEC; ++j) total += v[j] * v[j];
      }
      // The packed words are re-unpacked for the readout rather than kept as fp32 across the
      // reduction (the empty asm makes them opaque), which halves the row's registers.
#pragma unroll
      for (int u = 0; u < NV; ++u) asm volatile("" : "+v"(xr[u]));
      total = row_sum<TPR>(total, lds);
      const float scale = rms_scale<L2>(total, count, eps);
      typename St::T* op = out + (live ? row : 0) * ncols;
      // L2: the row's elements are divided through div_by_row; a lane holding an element
      // outside its exact range, or a row whose norm (or its reciprocal) is not a normal
      // number -- an infinite sum of squares, a denormal eps under an underflowed sum, an
      // eps of 2^126 or more -- stores div_rn results over them afterwards.
      const float inv = L2 ? 1.0f / scale : 0.0f;
      const float tiny = L2 ? __builtin_fmaxf(0x1p-100f, scale * 0x1p-125f) : 0.0f;
      bool redo = L2 && !(scale >= 0x1p-126f && scale <= 0x1p126f);
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const i64 e = (i64)(u * TPR + t) * VEC;
        if (e >= c1) continue;
        float v[VEC], g[VEC], y[VEC];
        St::unpack(xr[u], v);
        if constexpr (!L2) St::unpack(gr[u], g);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          if constexpr (L2) {
            y[j] = div_by_row(v[j], scale, inv);
            redo |= (__builtin_fabsf(v[j]) < tiny) & (v[j] != 0.0f);
          } else {
            y[j] = rms_readout<St, L2>(v[j], g[j], scale);
          }
        }
        store16(op + e, St::pack(y));
      }
      if constexpr (L2) {
        if (redo) {
#pragma unroll
          for (int u = 0; u < NV; ++u) {
            const i64 e = (i64)(u * TPR + t) * VEC;
            if (e >= c1) continue;
            float v[VEC], y[VEC];
            St::unpack(xr[u], v);
#pragma unroll
            for (int j = 0; j < VEC; ++j) y[j] = div_rn(v[j], scale);
            store16(op + e, St::pack(y));
          }
        }
      }
    }
  } else {
    float g[L2 ? 1 : NV];
    if constexpr (!L2) {
#pragma unroll
      for (int u = 0; u < NV; ++u) IO::load_gamma(gamma, stride_gamma, (i64)(u * TPR + t), ncols, g + u);
    }
    for (i64 base = (i64)blockIdx.x * RPW; base < rows; base += (i64)gridDim.x * RPW) {
      const i64 row = base + threadIdx.x / TPR;
      const bool live = row < rows;
      const i64 c1 = live ? ncols : 0;
      const typename St::T* rp = x + (live ? row : 0) * stride_row;
      float v[NV];
#pragma unroll
      for (int u = 0; u < NV; ++u) IO::load(rp, stride_col, (i64)(u * TPR + t), c1, v + u);
      float total = 0.0f;
#pragma unroll
      for (int u = 0; u < NV; ++u) total += v[u] * v[u];
      total = row_sum<TPR>(total, lds);
      const float scale = rms_scale<L2>(total, count, eps);
      typename St::T* op = out + (live ? row : 0) * ncols;
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        float y = rms_readout<St, L2>(v[u], L2 ? 0.0f : g[u], scale);
        IO::store(op, (i64)(u * TPR + t), c1, &y);
      }
    }
  }
}

// Split plan, partial statistics (emitters.py:597-610): virtual row vr = row*nparts + part
// covers columns [part*block, min(ncols, (part+1)*block)); writes (total fp32, count int64).
template <class St, int TPR, int NV, bool VECTOR, int WG>
__device__ __forceinline__ void rms_split_partial(const typename St::T* __restrict__ x,
                                                  float* __restrict__ totals,
                                                  i64* __restrict__ counts, i64 rows,
                                                  i64 ncols, i64 stride_row, i64 stride_col,
                                                  i64 nparts, i64 block) {
  typedef RowIO<St, VECTOR> IO;
  constexpr int VEC = IO::VEC;
  constexpr int RPW = WG / TPR;
  __shared__ float lds[WG / 64];
  const int t = threadIdx.x % TPR;
  for (i64 base = (i64)blockIdx.x * RPW; base < rows * nparts; base += (i64)gridDim.x * RPW) {
    const i64 vr = base + threadIdx.x / TPR;
    const bool live = vr < rows * nparts;
    const i64 row = live ? vr / nparts : 0, part = live ? vr % nparts : 0;
    const i64 c0 = part * block;
    i64 c1 = c0 + block < ncols ? c0 + block : ncols;
    if (!live) c1 = c0;
    const typename St::T* rp = x + row * stride_row + c0 * stride_col;
    float total = 0.0f;
    for (i64 off = 0; off < c1 - c0; off += (i64)TPR * NV * VEC) {
      float v[NV * VEC];
#pragma unroll
      for (int u = 0; u < NV; ++u)
        IO::load(rp, stride_col, off + (i64)(u * TPR + t) * VEC, c1 - c0, v + u * VEC);
#pragma unroll
      for (int k = 0; k < NV * VEC; ++k) total += v[k] * v[k];
    }
    total = row_sum<TPR>(total, lds);
    if (live && t == 0) {
      totals[vr] = total;
      counts[vr] = c1 - c0;
    }
  }
}

// Split plan, map kernel (emitters.py:613-627): every (row, tile) merges all of the row's
// partial statistics, then normalizes its own tile of `block` columns.
template <class St, int TPR, int NV, bool VECTOR, bool L2, int WG>
__device__ __forceinline__ void rms_split_map(const typename St::T* __restrict__ x,
                                              const typename St::T* __restrict__ gamma,
                                              const float* __restrict__ totals,
                                              const i64* __restrict__ counts,
                                              typename St::T* __restrict__ out, i64 rows,
                                              i64 ncols, i64 stride_row, i64 stride_col,
                                              i64 stride_gamma, i64 nparts, i64 block,
                                              float eps) {
  typedef RowIO<St, VECTOR> IO;
  constexpr int VEC = IO::VEC;
  constexpr int RPW = WG / TPR;
  __shared__ float lds[WG / 64];
  const int t = threadIdx.x % TPR;
  for (i64 base = (i64)blockIdx.x * RPW; base < rows * nparts; base += (i64)gridDim.x * RPW) {
    const i64 vr = base + threadIdx.x / TPR;
    const bool live = vr < rows * nparts;
    const i64 row = live ? vr / nparts : 0, tile = live ? vr % nparts : 0;
    float total = 0.0f, cnt = 0.0f;
    if (live) {
      i64 c = 0;
      for (i64 p = t; p < nparts; p += TPR) {
        total += totals[row * nparts + p];
        c += counts[row * nparts + p];
      }
      cnt = (float)c;  // per-lane count sums are exact in fp32 (width <= 2^22)
    }
    total = row_sum<TPR>(total, lds);
    cnt = row_sum<TPR>(cnt, lds);
    const float scale = rms_scale<L2>(total, cnt, eps);
    const i64 c0 = tile * block;
    i64 c1 = c0 + block < ncols ? c0 + block : ncols;
    if (!live) c1 = c0;
    const typename St::T* rp = x + row * stride_row + c0 * stride_col;
    const typename St::T* gp = gamma + c0 * stride_gamma;
    typename St::T* op = out + row * ncols + c0;
    for (i64 off = 0; off < c1 - c0; off += (i64)TPR * NV * VEC) {
#pragma unroll
      for (int u = 0; u < NV; ++u) {
        const i64 e = off + (i64)(u * TPR + t) * VEC;
        float v[VEC], g[VEC], y[VEC];
        IO::load(rp, stride_col, e, c1 - c0, v);
        if constexpr (!L2) IO::load_gamma(gp, stride_gamma, e, c1 - c0, g);
#pragma unroll
        for (int j = 0; j < VEC; ++j) y[j] = rms_readout<St, L2>(v[j], L2 ? 0.0f : g[j], scale);
        IO::store(op, e, c1 - c0, y);
      }
    }
  }
}

}  // namespace nep
