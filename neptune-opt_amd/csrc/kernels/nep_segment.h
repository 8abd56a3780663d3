// nep_segment.h -- CSR segment sum / mean with ordered storage-dtype rounding (gfx950).
//
// Numeric contract of the reference segment backend (neptune_codegen/torch_op.py:286-306,
// skeleton.py:218-221): for each (segment, channel) the accumulator starts at
// round_dtype(fp32(initial)); tokens are added strictly in order as
// acc = round_dtype(acc + fp32(x[token, channel])) with round-to-nearest-even; mean divides by
// fp32(round_dtype(count)) with a correctly rounded division; an empty mean is NaN unless an
// initial value was given; a malformed span [start, end) yields NaN and issues no load.
//
// For fp16 the per-token fp32-add-then-round equals the IEEE binary16 addition (binary32 has
// 24 >= 2*11+2 significand bits, so double rounding is innocuous); the vector path therefore
// adds packed halves (v_pk_add_f16).  bf16 and fp32 add in fp32 and round explicitly.
//
// Mapping: vector path -- LPS lanes per segment, each lane owns one 16-byte channel vector,
// 64/LPS segments per wavefront, UNR token rows prefetched per step; generic path -- one lane
// per channel, 64-channel tiles, any strides.
//
// Descriptor validation (the reference's device-side span asserts, torch_op.py:378-386) is
// fused into the fold: with `status` non-null, a lane whose span is malformed, or the last
// segment's lanes when its end differs from `cover` (>= 0: the coverage check of lengths
// input), store 0 to status[0] (which the caller set to 1).  Every writer stores the same
// value, so the unordered stores are benign.
#pragma once

namespace nep {

template <class St>
struct SegAcc;

template <>
struct SegAcc<F32> {
  float a[4];
  __device__ __forceinline__ void init(float v) {
    a[0] = a[1] = a[2] = a[3] = v;
  }
  __device__ __forceinline__ void add(const u32x4& w) {
    a[0] = a[0] + as_f32(w.x);
    a[1] = a[1] + as_f32(w.y);
    a[2] = a[2] + as_f32(w.z);
    a[3] = a[3] + as_f32(w.w);
  }
  __device__ __forceinline__ void get(float* o) const {
    for (int j = 0; j < 4; ++j) o[j] = a[j];
  }
};

template <>
struct SegAcc<BF16> {
  float a[8];
  __device__ __forceinline__ void init(float v) {
    for (int j = 0; j < 8; ++j) a[j] = v;
  }
  __device__ __forceinline__ void add(const u32x4& w) {
    float v[8];
    BF16::unpack(w, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = BF16::round(a[j] + v[j]);
  }
  __device__ __forceinline__ void get(float* o) const {
    for (int j = 0; j < 8; ++j) o[j] = a[j];
  }
};

template <>
struct SegAcc<F16> {
  half2_t a[4];
  __device__ __forceinline__ void init(float v) {
    half2_t h;
    h.x = (_Float16)v;
    h.y = h.x;
    a[0] = a[1] = a[2] = a[3] = h;
  }
  __device__ __forceinline__ void add(const u32x4& w) {
    a[0] = a[0] + as_half2(w.x);
    a[1] = a[1] + as_half2(w.y);
    a[2] = a[2] + as_half2(w.z);
    a[3] = a[3] + as_half2(w.w);
  }
  __device__ __forceinline__ void get(float* o) const {
    for (int j = 0; j < 4; ++j) {
      o[2 * j] = (float)a[j].x;
      o[2 * j + 1] = (float)a[j].y;
    }
  }
};

template <class SpanT>
__device__ __forceinline__ bool read_span(const SpanT* spans, i64 stride_span, i64 seg,
                                          i64 nrows, i64* start, i64* end) {
  const i64 s = (i64)spans[seg * stride_span];
  const i64 e = (i64)spans[(seg + 1) * stride_span];
  *start = s;
  *end = e;
  return s >= 0 && e >= s && e <= nrows;
}

__device__ __forceinline__ void segment_check(int* status, bool valid, i64 seg, i64 nsegments,
                                              i64 end, i64 cover) {
  if (status != nullptr && (!valid || (cover >= 0 && seg == nsegments - 1 && end != cover)))
    status[0] = 0;
}

template <class St, bool MEAN, bool INIT_NONE>
__device__ __forceinline__ float segment_readout(float acc, bool valid, i64 start, i64 end) {
  float r = acc;
  if constexpr (MEAN) {
    const float den = St::round((float)(end - start));
    r = div_rn(acc, den);
    if (end == start) r = INIT_NONE ? __builtin_nanf("") : acc;
  }
  return valid ? r : __builtin_nanf("");
}

// Vector path: channels == LPS * VEC, data rows 16-byte aligned with unit channel stride.
template <class St, class SpanT, bool MEAN, bool INIT_NONE, int LPS, int UNR, int WG>
__device__ __forceinline__ void segment_vector(const typename St::T* __restrict__ data,
                                               const SpanT* __restrict__ spans,
                                               typename St::T* __restrict__ out, i64 nrows,
                                               i64 channels, i64 nsegments, i64 stride_row,
                                               i64 stride_span, float initial, int* status,
                                               i64 cover) {
  constexpr int VEC = St::kVec;
  constexpr int SPW = WG / LPS;  // segments per workgroup
  const int l = threadIdx.x % LPS;
  const i64 seg = (i64)blockIdx.x * SPW + threadIdx.x / LPS;
  if (seg >= nsegments) return;
  i64 start, end;
  const bool valid = read_span(spans, stride_span, seg, nrows, &start, &end);
  segment_check(status, valid, seg, nsegments, end, cover);
  SegAcc<St> acc;
  acc.init(St::round(initial));
  if (valid) {
    const typename St::T* col = data + (i64)l * VEC;
    for (i64 t = start; t < end; t += UNR) {
      u32x4 w[UNR];
#pragma unroll
      for (int i = 0; i < UNR; ++i)
        if (t + i < end) w[i] = load16(col + (t + i) * stride_row);
#pragma unroll
      for (int i = 0; i < UNR; ++i)
        if (t + i < end) acc.add(w[i]);
    }
  }
  float a[VEC], r[VEC];
  acc.get(a);
#pragma unroll
  for (int j = 0; j < VEC; ++j) r[j] = segment_readout<St, MEAN, INIT_NONE>(a[j], valid, start, end);
  store16(out + seg * channels + (i64)l * VEC, St::pack(r));
}

// Generic path: grid (nsegments, ceil(channels / 64)), one lane per channel.
template <class St, class SpanT, bool MEAN, bool INIT_NONE, int UNR>
__device__ __forceinline__ void segment_generic(const typename St::T* __restrict__ data,
                                                const SpanT* __restrict__ spans,
                                                typename St::T* __restrict__ out, i64 nrows,
                                                i64 channels, i64 nsegments, i64 stride_row,
                                                i64 stride_channel, i64 stride_span,
                                                float initial, int* status, i64 cover) {
  const i64 seg = blockIdx.x;
  const i64 c = (i64)blockIdx.y * 64 + (threadIdx.x & 63);
  if (seg >= nsegments || c >= channels) return;
  i64 start, end;
  const bool valid = read_span(spans, stride_span, seg, nrows, &start, &end);
  segment_check(status, valid, seg, nsegments, end, cover);
  float acc = St::round(initial);
  if (valid) {
    const typename St::T* col = data + c * stride_channel;
    for (i64 t = start; t < end; t += UNR) {
      float v[UNR];
#pragma unroll
      for (int i = 0; i < UNR; ++i)
        if (t + i < end) v[i] = St::load(col + (t + i) * stride_row);
#pragma unroll
      for (int i = 0; i < UNR; ++i)
        if (t + i < end) acc = St::round(acc + v[i]);
    }
  }
  St::store(out + seg * channels + c, segment_readout<St, MEAN, INIT_NONE>(acc, valid, start, end));
}

// ---------------------------------------------------------------- lengths -> spans
// spans[0] = 0, spans[i + 1] = lengths[0] + ... + lengths[i] in int64: the reference's
// cat(0, cumsum(lengths)) (torch_op.py:370-387).  Two launches over blocks of kSpanBlock
// lengths: the block sums, then each block scans itself on top of the sum of the blocks before
// it (no inter-workgroup synchronisation).  Bad lengths are not judged here: the segment
// kernel's span checks see the resulting spans.
constexpr int kSpanThreads = 256;
constexpr int kSpanPer = 4;
constexpr i64 kSpanBlock = (i64)kSpanThreads * kSpanPer;

__device__ __forceinline__ i64 wave_sum_i64(i64 v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Sum over the workgroup, returned to every thread.
__device__ __forceinline__ i64 block_sum_i64(i64 v, i64* lds) {
  v = wave_sum_i64(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[wave] = v;
  __syncthreads();
  i64 total = 0;
#pragma unroll
  for (int w = 0; w < kSpanThreads / 64; ++w) total += lds[w];
  return total;
}

// Exclusive scan over the workgroup's threads (in thread order).
__device__ __forceinline__ i64 block_exclusive_i64(i64 v, i64* lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  i64 inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const i64 o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  __syncthreads();
  if (lane == 63) lds[wave] = inc;
  __syncthreads();
  i64 before = 0;
  for (int w = 0; w < wave; ++w) before += lds[w];
  return before + inc - v;
}

// Block sums of the lengths; block 0 also sets the segment kernel's status word to 1 (this
// launch precedes the segment kernel on the same stream, so no separate fill is needed).
template <class L>
__device__ __forceinline__ void spans_block_sums(const L* __restrict__ lengths, i64 n,
                                                 i64* __restrict__ sums, int* __restrict__ status) {
  __shared__ i64 lds[kSpanThreads / 64];
  if (status != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *status = 1;
  const i64 base = (i64)blockIdx.x * kSpanBlock + (i64)threadIdx.x * kSpanPer;
  i64 s = 0;
#pragma unroll
  for (int k = 0; k < kSpanPer; ++k)
    if (base + k < n) s += (i64)lengths[base + k];
  s = block_sum_i64(s, lds);
  if (threadIdx.x == 0) sums[blockIdx.x] = s;
}

template <class L>
__device__ __forceinline__ void spans_scan(const L* __restrict__ lengths, i64 n,
                                           const i64* __restrict__ sums,
                                           i64* __restrict__ spans) {
  __shared__ i64 lds[kSpanThreads / 64];
  i64 before = 0;
  for (i64 b = threadIdx.x; b < (i64)blockIdx.x; b += kSpanThreads) before += sums[b];
  before = block_sum_i64(before, lds);
  const i64 base = (i64)blockIdx.x * kSpanBlock + (i64)threadIdx.x * kSpanPer;
  i64 run[kSpanPer];
  i64 acc = 0;
#pragma unroll
  for (int k = 0; k < kSpanPer; ++k) {
    acc += base + k < n ? (i64)lengths[base + k] : 0;
    run[k] = acc;
  }
  const i64 offset = before + block_exclusive_i64(acc, lds);
#pragma unroll
  for (int k = 0; k < kSpanPer; ++k)
    if (base + k < n) spans[base + k + 1] = offset + run[k];
  if (blockIdx.x == 0 && threadIdx.x == 0) spans[0] = 0;
}

}  // namespace nep
