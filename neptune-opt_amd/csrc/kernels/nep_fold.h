// nep_fold.h -- row folds for scalar repair skeletons on gfx950.
//
// A fold reduces every row of a [rows, ncols] strided matrix to one value through the state
// (m, acc, seen, status): m is the producer value (a running max or sum), acc the consumer
// accumulator kept in the coordinate of m, seen whether any element was folded, status the
// NaN (bit 0) / +inf (bit 1) flags of exponential folds.  Semantics follow the reference's
// generated chunk / merge_state / finalize helpers (neptune_codegen/emitters.py:436-532); the
// algebra of one skeleton arrives as a policy struct F written by the HIP emitter:
//
//   static constexpr bool kLog, kProducerSum, kConsumerMax, kFloor, kHasBias;
//   static float phi(float v, float n)              producer operand of one element
//   static float term(float v, float den, float n)  consumer term at producer value den
//   static float rho(float q, float q2)             repair slope from coordinate q to q2
//   static float beta(float q, float q2)            repair bias (max consumers only)
//   static float finalize(float m, float acc, float n)
//
// Mapping (MI355X): TPR lanes cooperate on one row (TPR <= 64: several rows per wavefront;
// TPR > 64: several wavefronts per row, merged through LDS).  A row is walked in tiles of
// TPR*UNROLL*VEC elements; lane t of the row owns slot (u, t) = elements
// [tile + (u*TPR + t)*VEC, +VEC), so one wavefront-wide load instruction reads consecutive
// 16-byte segments.  VECTOR=false is the general strided path (one element per slot).
#pragma once

namespace nep {

struct State {
  float m;
  float acc;
  int seen;
  int status;
};

template <class F>
__device__ __forceinline__ float eff(float m) {
  if constexpr (F::kFloor) return __builtin_fmaxf(m, 1e-30f);
  else return m;
}

template <class F>
__device__ __forceinline__ float consumer_init() {
  return F::kConsumerMax ? -kInf : 0.0f;
}

// The reference's associative merge (emitters.py:491-517): sanitise both sides before the
// repair is evaluated, transport each accumulator to the combined coordinate, keep the
// non-empty side when only one is seen.  Commutative bit for bit, so butterfly partners agree.
template <class F>
__device__ __forceinline__ State merge_state(const State& A, const State& B) {
  const bool vA = A.seen != 0, vB = B.seen != 0, both = vA && vB;
  const float cm = F::kProducerSum ? (A.m + B.m) : __builtin_fmaxf(A.m, B.m);
  const float oldA = both ? A.m : 1.0f, oldB = both ? B.m : 1.0f, fresh = both ? cm : 1.0f;
  const float qA = eff<F>(oldA), qB = eff<F>(oldB), qN = eff<F>(fresh);
  const float sA = both ? A.acc : 0.0f, sB = both ? B.acc : 0.0f;
  float tA = sA * F::rho(qA, qN), tB = sB * F::rho(qB, qN);
  if constexpr (F::kHasBias) {
    tA += F::beta(qA, qN);
    tB += F::beta(qB, qN);
  }
  const float ca = F::kConsumerMax ? __builtin_fmaxf(tA, tB) : (tA + tB);
  State R;
  R.m = vA ? (vB ? cm : A.m) : B.m;
  R.acc = vA ? (vB ? ca : A.acc) : B.acc;
  R.seen = (vA || vB) ? 1 : 0;
  R.status = A.status | B.status;
  return R;
}

template <int S>
__device__ __forceinline__ State partner_state(const State& s) {
  State o;
  o.m = partner<S>(s.m);
  o.acc = partner<S>(s.acc);
  o.seen = partner<S>(s.seen);
  o.status = partner<S>(s.status);
  return o;
}

template <class F, int G>
__device__ __forceinline__ State group_merge(State s) {
  if constexpr (G >= 2) s = merge_state<F>(s, partner_state<1>(s));
  if constexpr (G >= 4) s = merge_state<F>(s, partner_state<2>(s));
  if constexpr (G >= 8) s = merge_state<F>(s, partner_state<4>(s));
  if constexpr (G >= 16) s = merge_state<F>(s, partner_state<8>(s));
  if constexpr (G >= 32) s = merge_state<F>(s, partner_state<16>(s));
  if constexpr (G >= 64) s = merge_state<F>(s, partner_state<32>(s));
  return s;
}

// Fast exponential-fold lane state: m = max finite phi so far (-inf when none), acc the sum of
// exp(phi - m).  NaN or +inf inputs poison acc (exp(NaN) / exp(inf - inf)); a NaN in a tile with
// no finite element sets `flag`.  Either marks the row for the exact path.
struct LogLane {
  float m;
  float acc;
  int flag;
};

__device__ __forceinline__ LogLane log_merge(const LogLane& A, const LogLane& B) {
  LogLane R;
  R.m = __builtin_fmaxf(A.m, B.m);
  const float a = A.acc * fast_exp(A.m - R.m) + B.acc * fast_exp(B.m - R.m);
  R.acc = (R.m == -kInf) ? 0.0f : a;
  R.flag = A.flag | B.flag;
  return R;
}


// ---------------------------------------------------------------- tile access
template <class St, int TPR, int UNROLL, bool VECTOR>
struct Tiles {
  typedef typename St::T T;
  static constexpr int VEC = VECTOR ? St::kVec : 1;
  static constexpr int K = UNROLL * VEC;
  static constexpr int TILE = TPR * K;

  // Load slot u of the tile starting at column `tile` into v[u*VEC ..]; returns whether the
  // slot lies inside [.., c1).  Out-of-range slots issue no load.
  __device__ static __forceinline__ bool load_slot(const T* row, i64 stride_col, i64 tile,
                                                   i64 c1, int t, int u, float* v) {
    const i64 e = tile + (i64)(u * TPR + t) * VEC;
    if (e >= c1) return false;
    if constexpr (VECTOR) {
      St::unpack(load16(row + e), v + u * VEC);
    } else {
      v[u] = St::load(row + e * stride_col);
    }
    return true;
  }
};

// ---------------------------------------------------------------- row-level combine
// Rows of TPR lanes: TPR <= 64 combines with in-wavefront butterflies; TPR > 64 additionally
// merges the row's wavefront results through LDS (WPR wavefronts per row).
template <int TPR>
struct RowComm {
  static constexpr int G = TPR < 64 ? TPR : 64;
  static constexpr int WPR = TPR > 64 ? TPR / 64 : 1;
};

// ---------------------------------------------------------------- exact path
// The reference chunk of an exponential fold (emitters.py:459-488) over one lane's UNROLL
// slots of VEC values.  slot(u, v) fills v[0..VEC) with slot u's values and returns whether
// the slot lies in the row; it is called once per pass, so a caller may hand out values it
// recomputes rather than holds.
template <class F, int UNROLL, int VEC, class Slot>
__device__ __forceinline__ State log_chunk(Slot slot, float n) {
  State c;
  int status = 0, seen = 0;
  float m = -kInf;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    float v[VEC];
    if (!slot(u, v)) continue;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float p = F::phi(v[j], n);
      if (is_nan(p)) status |= 1;
      if (p == kInf) status |= 2;
      if (is_finite(p)) {
        seen = 1;
        m = __builtin_fmaxf(m, p);
      }
    }
  }
  const float den = seen ? m : 0.0f;
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    float v[VEC];
    if (!slot(u, v)) continue;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float p = F::phi(v[j], n);
      if (is_finite(p)) acc += fast_exp(p - den);
    }
  }
  c.m = m;
  c.acc = acc;
  c.seen = seen;
  c.status = status;
  return c;
}

// The reference chunk over one thread's slots of one tile, merged into the running state.
// Used by every non-exponential fold and, for exponential folds, only on rows whose fast path
// met NaN or +inf.
template <class F, class St, int TPR, int UNROLL, bool VECTOR>
__device__ __forceinline__ void exact_tile(State& s, const typename St::T* row, i64 stride_col,
                                           i64 tile, i64 c1, int t, float n) {
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
  float v[TL::K];
  bool ok[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) ok[u] = TL::load_slot(row, stride_col, tile, c1, t, u, v);
  if constexpr (F::kLog) {
    auto slot = [&](int u, float* w) {
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) w[j] = v[u * TL::VEC + j];
      return ok[u];
    };
    s = merge_state<F>(s, log_chunk<F, UNROLL, TL::VEC>(slot, n));
  } else {
    // Streaming update (one repair per tile instead of merge_state's two): the tile's terms
    // are taken at the combined producer value, and only the carried accumulator is
    // transported, acc' = rho(s.m, m') * acc (+ beta).  In real arithmetic this equals
    // merge_state(s, chunk), whose chunk term is transported by rho(m_tile, m') instead.
    bool any = false;
    float mt = F::kProducerSum ? 0.0f : -kInf;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!ok[u]) continue;
      any = true;
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) {
        const float o = F::phi(v[u * TL::VEC + j], n);
        mt = F::kProducerSum ? (mt + o) : __builtin_fmaxf(mt, o);
      }
    }
    if (!any) return;
    const bool carried = s.seen != 0;
    const float m_new =
        carried ? (F::kProducerSum ? (s.m + mt) : __builtin_fmaxf(s.m, mt)) : mt;
    const float den = eff<F>(m_new);
    float acc = consumer_init<F>();
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!ok[u]) continue;
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) {
        const float tv = F::term(v[u * TL::VEC + j], den, n);
        acc = F::kConsumerMax ? __builtin_fmaxf(acc, tv) : (acc + tv);
      }
    }
    if (carried) {
      const float q = eff<F>(s.m);
      float moved = s.acc * F::rho(q, den);
      if constexpr (F::kHasBias) moved += F::beta(q, den);
      acc = F::kConsumerMax ? __builtin_fmaxf(moved, acc) : (moved + acc);
    }
    s.m = m_new;
    s.acc = acc;
    s.seen = 1;
  }
}

// A row's lane states merged (lanes in order, then waves in order), complete in every lane.
template <class F, int TPR>
__device__ __forceinline__ State row_state(State s, State* lds_state) {
  typedef RowComm<TPR> RC;
  s = group_merge<F, RC::G>(s);
  if constexpr (RC::WPR > 1) {
    const int wave = threadIdx.x >> 6, first = (wave / RC::WPR) * RC::WPR;
    __syncthreads();
    if (lane_id() == 0) lds_state[wave] = s;
    __syncthreads();
    State r = lds_state[first];
#pragma unroll
    for (int w = 1; w < RC::WPR; ++w) r = merge_state<F>(r, lds_state[first + w]);
    s = r;
  }
  return s;
}

template <class F>
__device__ __forceinline__ State empty_state() {
  State s;
  s.m = 0.0f;
  s.acc = consumer_init<F>();
  s.seen = 0;
  s.status = 0;
  return s;
}

// Exact state of the columns [c0, c1) of one row, complete in every lane of the row.
template <class F, class St, int TPR, int UNROLL, bool VECTOR>
__device__ __forceinline__ State exact_row_state(const typename St::T* row, i64 stride_col,
                                                 i64 c0, i64 c1, int t, float n,
                                                 State* lds_state) {
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
  State s = empty_state<F>();
  for (i64 tile = c0; tile < c1; tile += TL::TILE)
    exact_tile<F, St, TPR, UNROLL, VECTOR>(s, row, stride_col, tile, c1, t, n);
  return row_state<F, TPR>(s, lds_state);
}

// Final value of a row from its exact state (emitters.py:522-532 for exponential folds).
template <class F>
__device__ __forceinline__ float finalize_state(const State& s, float n) {
  if constexpr (F::kLog) {
    if (s.status & 1) return __builtin_nanf("");
    if (s.status & 2) return kInf;
    if (!s.seen) return -kInf;
    return F::finalize(s.m, s.acc, n);
  } else {
    return F::finalize(s.m, s.acc, n);
  }
}

// ---------------------------------------------------------------- fast exponential path
// Raw slots of one tile: 16-byte words (VECTOR) or one element each (strided path).  Slots
// past the row's end hold -inf elements, so a fold whose phi is the identity needs no per-element
// test of `ok` (-inf neither raises a max nor adds to an exponential sum).
template <class St, int UNROLL, bool VECTOR>
struct RawTile {
  u32x4 w[VECTOR ? UNROLL : 1];
  float s[VECTOR ? 1 : UNROLL];
  bool ok[UNROLL];
};

template <class St, int TPR, int UNROLL, bool VECTOR>
__device__ __forceinline__ void load_raw(RawTile<St, UNROLL, VECTOR>& r,
                                         const typename St::T* row, i64 stride_col, i64 tile,
                                         i64 c1, int t) {
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const i64 e = tile + (i64)(u * TPR + t) * TL::VEC;
    r.ok[u] = e < c1;
    if constexpr (VECTOR) {
      // a uniform base plus a 32-bit lane offset (the tile is below 2^31 elements)
      const u32 f = St::kNegInfWord;
      r.w[u] = r.ok[u] ? load16(row + tile + (u32)((u * TPR + t) * TL::VEC)) : u32x4{f, f, f, f};
    } else {
      r.s[u] = r.ok[u] ? St::load(row + e * stride_col) : -kInf;
    }
  }
}

// The held words of a raw tile, made opaque to the compiler: unpacks after this point cannot
// reuse values unpacked before it, so a pass over a held row re-derives its fp32 values from
// the 16-bit words instead of keeping them live (no instruction is emitted).
template <class St, int UNROLL, bool VECTOR>
__device__ __forceinline__ void reopen(RawTile<St, UNROLL, VECTOR>& r) {
  if constexpr (VECTOR) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) asm volatile("" : "+v"(r.w[u]));
  }
}

// Fold one raw tile into a lane's exponential state.  Per element: one max, one fma for the
// base-2 exponent, one exp2, one add.  The exponent p*log2e - m*log2e carries an absolute
// error of about |m| * 2^-23, which is relative to the readout m + log(acc): the row result
// keeps ~1e-7 relative accuracy.
//
// CENTERED evaluates exp2((p - m) * log2e) instead: p - m is exact, so an element equal to the
// row maximum contributes exactly 1 (one more VALU op per element).  The readout uses it, so
// that a log-probability of 0 comes out as 0 rather than as the rounding residue of m*log2e.
// The readout also holds its whole row in the raw words, so the centred fold recomputes phi
// from them in each pass rather than holding the K fp32 terms across the max (K = 64 for a
// 16-bit row of 8 slots: 64 VGPRs, which would cut the readout to one 8-wave workgroup per
// CU); the terms and their order are the same.  Only the identity term is recomputed: a
// term with arithmetic in it (softcap's tanh) is evaluated once and held, since evaluating it
// twice cost softcap_lse a quarter of its time (fp32 16384x4096: 41.8 -> 51.5 us).
template <class F, class St, int TPR, int UNROLL, bool VECTOR, bool CENTERED>
__device__ __forceinline__ void log_fold_tile(LogLane& s, RawTile<St, UNROLL, VECTOR>& cur,
                                              float n) {
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
  // The identity term is re-read from the raw words in each pass (only the words stay live);
  // any other term (a tanh, a scale, a bias) is evaluated once and held.
  float held[F::kPhiIdentity ? 1 : TL::K];
  if constexpr (!F::kPhiIdentity) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      float v[TL::VEC];
      if constexpr (VECTOR) St::unpack(cur.w[u], v);
      else v[0] = cur.s[u];
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j)
        held[u * TL::VEC + j] = cur.ok[u] ? F::phi(v[j], n) : -kInf;
    }
  }
  auto terms = [&](int u, float* p) {
    if constexpr (F::kPhiIdentity) {
      float v[TL::VEC];
      if constexpr (VECTOR) St::unpack(cur.w[u], v);
      else v[0] = cur.s[u];
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) p[j] = v[j];
    } else {
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) p[j] = held[u * TL::VEC + j];
    }
  };
  float tm = -kInf;
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    float p[TL::VEC];
    terms(u, p);
#pragma unroll
    for (int j = 0; j < TL::VEC; ++j) tm = __builtin_fmaxf(tm, p[j]);
  }
  if constexpr (CENTERED && F::kPhiIdentity) reopen(cur);
  const float mn = __builtin_fmaxf(s.m, tm);
  if (mn == -kInf) {
    // No finite or +inf value yet; a NaN would otherwise be skipped by the max.
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      float p[TL::VEC];
      terms(u, p);
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) s.flag |= is_nan(p[j]) ? 1 : 0;
    }
  } else {
    const float ml = mn * kLog2e;
    // |m| above ~2.3e38 overflows m*log2e: route the row to the exact (subtracting) path.
    if (!is_finite(ml) && is_finite(mn)) s.flag = 1;
    float a = s.acc * fast_exp(s.m - mn);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      float p[TL::VEC];
      terms(u, p);
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) {
        if constexpr (CENTERED) a += __builtin_amdgcn_exp2f((p[j] - mn) * kLog2e);
        else a += __builtin_amdgcn_exp2f(__builtin_fmaf(p[j], kLog2e, -ml));
      }
    }
    s.acc = a;
    s.m = mn;
  }
}

// One lane's exponential fold over its slots of [c0, c1).  The next tile's loads are issued
// before the current tile is folded, so each lane keeps up to 2*UNROLL loads in flight.
template <class F, class St, int TPR, int UNROLL, bool VECTOR, bool CENTERED = false>
__device__ __forceinline__ LogLane log_row_lane(const typename St::T* row, i64 stride_col,
                                                i64 c0, i64 c1, int t, float n) {
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
  LogLane s;
  s.m = -kInf;
  s.acc = 0.0f;
  s.flag = 0;
  if (c0 >= c1) return s;
  RawTile<St, UNROLL, VECTOR> cur;
  load_raw<St, TPR, UNROLL, VECTOR>(cur, row, stride_col, c0, c1, t);
  for (i64 tile = c0; tile < c1; tile += TL::TILE) {
    RawTile<St, UNROLL, VECTOR> nxt;
    const bool more = tile + TL::TILE < c1;
    if (more) load_raw<St, TPR, UNROLL, VECTOR>(nxt, row, stride_col, tile + TL::TILE, c1, t);
    log_fold_tile<F, St, TPR, UNROLL, VECTOR, CENTERED>(s, cur, n);
    if (more) cur = nxt;
  }
  return s;
}

// A row's lanes combine in two reductions instead of a tree of pairwise merges: the row max
// first, then each lane moves its sum to it once (one exponential per lane instead of one per
// tree level and partner) and the sums are added.  A lane with no finite value contributes 0;
// NaN sums (a +inf element) stay NaN and send the row to the exact path as before.
template <class F, int TPR>
__device__ __forceinline__ LogLane log_row_combine(LogLane s, LogLane* lds) {
  typedef RowComm<TPR> RC;
  {
    const float row_m = group_max<RC::G>(s.m);
    const float moved = (s.m == -kInf) ? 0.0f : s.acc * fast_exp(s.m - row_m);
    s.acc = group_sum<RC::G>(moved);
    s.m = row_m;
    s.flag = group_or<RC::G>(s.flag);
  }
  if constexpr (RC::WPR > 1) {
    const int wave = threadIdx.x >> 6, first = (wave / RC::WPR) * RC::WPR;
    if (lane_id() == 0) lds[wave] = s;
    __syncthreads();
    LogLane r = lds[first];
#pragma unroll
    for (int w = 1; w < RC::WPR; ++w) r = log_merge(r, lds[first + w]);
    s = r;
  }
  return s;
}

// ---------------------------------------------------------------- kernel bodies
// Serial plan: one output per row (template.py:41-54).  WG threads per workgroup, WG/TPR rows
// per workgroup (one row when TPR >= WG).
// The row's fp32 result in every lane of the row from the lanes' fast exponential states,
// with the exact fallback for rows that met NaN or +inf: exact(bad) returns the row's exact
// state (a lane passes bad = false to take part in the row's synchronisation only).  Every
// thread of the workgroup must call it (it synchronises when a row spans several wavefronts).
template <class F, int TPR, class Exact>
__device__ __forceinline__ float log_row_result(LogLane s, float n, LogLane* lds_lane,
                                                Exact exact) {
  float result;
  s = log_row_combine<F, TPR>(s, lds_lane);
  const bool bad = s.flag != 0 || is_nan(s.acc);
  // Rows with NaN/+inf take the exact reference path; `bad` is uniform across the row.
  bool any_bad = bad;
  if constexpr (TPR > 64) {
    any_bad = __syncthreads_or(bad ? 1 : 0) != 0;
  } else {
    any_bad = __builtin_amdgcn_ballot_w64(bad) != 0;
  }
  if (any_bad) {
    const State e = exact(bad);
    if (bad) result = finalize_state<F>(e, n);
  }
  if (!bad) result = (s.m == -kInf) ? -kInf : F::finalize(s.m, s.acc, n);
  return result;
}

// The same with the exact path re-reading the row from memory.
template <class F, class St, int TPR, int UNROLL, bool VECTOR>
__device__ __forceinline__ float log_row_finish(LogLane s, const typename St::T* rp,
                                                i64 stride_col, i64 c1, int t, float n,
                                                State* lds_state, LogLane* lds_lane) {
  return log_row_result<F, TPR>(s, n, lds_lane, [&](bool bad) {
    return exact_row_state<F, St, TPR, UNROLL, VECTOR>(rp, stride_col, 0, bad ? c1 : 0, t, n,
                                                       lds_state);
  });
}

template <class F, class St, int TPR, int UNROLL, bool VECTOR, bool CENTERED = false>
__device__ __forceinline__ float row_result(const typename St::T* rp, i64 stride_col, i64 c1,
                                            int t, float n, State* lds_state,
                                            LogLane* lds_lane) {
  if constexpr (F::kLog) {
    const LogLane s =
        log_row_lane<F, St, TPR, UNROLL, VECTOR, CENTERED>(rp, stride_col, 0, c1, t, n);
    return log_row_finish<F, St, TPR, UNROLL, VECTOR>(s, rp, stride_col, c1, t, n, lds_state,
                                                      lds_lane);
  } else {
    const State e = exact_row_state<F, St, TPR, UNROLL, VECTOR>(rp, stride_col, 0, c1, t, n,
                                                                 lds_state);
    return finalize_state<F>(e, n);
  }
}

template <class F, class St, int TPR, int UNROLL, bool VECTOR, int WG>
__device__ __forceinline__ void fold_serial(const typename St::T* __restrict__ x,
                                            typename St::T* __restrict__ out, i64 rows,
                                            i64 ncols, i64 stride_row, i64 stride_col) {
  static_assert(WG % 64 == 0 && (TPR <= 64 || WG % TPR == 0), "bad row mapping");
  constexpr int RPW = WG / TPR;  // rows per workgroup
  __shared__ State lds_state[WG / 64];
  __shared__ LogLane lds_lane[WG / 64];
  const int t = threadIdx.x % TPR;
  const i64 row = (i64)blockIdx.x * RPW + threadIdx.x / TPR;
  const bool live = row < rows;
  const typename St::T* rp = x + (live ? row : 0) * stride_row;
  const i64 c1 = live ? ncols : 0;
  const float n = (float)ncols;
  const float result =
      row_result<F, St, TPR, UNROLL, VECTOR>(rp, stride_col, c1, t, n, lds_state, lds_lane);
  if (live && t == 0) St::store(out + row, result);
}

// Readout of an exponential fold (log-softmax for logsumexp): out[row, c] = phi(x[row, c]) -
// r, r the row's fp32 result, computed in fp32 and rounded once to the storage type; with
// NAN_POSINF a row whose r is +inf (a +inf element) reads out NaN everywhere, as the lowered
// `where(lse == inf, nan, x - lse)` does.  `out` is contiguous [rows, ncols].  RESIDENT
// kernels take rows that fit in one tile (ncols <= TPR * UNROLL * VEC, checked by the host),
// which stay in registers between the fold and the readout (one HBM read); the others take
// any width and read the row twice.  The two are separate kernels so that each is allocated
// the registers of its own path.
template <class F, class St, int TPR, int UNROLL, bool VECTOR, int WG, bool NAN_POSINF,
          bool RESIDENT>
__device__ __forceinline__ void fold_readout(const typename St::T* __restrict__ x,
                                             typename St::T* __restrict__ out, i64 rows,
                                             i64 ncols, i64 stride_row, i64 stride_col) {
  static_assert(F::kLog, "the readout is defined for exponential folds");
  static_assert(WG % 64 == 0 && (TPR <= 64 || WG % TPR == 0), "bad row mapping");
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
  constexpr int RPW = WG / TPR;
  __shared__ State lds_state[WG / 64];
  __shared__ LogLane lds_lane[WG / 64];
  const int t = threadIdx.x % TPR;
  // one row per workgroup: the row, and so its base addresses, are wave-uniform
  const i64 row = RPW == 1 ? (i64)blockIdx.x : (i64)blockIdx.x * RPW + threadIdx.x / TPR;
  const bool live = row < rows;
  const typename St::T* rp = x + (live ? row : 0) * stride_row;
  typename St::T* op = out + (live ? row : 0) * ncols;
  const i64 c1 = live ? ncols : 0;
  const float n = (float)ncols;
  if constexpr (RESIDENT) {
    RawTile<St, UNROLL, VECTOR> keep;
    load_raw<St, TPR, UNROLL, VECTOR>(keep, rp, stride_col, 0, c1, t);
    LogLane s;
    s.m = -kInf;
    s.acc = 0.0f;
    s.flag = 0;
    log_fold_tile<F, St, TPR, UNROLL, VECTOR, true>(s, keep, n);
    // The exact fallback takes the row from the registers too: its state equals
    // exact_row_state's over the one tile (same slots, same order), without a second set of
    // fp32 values live beside `keep`.
    const float r = log_row_result<F, TPR>(s, n, lds_lane, [&](bool bad) {
      State e = empty_state<F>();
      if (bad) {
        auto slot = [&](int u, float* w) {
          if constexpr (VECTOR) {
            St::reunpack(keep.w[u], w);
          } else {
            w[0] = keep.s[u];
          }
          return keep.ok[u];
        };
        e = merge_state<F>(e, log_chunk<F, UNROLL, TL::VEC>(slot, n));
      }
      return row_state<F, TPR>(e, lds_state);
    });
    // A NaN row reads out phi(x) - NaN: NaN everywhere (such a row holds no NaN of its own,
    // which would have made r NaN), without a select per element.
    const float rr = (NAN_POSINF && r == kInf) ? __builtin_nanf("") : r;
    reopen(keep);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!keep.ok[u]) continue;
      const i64 e = (i64)(u * TPR + t) * TL::VEC;
      if constexpr (VECTOR) {
        float v[TL::VEC];
        St::unpack(keep.w[u], v);
#pragma unroll
        for (int j = 0; j < TL::VEC; ++j) v[j] = F::phi(v[j], n) - rr;
        store16(op + (u32)((u * TPR + t) * TL::VEC), St::pack(v));
      } else {
        St::store(op + e, F::phi(keep.s[u], n) - rr);
      }
    }
  } else {
    const float r = row_result<F, St, TPR, UNROLL, VECTOR, true>(rp, stride_col, c1, t, n,
                                                                lds_state, lds_lane);
    const float rr = (NAN_POSINF && r == kInf) ? __builtin_nanf("") : r;
    for (i64 tile = 0; tile < c1; tile += TL::TILE) {
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const i64 e = tile + (i64)(u * TPR + t) * TL::VEC;
        if (e >= c1) continue;
        if constexpr (VECTOR) {
          float v[TL::VEC];
          St::unpack(load16(rp + e), v);
#pragma unroll
          for (int j = 0; j < TL::VEC; ++j) v[j] = F::phi(v[j], n) - rr;
          store16(op + e, St::pack(v));
        } else {
          St::store(op + e, F::phi(St::load(rp + e * stride_col), n) - rr);
        }
      }
    }
  }
}

// Split plan, partial kernel (template.py:137-148): virtual row vr = row*nparts + part covers
// columns [part*block, min(ncols, (part+1)*block)) and writes its exact chunk state.
template <class F, class St, int TPR, int UNROLL, bool VECTOR, int WG>
__device__ __forceinline__ void fold_split_partial(const typename St::T* __restrict__ x,
                                                   float* __restrict__ pm,
                                                   float* __restrict__ pa,
                                                   int* __restrict__ pv,
                                                   int* __restrict__ ps, i64 rows, i64 ncols,
                                                   i64 stride_row, i64 stride_col,
                                                   i64 nparts, i64 block) {
  constexpr int RPW = WG / TPR;
  __shared__ State lds_state[WG / 64];
  __shared__ LogLane lds_lane[WG / 64];
  const int t = threadIdx.x % TPR;
  const i64 vr = (i64)blockIdx.x * RPW + threadIdx.x / TPR;
  const bool live = vr < rows * nparts;
  const i64 row = live ? vr / nparts : 0;
  const i64 part = live ? vr % nparts : 0;
  const typename St::T* rp = x + row * stride_row;
  const i64 c0 = part * block;
  i64 c1 = c0 + block;
  c1 = c1 < ncols ? c1 : ncols;
  if (!live) c1 = c0;
  const float n = (float)ncols;
  State out_state;
  if constexpr (F::kLog) {
    LogLane s = log_row_lane<F, St, TPR, UNROLL, VECTOR>(rp, stride_col, c0, c1, t, n);
    s = log_row_combine<F, TPR>(s, lds_lane);
    const bool bad = s.flag != 0 || is_nan(s.acc);
    bool any_bad;
    if constexpr (TPR > 64) any_bad = __syncthreads_or(bad ? 1 : 0) != 0;
    else any_bad = __builtin_amdgcn_ballot_w64(bad) != 0;
    out_state.m = s.m;
    out_state.acc = s.acc;
    out_state.seen = (s.m != -kInf) ? 1 : 0;
    out_state.status = 0;
    if (any_bad) {
      const State e = exact_row_state<F, St, TPR, UNROLL, VECTOR>(rp, stride_col, c0,
                                                                   bad ? c1 : c0, t, n,
                                                                   lds_state);
      if (bad) out_state = e;
    }
  } else {
    out_state = exact_row_state<F, St, TPR, UNROLL, VECTOR>(rp, stride_col, c0, c1, t, n,
                                                             lds_state);
  }
  if (live && t == 0) {
    pm[vr] = out_state.m;
    pa[vr] = out_state.acc;
    pv[vr] = out_state.seen;
    ps[vr] = out_state.status;
  }
}

// Split plan, merge kernel (template.py:151-164): one wavefront per row folds the row's
// nparts partial states with merge_state and finalizes.
template <class F, class St>
__device__ __forceinline__ void fold_split_merge(const float* __restrict__ pm,
                                                 const float* __restrict__ pa,
                                                 const int* __restrict__ pv,
                                                 const int* __restrict__ ps,
                                                 typename St::T* __restrict__ out, i64 rows,
                                                 i64 ncols, i64 nparts) {
  const int lane = threadIdx.x & 63;
  const i64 row = (i64)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const bool live = row < rows;
  State s;
  s.m = 0.0f;
  s.acc = consumer_init<F>();
  s.seen = 0;
  s.status = 0;
  if (live) {
    // four partial states per lane are loaded before any is merged, so one memory latency
    // covers up to 256 parts
    constexpr int PRE = 4;
    for (i64 p0 = lane; p0 < nparts; p0 += 64 * PRE) {
      State c[PRE];
      bool ok[PRE];
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
        const i64 p = p0 + 64 * u;
        ok[u] = p < nparts;
        if (ok[u]) {
          const i64 slot = row * nparts + p;
          c[u].m = pm[slot];
          c[u].acc = pa[slot];
          c[u].seen = pv[slot];
          c[u].status = ps[slot];
        }
      }
#pragma unroll
      for (int u = 0; u < PRE; ++u)
        if (ok[u]) s = merge_state<F>(s, c[u]);
    }
  }
  s = group_merge<F, 64>(s);
  if (live && lane == 0) St::store(out + row, finalize_state<F>(s, (float)ncols));
}

// Two-pass plan (template.py:62-103): pass 1 reduces the producer over the row, pass 2 the
// term with the producer held constant.  The second pass re-reads the row.
template <class F, class St, int TPR, int UNROLL, bool VECTOR, int WG>
__device__ __forceinline__ void fold_two_pass(const typename St::T* __restrict__ x,
                                              typename St::T* __restrict__ out, i64 rows,
                                              i64 ncols, i64 stride_row, i64 stride_col) {
  typedef Tiles<St, TPR, UNROLL, VECTOR> TL;
  typedef RowComm<TPR> RC;
  constexpr int RPW = WG / TPR;
  __shared__ float lds[WG / 64];
  const int t = threadIdx.x % TPR;
  const i64 row = (i64)blockIdx.x * RPW + threadIdx.x / TPR;
  const bool live = row < rows;
  const typename St::T* rp = x + (live ? row : 0) * stride_row;
  const i64 c1 = live ? ncols : 0;
  const float n = (float)ncols;
  const int wave = threadIdx.x >> 6, first = (wave / RC::WPR) * RC::WPR;
  // A row that fits in one tile stays in registers: pass 2 reads what pass 1 loaded, so the
  // row crosses HBM once (same values, same order as reading it twice).
  const bool resident = ncols <= TL::TILE;
  float keep[TL::K];
  bool kept[UNROLL];
  // pass 1: the producer
  float m = F::kProducerSum ? 0.0f : -kInf;
  if (resident) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      kept[u] = TL::load_slot(rp, stride_col, 0, c1, t, u, keep);
      if (!kept[u]) continue;
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) {
        const float o = F::phi(keep[u * TL::VEC + j], n);
        m = F::kProducerSum ? (m + o) : __builtin_fmaxf(m, o);
      }
    }
  } else {
    for (i64 tile = 0; tile < c1; tile += TL::TILE) {
      float v[TL::K];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        if (!TL::load_slot(rp, stride_col, tile, c1, t, u, v)) continue;
#pragma unroll
        for (int j = 0; j < TL::VEC; ++j) {
          const float o = F::phi(v[u * TL::VEC + j], n);
          m = F::kProducerSum ? (m + o) : __builtin_fmaxf(m, o);
        }
      }
    }
  }
  m = F::kProducerSum ? group_sum<RC::G>(m) : group_max<RC::G>(m);
  if constexpr (RC::WPR > 1) {
    if (lane_id() == 0) lds[wave] = m;
    __syncthreads();
    float r = lds[first];
#pragma unroll
    for (int w = 1; w < RC::WPR; ++w)
      r = F::kProducerSum ? (r + lds[first + w]) : __builtin_fmaxf(r, lds[first + w]);
    m = r;
    __syncthreads();
  }
  // pass 2: the term at the final producer value
  float acc = consumer_init<F>();
  if (resident) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (!kept[u]) continue;
#pragma unroll
      for (int j = 0; j < TL::VEC; ++j) {
        const float tv = F::term(keep[u * TL::VEC + j], m, n);
        acc = F::kConsumerMax ? __builtin_fmaxf(acc, tv) : (acc + tv);
      }
    }
  } else {
    for (i64 tile = 0; tile < c1; tile += TL::TILE) {
      float v[TL::K];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        if (!TL::load_slot(rp, stride_col, tile, c1, t, u, v)) continue;
#pragma unroll
        for (int j = 0; j < TL::VEC; ++j) {
          const float tv = F::term(v[u * TL::VEC + j], m, n);
          acc = F::kConsumerMax ? __builtin_fmaxf(acc, tv) : (acc + tv);
        }
      }
    }
  }
  acc = F::kConsumerMax ? group_max<RC::G>(acc) : group_sum<RC::G>(acc);
  if constexpr (RC::WPR > 1) {
    if (lane_id() == 0) lds[wave] = acc;
    __syncthreads();
    float r = lds[first];
#pragma unroll
    for (int w = 1; w < RC::WPR; ++w)
      r = F::kConsumerMax ? __builtin_fmaxf(r, lds[first + w]) : (r + lds[first + w]);
    acc = r;
  }
  if (live && t == 0) St::store(out + row, F::finalize(m, acc, n));
}

}  // namespace nep
