// rlk_ops.hpp -- the rl_triton estimators as producers/epilogues of the scan engine.
//
// Each struct turns its inputs into per-step affine coefficients (truncation and
// bootstrap handling folded in, so there is no extra pass) and turns the scanned
// values into the estimator's outputs.  Semantics follow the reference's fused Triton
// kernels (simonsays1980/rl-triton v0.1.3, src/rl_triton/kernels/*.py); each struct
// cites the lines it reproduces.  Padding steps (t >= T) are the identity map.
//
// Optional operands that change which arrays are read (truncations, TD(lambda)'s next
// values) are template parameters; loads are clamped into the row and absent per-row
// values are read from g_zero.
#pragma once
#include "rlk_engine.hpp"

namespace rlk {

template <int S>
__device__ __forceinline__ void fill_regs(float (&v)[S], float x) {
#pragma unroll
  for (int i = 0; i < S; ++i) v[i] = x;
}

// ------------------------------------------------------------------------------------------
// GAE: kernels/gae.py:121-180 (gae_fused_kernel), both HAS_TRUNCATIONS branches.
//   v_next = boot(t)  if t == T-1 or trunc[t] == 1,  values[t+1] otherwise
//   add = r + gamma*v_next*(1-term) - v,   mul = gamma*lambda*(1 - done)
//   done = min(term + trunc, 1) with truncations, term without;   x[T] = 0
// ------------------------------------------------------------------------------------------
template <bool TRUNC, class E = float>
struct GaeOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = false;
  static constexpr bool kBlockStats = false;  // no per-workgroup output statistics
  // long-row tiles: threads per workgroup and most 4-step segments per thread that stay
  // in registers (no spills at 1024 threads, whose cap is 128 VGPRs)
  static constexpr int kLongThreads = 1024, kLongMaxSegments = 4;
  using Halo = float;  // values[t+1]
  using Map = Affine;  // one carried value
  const E* r;
  const E* v;
  const E* term;
  const E* trunc;  // read iff TRUNC
  const E* boot;   // nullable, per boot_mode
  E* out;
  int boot_mode;
  float gamma, gl;  // gl = gamma*lambda


  template <int S>
  struct Regs {
    float r[S], v[S], te[S], tr[S], bt[S];
    float blast;
  };

  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    const int64_t o = row * (int64_t)T;
    load_seg<S, VEC>(r + o, t0, T, R.r);
    load_seg<S, VEC>(v + o, t0, T, R.v);
    load_seg<S, VEC>(term + o, t0, T, R.te);
    if constexpr (TRUNC) load_seg<S, VEC>(trunc + o, t0, T, R.tr);
    else fill_regs(R.tr, 0.f);
    boot_load<S, VEC, TRUNC>(boot, boot_mode, row, t0, T, R.bt, R.blast, r + o);
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>& R, int64_t, int t0, int T) const {
    boot_prepare<S, TRUNC>(boot_mode, t0, T, R.bt, R.blast);
  }
  template <int S>
  __device__ float export_first(const Regs<S>& R) const { return R.v[0]; }
  __device__ float halo_load(int64_t row, int t, int T) const { return to_f32(v[row * (int64_t)T + t]); }

  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, float vh, int64_t, int t0, int T, Affine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int t = t0 + i;
      const float raw = (i + 1 < S) ? R.v[i + 1] : vh;
      // kAligned: T % 4 == 0 and t0 % 4 == 0, so a segment is all in or all padding, and
      // only its last step can be T - 1 (one comparison per segment instead of one per step)
      const bool at_end = VEC == kAligned ? (i == S - 1 && t0 + S == T) : (t == T - 1);
      // `|`, not `||`: the short circuit compiled to a divergent branch on the path after
      // the loads (C2 [4096,128] 3.82 -> 3.80 us, bfloat16 3.28 -> 3.18 us on MI355X)
      const bool use_boot = at_end | (R.tr[i] == 1.f);
      const float vn = use_boot ? R.bt[i] : raw;
      const float done = TRUNC ? fminf(R.te[i] + R.tr[i], 1.f) : R.te[i];
      const float a = fmaf(gamma * vn, 1.f - R.te[i], R.r[i]) - R.v[i];
      const bool in = step_in<VEC>(t0, t, T);  // padding steps are the identity map
      m[i].add = in ? a : 0.f;
      m[i].mul = in ? gl * (1.f - done) : 1.f;
    }
  }
  __device__ const E* row_carry_src(int64_t, int) const { return nullptr; }

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>&, float, const float (&xs)[S], float, int64_t row, int t0,
                       int T) const {
    store_seg<S, VEC>(out + row * (int64_t)T, t0, T, xs, SP != 0);
  }
};

// ------------------------------------------------------------------------------------------
// GAE with returns and batch statistics: the first half of compute_gae_normalized (no
// counterpart in the reference, which has none of this; it is the "fused GAE + advantage
// normalisation" item of its ROADMAP.md:75-81).  The scan is GaeOp's; the epilogue writes
// the raw advantages A and the returns A + values, and each workgroup reduces the count,
// sum and sum of squares of its A in float64 into partials[3*blockIdx.x .. +2] (see
// block_stats in rlk_engine.hpp).  normalize_kernel then turns A into
// (A - mean) / (std + eps) in place.
// ------------------------------------------------------------------------------------------
template <bool TRUNC, class E = float>
struct GaeStatsOp : GaeOp<TRUNC, E> {
  static constexpr bool kBlockStats = true;
  E* returns;
  double* partials;
  template <int S>
  using Regs = typename GaeOp<TRUNC, E>::template Regs<S>;

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>& R, float, const float (&xs)[S], float, int64_t row, int t0,
                       int T) const {
    static_assert(VEC != kPhased, "stats() does not see the steps ahead of a phased row's tiles");
    float rt[S];
#pragma unroll
    for (int i = 0; i < S; ++i) rt[i] = xs[i] + R.v[i];
    const int64_t o = row * (int64_t)T;
    store_seg<S, VEC>(this->out + o, t0, T, xs, SP != 0);
    store_seg<S, VEC>(returns + o, t0, T, rt, SP != 0);
  }
  // every step of the row counts
  template <int S>
  __device__ void stats(const Regs<S>&, const float (&xs)[S], int t0, int T, Stats& st) const {
#pragma unroll
    for (int i = 0; i < S; ++i)
      if (t0 + i < T) st.add(xs[i]);
  }
};

// ------------------------------------------------------------------------------------------
// GAE with skipped steps: the "verl-style" masking of the reference's ROADMAP.md:131-140
// (not implemented in the reference).  Steps with mask == 0 leave the advantage and the
// next value unchanged, so credit and the continuation value pass across them (multi-turn
// rollouts whose observation tokens are not actions).  With nv = the value of the nearest
// kept step after t (boot(T-1) if there is none):
//   kept t:     v_next = boot(t) if trunc[t] == 1, nv otherwise
//               A[t] = r + gamma*v_next*(1-term) - v + gamma*lambda*(1-done)*A(after t)
//               nv <- v[t]
//   skipped t:  A[t] = A(after t) (0 if no kept step follows), nv unchanged
// With every step kept this is GaeOp.  The state {nv, A} is carried by SkipAffine maps:
// a kept step is (a, c, p, q, d) = (0, v, gamma*(1-term) [0 if truncated], gamma*lambda*
// (1-done), r - v [+ gamma*boot*(1-term) if truncated]); a skipped step is the identity.
// No halo: the next value arrives through the scan itself.
// ------------------------------------------------------------------------------------------
template <bool TRUNC, class E = float>
struct MaskedGaeOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = false;
  static constexpr bool kBlockStats = false;
  static constexpr int kLongThreads = 512, kLongMaxSegments = 4;  // five-word maps
  using Halo = NoHalo;
  using Map = SkipAffine;  // state {next value, advantage}
  const E* r;
  const E* v;
  const E* term;
  const E* trunc;  // read iff TRUNC
  const E* boot;   // nullable, per boot_mode
  const E* mask;
  E* out;
  int boot_mode;
  float gamma, gl;  // gl = gamma*lambda


  template <int S>
  struct Regs {
    float r[S], v[S], te[S], tr[S], bt[S], mk[S];
    float blast;
  };

  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    const int64_t o = row * (int64_t)T;
    load_seg<S, VEC>(r + o, t0, T, R.r);
    load_seg<S, VEC>(v + o, t0, T, R.v);
    load_seg<S, VEC>(term + o, t0, T, R.te);
    load_seg<S, VEC>(mask + o, t0, T, R.mk);
    if constexpr (TRUNC) {
      load_seg<S, VEC>(trunc + o, t0, T, R.tr);
      boot_load<S, VEC, true>(boot, boot_mode, row, t0, T, R.bt, R.blast, r + o);
    } else {
      fill_regs(R.tr, 0.f), fill_regs(R.bt, 0.f);
      R.blast = 0.f;
    }
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>& R, int64_t, int t0, int T) const {
    if constexpr (TRUNC) boot_prepare<S, true>(boot_mode, t0, T, R.bt, R.blast);
  }
  // state after the row: next value boot(T-1), advantage 0
  __device__ NvX row_state(int64_t row, int T) const {
    return NvX{to_f32(*boot_last(boot, boot_mode, row, T)), 0.f};
  }

  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, NoHalo, int64_t, int t0, int T, SkipAffine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const bool sel = TRUNC && R.tr[i] == 1.f;
      const float done = TRUNC ? fminf(R.te[i] + R.tr[i], 1.f) : R.te[i];
      const float g1 = gamma * (1.f - R.te[i]);
      const float d = sel ? fmaf(gamma * R.bt[i], 1.f - R.te[i], R.r[i]) - R.v[i] : R.r[i] - R.v[i];
      const bool kept = (step_in<VEC>(t0, t0 + i, T)) && R.mk[i] != 0.f;  // padding steps too
      m[i] = kept ? SkipAffine{0.f, R.v[i], sel ? 0.f : g1, gl * (1.f - done), d}
                  : SkipAffine::identity();
    }
  }

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>&, NoHalo, const NvX (&xs)[S], NvX, int64_t row, int t0,
                       int T) const {
    float a[S];
#pragma unroll
    for (int i = 0; i < S; ++i) a[i] = xs[i].x;
    store_seg<S, VEC>(out + row * (int64_t)T, t0, T, a, SP != 0);
  }
};

// ------------------------------------------------------------------------------------------
// Masked GAE with returns and statistics over the kept steps: the first half of
// compute_gae_normalized(..., mask=...), the masked whitening verl applies after its
// compute_gae_advantage_return.  Returns are A + values at every step; count, sum and sum of
// squares are of the kept steps only, and normalize_kernel rewrites every step's A.
// ------------------------------------------------------------------------------------------
template <bool TRUNC, class E = float>
struct MaskedGaeStatsOp : MaskedGaeOp<TRUNC, E> {
  static constexpr bool kBlockStats = true;
  E* returns;
  double* partials;
  template <int S>
  using Regs = typename MaskedGaeOp<TRUNC, E>::template Regs<S>;

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>& R, NoHalo, const NvX (&xs)[S], NvX, int64_t row, int t0,
                       int T) const {
    static_assert(VEC != kPhased, "stats() does not see the steps ahead of a phased row's tiles");
    float a[S], rt[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      a[i] = xs[i].x;
      rt[i] = xs[i].x + R.v[i];
    }
    const int64_t o = row * (int64_t)T;
    store_seg<S, VEC>(this->out + o, t0, T, a, SP != 0);
    store_seg<S, VEC>(returns + o, t0, T, rt, SP != 0);
  }
  template <int S>
  __device__ void stats(const Regs<S>& R, const NvX (&xs)[S], int t0, int T, Stats& st) const {
#pragma unroll
    for (int i = 0; i < S; ++i)
      if (t0 + i < T && R.mk[i] != 0.f) st.add(xs[i].x);
  }
};

// ------------------------------------------------------------------------------------------
// V-trace: kernels/vtrace_fused.py:90-196 (vtrace_fused_kernel).
//   rho = min(exp(lpt - lpb), rho_bar),  c = min(exp(lpt - lpb), c_bar)
//   truncations:  v_next = values[t+1]*[t < T-1 and trunc == 0] + boot(t)   (additive)
//   otherwise:    v_next = boot(T-1) at t = T-1, values[t+1] elsewhere
//   add = rho*(r + gamma*v_next*(1-term) - v),  mul = gamma*c*(1-done),  x[T] = 0
//   targets = x + v;  next target by the same rule as v_next with targets for values
//   advantages = rho*(r + gamma*next_target*(1-term) - v)
// The reference passes targets[t+1] through global memory (store, barrier, reload,
// vtrace_fused.py:149-152); here it is the neighbouring register or lane.
// ------------------------------------------------------------------------------------------
template <bool TRUNC, class E = float>
struct VtraceOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = false;
  static constexpr bool kBlockStats = false;  // no per-workgroup output statistics
  static constexpr int kLongThreads = 1024, kLongMaxSegments = 2;
  using Halo = float;  // values[t+1]
  using Map = Affine;  // one carried value
  const E* lpt;
  const E* lpb;
  const E* v;
  const E* r;
  const E* term;
  const E* trunc;  // read iff TRUNC
  const E* boot;   // nullable, per boot_mode
  E* targets;
  E* adv;
  int boot_mode;
  float gamma, rho_bar, c_bar;


  template <int S>
  struct Regs {
    float rho[S], c[S], v[S], r[S], te[S], tr[S], bt[S];  // rho, c: log-probs until prepare()
    float blast;
  };

  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    const int64_t o = row * (int64_t)T;
    load_seg<S, VEC>(lpt + o, t0, T, R.rho);
    load_seg<S, VEC>(lpb + o, t0, T, R.c);
    load_seg<S, VEC>(v + o, t0, T, R.v);
    load_seg<S, VEC>(r + o, t0, T, R.r);
    load_seg<S, VEC>(term + o, t0, T, R.te);
    if constexpr (TRUNC) load_seg<S, VEC>(trunc + o, t0, T, R.tr);
    else fill_regs(R.tr, 0.f);
    boot_load<S, VEC, TRUNC>(boot, boot_mode, row, t0, T, R.bt, R.blast, r + o);
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>& R, int64_t, int t0, int T) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      // hardware exp2 after a multiply by log2(e): a few ulp, far inside the parity
      // tolerance, and 2% off the [4096,128] call against the range-reduced expf
      const float ratio = __expf(R.rho[i] - R.c[i]);
      R.rho[i] = fminf(ratio, rho_bar);
      R.c[i] = fminf(ratio, c_bar);
    }
    boot_prepare<S, TRUNC>(boot_mode, t0, T, R.bt, R.blast);
  }
  template <int S>
  __device__ float export_first(const Regs<S>& R) const { return R.v[0]; }
  __device__ float halo_load(int64_t row, int t, int T) const { return to_f32(v[row * (int64_t)T + t]); }

  // continuation value at step t from the raw next-step value (values or targets)
  // last: t == T - 1
  __device__ __forceinline__ float next_value(float raw, float tr, float bt, bool last) const {
    if constexpr (TRUNC) return ((!last && tr == 0.f) ? raw : 0.f) + bt;
    return last ? bt : raw;
  }

  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, float vh, int64_t, int t0, int T, Affine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int t = t0 + i;
      const bool last = VEC == kAligned ? (i == S - 1 && t0 + S == T) : (t == T - 1);
      const float vn = next_value((i + 1 < S) ? R.v[i + 1] : vh, R.tr[i], R.bt[i], last);
      const float done = TRUNC ? fminf(R.te[i] + R.tr[i], 1.f) : R.te[i];
      const float a = R.rho[i] * (fmaf(gamma * vn, 1.f - R.te[i], R.r[i]) - R.v[i]);
      const bool in = step_in<VEC>(t0, t, T);
      m[i].add = in ? a : 0.f;
      m[i].mul = in ? gamma * R.c[i] * (1.f - done) : 1.f;
    }
  }
  __device__ const E* row_carry_src(int64_t, int) const { return nullptr; }

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>& R, float vh, const float (&xs)[S], float x_next, int64_t row,
                       int t0, int T) const {
    float tg[S], ad[S];
#pragma unroll
    for (int i = 0; i < S; ++i) tg[i] = xs[i] + R.v[i];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const float raw = (i + 1 < S) ? tg[i + 1] : x_next + vh;
      const bool last = VEC == kAligned ? (i == S - 1 && t0 + S == T) : (t0 + i == T - 1);
      const float nt = next_value(raw, R.tr[i], R.bt[i], last);
      ad[i] = R.rho[i] * (fmaf(gamma * nt, 1.f - R.te[i], R.r[i]) - R.v[i]);
    }
    const int64_t o = row * (int64_t)T;
    store_seg<S, VEC>(targets + o, t0, T, tg, SP != 0);
    store_seg<S, VEC>(adv + o, t0, T, ad, SP != 0);
  }
};

// ------------------------------------------------------------------------------------------
// Retrace(lambda): kernels/retrace_fused.py:116-201 (retrace_fused_kernel).
//   E_pi[Q'] = sum_a pi[t,a]*nq[t,a];  pi_a = pi[t, a_t] (0 if a_t outside [0, A))
//   rho = min(pi_a/mu, rho_bar),  c = lambda*min(pi_a/mu, c_bar)
//   add = r + gamma*E_pi[Q']*(1-term) - q,  mul = gamma*c[t+1]*(1-done),  c[T] = 0
//   Q_ret = x + q;  advantages = rho*(r + gamma*Q_ret[t+1]*(1-term) - q),  Q_ret[T] = 0
// NA > 0: compile-time action count (vector loads of the [S, A] block); NA == 0: runtime A.
// ------------------------------------------------------------------------------------------
template <int NA, bool TRUNC, class E = float>
struct RetraceOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = false;
  static constexpr bool kBlockStats = false;  // no per-workgroup output statistics
  static constexpr int kLongThreads = 512, kLongMaxSegments = 2;  // 256 VGPRs: the A-wide rows
  using Halo = Halo2;  // {c[t+1], q[t+1]}
  using Map = Affine;  // one carried value
  const E* pi;     // [E, T, A]
  const E* mu;     // [E, T]
  const E* q;
  const E* nq;     // [E, T, A]
  const int64_t* act;  // [E, T]
  const E* r;
  const E* term;
  const E* trunc;  // read iff TRUNC
  E* targets;
  E* adv;
  int A;
  float gamma, lambda, c_bar, rho_bar;


  template <int S>
  struct Regs {
    float q[S], r[S], te[S], tr[S], rho[S], c[S], enq[S];
  };

  // (rho, c, E_pi[Q']) at one step from its action row
  template <class P>
  __device__ __forceinline__ void step_terms(const P* p, const P* n, int64_t a_t, float m,
                                             float& rho, float& c, float& enq) const {
    float e = 0.f, pa = 0.f;
    const int na = NA > 0 ? NA : A;
    for (int a = 0; a < na; ++a) {
      const float pv = to_f32(p[a]);
      e = fmaf(pv, to_f32(n[a]), e);
      pa = (a == a_t) ? pv : pa;
    }
    const float ratio = pa / m;
    rho = fminf(ratio, rho_bar);
    c = lambda * fminf(ratio, c_bar);
    enq = e;
  }

  // Unlike the other ops, the [S, A] action blocks are reduced to (rho, c, E_pi[Q']) here,
  // at load time, so a segment holds three values per step instead of 2A.
  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    static_assert(VEC != kPhased, "the [E, T, A] arrays have no common row phase");
    const int64_t o = row * (int64_t)T;
    float m[S];
    load_seg<S, VEC>(q + o, t0, T, R.q);
    load_seg<S, VEC>(r + o, t0, T, R.r);
    load_seg<S, VEC>(term + o, t0, T, R.te);
    if constexpr (TRUNC) load_seg<S, VEC>(trunc + o, t0, T, R.tr);
    else fill_regs(R.tr, 0.f);
    load_seg<S, VEC>(mu + o, t0, T, m);
    int64_t at[S];
    if constexpr (VEC == kAligned) {
      // a quad of actions is 32 contiguous bytes, 16-byte aligned (the launch checks the
      // pointer): two 16-byte loads instead of four 8-byte ones (Retrace [4096,128]
      // 6.60 -> 6.53 us on MI355X); a quad beyond T reads the row's last quad
      typedef long long i64x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int qd = 0; qd < S / 4; ++qd) {
        const int t = t0 + 4 * qd;
        const i64x2* pq = reinterpret_cast<const i64x2*>(act + o + (t < T ? t : T - 4));
        const i64x2 u = pq[0], w = pq[1];
        at[4 * qd] = u.x, at[4 * qd + 1] = u.y, at[4 * qd + 2] = w.x, at[4 * qd + 3] = w.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < S; ++i) at[i] = act[o + clamp_step(t0 + i, T)];
    }
    if constexpr (NA > 0 && VEC == kAligned && (S * NA) % 4 == 0 && S * NA <= 16) {
      // the [S, NA] blocks are contiguous and 16-byte aligned; a quad beyond T reads the
      // row's first quad instead.  (Larger blocks take the per-step path below: two tiles
      // of them would not fit the register file.)
      float pb[S * NA], nb[S * NA];
      const E* pp = pi + (o + t0) * NA;
      const E* np = nq + (o + t0) * NA;
#pragma unroll
      for (int qd = 0; qd < S * NA / 4; ++qd) {
        const bool in = t0 + (4 * qd) / NA < T;
        const float4 a4 = load_quad(in ? pp + 4 * qd : pi + o * NA);
        const float4 b4 = load_quad(in ? np + 4 * qd : nq + o * NA);
        pb[4 * qd] = a4.x, pb[4 * qd + 1] = a4.y, pb[4 * qd + 2] = a4.z, pb[4 * qd + 3] = a4.w;
        nb[4 * qd] = b4.x, nb[4 * qd + 1] = b4.y, nb[4 * qd + 2] = b4.z, nb[4 * qd + 3] = b4.w;
      }
#pragma unroll
      for (int i = 0; i < S; ++i) step_terms(pb + i * NA, nb + i * NA, at[i], m[i], R.rho[i], R.c[i], R.enq[i]);
    } else {
      const int na = NA > 0 ? NA : A;
#pragma unroll
      for (int i = 0; i < S; ++i) {
        const int64_t base = (o + clamp_step(t0 + i, T)) * na;
        step_terms(pi + base, nq + base, at[i], m[i], R.rho[i], R.c[i], R.enq[i]);
      }
    }
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>&, int64_t, int, int) const {}
  template <int S>
  __device__ Halo2 export_first(const Regs<S>& R) const { return Halo2{R.c[0], R.q[0]}; }
  __device__ Halo2 halo_load(int64_t row, int t, int T) const {
    const int64_t i = row * (int64_t)T + t;
    const int na = NA > 0 ? NA : A;
    float rho, c, enq;
    step_terms(pi + i * na, nq + i * na, act[i], to_f32(mu[i]), rho, c, enq);
    return Halo2{c, to_f32(q[i])};
  }

  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, Halo2 h, int64_t, int t0, int T, Affine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int t = t0 + i;
      const bool before_end = VEC == kAligned ? (i < S - 1 ? t0 < T : t0 + S < T) : (t < T - 1);
      const float c_next = before_end ? ((i + 1 < S) ? R.c[i + 1] : h.a) : 0.f;
      const float done = fminf(R.te[i] + R.tr[i], 1.f);
      const float a = fmaf(gamma * R.enq[i], 1.f - R.te[i], R.r[i]) - R.q[i];
      const bool in = step_in<VEC>(t0, t, T);  // vector segments are all-in or all-out
      m[i].add = in ? a : 0.f;
      m[i].mul = in ? gamma * c_next * (1.f - done) : 1.f;
    }
  }
  __device__ const E* row_carry_src(int64_t, int) const { return nullptr; }

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>& R, Halo2 h, const float (&xs)[S], float x_next, int64_t row,
                       int t0, int T) const {
    float tg[S], ad[S];
#pragma unroll
    for (int i = 0; i < S; ++i) tg[i] = xs[i] + R.q[i];
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int t = t0 + i;
      const bool before_end = VEC == kAligned ? (i < S - 1 ? t0 < T : t0 + S < T) : (t < T - 1);
      const float nxt = before_end ? ((i + 1 < S) ? tg[i + 1] : x_next + h.b) : 0.f;
      ad[i] = R.rho[i] * (fmaf(gamma * nxt, 1.f - R.te[i], R.r[i]) - R.q[i]);
    }
    const int64_t o = row * (int64_t)T;
    store_seg<S, VEC>(targets + o, t0, T, tg, SP != 0);
    store_seg<S, VEC>(adv + o, t0, T, ad, SP != 0);
  }
};

// ------------------------------------------------------------------------------------------
// TD(lambda) returns: kernels/lambda_returns_fused.py:54-89.
//   nd = 1 - done;  add = r + gamma*(1-lambda)*nd*nv + gamma*trunc*boot(t);  mul = gamma*lambda*nd
//   x[T] = boot(T-1)
// Discounted returns: kernels/discounted_returns_fused.py:50-82 -- the same with
//   add = r + gamma*trunc*boot(t),  mul = gamma*nd  (NV = false: no next values).
// ------------------------------------------------------------------------------------------
template <bool NV, bool TRUNC, class E = float>
struct ReturnsOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = false;
  static constexpr bool kBlockStats = false;  // no per-workgroup output statistics
  // plain discounted returns (two arrays read): 512-thread tiles of up to 8 segments per
  // thread measured 3% faster at [16,131072] than 1024 threads of 2 (same tile size)
  static constexpr int kLongThreads = (NV || TRUNC) ? 1024 : 512;
  static constexpr int kLongMaxSegments = (NV || TRUNC) ? 4 : 8;
  using Halo = NoHalo;
  using Map = Affine;  // one carried value
  const E* r;
  const E* nv;     // read iff NV
  const E* term;
  const E* trunc;  // read iff TRUNC
  const E* boot;   // nullable, per boot_mode
  E* out;
  int boot_mode;
  float gamma, g1l, gl;  // gamma, gamma*(1-lambda), gamma*lambda (discounted: gl = gamma)


  template <int S>
  struct Regs {
    float r[S], nv[S], te[S], tr[S], bt[S];
    float blast;
  };

  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    const int64_t o = row * (int64_t)T;
    load_seg<S, VEC>(r + o, t0, T, R.r);
    if constexpr (NV) load_seg<S, VEC>(nv + o, t0, T, R.nv);
    else fill_regs(R.nv, 0.f);
    load_seg<S, VEC>(term + o, t0, T, R.te);
    if constexpr (TRUNC) {
      load_seg<S, VEC>(trunc + o, t0, T, R.tr);
      boot_load<S, VEC, true>(boot, boot_mode, row, t0, T, R.bt, R.blast, r + o);
    } else {
      fill_regs(R.tr, 0.f), fill_regs(R.bt, 0.f);
      R.blast = 0.f;
    }
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>& R, int64_t, int t0, int T) const {
    if constexpr (TRUNC) boot_prepare<S, true>(boot_mode, t0, T, R.bt, R.blast);
  }

  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, NoHalo, int64_t, int t0, int T, Affine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int t = t0 + i;
      const float nd = 1.f - (TRUNC ? fminf(R.te[i] + R.tr[i], 1.f) : R.te[i]);
      float a = NV ? fmaf(g1l * nd, R.nv[i], R.r[i]) : R.r[i];
      if constexpr (TRUNC) a = fmaf(gamma * R.tr[i], R.bt[i], a);
      const bool in = step_in<VEC>(t0, t, T);  // vector segments are all-in or all-out
      m[i].add = in ? a : 0.f;
      m[i].mul = in ? gl * nd : 1.f;
    }
  }
  __device__ const E* row_carry_src(int64_t row, int T) const {
    return boot_mode == kBootNone ? nullptr : boot_last(boot, boot_mode, row, T);
  }

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>&, NoHalo, const float (&xs)[S], float, int64_t row, int t0,
                       int T) const {
    store_seg<S, VEC>(out + row * (int64_t)T, t0, T, xs, SP != 0);
  }
};

// ------------------------------------------------------------------------------------------
// Forward scans gated on done.
//   eligibility traces (kernels/eligibility_traces_fused.py:67-84):
//       mul = gamma*lambda*(1 - done[t-1]), done[-1] = 0, add = g, x[-1] = seed
//   episodic prefix sum (kernels/prefix_sum_fused.py:63-84):
//       ends_at:   mul = 1 - done[t-1];  starts_at: mul = 1 - done[t];  add = x, x[-1] = seed
// (decay = gamma*lambda for traces, 1 for the prefix sum)
// ------------------------------------------------------------------------------------------
template <class E = float>
struct DoneGatedForwardOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = true;
  static constexpr bool kBlockStats = false;
  static constexpr int kLongThreads = 1024, kLongMaxSegments = 8;
  using Halo = float;  // done[t-1]
  using Map = Affine;  // one carried value
  const E* x;
  const E* dones;
  const E* seed;  // nullable
  E* out;
  float decay;
  int ends_at;


  template <int S>
  struct Regs {
    float x[S], d[S];
  };

  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    const int64_t o = row * (int64_t)T;
    load_seg<S, VEC>(x + o, t0, T, R.x);
    load_seg<S, VEC>(dones + o, t0, T, R.d);
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>&, int64_t, int, int) const {}
  template <int S>
  __device__ float export_last(const Regs<S>& R) const { return R.d[S - 1]; }
  __device__ float halo_load(int64_t row, int t, int T) const { return to_f32(dones[row * (int64_t)T + t]); }

  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, float dh, int64_t, int t0, int T, Affine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int t = t0 + i;
      float gate;
      if (ends_at) {
        // kPhased segments can hold step 0 past their first position, after steps of the
        // row before (done[-1] = 0 all the same)
        if constexpr (VEC == kPhased) gate = t == 0 ? 0.f : (i > 0 ? R.d[i - 1] : dh);
        else gate = (i > 0) ? R.d[i - 1] : (t == 0 ? 0.f : dh);
      } else {
        gate = R.d[i];
      }
      const bool in = step_in<VEC>(t0, t, T);  // vector segments are all-in or all-out
      m[i].mul = in ? decay * (1.f - gate) : 1.f;
      m[i].add = in ? R.x[i] : 0.f;
    }
  }
  __device__ const E* row_carry_src(int64_t row, int) const { return seed ? seed + row : nullptr; }

  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>&, float, const float (&xs)[S], float, int64_t row, int t0,
                       int T) const {
    store_seg<S, VEC>(out + row * (int64_t)T, t0, T, xs, SP != 0);
  }
};

// ------------------------------------------------------------------------------------------
// Generic affine scans (ops/_scan.py:69-213, kernels/scan.py:39-138):
//   backward A[t] = u[t] + v[t]*A[t+1], A[T] = carry;  forward e[t] = u[t] + v[t]*e[t-1], e[-1] = carry
// ------------------------------------------------------------------------------------------
template <bool FWD, class E = float>
struct AffineScanOp {
  using Elem = E;  // storage type of the float arrays
  static constexpr bool kForward = FWD;
  static constexpr bool kBlockStats = false;
  static constexpr int kLongThreads = 1024, kLongMaxSegments = 8;
  using Halo = NoHalo;
  using Map = Affine;  // one carried value
  const E* u;
  const E* v;
  const E* carry;  // nullable, [E]
  E* out;


  template <int S>
  struct Regs {
    float u[S], v[S];
  };
  template <int S, int VEC>
  __device__ void load(int64_t row, int t0, int T, Regs<S>& R) const {
    const int64_t o = row * (int64_t)T;
    load_seg<S, VEC>(u + o, t0, T, R.u);
    load_seg<S, VEC>(v + o, t0, T, R.v);
  }
  template <int S, int VEC>
  __device__ void prepare(Regs<S>&, int64_t, int, int) const {}
  template <int S, int VEC = kElementAligned>
  __device__ void coef(const Regs<S>& R, NoHalo, int64_t, int t0, int T, Affine (&m)[S]) const {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const bool in = step_in<VEC>(t0, t0 + i, T);
      m[i].mul = in ? R.v[i] : 1.f;
      m[i].add = in ? R.u[i] : 0.f;
    }
  }
  __device__ const E* row_carry_src(int64_t row, int) const { return carry ? carry + row : nullptr; }
  template <int S, int VEC, int SP = 0>
  __device__ void emit(const Regs<S>&, NoHalo, const float (&xs)[S], float, int64_t row, int t0,
                       int T) const {
    store_seg<S, VEC>(out + row * (int64_t)T, t0, T, xs, SP != 0);
  }
};

}  // namespace rlk
