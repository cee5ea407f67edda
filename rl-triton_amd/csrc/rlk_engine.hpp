// rlk_engine.hpp -- the scan engine shared by every rl_triton estimator on gfx950.
//
// Every estimator is one done-masked linear recurrence over a row of T steps,
//     backward:  x[t] = add[t] + mul[t] * x[t+1],   x[T]  = carry   (GAE, V-trace, ...)
//     forward:   x[t] = add[t] + mul[t] * x[t-1],   x[-1] = carry   (traces, prefix sum)
// evaluated as a scan over affine maps m(x) = add + mul * x.  Composition:
//     (m1 o m2)(x) = m1.add + m1.mul * m2.add  +  (m1.mul * m2.mul) * x.
//
// Work decomposition (rows are contiguous, row-major [E, T]; float32 arithmetic):
//   * a thread owns S consecutive steps of one row ("segment") and keeps its
//     inputs in registers; it folds them into one affine map serially;
//   * L threads (L = 2^k) form a row tile of L*S steps; their maps are combined by a
//     wavefront shuffle scan (width min(L, 64)) and, when L > 64, through LDS;
//   * short rows: a workgroup of NT threads holds NT/L whole rows, no inter-workgroup
//     traffic;
//   * long rows: a row is split into tiles, one per workgroup (by block index), chained
//     by a decoupled look-back over per-tile status words in a caller-provided workspace;
//     a workgroup that would wait on a predecessor not yet started computes that
//     predecessor's map itself.
//
// An estimator ("Op") supplies:
//   Regs                      per-thread registers for S steps
//   load(row, t0, T, R)       issue the segment's loads, clamped into the row
//   prepare(R, row, t0, T)    everything derived from the loaded values (exp, ratios,
//                             bootstrap selection)
//   Halo / export / halo_load the one-step neighbour data the producer needs (values[t+1]
//                             for GAE, done[t-1] for forward traces), passed lane to lane
//                             and read from global memory at wave/tile edges
//   coef(...)                 per-step (add, mul) with truncation/bootstrap folded in;
//                             padding steps (t >= T) are the identity map
//   row_carry_src(row, T)     address of x[T] (backward) or x[-1] (forward), or nullptr (0)
//   emit(...)                 outputs from the scanned x (and x one step further)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace rlk {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------
// Scan elements ("maps").  An op's steps are maps of one of two kinds; a kind provides its
// carried State, identity, apply, compose (outer o inner: inner first) and the number of
// look-back status words its aggregate and its state take.
//
//   Affine      x' = mul*x + add                              (State: x)
//   SkipAffine  nv' = a*nv + c,  x' = p*nv + q*x + d          (State: {nv, x})
//
// SkipAffine carries a second value beside x, a "next value" nv that skipped steps pass
// through unchanged; the steps of the masked GAE mode are of this kind (a step either
// replaces nv, a = 0, or keeps it, a = 1, so a stays exactly 0 or 1 under composition).
// ---------------------------------------------------------------------------------------
struct Affine {
  using State = float;
  static constexpr int kWords = 2;       // status words of an aggregate
  static constexpr int kStateWords = 1;  // status words of an inclusive value
  float mul;
  float add;
  __device__ static Affine identity() { return Affine{1.f, 0.f}; }
  __device__ float apply(float x) const { return fmaf(mul, x, add); }
  __device__ bool constant() const { return mul == 0.f; }  // apply() ignores its argument
  __device__ float word(int i) const { return i == 0 ? mul : add; }
  __device__ static Affine from_words(const float* w) { return Affine{w[0], w[1]}; }
};

__device__ __forceinline__ Affine compose(Affine outer, Affine inner) {
  // outer(inner(x))
  return Affine{outer.mul * inner.mul, fmaf(outer.mul, inner.add, outer.add)};
}

struct NvX {
  float nv;  // the carried next value
  float x;   // the scanned value
};

struct SkipAffine {
  using State = NvX;
  static constexpr int kWords = 5;
  static constexpr int kStateWords = 2;
  float a, c, p, q, d;
  __device__ static SkipAffine identity() { return SkipAffine{1.f, 0.f, 0.f, 1.f, 0.f}; }
  __device__ NvX apply(NvX s) const { return NvX{fmaf(a, s.nv, c), fmaf(p, s.nv, fmaf(q, s.x, d))}; }
  __device__ bool constant() const { return a == 0.f && p == 0.f && q == 0.f; }
  __device__ float word(int i) const { return i == 0 ? a : i == 1 ? c : i == 2 ? p : i == 3 ? q : d; }
  __device__ static SkipAffine from_words(const float* w) { return SkipAffine{w[0], w[1], w[2], w[3], w[4]}; }
};

__device__ __forceinline__ SkipAffine compose(SkipAffine o, SkipAffine i) {
  return SkipAffine{o.a * i.a, fmaf(o.a, i.c, o.c), fmaf(o.p, i.a, o.q * i.p), o.q * i.q,
                    fmaf(o.p, i.c, fmaf(o.q, i.d, o.d))};
}

// States as status words (an inclusive value): x first, so word 0 names the kind.
__device__ __forceinline__ float state_word(float x, int) { return x; }
__device__ __forceinline__ float state_word(NvX s, int i) { return i == 0 ? s.x : s.nv; }
template <class S>
__device__ __forceinline__ S state_from_words(const float* w);
template <>
__device__ __forceinline__ float state_from_words<float>(const float* w) { return w[0]; }
template <>
__device__ __forceinline__ NvX state_from_words<NvX>(const float* w) { return NvX{w[1], w[0]}; }

struct NoHalo {};

// ---------------------------------------------------------------------------------------
// Storage types.  Every array of a call is float32 or every one is bfloat16 (the upper half
// of an IEEE float32, here `bf16`); the arithmetic is float32 either way.  A bfloat16 load
// widens exactly; a store rounds to nearest even and turns any NaN into 0x7fc0, which is
// torch's float -> bfloat16 conversion, so a bfloat16 result is the float32 result as
// torch would round it.
// ---------------------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return __uint_as_float((uint32_t)x.bits << 16); }

template <class E>
__device__ __forceinline__ E from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
// gfx950's v_cvt_pk_bf16_f32 (what the compiler emits for a float -> __bf16 conversion)
// rounds to nearest even exactly as the integer form (u + 0x7fff + lsb) >> 16 does, for
// every non-NaN float, denormals and infinities included: the two agree on all 2^32 bit
// patterns on MI355X.  It keeps a NaN's sign and payload, so NaN is mapped to 0x7fc0
// after it.  Two values convert in one instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
  if (lo != lo) w = (w & 0xffff0000u) | 0x7fc0u;
  if (hi != hi) w = (w & 0x0000ffffu) | 0x7fc00000u;
  return w;
}
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) {
  return bf16{(uint16_t)pack_bf16x2(x, 0.f)};
}

// ---------------------------------------------------------------------------------------
// Streaming accesses.  Every input element is read once and every output written once.
// Where one wave instruction covers whole cache lines (a quad per lane, lanes contiguous),
// the row data goes through non-temporal loads and stores (NT = true, the `nt` cache
// policy): they do not displace other lines in L2, and the stores leave no dirty L2 lines
// for the end-of-kernel write-back.  On MI355X this took 6-10% off those configurations
// (V-trace [4096,128] 4.65 -> 4.35 us, V-trace [16,131072] 15.9 -> 14.2 us).  Where a line
// is shared by several instructions (8-step segments, Retrace's action blocks) it must stay
// in cache between them, so those use ordinary accesses: with `nt` there, Retrace
// [256,2048] went from 7.9 to 10.2 us.  Look-back status words and per-row values use
// ordinary accesses too.
// ---------------------------------------------------------------------------------------
typedef float nt_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t nt_u2 __attribute__((ext_vector_type(2)));

// Four consecutive elements (16 bytes of float32, 8 of bfloat16) as float32.
template <bool NT = false>
__device__ __forceinline__ float4 load_quad(const float* p) {
  if constexpr (NT) {
    const nt_f4 w = __builtin_nontemporal_load(reinterpret_cast<const nt_f4*>(p));
    return make_float4(w.x, w.y, w.z, w.w);
  } else {
    return *reinterpret_cast<const float4*>(p);
  }
}
template <bool NT = false>
__device__ __forceinline__ float4 load_quad(const bf16* p) {
  nt_u2 w;
  if constexpr (NT) w = __builtin_nontemporal_load(reinterpret_cast<const nt_u2*>(p));
  else w = *reinterpret_cast<const nt_u2*>(p);
  return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                     __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
}
template <bool NT = false>
__device__ __forceinline__ void store_quad(float* p, float4 v) {
  const nt_f4 w = {v.x, v.y, v.z, v.w};
  if constexpr (NT) __builtin_nontemporal_store(w, reinterpret_cast<nt_f4*>(p));
  else *reinterpret_cast<nt_f4*>(p) = w;
}
template <bool NT = false>
__device__ __forceinline__ void store_quad(bf16* p, float4 v) {
  const nt_u2 w = {pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
  if constexpr (NT) __builtin_nontemporal_store(w, reinterpret_cast<nt_u2*>(p));
  else *reinterpret_cast<nt_u2*>(p) = w;
}
// The same stores with the sc1 cache-policy bit (write-through towards memory) instead of
// nt.  Which of the two a launch uses is the launcher's choice, by call shape: the kernels'
// SP template argument (0 non-temporal, 1 write-through), passed on to the op's emit, so
// that each kernel instance holds the stores of one policy only (a runtime branch around
// two copies of the output loop made kernels up to 3.5% slower on MI355X).
// A VALU write to the data registers of a store of more than 8 bytes must come at least 2
// wait states after it on gfx950, or the store may send the new values; the compiler pads
// its own stores for this but not inline assembly, so the 16-byte form carries its own
// s_nop 1 (2 wait states).
__device__ __forceinline__ void store_quad_wt(float* p, float4 v) {
  const nt_f4 w = {v.x, v.y, v.z, v.w};
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(w) : "memory");
}
__device__ __forceinline__ void store_quad_wt(bf16* p, float4 v) {
  const nt_u2 w = {pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
  asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(w) : "memory");
}
// Four consecutive elements at any element boundary: one 16-byte (bfloat16: 8-byte) access
// that need not be aligned to its size.  gfx950 runs compute in unaligned access mode, and
// the compiler emits a single dwordx4 (dwordx2) access for these element-aligned vector
// types; an unaligned quad costs ~6% more than an aligned one on a streaming pattern,
// against ~45% for four single-element accesses.
typedef float ua_f4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t ua_u2 __attribute__((ext_vector_type(2), aligned(2)));
__device__ __forceinline__ float4 load_quad_ua(const float* p) {
  const ua_f4 w = *reinterpret_cast<const ua_f4*>(p);
  return make_float4(w.x, w.y, w.z, w.w);
}
__device__ __forceinline__ float4 load_quad_ua(const bf16* p) {
  const ua_u2 w = *reinterpret_cast<const ua_u2*>(p);
  return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                     __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
}
__device__ __forceinline__ void store_quad_ua(float* p, float4 v) {
  *reinterpret_cast<ua_f4*>(p) = ua_f4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void store_quad_ua(bf16* p, float4 v) {
  *reinterpret_cast<ua_u2*>(p) = ua_u2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
}
// Element k of a quad, k >= 3 giving the last one.
__device__ __forceinline__ float quad_elem(float4 f, int k) {
  return k <= 0 ? f.x : k == 1 ? f.y : k == 2 ? f.z : f.w;
}

// One element, non-temporal (lanes contiguous).
__device__ __forceinline__ float load_one_nt(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float load_one_nt(const bf16* p) {
  return to_f32(bf16{__builtin_nontemporal_load(&p->bits)});
}
__device__ __forceinline__ void store_one_nt(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_one_nt(bf16* p, float v) {
  __builtin_nontemporal_store(from_f32<bf16>(v).bits, &p->bits);
}

// ---------------------------------------------------------------------------------------
// Segment loads / stores, in one of three access modes (the VEC template argument):
//
// kAligned (1): T % 4 == 0 and every base pointer aligned to four elements (16 bytes for
// float32, 8 for bfloat16), so a segment start t0 (a multiple of 4) is aligned and each
// quad is all-in or all-out.  A 4-step segment is one quad per lane with the lanes of a
// wave on consecutive quads (every kernel lays segments out that way), so it streams
// non-temporally.
//
// kPhased (2, long rows only): T % 4 != 0, and every [E, T] array of the call starts at the
// same element phase (address / element size, mod 4).  Each row's segments are shifted to
// its own four-element boundary (t0 = 4j + shift, shift = -ph backward, (4 - ph) % 4
// forward, ph the row's phase 0..3; see chain_kernel), so every quad is one aligned access
// again.  A row's first quad reaches up to 3 steps before step 0, its last up to 3 beyond
// step T - 1: both stay inside the aligned 16-byte (bfloat16: 8-byte) block that holds the
// row's first (last) element, so they never leave a mapped page, and their foreign steps
// are masked (step_in) and not stored.  Stores of those two quads go element by element.
//
// kElementAligned (0): every other case.  A quad wholly inside the row is still one access
// (load_quad_ua); the row's partial last quad is read as the row's last four elements and
// shifted into place.  Rows shorter than four steps use segments of one step (S = 1),
// element by element.
//
// Loads are unconditional: a step beyond T reads the row's last element (kAligned,
// kPhased: its last quad).  Padding steps are masked to the identity map in coef() and are
// not stored, so their register contents never matter.
// ---------------------------------------------------------------------------------------
constexpr int kElementAligned = 0, kAligned = 1, kPhased = 2;

// Step t (of a segment starting at t0) lies inside the row [0, T).  kAligned segments are
// all-in or all-out; only kPhased steps can lie before the row.
template <int VEC>
__device__ __forceinline__ bool step_in(int t0, int t, int T) {
  if constexpr (VEC == kAligned) return t0 < T;
  else if constexpr (VEC == kPhased) return (unsigned)t < (unsigned)T;
  else return t < T;
}
__device__ __forceinline__ int clamp_step(int t, int T) { return t < 0 ? 0 : (t < T ? t : T - 1); }

template <int S, int VEC, class E>
__device__ __forceinline__ void load_seg(const E* __restrict__ p, int t0, int T, float (&v)[S]) {
  static_assert(VEC == kElementAligned || S % 4 == 0, "vector segments hold whole quads");
  if constexpr (VEC == kPhased) {
    // t0 + ph is a multiple of 4 (ph the row's phase): every quad start is aligned.  Quads
    // beyond the row read the one that holds step T - 1 (tq, at the same phase).
    const int tq = (T - 1) - ((T - 1 - t0) & 3);
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      const float4 f = load_quad<S == 4>(p + (t < T ? t : tq));
      v[4 * q + 0] = f.x;
      v[4 * q + 1] = f.y;
      v[4 * q + 2] = f.z;
      v[4 * q + 3] = f.w;
    }
  } else if constexpr (VEC == kAligned) {
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      const float4 f = load_quad<S == 4>(p + (t < T ? t : T - 4));
      v[4 * q + 0] = f.x;
      v[4 * q + 1] = f.y;
      v[4 * q + 2] = f.z;
      v[4 * q + 3] = f.w;
    }
  } else if constexpr (S % 4 == 0) {
    // element-aligned quads; the launch guarantees T >= 4.  No branch around the load: a
    // join after it would make the compiler wait for the load there, and the loads of a
    // segment's arrays would no longer overlap.  Segments start at multiples of four, so
    // the one partial quad of a row (T % 4 != 0) starts at 4 * (T / 4); it is read as the
    // row's last four elements, and its steps sit c = 4 - T % 4 places further in: one
    // shift for the whole row.  Padding quads beyond it read the same four elements (their
    // values never matter).  Per quad only a lane mask (inside the row or not) stays live
    // until the load returns, not a per-lane shift.
    const int c = 4 - (T & 3);
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      const bool edge = t + 4 > T;  // the partial quad, or padding
      const float4 f = load_quad_ua(p + (edge ? T - 4 : t));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * q + i] = edge ? quad_elem(f, i + c) : quad_elem(f, i);
    }
  } else {
    // segments of 1-3 steps (rows shorter than four steps)
#pragma unroll
    for (int i = 0; i < S; ++i) v[i] = to_f32(p[t0 + i < T ? t0 + i : T - 1]);
  }
}

// Steps beyond T are not stored.  wt: vector quads take store_quad_wt.
template <int S, int VEC, class E>
__device__ __forceinline__ void store_seg(E* __restrict__ p, int t0, int T, const float (&v)[S],
                                          bool wt = false) {
  static_assert(VEC == kElementAligned || S % 4 == 0, "vector segments hold whole quads");
  if constexpr (VEC == kPhased) {
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      if (t >= 0 && t + 4 <= T) {
        const float4 f = make_float4(v[4 * q + 0], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        if (wt) store_quad_wt(p + t, f);
        else store_quad<S == 4>(p + t, f);
      } else if (t < T) {  // the row's first or last quad: its own steps only
        // Not step_in's test: written as that, the compiler kept coef's per-step masks (one
        // per step of every segment) live up to here, and the 1024-thread instances spilled
        // 24-176 B per lane.
        const int lo = -t, hi = T - t;  // element i of the quad is step t + i
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (i >= lo && i < hi) p[t + i] = from_f32<E>(v[4 * q + i]);
      }
    }
  } else if constexpr (VEC == kAligned) {
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      const float4 f = make_float4(v[4 * q + 0], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
      if (t < T) {
        if (wt) store_quad_wt(p + t, f);
        else store_quad<S == 4>(p + t, f);
      }
    }
  } else if constexpr (S % 4 == 0) {
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      if (t + 4 <= T) {
        store_quad_ua(p + t, make_float4(v[4 * q + 0], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (t + i < T) p[t + i] = from_f32<E>(v[4 * q + i]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < S; ++i)
      if (t0 + i < T) p[t0 + i] = from_f32<E>(v[i]);
  }
}

// A 0.0f that is never written: the source of an unconditional load whose operand is absent.
// Global (not __constant__) memory, so that selecting between it and a global operand keeps
// a global load (a flat load would also count against the LDS counter).  All-zero bits are
// also a bfloat16 zero.
__device__ float g_zero[4] = {0.f, 0.f, 0.f, 0.f};
template <class E>
__device__ __forceinline__ const E* zero_src() { return reinterpret_cast<const E*>(g_zero); }

// Bootstrap argument shared by the backward estimators: none, one value per row, or
// one value per step (the reference's last_value / bootstrap_values pair).
enum BootMode : int { kBootNone = 0, kBootRow = 1, kBootFull = 2 };

// Address of boot(T-1) for `row` (g_zero when there is no bootstrap).
template <class E>
__device__ __forceinline__ const E* boot_last(const E* boot, int mode, int64_t row, int T) {
  return mode == kBootFull ? boot + row * (int64_t)T + (T - 1)
       : mode == kBootRow  ? boot + row
                           : zero_src<E>();
}

// The bootstrap in two halves, load (raw, unconditional) and prepare:
//   PER_STEP = false: the caller only uses boot(T-1) (no truncations), so only that value
//                     is read (a per-step array at its last column);
//   PER_STEP = true:  a per-step array is read in full; with a per-row value (or none) the
//                     segment loads read `any_row` (any readable [T] row) and are discarded.
// boot_prepare turns the raw registers into bt[i] = boot(t0 + i).
template <int S, int VEC, bool PER_STEP, class E>
__device__ __forceinline__ void boot_load(const E* __restrict__ boot, int mode, int64_t row,
                                          int t0, int T, float (&seg)[S], float& last,
                                          const E* any_row) {
  if constexpr (PER_STEP) {
    load_seg<S, VEC>(mode == kBootFull ? boot + row * (int64_t)T : any_row, t0, T, seg);
    // a per-step array already holds boot(T-1) in the segment that contains T-1
    last = mode == kBootFull ? 0.f : to_f32(*boot_last(boot, mode, row, T));
  } else {
    last = to_f32(*boot_last(boot, mode, row, T));
  }
}
template <int S, bool PER_STEP>
__device__ __forceinline__ void boot_prepare(int mode, int t0, int T, float (&bt)[S], float last) {
#pragma unroll
  for (int i = 0; i < S; ++i) {
    const float at_last = (t0 + i == T - 1) ? last : 0.f;
    bt[i] = (PER_STEP && mode == kBootFull) ? bt[i] : at_last;
  }
}

// The row's carry x[T] (backward) / x[-1] (forward): op.row_carry_src() gives its address,
// nullptr for 0.
// Ops whose map is not Affine give their row's carried state by op.row_state(row, T).
template <class Op>
__device__ __forceinline__ typename Op::Map::State row_carry(const Op& op, int64_t row, int T) {
  if constexpr (std::is_same<typename Op::Map, Affine>::value) {
    const auto* src = op.row_carry_src(row, T);
    return src ? to_f32(*src) : 0.f;
  } else {
    return op.row_state(row, T);
  }
}

// A halo value of two floats (Retrace: c[t+1] and q[t+1]).
struct Halo2 {
  float a, b;
};

// ---------------------------------------------------------------------------------------
// Decoupled look-back status words.  Per tile kStatusWords 64-bit words {tag:32 | value:32}:
//   AGG (the tile's map):           words 0..Map::kWords-1 = the map's coefficients
//   INC (the state at the tile's outgoing edge): words 0..kStateWords-1 (x first)
// Every word carries its own tag, so a reader accepts a map or a state only when all of
// its words carry the same current tag.
// tag = (epoch << 2) | kind, kind 1 = AGG, 2 = INC.  A word whose epoch differs from the
// current call's is "not yet published", so the workspace needs clearing only once.
//
// Workspace (uint64 words), the same layout for every shape so that one buffer serves
// calls of any shape in stream order:
//   header   [0..7]               [3] error flag (a bounded wait gave up, or counters were
//                                 not at rest); others reserved
//   slots    [8 + 32*s], s < 64   slot s (256 bytes each), rows r = s mod 64:
//                                 +16 counter of the slot's workgroups that have started,
//                                 +24 epoch of the slot's calls
//   status   [8 + 32*64 ...]      kStatusWords words per tile, tiles of row r at
//                                 r*tiles_per_row: what the tile's own workgroup publishes
//   second   [status + kStatusWords*tiles ...]  the same layout: what other workgroups
//                                 publish for a tile they computed in its place
// (tiles counted at the smallest tile; see rlk_workspace_bytes).  Device-scope atomics on
// one address serialise (~12 ns each on MI355X), so the start counters are spread over 64
// slots.  Each slot holds a copy of the epoch, and all 64 copies advance once per call
// (each as soon as every workgroup that reads it has done so: the one that completes a
// slot's start count advances the copies of its residue class), so they stay equal, a
// status word left by any earlier call never matches the current epoch, and no workgroup
// issues an atomic on its way out of the kernel.
// ---------------------------------------------------------------------------------------
constexpr int kHeaderWords = 8;
constexpr int kSlots = 64;
constexpr int kSlotWords = 32;
constexpr int kStatusOffset = kHeaderWords + kSlots * kSlotWords;
constexpr int kStatusWords = 5;  // the largest map (SkipAffine); Affine tiles use 2 of them
constexpr uint32_t kAgg = 1, kInc = 2;
constexpr uint32_t kEpochMask = 0x3fffffffu;
constexpr int kSpinLimit = 1 << 20;  // polls before a wait gives up (~1 s), never reached when correct

// The carry of a tile whose look-back gave up: NaN in every component.
template <class S>
__device__ __forceinline__ S nan_state();
template <>
__device__ __forceinline__ float nan_state<float>() { return __builtin_nanf(""); }
template <>
__device__ __forceinline__ NvX nan_state<NvX>() { return NvX{__builtin_nanf(""), __builtin_nanf("")}; }

__device__ __forceinline__ uint64_t atomic_ld(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_st(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t pack(uint32_t tag, float v) {
  return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}

// ---------------------------------------------------------------------------------------
// Segment pieces shared by both kernels.
// ---------------------------------------------------------------------------------------

// The segment's map: steps composed in scan order, starting from the first step itself
// (composing with the identity would cost a multiply and an fma the compiler cannot drop:
// x * 1 and fma(x, 0, y) are not exact identities for inf or nan).
template <bool FWD, int S, class M>
__device__ __forceinline__ M fold_segment(const M (&steps)[S]) {
  if constexpr (FWD) {
    M m = steps[0];
#pragma unroll
    for (int i = 1; i < S; ++i) m = compose(steps[i], m);
    return m;
  } else {
    M m = steps[S - 1];
#pragma unroll
    for (int i = S - 2; i >= 0; --i) m = compose(steps[i], m);
    return m;
  }
}

// Every step's state from the state entering the segment.
template <bool FWD, int S, class M>
__device__ __forceinline__ void replay(const M (&steps)[S], typename M::State x_in,
                                       typename M::State (&xs)[S]) {
  typename M::State x = x_in;
  if constexpr (FWD) {
#pragma unroll
    for (int i = 0; i < S; ++i) xs[i] = x = steps[i].apply(x);
  } else {
#pragma unroll
    for (int i = S - 1; i >= 0; --i) xs[i] = x = steps[i].apply(x);
  }
}

// ---------------------------------------------------------------------------------------
// Cross-lane moves by DPP (gfx9 data-parallel primitives): a VALU modifier, no trip through
// the LDS crossbar.  update_dpp(old, src): a lane whose source lane is invalid, or whose
// row is masked off, keeps `old`.
// ---------------------------------------------------------------------------------------
constexpr int kDppRowShr = 0x110;     // + n: lane i <- lane i-n within its row of 16
constexpr int kDppWaveShr1 = 0x138;   // lane i <- lane i-1 across the wave
constexpr int kDppRowBcast15 = 0x142; // lane 15 of each row -> the next row
constexpr int kDppRowBcast31 = 0x143; // lane 31 -> rows 2 and 3

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp(float src, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src), CTRL,
                                                    ROW_MASK, 0xf, false));
}

// ---------------------------------------------------------------------------------------
// Per-workgroup output statistics (ops with kBlockStats): float64 count, sum and sum of
// squares of the outputs the op counts (op.stats()), reduced in a fixed order (lanes by
// wave_total's DPP steps, waves in index order), so the partial a workgroup writes is the
// same bit pattern on every run.  kStatWords doubles per workgroup.
// ---------------------------------------------------------------------------------------
constexpr int kStatWords = 3;

struct Stats {
  double n = 0.0, sum = 0.0, sq = 0.0;
  __device__ void add(float v) {
    const double x = (double)v;
    n += 1.0;
    sum += x;
    sq = fma(x, x, sq);
  }
};

// A double moved by a DPP control (both halves alike); lanes without a source get 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_or_zero(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROW_MASK, 0xf, false);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROW_MASK, 0xf, false);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// The wave's sum of v, in lane 63 (other lanes hold partial sums): prefixes within each row
// of 16 lanes (row_shr 1, 2, 4, 8), then rows 0+1 and 2+3 (row_bcast 15), then all four
// (row_bcast 31).  A fixed order, and all of it in VALU: a butterfly of ds_bpermute round
// trips through the LDS crossbar costs one LDS latency per level.
__device__ __forceinline__ double wave_total(double v) {
  v += dpp_or_zero<kDppRowShr + 1, 0xf>(v);
  v += dpp_or_zero<kDppRowShr + 2, 0xf>(v);
  v += dpp_or_zero<kDppRowShr + 4, 0xf>(v);
  v += dpp_or_zero<kDppRowShr + 8, 0xf>(v);
  v += dpp_or_zero<kDppRowBcast15, 0xa>(v);
  v += dpp_or_zero<kDppRowBcast31, 0xc>(v);
  return v;
}

// Every thread of the workgroup calls this once; thread 0 writes
// partials[kStatWords*blockIdx.x + {0,1,2}] = {n, sum, sum of squares}.
template <int NT>
__device__ __forceinline__ void block_stats(Stats st, double* __restrict__ partials) {
  constexpr int NW = NT / kWave;
  __shared__ double s_st[kStatWords][NW];
  st.n = wave_total(st.n);
  st.sum = wave_total(st.sum);
  st.sq = wave_total(st.sq);
  const int wave = threadIdx.x / kWave;
  if (__lane_id() == kWave - 1) {
    s_st[0][wave] = st.n;
    s_st[1][wave] = st.sum;
    s_st[2][wave] = st.sq;
  }
  __syncthreads();
  if (threadIdx.x < kStatWords) {
    double a = 0.0;
    for (int w = 0; w < NW; ++w) a += s_st[threadIdx.x][w];
    partials[kStatWords * blockIdx.x + threadIdx.x] = a;
  }
}

// One level of a tree over the partials, for first launches of many workgroups: workgroup j
// sums the triples j*kReduceSlice .. (j+1)*kReduceSlice - 1 of `in` (n triples in all; thread
// i takes i, i+NT, ... in order, then block_stats' fixed lane and wave order) into out[j].
// Without it every workgroup of normalize_kernel reads every triple: at [2^20, 128] (65536
// triples, 2048 normalising workgroups) that is 3.2 GB of cache reads ahead of the
// workgroups' first stores.
constexpr int kReduceNT = 256, kReducePerThread = 8;
constexpr int kReduceSlice = kReduceNT * kReducePerThread;

template <int NT>
__global__ __launch_bounds__(NT) void reduce_partials_kernel(const double* __restrict__ in, int n,
                                                             double* __restrict__ out) {
  static_assert(NT * kReducePerThread == kReduceSlice, "one slice per workgroup");
  const int64_t first = (int64_t)blockIdx.x * kReduceSlice + threadIdx.x;
  double p[kReducePerThread][kStatWords];
#pragma unroll
  for (int k = 0; k < kReducePerThread; ++k) {
    const int64_t i = first + k * NT;
#pragma unroll
    for (int w = 0; w < kStatWords; ++w) p[k][w] = i < n ? in[kStatWords * i + w] : 0.0;
  }
  Stats st;
#pragma unroll
  for (int k = 0; k < kReducePerThread; ++k) {
    st.n += p[k][0];
    st.sum += p[k][1];
    st.sq += p[k][2];
  }
  block_stats<NT>(st, out);
}

// Second launch of the normalisation: every workgroup combines the per-workgroup partials
// of the first launch in one fixed order (thread i sums partials i, i+NT, ...; the lanes by
// wave_total; the waves in index order), so all agree on the statistics, then rewrites its
// share of the n_all elements of x as (x - mean) / (std + eps): mean and std (unbiased,
// count - 1, as torch computes x.std()) over the elements the first launch counted, which
// are all of them, or the kept steps of a masked call.
template <int NT, bool VEC, class E>
__global__ __launch_bounds__(NT) void normalize_kernel(E* __restrict__ x,
                                                       const double* __restrict__ partials,
                                                       int nparts, int64_t n_all, float eps) {
  constexpr int NW = NT / kWave;
  __shared__ double s_st[kStatWords][NW];
  const int tid = threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * NT;
  const int64_t first = (int64_t)blockIdx.x * NT + tid;
  const int64_t units = VEC ? n_all / 4 : n_all;
  // this thread's first element is loaded before the statistics, so the two round trips
  // overlap
  float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (first < units) {
    if constexpr (VEC) v0 = load_quad<true>(x + 4 * first);
    else v0.x = load_one_nt(x + first);
  }
  // four triples' loads in flight per round, summed in index order (at 1024-2048 triples
  // 6-7% faster per call than one triple per round)
  double acc[kStatWords] = {0.0, 0.0, 0.0};
  int i = tid;
  for (; i + 3 * NT < nparts; i += 4 * NT) {
    double p[4][kStatWords];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int k = 0; k < kStatWords; ++k) p[u][k] = partials[kStatWords * (i + u * NT) + k];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int k = 0; k < kStatWords; ++k) acc[k] += p[u][k];
    }
  }
  for (; i < nparts; i += NT) {
#pragma unroll
    for (int k = 0; k < kStatWords; ++k) acc[k] += partials[kStatWords * i + k];
  }
#pragma unroll
  for (int k = 0; k < kStatWords; ++k) acc[k] = wave_total(acc[k]);
  if (__lane_id() == kWave - 1) {
#pragma unroll
    for (int k = 0; k < kStatWords; ++k) s_st[k][tid / kWave] = acc[k];
  }
  __syncthreads();
  double n = 0.0, sum = 0.0, sq = 0.0;
  for (int w = 0; w < NW; ++w) {
    n += s_st[0][w];
    sum += s_st[1][w];
    sq += s_st[2][w];
  }
  const double mean = sum / n;  // nan when nothing was counted
  double var = (sq - sum * mean) / (n - 1.0);
  var = var > 0.0 ? var : 0.0;
  if (!(n >= 2.0)) var = __builtin_nan("");  // torch: the unbiased std of one element is nan
  const float m = (float)mean;
  const float d = (float)sqrt(var) + eps;
  if constexpr (VEC) {
    for (int64_t i = first; i < units; i += stride) {
      float4 v = i == first ? v0 : load_quad<true>(x + 4 * i);
      v.x = (v.x - m) / d;
      v.y = (v.y - m) / d;
      v.z = (v.z - m) / d;
      v.w = (v.w - m) / d;
      store_quad<true>(x + 4 * i, v);
    }
  } else {
    for (int64_t i = first; i < units; i += stride)
      store_one_nt(x + i, ((i == first ? v0.x : load_one_nt(x + i)) - m) / d);
  }
}

// The previous lane's value (lane 0 keeps its own).
__device__ __forceinline__ float lane_prev(float v) { return dpp<kDppWaveShr1, 0xf>(v, v); }
__device__ __forceinline__ Halo2 lane_prev(Halo2 h) { return Halo2{lane_prev(h.a), lane_prev(h.b)}; }
__device__ __forceinline__ NoHalo lane_prev(NoHalo h) { return h; }
__device__ __forceinline__ NvX lane_prev(NvX s) { return NvX{lane_prev(s.nv), lane_prev(s.x)}; }

// A map moved by a DPP control; lanes without a source get the identity.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ Affine dpp_map(Affine m) {
  return Affine{dpp<CTRL, ROW_MASK>(m.mul, 1.f), dpp<CTRL, ROW_MASK>(m.add, 0.f)};
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ SkipAffine dpp_map(SkipAffine m) {
  return SkipAffine{dpp<CTRL, ROW_MASK>(m.a, 1.f), dpp<CTRL, ROW_MASK>(m.c, 0.f),
                    dpp<CTRL, ROW_MASK>(m.p, 0.f), dpp<CTRL, ROW_MASK>(m.q, 1.f),
                    dpp<CTRL, ROW_MASK>(m.d, 0.f)};
}

// The data of a segment that the next segment in scan order needs: its last step (forward
// scans: done[t-1]) or its first step (backward scans: values[t+1], ...).
template <class Op, int S>
__device__ __forceinline__ typename Op::Halo scan_export(const Op& op, const typename Op::template Regs<S>& R) {
  if constexpr (Op::kForward) return op.template export_last<S>(R);
  else return op.template export_first<S>(R);
}

template <int D, class M>
__device__ __forceinline__ M scan_step_rows(M m, int li, int W) {
  M prev = dpp_map<kDppRowShr + D, 0xf>(m);
  // groups narrower than a DPP row: the source may be in another group.  (From 16 lanes up
  // a group starts a row, where row_shr already leaves the identity.)
  if (W < 16 && li < D) prev = M::identity();
  return compose(m, prev);
}

// Inclusive scan of maps towards higher lanes, in groups of W lanes (W a power of two <= 64,
// wave-uniform): lane i ends up with m_i o m_{i-1} o ... o m_0 of its group.  Kogge-Stone
// within rows of 16 lanes, then row_bcast to join rows.
template <class M>
__device__ __forceinline__ M lane_scan(M m, int W) {
  const int li = __lane_id() & (W - 1);
  if (W > 1) m = scan_step_rows<1>(m, li, W);
  if (W > 2) m = scan_step_rows<2>(m, li, W);
  if (W > 4) m = scan_step_rows<4>(m, li, W);
  if (W > 8) m = scan_step_rows<8>(m, li, W);
  if (W > 16) m = compose(m, dpp_map<kDppRowBcast15, 0xa>(m));
  if (W > 32) m = compose(m, dpp_map<kDppRowBcast31, 0xc>(m));
  return m;
}

// ---------------------------------------------------------------------------------------
// Short rows: a workgroup of NT threads holds NT/L whole rows of L threads each
// (L = 2^log2L, L*S >= T).  Launch: grid = ceil(E / (NT/L)).
//
// Lane space.  A row's segments are assigned to its L threads in scan order: in time order
// for forward scans, reversed for backward scans (thread i of the row holds segment L-1-i).
// Every scan then runs towards higher lanes whatever the op's direction, which is the
// direction DPP row broadcasts go; memory accesses stay coalesced (lane order within a
// wave does not matter to them).  The segment before a thread's own in scan order is in
// the previous lane, so the neighbour step's data, and the value entering the segment,
// come from there.
// ---------------------------------------------------------------------------------------
// WT: the scan width W fixed at compile time (16, 32 or 64), or 0 for a width taken from
// log2L at run time.  With W = 16 or 32, L = W is fixed too.  A fixed width leaves the lane
// scan and the index arithmetic straight-line code the compiler schedules across: V-trace
// [4096,128] 4.12 -> 3.99 us, GAE 3.99 -> 3.80 us, GAE [8192,64] 3.97 -> 3.78 us, TD(lambda)
// [256,2048] 3.61 -> 3.48 us, element-aligned V-trace [4096,127] 4.80 -> 4.66 us on MI355X
// (bit-identical results).
template <class Op, int NT, int S, int VEC, int WT = 0, int SP = 0>
__global__ __launch_bounds__(NT) void rows_kernel(const Op op, int64_t E, int T, int log2L_arg) {
  static_assert(VEC != kPhased, "phased access is for long rows");
  constexpr bool FWD = Op::kForward;
  constexpr int NW = NT / kWave;
  using Regs = typename Op::template Regs<S>;
  using Halo = typename Op::Halo;
  using Map = typename Op::Map;
  using State = typename Map::State;
  constexpr bool HAS_HALO = !std::is_same<Halo, NoHalo>::value;
  __shared__ Map s_map[NW];

  const int tid = threadIdx.x;
  const int lane = __lane_id();
  const int wave = tid / kWave;
  static_assert(WT == 0 || WT == 16 || WT == 32 || WT == kWave, "fixed scan widths");
  const int log2L = WT == 16 ? 4 : WT == 32 ? 5 : log2L_arg;
  const int L = 1 << log2L;
  const int W = WT > 0 ? WT : (L < kWave ? L : kWave);
  const int li = tid & (L - 1);  // position in scan order
  const int64_t row_id = (int64_t)blockIdx.x * (NT >> log2L) + (tid >> log2L);
  const bool active = row_id < E;
  const int64_t row = active ? row_id : E - 1;  // idle lanes of the last workgroup read a real row
  const int t0 = (FWD ? li : L - 1 - li) * S;

  Regs R;
  op.template load<S, VEC>(row, t0, T, R);
  // the first lane of a wave that is not the first of its row reads the neighbour step
  Halo edge{};
  if constexpr (HAS_HALO) {
    if (lane == 0 && li > 0) edge = op.halo_load(row, clamp_step(FWD ? t0 - 1 : t0 + S, T), T);
  }
  State carry = row_carry(op, row, T);
  op.template prepare<S, VEC>(R, row, t0, T);
  Halo h{};
  if constexpr (HAS_HALO) {
    h = lane_prev(scan_export<Op, S>(op, R));
    if (lane == 0) h = edge;  // unused when li == 0: the row's first segment in scan order
  }

  Map steps[S];
  op.template coef<S, VEC>(R, h, row, t0, T, steps);
  const Map m = lane_scan(fold_segment<FWD, S>(steps), W);

  if (L > kWave) {
    // rows spanning several waves: combine the wave aggregates of the row through LDS
    if (lane == kWave - 1) s_map[wave] = m;
    __syncthreads();
    const int first = (wave / (L / kWave)) * (L / kWave);
    for (int v = first; v < wave; ++v) carry = s_map[v].apply(carry);
  }
  // state entering the segment: the previous lane's outgoing state, or the carry
  State x_in = lane_prev(m.apply(carry));
  if ((li & (W - 1)) == 0) x_in = carry;
  State xs[S];
  replay<FWD, S>(steps, x_in, xs);
  if (active) op.template emit<S, VEC, SP>(R, h, xs, x_in, row, t0, T);
  if constexpr (Op::kBlockStats) {
    Stats st;
    if (active) op.template stats<S>(R, xs, t0, T, st);
    block_stats<NT>(st, op.partials);
  }
}

// Two row groups per thread (float32 Retrace on rows of 65..128 steps, chosen by the
// launcher): a workgroup of NT threads holds 2*NT/L rows, in two groups of NT/L consecutive
// rows, and each thread one row of each.  Rows stay within one wave (W = L = 16 or 32).
// Launch: grid = ceil(E / (2*NT/L)).
//
// The source order below, with the wave-edge neighbour read of rows_kernel kept (it never
// fires here: a row's first lane is a wave's first lane or follows another of its row), is
// the one for which the compiler issues every load of both rows before the arithmetic on
// them.  Orders without that read (one row scanned and stored after the other, or both
// scanned first) interleaved the second row's loads with the first row's arithmetic, and
// C4 Retrace [4096,128] took 6.95 us instead of 6.41.
template <class Op, int NT, int WT, int SP = 0>
__global__ __launch_bounds__(NT) void rows_pair_kernel(const Op op, int64_t E, int T, int) {
  constexpr bool FWD = Op::kForward;
  constexpr int S = 4, RPT = 2;
  using Regs = typename Op::template Regs<S>;
  using Halo = typename Op::Halo;
  using Map = typename Op::Map;
  using State = typename Map::State;
  constexpr bool HAS_HALO = !std::is_same<Halo, NoHalo>::value;
  static_assert(WT == 16 || WT == 32, "rows within one wave");
  static_assert(!Op::kBlockStats, "no statistics epilogue");
  constexpr int log2L = WT == 16 ? 4 : 5;
  constexpr int L = WT;
  const int tid = threadIdx.x;
  const int lane = __lane_id();
  const int li = tid & (L - 1);  // position in scan order
  const int t0 = (FWD ? li : L - 1 - li) * S;
  int64_t row[RPT];
  bool active[RPT];
  Regs R[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t row_id = ((int64_t)blockIdx.x * RPT + u) * (NT >> log2L) + (tid >> log2L);
    active[u] = row_id < E;
    row[u] = active[u] ? row_id : E - 1;  // idle lanes of the last workgroup read a real row
    op.template load<S, kAligned>(row[u], t0, T, R[u]);
  }
  Halo edge{};
  if constexpr (HAS_HALO) {
    if (lane == 0 && li > 0) edge = op.halo_load(row[0], clamp_step(FWD ? t0 - 1 : t0 + S, T), T);
  }
  State carry[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    carry[u] = row_carry(op, row[u], T);
    op.template prepare<S, kAligned>(R[u], row[u], t0, T);
  }
  Halo h[RPT];
  Map steps[RPT][S];
  Map m[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    if constexpr (HAS_HALO) {
      h[u] = lane_prev(scan_export<Op, S>(op, R[u]));
      if (lane == 0) h[u] = edge;  // unused: the row's first segment in scan order
    }
    op.template coef<S, kAligned>(R[u], h[u], row[u], t0, T, steps[u]);
    m[u] = lane_scan(fold_segment<FWD, S>(steps[u]), WT);
  }
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    // state entering the segment: the previous lane's outgoing state, or the carry
    State x_in = lane_prev(m[u].apply(carry[u]));
    if (li == 0) x_in = carry[u];
    State xs[S];
    replay<FWD, S>(steps[u], x_in, xs);
    if (active[u]) op.template emit<S, kAligned, SP>(R[u], h[u], xs, x_in, row[u], t0, T);
  }
}

// ---------------------------------------------------------------------------------------
// Long rows: the decoupled look-back.
// ---------------------------------------------------------------------------------------
__host__ __device__ inline int lookback_slots(int64_t E) { return E < kSlots ? (int)E : kSlots; }

// s_waitcnt vmcnt(0): the look-back wave's own traffic is complete before its path rejoins
// the other waves', so nothing it issued looks pending to the compiler afterwards.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Lane 0's value of a 64-bit register, in every lane.
__device__ __forceinline__ uint64_t lane0_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, 0);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 0);
  return ((uint64_t)hi << 32) | lo;
}

// What one look-back read finds for a tile: lane l examines tile k -/+ (1 + base + l) of
// the row, in its own status words (st) and in those another workgroup published for it
// (sf, see chain_kernel).  kind: 0 (nothing usable yet), kAgg or kInc; absent: nothing of
// this call in either place (its workgroup has not published yet).
template <class M>
struct Probe {
  uint32_t kind;
  bool absent;
  float w[M::kWords];
};

template <bool FWD, class M>
__device__ __forceinline__ Probe<M> probe_tiles(const uint64_t* st, const uint64_t* sf, int k,
                                                int base, int tiles_per_row, uint32_t epoch,
                                                int lane) {
  constexpr int NWD = M::kWords, NSW = M::kStateWords;
  const uint32_t tag_agg = (epoch << 2) | kAgg, tag_inc = (epoch << 2) | kInc;
  Probe<M> p;
  p.kind = 0;
  p.absent = false;
#pragma unroll
  for (int i = 0; i < NWD; ++i) p.w[i] = 0.f;
  const int jj = FWD ? k - 1 - base - lane : k + 1 + base + lane;
  if (FWD ? jj >= 0 : jj < tiles_per_row) {
    // All words in flight at once.  Each word is written at most once per call, kind and
    // place (by identical values when two workgroups write one place), so words that all
    // carry the current AGG tag (or INC tag) are one consistent map (or state); a word
    // with another tag just means "not yet".
    uint64_t a[NWD], b[NWD];
#pragma unroll
    for (int i = 0; i < NWD; ++i) a[i] = atomic_ld(st + NWD * jj + i);
#pragma unroll
    for (int i = 0; i < NWD; ++i) b[i] = atomic_ld(sf + NWD * jj + i);
    auto kind_of = [&](const uint64_t(&x)[NWD]) -> uint32_t {
      const uint32_t tag0 = (uint32_t)(x[0] >> 32);
      const uint32_t kd = tag0 & 3u;
      if ((tag0 >> 2) != epoch || (kd != kAgg && kd != kInc)) return 0u;
      const uint32_t want = kd == kAgg ? tag_agg : tag_inc;
      const int nw = kd == kAgg ? NWD : NSW;
#pragma unroll
      for (int i = 1; i < NWD; ++i)
        if (i < nw && (uint32_t)(x[i] >> 32) != want) return 0u;
      return kd;
    };
    auto touched = [&](uint64_t w0) {  // word 0 (written last) names this call's publish
      const uint32_t tag0 = (uint32_t)(w0 >> 32);
      return (tag0 >> 2) == epoch && (tag0 & 3u) != 0u;
    };
    const uint32_t ka = kind_of(a), kb = kind_of(b);
    const bool use_b = kb == kInc ? ka != kInc : (ka == 0u && kb != 0u);  // a state first
    p.kind = use_b ? kb : ka;
#pragma unroll
    for (int i = 0; i < NWD; ++i) p.w[i] = __uint_as_float((uint32_t)(use_b ? b[i] : a[i]));
    p.absent = !touched(a[0]) && !touched(b[0]);
  }
  return p;
}

// The state a lane's tile publishes (INC words), as seen by every lane.
template <class M>
__device__ __forceinline__ typename M::State probe_state(const Probe<M>& p, int l) {
  float iw[M::kStateWords];
#pragma unroll
  for (int i = 0; i < M::kStateWords; ++i) iw[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.w[i]), l));
  return state_from_words<typename M::State>(iw);
}
// The map a lane's tile publishes (AGG words), as seen by every lane.
template <class M>
__device__ __forceinline__ M probe_map(const Probe<M>& p, int l) {
  float aw[M::kWords];
#pragma unroll
  for (int i = 0; i < M::kWords; ++i) aw[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p.w[i]), l));
  return M::from_words(aw);
}

// Carry entering tile k of `row` (one wave, all 64 lanes): publish the tile's map and look
// back.  Predecessors are read 64 at a time (lane i <-> i+1 tiles away).  Once the nearest
// published state X has only maps between it and this tile, they are applied to X one at a
// time, nearest last, so every published state equals the sequential chain
// X_k = A_k(X_{k+1}) however far the look-back reached, and whichever state it found:
// results are bit-reproducible.
//
// Tiles come from the block index, not from an ordered ticket, so a predecessor's
// workgroup may not have started.  The look-back never depends on it: after
// `fallback_polls` polls,
//   * a predecessor with nothing published is handed back (need = its tile): the
//     workgroup computes that tile's map itself, publishes it in the predecessor's second
//     place (sf), and looks back again;
//   * a window of 64 maps and no state makes the look-back walk further back, window by
//     window, to a state, and then apply every map from there, one by one.
// A bounded wait (spin_limit polls in all) gives up rather than hang: it sets the error
// flag and takes a NaN carry, so the tile's outputs, and those of every tile that chains
// through its state, are NaN instead of plausible values.
// The first tile of a row (in scan order) takes `row_c`, the row's own carry.
// Tile k's status words are st[M::kWords * k + i] (kStatusWords bounds M::kWords).
template <bool FWD, class M>
__device__ __forceinline__ typename M::State tile_carry(M tm, typename M::State row_c, int64_t row,
                                                        int k, int tiles_per_row, uint32_t epoch,
                                                        uint64_t* ws, uint64_t* fb, int lane,
                                                        int spin_limit, int fallback_polls,
                                                        int& need) {
  using State = typename M::State;
  constexpr int NWD = M::kWords, NSW = M::kStateWords;
  static_assert(NWD <= kStatusWords && NSW <= NWD, "status words per tile");
  uint64_t* st = ws + kStatusOffset + NWD * (row * (int64_t)tiles_per_row);
  const uint64_t* sf = fb + NWD * (row * (int64_t)tiles_per_row);
  const uint32_t tag_agg = (epoch << 2) | kAgg, tag_inc = (epoch << 2) | kInc;
  need = -1;
  // word 0 last: it names the kind
  auto publish_inc = [&](State x) {
#pragma unroll
    for (int i = NSW - 1; i >= 0; --i) atomic_st(st + NWD * k + i, pack(tag_inc, state_word(x, i)));
  };
  if (FWD ? (k == 0) : (k == tiles_per_row - 1)) {
    wait_vmem();
    if (lane == 0) publish_inc(tm.apply(row_c));
    return row_c;
  }
  if (lane == 0) {
    if (tm.constant()) {
      // the tile's outgoing state does not depend on its carry
      publish_inc(tm.apply(State{}));
    } else {
#pragma unroll
      for (int i = NWD - 1; i >= 0; --i) atomic_st(st + NWD * k + i, pack(tag_agg, tm.word(i)));
    }
  }
  auto tile_at = [&](int base, int l) { return FWD ? k - 1 - base - l : k + 1 + base + l; };
  auto first_of = [](uint64_t mask) { return mask ? __ffsll((long long)mask) - 1 : kWave; };
  State c{};
  bool done = false;
  int spins = 0;
  // the nearest 64 tiles
  bool walk = false;
  for (;; ++spins) {
    const Probe<M> p = probe_tiles<FWD, M>(st, sf, k, 0, tiles_per_row, epoch, lane);
    const int first_inc = first_of(__ballot(p.kind == kInc));
    const int first_bad = first_of(__ballot(p.kind == 0u));
    const uint64_t absent = __ballot(p.absent);
    if (first_inc < first_bad) {
      State x = probe_state(p, first_inc);
      for (int l = first_inc - 1; l >= 0; --l) x = probe_map(p, l).apply(x);
      c = x;
      done = true;
      break;
    }
    if (spins >= spin_limit) break;
    if (spins >= fallback_polls) {
      if (first_bad < kWave && ((absent >> first_bad) & 1u)) {
        need = tile_at(0, first_bad);
        wait_vmem();
        return c;
      }
      if (first_bad == kWave) {  // 64 maps, no state: walk back
        walk = true;
        break;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (walk) {
    // windows further back, to the first that holds a state before anything unusable
    int base = kWave, found = -1;
    Probe<M> p{};
    for (; spins < spin_limit; ++spins) {
      p = probe_tiles<FWD, M>(st, sf, k, base, tiles_per_row, epoch, lane);
      const int first_inc = first_of(__ballot(p.kind == kInc));
      const int first_bad = first_of(__ballot(p.kind == 0u));
      const uint64_t absent = __ballot(p.absent);
      if (first_inc < first_bad) {
        found = first_inc;
        break;
      }
      if (first_bad < kWave) {
        if ((absent >> first_bad) & 1u) {
          need = tile_at(base, first_bad);
          wait_vmem();
          return c;
        }
        __builtin_amdgcn_s_sleep(1);  // published, not complete yet: read this window again
        continue;
      }
      base += kWave;
    }
    if (found >= 0) {
      // from that state, every map between it and this tile, one by one, nearest last (a
      // tile that has published its state meanwhile gives that state: the same bits)
      State x = probe_state(p, found);
      for (int l = found - 1; l >= 0; --l) x = probe_map(p, l).apply(x);
      for (base -= kWave; base >= 0 && spins < spin_limit; base -= kWave) {
        for (; spins < spin_limit; ++spins) {
          p = probe_tiles<FWD, M>(st, sf, k, base, tiles_per_row, epoch, lane);
          if (__ballot(p.kind == 0u) == 0) break;
          __builtin_amdgcn_s_sleep(1);
        }
        if (spins >= spin_limit) break;
        for (int l = kWave - 1; l >= 0; --l) {
          const uint32_t kl = (uint32_t)__builtin_amdgcn_readlane((int)p.kind, l);
          x = kl == kInc ? probe_state(p, l) : probe_map(p, l).apply(x);
        }
      }
      if (base < 0) {
        c = x;
        done = true;
      }
    }
  }
  if (!done) {
    if (lane == 0) atomic_st(ws + 3, (uint64_t)1);
    c = nan_state<State>();
  }
  wait_vmem();
  if (lane == 0 && !tm.constant()) publish_inc(tm.apply(c));
  return c;
}

// A tile's map (or, for a row's first tile or a tile whose map ignores its carry, its
// state) computed by a workgroup that is not the tile's own: published in the tile's second
// place, which only such workgroups write, all with the same values.
template <bool FWD, class M>
__device__ __forceinline__ void publish_for(M tm, typename M::State row_c, int64_t row, int k,
                                            int tiles_per_row, uint32_t epoch, uint64_t* fb,
                                            int lane) {
  using State = typename M::State;
  constexpr int NWD = M::kWords, NSW = M::kStateWords;
  uint64_t* sf = fb + NWD * (row * (int64_t)tiles_per_row);
  const uint32_t tag_agg = (epoch << 2) | kAgg, tag_inc = (epoch << 2) | kInc;
  const bool first = FWD ? (k == 0) : (k == tiles_per_row - 1);
  if (lane == 0) {
    if (first || tm.constant()) {
      const State x = tm.apply(first ? row_c : State{});
#pragma unroll
      for (int i = NSW - 1; i >= 0; --i) atomic_st(sf + NWD * k + i, pack(tag_inc, state_word(x, i)));
    } else {
#pragma unroll
      for (int i = NWD - 1; i >= 0; --i) atomic_st(sf + NWD * k + i, pack(tag_agg, tm.word(i)));
    }
  }
  wait_vmem();
}

// ---------------------------------------------------------------------------------------
// Long rows, one tile per workgroup.
//
// Tile = NT threads x Q segments of 4 steps, held in registers.  The segments are strided
// by the wave so that every vector load and store of a wave covers 1 KB of consecutive
// memory: in wave w's chunk of Q*256 steps, segment q of lane l starts at step
// (q*64 + l)*4.  Like the short-row kernel the tile is laid out in lane space, so that
// every scan runs towards higher lanes: for backward ops the waves, the segment rows and
// the lanes are all taken in reverse.  Each of the Q segment rows is scanned across the 64
// lanes by DPP, and the rows are chained in scan order.
//
// A workgroup's tile (row, position in scan order) follows from its block index
// (slot = blockIdx % nslots); it loads and scans the tile, wave 0 publishes the tile's map
// and looks back for the carry, then every thread replays and stores.  Any residency makes
// progress: when a predecessor's workgroup has published nothing after a while, the
// look-back hands that tile back, and the workgroup loads and scans it, publishes its map
// in the predecessor's second place, and looks back again (tile_carry).  No ordered ticket
// is drawn, so a row's tiles do not queue on one counter.  Large tiles keep the look-back
// chain along a row short for the shapes this path serves (a few rows of 10^4..10^6
// steps).  Launch: grid = nslots * (tiles of the fullest slot), block = NT.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float lane_bcast(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ Halo2 lane_bcast(Halo2 h, int l) { return Halo2{lane_bcast(h.a, l), lane_bcast(h.b, l)}; }
__device__ __forceinline__ NoHalo lane_bcast(NoHalo h, int) { return h; }
__device__ __forceinline__ Affine lane_bcast(Affine m, int l) {
  return Affine{lane_bcast(m.mul, l), lane_bcast(m.add, l)};
}
__device__ __forceinline__ SkipAffine lane_bcast(SkipAffine m, int l) {
  return SkipAffine{lane_bcast(m.a, l), lane_bcast(m.c, l), lane_bcast(m.p, l), lane_bcast(m.q, l),
                    lane_bcast(m.d, l)};
}

constexpr int kSeg = 4;  // steps per segment of the long-row path

// Rows of 1025..2048 steps, one per workgroup, with the long-row tile layout: NT threads
// hold Q segments of 4 steps each, strided by the wave (segment q of lane l at step
// (q*64 + l)*4 of the wave's chunk), so every vector access of a wave covers 1 KB.  Against
// one segment per thread (rows_kernel with NT = 512) a row has half the waves, so its wave
// maps chain through LDS in at most NW - 1 = 3 applies instead of 7.  Launch: grid = E.
template <class Op, int NT, int Q, int VEC, int SP = 0>
__global__ __launch_bounds__(NT) void rows_strided_kernel(const Op op, int64_t E, int T, int) {
  static_assert(VEC != kPhased, "phased access is for long rows");
  constexpr bool FWD = Op::kForward;
  constexpr int NW = NT / kWave;
  constexpr int S = 4;
  constexpr int WSTEPS = Q * kWave * S;  // steps per wave chunk
  using Regs = typename Op::template Regs<S>;
  using Halo = typename Op::Halo;
  using Map = typename Op::Map;
  using State = typename Map::State;
  constexpr bool HAS_HALO = !std::is_same<Halo, NoHalo>::value;
  __shared__ Map s_map[NW];

  const int tid = threadIdx.x;
  const int lane = __lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t row = blockIdx.x;
  // lane space -> time: this wave's chunk, and the first step of segment row r
  const int wbase = (FWD ? wave : NW - 1 - wave) * WSTEPS;
  const int lt = FWD ? lane : kWave - 1 - lane;
  auto seg_t0 = [&](int r) { return wbase + ((FWD ? r : Q - 1 - r) * kWave + lt) * S; };

  Regs R[Q];
#pragma unroll
  for (int r = 0; r < Q; ++r) op.template load<S, VEC>(row, seg_t0(r), T, R[r]);
  Halo edge{};
  if constexpr (HAS_HALO) {
    if (lane == 0 && (FWD ? wbase > 0 : wbase + WSTEPS < T))
      edge = op.halo_load(row, clamp_step(FWD ? wbase - 1 : wbase + WSTEPS, T), T);
  }
  State carry = row_carry(op, row, T);
#pragma unroll
  for (int r = 0; r < Q; ++r) op.template prepare<S, VEC>(R[r], row, seg_t0(r), T);

  // neighbour step of each segment (the one before it in scan order): the previous lane,
  // lane 63 of the previous segment row, or the edge load
  Halo h[Q];
#pragma unroll
  for (int r = 0; r < Q; ++r) {
    if constexpr (HAS_HALO) {
      const Halo prev = lane_prev(scan_export<Op, S>(op, R[r]));
      const Halo wrap = r > 0 ? lane_bcast(scan_export<Op, S>(op, R[r > 0 ? r - 1 : 0]), kWave - 1) : edge;
      h[r] = lane == 0 ? wrap : prev;
    }
  }
  Map steps[Q][S];
  Map m[Q];
  Map rowagg[Q];  // map of each segment row (wave-uniform)
#pragma unroll
  for (int r = 0; r < Q; ++r) {
    op.template coef<S, VEC>(R[r], h[r], row, seg_t0(r), T, steps[r]);
    m[r] = lane_scan(fold_segment<FWD, S>(steps[r]), kWave);
    rowagg[r] = lane_bcast(m[r], kWave - 1);
  }
  // the chunk's map: segment rows composed in scan order
  Map wm = rowagg[0];
#pragma unroll
  for (int r = 1; r < Q; ++r) wm = compose(rowagg[r], wm);
  if (lane == 0) s_map[wave] = wm;
  __syncthreads();
  // state entering this wave's chunk, then each segment row, then each lane
  for (int v = 0; v < wave; ++v) carry = s_map[v].apply(carry);
  Stats st;
#pragma unroll
  for (int r = 0; r < Q; ++r) {
    State x_in = lane_prev(m[r].apply(carry));
    if (lane == 0) x_in = carry;
    carry = rowagg[r].apply(carry);
    State xs[S];
    replay<FWD, S>(steps[r], x_in, xs);
    op.template emit<S, VEC, SP>(R[r], h[r], xs, x_in, row, seg_t0(r), T);
    if constexpr (Op::kBlockStats) op.template stats<S>(R[r], xs, seg_t0(r), T, st);
  }
  if constexpr (Op::kBlockStats) block_stats<NT>(st, op.partials);
}


template <class Op, int NT, int Q, int VEC, int SP = 0>
__global__ __launch_bounds__(NT) void chain_kernel(const Op op, int64_t E, int T, int tiles_per_row,
                                                   uint64_t* __restrict__ ws, uint64_t* __restrict__ fb,
                                                   int spin_limit, int fallback_polls,
                                                   int row_major, int phase0) {
  constexpr bool FWD = Op::kForward;
  constexpr int NW = NT / kWave;
  constexpr int WSTEPS = Q * kWave * kSeg;  // steps per wave chunk
  static_assert(NT % kWave == 0, "whole waves");
  using Regs = typename Op::template Regs<kSeg>;
  using Halo = typename Op::Halo;
  using Map = typename Op::Map;
  using State = typename Map::State;
  constexpr bool HAS_HALO = !std::is_same<Halo, NoHalo>::value;
  __shared__ Map s_map[NW];
  __shared__ Map s_pref[NW];  // s_map[v] o ... o s_map[0]: the tile's maps up to each wave
  __shared__ State s_carry;
  __shared__ int s_next;
  __shared__ uint32_t s_epoch;

  const int tid = threadIdx.x;
  const int lane = __lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int nslots = lookback_slots(E);
  const uint64_t wgs_per_slot = gridDim.x / (unsigned)nslots;
  // Placement of the slots' tiles in the block index (see launch_chain): slot-interleaved,
  // block b -> slot b % nslots at position b / nslots, or row-major, the blocks of a slot
  // consecutive (slot b / wgs_per_slot at position b % wgs_per_slot).  One division either
  // way.
  const unsigned pl_div = row_major ? (unsigned)wgs_per_slot : (unsigned)nslots;
  const unsigned pl_quo = blockIdx.x / pl_div, pl_rem = blockIdx.x - pl_quo * pl_div;
  const int slot = (int)(row_major ? pl_quo : pl_rem);
  uint64_t* sc = ws + kHeaderWords + kSlotWords * slot;
  const int64_t rows_in_slot = (E - slot + nslots - 1) / nslots;
  const uint64_t tiles_in_slot = (uint64_t)rows_in_slot * (uint64_t)tiles_per_row;
  // The workgroup's tile, from its block index: slot, then position in the slot's scan
  // order (lower block indices first, so a tile's predecessors are normally dispatched
  // before it; the look-back does not rely on that).
  const uint64_t q_t = row_major ? pl_rem : pl_quo;

  // The slot's epoch is read first and used once the tile's loads are in flight.  Every
  // workgroup counts itself in the slot's counter once it has the epoch.  The one that
  // completes the count has then seen every workgroup of the slot read the epoch: once its
  // tile's look-back is done (the count's result is back long before) it resets the count
  // and advances the slot's epoch for the next call.
  //
  // "Once it has the epoch" is a data dependency, not an assumption about the schedule: the
  // count's increment is computed from the loaded epoch word (1 + its upper half, which is
  // always 0: the word holds an epoch below 2^30), so the atomic cannot issue before the
  // load has returned its value.  Without it the two relaxed accesses to different
  // addresses could be performed in either order, and a workgroup whose count came first
  // could read the epoch its slot's last workgroup had already advanced, then tag its
  // status words with the next call's epoch (a silently wrong carry in that call).
  uint64_t e_raw = 0, drawn = 0;
  // A call of one tile per row has no tile that waits on another: it skips the protocol
  // (the epoch, the count, the status words), and leaves the workspace as it found it, so
  // every slot's epoch is still the next call's (1.5-5% faster on such calls, MI355X:
  // TD(lambda) [4096,2560] 31.5 -> 30.1 us, discounted returns [150,10000] 6.56 -> 6.23).
  // Not in the 32768-step instances or the statistics ops, which sit at the VGPR limit:
  // there the check spilled 12 B per lane (prefix sum [8,2^20-1], phased, 19.6 -> 20.1 us).
  constexpr bool kSolo = NT * Q < 8192 && !Op::kBlockStats;
  const bool chained = !kSolo || tiles_per_row > 1;
  if (tid == 0 && chained) e_raw = atomic_ld(sc + 24);
  auto count_drawn = [&]() {
    const uint64_t one = 1 + (e_raw >> 32);
    drawn = __hip_atomic_fetch_add(sc + 16, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (drawn >= wgs_per_slot) atomic_st(ws + 3, (uint64_t)1);  // counters were not at rest
  };
  // It advances the epoch of every slot this call leaves unused whose index falls on its
  // slot modulo nslots as well, so that every call advances all 64 epochs once and they stay
  // equal: a call of another row count maps rows to other slots and other status words, and
  // a word some earlier call left there must not carry a slot's current epoch.
  // Called by all of wave 0 (the count is thread 0's) once its look-back is done: one copy
  // per lane, one store.
  auto advance_slot = [&](uint32_t epoch) {
    if (lane0_u64(drawn) == wgs_per_slot - 1) {
      if (lane == 0) atomic_st(sc + 16, 0);
      const int s2 = slot + lane * nslots;
      if (s2 < kSlots) atomic_st(ws + kHeaderWords + kSlotWords * s2 + 24, (uint64_t)((epoch + 1) & kEpochMask));
    }
  };

  Stats st;  // output statistics (ops with kBlockStats)
  if (q_t < tiles_in_slot) {
    const int64_t lr = (int64_t)(q_t / (uint64_t)tiles_per_row);
    const int jpos = (int)(q_t - (uint64_t)lr * tiles_per_row);
    const int64_t row = slot + (int64_t)nslots * lr;
    const int k_own = FWD ? jpos : tiles_per_row - 1 - jpos;
    // kPhased: the row's element phase ph (phase0 is row 0's) shifts its tiles to the row's
    // four-element boundaries: backward by -ph, so they cover [-ph, tiles*tile - ph) and
    // leave the row's last steps from tiles*tile - ph on (0..3 of them); forward by
    // (4 - ph) % 4, leaving steps 0 .. shift-1.  Those steps come first in scan order: the
    // first tile in scan order takes them as one more quad (pre_t0) ahead of its own,
    // applied to the row's carry.  The tile count stays ceil(T / tile).
    int shift = 0;
    if constexpr (VEC == kPhased) {
      const int ph = (int)(((uint64_t)phase0 + (uint64_t)row * (uint64_t)T) & 3u);
      shift = FWD ? ((4 - ph) & 3) : -ph;
    }
    const int pre_t0 = FWD ? shift - kSeg : tiles_per_row * (NW * WSTEPS) + shift;
    // ... when they hold a step of the row (otherwise the quad would lie wholly outside it)
    const bool pre_live = VEC == kPhased && (FWD ? shift > 0 : pre_t0 < T);
    // Tile k_own, or first a predecessor the look-back hands back (its map computed here,
    // then this tile again from its loads).
    for (int k = k_own, it = 0;; ++it) {
      // lane space -> time: this wave's chunk, and the first step of segment row r
      const int wbase = (k * NW + (FWD ? wave : NW - 1 - wave)) * WSTEPS + shift;
      const int lt = FWD ? lane : kWave - 1 - lane;
      auto seg_t0 = [&](int r) { return wbase + ((FWD ? r : Q - 1 - r) * kWave + lt) * kSeg; };

      // loads: Q segments, plus the neighbour step before the chunk in scan order
      Regs R[Q];
#pragma unroll
      for (int r = 0; r < Q; ++r) op.template load<kSeg, VEC>(row, seg_t0(r), T, R[r]);
      Halo edge{};
      if constexpr (HAS_HALO) {
        if (lane == 0 && (FWD ? wbase > 0 : wbase + WSTEPS < T))
          edge = op.halo_load(row, clamp_step(FWD ? wbase - 1 : wbase + WSTEPS, T), T);
      }
      const bool first = FWD ? (k == 0) : (k == tiles_per_row - 1);
      State rc = (first && wave == 0) ? row_carry(op, row, T) : State{};
      [[maybe_unused]] Regs Rp;  // kPhased: the steps ahead of the row's tiles (below)
      if (it == 0 && tid == 0 && chained) {  // the epoch load was issued before the tile's loads
        s_epoch = (uint32_t)e_raw & kEpochMask;
        count_drawn();
      }

#pragma unroll
      for (int r = 0; r < Q; ++r) op.template prepare<kSeg, VEC>(R[r], row, seg_t0(r), T);

      // neighbour step of each segment (the one before it in scan order): the previous lane,
      // lane 63 of the previous segment row, or the edge load
      Halo h[Q];
#pragma unroll
      for (int r = 0; r < Q; ++r) {
        if constexpr (HAS_HALO) {
          const Halo prev = lane_prev(scan_export<Op, kSeg>(op, R[r]));
          const Halo wrap = r > 0 ? lane_bcast(scan_export<Op, kSeg>(op, R[r > 0 ? r - 1 : 0]), kWave - 1) : edge;
          h[r] = lane == 0 ? wrap : prev;
        }
      }

      Map steps[Q][kSeg];
      Map m[Q];
      Map rowagg[Q];  // map of each segment row (wave-uniform)
#pragma unroll
      for (int r = 0; r < Q; ++r) {
        op.template coef<kSeg, VEC>(R[r], h[r], row, seg_t0(r), T, steps[r]);
        m[r] = lane_scan(fold_segment<FWD, kSeg>(steps[r]), kWave);
        rowagg[r] = lane_bcast(m[r], kWave - 1);
      }
      if constexpr (VEC == kPhased) {
        // The steps ahead of the row's tiles (pre_t0), on every lane of wave 0 alike: the
        // row's carry through them, and their outputs, stored by lane 0 of the tile's own
        // workgroup.  Loaded here, after the tile's coefficients: loaded with the tile's
        // own loads, the quad's registers stayed live across them and the 1024-thread
        // instances spilled 20-68 B per lane; here it costs wave 0 of one tile per row one
        // load's latency (prefix sum [8,2^20-1] 20.59 -> 19.55 us, GAE [64,40001]
        // 19.41 -> 17.52 us on MI355X).
        if (first && wave == 0 && pre_live) {
          op.template load<kSeg, VEC>(row, pre_t0, T, Rp);
          op.template prepare<kSeg, VEC>(Rp, row, pre_t0, T);
          Halo hp{};
          if constexpr (HAS_HALO) hp = op.halo_load(row, clamp_step(FWD ? pre_t0 - 1 : pre_t0 + kSeg, T), T);
          Map sp[kSeg];
          op.template coef<kSeg, VEC>(Rp, hp, row, pre_t0, T, sp);
          State xp[kSeg];
          replay<FWD, kSeg>(sp, rc, xp);
          if (k == k_own && lane == 0) op.template emit<kSeg, VEC, SP>(Rp, hp, xp, rc, row, pre_t0, T);
          rc = fold_segment<FWD, kSeg>(sp).apply(rc);
        }
      }
      // the chunk's map: segment rows composed in scan order
      Map wm = Map::identity();
#pragma unroll
      for (int r = 0; r < Q; ++r) wm = compose(rowagg[r], wm);
      if (lane == 0) s_map[wave] = wm;
      __syncthreads();
      const uint32_t epoch = s_epoch;
      if (wave == 0) {
        // The wave maps' inclusive prefixes by one lane scan (lane v: waves 0..v), kept in
        // LDS, so that a wave's entering state is one application once the tile's carry is
        // known instead of a chain through the waves before it (prefix sum [8,2^20]
        // 19.18 -> 18.96 us, discounted returns [3,500000] 7.65 -> 7.40 us on MI355X).
        Map pm = lane < NW ? s_map[lane < NW ? lane : 0] : Map::identity();
        pm = lane_scan(pm, NW);
        if (lane < NW) s_pref[lane] = pm;
        const Map tm = lane_bcast(pm, NW - 1);
        if (!chained) {  // the row's own carry
          if (lane == 0) {
            s_carry = rc;
            s_next = -1;
          }
        } else if (k != k_own) {
          publish_for<FWD>(tm, rc, row, k, tiles_per_row, epoch, fb, lane);
          if (lane == 0) s_next = k_own;
        } else {
          int need;
          const State c = tile_carry<FWD>(tm, rc, row, k, tiles_per_row, epoch, ws, fb, lane,
                                          spin_limit, fallback_polls, need);
          if (lane == 0) {
            s_carry = c;
            s_next = need;
          }
        }
        if (it == 0 && chained) advance_slot(epoch);  // after the look-back: off its path
      }
      __syncthreads();
      const int next = s_next;
      if (k != k_own || next >= 0) {
        k = k != k_own ? k_own : next;
        continue;
      }
      // state entering this wave's chunk, then each segment row, then each lane
      State carry = s_carry;
      if (wave > 0) carry = s_pref[wave > 0 ? wave - 1 : 0].apply(carry);
#pragma unroll
      for (int r = 0; r < Q; ++r) {
        State x_in = lane_prev(m[r].apply(carry));
        if (lane == 0) x_in = carry;
        carry = rowagg[r].apply(carry);
        State xs[kSeg];
        replay<FWD, kSeg>(steps[r], x_in, xs);
        op.template emit<kSeg, VEC, SP>(R[r], h[r], xs, x_in, row, seg_t0(r), T);
        if constexpr (Op::kBlockStats) op.template stats<kSeg>(R[r], xs, seg_t0(r), T, st);
      }
      break;
    }
  } else if (wave == 0 && chained) {  // a slot with fewer rows than the fullest: only the count
    if (tid == 0) count_drawn();
    advance_slot((uint32_t)lane0_u64(e_raw) & kEpochMask);
  }
  if constexpr (Op::kBlockStats) block_stats<NT>(st, op.partials);
}

}  // namespace rlk
