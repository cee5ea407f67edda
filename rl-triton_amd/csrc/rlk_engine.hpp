// rlk_engine.hpp -- the scan engine shared by every rl_triton estimator on gfx950.
//
// Every estimator is one done-masked linear recurrence over a row of T steps,
//     backward:  x[t] = add[t] + mul[t] * x[t+1],   x[T]  = carry   (GAE, V-trace, ...)
//     forward:   x[t] = add[t] + mul[t] * x[t-1],   x[-1] = carry   (traces, prefix sum)
// evaluated as a scan over affine maps m(x) = add + mul * x.  Composition:
//     (m1 o m2)(x) = m1.add + m1.mul * m2.add  +  (m1.mul * m2.mul) * x.
//
// Work decomposition (rows are contiguous, row-major [E, T] fp32):
//   * a thread owns S consecutive steps of one row ("segment") and keeps its
//     inputs in registers; it folds them into one affine map serially;
//   * L threads (L = 2^k) form a row tile of L*S steps; their maps are combined by a
//     wavefront shuffle scan (width min(L, 64)) and, when L > 64, through LDS;
//   * short rows: a workgroup of NT threads holds NT/L whole rows, no inter-workgroup
//     traffic;
//   * long rows: a row is split into tiles of NTD*S steps, handed out by per-slot atomic
//     tickets in scan order to a persistent grid and chained by a decoupled look-back over
//     per-tile status words in a caller-provided workspace; a coordinator wave per
//     workgroup does the look-back while the data waves prefetch the next tile.
//
// An estimator ("Op") supplies:
//   Regs                      per-thread registers for S steps
//   load(row, t0, T, R)       issue the segment's loads: unconditional, raw, nothing
//                             computed from them (see load_seg)
//   prepare(R, row, t0, T)    everything derived from the loaded values (exp, ratios,
//                             bootstrap selection), run when the tile is processed
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

struct Affine {
  float mul;
  float add;
};

__device__ __forceinline__ Affine compose(Affine outer, Affine inner) {
  // outer(inner(x))
  return Affine{outer.mul * inner.mul, fmaf(outer.mul, inner.add, outer.add)};
}

struct NoHalo {};

// ---------------------------------------------------------------------------------------
// Segment loads / stores.  VEC: T % 4 == 0 and every base pointer 16-byte aligned, so a
// segment start t0 (a multiple of 4) is 16-byte aligned and each quad is all-in or all-out.
//
// Loads are unconditional and raw: a step beyond T reads the row's last quad (or step),
// and nothing is computed from the loaded values until the op's prepare() -- padding
// steps are masked to the identity map in coef() and their stores go to the sink, so
// their register contents never matter.  Every lane then issues the same memory
// instructions in every tile, and no instruction touches a prefetched register before the
// tile is processed, so the look-back kernel's prefetch really stays in flight (vector
// loads return in order; a load under a branch, or an early use, forces an early wait).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int clamp_step(int t, int T) { return t < 0 ? 0 : (t < T ? t : T - 1); }

template <int S, bool VEC>
__device__ __forceinline__ void load_seg(const float* __restrict__ p, int t0, int T, float (&v)[S]) {
  if constexpr (VEC) {
    static_assert(S % 4 == 0, "vector segments hold whole quads");
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      const float4 f = *reinterpret_cast<const float4*>(p + (t < T ? t : T - 4));
      v[4 * q + 0] = f.x;
      v[4 * q + 1] = f.y;
      v[4 * q + 2] = f.z;
      v[4 * q + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < S; ++i) v[i] = p[t0 + i < T ? t0 + i : T - 1];
  }
}

// sink == nullptr: steps beyond T are skipped.  Otherwise every quad (step) is stored and
// those beyond T go to the lane's own 16-byte slot of `sink` (kSinkWords of scratch), so
// that the number of memory instructions does not depend on the tile either.
template <int S, bool VEC>
__device__ __forceinline__ void store_seg(float* __restrict__ p, int t0, int T, const float (&v)[S],
                                          float* sink) {
  float* const slot = sink ? sink + 4 * __lane_id() : nullptr;
  if constexpr (VEC) {
#pragma unroll
    for (int q = 0; q < S / 4; ++q) {
      const int t = t0 + 4 * q;
      const float4 f = make_float4(v[4 * q + 0], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
      if (slot) *reinterpret_cast<float4*>(t < T ? p + t : slot) = f;
      else if (t < T) *reinterpret_cast<float4*>(p + t) = f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < S; ++i) {
      if (slot) *(t0 + i < T ? p + t0 + i : slot) = v[i];
      else if (t0 + i < T) p[t0 + i] = v[i];
    }
  }
}

// A 0.0f that is never written: the source of an unconditional load whose operand is absent.
// Global (not __constant__) memory, so that selecting between it and a global operand keeps
// a global load: a flat load would count against the LDS counter too and make the next LDS
// wait drain the whole prefetch.
__device__ float g_zero[4] = {0.f, 0.f, 0.f, 0.f};

// Bootstrap argument shared by the backward estimators: none, one value per row, or
// one value per step (the reference's last_value / bootstrap_values pair).
enum BootMode : int { kBootNone = 0, kBootRow = 1, kBootFull = 2 };

// Address of boot(T-1) for `row` (g_zero when there is no bootstrap).
__device__ __forceinline__ const float* boot_last(const float* boot, int mode, int64_t row, int T) {
  return mode == kBootFull ? boot + row * (int64_t)T + (T - 1)
       : mode == kBootRow  ? boot + row
                           : g_zero;
}

// The bootstrap in two halves, load (raw, unconditional) and prepare:
//   PER_STEP = false: the caller only uses boot(T-1) (no truncations), so only that value
//                     is read (a per-step array at its last column);
//   PER_STEP = true:  a per-step array is read in full; with a per-row value (or none) the
//                     segment loads read `any_row` (any readable [T] row) and are discarded.
// boot_prepare turns the raw registers into bt[i] = boot(t0 + i).
template <int S, bool VEC, bool PER_STEP>
__device__ __forceinline__ void boot_load(const float* __restrict__ boot, int mode, int64_t row,
                                          int t0, int T, float (&seg)[S], float& last,
                                          const float* any_row) {
  last = *boot_last(boot, mode, row, T);
  if constexpr (PER_STEP) load_seg<S, VEC>(mode == kBootFull ? boot + row * (int64_t)T : any_row, t0, T, seg);
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
template <class Op>
__device__ __forceinline__ float row_carry(const Op& op, int64_t row, int T) {
  const float* src = op.row_carry_src(row, T);
  return src ? *src : 0.f;
}

// ---------------------------------------------------------------------------------------
// Lane shuffles of a halo value (float or a small struct of floats).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float shfl_next(float v) { return __shfl_down(v, 1, kWave); }
__device__ __forceinline__ float shfl_prev(float v) { return __shfl_up(v, 1, kWave); }

struct Halo2 {
  float a, b;
};
__device__ __forceinline__ Halo2 shfl_next(Halo2 h) { return Halo2{shfl_next(h.a), shfl_next(h.b)}; }
__device__ __forceinline__ Halo2 shfl_prev(Halo2 h) { return Halo2{shfl_prev(h.a), shfl_prev(h.b)}; }

// Inclusive scan of affine maps across groups of W lanes (W a power of two <= 64).
// Backward (FWD=false): lane i ends up with m_i o m_{i+1} o ... o m_{W-1} of its group.
// Forward  (FWD=true):  lane i ends up with m_i o m_{i-1} o ... o m_0.
template <bool FWD>
__device__ __forceinline__ Affine group_scan(Affine m, int W) {
  const int li = __lane_id() & (W - 1);
  for (int d = 1; d < W; d <<= 1) {
    float omul, oadd;
    bool ok;
    if constexpr (FWD) {
      omul = __shfl_up(m.mul, d, W);
      oadd = __shfl_up(m.add, d, W);
      ok = li >= d;
    } else {
      omul = __shfl_down(m.mul, d, W);
      oadd = __shfl_down(m.add, d, W);
      ok = li + d < W;
    }
    if (ok) m = compose(m, Affine{omul, oadd});
  }
  return m;
}

// ---------------------------------------------------------------------------------------
// Decoupled look-back status words.  Per tile two 64-bit words {tag:32 | value:32}:
//   word0 = AGG: mul   or INC: x at the tile's outgoing edge
//   word1 = AGG: add
// tag = (epoch << 2) | kind, kind 1 = AGG, 2 = INC.  A word whose epoch differs from the
// current call's is "not yet published", so the workspace needs clearing only once.
//
// Workspace (uint64 words), the same layout for every shape so that one buffer serves
// calls of any shape in stream order:
//   header   [0..7]               [1] finished-slot counter, [2] epoch of the call,
//                                 [3] error flag (a bounded wait gave up, or counters were
//                                 not at rest); others reserved
//   slots    [8 + 32*s], s < 64   ticket counter slot s (256 bytes each): +0 ticket,
//                                 +16 finished-workgroup counter (its own 128-byte line)
//   sink     [8 + 32*64, +128)    1 KB that takes the stores of steps beyond T (garbage)
//   status   [8 + 32*64 + 128...] two words per tile, tiles of row r at r*tiles_per_row
// Device-scope atomics on one address serialise (~12 ns each on MI355X), so tickets come
// from up to 64 counters: row r draws from slot r % 64, and since a tile only ever waits
// on tiles of its own row, handing out each slot's tiles in scan order is enough for
// forward progress.  The epoch is global and advances once per call, after every slot
// has finished, so a status word left by any earlier call never matches the current one.
// ---------------------------------------------------------------------------------------
constexpr int kHeaderWords = 8;
constexpr int kSlots = 64;
constexpr int kSlotWords = 32;
constexpr int kSinkOffset = kHeaderWords + kSlots * kSlotWords;
constexpr int kSinkWords = 128;  // 64 lanes x 16 bytes
constexpr int kStatusOffset = kSinkOffset + kSinkWords;
constexpr uint32_t kAgg = 1, kInc = 2;
constexpr uint32_t kEpochMask = 0x3fffffffu;
constexpr int kSpinLimit = 1 << 20;  // polls before a wait gives up (~1 s), never reached when correct

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

// Issue the loads of this thread's segment, and of the neighbour step for the edge lane
// whose neighbour lives outside its wave, together: the edge lane must not pay a second
// memory round trip after its segment has arrived.
//   UNIFORM = false: only the edge lane loads the neighbour step, when it exists.
//   UNIFORM = true:  every lane loads it (one wave-uniform address, clamped into the row),
//                    so the instruction stream does not depend on the lane or the tile.
template <class Op, int S, bool VEC, bool UNIFORM>
__device__ __forceinline__ void load_segment(const Op& op, int64_t row, int t0, int T, int lane,
                                             typename Op::template Regs<S>& R,
                                             typename Op::Halo& edge) {
  if constexpr (!std::is_same<typename Op::Halo, NoHalo>::value) {
    if constexpr (UNIFORM) {
      const int te = Op::kForward ? t0 - lane * S - 1 : t0 + (kWave - lane) * S;
      edge = op.halo_load(row, clamp_step(te, T), T);
    } else if constexpr (Op::kForward) {
      if (lane == 0 && t0 > 0) edge = op.halo_load(row, t0 - 1, T);
    } else {
      if (lane == kWave - 1 && t0 + S < T) edge = op.halo_load(row, t0 + S, T);
    }
  }
  op.template load<S, VEC>(row, t0, T, R);
}

// The neighbour step's data: from the adjacent lane, or the edge load.
template <class Op, int S>
__device__ __forceinline__ typename Op::Halo neighbour(const Op& op,
                                                       const typename Op::template Regs<S>& R,
                                                       typename Op::Halo edge, int lane, int t0,
                                                       int T) {
  typename Op::Halo h{};
  if constexpr (!std::is_same<typename Op::Halo, NoHalo>::value) {
    if constexpr (Op::kForward) {
      h = shfl_prev(op.template export_last<S>(R));
      if (lane == 0 && t0 > 0) h = edge;
    } else {
      h = shfl_next(op.template export_first<S>(R));
      if (lane == kWave - 1 && t0 + S < T) h = edge;
    }
  }
  return h;
}

// The segment's map: steps composed in scan order.
template <bool FWD, int S>
__device__ __forceinline__ Affine fold_segment(const float (&mul)[S], const float (&add)[S]) {
  Affine m{1.f, 0.f};
  if constexpr (FWD) {
#pragma unroll
    for (int i = 0; i < S; ++i) m = compose(Affine{mul[i], add[i]}, m);
  } else {
#pragma unroll
    for (int i = S - 1; i >= 0; --i) m = compose(Affine{mul[i], add[i]}, m);
  }
  return m;
}

// Every step's value from the value entering the segment.
template <bool FWD, int S>
__device__ __forceinline__ void replay(const float (&mul)[S], const float (&add)[S], float x_in,
                                       float (&xs)[S]) {
  float x = x_in;
  if constexpr (FWD) {
#pragma unroll
    for (int i = 0; i < S; ++i) xs[i] = x = fmaf(mul[i], x, add[i]);
  } else {
#pragma unroll
    for (int i = S - 1; i >= 0; --i) xs[i] = x = fmaf(mul[i], x, add[i]);
  }
}

// The value entering each lane's segment, given the value entering its group of W lanes
// (`carry`) and the lane's inclusive group-scan map `m`: the neighbour lane's outgoing value.
template <bool FWD>
__device__ __forceinline__ float lane_input(Affine m, float carry, int lane, int W) {
  const float y = fmaf(m.mul, carry, m.add);
  const int gl = lane & (W - 1);
  float x_in;
  if constexpr (FWD) {
    x_in = __shfl_up(y, 1, kWave);
    if (gl == 0) x_in = carry;
  } else {
    x_in = __shfl_down(y, 1, kWave);
    if (gl == W - 1) x_in = carry;
  }
  return x_in;
}

// ---------------------------------------------------------------------------------------
// Short rows: a workgroup of NT threads holds NT/L whole rows of L threads each
// (L = 2^log2L, L*S >= T).  Launch: grid = ceil(E / (NT/L)).
// ---------------------------------------------------------------------------------------
template <class Op, int NT, int S, bool VEC>
__global__ __launch_bounds__(NT) void rows_kernel(const Op op, int64_t E, int T, int log2L) {
  constexpr bool FWD = Op::kForward;
  constexpr int NW = NT / kWave;
  using Regs = typename Op::template Regs<S>;
  using Halo = typename Op::Halo;
  __shared__ float s_mul[NW], s_add[NW];

  const int tid = threadIdx.x;
  const int lane = __lane_id();
  const int wave = tid / kWave;
  const int L = 1 << log2L;
  const int W = L < kWave ? L : kWave;
  const int li = tid & (L - 1);
  const int64_t row_id = (int64_t)blockIdx.x * (NT >> log2L) + (tid >> log2L);
  const bool active = row_id < E;
  const int64_t row = active ? row_id : E - 1;  // idle lanes of the last workgroup read a real row
  const int t0 = li * S;

  Regs R;
  Halo edge{};
  load_segment<Op, S, VEC, false>(op, row, t0, T, lane, R, edge);
  float carry = row_carry(op, row, T);
  op.template prepare<S, VEC>(R, row, t0, T);
  const Halo h = neighbour<Op, S>(op, R, edge, lane, t0, T);

  float mul[S], add[S];
  op.template coef<S>(R, h, row, t0, T, mul, add);
  const Affine m = group_scan<FWD>(fold_segment<FWD, S>(mul, add), W);

  if (L > kWave) {
    // rows spanning several waves: combine the wave aggregates of the row through LDS
    if (lane == (FWD ? kWave - 1 : 0)) {
      s_mul[wave] = m.mul;
      s_add[wave] = m.add;
    }
    __syncthreads();
    const int wpr = L / kWave;
    const int first = (wave / wpr) * wpr, last = first + wpr - 1;
    if constexpr (FWD) {
      for (int v = first; v < wave; ++v) carry = fmaf(s_mul[v], carry, s_add[v]);
    } else {
      for (int v = last; v > wave; --v) carry = fmaf(s_mul[v], carry, s_add[v]);
    }
  }
  const float x_in = lane_input<FWD>(m, carry, lane, W);
  float xs[S];
  replay<FWD, S>(mul, add, x_in, xs);
  if (active) op.template emit<S, VEC>(R, h, xs, x_in, row, t0, T, nullptr);
}

// ---------------------------------------------------------------------------------------
// Long rows: rows split into tiles of NTD*S steps chained by a decoupled look-back.
//
// Persistent and software-pipelined: a workgroup keeps drawing tiles from its slot's
// ticket counter (slot = blockIdx % nslots, nslots = min(E, 64); each slot hands out the
// tiles of rows r = slot (mod nslots) in scan order) and works one tile ahead.  A
// workgroup only ever waits on tiles with smaller tickets of its own slot, whose holders
// are running, so any grid size makes progress.  Launch: grid = nslots * wgs_per_slot,
// block = NTD + 64.
//
// Roles.  Vector loads of one wave complete in order, so a wave that polls status words
// behind its own prefetch waits for the prefetch too.  Wave 0 is therefore a coordinator
// that holds no tile data: it draws tickets, publishes the tile's status and looks back,
// and its memory queue holds nothing else.  The NTD/64 data waves prefetch the next tile,
// scan the current one, and replay and store it once the coordinator has its carry; all
// their loads and stores are unconditional (clamped, or sent to the sink), so the next
// tile's loads stay in flight across the look-back.
// ---------------------------------------------------------------------------------------
__host__ __device__ inline int lookback_slots(int64_t E) { return E < kSlots ? (int)E : kSlots; }

// Last act of a look-back workgroup: count it finished in its slot; the slot's last one
// leaves the slot at rest, and the last slot to finish advances the epoch.
__device__ __forceinline__ void lookback_finish(uint64_t* ws, uint64_t* sc, uint64_t wgs_per_slot,
                                                int nslots, uint32_t epoch) {
  const uint64_t fin =
      __hip_atomic_fetch_add(sc + 16, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (fin == wgs_per_slot - 1) {
    atomic_st(sc + 0, 0);
    atomic_st(sc + 16, 0);
    const uint64_t slots_done =
        __hip_atomic_fetch_add(ws + 1, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (slots_done == (uint64_t)nslots - 1) {
      atomic_st(ws + 1, 0);
      atomic_st(ws + 2, (uint64_t)((epoch + 1) & kEpochMask));
    }
  }
}

__device__ __forceinline__ uint64_t draw_ticket(uint64_t* sc) {
  return __hip_atomic_fetch_add(sc, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// s_waitcnt vmcnt(0): the coordinator's own traffic is complete before its path rejoins
// the data waves', so nothing it issued looks pending to the compiler afterwards.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Carry entering tile k of `row` (the coordinator wave, all 64 lanes): publish the tile's
// map and look back.  Predecessors are read 64 at a time (lane i <-> i+1 tiles away).
// Once the nearest published inclusive value X has only aggregates between it and this
// tile, they are applied to X one at a time, nearest last, so every published X equals the
// sequential chain X_k = fma(A_k, X_{k+1}, B_k) however far the look-back reached: results
// are bit-reproducible.  A bounded wait gives up (error flag, carry 0) rather than hang.
// The first tile of a row (in scan order) takes `row_c`, the row's own carry.
template <bool FWD>
__device__ __forceinline__ float tile_carry(Affine tm, float row_c, int64_t row, int k,
                                            int tiles_per_row, uint32_t epoch, uint64_t* ws,
                                            int lane) {
  uint64_t* st = ws + kStatusOffset + 2 * (row * (int64_t)tiles_per_row);
  const uint32_t tag_agg = (epoch << 2) | kAgg, tag_inc = (epoch << 2) | kInc;
  if (FWD ? (k == 0) : (k == tiles_per_row - 1)) {
    wait_vmem();
    if (lane == 0) atomic_st(st + 2 * k, pack(tag_inc, fmaf(tm.mul, row_c, tm.add)));
    return row_c;
  }
  if (lane == 0) {
    if (tm.mul == 0.f) {
      // the tile's outgoing value does not depend on its carry
      atomic_st(st + 2 * k, pack(tag_inc, tm.add));
    } else {
      atomic_st(st + 2 * k + 1, pack(tag_agg, tm.add));
      atomic_st(st + 2 * k, pack(tag_agg, tm.mul));
    }
  }
  float c = 0.f;
  for (int spins = 0;; ++spins) {
    const int jj = FWD ? k - 1 - lane : k + 1 + lane;
    const bool inr = FWD ? (jj >= 0) : (jj < tiles_per_row);
    uint32_t kind = 0;
    float v0 = 1.f, v1 = 0.f;
    if (inr) {
      // Both words in flight at once.  word1 is written once per call, before word0's AGG,
      // so a current-epoch AGG word0 with a current-epoch word1 is a consistent (mul, add)
      // pair; a stale word1 just means "not yet".
      const uint64_t w0 = atomic_ld(st + 2 * jj);
      const uint64_t w1 = atomic_ld(st + 2 * jj + 1);
      const uint32_t tag0 = (uint32_t)(w0 >> 32);
      v0 = __uint_as_float((uint32_t)w0);
      if ((tag0 >> 2) == epoch) kind = tag0 & 3u;
      if (kind == kAgg) {
        if ((uint32_t)(w1 >> 32) == tag_agg) v1 = __uint_as_float((uint32_t)w1);
        else kind = 0;
      }
    }
    const uint64_t inc_mask = __ballot(kind == kInc);
    const uint64_t bad_mask = __ballot(kind == 0);
    const int first_inc = inc_mask ? __ffsll((long long)inc_mask) - 1 : kWave;
    const int first_bad = bad_mask ? __ffsll((long long)bad_mask) - 1 : kWave;
    if (first_inc < first_bad) {
      float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v0), first_inc));
      for (int l = first_inc - 1; l >= 0; --l) {
        const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v0), l));
        const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v1), l));
        x = fmaf(a, x, b);
      }
      c = x;
      break;
    }
    if (spins >= kSpinLimit) {
      if (lane == 0) atomic_st(ws + 3, (uint64_t)1);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  wait_vmem();
  if (lane == 0 && tm.mul != 0.f) atomic_st(st + 2 * k, pack(tag_inc, fmaf(tm.mul, c, tm.add)));
  return c;
}

template <class Op, int NTD, int S, bool VEC>
__global__ __launch_bounds__(NTD + kWave) void lookback_kernel(const Op op, int64_t E, int T,
                                                               int tiles_per_row,
                                                               uint64_t* __restrict__ ws) {
  constexpr bool FWD = Op::kForward;
  constexpr int NWD = NTD / kWave;  // data waves
  static_assert(NTD % kWave == 0, "whole data waves");
  using Regs = typename Op::template Regs<S>;
  using Halo = typename Op::Halo;
  // wave aggregates, double-buffered by tile parity: a data wave may write the next tile's
  // while a slower one still reads this tile's
  __shared__ float s_mul[2][NWD], s_add[2][NWD];
  __shared__ float s_carry;
  __shared__ uint64_t s_q;  // the workgroup's next ticket

  const int tid = threadIdx.x;
  const int lane = __lane_id();
  // wave-uniform as far as the compiler knows: role branches become scalar branches, and a
  // wave never executes (or waits in) the other role's code
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const bool coord = wave == 0;
  const int wd = wave - 1;      // data wave index
  const int d = tid - kWave;    // data thread index
  const int nslots = lookback_slots(E);
  const int slot = (int)(blockIdx.x % (unsigned)nslots);
  const uint64_t wgs_per_slot = gridDim.x / (unsigned)nslots;
  uint64_t* sc = ws + kHeaderWords + kSlotWords * slot;
  const int64_t rows_in_slot = (E - slot + nslots - 1) / nslots;
  const uint64_t tiles_in_slot = (uint64_t)rows_in_slot * (uint64_t)tiles_per_row;
  float* const sink = reinterpret_cast<float*>(ws + kSinkOffset);

  uint32_t epoch = 0;
  if (coord) {
    if (lane == 0) s_q = draw_ticket(sc);
    epoch = (uint32_t)atomic_ld(ws + 2) & kEpochMask;
  }
  __syncthreads();
  uint64_t q = s_q;
  // every workgroup draws exactly one ticket beyond the slot's tiles
  if (tid == 0 && q >= tiles_in_slot + wgs_per_slot) atomic_st(ws + 3, (uint64_t)1);  // not at rest

  // ticket -> (row, tile index in scan order -> tile position k)
  auto decode = [&](uint64_t qq, int64_t& row, int& k) {
    const int64_t lr = (int64_t)(qq / (uint64_t)tiles_per_row);
    const int j = (int)(qq - (uint64_t)lr * tiles_per_row);
    row = slot + (int64_t)nslots * lr;
    k = FWD ? j : tiles_per_row - 1 - j;
  };

  // The two roles run separate loops over the same ticket sequence and meet at two
  // barriers per tile: A (the data waves' aggregates and the next ticket are in LDS) and B
  // (the carry is in LDS).  Neither loop contains the other's memory traffic.  Tickets are
  // drawn one tile ahead, at the top of the coordinator's iteration, so a workgroup holds
  // at most one tile it has not started (a deeper lead lets one slow tile hold up the
  // tiles after it); the next tile's loads are issued right after A and stay in flight
  // across the look-back and this tile's stores.
  int64_t row = 0;
  int k = 0;
  if (q < tiles_in_slot) decode(q, row, k);
  if (coord) {
    for (int parity = 0; q < tiles_in_slot; parity ^= 1) {
      uint64_t qn = ~(uint64_t)0;
      if (lane == 0) qn = draw_ticket(sc);
      const bool first = FWD ? (k == 0) : (k == tiles_per_row - 1);
      const float rc = first ? row_carry(op, row, T) : 0.f;
      wait_vmem();
      if (lane == 0) s_q = qn;
      __syncthreads();  // A
      Affine tm{1.f, 0.f};
      if constexpr (FWD) {
        for (int v = 0; v < NWD; ++v) tm = compose(Affine{s_mul[parity][v], s_add[parity][v]}, tm);
      } else {
        for (int v = NWD - 1; v >= 0; --v) tm = compose(Affine{s_mul[parity][v], s_add[parity][v]}, tm);
      }
      const uint64_t q_next = s_q;
      const float c = tile_carry<FWD>(tm, rc, row, k, tiles_per_row, epoch, ws, lane);
      if (lane == 0) s_carry = c;
      __syncthreads();  // B
      q = q_next;
      if (q < tiles_in_slot) decode(q, row, k);
    }
    if (lane == 0) lookback_finish(ws, sc, wgs_per_slot, nslots, epoch);
    return;
  }

  Regs cur;
  Halo ecur{};
  if (q < tiles_in_slot) load_segment<Op, S, VEC, true>(op, row, (k * NTD + d) * S, T, lane, cur, ecur);
  for (int parity = 0; q < tiles_in_slot; parity ^= 1) {
    const int t0 = (k * NTD + d) * S;
    op.template prepare<S, VEC>(cur, row, t0, T);
    const Halo h = neighbour<Op, S>(op, cur, ecur, lane, t0, T);
    float mul[S], add[S];
    op.template coef<S>(cur, h, row, t0, T, mul, add);
    const Affine m = group_scan<FWD>(fold_segment<FWD, S>(mul, add), kWave);
    if (lane == (FWD ? kWave - 1 : 0)) {
      s_mul[parity][wd] = m.mul;
      s_add[parity][wd] = m.add;
    }
    __syncthreads();  // A
    // prefetch the next tile (this one again when there is none)
    const uint64_t qn = s_q;
    int64_t nrow = row;
    int nk = k;
    if (qn < tiles_in_slot) decode(qn, nrow, nk);
    Regs nxt;
    Halo enxt{};
    load_segment<Op, S, VEC, true>(op, nrow, (nk * NTD + d) * S, T, lane, nxt, enxt);
    __syncthreads();  // B
    float carry = s_carry;
    if constexpr (FWD) {
      for (int v = 0; v < wd; ++v) carry = fmaf(s_mul[parity][v], carry, s_add[parity][v]);
    } else {
      for (int v = NWD - 1; v > wd; --v) carry = fmaf(s_mul[parity][v], carry, s_add[parity][v]);
    }
    const float x_in = lane_input<FWD>(m, carry, lane, kWave);
    float xs[S];
    replay<FWD, S>(mul, add, x_in, xs);
    op.template emit<S, VEC>(cur, h, xs, x_in, row, t0, T, sink);
    cur = nxt;
    ecur = enxt;
    q = qn;
    row = nrow;
    k = nk;
  }
}

}  // namespace rlk
