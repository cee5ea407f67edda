// rlk_capi.hip -- extern "C" entry points of librl_triton_amd.so (declared in
// include/rl_triton_amd.h): argument checks, launch planning and kernel launches.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "rl_triton_amd.h"
#include "rlk_ops.hpp"

namespace rlk {
namespace {

// Launch geometry.
constexpr int kNT = 256;          // short rows: threads per workgroup of small calls (4 wavefronts)
constexpr int kNTWide = 512;      // short rows otherwise (8 wavefronts; one row of 1025..2048
                                  // steps where rows_strided_kernel is not used)
constexpr int kShortMaxT = 2048;  // rows up to this length are kept whole in one workgroup
constexpr int kStridedThreads = 256, kStridedSegments = 2;  // rows_strided_kernel's tile
static_assert(kNTWide >= kShortMaxT / 4, "a short row (up to 512 threads of 4 steps) fits one workgroup");
// Long rows: each op fixes its threads per workgroup (kLongThreads) and the most 4-step
// segments per thread its registers hold without spilling (kLongMaxSegments, 2..8).  The
// smallest tile any op uses sizes the workspace.
constexpr int kMinQ = 2;
constexpr int64_t kMinTile = (int64_t)512 * kSeg * kMinQ;  // 4096 steps

int ceil_log2(int64_t x) {
  int k = 0;
  while ((int64_t{1} << k) < x) ++k;
  return k;
}

// Compute units of the current device (cached per device; 256 on MI355X).  Threads that
// race on the first call store the same value.
int device_cus() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Long rows: segments per thread.  Tiles are as large as the op's registers allow while
// the call still has one tile per compute unit: a longer tile shortens the look-back
// chain along a row, and a tile per CU keeps every CU streaming.
template <class Op>
int long_segments(int64_t E, int64_t T) {
  const int64_t cus = device_cus();
  for (int q = Op::kLongMaxSegments; q > kMinQ; q /= 2) {
    const int64_t tile = (int64_t)Op::kLongThreads * kSeg * q;
    if (E * ((T + tile - 1) / tile) >= cus) return q;
  }
  return kMinQ;
}

// Workspace for a long-row call: two places of status words for its tiles (the tile's own,
// and the one other workgroups publish into), counted at the smallest tile.
int64_t status_tiles(int64_t E, int64_t T) { return E * ((T + kMinTile - 1) / kMinTile); }
size_t workspace_bytes(int64_t E, int64_t T) {
  if (E <= 0 || T <= kShortMaxT) return 0;
  return (size_t)(kStatusOffset + 2 * kStatusWords * status_tiles(E, T)) * sizeof(uint64_t);
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Short rows: S steps per thread, L = 2^ceil(log2(ceil(T/S))) threads per row, NT/L rows
// per workgroup, grid = ceil(E / (NT/L)).
int64_t rows_grid(int64_t E, int64_t T, int S, int NT) {
  const int64_t rows_per_block = NT >> ceil_log2((T + S - 1) / S);
  return (E + rows_per_block - 1) / rows_per_block;
}

// Threads per workgroup of a short-row launch: 512 for rows over 1024 steps (one row per
// workgroup), and for shorter rows whenever 512-thread workgroups still give every compute
// unit one (GAE [4096,128] measured 4.26 -> 4.08 us, TD(lambda) 3.41 -> 3.26 us); 256 for
// smaller calls, which need the finer grid to reach the CUs.
int rows_threads(int64_t E, int64_t T) {
  if (T > 1024) return kNTWide;
  return rows_grid(E, T, 4, kNTWide) >= device_cus() ? kNTWide : kNT;
}

int64_t chain_grid(int64_t E, int64_t T, int NT, int Q) {
  const int64_t tile = (int64_t)NT * kSeg * Q;
  const int64_t nslots = lookback_slots(E);
  return nslots * (((E + nslots - 1) / nslots) * ((T + tile - 1) / tile));
}

// Short rows: steps per segment.  Four (one quad per array per thread) from four steps
// up; rows of 1-3 steps take one step per thread, element by element.
int rows_seg(int64_t T) { return T < 4 ? 1 : 4; }

// Long-row tile shapes (threads x 4-step segments per thread).  Each op has its own thread
// count and largest segment count (kLongThreads, kLongMaxSegments), and long_segments picks
// the largest tile that still gives every CU one.  Three kinds of call change the shape,
// where measured faster on MI355X (A/B twice, same box, both storage types alike so that a
// bfloat16 result stays the float32 result rounded):
//   * discounted returns without truncations (512-thread tiles of up to 8 segments), a call
//     that gives every CU a 16384-step tile: 1024 x 4 instead of 512 x 8, the same tiles
//     ([64,65536] 11.2 -> 10.3 us, [8,2^20] 23.1 -> 22.0 us; C5 [16,131072] keeps 512 x 4,
//     8.12 us, against 8.41 at 1024 x 2);
//   * discounted returns on rows of at least eight 8192-step tiles, whose 8192-step tiles
//     reach half the CUs but not all of them: 1024 x 2 (those tiles) instead of 512 x 2
//     (4096-step tiles, enough for every CU): [2,10^6] 10.3 -> 8.9 us, [3,500000]
//     8.20 -> 7.62 us, [8,200000] 9.15 -> 8.12 us; bfloat16 [3,500000] 7.60 -> 7.00 us.
//     Shorter rows lose to the last tile's padding ([100,10000] 6.19 -> 6.44 us);
//   * 1024-thread ops whose 8192-step tiles (1024 x 2) outnumber the CUs but not twice
//     over: a CU holds one 1024-thread workgroup of these kernels, so the tiles would run in
//     two rounds; 512 x 4 (the same tiles) fits two workgroups per CU.  TD(lambda)
//     [64,40000] 13.17 -> 11.89 us, [96,30000] 13.62 -> 11.92 us (bfloat16 11.53 -> 8.87),
//     [200,10000] 12.12 -> 10.37 us; GAE [64,40000] 17.46 -> 16.16 us, [200,10000]
//     16.16 -> 14.41 us; prefix sum [64,40000] 11.18 -> 8.93 us.  V-trace's registers allow
//     one 512 x 4 workgroup per CU, so it takes 512 x 2 (4096-step tiles, two workgroups
//     per CU): [64,40000] 18.6 -> 16.4 us, [200,10000] 17.2 -> 15.4 us, bfloat16
//     [96,30000] 15.7 -> 15.0 us, float32 [96,30000] 19.4 -> 19.7 us.  (Ops whose tile can
//     double take twice the tile first in these calls, one round of 16384-step tiles,
//     faster still (cu_shape); only V-trace still takes this rule.)
struct LongShape {
  int threads, segments;
};
template <class Op>
struct wide_long_tiles : std::false_type {};
template <class E>
struct wide_long_tiles<ReturnsOp<false, false, E>> : std::true_type {};
// segments per thread of the 512-thread tiles a 1024 x 2 call between one and two tiles
// per CU takes instead (0: keeps 1024 x 2)
template <class Op>
struct half_width_segments : std::integral_constant<int, 0> {};
template <bool TRUNC, class E>
struct half_width_segments<GaeOp<TRUNC, E>> : std::integral_constant<int, 4> {};
template <bool TRUNC, class E>
struct half_width_segments<GaeStatsOp<TRUNC, E>> : std::integral_constant<int, 4> {};
template <bool NV, bool TRUNC, class E>
struct half_width_segments<ReturnsOp<NV, TRUNC, E>> : std::integral_constant<int, (NV || TRUNC) ? 4 : 0> {};
template <class E>
struct half_width_segments<DoneGatedForwardOp<E>> : std::integral_constant<int, 4> {};
template <bool FWD, class E>
struct half_width_segments<AffineScanOp<FWD, E>> : std::integral_constant<int, 4> {};
template <bool TRUNC, class E>
struct half_width_segments<VtraceOp<TRUNC, E>> : std::integral_constant<int, 2> {};

template <class Op>
LongShape cu_shape(int64_t E, int64_t T) {
  const int64_t cus = device_cus();
  auto tiles = [&](int64_t tile) { return E * ((T + tile - 1) / tile); };
  if constexpr (wide_long_tiles<Op>::value) {
    if (tiles(1024 * kSeg * 4) >= cus) return {1024, 4};
    const int64_t t8 = tiles(1024 * kSeg * 2);
    if (T >= 8 * 8192 && t8 < cus && 2 * t8 >= cus) return {1024, 2};
  }
  int q = long_segments<Op>(E, T);
  // More tiles than CUs at that size, fewer at twice the size: the larger tiles, in one
  // round with some CUs idle, beat the smaller ones in two.  Measured on MI355X (the
  // larger tiles' share of the CUs 0.53-0.88, A/B in one process): GAE [150,10000]
  // 13.7 -> 10.3 us, [64,40000] 16.1 -> 14.2, TD(lambda) [160,10000] 10.1 -> 7.6, prefix
  // sum [48,131072] 18.6 -> 14.9, [40,100000] 14.6 -> 12.5.  Calls whose tiles already fit
  // one round keep them ([128,12000], [16,131072]: twice the tile lost 6-25%).
  if (q < Op::kLongMaxSegments) {
    const int64_t tile = (int64_t)Op::kLongThreads * kSeg * q;
    if (tiles(tile) > cus && tiles(2 * tile) < cus) q *= 2;
  }
  // (Below, q == 2 with more 8192-step tiles than CUs is left only to ops whose largest
  // tile that is: V-trace.)
  constexpr int hq = half_width_segments<Op>::value;
  if constexpr (hq != 0) {
    static_assert(Op::kLongThreads == 1024, "a 1024 x 2 call becomes 512 x hq");
    const int64_t t8 = tiles(1024 * kSeg * 2);
    if (q == 2 && t8 > cus && t8 <= 2 * cus) return {512, hq};
  }
  return {Op::kLongThreads, q};
}

inline int64_t tile_steps(LongShape s) { return (int64_t)s.threads * kSeg * s.segments; }

// The long-row tile shape of a call: cu_shape's, then two corrections.
//   * Calls that leave CUs idle even at the op's own smallest tile take 4096-step tiles
//     while those fit one round (below).
//   * Rows much shorter than the tiles.  cu_shape sizes a tile for the CUs and the
//     look-back chain along a row, so a call of many rows of a few thousand steps ran one
//     tile per row that was mostly padding: a 2560-step row in a 32768-step tile, the
//     prefix sum [4096,2560] at 114 us against 22 us for a streaming kernel of its bytes.
//     Where more than a quarter of a row's tile steps would be padding, the call takes the
//     largest of the op's tiles that pads a row by at most a quarter, or else the one that
//     pads it least (the larger on a tie), unless its tiles fit the CUs in one round and
//     the smaller ones would not.
// Tiles of one size run at the op's own thread count, 4096-step tiles at 512 threads; an
// 8192-step tile of a 1024-thread op between one and two tiles per CU takes 512 threads,
// as in cu_shape.
template <class Op>
LongShape long_shape(int64_t E, int64_t T) {
  LongShape sh = cu_shape<Op>(E, T);
  {
    // Fewer tiles than CUs even at the op's own smallest tile (8192 steps for the
    // 1024-thread ops): 4096-step tiles, while those still fit the CUs in one round.  GAE
    // [16,40000] 8.07 -> 6.94 us, V-trace [24,20000] 8.11 -> 6.83, TD(lambda) [16,65536]
    // 6.90 -> 6.52, prefix sum [40,16384] 5.77 -> 5.22; calls that fill the CUs unchanged.
    const int64_t cus = device_cus(), tile = tile_steps(sh);
    const int64_t now = E * ((T + tile - 1) / tile), small = E * ((T + kMinTile - 1) / kMinTile);
    if (tile > kMinTile && now < cus && small > now && small <= cus) sh = {512, kMinQ};
  }
  auto padded = [&](int64_t tile) { return (T + tile - 1) / tile * tile; };
  auto fits = [&](int64_t tile) { return 4 * padded(tile) <= 5 * T; };  // padding <= T / 4
  if (fits(tile_steps(sh))) return sh;
  // the op's tiles, largest first: kLongThreads x q for q = kLongMaxSegments .. kMinQ, then
  // the 4096-step tile of 512 x kMinQ
  int64_t tiles[8];
  int n = 0;
  for (int q = Op::kLongMaxSegments; q >= kMinQ; q /= 2) tiles[n++] = (int64_t)Op::kLongThreads * kSeg * q;
  if (tiles[n - 1] > kMinTile) tiles[n++] = kMinTile;
  int64_t best = tiles[0];
  for (int i = 0; i < n; ++i) {
    if (fits(tiles[i])) {
      best = tiles[i];
      break;
    }
    if (padded(tiles[i]) < padded(best)) best = tiles[i];
  }
  // a call whose tiles fit the CUs in one round keeps them rather than take smaller tiles
  // in more than one
  const int64_t cus = device_cus(), t = E * ((T + best - 1) / best);
  const int64_t t_sh = E * ((T + tile_steps(sh) - 1) / tile_steps(sh));
  if (t_sh <= cus && t > cus) return sh;
  if (best == kMinTile) return {512, kMinQ};
  const LongShape r{Op::kLongThreads, (int)(best / ((int64_t)Op::kLongThreads * kSeg))};
  constexpr int hq = half_width_segments<Op>::value;
  if constexpr (hq != 0) {
    if (r.segments == 2 && t > cus && t <= 2 * cus) return {512, hq};
  }
  return r;
}

// Workgroups of the launch that launch() makes for Op at [E, T] (E, T > 0).
template <class Op>
int64_t launch_grid(int64_t E, int64_t T) {
  if (T > kShortMaxT) {
    const LongShape sh = long_shape<Op>(E, T);
    return chain_grid(E, T, sh.threads, sh.segments);
  }
  if (rows_seg(T) == 1) return rows_grid(E, T, 1, kNT);
  return rows_grid(E, T, 4, rows_threads(E, T));
}

// Ops whose aligned short rows of 65..128 steps run two row groups per thread
// (rows_pair_kernel): in place of a 512-thread workgroup, a 256-thread one whose threads
// each hold a row of the first and of the second half (same grid, half the waves, twice the
// loads in flight per wave).  float32 Retrace (nine arrays per step) gains from it: C4
// [4096,128] 6.55 -> 6.41 us on MI355X.  Elsewhere the second row's scan lengthens each
// wave's path after its loads: GAE [4096,128] 3.81 -> 3.98 us, V-trace 3.99 -> 4.22 us,
// TD(lambda) 3.11 -> 3.18 us, bfloat16 Retrace 4.77 -> 5.20 us; Retrace [8192,64] is
// unchanged (6.39-6.58 us either way).
template <class Op>
struct paired_rows : std::false_type {};
template <int NA, bool TRUNC>
struct paired_rows<RetraceOp<NA, TRUNC, float>> : std::true_type {};

template <class Op, int NT, int S, int VEC, int SP>
hipError_t launch_rows(const Op& op, int64_t E, int T, hipStream_t stream) {
  int log2L = ceil_log2((T + S - 1) / S);
  const int64_t grid = rows_grid(E, T, S, NT);
  if (grid * NT > 0xffffffffLL) return hipErrorInvalidValue;  // launch() splits such calls
  void* args[] = {const_cast<Op*>(&op), &E, &T, &log2L};
  // 4-step rows of 33..2048 steps: the instance whose scan width is fixed
  const void* k = reinterpret_cast<const void*>(&rows_kernel<Op, NT, S, VEC, 0, SP>);
  if constexpr (S == 4 && VEC == kAligned && NT == kNTWide && paired_rows<Op>::value) {
    if (log2L == 5) {
      k = reinterpret_cast<const void*>(&rows_pair_kernel<Op, NT / 2, 32, SP>);
      return hipLaunchKernel(k, dim3((unsigned)grid), dim3(NT / 2), args, 0, stream);
    }
  }
  if constexpr (S == 4) {
    if (log2L == 4) k = reinterpret_cast<const void*>(&rows_kernel<Op, NT, S, VEC, 16, SP>);
    else if (log2L == 5) k = reinterpret_cast<const void*>(&rows_kernel<Op, NT, S, VEC, 32, SP>);
    else if (log2L >= 6) k = reinterpret_cast<const void*>(&rows_kernel<Op, NT, S, VEC, kWave, SP>);
  }
  return hipLaunchKernel(k, dim3((unsigned)grid), dim3(NT), args, 0, stream);
}

// Aligned rows of 1025..2048 steps: one row per 256-thread workgroup, two wave-strided
// segments per thread (rows_strided_kernel), grid = E, for every op but V-trace and
// Retrace, in both storage types (so that a bfloat16 result stays the float32 kernels'
// result rounded).  Against rows_kernel's 512 threads of one segment, on MI355X:
// TD(lambda) [256,2048] 3.47 -> 3.35 us, prefix sum [256,2048] 3.28 -> 3.09 us (bfloat16
// 3.12 -> 3.06), GAE [256,2048] 4.33 -> 4.27 us, TD(lambda) [512,1100] 4.14 -> 4.00 us,
// the other bfloat16 calls unchanged.  V-trace (4.42 -> 4.44 us, bfloat16 3.88 -> 3.99)
// and Retrace (6.66 -> 6.64 us, bfloat16 5.47 -> 5.74) keep rows_kernel, as do
// element-aligned rows ([256,2047] 3.76 -> 3.78 us).
template <class Op>
struct strided_rows : std::true_type {};
template <bool TRUNC, class E>
struct strided_rows<VtraceOp<TRUNC, E>> : std::false_type {};
template <int NA, bool TRUNC, class E>
struct strided_rows<RetraceOp<NA, TRUNC, E>> : std::false_type {};

template <class Op, int SP>
hipError_t launch_strided(const Op& op, int64_t E, int T, hipStream_t stream) {
  static_assert(kStridedThreads * kSeg * kStridedSegments == kShortMaxT, "one row per workgroup");
  if (E * kStridedThreads > 0xffffffffLL) return hipErrorInvalidValue;  // launch() splits such calls
  int unused = 0;
  void* args[] = {const_cast<Op*>(&op), &E, &T, &unused};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rows_strided_kernel<Op, kStridedThreads, kStridedSegments, kAligned, SP>),
                         dim3((unsigned)E), dim3(kStridedThreads), args, 0, stream);
}

// Look-back poll budgets (rlk_debug_lookback): polls before a wait gives up (~1 s), and
// polls before a wait on a predecessor that has published nothing computes it instead.
constexpr int kFallbackPolls = 256;
std::atomic<int> g_spin_limit{kSpinLimit};
std::atomic<int> g_fallback_polls{kFallbackPolls};

// Long rows: one tile of kLongThreads * 4 * Q steps per workgroup, grid = nslots * (tiles
// of the fullest slot) (see chain_kernel in rlk_engine.hpp).
//
// Placement of the tiles in the block index.  By default the slots interleave (block b
// holds a tile of slot b % nslots), so position j of every row is dispatched before
// position j + 1 of any, and with 8 XCDs taking blocks round-robin a row's tiles share one
// XCD.  A call of at most 16 rows whose tiles fill every CU at least once takes the rows
// one after another instead (a row's tiles consecutive, spread over the XCDs).  Measured on
// MI355X, A/B twice in one process, bit-identical results: V-trace [16,131072]
// 13.39 -> 12.50 us, GAE [16,131072] 12.78 -> 11.69, TD(lambda) [16,131072] 9.65 -> 8.86,
// discounted returns [8,262144] 9.18 -> 8.46 and [16,131072] 8.28 -> 8.22, prefix sum
// [16,131072] 8.32 -> 7.80; [8,2^20], [4,2^19..2^21] unchanged.  Where the grid is smaller
// than the chip ([16,65536], [12,131072], [16,40000]) or the rows are many ([32..200] rows)
// the row-major order lost up to 1.35 us (TD(lambda) [96,30000]), so those keep the
// interleave.
inline int chain_row_major(int64_t E, int64_t grid) { return E <= 16 && grid >= device_cus() ? 1 : 0; }

// VEC = kPhased: phase0 = the element phase of row 0's arrays.
template <class Op, int Q, int VEC, int SP, int NT = Op::kLongThreads>
hipError_t launch_chain(const Op& op, int64_t E, int T, uint64_t* ws, hipStream_t stream, int phase0) {
  static_assert(NT * kSeg * Q >= kMinTile, "the workspace is sized for the smallest tile");
  constexpr int64_t tile = (int64_t)NT * kSeg * Q;
  int tpr = (int)((T + tile - 1) / tile);
  const int64_t grid = chain_grid(E, T, NT, Q);
  if (grid * NT > 0xffffffffLL) return hipErrorInvalidValue;  // launch() splits such calls
  uint64_t* fb = ws + kStatusOffset + kStatusWords * status_tiles(E, T);
  int spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  int fallback_polls = g_fallback_polls.load(std::memory_order_relaxed);
  int row_major = chain_row_major(E, grid);
  void* args[] = {const_cast<Op*>(&op), &E, &T, &tpr, &ws, &fb, &spin_limit, &fallback_polls,
                  &row_major, &phase0};
  return hipLaunchKernel(reinterpret_cast<const void*>(&chain_kernel<Op, NT, Q, VEC, SP>),
                         dim3((unsigned)grid), dim3(NT), args, 0, stream);
}

template <class Op, int VEC, int SP>
hipError_t launch_long(const Op& op, int64_t E, int T, uint64_t* ws, hipStream_t stream, int phase0) {
  const LongShape sh = long_shape<Op>(E, T);
  if constexpr (wide_long_tiles<Op>::value) {
    if (sh.threads == 1024 && sh.segments == 4) return launch_chain<Op, 4, VEC, SP, 1024>(op, E, T, ws, stream, phase0);
    if (sh.threads == 1024 && sh.segments == 2) return launch_chain<Op, 2, VEC, SP, 1024>(op, E, T, ws, stream, phase0);
  }
  constexpr int hq = half_width_segments<Op>::value;
  if constexpr (hq != 0) {
    if (sh.threads == 512 && sh.segments == hq) return launch_chain<Op, hq, VEC, SP, 512>(op, E, T, ws, stream, phase0);
  }
  if constexpr (Op::kLongThreads == 1024 && hq != kMinQ) {
    if (sh.threads == 512 && sh.segments == kMinQ) return launch_chain<Op, kMinQ, VEC, SP, 512>(op, E, T, ws, stream, phase0);
  }
  const int q = sh.segments;
  if constexpr (Op::kLongMaxSegments >= 8)
    if (q == 8) return launch_chain<Op, 8, VEC, SP>(op, E, T, ws, stream, phase0);
  if constexpr (Op::kLongMaxSegments >= 4)
    if (q == 4) return launch_chain<Op, 4, VEC, SP>(op, E, T, ws, stream, phase0);
  return launch_chain<Op, 2, VEC, SP>(op, E, T, ws, stream, phase0);
}

// Output stores: non-temporal (the default) or write-through (sc1, store_quad_wt), per
// launch, by what measured faster on MI355X (one process, three builds -- nt, sc1 and
// plain stores -- alternated, 88 op x shape x storage cases; µs, nt -> sc1):
//   * bfloat16 outputs: sc1 everywhere, 1-4% faster in every case but one (Retrace
//     [4096,128], equal): V-trace [4096,128] 3.49 -> 3.34, prefix sum [16,131072]
//     6.77 -> 6.54, TD(lambda) [16,131072] 7.07 -> 6.83;
//   * float32 short rows that span several waves (more than 256 steps) in launches writing
//     at least 1 MB, or launches writing at least 12 MB: sc1, 2-4% (TD(lambda) [256,2048]
//     3.35 -> 3.25, Retrace [256,2048] 6.71 -> 6.49, V-trace [1024,512] 4.38 -> 4.21,
//     V-trace [16384,128] 11.19 -> 10.75); rows of up to 256 steps in smaller launches keep
//     nt (GAE [4096,128] 3.77 against 3.94, V-trace 3.99 against 4.20, GAE [2048,256] 3.83
//     against 3.98), as does GAE [64,512] (128 KB written, 2.25 against 2.27);
//   * float32 long rows: sc1 when the grid is at most one tile per CU, for every op but
//     V-trace and Retrace (discounted returns [16,131072] 8.00 -> 7.86, prefix sum
//     [16,131072] 7.66 -> 7.49, TD(lambda) [8,262144] 8.92 -> 8.79); nt with more tiles
//     (discounted [64,40000] 8.99 against 9.58) and for V-trace ([16,131072] 12.40 against
//     12.70, [256,8192] 11.46 against 12.15).
// Plain stores were never the fastest by more than 3% and lost up to 13% elsewhere.  The
// policy is a kernel template argument (SP), so a non-temporal instance is the same code
// as before write-through stores existed.
template <class Op>
struct n_outputs : std::integral_constant<int, 1> {};
template <bool TRUNC, class E>
struct n_outputs<VtraceOp<TRUNC, E>> : std::integral_constant<int, 2> {};
template <int NA, bool TRUNC, class E>
struct n_outputs<RetraceOp<NA, TRUNC, E>> : std::integral_constant<int, 2> {};
template <bool TRUNC, class E>
struct n_outputs<GaeStatsOp<TRUNC, E>> : std::integral_constant<int, 2> {};
template <bool TRUNC, class E>
struct n_outputs<MaskedGaeStatsOp<TRUNC, E>> : std::integral_constant<int, 2> {};
template <class Op>
struct long_rows_write_through : std::true_type {};
template <bool TRUNC, class E>
struct long_rows_write_through<VtraceOp<TRUNC, E>> : std::false_type {};
template <int NA, bool TRUNC, class E>
struct long_rows_write_through<RetraceOp<NA, TRUNC, E>> : std::false_type {};

enum class Kernel { kRows, kStrided, kChain };
// The policies a kernel can be launched with for an op: bfloat16 outputs and the strided
// rows kernel always write through, float32 V-trace and Retrace long rows never; only the
// policies listed here are instantiated.
template <class Op, Kernel K>
struct store_policies {
  static constexpr bool kBf16 = std::is_same<typename Op::Elem, bf16>::value;
  static constexpr bool kWriteThrough = kBf16 || K != Kernel::kChain || long_rows_write_through<Op>::value;
  static constexpr bool kNonTemporal = !kBf16 && K != Kernel::kStrided;
  static_assert(kWriteThrough || kNonTemporal, "some store policy");
};
template <class Op, Kernel K>
int store_write_through(int64_t E, int64_t T) {
  using P = store_policies<Op, K>;
  if constexpr (!P::kNonTemporal) return 1;
  if constexpr (!P::kWriteThrough) return 0;
  if constexpr (K == Kernel::kChain) return launch_grid<Op>(E, T) <= device_cus() ? 1 : 0;
  const int64_t out_bytes = E * T * (int64_t)sizeof(float) * n_outputs<Op>::value;
  return (((T + 3) / 4 > kWave && out_bytes >= (int64_t{1} << 20)) || out_bytes >= (int64_t{12} << 20)) ? 1 : 0;
}
// rlk_debug_store_policy: -1 the rule above, 0 / 1 non-temporal / write-through wherever
// the launch has an instance of that policy.
std::atomic<int> g_store_policy{-1};

// Calls f(std::integral_constant<int, SP>) with SP the launch's store policy.
template <class Op, Kernel K, class F>
hipError_t dispatch_store_policy(int64_t E, int64_t T, F&& f) {
  using P = store_policies<Op, K>;
  if constexpr (P::kWriteThrough && P::kNonTemporal) {
    const int forced = g_store_policy.load(std::memory_order_relaxed);
    if (forced >= 0 ? forced == 1 : store_write_through<Op, K>(E, T) != 0)
      return f(std::integral_constant<int, 1>{});
    return f(std::integral_constant<int, 0>{});
  } else {
    return f(std::integral_constant<int, P::kWriteThrough ? 1 : 0>{});
  }
}

// Ops that take long rows in the phased access mode: all but Retrace (whose [E, T, A]
// arrays have no common row phase) and the statistics ops of compute_gae_normalized (the
// steps a phased row takes ahead of its tiles would be missing from their statistics).
template <class Op>
struct phased_rows : std::true_type {};
template <int NA, bool TRUNC, class E>
struct phased_rows<RetraceOp<NA, TRUNC, E>> : std::false_type {};
template <bool TRUNC, class E>
struct phased_rows<GaeStatsOp<TRUNC, E>> : std::false_type {};
template <bool TRUNC, class E>
struct phased_rows<MaskedGaeStatsOp<TRUNC, E>> : std::false_type {};

// ---------------------------------------------------------------------------------------
// Calls beyond one launch.  HIP launches at most 2^32 - 1 work-items per grid dimension
// (hip_runtime_api.h, hipLaunchKernel), and every launch here is one-dimensional with at
// most 1024 threads per workgroup.  Rows are independent, so a call whose launch would
// need more than kMaxLaunchBlocks workgroups runs as calls over consecutive row ranges,
// in row order on the same stream, each within the limit.  Short rows reach it from 0.8
// billion steps (3-step rows, 64 per workgroup: 3.2 GB per float32 array) to 8.6 billion,
// long rows from ~4.2 million rows of one tile each: sizes MI355X's 288 GB holds.
// ---------------------------------------------------------------------------------------
constexpr int64_t kMaxLaunchBlocks = ((int64_t{1} << 32) - 1) / 1024;

template <class P>
void skip(P*& p, int64_t n) {
  if (p != nullptr) p += n;
}
// boot: one value per row (RLK_BOOT_ROW) or [E, T] (RLK_BOOT_FULL)
template <class E>
void skip_boot(const E*& boot, int boot_mode, int64_t r0, int64_t T) {
  skip(boot, boot_mode == RLK_BOOT_FULL ? r0 * T : r0);
}

// An op's arrays advanced by r0 rows: [E, T] arrays by r0 * T elements, [E, T, A] ones by
// r0 * T * A, per-row ones by r0.  (The statistics ops' partials are placed by the caller.)
template <bool TR, class E>
void skip_rows(GaeOp<TR, E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.r, n), skip(op.v, n), skip(op.term, n), skip(op.trunc, n), skip(op.out, n);
  skip_boot(op.boot, op.boot_mode, r0, T);
}
template <bool TR, class E>
void skip_rows(GaeStatsOp<TR, E>& op, int64_t r0, int64_t T) {
  skip_rows(static_cast<GaeOp<TR, E>&>(op), r0, T);
  skip(op.returns, r0 * T);
}
template <bool TR, class E>
void skip_rows(MaskedGaeOp<TR, E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.r, n), skip(op.v, n), skip(op.term, n), skip(op.trunc, n), skip(op.mask, n);
  skip(op.out, n);
  skip_boot(op.boot, op.boot_mode, r0, T);
}
template <bool TR, class E>
void skip_rows(MaskedGaeStatsOp<TR, E>& op, int64_t r0, int64_t T) {
  skip_rows(static_cast<MaskedGaeOp<TR, E>&>(op), r0, T);
  skip(op.returns, r0 * T);
}
template <bool TR, class E>
void skip_rows(VtraceOp<TR, E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.lpt, n), skip(op.lpb, n), skip(op.v, n), skip(op.r, n), skip(op.term, n);
  skip(op.trunc, n), skip(op.targets, n), skip(op.adv, n);
  skip_boot(op.boot, op.boot_mode, r0, T);
}
template <int NA, bool TR, class E>
void skip_rows(RetraceOp<NA, TR, E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.pi, n * op.A), skip(op.nq, n * op.A);
  skip(op.mu, n), skip(op.q, n), skip(op.act, n), skip(op.r, n), skip(op.term, n);
  skip(op.trunc, n), skip(op.targets, n), skip(op.adv, n);
}
template <bool NV, bool TR, class E>
void skip_rows(ReturnsOp<NV, TR, E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.r, n), skip(op.nv, n), skip(op.term, n), skip(op.trunc, n), skip(op.out, n);
  skip_boot(op.boot, op.boot_mode, r0, T);
}
template <class E>
void skip_rows(DoneGatedForwardOp<E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.x, n), skip(op.dones, n), skip(op.out, n), skip(op.seed, r0);
}
template <bool FWD, class E>
void skip_rows(AffineScanOp<FWD, E>& op, int64_t r0, int64_t T) {
  const int64_t n = r0 * T;
  skip(op.u, n), skip(op.v, n), skip(op.out, n), skip(op.carry, r0);
}

// Rows per launch of a call: all E when one launch holds the call, else the most rows
// (a multiple of 512 where that is at least 512: whole workgroups of every short-row shape)
// whose launch stays within kMaxLaunchBlocks.
template <class Op>
int64_t rows_per_launch(int64_t E, int64_t T) {
  const int64_t g = launch_grid<Op>(E, T);
  if (g <= kMaxLaunchBlocks) return E;
  int64_t n = (int64_t)((double)E * (double)kMaxLaunchBlocks / (double)g);  // grid ~ rows
  n = n < 1 ? 1 : n > E ? E : n;
  for (const int64_t unit : {int64_t{512}, int64_t{1}}) {
    if (n < unit) continue;
    int64_t m = n / unit * unit;
    while (m > unit && launch_grid<Op>(m, T) > kMaxLaunchBlocks) m -= unit;
    if (launch_grid<Op>(m, T) <= kMaxLaunchBlocks) return m;
  }
  return 1;  // one row of at most 2^30 steps is at most 2^18 tiles
}

// Workgroups of all the launches of a call, following launch()'s row ranges: the
// statistics ops write one partial per workgroup.
template <class Op>
int64_t call_blocks(int64_t E, int64_t T) {
  if (E <= 0 || T <= 0) return 0;
  const int64_t rows = rows_per_launch<Op>(E, T);
  if (rows >= E) return launch_grid<Op>(E, T);
  int64_t total = 0;
  for (int64_t r0 = 0; r0 < E; r0 += rows) total += call_blocks<Op>(rows < E - r0 ? rows : E - r0, T);
  return total;
}

// vec: kAligned access.  phase0 >= 0: the element phase every [E, T] array of the call
// shares at row 0 (common_phase), for the phased access of long rows when T % 4 != 0.
template <class Op>
int launch(const Op& op, int64_t E, int64_t T, bool vec, void* workspace, size_t workspace_bytes_given,
           void* stream, int phase0 = -1) {
  if (E < 0 || T < 0 || T > (int64_t{1} << 30)) return RLK_ERR_INVALID_ARGUMENT;
  if (E == 0 || T == 0) return RLK_OK;
  const int64_t rows = rows_per_launch<Op>(E, T);
  if (rows < E) {
    int64_t blocks = 0;  // the statistics ops' partials of the ranges before this one
    for (int64_t r0 = 0; r0 < E; r0 += rows) {
      const int64_t n = rows < E - r0 ? rows : E - r0;
      Op part = op;
      skip_rows(part, r0, T);
      if constexpr (Op::kBlockStats) part.partials = op.partials + kStatWords * blocks;
      const int ph = phase0 < 0 ? -1 : (int)((phase0 + (r0 & 3) * (T & 3)) & 3);
      const int st = launch(part, n, T, vec, workspace, workspace_bytes_given, stream, ph);
      if (st != RLK_OK) return st;
      blocks += call_blocks<Op>(n, T);
    }
    return RLK_OK;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int Ti = (int)T;
  hipError_t e;
  if (T > kShortMaxT) {
    uint64_t* ws = reinterpret_cast<uint64_t*>(workspace);
    if (ws == nullptr || workspace_bytes_given < workspace_bytes(E, T) || !aligned16(ws))
      return RLK_ERR_WORKSPACE;
    const bool phased = phased_rows<Op>::value && !vec && phase0 >= 0 && T % 4 != 0;
    e = dispatch_store_policy<Op, Kernel::kChain>(E, T, [&](auto sp) {
      constexpr int SP = decltype(sp)::value;
      if constexpr (phased_rows<Op>::value) {
        if (phased) return launch_long<Op, kPhased, SP>(op, E, Ti, ws, s, phase0);
      }
      return vec ? launch_long<Op, kAligned, SP>(op, E, Ti, ws, s, 0)
                 : launch_long<Op, kElementAligned, SP>(op, E, Ti, ws, s, 0);
    });
  } else if (strided_rows<Op>::value && vec && T > kShortMaxT / 2) {
    e = dispatch_store_policy<Op, Kernel::kStrided>(E, T, [&](auto sp) {
      return launch_strided<Op, decltype(sp)::value>(op, E, Ti, s);
    });
  } else {
    e = dispatch_store_policy<Op, Kernel::kRows>(E, T, [&](auto sp) {
      constexpr int SP = decltype(sp)::value;
      if (rows_seg(T) == 1) return launch_rows<Op, kNT, 1, kElementAligned, SP>(op, E, Ti, s);
      if (rows_threads(E, T) == kNT)
        return vec ? launch_rows<Op, kNT, 4, kAligned, SP>(op, E, Ti, s)
                   : launch_rows<Op, kNT, 4, kElementAligned, SP>(op, E, Ti, s);
      return vec ? launch_rows<Op, kNTWide, 4, kAligned, SP>(op, E, Ti, s)
                 : launch_rows<Op, kNTWide, 4, kElementAligned, SP>(op, E, Ti, s);
    });
  }
  return e == hipSuccess ? RLK_OK : RLK_ERR_LAUNCH;
}

// Empty shapes are a successful no-op (their data pointers may be null); negative sizes
// are rejected by launch().
bool is_empty(int64_t E, int64_t T) { return (E == 0 && T >= 0) || (T == 0 && E >= 0); }

bool valid_boot(const void* boot, int mode) {
  if (mode == RLK_BOOT_NONE) return true;
  if (mode == RLK_BOOT_ROW || mode == RLK_BOOT_FULL) return boot != nullptr;
  return false;
}

// Vector segments need every [E, T] array aligned to four elements (absent ones pass).
template <class E>
bool quad_aligned(const E* p) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % (4 * sizeof(E))) == 0;
}
template <class E, class... R>
bool quad_aligned(const E* p, const R*... rest) {
  return quad_aligned(p) && quad_aligned(rest...);
}
// The element phase (address / sizeof(E), mod 4) that every non-null array shares, or -1
// when two differ or one is not element-aligned.  Arrays of one call hold [E, T] rows at
// the same offsets, so a shared phase at row 0 makes every row's phase shared too.
template <class E, class... P>
int common_phase(const P*... ptrs) {
  int ph = -1;
  for (const E* p : {static_cast<const E*>(ptrs)...}) {
    if (p == nullptr) continue;
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    if (a % sizeof(E) != 0) return -1;
    const int q = (int)((a / sizeof(E)) & 3);
    if (ph >= 0 && q != ph) return -1;
    ph = q;
  }
  return ph;
}

// ---------------------------------------------------------------------------------------
// Entry points, one template per estimator over the storage type E (float or bf16); the
// extern "C" functions below instantiate them.
// ---------------------------------------------------------------------------------------
template <class E>
int gae_impl(const E* rewards, const E* values, const E* terminateds, const E* truncateds,
             const E* bootstrap, int boot_mode, E* advantages, int64_t num_envs, int64_t seq_len,
             float gamma, float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !values || !terminateds || !advantages || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const E* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 &&
                   quad_aligned(rewards, values, terminateds, truncateds, advantages) &&
                   (boot_mode != RLK_BOOT_FULL || quad_aligned(bootstrap));
  const int ph = common_phase<E>(rewards, values, terminateds, truncateds, advantages,
                                 boot_mode == RLK_BOOT_FULL ? bootstrap : nullptr);
  if (truncateds) {
    GaeOp<true, E> op{rewards, values, terminateds, truncateds, boot, advantages, boot_mode, gamma,
                      gamma * lambda_};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
  }
  GaeOp<false, E> op{rewards, values, terminateds, nullptr, boot, advantages, boot_mode, gamma,
                     gamma * lambda_};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
}

template <class E>
int gae_masked_impl(const E* rewards, const E* values, const E* terminateds, const E* truncateds,
                    const E* bootstrap, int boot_mode, const E* mask, E* advantages,
                    int64_t num_envs, int64_t seq_len, float gamma, float lambda_,
                    void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !values || !terminateds || !mask || !advantages ||
      !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const E* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 &&
                   quad_aligned(rewards, values, terminateds, truncateds, mask, advantages) &&
                   (boot_mode != RLK_BOOT_FULL || quad_aligned(bootstrap));
  const int ph = common_phase<E>(rewards, values, terminateds, truncateds, mask, advantages,
                                 boot_mode == RLK_BOOT_FULL ? bootstrap : nullptr);
  if (truncateds) {
    MaskedGaeOp<true, E> op{rewards, values, terminateds, truncateds, boot, mask, advantages,
                            boot_mode, gamma, gamma * lambda_};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
  }
  MaskedGaeOp<false, E> op{rewards, values, terminateds, nullptr, boot, mask, advantages,
                           boot_mode, gamma, gamma * lambda_};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
}

// First launches of more workgroups than this have their partials summed by a tree of
// reduce_partials_kernel levels (kReduceSlice triples into one per level) until at most
// this many remain, which normalize_kernel's workgroups then each read.  The crossover,
// measured on MI355X (float32, µs per call): 2048 triples read directly 24.1, through one
// level 24.7 ([32768,128]); 4096 triples 44.9 directly, 42.5 through a level ([65536,128]).
// Against every normalising workgroup reading every triple, the tree takes [2^20,128]
// (65536 triples) from 761 to 630 µs and [16384,2048] from 167 to 139 µs.
constexpr int64_t kDirectParts = 2048;

// Triples of the partials buffer for a first launch of `nparts` workgroups: its own, then
// each tree level's.
int64_t partials_triples(int64_t nparts) {
  int64_t total = nparts;
  for (int64_t n = nparts; n > kDirectParts;) {
    n = (n + kReduceSlice - 1) / kReduceSlice;
    total += n;
  }
  return total;
}

// Partials of compute_gae_normalized: kStatWords doubles per workgroup of the first launch
// and per tree level, for the larger of the two ops' grids (the masked op uses narrower
// long-row tiles).
size_t gae_normalized_partials(int64_t num_envs, int64_t seq_len) {
  if (num_envs <= 0 || seq_len <= 0) return 0;
  const int64_t a = call_blocks<GaeStatsOp<true>>(num_envs, seq_len);
  const int64_t b = call_blocks<MaskedGaeStatsOp<true>>(num_envs, seq_len);
  return (size_t)partials_triples(a > b ? a : b) * kStatWords * sizeof(double);
}

// The two launches of a normalised GAE: `op` (GaeStatsOp or MaskedGaeStatsOp, partials not
// yet set) writes A, the returns and the per-workgroup statistics; normalize_kernel then
// rewrites A as (A - mean) / (std + eps).
template <class StatsOp, class E>
int normalized_launch(StatsOp op, E* advantages, int64_t num_envs, int64_t seq_len, bool vec,
                      float eps, void* workspace, size_t workspace_bytes, void* partials,
                      size_t partials_bytes, void* stream) {
  if (num_envs < 0 || seq_len < 0 || seq_len > (int64_t{1} << 30)) return RLK_ERR_INVALID_ARGUMENT;
  double* parts = reinterpret_cast<double*>(partials);
  const int64_t nparts = call_blocks<StatsOp>(num_envs, seq_len);
  if (parts == nullptr || (reinterpret_cast<uintptr_t>(parts) & 7u) != 0 ||
      partials_bytes < (size_t)partials_triples(nparts) * kStatWords * sizeof(double) ||
      nparts > 0x7fffffffLL)
    return RLK_ERR_WORKSPACE;
  op.partials = parts;
  const int st = launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
  if (st != RLK_OK) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int np = (int)nparts;
  while (np > kDirectParts) {
    const int next = (np + kReduceSlice - 1) / kReduceSlice;
    double* up = parts + kStatWords * (int64_t)np;
    void* rargs[] = {&parts, &np, &up};
    if (hipLaunchKernel(reinterpret_cast<const void*>(&reduce_partials_kernel<kReduceNT>),
                        dim3((unsigned)next), dim3(kReduceNT), rargs, 0, s) != hipSuccess)
      return RLK_ERR_LAUNCH;
    parts = up;
    np = next;
  }
  constexpr int kNormNT = 256;
  int64_t n = num_envs * seq_len;
  const bool nvec = n % 4 == 0 && quad_aligned(advantages);
  const int64_t units = nvec ? n / 4 : n;
  int64_t grid = (units + kNormNT - 1) / kNormNT;
  if (grid > 2048) grid = 2048;
  void* args[] = {&advantages, &parts, &np, &n, &eps};
  const void* kernel = nvec ? reinterpret_cast<const void*>(&normalize_kernel<kNormNT, true, E>)
                            : reinterpret_cast<const void*>(&normalize_kernel<kNormNT, false, E>);
  const hipError_t e = hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(kNormNT), args, 0, s);
  return e == hipSuccess ? RLK_OK : RLK_ERR_LAUNCH;
}

// mask == nullptr: every step counts (GaeStatsOp); otherwise the masked op
template <class E>
int gae_normalized_impl(const E* rewards, const E* values, const E* terminateds,
                        const E* truncateds, const E* bootstrap, int boot_mode, const E* mask,
                        E* advantages, E* returns, int64_t num_envs, int64_t seq_len, float gamma,
                        float lambda_, float eps, void* workspace, size_t workspace_bytes,
                        void* partials, size_t partials_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !values || !terminateds || !advantages || !returns ||
      !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const E* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 &&
                   quad_aligned(rewards, values, terminateds, truncateds, mask, advantages,
                                returns) &&
                   (boot_mode != RLK_BOOT_FULL || quad_aligned(bootstrap));
  const float gl = gamma * lambda_;
  auto run = [&](auto op) {
    return normalized_launch(op, advantages, num_envs, seq_len, vec, eps, workspace,
                             workspace_bytes, partials, partials_bytes, stream);
  };
  if (mask) {
    if (truncateds)
      return run(MaskedGaeStatsOp<true, E>{{rewards, values, terminateds, truncateds, boot, mask,
                                             advantages, boot_mode, gamma, gl},
                                            returns, nullptr});
    return run(MaskedGaeStatsOp<false, E>{{rewards, values, terminateds, nullptr, boot, mask,
                                            advantages, boot_mode, gamma, gl},
                                           returns, nullptr});
  }
  if (truncateds)
    return run(GaeStatsOp<true, E>{{rewards, values, terminateds, truncateds, boot, advantages,
                                     boot_mode, gamma, gl},
                                    returns, nullptr});
  return run(GaeStatsOp<false, E>{{rewards, values, terminateds, nullptr, boot, advantages,
                                    boot_mode, gamma, gl},
                                   returns, nullptr});
}

template <class E>
int vtrace_impl(const E* log_pi_target, const E* log_pi_behavior, const E* values,
                const E* rewards, const E* terminateds, const E* truncateds, const E* bootstrap,
                int boot_mode, E* targets, E* advantages, int64_t num_envs, int64_t seq_len,
                float gamma, float rho_bar, float c_bar, void* workspace, size_t workspace_bytes,
                void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!log_pi_target || !log_pi_behavior || !values || !rewards || !terminateds || !targets ||
      !advantages || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const E* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 &&
                   quad_aligned(log_pi_target, log_pi_behavior, values, rewards, terminateds,
                                truncateds, targets, advantages) &&
                   (boot_mode != RLK_BOOT_FULL || quad_aligned(bootstrap));
  const int ph = common_phase<E>(log_pi_target, log_pi_behavior, values, rewards, terminateds,
                                 truncateds, targets, advantages,
                                 boot_mode == RLK_BOOT_FULL ? bootstrap : nullptr);
  if (truncateds) {
    VtraceOp<true, E> op{log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds,
                         boot, targets, advantages, boot_mode, gamma, rho_bar, c_bar};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
  }
  VtraceOp<false, E> op{log_pi_target, log_pi_behavior, values, rewards, terminateds, nullptr,
                        boot, targets, advantages, boot_mode, gamma, rho_bar, c_bar};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
}

template <class E>
int retrace_impl(const E* action_probs_target, const E* action_probs_behavior, const E* q_values,
                 const E* next_q_values_all, const int64_t* actions, const E* rewards,
                 const E* terminateds, const E* truncateds, E* targets, E* advantages,
                 int64_t num_envs, int64_t seq_len, int64_t num_actions, float gamma,
                 float lambda_, float c_bar, float rho_bar, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!action_probs_target || !action_probs_behavior || !q_values || !next_q_values_all ||
      !actions || !rewards || !terminateds || !targets || !advantages || num_actions <= 0 ||
      num_actions > (1 << 20))
    return RLK_ERR_INVALID_ARGUMENT;
  const bool vec = seq_len % 4 == 0 &&
                   quad_aligned(action_probs_target, action_probs_behavior, q_values,
                                next_q_values_all, rewards, terminateds, truncateds, targets,
                                advantages) &&
                   aligned16(actions);
  const int A = (int)num_actions;
#define RLK_RETRACE(NA)                                                                          \
  {                                                                                              \
    if (truncateds) {                                                                            \
      RetraceOp<NA, true, E> op{action_probs_target, action_probs_behavior, q_values,            \
                                next_q_values_all, actions, rewards, terminateds, truncateds,    \
                                targets, advantages, A, gamma, lambda_, c_bar, rho_bar};         \
      return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);             \
    }                                                                                            \
    RetraceOp<NA, false, E> op{action_probs_target, action_probs_behavior, q_values,             \
                               next_q_values_all, actions, rewards, terminateds, nullptr,        \
                               targets, advantages, A, gamma, lambda_, c_bar, rho_bar};          \
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);               \
  }
  switch (A) {
    case 1: RLK_RETRACE(1)
    case 2: RLK_RETRACE(2)
    case 4: RLK_RETRACE(4)
    default: RLK_RETRACE(0)
  }
#undef RLK_RETRACE
}

template <class E>
int lambda_returns_impl(const E* rewards, const E* next_values, const E* terminateds,
                        const E* truncateds, const E* bootstrap, int boot_mode, E* returns,
                        int64_t num_envs, int64_t seq_len, float gamma, float lambda_,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !next_values || !terminateds || !returns || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const E* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 &&
                   quad_aligned(rewards, next_values, terminateds, truncateds, returns) &&
                   (boot_mode != RLK_BOOT_FULL || quad_aligned(bootstrap));
  const int ph = common_phase<E>(rewards, next_values, terminateds, truncateds, returns,
                                 boot_mode == RLK_BOOT_FULL ? bootstrap : nullptr);
  if (truncateds) {
    ReturnsOp<true, true, E> op{rewards, next_values, terminateds, truncateds, boot, returns,
                                boot_mode, gamma, gamma * (1.f - lambda_), gamma * lambda_};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
  }
  ReturnsOp<true, false, E> op{rewards, next_values, terminateds, nullptr, boot, returns,
                               boot_mode, gamma, gamma * (1.f - lambda_), gamma * lambda_};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
}

template <class E>
int discounted_returns_impl(const E* rewards, const E* terminateds, const E* truncateds,
                            const E* bootstrap, int boot_mode, E* returns, int64_t num_envs,
                            int64_t seq_len, float gamma, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !terminateds || !returns || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const E* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 && quad_aligned(rewards, terminateds, truncateds, returns) &&
                   (boot_mode != RLK_BOOT_FULL || quad_aligned(bootstrap));
  const int ph = common_phase<E>(rewards, terminateds, truncateds, returns,
                                 boot_mode == RLK_BOOT_FULL ? bootstrap : nullptr);
  if (truncateds) {
    ReturnsOp<false, true, E> op{rewards, nullptr, terminateds, truncateds, boot, returns,
                                 boot_mode, gamma, 0.f, gamma};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
  }
  ReturnsOp<false, false, E> op{rewards, nullptr, terminateds, nullptr, boot, returns, boot_mode,
                                gamma, 0.f, gamma};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
}

// eligibility traces (decay = gamma * lambda, gated on done[t-1]) and the episodic prefix
// sum (decay 1, ends_at or starts_at) share one op
template <class E>
int done_gated_impl(const E* x, const E* dones, const E* seed, E* out, int64_t num_envs,
                    int64_t seq_len, float decay, int ends_at, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!x || !dones || !out) return RLK_ERR_INVALID_ARGUMENT;
  DoneGatedForwardOp<E> op{x, dones, seed, out, decay, ends_at};
  const bool vec = seq_len % 4 == 0 && quad_aligned(x, dones, out);
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream,
                common_phase<E>(x, dones, out));
}

template <class E>
int affine_scan_impl(const E* u, const E* v, const E* carry, E* out, int64_t num_envs,
                     int64_t seq_len, int direction, void* workspace, size_t workspace_bytes,
                     void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!u || !v || !out || (direction != RLK_BACKWARD && direction != RLK_FORWARD))
    return RLK_ERR_INVALID_ARGUMENT;
  const bool vec = seq_len % 4 == 0 && quad_aligned(u, v, out);
  const int ph = common_phase<E>(u, v, out);
  if (direction == RLK_FORWARD) {
    AffineScanOp<true, E> op{u, v, carry, out};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
  }
  AffineScanOp<false, E> op{u, v, carry, out};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream, ph);
}

// ---------------------------------------------------------------------------------------
// rlk_gae_noalloc: the look-back workspace of long rows in a static device array instead of
// a caller's buffer, for callers that cannot allocate.  Each GPU holds its own copy of
// `scratch`; host code never uses the array's name as an address (on the host it is only a
// stand-in) but the address hipGetSymbolAddress returns for the current device, kept per
// device.  The array must start from zero (the look-back's counters at rest, no status
// word tagged with the current call count): clear_scratch zeroes it on the first eager call
// on a device, every RLK_WORKSPACE_MAX_CALLS calls after that (before the status words'
// 30-bit call count can wrap), and in every captured call, so that each graph replay starts
// from zero.  The whole array is cleared, not just the call's share: a clear also resets the
// call count, and words of an earlier, larger call must not outlive it.
// ---------------------------------------------------------------------------------------
constexpr int64_t kNoAllocWords = RLK_NOALLOC_SCRATCH_BYTES / (int64_t)sizeof(uint64_t);
static __device__ __align__(256) uint64_t scratch[kNoAllocWords];

__global__ __launch_bounds__(256) void clear_scratch(uint64_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0;
}

constexpr int kMaxDevices = 64;
struct NoAllocDevice {
  std::mutex mu;
  uint64_t* ptr = nullptr;  // this device's copy of `scratch`
  bool cleared = false;     // an eager clear has been enqueued since set-up
  uint64_t calls = 0;       // long-row eager calls since that clear
};
NoAllocDevice g_noalloc[kMaxDevices];

// The current device's scratch, cleared first when due (on `stream`).
int noalloc_scratch(void* stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RLK_ERR_DEVICE;
  NoAllocDevice& d = g_noalloc[dev];
  std::lock_guard<std::mutex> lock(d.mu);
  if (d.ptr == nullptr) {  // set-up, once per device, with that device current
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return RLK_ERR_DEVICE;
    d.ptr = static_cast<uint64_t*>(p);
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) return RLK_ERR_DEVICE;
  const bool capturing = cs != hipStreamCaptureStatusNone;
  if (capturing || !d.cleared || d.calls >= (uint64_t)RLK_WORKSPACE_MAX_CALLS) {
    uint64_t* p = d.ptr;
    int64_t n = kNoAllocWords;
    void* args[] = {&p, &n};
    if (hipLaunchKernel(reinterpret_cast<const void*>(&clear_scratch), dim3(128), dim3(256), args,
                        0, s) != hipSuccess)
      return RLK_ERR_LAUNCH;
    if (!capturing) {
      d.cleared = true;
      d.calls = 0;
    }
  }
  if (!capturing) ++d.calls;
  *out = d.ptr;
  return RLK_OK;
}

// rlk_bf16 (raw bits) <-> the kernels' bf16 storage type
const bf16* B(const rlk_bf16* p) { return reinterpret_cast<const bf16*>(p); }
bf16* B(rlk_bf16* p) { return reinterpret_cast<bf16*>(p); }

}  // namespace
}  // namespace rlk

using namespace rlk;

extern "C" {

int rlk_version(void) { return 100; }

const char* rlk_status_string(int status) {
  switch (status) {
    case RLK_OK: return "ok";
    case RLK_ERR_INVALID_ARGUMENT: return "invalid argument";
    case RLK_ERR_WORKSPACE: return "workspace missing, too small or misaligned";
    case RLK_ERR_LAUNCH: return "kernel launch failed";
    case RLK_ERR_SCRATCH_LIMIT:
      return "the call needs more look-back scratch than rlk_gae_noalloc's static buffer "
             "(RLK_NOALLOC_SCRATCH_BYTES) holds";
    case RLK_ERR_DEVICE: return "HIP device query or set-up failed";
    default: return "unknown status";
  }
}

size_t rlk_workspace_bytes(int64_t num_envs, int64_t seq_len) {
  return workspace_bytes(num_envs, seq_len);
}

int rlk_debug_lookback(int give_up_polls, int fallback_polls) {
  g_spin_limit.store(give_up_polls < 0 ? kSpinLimit : give_up_polls, std::memory_order_relaxed);
  g_fallback_polls.store(fallback_polls < 0 ? kFallbackPolls : fallback_polls, std::memory_order_relaxed);
  return RLK_OK;
}

int rlk_debug_store_policy(int policy) {
  if (policy < -1 || policy > 1) return RLK_ERR_INVALID_ARGUMENT;
  g_store_policy.store(policy, std::memory_order_relaxed);
  return RLK_OK;
}

int rlk_gae(const float* rewards, const float* values, const float* terminateds,
            const float* truncateds, const float* bootstrap, int boot_mode, float* advantages,
            int64_t num_envs, int64_t seq_len, float gamma, float lambda_, void* workspace,
            size_t workspace_bytes, void* stream) {
  return gae_impl(rewards, values, terminateds, truncateds, bootstrap, boot_mode, advantages,
                  num_envs, seq_len, gamma, lambda_, workspace, workspace_bytes, stream);
}

int rlk_gae_noalloc(const float* rewards, const float* values, const float* terminateds,
                    const float* truncateds, const float* bootstrap, int boot_mode,
                    float* advantages, int64_t num_envs, int64_t seq_len, float gamma,
                    float lambda_, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (num_envs < 0 || seq_len < 0 || seq_len > (int64_t{1} << 30)) return RLK_ERR_INVALID_ARGUMENT;
  void* ws = nullptr;
  const size_t need = workspace_bytes(num_envs, seq_len);
  if (need > 0) {
    if (num_envs > kNoAllocWords || need > (size_t)RLK_NOALLOC_SCRATCH_BYTES)
      return RLK_ERR_SCRATCH_LIMIT;
    const int st = noalloc_scratch(stream, &ws);
    if (st != RLK_OK) return st;
  }
  return gae_impl(rewards, values, terminateds, truncateds, bootstrap, boot_mode, advantages,
                  num_envs, seq_len, gamma, lambda_, ws, ws ? (size_t)RLK_NOALLOC_SCRATCH_BYTES : 0,
                  stream);
}

int rlk_gae_bf16(const rlk_bf16* rewards, const rlk_bf16* values, const rlk_bf16* terminateds,
                 const rlk_bf16* truncateds, const rlk_bf16* bootstrap, int boot_mode,
                 rlk_bf16* advantages, int64_t num_envs, int64_t seq_len, float gamma,
                 float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  return gae_impl(B(rewards), B(values), B(terminateds), B(truncateds), B(bootstrap), boot_mode,
                  B(advantages), num_envs, seq_len, gamma, lambda_, workspace, workspace_bytes,
                  stream);
}

int rlk_gae_masked(const float* rewards, const float* values, const float* terminateds,
                   const float* truncateds, const float* bootstrap, int boot_mode,
                   const float* mask, float* advantages, int64_t num_envs, int64_t seq_len,
                   float gamma, float lambda_, void* workspace, size_t workspace_bytes,
                   void* stream) {
  return gae_masked_impl(rewards, values, terminateds, truncateds, bootstrap, boot_mode, mask,
                         advantages, num_envs, seq_len, gamma, lambda_, workspace,
                         workspace_bytes, stream);
}

int rlk_gae_masked_bf16(const rlk_bf16* rewards, const rlk_bf16* values,
                        const rlk_bf16* terminateds, const rlk_bf16* truncateds,
                        const rlk_bf16* bootstrap, int boot_mode, const rlk_bf16* mask,
                        rlk_bf16* advantages, int64_t num_envs, int64_t seq_len, float gamma,
                        float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  return gae_masked_impl(B(rewards), B(values), B(terminateds), B(truncateds), B(bootstrap),
                         boot_mode, B(mask), B(advantages), num_envs, seq_len, gamma, lambda_,
                         workspace, workspace_bytes, stream);
}

size_t rlk_gae_normalized_partials_bytes(int64_t num_envs, int64_t seq_len) {
  return gae_normalized_partials(num_envs, seq_len);
}

int rlk_gae_normalized(const float* rewards, const float* values, const float* terminateds,
                       const float* truncateds, const float* bootstrap, int boot_mode,
                       float* advantages, float* returns, int64_t num_envs, int64_t seq_len,
                       float gamma, float lambda_, float eps, void* workspace,
                       size_t workspace_bytes, void* partials, size_t partials_bytes,
                       void* stream) {
  return gae_normalized_impl<float>(rewards, values, terminateds, truncateds, bootstrap,
                                    boot_mode, nullptr, advantages, returns, num_envs, seq_len,
                                    gamma, lambda_, eps, workspace, workspace_bytes, partials,
                                    partials_bytes, stream);
}

int rlk_gae_normalized_bf16(const rlk_bf16* rewards, const rlk_bf16* values,
                            const rlk_bf16* terminateds, const rlk_bf16* truncateds,
                            const rlk_bf16* bootstrap, int boot_mode, rlk_bf16* advantages,
                            rlk_bf16* returns, int64_t num_envs, int64_t seq_len, float gamma,
                            float lambda_, float eps, void* workspace, size_t workspace_bytes,
                            void* partials, size_t partials_bytes, void* stream) {
  return gae_normalized_impl<bf16>(B(rewards), B(values), B(terminateds), B(truncateds),
                                   B(bootstrap), boot_mode, nullptr, B(advantages), B(returns),
                                   num_envs, seq_len, gamma, lambda_, eps, workspace,
                                   workspace_bytes, partials, partials_bytes, stream);
}

int rlk_gae_normalized_masked(const float* rewards, const float* values,
                              const float* terminateds, const float* truncateds,
                              const float* bootstrap, int boot_mode, const float* mask,
                              float* advantages, float* returns, int64_t num_envs,
                              int64_t seq_len, float gamma, float lambda_, float eps,
                              void* workspace, size_t workspace_bytes, void* partials,
                              size_t partials_bytes, void* stream) {
  if (!is_empty(num_envs, seq_len) && !mask) return RLK_ERR_INVALID_ARGUMENT;
  return gae_normalized_impl<float>(rewards, values, terminateds, truncateds, bootstrap,
                                    boot_mode, mask, advantages, returns, num_envs, seq_len,
                                    gamma, lambda_, eps, workspace, workspace_bytes, partials,
                                    partials_bytes, stream);
}

int rlk_gae_normalized_masked_bf16(const rlk_bf16* rewards, const rlk_bf16* values,
                                   const rlk_bf16* terminateds, const rlk_bf16* truncateds,
                                   const rlk_bf16* bootstrap, int boot_mode, const rlk_bf16* mask,
                                   rlk_bf16* advantages, rlk_bf16* returns, int64_t num_envs,
                                   int64_t seq_len, float gamma, float lambda_, float eps,
                                   void* workspace, size_t workspace_bytes, void* partials,
                                   size_t partials_bytes, void* stream) {
  if (!is_empty(num_envs, seq_len) && !mask) return RLK_ERR_INVALID_ARGUMENT;
  return gae_normalized_impl<bf16>(B(rewards), B(values), B(terminateds), B(truncateds),
                                   B(bootstrap), boot_mode, B(mask), B(advantages), B(returns),
                                   num_envs, seq_len, gamma, lambda_, eps, workspace,
                                   workspace_bytes, partials, partials_bytes, stream);
}

int rlk_vtrace(const float* log_pi_target, const float* log_pi_behavior, const float* values,
               const float* rewards, const float* terminateds, const float* truncateds,
               const float* bootstrap, int boot_mode, float* targets, float* advantages,
               int64_t num_envs, int64_t seq_len, float gamma, float rho_bar, float c_bar,
               void* workspace, size_t workspace_bytes, void* stream) {
  return vtrace_impl(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds,
                     bootstrap, boot_mode, targets, advantages, num_envs, seq_len, gamma, rho_bar,
                     c_bar, workspace, workspace_bytes, stream);
}

int rlk_vtrace_bf16(const rlk_bf16* log_pi_target, const rlk_bf16* log_pi_behavior,
                    const rlk_bf16* values, const rlk_bf16* rewards, const rlk_bf16* terminateds,
                    const rlk_bf16* truncateds, const rlk_bf16* bootstrap, int boot_mode,
                    rlk_bf16* targets, rlk_bf16* advantages, int64_t num_envs, int64_t seq_len,
                    float gamma, float rho_bar, float c_bar, void* workspace,
                    size_t workspace_bytes, void* stream) {
  return vtrace_impl(B(log_pi_target), B(log_pi_behavior), B(values), B(rewards), B(terminateds),
                     B(truncateds), B(bootstrap), boot_mode, B(targets), B(advantages), num_envs,
                     seq_len, gamma, rho_bar, c_bar, workspace, workspace_bytes, stream);
}

int rlk_retrace(const float* action_probs_target, const float* action_probs_behavior,
                const float* q_values, const float* next_q_values_all, const int64_t* actions,
                const float* rewards, const float* terminateds, const float* truncateds,
                float* targets, float* advantages, int64_t num_envs, int64_t seq_len,
                int64_t num_actions, float gamma, float lambda_, float c_bar, float rho_bar,
                void* workspace, size_t workspace_bytes, void* stream) {
  return retrace_impl(action_probs_target, action_probs_behavior, q_values, next_q_values_all,
                      actions, rewards, terminateds, truncateds, targets, advantages, num_envs,
                      seq_len, num_actions, gamma, lambda_, c_bar, rho_bar, workspace,
                      workspace_bytes, stream);
}

int rlk_retrace_bf16(const rlk_bf16* action_probs_target, const rlk_bf16* action_probs_behavior,
                     const rlk_bf16* q_values, const rlk_bf16* next_q_values_all,
                     const int64_t* actions, const rlk_bf16* rewards,
                     const rlk_bf16* terminateds, const rlk_bf16* truncateds, rlk_bf16* targets,
                     rlk_bf16* advantages, int64_t num_envs, int64_t seq_len,
                     int64_t num_actions, float gamma, float lambda_, float c_bar, float rho_bar,
                     void* workspace, size_t workspace_bytes, void* stream) {
  return retrace_impl(B(action_probs_target), B(action_probs_behavior), B(q_values),
                      B(next_q_values_all), actions, B(rewards), B(terminateds), B(truncateds),
                      B(targets), B(advantages), num_envs, seq_len, num_actions, gamma, lambda_,
                      c_bar, rho_bar, workspace, workspace_bytes, stream);
}

int rlk_lambda_returns(const float* rewards, const float* next_values, const float* terminateds,
                       const float* truncateds, const float* bootstrap, int boot_mode,
                       float* returns, int64_t num_envs, int64_t seq_len, float gamma,
                       float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  return lambda_returns_impl(rewards, next_values, terminateds, truncateds, bootstrap, boot_mode,
                             returns, num_envs, seq_len, gamma, lambda_, workspace,
                             workspace_bytes, stream);
}

int rlk_lambda_returns_bf16(const rlk_bf16* rewards, const rlk_bf16* next_values,
                            const rlk_bf16* terminateds, const rlk_bf16* truncateds,
                            const rlk_bf16* bootstrap, int boot_mode, rlk_bf16* returns,
                            int64_t num_envs, int64_t seq_len, float gamma, float lambda_,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return lambda_returns_impl(B(rewards), B(next_values), B(terminateds), B(truncateds),
                             B(bootstrap), boot_mode, B(returns), num_envs, seq_len, gamma,
                             lambda_, workspace, workspace_bytes, stream);
}

int rlk_discounted_returns(const float* rewards, const float* terminateds,
                           const float* truncateds, const float* bootstrap, int boot_mode,
                           float* returns, int64_t num_envs, int64_t seq_len, float gamma,
                           void* workspace, size_t workspace_bytes, void* stream) {
  return discounted_returns_impl(rewards, terminateds, truncateds, bootstrap, boot_mode, returns,
                                 num_envs, seq_len, gamma, workspace, workspace_bytes, stream);
}

int rlk_discounted_returns_bf16(const rlk_bf16* rewards, const rlk_bf16* terminateds,
                                const rlk_bf16* truncateds, const rlk_bf16* bootstrap,
                                int boot_mode, rlk_bf16* returns, int64_t num_envs,
                                int64_t seq_len, float gamma, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return discounted_returns_impl(B(rewards), B(terminateds), B(truncateds), B(bootstrap),
                                 boot_mode, B(returns), num_envs, seq_len, gamma, workspace,
                                 workspace_bytes, stream);
}

int rlk_eligibility_traces(const float* gradients, const float* dones, const float* seed_values,
                           float* traces, int64_t num_envs, int64_t seq_len, float gamma,
                           float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  return done_gated_impl(gradients, dones, seed_values, traces, num_envs, seq_len,
                         gamma * lambda_, 1, workspace, workspace_bytes, stream);
}

int rlk_eligibility_traces_bf16(const rlk_bf16* gradients, const rlk_bf16* dones,
                                const rlk_bf16* seed_values, rlk_bf16* traces, int64_t num_envs,
                                int64_t seq_len, float gamma, float lambda_, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return done_gated_impl(B(gradients), B(dones), B(seed_values), B(traces), num_envs, seq_len,
                         gamma * lambda_, 1, workspace, workspace_bytes, stream);
}

int rlk_prefix_sum(const float* inputs, const float* dones, const float* seed_values,
                   float* prefix_sums, int64_t num_envs, int64_t seq_len, int ends_at,
                   void* workspace, size_t workspace_bytes, void* stream) {
  return done_gated_impl(inputs, dones, seed_values, prefix_sums, num_envs, seq_len, 1.f,
                         ends_at ? 1 : 0, workspace, workspace_bytes, stream);
}

int rlk_prefix_sum_bf16(const rlk_bf16* inputs, const rlk_bf16* dones,
                        const rlk_bf16* seed_values, rlk_bf16* prefix_sums, int64_t num_envs,
                        int64_t seq_len, int ends_at, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return done_gated_impl(B(inputs), B(dones), B(seed_values), B(prefix_sums), num_envs, seq_len,
                         1.f, ends_at ? 1 : 0, workspace, workspace_bytes, stream);
}

int rlk_affine_scan(const float* u, const float* v, const float* carry, float* out,
                    int64_t num_envs, int64_t seq_len, int direction, void* workspace,
                    size_t workspace_bytes, void* stream) {
  return affine_scan_impl(u, v, carry, out, num_envs, seq_len, direction, workspace,
                          workspace_bytes, stream);
}

int rlk_affine_scan_bf16(const rlk_bf16* u, const rlk_bf16* v, const rlk_bf16* carry,
                         rlk_bf16* out, int64_t num_envs, int64_t seq_len, int direction,
                         void* workspace, size_t workspace_bytes, void* stream) {
  return affine_scan_impl(B(u), B(v), B(carry), B(out), num_envs, seq_len, direction, workspace,
                          workspace_bytes, stream);
}

}  // extern "C"
