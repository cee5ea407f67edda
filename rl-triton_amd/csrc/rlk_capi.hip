// rlk_capi.hip -- extern "C" entry points of librl_triton_amd.so (declared in
// include/rl_triton_amd.h): argument checks, launch planning and kernel launches.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

#include "rl_triton_amd.h"
#include "rlk_ops.hpp"

namespace rlk {
namespace {

// Launch geometry.  The macros only exist so that tuning sweeps can rebuild the library
// with other values; the defaults are the shipped configuration.
#ifndef RLK_LB_NTD
#define RLK_LB_NTD 512
#endif
#ifndef RLK_LB_S
#define RLK_LB_S 8
#endif
constexpr int kNT = 256;             // short rows: threads per workgroup (4 wavefronts)
constexpr int kShortMaxT = 2048;     // rows up to this length are kept whole in one workgroup
constexpr int kLbNTD = RLK_LB_NTD;   // look-back path: data threads per workgroup
constexpr int kLbBlock = kLbNTD + kWave;  // ... plus the coordinator wave
constexpr int kTileS = RLK_LB_S;     // look-back path: steps per data thread
constexpr int kTile = kLbNTD * kTileS;

struct Plan {
  bool lookback;
  int S;
  int log2L;
  int tiles_per_row;
  int64_t grid;
};

int ceil_log2(int64_t x) {
  int k = 0;
  while ((int64_t{1} << k) < x) ++k;
  return k;
}

// Short rows: S steps per thread, L = 2^ceil(log2(ceil(T/S))) threads per row, 256/L
// rows per workgroup.  Long rows: tiles of kTile steps, drawn by a persistent grid of
// min(E, 64) * k workgroups (see lookback_kernel in rlk_engine.hpp).
Plan make_plan(int64_t E, int64_t T) {
  Plan p{};
  if (T <= kShortMaxT) {
    p.lookback = false;
    p.S = (T <= 1024) ? 4 : 8;
    p.log2L = ceil_log2((T + p.S - 1) / p.S);
    p.tiles_per_row = 1;
    const int64_t rows_per_block = kNT >> p.log2L;
    p.grid = (E + rows_per_block - 1) / rows_per_block;
  } else {
    p.lookback = true;
    p.S = kTileS;
    p.log2L = 0;
    p.tiles_per_row = (int)((T + kTile - 1) / kTile);
    p.grid = E * p.tiles_per_row;  // upper bound; the persistent grid is smaller
  }
  return p;
}

size_t workspace_bytes(int64_t E, int64_t T) {
  if (E <= 0 || T <= kShortMaxT) return 0;
  const int64_t tiles = E * ((T + kTile - 1) / kTile);
  return (size_t)(kStatusOffset + 2 * tiles) * sizeof(uint64_t);
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Resident workgroups of `kernel` on the current device (occupancy x compute units),
// cached per kernel and device: the persistent look-back grid is sized to it.
int resident_workgroups(const void* kernel, int nt) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({kernel, dev});
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, nt, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int n = per_cu * cus;
  cache[{kernel, dev}] = n;
  return n;
}

template <class Op, int S, bool VEC>
hipError_t launch_rows(const Op& op, int64_t E, int T, int log2L, int64_t grid, hipStream_t stream) {
  void* args[] = {const_cast<Op*>(&op), &E, &T, &log2L};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rows_kernel<Op, kNT, S, VEC>),
                         dim3((unsigned)grid), dim3(kNT), args, 0, stream);
}

template <class Op, bool VEC>
hipError_t launch_lookback(const Op& op, int64_t E, int T, int tpr, uint64_t* ws, hipStream_t stream) {
  const void* kernel = reinterpret_cast<const void*>(&lookback_kernel<Op, kLbNTD, kTileS, VEC>);
  const int64_t nslots = lookback_slots(E);
  const int64_t tiles_per_slot = ((E + nslots - 1) / nslots) * (int64_t)tpr;
  int64_t wgs = resident_workgroups(kernel, kLbBlock) / nslots;
  if (wgs < 1) wgs = 1;
  if (wgs > tiles_per_slot) wgs = tiles_per_slot;
  const int64_t grid = nslots * wgs;
  void* args[] = {const_cast<Op*>(&op), &E, &T, &tpr, &ws};
  return hipLaunchKernel(kernel, dim3((unsigned)grid), dim3(kLbBlock), args, 0, stream);
}

template <class Op>
int launch(const Op& op, int64_t E, int64_t T, bool vec, void* workspace, size_t workspace_bytes_given,
           void* stream) {
  if (E < 0 || T < 0 || T > (int64_t{1} << 30)) return RLK_ERR_INVALID_ARGUMENT;
  if (E == 0 || T == 0) return RLK_OK;
  const Plan p = make_plan(E, T);
  if (p.grid > 0x7fffffffLL) return RLK_ERR_INVALID_ARGUMENT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint64_t* ws = reinterpret_cast<uint64_t*>(workspace);
  const int Ti = (int)T;
  hipError_t e;
  if (p.lookback) {
    if (ws == nullptr || workspace_bytes_given < workspace_bytes(E, T) || !aligned16(ws))
      return RLK_ERR_WORKSPACE;
    e = vec ? launch_lookback<Op, true>(op, E, Ti, p.tiles_per_row, ws, s)
            : launch_lookback<Op, false>(op, E, Ti, p.tiles_per_row, ws, s);
  } else if (p.S == 4) {
    e = vec ? launch_rows<Op, 4, true>(op, E, Ti, p.log2L, p.grid, s)
            : launch_rows<Op, 4, false>(op, E, Ti, p.log2L, p.grid, s);
  } else {
    e = vec ? launch_rows<Op, 8, true>(op, E, Ti, p.log2L, p.grid, s)
            : launch_rows<Op, 8, false>(op, E, Ti, p.log2L, p.grid, s);
  }
  return e == hipSuccess ? RLK_OK : RLK_ERR_LAUNCH;
}

// Empty shapes are a successful no-op (their data pointers may be null); negative sizes
// are rejected by launch().
bool is_empty(int64_t E, int64_t T) { return (E == 0 && T >= 0) || (T == 0 && E >= 0); }

bool valid_boot(const float* boot, int mode) {
  if (mode == RLK_BOOT_NONE) return true;
  if (mode == RLK_BOOT_ROW || mode == RLK_BOOT_FULL) return boot != nullptr;
  return false;
}

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
    default: return "unknown status";
  }
}

size_t rlk_workspace_bytes(int64_t num_envs, int64_t seq_len) {
  return workspace_bytes(num_envs, seq_len);
}

int rlk_gae(const float* rewards, const float* values, const float* terminateds,
            const float* truncateds, const float* bootstrap, int boot_mode, float* advantages,
            int64_t num_envs, int64_t seq_len, float gamma, float lambda_, void* workspace,
            size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !values || !terminateds || !advantages || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const float* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 && aligned16(rewards) && aligned16(values) &&
                   aligned16(terminateds) && aligned16(truncateds) && aligned16(advantages) &&
                   (boot_mode != RLK_BOOT_FULL || aligned16(bootstrap));
  if (truncateds) {
    GaeOp<true> op{rewards, values, terminateds, truncateds, boot, advantages, boot_mode, gamma,
                   gamma * lambda_};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
  }
  GaeOp<false> op{rewards, values, terminateds, nullptr, boot, advantages, boot_mode, gamma,
                  gamma * lambda_};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

int rlk_vtrace(const float* log_pi_target, const float* log_pi_behavior, const float* values,
               const float* rewards, const float* terminateds, const float* truncateds,
               const float* bootstrap, int boot_mode, float* targets, float* advantages,
               int64_t num_envs, int64_t seq_len, float gamma, float rho_bar, float c_bar,
               void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!log_pi_target || !log_pi_behavior || !values || !rewards || !terminateds || !targets ||
      !advantages || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const float* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 && aligned16(log_pi_target) && aligned16(log_pi_behavior) &&
                   aligned16(values) && aligned16(rewards) && aligned16(terminateds) &&
                   aligned16(truncateds) && aligned16(targets) && aligned16(advantages) &&
                   (boot_mode != RLK_BOOT_FULL || aligned16(bootstrap));
  if (truncateds) {
    VtraceOp<true> op{log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds,
                      boot, targets, advantages, boot_mode, gamma, rho_bar, c_bar};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
  }
  VtraceOp<false> op{log_pi_target, log_pi_behavior, values, rewards, terminateds, nullptr,
                     boot, targets, advantages, boot_mode, gamma, rho_bar, c_bar};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

int rlk_retrace(const float* action_probs_target, const float* action_probs_behavior,
                const float* q_values, const float* next_q_values_all, const int64_t* actions,
                const float* rewards, const float* terminateds, const float* truncateds,
                float* targets, float* advantages, int64_t num_envs, int64_t seq_len,
                int64_t num_actions, float gamma, float lambda_, float c_bar, float rho_bar,
                void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!action_probs_target || !action_probs_behavior || !q_values || !next_q_values_all ||
      !actions || !rewards || !terminateds || !targets || !advantages || num_actions <= 0 ||
      num_actions > (1 << 20))
    return RLK_ERR_INVALID_ARGUMENT;
  const bool vec = seq_len % 4 == 0 && aligned16(action_probs_target) &&
                   aligned16(action_probs_behavior) && aligned16(q_values) &&
                   aligned16(next_q_values_all) && aligned16(actions) && aligned16(rewards) &&
                   aligned16(terminateds) && aligned16(truncateds) && aligned16(targets) &&
                   aligned16(advantages);
  const int A = (int)num_actions;
#define RLK_RETRACE(NA)                                                                          \
  {                                                                                              \
    if (truncateds) {                                                                            \
      RetraceOp<NA, true> op{action_probs_target, action_probs_behavior, q_values,               \
                             next_q_values_all, actions, rewards, terminateds, truncateds,       \
                             targets, advantages, A, gamma, lambda_, c_bar, rho_bar};            \
      return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);             \
    }                                                                                            \
    RetraceOp<NA, false> op{action_probs_target, action_probs_behavior, q_values,                \
                            next_q_values_all, actions, rewards, terminateds, nullptr, targets,  \
                            advantages, A, gamma, lambda_, c_bar, rho_bar};                      \
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

int rlk_lambda_returns(const float* rewards, const float* next_values, const float* terminateds,
                       const float* truncateds, const float* bootstrap, int boot_mode,
                       float* returns, int64_t num_envs, int64_t seq_len, float gamma,
                       float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !next_values || !terminateds || !returns || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const float* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 && aligned16(rewards) && aligned16(next_values) &&
                   aligned16(terminateds) && aligned16(truncateds) && aligned16(returns) &&
                   (boot_mode != RLK_BOOT_FULL || aligned16(bootstrap));
  if (truncateds) {
    ReturnsOp<true, true> op{rewards, next_values, terminateds, truncateds, boot, returns,
                             boot_mode, gamma, gamma * (1.f - lambda_), gamma * lambda_};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
  }
  ReturnsOp<true, false> op{rewards, next_values, terminateds, nullptr, boot, returns, boot_mode,
                            gamma, gamma * (1.f - lambda_), gamma * lambda_};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

int rlk_discounted_returns(const float* rewards, const float* terminateds,
                           const float* truncateds, const float* bootstrap, int boot_mode,
                           float* returns, int64_t num_envs, int64_t seq_len, float gamma,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!rewards || !terminateds || !returns || !valid_boot(bootstrap, boot_mode))
    return RLK_ERR_INVALID_ARGUMENT;
  const float* boot = boot_mode == RLK_BOOT_NONE ? nullptr : bootstrap;
  const bool vec = seq_len % 4 == 0 && aligned16(rewards) && aligned16(terminateds) &&
                   aligned16(truncateds) && aligned16(returns) &&
                   (boot_mode != RLK_BOOT_FULL || aligned16(bootstrap));
  if (truncateds) {
    ReturnsOp<false, true> op{rewards, nullptr, terminateds, truncateds, boot, returns, boot_mode,
                              gamma, 0.f, gamma};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
  }
  ReturnsOp<false, false> op{rewards, nullptr, terminateds, nullptr, boot, returns, boot_mode,
                             gamma, 0.f, gamma};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

int rlk_eligibility_traces(const float* gradients, const float* dones, const float* seed_values,
                           float* traces, int64_t num_envs, int64_t seq_len, float gamma,
                           float lambda_, void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!gradients || !dones || !traces) return RLK_ERR_INVALID_ARGUMENT;
  DoneGatedForwardOp op{gradients, dones, seed_values, traces, gamma * lambda_, 1};
  const bool vec = seq_len % 4 == 0 && aligned16(gradients) && aligned16(dones) && aligned16(traces);
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

int rlk_prefix_sum(const float* inputs, const float* dones, const float* seed_values,
                   float* prefix_sums, int64_t num_envs, int64_t seq_len, int ends_at,
                   void* workspace, size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!inputs || !dones || !prefix_sums) return RLK_ERR_INVALID_ARGUMENT;
  DoneGatedForwardOp op{inputs, dones, seed_values, prefix_sums, 1.f, ends_at ? 1 : 0};
  const bool vec = seq_len % 4 == 0 && aligned16(inputs) && aligned16(dones) && aligned16(prefix_sums);
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

int rlk_affine_scan(const float* u, const float* v, const float* carry, float* out,
                    int64_t num_envs, int64_t seq_len, int direction, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (is_empty(num_envs, seq_len)) return RLK_OK;
  if (!u || !v || !out || (direction != RLK_BACKWARD && direction != RLK_FORWARD))
    return RLK_ERR_INVALID_ARGUMENT;
  const bool vec = seq_len % 4 == 0 && aligned16(u) && aligned16(v) && aligned16(out);
  if (direction == RLK_FORWARD) {
    AffineScanOp<true> op{u, v, carry, out};
    return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
  }
  AffineScanOp<false> op{u, v, carry, out};
  return launch(op, num_envs, seq_len, vec, workspace, workspace_bytes, stream);
}

}  // extern "C"
