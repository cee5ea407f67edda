/*
 * rl_triton_amd.h -- C ABI of the MI355X (gfx950) return-estimation kernels.
 *
 * The reference (simonsays1980/rl-triton v0.1.3) has no C ABI: its boundary is the
 * Python functions in src/rl_triton/ops/, each of which validates its tensors and
 * launches one Triton kernel on torch's current stream.  Each entry point below is
 * the device-side half of one of those functions; the rl_triton Python package in
 * this repository calls them with tensor data pointers (ctypes), after raising the
 * reference's AssertionErrors itself.
 *
 * Conventions shared by every entry point
 *   - Tensors are contiguous row-major float32 [num_envs, seq_len] device arrays (the
 *     `_bf16` twins: bfloat16)
 *     (Retrace: [num_envs, seq_len, num_actions] for the per-action inputs, int64
 *     actions).  Outputs are written, never read; inputs are never written.
 *   - All work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 *     default stream).  Nothing allocates and nothing synchronises.
 *   - Any element-aligned pointers are accepted.  The fastest form is seq_len % 4 == 0
 *     with every [num_envs, seq_len] array 16-byte aligned (bfloat16: 8-byte), which
 *     the kernels read and write with aligned non-temporal 16-byte accesses.  Rows longer
 *     than 2048 steps of seq_len % 4 != 0 whose arrays all start at the same element
 *     offset modulo 4 (freshly allocated arrays do) are shifted to their own 16-byte
 *     boundaries and keep aligned accesses (within ~5% of the aligned form); Retrace and
 *     the normalised GAE entries excepted.  Other calls use element-aligned 16-byte
 *     accesses (about 10-20% slower).
 *   - Bootstrap mode: RLK_BOOT_NONE (bootstrap == NULL, value 0), RLK_BOOT_ROW
 *     (bootstrap is [num_envs]: the continuation value after step seq_len-1, the
 *     reference's `last_value`), RLK_BOOT_FULL (bootstrap is [num_envs, seq_len], the
 *     reference's `bootstrap_values`).
 *   - Workspace: rows longer than one workgroup tile are split into tiles chained by a
 *     decoupled look-back.  Those calls need `workspace` of at least
 *     rlk_workspace_bytes(num_envs, seq_len) bytes, ZERO-FILLED BEFORE ITS FIRST USE.
 *     Each call leaves the workspace ready for the next one, so zero it once and reuse
 *     it, across calls of any shape; calls that share a workspace must be ordered on one
 *     stream (concurrent use races).  Zero it again after at most
 *     RLK_WORKSPACE_MAX_CALLS long-row calls: the status words carry a 30-bit count of
 *     the calls made on the workspace, which wraps after 2^30 calls, and a word left by
 *     a call 2^30 calls earlier would then read as current (a silently wrong carry).
 *     Calls that need no workspace ignore the argument (NULL is fine).
 *     Layout (uint64 words): [0..7] header, word [3] the error flag -- nonzero if a
 *     look-back wait gave up or the counters were not at rest (results of that call are
 *     invalid); [8..2055] 64 slots (start counter and epoch of a slot of rows); then two
 *     places of up to five status words per tile.
 *   - Sizes: num_envs up to what device memory holds, seq_len up to 2^30.  HIP launches at
 *     most 2^32 - 1 work-items per grid dimension; a call whose launch would need more
 *     (from about 3.2 billion steps of 3-step rows, or about 4.2 million rows of 2049
 *     steps) is issued as launches over consecutive row ranges, in row order on `stream`.
 *     Rows are independent, so only the number of launches changes (the normalised GAE's
 *     statistics cover all of them).  The reference's Triton kernels compute a row's
 *     offset as program_id * stride in 32-bit integers (src/rl_triton/kernels/gae.py:38-39).
 *   - Return value: RLK_OK or a negative RLK_ERR_* code; rlk_status_string() names it.
 *     Empty inputs (num_envs == 0 or seq_len == 0) return RLK_OK without a launch.
 *   - bfloat16 I/O: every estimator has an `_bf16` twin whose float arrays (inputs,
 *     bootstrap, seed and outputs alike) are bfloat16, passed as rlk_bf16 (the raw 16
 *     bits).  The arithmetic stays float32: a bfloat16 result is the float32 entry
 *     point's result on the same (widened) inputs, rounded to nearest even as torch's
 *     float -> bfloat16 conversion on the GPU rounds it (NaN -> 0x7fc0).  The reference accepts
 *     float32 only (its ROADMAP.md:82-99 lists this as planned); the twins have no
 *     counterpart there.
 */
#ifndef RL_TRITON_AMD_H
#define RL_TRITON_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RLK_OK 0
#define RLK_ERR_INVALID_ARGUMENT (-1)
#define RLK_ERR_WORKSPACE (-2)
#define RLK_ERR_LAUNCH (-3)
#define RLK_ERR_SCRATCH_LIMIT (-4) /* rlk_gae_noalloc: the call needs more than its static buffer */
#define RLK_ERR_DEVICE (-5)        /* a HIP device query or set-up call failed */

#define RLK_BOOT_NONE 0
#define RLK_BOOT_ROW 1
#define RLK_BOOT_FULL 2

#define RLK_BACKWARD 0
#define RLK_FORWARD 1

/* Long-row calls a workspace may serve between two zero-fills (see Workspace above). */
#define RLK_WORKSPACE_MAX_CALLS (1 << 29)

/* A bfloat16 value as its raw bits (the upper half of an IEEE float32). */
typedef uint16_t rlk_bf16;

/* Library version, major*10000 + minor*100 + patch. */
int rlk_version(void);

/* Static text for a status code. */
const char *rlk_status_string(int status);

/* Workspace bytes a call on [num_envs, seq_len] needs (0 when none is needed). */
size_t rlk_workspace_bytes(int64_t num_envs, int64_t seq_len);

/* For tests of the look-back's rare paths only; no counterpart in the reference.  Sets,
 * for the long-row calls launched after it (process-wide), how many polls a look-back wait
 * makes before it gives up (give_up_polls; default about one second) and before a wait on
 * a predecessor tile that has published nothing computes that tile itself, or a wait for
 * a state walks further back (fallback_polls; default 256).  Negative values restore the
 * defaults.  A wait that gives up sets the workspace error flag and writes NaN for its
 * tile and every tile that chains through it; with the defaults a correct run never gets
 * there.  The fallback paths give the same bits as the ordinary one.  Returns RLK_OK. */
int rlk_debug_lookback(int give_up_polls, int fallback_polls);

/* For tests of the output stores only; no counterpart in the reference.  The kernels store
 * their outputs non-temporally or write-through, chosen per launch by the call's shape and
 * storage type (a speed choice; the bits stored are the same).  policy 0 or 1 forces
 * non-temporal or write-through stores, process-wide, for the calls launched after it,
 * wherever the launch is built with that policy (bfloat16 outputs and the 1025..2048-step
 * strided rows are write-through only; float32 V-trace and Retrace long rows non-temporal
 * only); -1 restores the rule.  Returns RLK_OK, or RLK_ERR_INVALID_ARGUMENT for another
 * value. */
int rlk_debug_store_policy(int policy);

/* GAE advantages.  Replaces the gae_fused_kernel launch in compute_gae
 * (src/rl_triton/ops/gae.py:164-190; kernel src/rl_triton/kernels/gae.py:62-180), and
 * its chunked fallback for seq_len > 131072 (ops/gae.py:192-215).
 * truncateds may be NULL (done = terminateds). */
int rlk_gae(const float *rewards, const float *values, const float *terminateds,
            const float *truncateds, const float *bootstrap, int boot_mode, float *advantages,
            int64_t num_envs, int64_t seq_len, float gamma, float lambda_, void *workspace,
            size_t workspace_bytes, void *stream);

/* GAE that allocates nothing and takes no workspace.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Arguments, results and error codes are
 * rlk_gae's without `workspace`/`workspace_bytes`.  Rows longer than 2048 steps keep their
 * look-back status words in a static device buffer of the library, RLK_NOALLOC_SCRATCH_BYTES
 * (1 MiB) on each GPU it runs on, held until the process ends; a call whose
 * rlk_workspace_bytes(num_envs, seq_len) exceeds it (more than 12900 row tiles of 4096
 * steps, e.g. [4096, 16384]) returns RLK_ERR_SCRATCH_LIMIT and launches nothing.  All calls
 * on one GPU share that GPU's buffer, which keeps the last call's contents: calls that
 * overlap on one GPU (other streams, other host threads) race.  The first call on a device
 * that needs the buffer also enqueues a small kernel on `stream` that clears it, as does
 * every RLK_WORKSPACE_MAX_CALLS-th such call after that, and every such call made while
 * `stream` captures a graph (so each replay starts from a clear buffer).  No memset and
 * no allocating routine is called.  The look-back error flag (word 3 of a workspace, see
 * Workspace above) lives in that buffer too, where the caller cannot read it: NaN in the
 * outputs is this entry's only sign of a wait that gave up, and overlapping calls are not
 * detected. */
#define RLK_NOALLOC_SCRATCH_BYTES (1 << 20)
int rlk_gae_noalloc(const float *rewards, const float *values, const float *terminateds,
                    const float *truncateds, const float *bootstrap, int boot_mode,
                    float *advantages, int64_t num_envs, int64_t seq_len, float gamma,
                    float lambda_, void *stream);

/* GAE with skipped steps ("verl-style" masking, listed in the reference's
 * ROADMAP.md:131-140; no counterpart in the reference).  mask [num_envs, seq_len]: a step
 * with mask == 0 is skipped -- its advantage is the next kept step's (0 if none) and the
 * next value passes across it, so a kept step's TD target uses the value of the nearest
 * kept step after it (bootstrap(T-1) after the last one).  Kept steps follow rlk_gae's
 * rules (terminations, truncations with bootstrap_values); with every step kept the result
 * is rlk_gae's.  The other arguments are rlk_gae's. */
int rlk_gae_masked(const float *rewards, const float *values, const float *terminateds,
                   const float *truncateds, const float *bootstrap, int boot_mode,
                   const float *mask, float *advantages, int64_t num_envs, int64_t seq_len,
                   float gamma, float lambda_, void *workspace, size_t workspace_bytes,
                   void *stream);

/* GAE with returns and batch-normalised advantages (no counterpart in the reference: the
 * "fused GAE + advantage normalisation" item of its ROADMAP.md:75-81).  Writes
 *   returns    = A + values
 *   advantages = (A - mean(A)) / (std(A) + eps)
 * with A the advantages of rlk_gae on the same arguments, mean and std over all
 * num_envs * seq_len elements (std unbiased, as torch's Tensor.std()), computed in float64
 * in a fixed order.  Two launches: the scan writes A, the returns and one float64
 * (count, sum, sum of squares) triple per workgroup into `partials` (at least
 * rlk_gae_normalized_partials_bytes(num_envs, seq_len) bytes, 8-byte aligned, no
 * initialisation needed); a second kernel normalises A in place.  Scans of more than 2048
 * workgroups first sum their triples in a tree of 2048 to one (one more launch per level,
 * its triples in the same buffer).  `workspace` as for rlk_gae. */
size_t rlk_gae_normalized_partials_bytes(int64_t num_envs, int64_t seq_len);
int rlk_gae_normalized(const float *rewards, const float *values, const float *terminateds,
                       const float *truncateds, const float *bootstrap, int boot_mode,
                       float *advantages, float *returns, int64_t num_envs, int64_t seq_len,
                       float gamma, float lambda_, float eps, void *workspace,
                       size_t workspace_bytes, void *partials, size_t partials_bytes,
                       void *stream);

/* rlk_gae_normalized with skipped steps (rlk_gae_masked's mask, which must not be NULL): the
 * advantages are rlk_gae_masked's, the returns A + values at every step, and mean and std
 * are taken over the kept steps (mask != 0) only -- the masked whitening verl applies to
 * multi-turn advantages -- then applied to every step.  Fewer than two kept steps give nan
 * advantages, as above.  partials sized by rlk_gae_normalized_partials_bytes. */
int rlk_gae_normalized_masked(const float *rewards, const float *values,
                              const float *terminateds, const float *truncateds,
                              const float *bootstrap, int boot_mode, const float *mask,
                              float *advantages, float *returns, int64_t num_envs,
                              int64_t seq_len, float gamma, float lambda_, float eps,
                              void *workspace, size_t workspace_bytes, void *partials,
                              size_t partials_bytes, void *stream);

/* V-trace targets and advantages.  Replaces vtrace_fused_kernel in compute_vtrace_fused
 * (src/rl_triton/ops/vtrace_fused.py:161-219; kernel kernels/vtrace_fused.py:7-196) and
 * the torch + chunked-scan path of compute_vtrace (ops/vtrace.py:161-201).
 * truncateds may be NULL. */
int rlk_vtrace(const float *log_pi_target, const float *log_pi_behavior, const float *values,
               const float *rewards, const float *terminateds, const float *truncateds,
               const float *bootstrap, int boot_mode, float *targets, float *advantages,
               int64_t num_envs, int64_t seq_len, float gamma, float rho_bar, float c_bar,
               void *workspace, size_t workspace_bytes, void *stream);

/* Retrace(lambda) targets and advantages.  Replaces retrace_fused_kernel in
 * compute_retrace_fused (src/rl_triton/ops/retrace_fused.py:93-118; kernel
 * kernels/retrace_fused.py:7-201) and the torch + _run_scan path of compute_retrace
 * (ops/retrace.py:173-196).  action_probs_target / next_q_values_all are
 * [num_envs, seq_len, num_actions]; actions is int64 [num_envs, seq_len];
 * truncateds may be NULL. */
int rlk_retrace(const float *action_probs_target, const float *action_probs_behavior,
                const float *q_values, const float *next_q_values_all, const int64_t *actions,
                const float *rewards, const float *terminateds, const float *truncateds,
                float *targets, float *advantages, int64_t num_envs, int64_t seq_len,
                int64_t num_actions, float gamma, float lambda_, float c_bar, float rho_bar,
                void *workspace, size_t workspace_bytes, void *stream);

/* TD(lambda) returns.  Replaces lambda_returns_fused_kernel in compute_lambda_returns
 * (src/rl_triton/ops/returns.py:113-140; kernel kernels/lambda_returns_fused.py:7-89) and
 * its chunked fallback (ops/returns.py:142-152).  truncateds may be NULL. */
int rlk_lambda_returns(const float *rewards, const float *next_values, const float *terminateds,
                       const float *truncateds, const float *bootstrap, int boot_mode,
                       float *returns, int64_t num_envs, int64_t seq_len, float gamma,
                       float lambda_, void *workspace, size_t workspace_bytes, void *stream);

/* Discounted returns.  Replaces discounted_returns_fused_kernel in
 * compute_discounted_returns (src/rl_triton/ops/returns.py:225-252; kernel
 * kernels/discounted_returns_fused.py:7-82) and its chunked fallback
 * (ops/returns.py:254-263).  truncateds may be NULL. */
int rlk_discounted_returns(const float *rewards, const float *terminateds,
                           const float *truncateds, const float *bootstrap, int boot_mode,
                           float *returns, int64_t num_envs, int64_t seq_len, float gamma,
                           void *workspace, size_t workspace_bytes, void *stream);

/* Eligibility traces (forward).  Replaces eligibility_traces_fused_kernel in
 * compute_eligibility_traces (src/rl_triton/ops/returns.py:337-346; kernel
 * kernels/eligibility_traces_fused.py:7-84).  Unlike the reference, seq_len is not
 * limited to 131072 (ops/returns.py:319-322).  seed_values may be NULL. */
int rlk_eligibility_traces(const float *gradients, const float *dones, const float *seed_values,
                           float *traces, int64_t num_envs, int64_t seq_len, float gamma,
                           float lambda_, void *workspace, size_t workspace_bytes, void *stream);

/* Episodic prefix sum (forward).  Replaces prefix_sum_fused_kernel in
 * compute_episodic_prefix_sum (src/rl_triton/ops/prefix_sum.py:101-110; kernel
 * kernels/prefix_sum_fused.py:7-84).  ends_at = 1: boundary="ends_at", 0: "starts_at".
 * Not limited to seq_len <= 131072 (ops/prefix_sum.py:83-86).  seed_values may be NULL. */
int rlk_prefix_sum(const float *inputs, const float *dones, const float *seed_values,
                   float *prefix_sums, int64_t num_envs, int64_t seq_len, int ends_at,
                   void *workspace, size_t workspace_bytes, void *stream);

/* Generic affine scan.  direction RLK_BACKWARD: out[t] = u[t] + v[t]*out[t+1],
 * out[T] = carry; RLK_FORWARD: out[t] = u[t] + v[t]*out[t-1], out[-1] = carry.
 * carry ([num_envs]) may be NULL (0).  Replaces _run_scan / _run_scan_forward
 * (src/rl_triton/ops/_scan.py:69-213; kernels kernels/scan.py:39-138,
 * kernels/scan_chunked.py:7-85). */
int rlk_affine_scan(const float *u, const float *v, const float *carry, float *out,
                    int64_t num_envs, int64_t seq_len, int direction, void *workspace,
                    size_t workspace_bytes, void *stream);

/* bfloat16 twins of the entry points above: the same arguments, with rlk_bf16 for every
 * float array.  See "bfloat16 I/O" at the top of this file. */
int rlk_gae_bf16(const rlk_bf16 *rewards, const rlk_bf16 *values, const rlk_bf16 *terminateds,
                 const rlk_bf16 *truncateds, const rlk_bf16 *bootstrap, int boot_mode,
                 rlk_bf16 *advantages, int64_t num_envs, int64_t seq_len, float gamma,
                 float lambda_, void *workspace, size_t workspace_bytes, void *stream);

int rlk_gae_masked_bf16(const rlk_bf16 *rewards, const rlk_bf16 *values,
                        const rlk_bf16 *terminateds, const rlk_bf16 *truncateds,
                        const rlk_bf16 *bootstrap, int boot_mode, const rlk_bf16 *mask,
                        rlk_bf16 *advantages, int64_t num_envs, int64_t seq_len, float gamma,
                        float lambda_, void *workspace, size_t workspace_bytes, void *stream);

/* The bfloat16 results of rlk_gae_normalized.  The statistics are those of the float32
 * advantages; the second launch normalises the stored (bfloat16) advantages, so each
 * normalised value is rounded twice. */
int rlk_gae_normalized_bf16(const rlk_bf16 *rewards, const rlk_bf16 *values,
                            const rlk_bf16 *terminateds, const rlk_bf16 *truncateds,
                            const rlk_bf16 *bootstrap, int boot_mode, rlk_bf16 *advantages,
                            rlk_bf16 *returns, int64_t num_envs, int64_t seq_len, float gamma,
                            float lambda_, float eps, void *workspace, size_t workspace_bytes,
                            void *partials, size_t partials_bytes, void *stream);

int rlk_gae_normalized_masked_bf16(const rlk_bf16 *rewards, const rlk_bf16 *values,
                                   const rlk_bf16 *terminateds, const rlk_bf16 *truncateds,
                                   const rlk_bf16 *bootstrap, int boot_mode, const rlk_bf16 *mask,
                                   rlk_bf16 *advantages, rlk_bf16 *returns, int64_t num_envs,
                                   int64_t seq_len, float gamma, float lambda_, float eps,
                                   void *workspace, size_t workspace_bytes, void *partials,
                                   size_t partials_bytes, void *stream);

int rlk_vtrace_bf16(const rlk_bf16 *log_pi_target, const rlk_bf16 *log_pi_behavior,
                    const rlk_bf16 *values, const rlk_bf16 *rewards, const rlk_bf16 *terminateds,
                    const rlk_bf16 *truncateds, const rlk_bf16 *bootstrap, int boot_mode,
                    rlk_bf16 *targets, rlk_bf16 *advantages, int64_t num_envs, int64_t seq_len,
                    float gamma, float rho_bar, float c_bar, void *workspace,
                    size_t workspace_bytes, void *stream);

/* actions stay int64. */
int rlk_retrace_bf16(const rlk_bf16 *action_probs_target, const rlk_bf16 *action_probs_behavior,
                     const rlk_bf16 *q_values, const rlk_bf16 *next_q_values_all,
                     const int64_t *actions, const rlk_bf16 *rewards,
                     const rlk_bf16 *terminateds, const rlk_bf16 *truncateds, rlk_bf16 *targets,
                     rlk_bf16 *advantages, int64_t num_envs, int64_t seq_len,
                     int64_t num_actions, float gamma, float lambda_, float c_bar, float rho_bar,
                     void *workspace, size_t workspace_bytes, void *stream);

int rlk_lambda_returns_bf16(const rlk_bf16 *rewards, const rlk_bf16 *next_values,
                            const rlk_bf16 *terminateds, const rlk_bf16 *truncateds,
                            const rlk_bf16 *bootstrap, int boot_mode, rlk_bf16 *returns,
                            int64_t num_envs, int64_t seq_len, float gamma, float lambda_,
                            void *workspace, size_t workspace_bytes, void *stream);

int rlk_discounted_returns_bf16(const rlk_bf16 *rewards, const rlk_bf16 *terminateds,
                                const rlk_bf16 *truncateds, const rlk_bf16 *bootstrap,
                                int boot_mode, rlk_bf16 *returns, int64_t num_envs,
                                int64_t seq_len, float gamma, void *workspace,
                                size_t workspace_bytes, void *stream);

int rlk_eligibility_traces_bf16(const rlk_bf16 *gradients, const rlk_bf16 *dones,
                                const rlk_bf16 *seed_values, rlk_bf16 *traces, int64_t num_envs,
                                int64_t seq_len, float gamma, float lambda_, void *workspace,
                                size_t workspace_bytes, void *stream);

int rlk_prefix_sum_bf16(const rlk_bf16 *inputs, const rlk_bf16 *dones,
                        const rlk_bf16 *seed_values, rlk_bf16 *prefix_sums, int64_t num_envs,
                        int64_t seq_len, int ends_at, void *workspace, size_t workspace_bytes,
                        void *stream);

int rlk_affine_scan_bf16(const rlk_bf16 *u, const rlk_bf16 *v, const rlk_bf16 *carry,
                         rlk_bf16 *out, int64_t num_envs, int64_t seq_len, int direction,
                         void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RL_TRITON_AMD_H */
