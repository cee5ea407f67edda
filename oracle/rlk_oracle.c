/*
 * rlk_oracle.c -- CPU oracle for the rl_triton return-estimation path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the rl_triton package or
 * the HIP library) links, loads or calls this file.  Only tests/, the smoke()
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py use it, and
 * only as the checker.
 *
 * A sequential restatement, in double precision, of the reference's own
 * PyTorch test loops (simonsays1980/rl-triton v0.1.3).  Each function cites
 * the reference loop it follows.  Inputs are the same float32 row-major
 * [E, T] (or [E, T, A]) arrays the GPU path receives; outputs are float64.
 * Every recurrence is evaluated one element at a time in time order, so the
 * result is the exact-arithmetic value rounded only by float64 steps.
 *
 * Bootstrap modes (shared by the backward estimators):
 *   ORC_BOOT_NONE   (0)  no bootstrap: boot(t) = 0
 *   ORC_BOOT_ROW    (1)  one value per row [E]: boot(T-1) = boot[n], else 0
 *   ORC_BOOT_FULL   (2)  per step [E, T]: boot(t) = boot[n, t]
 * (the reference's last_value / bootstrap_values pair, ops/gae.py:153-160)
 *
 * Built with -ffp-contract=off so no multiply-add is fused.
 */
#include <stdint.h>
#include <stddef.h>
#include <math.h>

#define ORC_BOOT_NONE 0
#define ORC_BOOT_ROW 1
#define ORC_BOOT_FULL 2

static double boot_at(const float *boot, int mode, int64_t n, int64_t t, int64_t T)
{
    if (!boot || mode == ORC_BOOT_NONE) return 0.0;
    if (mode == ORC_BOOT_ROW) return (t == T - 1) ? (double)boot[n] : 0.0;
    return (double)boot[n * T + t];
}

static double dmin(double a, double b) { return a < b ? a : b; }

/* Generic backward scan A[t] = u[t] + v[t]*A[t+1], A[T] = boot[n] (or 0).
 * Follows _reference_scan, tests/test_scan_chunked.py:15-29. */
int orc_backward_scan(int64_t E, int64_t T, const float *u, const float *v,
                      const float *boot, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = boot ? (double)boot[n] : 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            carry = (double)u[i] + (double)v[i] * carry;
            out[i] = carry;
        }
    }
    return 0;
}

/* Generic forward scan e[t] = u[t] + v[t]*e[t-1], e[-1] = seed[n] (or 0).
 * Restates the forward recurrence of kernels/scan.py:91-138 (_run_scan_forward,
 * ops/_scan.py:147-213) as a loop. */
int orc_forward_scan(int64_t E, int64_t T, const float *u, const float *v,
                     const float *seed, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = seed ? (double)seed[n] : 0.0;
        for (int64_t t = 0; t < T; ++t) {
            int64_t i = n * T + t;
            carry = (double)u[i] + (double)v[i] * carry;
            out[i] = carry;
        }
    }
    return 0;
}

/* GAE.  Follows _ref_gae_sequential, tests/test_gae.py:418-450 (truncation
 * path) and reference_gae, tests/test_gae.py:34-60 (no truncations; the
 * bootstrap is the next-state value at t = T-1 only).  Semantics of the fused
 * kernel, kernels/gae.py:128-180:
 *   v_next = boot(t)          if t == T-1 or trunc[t] == 1
 *          = values[t+1]      otherwise
 *   done   = min(term + trunc, 1)
 *   delta  = r + gamma*(1-term)*v_next - values
 *   A[t]   = delta + gamma*lambda*(1-done)*A[t+1],   A[T] = 0 */
int orc_gae(int64_t E, int64_t T, const float *r, const float *val,
            const float *term, const float *trunc, const float *boot, int boot_mode,
            double gamma, double lambda, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            double tr = trunc ? (double)trunc[i] : 0.0;
            double te = (double)term[i];
            double v_next = (t == T - 1 || tr == 1.0) ? boot_at(boot, boot_mode, n, t, T)
                                                      : (double)val[i + 1];
            double done = dmin(te + tr, 1.0);
            double delta = (double)r[i] + gamma * (1.0 - te) * v_next - (double)val[i];
            carry = delta + gamma * lambda * (1.0 - done) * carry;
            out[i] = carry;
        }
    }
    return 0;
}

/* GAE with skipped steps: the "verl-style" masking of the reference's ROADMAP.md:131-140,
 * which the reference does not implement.  Restates verl's compute_gae_advantage_return
 * (verl/trainer/ppo/core_algos.py, the multi-turn form, verl is not a dependency of the
 * reference), whose loop keeps `nextvalues` and `lastgaelam` across steps with
 * response_mask == 0:
 *     delta       = r + gamma * nextvalues - values
 *     lastgaelam' = delta + gamma * lam * lastgaelam
 *     nextvalues  = mask ? values : nextvalues;   lastgaelam = mask ? lastgaelam' : lastgaelam
 *     A[t]        = lastgaelam
 * with this library's boundary rules at kept steps (the GAE above): nextvalues starts at
 * boot(T-1); a truncated step takes boot(t) as its next value; (1 - term) masks the TD
 * target and (1 - done) cuts lastgaelam.  A step is kept when mask != 0. */
int orc_gae_masked(int64_t E, int64_t T, const float *r, const float *val,
                   const float *term, const float *trunc, const float *boot, int boot_mode,
                   const float *mask, double gamma, double lambda, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double nv = boot_at(boot, boot_mode, n, T - 1, T);
        double a = 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            if (mask[i] != 0.0f) {
                double tr = trunc ? (double)trunc[i] : 0.0;
                double te = (double)term[i];
                double v_next = (tr == 1.0) ? boot_at(boot, boot_mode, n, t, T) : nv;
                double done = dmin(te + tr, 1.0);
                double delta = (double)r[i] + gamma * (1.0 - te) * v_next - (double)val[i];
                a = delta + gamma * lambda * (1.0 - done) * a;
                nv = (double)val[i];
            }
            out[i] = a;
        }
    }
    return 0;
}

/* V-trace.  Follows reference_vtrace, tests/test_vtrace.py:56-101 and
 * _ref_vtrace_sequential, tests/test_vtrace.py:424-480, with the fused
 * kernel's bootstrap rule (kernels/vtrace_fused.py:109-196):
 *   rho = min(rho_bar, exp(lpt - lpb)),  c = min(c_bar, exp(lpt - lpb))
 *   no truncations: v_next = boot(T-1) at t = T-1, values[t+1] otherwise
 *   truncations:    v_next = values[t+1]*[t < T-1 and trunc == 0] + boot(t)
 *   delta = rho*(r + gamma*v_next*(1-term) - values)
 *   Delta[t] = delta + gamma*c*(1-done)*Delta[t+1],  Delta[T] = 0
 *   vs = Delta + values
 *   next_vs follows the same rule as v_next with vs in place of values
 *   adv = rho*(r + gamma*next_vs*(1-term) - values) */
int orc_vtrace(int64_t E, int64_t T, const float *lpt, const float *lpb,
               const float *val, const float *r, const float *term, const float *trunc,
               const float *boot, int boot_mode, double gamma, double rho_bar,
               double c_bar, double *targets, double *adv)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            double ratio = exp((double)lpt[i] - (double)lpb[i]);
            double rho = dmin(ratio, rho_bar);
            double c = dmin(ratio, c_bar);
            double te = (double)term[i];
            double tr = trunc ? (double)trunc[i] : 0.0;
            double done = dmin(te + tr, 1.0);
            double v_next;
            if (trunc) {
                double raw = (t < T - 1 && tr == 0.0) ? (double)val[i + 1] : 0.0;
                v_next = raw + boot_at(boot, boot_mode, n, t, T);
            } else {
                v_next = (t == T - 1) ? boot_at(boot, boot_mode, n, t, T) : (double)val[i + 1];
            }
            double delta = rho * ((double)r[i] + gamma * v_next * (1.0 - te) - (double)val[i]);
            carry = delta + gamma * c * (1.0 - done) * carry;
            targets[i] = carry + (double)val[i];
        }
        for (int64_t t = 0; t < T; ++t) {
            int64_t i = n * T + t;
            double ratio = exp((double)lpt[i] - (double)lpb[i]);
            double rho = dmin(ratio, rho_bar);
            double te = (double)term[i];
            double tr = trunc ? (double)trunc[i] : 0.0;
            double nxt;
            if (trunc) {
                double raw = (t < T - 1 && tr == 0.0) ? targets[i + 1] : 0.0;
                nxt = raw + boot_at(boot, boot_mode, n, t, T);
            } else {
                nxt = (t == T - 1) ? boot_at(boot, boot_mode, n, t, T) : targets[i + 1];
            }
            adv[i] = rho * ((double)r[i] + gamma * nxt * (1.0 - te) - (double)val[i]);
        }
    }
    return 0;
}

/* Retrace(lambda).  Follows reference_retrace, tests/test_retrace.py:19-60.
 *   pi_a  = pi[t, a_t] (0 when a_t is outside [0, A), as the fused kernel's
 *           one-hot select gives, kernels/retrace_fused.py:166-172)
 *   rho   = min(rho_bar, pi_a/mu),  c = lambda*min(c_bar, pi_a/mu)
 *   u     = r + gamma*sum_a(pi*nq)*(1-term) - q
 *   v     = gamma*c[t+1]*(1-done),  c[T] = 0,  done = min(term + trunc, 1)
 *   Delta[t] = u + v*Delta[t+1],  Delta[T] = 0;  Q_ret = Delta + q
 *   adv   = rho*(r + gamma*Q_ret[t+1]*(1-term) - q),  Q_ret[T] = 0 */
int orc_retrace(int64_t E, int64_t T, int64_t A, const float *pi, const float *mu,
                const float *q, const float *nq, const int64_t *actions, const float *r,
                const float *term, const float *trunc, double gamma, double lambda,
                double c_bar, double rho_bar, double *targets, double *adv)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = 0.0;
        double c_next = 0.0; /* c[T] = 0 */
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            double exp_nq = 0.0, pi_a = 0.0;
            int64_t act = actions[i];
            for (int64_t a = 0; a < A; ++a) {
                double p = (double)pi[i * A + a];
                exp_nq += p * (double)nq[i * A + a];
                if (a == act) pi_a = p;
            }
            double ratio = pi_a / (double)mu[i];
            double te = (double)term[i];
            double tr = trunc ? (double)trunc[i] : 0.0;
            double done = dmin(te + tr, 1.0);
            double u = (double)r[i] + gamma * exp_nq * (1.0 - te) - (double)q[i];
            double v = gamma * c_next * (1.0 - done);
            carry = u + v * carry;
            targets[i] = carry + (double)q[i];
            c_next = lambda * dmin(ratio, c_bar);
        }
        for (int64_t t = 0; t < T; ++t) {
            int64_t i = n * T + t;
            double pi_a = 0.0;
            int64_t act = actions[i];
            if (act >= 0 && act < A) pi_a = (double)pi[i * A + act];
            double rho = dmin(pi_a / (double)mu[i], rho_bar);
            double nxt = (t < T - 1) ? targets[i + 1] : 0.0;
            adv[i] = rho * ((double)r[i] + gamma * nxt * (1.0 - (double)term[i]) - (double)q[i]);
        }
    }
    return 0;
}

/* TD(lambda) lambda-returns.  Follows reference_lambda_returns,
 * tests/test_returns.py:19-38 and _ref_lambda_sequential,
 * tests/test_returns.py:451-485:
 *   nd = 1 - min(term + trunc, 1)
 *   G[t] = r + gamma*(1-lambda)*nd*nv + gamma*trunc*boot(t) + gamma*lambda*nd*G[t+1]
 *   G[T] = boot(T-1) */
int orc_lambda_returns(int64_t E, int64_t T, const float *r, const float *nv,
                       const float *term, const float *trunc, const float *boot,
                       int boot_mode, double gamma, double lambda, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = boot_at(boot, boot_mode, n, T - 1, T);
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            double tr = trunc ? (double)trunc[i] : 0.0;
            double nd = 1.0 - dmin((double)term[i] + tr, 1.0);
            carry = (double)r[i] + gamma * (1.0 - lambda) * nd * (double)nv[i]
                    + gamma * tr * boot_at(boot, boot_mode, n, t, T)
                    + gamma * lambda * nd * carry;
            out[i] = carry;
        }
    }
    return 0;
}

/* Discounted returns.  Follows reference_discounted_returns,
 * tests/test_returns.py:41-57 and _ref_discounted_sequential,
 * tests/test_returns.py:488-510:
 *   G[t] = r + gamma*(1 - min(term + trunc, 1))*G[t+1] + gamma*trunc*boot(t)
 *   G[T] = boot(T-1) */
int orc_discounted_returns(int64_t E, int64_t T, const float *r, const float *term,
                           const float *trunc, const float *boot, int boot_mode,
                           double gamma, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = boot_at(boot, boot_mode, n, T - 1, T);
        for (int64_t t = T - 1; t >= 0; --t) {
            int64_t i = n * T + t;
            double tr = trunc ? (double)trunc[i] : 0.0;
            double nd = 1.0 - dmin((double)term[i] + tr, 1.0);
            carry = (double)r[i] + gamma * nd * carry + gamma * tr * boot_at(boot, boot_mode, n, t, T);
            out[i] = carry;
        }
    }
    return 0;
}

/* Eligibility traces (forward).  Follows reference_eligibility_traces,
 * tests/test_returns.py:362-384:
 *   z[t] = g[t] + gamma*lambda*(1 - done[t-1])*z[t-1],  z[-1] = seed,  done[-1] = 0 */
int orc_eligibility_traces(int64_t E, int64_t T, const float *g, const float *dones,
                           double gamma, double lambda, const float *seed, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = seed ? (double)seed[n] : 0.0;
        double prev_done = 0.0;
        for (int64_t t = 0; t < T; ++t) {
            int64_t i = n * T + t;
            carry = (double)g[i] + gamma * lambda * (1.0 - prev_done) * carry;
            out[i] = carry;
            prev_done = (double)dones[i];
        }
    }
    return 0;
}

/* Episodic prefix sum (forward).  Follows reference_episodic_prefix_sum,
 * tests/test_prefix_sum.py:18-56:
 *   ends_at:   C[t] = x[t] + (1 - done[t-1])*C[t-1],  done[-1] = 0
 *   starts_at: C[t] = x[t] + (1 - done[t])*C[t-1]
 *   C[-1] = seed */
int orc_prefix_sum(int64_t E, int64_t T, const float *x, const float *dones,
                   const float *seed, int ends_at, double *out)
{
    for (int64_t n = 0; n < E; ++n) {
        double carry = seed ? (double)seed[n] : 0.0;
        double prev_done = 0.0;
        for (int64_t t = 0; t < T; ++t) {
            int64_t i = n * T + t;
            double gate = ends_at ? prev_done : (double)dones[i];
            carry = (double)x[i] + (1.0 - gate) * carry;
            out[i] = carry;
            prev_done = (double)dones[i];
        }
    }
    return 0;
}
