/*
 * rlk_loops_f32.c -- float32 sequential loops of the reference's own PyTorch tests.
 *
 * TEST INFRASTRUCTURE ONLY, like rlk_oracle.c (built into the same liboracle.so): the
 * rl_triton package never links, loads or calls it.
 *
 * The reference's correctness tests compare its kernels with PyTorch loops that step
 * through time one vectorised float32 operation at a time.  These functions restate
 * those loops in C with the same operation order, so every statement rounds to float32
 * exactly where a torch CPU elementwise operation does: a product of two Python floats
 * (gamma * lambda_) is formed in double and rounded once when it meets a tensor, and
 * nothing is fused (built with -ffp-contract=off).  tests/test_oracle_cpu.py checks them
 * bit for bit against the torch loops of oracle/torch_loops.py.  They exist so that the
 * full-size parity tests can measure the error of "the reference's float32 sequential
 * loop" against the float64 oracle in milliseconds (a torch loop takes ~18 us per step,
 * ~20 s at a million steps), and bound the GPU's error by it.
 *
 * Bootstrap modes as in rlk_oracle.c: 0 none, 1 one value per row (boot(T-1)), 2 per step.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

static float boot32(const float *boot, int mode, int64_t n, int64_t t, int64_t T)
{
    if (!boot || mode == 0) return 0.0f;
    if (mode == 1) return (t == T - 1) ? boot[n] : 0.0f;
    return boot[n * T + t];
}

/* torch.clamp(x, max=m) */
static float clampmax(float x, float m) { return x > m ? m : x; }
static float clamp1(float x) { return x > 1.0f ? 1.0f : x; }

/* GAE: reference_gae, tests/test_gae.py:34-60 (no truncations) and _ref_gae_trunc,
 * tests/bench_release.py:128-156 (truncations), as oracle/torch_loops.py gae_loop:
 *   v_next = boot(T-1) at t = T-1; with truncations where(trunc, boot(t), values[t+1])
 *   delta  = r + gamma*(1-term)*v_next - values
 *   carry  = delta + gamma*lambda*(1-done)*carry,   carry = 0 at T */
int f32_gae(int64_t E, int64_t T, const float *r, const float *val, const float *term,
            const float *trunc, const float *boot, int boot_mode, double gamma, double lambda,
            float *out)
{
    const float g = (float)gamma, gl = (float)(gamma * lambda);
    for (int64_t n = 0; n < E; ++n) {
        float carry = 0.0f;
        for (int64_t t = T - 1; t >= 0; --t) {
            const int64_t i = n * T + t;
            float v_next;
            if (t == T - 1) v_next = boot32(boot, boot_mode, n, t, T);
            else if (trunc && trunc[i] != 0.0f) v_next = boot32(boot, boot_mode, n, t, T);
            else v_next = val[i + 1];
            const float done = trunc ? clamp1(term[i] + trunc[i]) : term[i];
            float a = g * (1.0f - term[i]);
            a = a * v_next;
            float delta = r[i] + a;
            delta = delta - val[i];
            float d = gl * (1.0f - done);
            d = d * carry;
            carry = delta + d;
            out[i] = carry;
        }
    }
    return 0;
}

/* V-trace without truncations: numpy_vtrace_cpu, tests/bench_release.py:296-320 and
 * reference_vtrace, tests/test_vtrace.py:56-101, as oracle/torch_loops.py vtrace_loop:
 *   ratio = exp(lpt - lpb), rho = clamp(ratio, max=rho_bar), c = clamp(ratio, max=c_bar)
 *   disc = gamma*(1-term);  delta = rho*(r + disc*v_next - values)
 *   carry = delta + disc*c*carry;  targets = carry + values
 *   adv = rho*(r + disc*next_target - values), next_target[T-1] = last_value (or 0)
 * exp is the C library's expf (torch's CPU exp may differ from it in the last place). */
int f32_vtrace(int64_t E, int64_t T, const float *lpt, const float *lpb, const float *val,
               const float *r, const float *term, const float *last_value, double gamma,
               double rho_bar, double c_bar, float *targets, float *adv)
{
    const float g = (float)gamma, rb = (float)rho_bar, cb = (float)c_bar;
    for (int64_t n = 0; n < E; ++n) {
        const float lv = last_value ? last_value[n] : 0.0f;
        float carry = 0.0f;
        for (int64_t t = T - 1; t >= 0; --t) {
            const int64_t i = n * T + t;
            const float ratio = expf(lpt[i] - lpb[i]);
            const float rho = clampmax(ratio, rb), c = clampmax(ratio, cb);
            const float disc = g * (1.0f - term[i]);
            const float shifted = (t == T - 1) ? lv : val[i + 1];
            float x = disc * shifted;
            x = r[i] + x;
            x = x - val[i];
            const float delta = rho * x;
            float d = disc * c;
            d = d * carry;
            carry = delta + d;
            targets[i] = carry + val[i];
        }
        for (int64_t t = 0; t < T; ++t) {
            const int64_t i = n * T + t;
            const float ratio = expf(lpt[i] - lpb[i]);
            const float rho = clampmax(ratio, rb);
            const float disc = g * (1.0f - term[i]);
            const float nxt = (t == T - 1) ? lv : targets[i + 1];
            float x = disc * nxt;
            x = r[i] + x;
            x = x - val[i];
            adv[i] = rho * x;
        }
    }
    return 0;
}

/* Retrace(lambda): reference_retrace, tests/test_retrace.py:19-60:
 *   dones = clamp(term + trunc, max=1);  E_pi[Q'] = sum over actions of pi*Q'
 *   deltas = r + gamma*E_pi[Q']*(1-term) - q
 *   c = lambda*clamp(pi_a/mu, max=c_bar),  rho = clamp(pi_a/mu, max=rho_bar)
 *   carry = deltas + gamma*c[t+1]*(1-dones)*carry  (c[T] = 0);  targets = carry + q
 *   adv = rho*(r + gamma*targets[t+1]*(1-term) - q),  targets[T] = 0
 * The sum over actions is taken in action order. */
int f32_retrace(int64_t E, int64_t T, int64_t A, const float *pi, const float *mu,
                const float *q, const float *nq, const int64_t *actions, const float *r,
                const float *term, const float *trunc, double gamma, double lambda,
                double c_bar, double rho_bar, float *targets, float *adv)
{
    const float g = (float)gamma, lam = (float)lambda, cb = (float)c_bar, rb = (float)rho_bar;
    for (int64_t n = 0; n < E; ++n) {
        float carry = 0.0f, c_next = 0.0f;
        for (int64_t t = T - 1; t >= 0; --t) {
            const int64_t i = n * T + t;
            float enq = 0.0f;
            for (int64_t a = 0; a < A; ++a) {
                const float p = pi[i * A + a] * nq[i * A + a];
                enq = a == 0 ? p : enq + p;
            }
            const float done = clamp1(term[i] + (trunc ? trunc[i] : 0.0f));
            float x = g * enq;
            x = x * (1.0f - term[i]);
            x = r[i] + x;
            const float delta = x - q[i];
            float d = g * c_next;
            d = d * (1.0f - done);
            d = d * carry;
            carry = delta + d;
            targets[i] = carry + q[i];
            const int64_t act = actions[i];
            const float pa = (act >= 0 && act < A) ? pi[i * A + act] : 0.0f;
            c_next = lam * clampmax(pa / mu[i], cb);
        }
        for (int64_t t = 0; t < T; ++t) {
            const int64_t i = n * T + t;
            const int64_t act = actions[i];
            const float pa = (act >= 0 && act < A) ? pi[i * A + act] : 0.0f;
            const float rho = clampmax(pa / mu[i], rb);
            const float nxt = (t < T - 1) ? targets[i + 1] : 0.0f;
            float x = g * nxt;
            x = x * (1.0f - term[i]);
            x = r[i] + x;
            x = x - q[i];
            adv[i] = rho * x;
        }
    }
    return 0;
}

/* TD(lambda): reference_lambda_returns, tests/test_returns.py:19-38 (no truncations) and
 * _ref_lambda_sequential, tests/test_returns.py:449-485 (truncations):
 *   not_done = 1 - clamp(term + trunc, max=1)
 *   carry = r + gamma*(1-lambda)*not_done*nv [+ gamma*trunc*boot(t)] + gamma*lambda*not_done*carry
 *   carry = boot(T-1) at T */
int f32_lambda_returns(int64_t E, int64_t T, const float *r, const float *nv, const float *term,
                       const float *trunc, const float *boot, int boot_mode, double gamma,
                       double lambda, float *out)
{
    const float g = (float)gamma, g1l = (float)(gamma * (1.0 - lambda)), gl = (float)(gamma * lambda);
    for (int64_t n = 0; n < E; ++n) {
        float carry = boot32(boot, boot_mode, n, T - 1, T);
        for (int64_t t = T - 1; t >= 0; --t) {
            const int64_t i = n * T + t;
            const float nd = trunc ? 1.0f - clamp1(term[i] + trunc[i]) : 1.0f - term[i];
            float a = g1l * nd;
            a = a * nv[i];
            float u = r[i] + a;
            if (trunc) {
                float b = g * trunc[i];
                b = b * boot32(boot, boot_mode, n, t, T);
                u = u + b;
            }
            float d = gl * nd;
            d = d * carry;
            carry = u + d;
            out[i] = carry;
        }
    }
    return 0;
}

/* Discounted returns: reference_discounted_returns, tests/test_returns.py:41-57 and
 * _ref_discounted_sequential, tests/test_returns.py:488-510:
 *   carry = r + gamma*not_done*carry [+ gamma*trunc*boot(t)],  carry = boot(T-1) at T */
int f32_discounted_returns(int64_t E, int64_t T, const float *r, const float *term,
                           const float *trunc, const float *boot, int boot_mode, double gamma,
                           float *out)
{
    const float g = (float)gamma;
    for (int64_t n = 0; n < E; ++n) {
        float carry = boot32(boot, boot_mode, n, T - 1, T);
        for (int64_t t = T - 1; t >= 0; --t) {
            const int64_t i = n * T + t;
            const float nd = trunc ? 1.0f - clamp1(term[i] + trunc[i]) : 1.0f - term[i];
            float d = g * nd;
            d = d * carry;
            float x = r[i] + d;
            if (trunc) {
                float b = g * trunc[i];
                b = b * boot32(boot, boot_mode, n, t, T);
                x = x + b;
            }
            carry = x;
            out[i] = carry;
        }
    }
    return 0;
}

/* Eligibility traces: reference_eligibility_traces, tests/test_returns.py:362-384:
 *   carry = g + gamma*lambda*(1-prev_done)*carry,  prev_done = dones[t-1] (0 at t = 0) */
int f32_eligibility_traces(int64_t E, int64_t T, const float *grad, const float *dones,
                           double gamma, double lambda, const float *seed, float *out)
{
    const float gl = (float)(gamma * lambda);
    for (int64_t n = 0; n < E; ++n) {
        float carry = seed ? seed[n] : 0.0f, prev = 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            const int64_t i = n * T + t;
            float d = gl * (1.0f - prev);
            d = d * carry;
            carry = grad[i] + d;
            out[i] = carry;
            prev = dones[i];
        }
    }
    return 0;
}

/* Episodic prefix sum: reference_episodic_prefix_sum, tests/test_prefix_sum.py:18-56:
 *   ends_at: carry = x + (1-prev_done)*carry;  starts_at: carry = x + (1-dones[t])*carry */
int f32_prefix_sum(int64_t E, int64_t T, const float *x, const float *dones, const float *seed,
                   int ends_at, float *out)
{
    for (int64_t n = 0; n < E; ++n) {
        float carry = seed ? seed[n] : 0.0f, prev = 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            const int64_t i = n * T + t;
            const float gate = ends_at ? prev : dones[i];
            const float d = (1.0f - gate) * carry;
            carry = x[i] + d;
            out[i] = carry;
            prev = dones[i];
        }
    }
    return 0;
}

/* Generic scans: _reference_scan, tests/test_scan_chunked.py:15-29 (backward,
 *   carry = deltas + decays*carry, carry = bootstrap at T), and its forward mirror
 *   (carry = u + v*carry from the seed at t = -1; _run_scan_forward has no reference loop). */
int f32_backward_scan(int64_t E, int64_t T, const float *u, const float *v, const float *carry0,
                      float *out)
{
    for (int64_t n = 0; n < E; ++n) {
        float carry = carry0 ? carry0[n] : 0.0f;
        for (int64_t t = T - 1; t >= 0; --t) {
            const int64_t i = n * T + t;
            const float d = v[i] * carry;
            carry = u[i] + d;
            out[i] = carry;
        }
    }
    return 0;
}

int f32_forward_scan(int64_t E, int64_t T, const float *u, const float *v, const float *carry0,
                     float *out)
{
    for (int64_t n = 0; n < E; ++n) {
        float carry = carry0 ? carry0[n] : 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            const int64_t i = n * T + t;
            const float d = v[i] * carry;
            carry = u[i] + d;
            out[i] = carry;
        }
    }
    return 0;
}
