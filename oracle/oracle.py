"""NumPy front end for the C oracle in ``oracle/rlk_oracle.c``.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, always as the checker.  The
rl_triton package never imports it.

Every function takes float32 (int64 for Retrace actions) NumPy arrays shaped
like the rl_triton API arguments and returns float64 arrays computed by a
sequential double-precision loop that restates the reference's own PyTorch
test loops (see the file:line citations in rlk_oracle.c).

``loop32`` is the other kind: the reference's float32 torch
loops restated in C with the same operation order and rounding
(rlk_loops_f32.c), returning float32 arrays.  They measure the error level of
"the reference's float32 sequential loop" at full size in milliseconds.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

BOOT_NONE, BOOT_ROW, BOOT_FULL = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_D = ctypes.c_double
_INT = ctypes.c_int

_SIGS = {
    "orc_backward_scan": [_I64, _I64, _P, _P, _P, _P],
    "orc_forward_scan": [_I64, _I64, _P, _P, _P, _P],
    "orc_gae": [_I64, _I64, _P, _P, _P, _P, _P, _INT, _D, _D, _P],
    "orc_gae_masked": [_I64, _I64, _P, _P, _P, _P, _P, _INT, _P, _D, _D, _P],
    "orc_vtrace": [_I64, _I64, _P, _P, _P, _P, _P, _P, _P, _INT, _D, _D, _D, _P, _P],
    "orc_retrace": [_I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _D, _D, _D, _D, _P, _P],
    "orc_lambda_returns": [_I64, _I64, _P, _P, _P, _P, _P, _INT, _D, _D, _P],
    "orc_discounted_returns": [_I64, _I64, _P, _P, _P, _P, _INT, _D, _P],
    "orc_eligibility_traces": [_I64, _I64, _P, _P, _D, _D, _P, _P],
    "orc_prefix_sum": [_I64, _I64, _P, _P, _P, _INT, _P],
    # float32 loops (rlk_loops_f32.c)
    "f32_gae": [_I64, _I64, _P, _P, _P, _P, _P, _INT, _D, _D, _P],
    "f32_vtrace": [_I64, _I64, _P, _P, _P, _P, _P, _P, _D, _D, _D, _P, _P],
    "f32_retrace": [_I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _D, _D, _D, _D, _P, _P],
    "f32_lambda_returns": [_I64, _I64, _P, _P, _P, _P, _P, _INT, _D, _D, _P],
    "f32_discounted_returns": [_I64, _I64, _P, _P, _P, _P, _INT, _D, _P],
    "f32_eligibility_traces": [_I64, _I64, _P, _P, _D, _D, _P, _P],
    "f32_prefix_sum": [_I64, _I64, _P, _P, _P, _INT, _P],
    "f32_backward_scan": [_I64, _I64, _P, _P, _P, _P],
    "f32_forward_scan": [_I64, _I64, _P, _P, _P, _P],
}


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile next to this file."""
    if force or not os.path.exists(_LIB_PATH):
        cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
        subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        for name, argtypes in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib = lib
    return _lib


def _f32(a):
    if a is None:
        return None
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return a


def _ptr(a):
    return None if a is None else a.ctypes.data


def _boot(boot, E, T):
    """Classify a bootstrap argument: None, per-row [E] or per-step [E, T]."""
    if boot is None:
        return None, BOOT_NONE
    b = _f32(boot)
    if b.shape == (E,):
        return b, BOOT_ROW
    if b.shape == (E, T):
        return b, BOOT_FULL
    raise ValueError(f"bootstrap shape {b.shape} is neither [{E}] nor [{E}, {T}]")


def backward_scan(u, v, bootstrap=None):
    u, v = _f32(u), _f32(v)
    E, T = u.shape
    b = _f32(bootstrap)
    out = np.empty((E, T), np.float64)
    _load().orc_backward_scan(E, T, _ptr(u), _ptr(v), _ptr(b), _ptr(out))
    return out


def forward_scan(u, v, seed=None):
    u, v = _f32(u), _f32(v)
    E, T = u.shape
    s = _f32(seed)
    out = np.empty((E, T), np.float64)
    _load().orc_forward_scan(E, T, _ptr(u), _ptr(v), _ptr(s), _ptr(out))
    return out


def gae(rewards, values, terminateds, truncateds=None, gamma=0.99, lambda_=0.95,
        bootstrap=None):
    """``bootstrap`` is ``last_value`` ([E]) or ``bootstrap_values`` ([E, T])."""
    r, v, te, tr = map(_f32, (rewards, values, terminateds, truncateds))
    E, T = r.shape
    b, mode = _boot(bootstrap, E, T)
    out = np.empty((E, T), np.float64)
    _load().orc_gae(E, T, _ptr(r), _ptr(v), _ptr(te), _ptr(tr), _ptr(b), mode,
                    gamma, lambda_, _ptr(out))
    return out


def gae_masked(rewards, values, terminateds, mask, truncateds=None, gamma=0.99, lambda_=0.95,
               bootstrap=None):
    """GAE in which steps with mask == 0 pass the advantage and the next value through."""
    r, v, te, mk, tr = map(_f32, (rewards, values, terminateds, mask, truncateds))
    E, T = r.shape
    b, mode = _boot(bootstrap, E, T)
    out = np.empty((E, T), np.float64)
    _load().orc_gae_masked(E, T, _ptr(r), _ptr(v), _ptr(te), _ptr(tr), _ptr(b), mode, _ptr(mk),
                           gamma, lambda_, _ptr(out))
    return out


def vtrace(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds=None,
           gamma=0.99, rho_bar=1.0, c_bar=1.0, bootstrap=None):
    lpt, lpb, v, r, te, tr = map(_f32, (log_pi_target, log_pi_behavior, values, rewards,
                                        terminateds, truncateds))
    E, T = r.shape
    b, mode = _boot(bootstrap, E, T)
    tg = np.empty((E, T), np.float64)
    adv = np.empty((E, T), np.float64)
    _load().orc_vtrace(E, T, _ptr(lpt), _ptr(lpb), _ptr(v), _ptr(r), _ptr(te), _ptr(tr),
                       _ptr(b), mode, gamma, rho_bar, c_bar, _ptr(tg), _ptr(adv))
    return tg, adv


def retrace(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions,
            rewards, terminateds, truncateds, gamma, lambda_=1.0, c_bar=1.0, rho_bar=1.0):
    pi, mu, q, nq, r, te, tr = map(_f32, (action_probs_target, action_probs_behavior, q_values,
                                          next_q_values_all, rewards, terminateds, truncateds))
    act = np.ascontiguousarray(np.asarray(actions, dtype=np.int64))
    E, T, A = pi.shape
    tg = np.empty((E, T), np.float64)
    adv = np.empty((E, T), np.float64)
    _load().orc_retrace(E, T, A, _ptr(pi), _ptr(mu), _ptr(q), _ptr(nq), _ptr(act), _ptr(r),
                        _ptr(te), _ptr(tr), gamma, lambda_, c_bar, rho_bar, _ptr(tg), _ptr(adv))
    return tg, adv


def lambda_returns(rewards, next_values, terminateds, truncateds=None, gamma=0.99,
                   lambda_=0.95, bootstrap=None):
    r, nv, te, tr = map(_f32, (rewards, next_values, terminateds, truncateds))
    E, T = r.shape
    b, mode = _boot(bootstrap, E, T)
    out = np.empty((E, T), np.float64)
    _load().orc_lambda_returns(E, T, _ptr(r), _ptr(nv), _ptr(te), _ptr(tr), _ptr(b), mode,
                               gamma, lambda_, _ptr(out))
    return out


def discounted_returns(rewards, terminateds, truncateds=None, gamma=0.99, bootstrap=None):
    r, te, tr = map(_f32, (rewards, terminateds, truncateds))
    E, T = r.shape
    b, mode = _boot(bootstrap, E, T)
    out = np.empty((E, T), np.float64)
    _load().orc_discounted_returns(E, T, _ptr(r), _ptr(te), _ptr(tr), _ptr(b), mode, gamma,
                                   _ptr(out))
    return out


def eligibility_traces(gradients, dones, gamma, lambda_, seed_values=None):
    g, d, s = map(_f32, (gradients, dones, seed_values))
    E, T = g.shape
    out = np.empty((E, T), np.float64)
    _load().orc_eligibility_traces(E, T, _ptr(g), _ptr(d), gamma, lambda_, _ptr(s), _ptr(out))
    return out


def episodic_prefix_sum(inputs, dones, seed_values=None, boundary="ends_at"):
    if boundary not in ("ends_at", "starts_at"):
        raise ValueError(boundary)
    x, d, s = map(_f32, (inputs, dones, seed_values))
    E, T = x.shape
    out = np.empty((E, T), np.float64)
    _load().orc_prefix_sum(E, T, _ptr(x), _ptr(d), _ptr(s), int(boundary == "ends_at"),
                           _ptr(out))
    return out


# ---------------------------------------------------------------------------------------
# the reference's float32 sequential loops (rlk_loops_f32.c): float32 results
# ---------------------------------------------------------------------------------------
def loop32(op, inp, params):
    """The float32 loop of `op` on a case dict (the keys of the rl_triton API arguments),
    as a tuple of float32 arrays in the order of the API's outputs."""
    g = inp.get
    lib = _load()
    if op == "gae":
        r, v, te, tr = map(_f32, (g("rewards"), g("values"), g("terminateds"), g("truncateds")))
        E, T = r.shape
        b, mode = _boot(g("last_value") if g("last_value") is not None else g("bootstrap_values"), E, T)
        out = np.empty((E, T), np.float32)
        lib.f32_gae(E, T, _ptr(r), _ptr(v), _ptr(te), _ptr(tr), _ptr(b), mode,
                    params["gamma"], params["lambda_"], _ptr(out))
        return (out,)
    if op == "vtrace":
        if g("truncateds") is not None or g("bootstrap_values") is not None:
            raise ValueError("the reference's float32 V-trace loop takes last_value only")
        lpt, lpb, v, r, te, lv = map(_f32, (g("log_pi_target"), g("log_pi_behavior"), g("values"),
                                            g("rewards"), g("terminateds"), g("last_value")))
        E, T = r.shape
        tg, adv = np.empty((E, T), np.float32), np.empty((E, T), np.float32)
        lib.f32_vtrace(E, T, _ptr(lpt), _ptr(lpb), _ptr(v), _ptr(r), _ptr(te), _ptr(lv),
                       params["gamma"], params.get("rho_bar", 1.0), params.get("c_bar", 1.0),
                       _ptr(tg), _ptr(adv))
        return tg, adv
    if op == "retrace":
        pi, mu, q, nq, r, te, tr = map(_f32, (g("action_probs_target"), g("action_probs_behavior"),
                                              g("q_values"), g("next_q_values_all"), g("rewards"),
                                              g("terminateds"), g("truncateds")))
        act = np.ascontiguousarray(np.asarray(g("actions"), dtype=np.int64))
        E, T, A = pi.shape
        tg, adv = np.empty((E, T), np.float32), np.empty((E, T), np.float32)
        lib.f32_retrace(E, T, A, _ptr(pi), _ptr(mu), _ptr(q), _ptr(nq), _ptr(act), _ptr(r),
                        _ptr(te), _ptr(tr), params["gamma"], params.get("lambda_", 1.0),
                        params.get("c_bar", 1.0), params.get("rho_bar", 1.0), _ptr(tg), _ptr(adv))
        return tg, adv
    if op == "lambda_returns":
        r, nv, te, tr = map(_f32, (g("rewards"), g("next_values"), g("terminateds"), g("truncateds")))
        E, T = r.shape
        b, mode = _boot(g("bootstrap_values"), E, T)
        out = np.empty((E, T), np.float32)
        lib.f32_lambda_returns(E, T, _ptr(r), _ptr(nv), _ptr(te), _ptr(tr), _ptr(b), mode,
                               params["gamma"], params["lambda_"], _ptr(out))
        return (out,)
    if op == "discounted_returns":
        r, te, tr = map(_f32, (g("rewards"), g("terminateds"), g("truncateds")))
        E, T = r.shape
        b, mode = _boot(g("bootstrap_values"), E, T)
        out = np.empty((E, T), np.float32)
        lib.f32_discounted_returns(E, T, _ptr(r), _ptr(te), _ptr(tr), _ptr(b), mode,
                                   params["gamma"], _ptr(out))
        return (out,)
    if op == "eligibility_traces":
        x, d, s = map(_f32, (g("gradients"), g("dones"), g("seed_values")))
        E, T = x.shape
        out = np.empty((E, T), np.float32)
        lib.f32_eligibility_traces(E, T, _ptr(x), _ptr(d), params["gamma"], params["lambda_"],
                                   _ptr(s), _ptr(out))
        return (out,)
    if op == "prefix_sum":
        x, d, s = map(_f32, (g("inputs"), g("dones"), g("seed_values")))
        E, T = x.shape
        out = np.empty((E, T), np.float32)
        lib.f32_prefix_sum(E, T, _ptr(x), _ptr(d), _ptr(s),
                           int(params.get("boundary", "ends_at") == "ends_at"), _ptr(out))
        return (out,)
    if op in ("backward_scan", "forward_scan"):
        u, v = _f32(g("u")), _f32(g("v"))
        c = _f32(g("bootstrap") if op == "backward_scan" else g("seed"))
        E, T = u.shape
        out = np.empty((E, T), np.float32)
        fn = lib.f32_backward_scan if op == "backward_scan" else lib.f32_forward_scan
        fn(E, T, _ptr(u), _ptr(v), _ptr(c), _ptr(out))
        return (out,)
    raise KeyError(op)


def has_loop32(op, inp) -> bool:
    """Whether the reference has a float32 loop for this call (its V-trace loop takes no
    truncations and no per-step bootstrap)."""
    if op == "vtrace":
        return inp.get("truncateds") is None and inp.get("bootstrap_values") is None
    return op in ("gae", "retrace", "lambda_returns", "discounted_returns", "eligibility_traces",
                  "prefix_sum", "backward_scan", "forward_scan")
