"""ctypes binding of librl_triton_amd.so, the gfx950 HIP kernels behind every op.

The library's C ABI (include/rl_triton_amd.h) takes plain device pointers, sizes and
a hipStream_t.  This module turns tensors into those arguments, launches on torch's
current stream for the tensors' device, owns the per-(device, stream) look-back
workspace, and maps error codes to exceptions.

There is no fallback: if the library is missing or cannot be loaded, every op
raises.  All tensors reaching this module are checked (device, dtype, contiguity,
shape) before any pointer is handed to a kernel, so a malformed call raises here
instead of reaching the GPU.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_NAME = "librl_triton_amd.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

BOOT_NONE, BOOT_ROW, BOOT_FULL = 0, 1, 2
BACKWARD, FORWARD = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> argtypes (must match include/rl_triton_amd.h)
SIGNATURES = {
    "rlk_gae": [_P, _P, _P, _P, _P, _INT, _P, _I64, _I64, _F, _F, _P, _SZ, _P],
    "rlk_gae_noalloc": [_P, _P, _P, _P, _P, _INT, _P, _I64, _I64, _F, _F, _P],
    "rlk_gae_masked": [_P, _P, _P, _P, _P, _INT, _P, _P, _I64, _I64, _F, _F, _P, _SZ, _P],
    "rlk_gae_normalized": [_P, _P, _P, _P, _P, _INT, _P, _P, _I64, _I64, _F, _F, _F, _P, _SZ, _P,
                           _SZ, _P],
    "rlk_gae_normalized_masked": [_P, _P, _P, _P, _P, _INT, _P, _P, _P, _I64, _I64, _F, _F, _F, _P,
                                  _SZ, _P, _SZ, _P],
    "rlk_gae_normalized_partials_bytes": [_I64, _I64],
    "rlk_vtrace": [_P, _P, _P, _P, _P, _P, _P, _INT, _P, _P, _I64, _I64, _F, _F, _F, _P, _SZ, _P],
    "rlk_retrace": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _F, _F, _F, _P,
                    _SZ, _P],
    "rlk_lambda_returns": [_P, _P, _P, _P, _P, _INT, _P, _I64, _I64, _F, _F, _P, _SZ, _P],
    "rlk_discounted_returns": [_P, _P, _P, _P, _INT, _P, _I64, _I64, _F, _P, _SZ, _P],
    "rlk_eligibility_traces": [_P, _P, _P, _P, _I64, _I64, _F, _F, _P, _SZ, _P],
    "rlk_prefix_sum": [_P, _P, _P, _P, _I64, _I64, _INT, _P, _SZ, _P],
    "rlk_affine_scan": [_P, _P, _P, _P, _I64, _I64, _INT, _P, _SZ, _P],
    "rlk_workspace_bytes": [_I64, _I64],
    "rlk_status_string": [_INT],
    "rlk_version": [],
    "rlk_debug_lookback": [_INT, _INT],
    "rlk_debug_store_policy": [_INT],
}
# the bfloat16 twins take the same arguments (rlk_bf16 arrays in place of float ones)
for _name in ("rlk_gae", "rlk_gae_masked", "rlk_gae_normalized", "rlk_gae_normalized_masked", "rlk_vtrace", "rlk_retrace", "rlk_lambda_returns",
              "rlk_discounted_returns", "rlk_eligibility_traces", "rlk_prefix_sum",
              "rlk_affine_scan"):
    SIGNATURES[_name + "_bf16"] = SIGNATURES[_name]
del _name
_RESTYPES = {"rlk_workspace_bytes": _SZ, "rlk_gae_normalized_partials_bytes": _SZ,
             "rlk_status_string": ctypes.c_char_p}

_lib = None
_lock = threading.Lock()

# The tensor-level fast path (csrc/rlk_torch.cpp, built next to this file): a well-formed
# call goes from the API straight to the C ABI with its checks done in C++; it returns None
# for any call it does not take, and the op's Python path handles that call.  None here if
# the module is not built (the Python path then serves every call, through ctypes); a
# module that is built but does not load is an error.
_FAST_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_rlk_torch.so")
if os.path.exists(_FAST_PATH):
    from rl_triton import _rlk_torch as fast
else:
    fast = None


def public_entry(pyfunc, op):
    """`pyfunc` (a compute_* implementation) behind the C++ fast path: a callable with the
    same signature, defaults, name and docstring that launches well-formed calls directly
    and passes every other call, arguments untouched, to `pyfunc` (see Entry in
    csrc/rlk_torch.cpp).  `pyfunc` itself when the fast path is not built."""
    if fast is None:
        return pyfunc
    import functools
    import inspect
    params = list(inspect.signature(pyfunc).parameters.values())
    names = tuple(p.name for p in params)
    npos = sum(p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD) for p in params)
    defaults = tuple(p.default for p in params)
    entry = fast.entry(op, names, npos, defaults, inspect.Parameter.empty, pyfunc)
    return functools.update_wrapper(entry, pyfunc)


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or failed to load; there is no other backend."""


def library_path() -> str:
    return _LIB_PATH


def load():
    """Load (once) and return the ctypes handle of librl_triton_amd.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise NativeLibraryError(
                    f"{_LIB_PATH} is not built; run `python rl-triton_amd/build.py` "
                    "(rl_triton has no non-HIP backend)")
            try:
                lib = ctypes.CDLL(_LIB_PATH)
            except OSError as e:
                raise NativeLibraryError(f"cannot load {_LIB_PATH}: {e}") from e
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


# ---------------------------------------------------------------------------------------
# argument checks (the last line of defence before pointers reach a kernel).  Written for
# a short per-call path: a few C-level tensor queries per argument.
# ---------------------------------------------------------------------------------------
_F32 = torch.float32
_BF16 = torch.bfloat16
_I64 = torch.int64
_raw_stream = torch._C._cuda_getCurrentRawStream
_cur_device = torch._C._cuda_getDevice


def _ptr(t, name, shape, dev, dtype=_F32) -> int:
    """Data pointer of `t` after checking device index, dtype, shape and contiguity."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(t).__name__}")
    if t.get_device() != dev or t.dtype is not dtype or t.shape != shape or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous {dtype} tensor of shape {list(shape)} on "
                         f"cuda:{dev}, got {t.dtype} {list(t.shape)} on {t.device} "
                         f"(contiguous={t.is_contiguous()})")
    return t.data_ptr()


def _opt(t, name, shape, dev, dtype=_F32):
    return None if t is None else _ptr(t, name, shape, dev, dtype)


def _entry(lib, name, dtype):
    """The C entry point for arrays of `dtype`: `name` for float32, its `_bf16` twin for
    bfloat16 (every float array of a call has the leading tensor's dtype)."""
    if dtype is _F32:
        return getattr(lib, name)
    if dtype is _BF16:
        return getattr(lib, name + "_bf16")
    raise ValueError(f"{name}: expected float32 or bfloat16 tensors, got {dtype}")


def _device_of(t) -> int:
    dev = t.get_device() if isinstance(t, torch.Tensor) else -1
    if dev < 0 or t.device.type != "cuda":
        raise ValueError("rl_triton kernels need GPU tensors (device type 'cuda' on ROCm)")
    return dev


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = load().rlk_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


# ---------------------------------------------------------------------------------------
# look-back workspace: one zero-initialised buffer per (device, stream), grown on demand and
# reused by calls of every shape (the kernels leave it ready for the next call).  Calls on
# one stream are ordered, which is what sharing a workspace requires.
# ---------------------------------------------------------------------------------------
_workspaces: dict = {}
_ws_need: dict = {}
# Status words carry a 30-bit count of the calls made on their workspace, which wraps after
# 2^30 long-row calls; a word left 2^30 calls earlier would then read as current.  A cached
# workspace is therefore zero-filled again (a fill kernel on its own stream, ordered before
# the call) once it has served WORKSPACE_MAX_CALLS long-row calls -- the C ABI's
# RLK_WORKSPACE_MAX_CALLS, which tests may lower.
WORKSPACE_MAX_CALLS = 1 << 29
_ws_calls: dict = {}
_ws_clears = 0


def _count_call(key, ws) -> None:
    """Count one long-row call on workspace `ws` (cache key `key`), zero-filling it first
    when it has already served WORKSPACE_MAX_CALLS calls since it was last zeroed."""
    global _ws_clears
    n = _ws_calls.get(key, 0)
    if n >= WORKSPACE_MAX_CALLS:
        ws.zero_()
        _ws_clears += 1
        n = 0
    _ws_calls[key] = n + 1
# Buffers of calls captured into a HIP graph.  A captured call gets its own, allocated (and
# zero-filled, by a kernel the graph records) inside the capture, so every replay starts
# from a clean buffer and no replay shares one with eager calls, whatever streams they run
# on.  Kept alive here for the life of the process (a few KB each).
_captured: list = []


def _capturing() -> bool:
    return torch.cuda.is_current_stream_capturing()


def _workspace(dev: int, stream: int, n_env: int, n_t: int):
    key = (n_env, n_t)
    need = _ws_need.get(key)
    if need is None:
        need = _ws_need[key] = load().rlk_workspace_bytes(n_env, n_t)
    if need == 0:
        return None, 0
    if _capturing():
        ws = torch.zeros((need + 255) // 256 * 256, dtype=torch.uint8, device=torch.device("cuda", dev))
        _captured.append(ws)
        return ws.data_ptr(), ws.numel()
    ws = _workspaces.get((dev, stream))
    if ws is None or ws.numel() < need:
        size = max(need, 2 * ws.numel() if ws is not None else 0)
        size = (size + 255) // 256 * 256
        cur = torch.cuda.current_stream(dev)
        if cur.cuda_stream != stream:
            raise RuntimeError("workspace stream mismatch")
        ws = torch.zeros(size, dtype=torch.uint8, device=torch.device("cuda", dev))
        _workspaces[(dev, stream)] = ws
        _ws_calls[(dev, stream)] = 0
    _count_call((dev, stream), ws)
    return ws.data_ptr(), ws.numel()


def workspace_error(device=None) -> bool:
    """True if any cached workspace on `device` (this module's and the fast path's) recorded
    a look-back wait that gave up."""
    want = None if device is None else torch.device(device).index
    for (dev, _), ws in list(_workspaces.items()):
        if want is not None and dev != want:
            continue
        if ws[24:32].cpu().view(torch.int64).item() != 0:
            return True
    if fast is not None:
        devs = [want] if want is not None else range(torch.cuda.device_count())
        return any(fast.workspace_error(d) for d in devs)
    return False


# per-workgroup partial sums of compute_gae_normalized: one uninitialised buffer per
# (device, stream), grown on demand (every workgroup writes its own entry before the second
# launch reads them; calls on one stream are ordered).
_partials: dict = {}


def _partials_buffer(dev: int, stream: int, n_env: int, n_t: int):
    need = load().rlk_gae_normalized_partials_bytes(n_env, n_t)
    if _capturing():
        buf = torch.empty(max(need, 256), dtype=torch.uint8, device=torch.device("cuda", dev))
        _captured.append(buf)
        return buf.data_ptr(), buf.numel()
    buf = _partials.get((dev, stream))
    if buf is None or buf.numel() < need:
        size = max(need, 2 * buf.numel() if buf is not None else 0, 256)
        buf = torch.empty(size, dtype=torch.uint8, device=torch.device("cuda", dev))
        _partials[(dev, stream)] = buf
    return buf.data_ptr(), buf.numel()


def _launch(fn, what, dev, n_env, n_t, *args):
    """Call C entry `fn` with `args` + (workspace, bytes, stream) on the current stream of
    device `dev` (made current for the call if it is not)."""
    if dev != _cur_device():
        with torch.cuda.device(dev):
            return _launch(fn, what, dev, n_env, n_t, *args)
    stream = _raw_stream(dev)
    ws, wsb = _workspace(dev, stream, n_env, n_t)
    status = fn(*args, ws, wsb, stream)
    if status != 0:
        _check(status, what)


def _boot_args(boot, n_env, n_t, dev, dtype=_F32):
    if boot is None:
        return None, BOOT_NONE
    if boot.dim() == 1:
        return _ptr(boot, "bootstrap", torch.Size((n_env,)), dev, dtype), BOOT_ROW
    return _ptr(boot, "bootstrap", torch.Size((n_env, n_t)), dev, dtype), BOOT_FULL


# ---------------------------------------------------------------------------------------
# ops.  Every argument is already contiguous; outputs are preallocated by the caller.
# ---------------------------------------------------------------------------------------
def gae(rewards, values, terminateds, truncateds, bootstrap, out, gamma, lambda_):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    lib = _lib or load()
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev, dt)
    _launch(_entry(lib, "rlk_gae", dt), "rlk_gae", dev, n_env, n_t,
            _ptr(rewards, "rewards", shape, dev, dt), _ptr(values, "values", shape, dev, dt),
            _ptr(terminateds, "terminateds", shape, dev, dt), _opt(truncateds, "truncateds", shape, dev, dt),
            bp, mode, _ptr(out, "out", shape, dev, dt), n_env, n_t, gamma, lambda_)
    return out


def gae_masked(rewards, values, terminateds, truncateds, bootstrap, mask, out, gamma, lambda_):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    lib = _lib or load()
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev, dt)
    _launch(_entry(lib, "rlk_gae_masked", dt), "rlk_gae_masked", dev, n_env, n_t,
            _ptr(rewards, "rewards", shape, dev, dt), _ptr(values, "values", shape, dev, dt),
            _ptr(terminateds, "terminateds", shape, dev, dt),
            _opt(truncateds, "truncateds", shape, dev, dt), bp, mode,
            _ptr(mask, "mask", shape, dev, dt), _ptr(out, "out", shape, dev, dt), n_env, n_t,
            gamma, lambda_)
    return out


def gae_normalized(rewards, values, terminateds, truncateds, bootstrap, advantages, returns, gamma,
                   lambda_, eps, mask=None):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    lib = _lib or load()
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev, dt)
    head = (_ptr(rewards, "rewards", shape, dev, dt), _ptr(values, "values", shape, dev, dt),
            _ptr(terminateds, "terminateds", shape, dev, dt),
            _opt(truncateds, "truncateds", shape, dev, dt), bp, mode)
    if mask is not None:
        head = head + (_ptr(mask, "mask", shape, dev, dt),)
    args = head + (_ptr(advantages, "advantages", shape, dev, dt),
                   _ptr(returns, "returns", shape, dev, dt), n_env, n_t, gamma, lambda_, eps)
    if dev != _cur_device():
        with torch.cuda.device(dev):
            return gae_normalized(rewards, values, terminateds, truncateds, bootstrap, advantages,
                                  returns, gamma, lambda_, eps, mask)
    stream = _raw_stream(dev)
    ws, wsb = _workspace(dev, stream, n_env, n_t)
    pp, ppb = _partials_buffer(dev, stream, n_env, n_t) if n_env * n_t > 0 else (None, 0)
    name = "rlk_gae_normalized" if mask is None else "rlk_gae_normalized_masked"
    status = _entry(lib, name, dt)(*args, ws, wsb, pp, ppb, stream)
    if status != 0:
        _check(status, name)
    return advantages, returns


def vtrace(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds, bootstrap,
           targets, advantages, gamma, rho_bar, c_bar):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    lib = _lib or load()
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev, dt)
    _launch(_entry(lib, "rlk_vtrace", dt), "rlk_vtrace", dev, n_env, n_t,
            _ptr(log_pi_target, "log_pi_target", shape, dev, dt),
            _ptr(log_pi_behavior, "log_pi_behavior", shape, dev, dt),
            _ptr(values, "values", shape, dev, dt), _ptr(rewards, "rewards", shape, dev, dt),
            _ptr(terminateds, "terminateds", shape, dev, dt), _opt(truncateds, "truncateds", shape, dev, dt),
            bp, mode, _ptr(targets, "targets", shape, dev, dt), _ptr(advantages, "advantages", shape, dev, dt),
            n_env, n_t, gamma, rho_bar, c_bar)
    return targets, advantages


def retrace(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions,
            rewards, terminateds, truncateds, targets, advantages, gamma, lambda_, c_bar, rho_bar):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    if action_probs_target.dim() != 3:
        raise ValueError("action_probs_target must be [num_envs, seq_len, num_actions]")
    n_act = action_probs_target.shape[2]
    shape3 = torch.Size((n_env, n_t, n_act))
    if n_act == 0 and n_env * n_t > 0:
        raise ValueError("num_actions must be positive")
    lib = _lib or load()
    _launch(_entry(lib, "rlk_retrace", dt), "rlk_retrace", dev, n_env, n_t,
            _ptr(action_probs_target, "action_probs_target", shape3, dev, dt),
            _ptr(action_probs_behavior, "action_probs_behavior", shape, dev, dt),
            _ptr(q_values, "q_values", shape, dev, dt),
            _ptr(next_q_values_all, "next_q_values_all", shape3, dev, dt),
            _ptr(actions, "actions", shape, dev, _I64),
            _ptr(rewards, "rewards", shape, dev, dt), _ptr(terminateds, "terminateds", shape, dev, dt),
            _opt(truncateds, "truncateds", shape, dev, dt),
            _ptr(targets, "targets", shape, dev, dt), _ptr(advantages, "advantages", shape, dev, dt),
            n_env, n_t, max(n_act, 1), gamma, lambda_, c_bar, rho_bar)
    return targets, advantages


def lambda_returns(rewards, next_values, terminateds, truncateds, bootstrap, out, gamma, lambda_):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    lib = _lib or load()
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev, dt)
    _launch(_entry(lib, "rlk_lambda_returns", dt), "rlk_lambda_returns", dev, n_env, n_t,
            _ptr(rewards, "rewards", shape, dev, dt), _ptr(next_values, "next_values", shape, dev, dt),
            _ptr(terminateds, "terminateds", shape, dev, dt), _opt(truncateds, "truncateds", shape, dev, dt),
            bp, mode, _ptr(out, "out", shape, dev, dt), n_env, n_t, gamma, lambda_)
    return out


def discounted_returns(rewards, terminateds, truncateds, bootstrap, out, gamma):
    dev = _device_of(rewards)
    shape = rewards.shape
    dt = rewards.dtype
    n_env, n_t = shape
    lib = _lib or load()
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev, dt)
    _launch(_entry(lib, "rlk_discounted_returns", dt), "rlk_discounted_returns", dev, n_env, n_t,
            _ptr(rewards, "rewards", shape, dev, dt), _ptr(terminateds, "terminateds", shape, dev, dt),
            _opt(truncateds, "truncateds", shape, dev, dt), bp, mode,
            _ptr(out, "out", shape, dev, dt), n_env, n_t, gamma)
    return out


def eligibility_traces(gradients, dones, seed, out, gamma, lambda_):
    dev = _device_of(gradients)
    shape = gradients.shape
    dt = gradients.dtype
    n_env, n_t = shape
    lib = _lib or load()
    _launch(_entry(lib, "rlk_eligibility_traces", dt), "rlk_eligibility_traces", dev, n_env, n_t,
            _ptr(gradients, "gradients", shape, dev, dt), _ptr(dones, "dones", shape, dev, dt),
            _opt(seed, "seed_values", torch.Size((n_env,)), dev, dt), _ptr(out, "out", shape, dev, dt),
            n_env, n_t, gamma, lambda_)
    return out


def prefix_sum(inputs, dones, seed, out, ends_at):
    dev = _device_of(inputs)
    shape = inputs.shape
    dt = inputs.dtype
    n_env, n_t = shape
    lib = _lib or load()
    _launch(_entry(lib, "rlk_prefix_sum", dt), "rlk_prefix_sum", dev, n_env, n_t,
            _ptr(inputs, "inputs", shape, dev, dt), _ptr(dones, "dones", shape, dev, dt),
            _opt(seed, "seed_values", torch.Size((n_env,)), dev, dt), _ptr(out, "out", shape, dev, dt),
            n_env, n_t, int(bool(ends_at)))
    return out


def affine_scan(u, v, carry, out, direction):
    dev = _device_of(u)
    shape = u.shape
    dt = u.dtype
    n_env, n_t = shape
    lib = _lib or load()
    _launch(_entry(lib, "rlk_affine_scan", dt), "rlk_affine_scan", dev, n_env, n_t,
            _ptr(u, "u", shape, dev, dt), _ptr(v, "v", shape, dev, dt),
            _opt(carry, "bootstrap" if direction == BACKWARD else "seed", torch.Size((n_env,)), dev, dt),
            _ptr(out, "out", shape, dev, dt), n_env, n_t, direction)
    return out
