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
}
_RESTYPES = {"rlk_workspace_bytes": _SZ, "rlk_status_string": ctypes.c_char_p}

_lib = None
_lock = threading.Lock()


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
# argument checks (the last line of defence before pointers reach a kernel)
# ---------------------------------------------------------------------------------------
def _require(t: torch.Tensor, name: str, shape, device, dtype=torch.float32) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor, got {type(t).__name__}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if t.dtype != dtype:
        raise ValueError(f"{name}: expected {dtype}, got {t.dtype}")
    if tuple(t.shape) != shape:
        raise ValueError(f"{name}: expected shape {list(shape)}, got {list(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _opt(t, name, shape, device):
    return None if t is None else _require(t, name, shape, device)


def _device_of(t: torch.Tensor) -> torch.device:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError("rl_triton kernels need GPU tensors (device type 'cuda' on ROCm)")
    return t.device


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = load().rlk_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


# ---------------------------------------------------------------------------------------
# look-back workspace: one zero-initialised buffer per (device, stream), grown on demand.
# Calls on one stream are ordered, which is what the kernels require of a shared
# workspace.
# ---------------------------------------------------------------------------------------
_workspaces: dict = {}


def _workspace(device: torch.device, stream: torch.cuda.Stream, n_env: int, n_t: int):
    need = load().rlk_workspace_bytes(n_env, n_t)
    if need == 0:
        return None, 0
    key = (device.index, stream.cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < need:
        size = max(need, 2 * ws.numel() if ws is not None else 0)
        size = (size + 255) // 256 * 256
        with torch.cuda.stream(stream):
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws.data_ptr(), ws.numel()


def workspace_error(device=None) -> bool:
    """True if any cached workspace on `device` recorded a look-back wait that gave up."""
    for (dev, _), ws in list(_workspaces.items()):
        if device is not None and dev != torch.device(device).index:
            continue
        flag = ws[24:32].cpu().view(torch.int64).item()
        if flag != 0:
            return True
    return False


class _Launch:
    """Current device / stream context for one call."""

    __slots__ = ("device", "stream", "guard")

    def __init__(self, device: torch.device):
        self.device = device
        self.guard = None
        if device.index is not None and device.index != torch.cuda.current_device():
            self.guard = torch.cuda.device(device)
        self.stream = torch.cuda.current_stream(device)

    def __enter__(self):
        if self.guard is not None:
            self.guard.__enter__()
        return self

    def __exit__(self, *exc):
        if self.guard is not None:
            self.guard.__exit__(*exc)
        return False


def _boot_args(boot, n_env, n_t, device):
    if boot is None:
        return None, BOOT_NONE
    if tuple(boot.shape) == (n_env,):
        return _require(boot, "bootstrap", (n_env,), device), BOOT_ROW
    return _require(boot, "bootstrap", (n_env, n_t), device), BOOT_FULL


# ---------------------------------------------------------------------------------------
# ops.  Every argument is already contiguous; outputs are preallocated by the caller.
# ---------------------------------------------------------------------------------------
def gae(rewards, values, terminateds, truncateds, bootstrap, out, gamma, lambda_):
    dev = _device_of(rewards)
    shape = tuple(rewards.shape)
    n_env, n_t = shape
    args = [_require(rewards, "rewards", shape, dev), _require(values, "values", shape, dev),
            _require(terminateds, "terminateds", shape, dev),
            _opt(truncateds, "truncateds", shape, dev)]
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev)
    o = _require(out, "out", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_gae(*args, bp, mode, o, n_env, n_t, gamma, lambda_, ws, wsb,
                              L.stream.cuda_stream), "rlk_gae")
    return out


def vtrace(log_pi_target, log_pi_behavior, values, rewards, terminateds, truncateds, bootstrap,
           targets, advantages, gamma, rho_bar, c_bar):
    dev = _device_of(rewards)
    shape = tuple(rewards.shape)
    n_env, n_t = shape
    args = [_require(log_pi_target, "log_pi_target", shape, dev),
            _require(log_pi_behavior, "log_pi_behavior", shape, dev),
            _require(values, "values", shape, dev), _require(rewards, "rewards", shape, dev),
            _require(terminateds, "terminateds", shape, dev),
            _opt(truncateds, "truncateds", shape, dev)]
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev)
    tg = _require(targets, "targets", shape, dev)
    ad = _require(advantages, "advantages", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_vtrace(*args, bp, mode, tg, ad, n_env, n_t, gamma, rho_bar, c_bar, ws,
                                 wsb, L.stream.cuda_stream), "rlk_vtrace")
    return targets, advantages


def retrace(action_probs_target, action_probs_behavior, q_values, next_q_values_all, actions,
            rewards, terminateds, truncateds, targets, advantages, gamma, lambda_, c_bar, rho_bar):
    dev = _device_of(rewards)
    shape = tuple(rewards.shape)
    n_env, n_t = shape
    if action_probs_target.dim() != 3:
        raise ValueError("action_probs_target must be [num_envs, seq_len, num_actions]")
    n_act = action_probs_target.shape[2]
    shape3 = (n_env, n_t, n_act)
    args = [_require(action_probs_target, "action_probs_target", shape3, dev),
            _require(action_probs_behavior, "action_probs_behavior", shape, dev),
            _require(q_values, "q_values", shape, dev),
            _require(next_q_values_all, "next_q_values_all", shape3, dev),
            _require(actions, "actions", shape, dev, torch.int64),
            _require(rewards, "rewards", shape, dev),
            _require(terminateds, "terminateds", shape, dev),
            _opt(truncateds, "truncateds", shape, dev)]
    tg = _require(targets, "targets", shape, dev)
    ad = _require(advantages, "advantages", shape, dev)
    if n_act == 0 and n_env * n_t > 0:
        raise ValueError("num_actions must be positive")
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        if n_env * n_t == 0:
            return targets, advantages
        _check(load().rlk_retrace(*args, tg, ad, n_env, n_t, n_act, gamma, lambda_, c_bar, rho_bar,
                                  ws, wsb, L.stream.cuda_stream), "rlk_retrace")
    return targets, advantages


def lambda_returns(rewards, next_values, terminateds, truncateds, bootstrap, out, gamma, lambda_):
    dev = _device_of(rewards)
    shape = tuple(rewards.shape)
    n_env, n_t = shape
    args = [_require(rewards, "rewards", shape, dev),
            _require(next_values, "next_values", shape, dev),
            _require(terminateds, "terminateds", shape, dev),
            _opt(truncateds, "truncateds", shape, dev)]
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev)
    o = _require(out, "out", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_lambda_returns(*args, bp, mode, o, n_env, n_t, gamma, lambda_, ws, wsb,
                                         L.stream.cuda_stream), "rlk_lambda_returns")
    return out


def discounted_returns(rewards, terminateds, truncateds, bootstrap, out, gamma):
    dev = _device_of(rewards)
    shape = tuple(rewards.shape)
    n_env, n_t = shape
    args = [_require(rewards, "rewards", shape, dev),
            _require(terminateds, "terminateds", shape, dev),
            _opt(truncateds, "truncateds", shape, dev)]
    bp, mode = _boot_args(bootstrap, n_env, n_t, dev)
    o = _require(out, "out", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_discounted_returns(*args, bp, mode, o, n_env, n_t, gamma, ws, wsb,
                                             L.stream.cuda_stream), "rlk_discounted_returns")
    return out


def eligibility_traces(gradients, dones, seed, out, gamma, lambda_):
    dev = _device_of(gradients)
    shape = tuple(gradients.shape)
    n_env, n_t = shape
    g = _require(gradients, "gradients", shape, dev)
    d = _require(dones, "dones", shape, dev)
    s = _opt(seed, "seed_values", (n_env,), dev)
    o = _require(out, "out", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_eligibility_traces(g, d, s, o, n_env, n_t, gamma, lambda_, ws, wsb,
                                             L.stream.cuda_stream), "rlk_eligibility_traces")
    return out


def prefix_sum(inputs, dones, seed, out, ends_at):
    dev = _device_of(inputs)
    shape = tuple(inputs.shape)
    n_env, n_t = shape
    x = _require(inputs, "inputs", shape, dev)
    d = _require(dones, "dones", shape, dev)
    s = _opt(seed, "seed_values", (n_env,), dev)
    o = _require(out, "out", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_prefix_sum(x, d, s, o, n_env, n_t, int(bool(ends_at)), ws, wsb,
                                     L.stream.cuda_stream), "rlk_prefix_sum")
    return out


def affine_scan(u, v, carry, out, direction):
    dev = _device_of(u)
    shape = tuple(u.shape)
    n_env, n_t = shape
    up = _require(u, "u", shape, dev)
    vp = _require(v, "v", shape, dev)
    c = _opt(carry, "bootstrap" if direction == BACKWARD else "seed", (n_env,), dev)
    o = _require(out, "out", shape, dev)
    with _Launch(dev) as L:
        ws, wsb = _workspace(dev, L.stream, n_env, n_t)
        _check(load().rlk_affine_scan(up, vp, c, o, n_env, n_t, direction, ws, wsb,
                                      L.stream.cuda_stream), "rlk_affine_scan")
    return out
