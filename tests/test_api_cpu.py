"""CPU-side checks of the boundary: the C-ABI library and the drop-in API contract.

No kernel runs here.  The library is loaded (a HIP fat binary loads without a GPU), its
exported symbols are compared with include/rl_triton_amd.h, host-only entry points are
called, and the reference's always-on AssertionErrors are raised on CPU tensors before
any launch (ops/gae.py:106-129 and the matching blocks of the other ops).
"""
import ctypes
import os
import re

import pytest
import torch

import rl_triton
from rl_triton import _native
from rl_triton.ops._scan import _FLAT_MAX_SEQ_LEN, _run_scan, _run_scan_forward
from rl_triton.ops.retrace_fused import compute_retrace_fused
from rl_triton.ops.vtrace_fused import compute_vtrace_fused

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rl_triton_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char \*)\s*(rlk_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_native.library_path())
    names = _declared()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), f"{name} declared in rl_triton_amd.h but not exported"
    assert set(names) == set(_native.SIGNATURES), "binding signatures out of sync with the header"


@pytest.mark.parametrize("lang", ["c", "c++"])
def test_headers_compile_as_plain_c_and_cpp(lang, tmp_path):
    """The C ABI headers need nothing beyond the C standard headers: a C99 (and a C++17)
    translation unit that includes them compiles with every warning an error."""
    import subprocess
    src = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    src.write_text('#include "rl_triton_amd.h"\n#include "rlk_stream_ceiling.h"\n'
                   "int main(void) { return rlk_version() > 0 ? 0 : 1; }\n")
    cc, std = ("gcc", "-std=c99") if lang == "c" else ("g++", "-std=c++17")
    r = subprocess.run([cc, std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


CEILING_HEADER = os.path.join(ROOT, "include", "rlk_stream_ceiling.h")
CEILING_LIB = os.path.join(ROOT, "rl-triton_amd", "rl_triton", "librlk_stream_ceiling.so")


def test_stream_ceiling_library_exports_and_rejects_bad_arguments():
    """The benchmark's streaming-ceiling library: its one declared symbol is exported and
    invalid arguments are refused before any launch."""
    text = open(CEILING_HEADER).read()
    names = re.findall(r"^\s*int\s+(rlk_\w+)\s*\(", text, re.M)
    assert names == ["rlk_stream_ceiling"]
    lib = ctypes.CDLL(CEILING_LIB)
    fn = lib.rlk_stream_ceiling
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                   ctypes.c_int, ctypes.c_int64, ctypes.c_void_p]
    P = ctypes.c_void_p
    ins, outs = (P * 6)(*[16 * (i + 1) for i in range(6)]), (P * 2)(1024, 2048)
    assert fn(ins, 0, outs, 1, 16, None) == -1          # no inputs
    assert fn(ins, 7, outs, 1, 16, None) == -1          # too many inputs
    assert fn(ins, 5, outs, 3, 16, None) == -1          # too many outputs
    assert fn(ins, 5, outs, 1, 18, None) == -1          # n not a multiple of 4
    assert fn(ins, 5, outs, 1, -4, None) == -1
    assert fn((P * 1)(8), 1, outs, 1, 16, None) == -1   # misaligned input
    assert fn((P * 1)(None), 1, outs, 1, 16, None) == -1
    assert fn(ins, 5, outs, 2, 0, None) == 0            # empty: no launch


def test_host_only_entry_points():
    lib = _native.load()
    assert lib.rlk_version() >= 100
    assert lib.rlk_status_string(0) == b"ok"
    assert b"workspace" in lib.rlk_status_string(-2)
    # short rows need no workspace; long rows need one, growing with the tile count
    assert lib.rlk_workspace_bytes(4096, 128) == 0
    assert lib.rlk_workspace_bytes(256, 2048) == 0
    a = lib.rlk_workspace_bytes(8, 1 << 20)
    b = lib.rlk_workspace_bytes(16, 1 << 20)
    assert 0 < a < b and a % 8 == 0
    assert lib.rlk_workspace_bytes(0, 1 << 20) == 0
    # 80 B per 4096-step tile of every row, whatever the row's alignment
    w = lib.rlk_workspace_bytes
    assert w(1, 8192) == w(1, 4097) == w(1, 8189) and w(1, 8193) - w(1, 8192) == 80
    assert w(3, 8191) == w(3, 8192) and w(3, 8193) - w(3, 8192) == 240


def test_entry_points_reject_bad_arguments_without_launching():
    lib = _native.load()
    # empty shapes succeed with null pointers; missing required pointers are refused
    assert lib.rlk_gae(None, None, None, None, None, 0, None, 0, 128, 0.99, 0.95, None, 0, None) == 0
    assert lib.rlk_gae(None, None, None, None, None, 0, None, 4, 128, 0.99, 0.95, None, 0, None) == -1
    assert lib.rlk_prefix_sum(None, None, None, None, 4, 4, 1, None, 0, None) == -1
    assert lib.rlk_affine_scan(None, None, None, None, 2, 8, 7, None, 0, None) == -1
    fake = ctypes.c_void_p(16)  # never dereferenced: the call fails before any launch
    # invalid bootstrap mode / missing bootstrap pointer
    assert lib.rlk_gae(fake, fake, fake, None, None, 2, fake, 4, 8, 0.99, 0.95, None, 0, None) == -1
    assert lib.rlk_gae(fake, fake, fake, None, fake, 9, fake, 4, 8, 0.99, 0.95, None, 0, None) == -1
    # long rows without a workspace
    assert lib.rlk_prefix_sum(fake, fake, None, fake, 2, 1 << 20, 1, None, 0, None) == -2
    # masked entry points need their mask; the bfloat16 twins check like their float32 ones
    assert lib.rlk_gae_masked(fake, fake, fake, None, None, 0, None, fake, 4, 8, 0.99, 0.95,
                              None, 0, None) == -1
    assert lib.rlk_gae_normalized_masked(fake, fake, fake, None, None, 0, None, fake, fake, 4, 8,
                                         0.99, 0.95, 1e-8, None, 0, fake, 1 << 20, None) == -1
    assert lib.rlk_gae_bf16(fake, fake, fake, None, fake, 9, fake, 4, 8, 0.99, 0.95, None, 0,
                            None) == -1
    assert lib.rlk_prefix_sum_bf16(fake, fake, None, fake, 2, 1 << 20, 1, None, 0, None) == -2
    assert lib.rlk_affine_scan_bf16(None, None, None, None, 2, 8, 7, None, 0, None) == -1
    # empty shapes are a no-op for every twin
    for name in ("rlk_gae_bf16", "rlk_gae_masked", "rlk_gae_masked_bf16"):
        argc = len(_native.SIGNATURES[name])
        args = [None] * argc
        i_e = [i for i, t in enumerate(_native.SIGNATURES[name]) if t is ctypes.c_int64]
        args[i_e[0]], args[i_e[1]] = 0, 8
        for i, t in enumerate(_native.SIGNATURES[name]):
            if args[i] is None and t is not ctypes.c_void_p:
                args[i] = 0
        assert getattr(lib, name)(*args) == 0, name
    # a normalised call's partials must hold three float64 per workgroup of the first launch
    # (512-thread workgroups of 16 rows at T = 128, 4 at T = 300, 256 one-step rows), then,
    # above 2048 of them, one per 2048 for each level of the tree that sums them
    need = lib.rlk_gae_normalized_partials_bytes(4096, 128)
    assert need == 256 * 24
    p = lib.rlk_gae_normalized_partials_bytes
    assert p(8192, 300) == 2048 * 24 and p(8193, 300) == (2049 + 2) * 24
    assert p(65536, 128) == (4096 + 2) * 24
    assert p(4096 * 524291, 1) == (8388656 + 4097 + 3) * 24
    # beyond one launch (2^32 work-items): two launches over 268434944 and 4608 rows of
    # 64 per workgroup, one partial per workgroup of each
    assert p(4096 * 65537, 3) == (4194296 + 72 + 2049 + 2) * 24
    assert lib.rlk_gae_normalized(fake, fake, fake, None, None, 0, fake, fake, 4096, 128, 0.99,
                                  0.95, 1e-8, None, 0, fake, need - 8, None) == -2


def _cpu(*shape):
    return torch.zeros(*shape)


def test_gae_reference_assertions():
    r = _cpu(4, 16)
    with pytest.raises(AssertionError, match="rewards must be on CUDA"):
        rl_triton.compute_gae(r, r, r)


def test_vtrace_reference_assertions():
    r = _cpu(4, 16)
    with pytest.raises(AssertionError, match="log_pi_target must be on CUDA"):
        rl_triton.compute_vtrace(r, r, r, r, r)
    with pytest.raises(AssertionError, match="log_pi_target must be on CUDA"):
        compute_vtrace_fused(r, r, r, r, r)


def test_retrace_and_returns_reference_assertions():
    r = _cpu(4, 16)
    a3 = _cpu(4, 16, 2)
    act = torch.zeros(4, 16, dtype=torch.int64)
    with pytest.raises(AssertionError, match="must be on CUDA"):
        rl_triton.compute_retrace(a3, r, r, a3, act, r, r, r, gamma=0.99)
    with pytest.raises(AssertionError, match="rewards must be on CUDA"):
        rl_triton.compute_lambda_returns(r, r, r)
    with pytest.raises(AssertionError, match="rewards must be on CUDA"):
        rl_triton.compute_discounted_returns(r, r)
    with pytest.raises(AssertionError, match="gradients and dones must be on CUDA"):
        rl_triton.compute_eligibility_traces(r, r, 0.99, 0.95)


def test_flag_gated_paths_still_refuse_cpu_tensors(monkeypatch):
    """Prefix sum and _run_scan check only under RL_TRITON_CORRECTNESS_WARNINGS (as in the
    reference); without it the GPU binding itself refuses host tensors."""
    monkeypatch.setenv("RL_TRITON_CORRECTNESS_WARNINGS", "0")
    r = _cpu(4, 16)
    with pytest.raises(ValueError, match="GPU tensors"):
        rl_triton.compute_episodic_prefix_sum(r, r)
    with pytest.raises(ValueError, match="GPU tensors"):
        _run_scan(r, r)
    with pytest.raises(ValueError, match="GPU tensors"):
        _run_scan_forward(r, r)
    with pytest.raises(ValueError, match="boundary"):
        rl_triton.compute_episodic_prefix_sum(r, r, boundary="middle")
    monkeypatch.setenv("RL_TRITON_CORRECTNESS_WARNINGS", "1")
    with pytest.raises(AssertionError, match="must be on CUDA"):
        rl_triton.compute_episodic_prefix_sum(r, r)


def test_public_surface_matches_reference():
    assert rl_triton.__version__ == "0.1.3"
    reference = ["compute_discounted_returns", "compute_eligibility_traces",
                 "compute_episodic_prefix_sum", "compute_gae", "compute_lambda_returns",
                 "compute_retrace", "compute_vtrace"]
    # the reference's seven functions, plus one extension it lists on its ROADMAP.md:75-81
    assert sorted(rl_triton.__all__) == sorted(reference + ["compute_gae_normalized"])
    assert _FLAT_MAX_SEQ_LEN == 131072
    assert callable(compute_retrace_fused)


def test_fast_path_declines_cpu_tensors():
    """The C++ fast path takes GPU tensors only; CPU calls reach the Python path and its
    reference assertions."""
    from rl_triton import _native
    if _native.fast is None:
        pytest.skip("rl_triton._rlk_torch is not built")
    x = torch.zeros(4, 8)
    f = _native.fast
    assert f.gae(x, x, x, None, 0.99, 0.95, None, None, None) is None
    assert f.vtrace(x, x, x, x, x, None, 0.99, 1.0, 1.0, None, None) is None
    assert f.prefix_sum(x, x, None, True) is None
    assert f.affine_scan(x, x, None, 0) is None
    with pytest.raises(TypeError):
        f.gae(x)
    import rl_triton
    with pytest.raises(AssertionError, match="must be on CUDA"):
        rl_triton.compute_gae(x, x, x)


def test_gae_normalized_checks_match_compute_gae():
    """compute_gae_normalized raises compute_gae's assertions: both call one check helper."""
    from rl_triton.ops.gae import _check_gae_args

    class _Gpu:  # passes the device, dtype and shape checks without a GPU
        def __init__(self, *shape):
            self.shape, self.is_cuda, self.dtype = torch.Size(shape), True, torch.float32

    x = torch.zeros(4, 8)
    for fn in (rl_triton.compute_gae, rl_triton.compute_gae_normalized):
        with pytest.raises(AssertionError, match="rewards must be on CUDA"):
            fn(x, x, x)
    t = _Gpu(4, 8)
    with pytest.raises(AssertionError, match="not both"):
        _check_gae_args(t, t, t, None, t, _Gpu(4))
    with pytest.raises(AssertionError, match="cannot be combined with truncateds"):
        _check_gae_args(t, t, t, t, None, _Gpu(4))


def test_workspace_call_limit_is_below_the_epoch_wrap():
    """The call limit between zero-fills of a workspace (RLK_WORKSPACE_MAX_CALLS, mirrored by
    the Python binding) is below the 2^30 calls after which the status words' call count
    (kEpochMask in the engine) wraps."""
    text = open(HEADER).read()
    limit = int(eval(re.search(r"#define RLK_WORKSPACE_MAX_CALLS \(([^)]*)\)", text).group(1)))
    engine = open(os.path.join(ROOT, "rl-triton_amd", "csrc", "rlk_engine.hpp")).read()
    mask = int(re.search(r"kEpochMask = (0x[0-9a-fA-F]+)u", engine).group(1), 16)
    assert limit == _native.WORKSPACE_MAX_CALLS == 1 << 29
    assert limit < mask + 1


def test_workspace_rezeroed_at_call_limit(monkeypatch):
    """A cached workspace that has served WORKSPACE_MAX_CALLS long-row calls is zero-filled
    before the next one (here on a CPU stand-in with the limit lowered to 3)."""
    monkeypatch.setattr(_native, "WORKSPACE_MAX_CALLS", 3)
    key = ("cpu-test", 0)
    monkeypatch.setitem(_native._ws_calls, key, 0)
    ws = torch.full((64,), 7, dtype=torch.uint8)
    zeroed_before = []
    for call in range(1, 11):
        _native._count_call(key, ws)
        zeroed_before.append(bool((ws == 0).all()))
        ws.fill_(7)
    assert [c for c, z in zip(range(1, 11), zeroed_before) if z] == [4, 7, 10]
    del _native._ws_calls[key]


def test_noalloc_entry_refuses_before_any_device_call():
    """rlk_gae_noalloc checks sizes on the host: a call whose look-back status words exceed
    its static buffer, or with negative sizes, is refused without a HIP call (so also here,
    without a GPU); an empty call is a no-op."""
    lib = _native.load()
    p = 4096  # never dereferenced
    assert lib.rlk_gae_noalloc(p, p, p, None, None, 0, p, 4096, 16384, 0.99, 0.95, None) == -4
    assert lib.rlk_gae_noalloc(p, p, p, None, None, 0, p, -1, 5000, 0.99, 0.95, None) == -1
    assert lib.rlk_gae_noalloc(None, None, None, None, None, 0, None, 0, 5000, 0.99, 0.95, None) == 0
    assert b"static buffer" in lib.rlk_status_string(-4)
    assert b"device" in lib.rlk_status_string(-5)
