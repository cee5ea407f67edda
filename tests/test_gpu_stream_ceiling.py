"""The benchmark's streaming-ceiling kernel (librlk_stream_ceiling.so) writes what its
header promises: output k = (k + 1) * the sum of the inputs, over every element, for each
read/write count the library accepts, including a grid whose last workgroup is partial."""
import ctypes
import os

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "rl-triton_amd", "rl_triton", "librlk_stream_ceiling.so")

pytestmark = pytest.mark.gpu


def _fn():
    fn = ctypes.CDLL(LIB).rlk_stream_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                   ctypes.c_int, ctypes.c_int64, ctypes.c_void_p]
    return fn


@pytest.mark.parametrize("n", [4, 2048 + 4, 4096 * 128])
@pytest.mark.parametrize("n_in,n_out", [(1, 1), (2, 1), (5, 1), (5, 2), (6, 2)])
def test_stream_ceiling_writes_the_sum(n, n_in, n_out):
    print(f"stream ceiling n={n} reads={n_in} writes={n_out}", flush=True)
    fn = _fn()
    g = torch.Generator().manual_seed(n + 10 * n_in + n_out)
    ins = [torch.randn(n, generator=g).cuda() for _ in range(n_in)]
    outs = [torch.full((n + 4,), 7.0, device="cuda") for _ in range(n_out)]
    P = ctypes.c_void_p
    stream = P(torch.cuda.current_stream().cuda_stream)
    rc = fn((P * n_in)(*[t.data_ptr() for t in ins]), n_in,
            (P * n_out)(*[t.data_ptr() for t in outs]), n_out, n, stream)
    assert rc == 0
    torch.cuda.synchronize()
    total = sum(t.double() for t in ins).float()
    for k, o in enumerate(outs):
        torch.testing.assert_close(o[:n], total * (k + 1), rtol=1e-6, atol=1e-5)
        assert torch.equal(o[n:], torch.full((4,), 7.0, device="cuda")), "wrote past n"
