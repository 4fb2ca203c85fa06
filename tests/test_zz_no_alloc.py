"""ckh_amax_scale_noalloc (the entry point that allocates nothing) against ckh_amax_scale.

Both are called through the C ABI with ctypes, on torch's current stream.  The two must
agree bit for bit on consecutive calls, the second on a smaller input than the first:
the no-allocation variant keeps its per-workgroup partial maxima in one device array
per GPU that the previous call left filled, so a stale word would show as a wrong
(too large) amax on the smaller call.
"""
import pytest
import torch

import comfy_kitchen.backends.hip as hb
from comfy_kitchen.ops import DTYPE_TO_CODE

pytestmark = pytest.mark.gpu


def _with_workspace(lib, x, divisor):
    out = torch.empty((), dtype=torch.float32, device=x.device)
    work = torch.empty(hb.AMAX_WORKSPACE_BYTES // 4, dtype=torch.int32, device=x.device)
    rc = lib.ckh_amax_scale(x.data_ptr(), x.numel(), DTYPE_TO_CODE[x.dtype], divisor, out.data_ptr(),
                            work.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.ckh_last_error()
    return out


def _no_alloc(lib, x, divisor):
    out = torch.empty((), dtype=torch.float32, device=x.device)
    rc = lib.ckh_amax_scale_noalloc(x.data_ptr(), x.numel(), DTYPE_TO_CODE[x.dtype], divisor, out.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.ckh_last_error()
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("divisor", [448.0, 2688.0])
def test_no_alloc_matches_workspace_entry_point(dtype, divisor, hip):
    lib = hb.load_library()
    g = torch.Generator().manual_seed(7)
    big = (torch.randn(8192 * 5120, generator=g) * 0.5).to(dtype)
    big[12345] = 900.0  # the first call's amax, far above anything in the second input
    small = (torch.randn(300_001, generator=g) * 0.5).to(dtype)
    small[-1] = -3.5
    for x in (big.cuda(), small.cuda()[1:]):  # the second call: smaller and misaligned
        want = _with_workspace(lib, x, divisor)
        got = _no_alloc(lib, x, divisor)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (float(got), float(want))
    assert float(got) == float((torch.amax(small[1:].abs().cuda()) / divisor).float())


def test_no_alloc_under_graph_capture(hip):
    """The callers it is for: captured in a HIP graph (after one eager call on the device,
    which resolves the array's address), two calls of different sizes, the graph replayed
    several times with eager work that changes the inputs between replays; every replay's
    scales equal the workspace entry point's on the same inputs."""
    lib = hb.load_library()
    g = torch.Generator().manual_seed(11)
    big = torch.randn(4096 * 3072, generator=g).bfloat16().cuda()
    small = (torch.randn(70_001, generator=g) * 3).bfloat16().cuda()
    _no_alloc(lib, small, 448.0)  # the first call on this device: outside capture
    torch.cuda.synchronize()
    outs = [torch.zeros((), dtype=torch.float32, device="cuda") for _ in range(2)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for x, o in zip((big, small), outs):
                rc = lib.ckh_amax_scale_noalloc(x.data_ptr(), x.numel(), DTYPE_TO_CODE[x.dtype], 448.0, o.data_ptr(),
                                                stream.cuda_stream)
                assert rc == 0, lib.ckh_last_error()
    torch.cuda.synchronize()
    for rep in range(4):
        big.mul_(1.5 if rep % 2 else 0.75)
        small[rep * 1000] = 50.0 * (rep + 1)  # the small input's amax changes every replay
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for x, o in zip((big, small), outs):
            want = _with_workspace(lib, x, 448.0)
            torch.cuda.synchronize()
            assert torch.equal(o.view(torch.int32), want.view(torch.int32)), (rep, float(o), float(want))
    assert float(outs[1]) == float((torch.amax(small.abs()) / 448.0).float())
