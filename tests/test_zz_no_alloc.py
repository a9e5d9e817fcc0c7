"""GPU: moe_ffn_noalloc (the decode path of moe_ffn with its h scratch in a static device
array, for callers that cannot allocate) against moe_ffn on the same inputs: calls in a row,
each with fewer tokens than the one before (M = 8 down to the M = 1 kernels, which use no
plan block), each bit-identical to moe_ffn's output (same kernels, only the scratch differs);
no device memory taken by the calls; replays of a graph that captured a call.  Runs alone in
a fresh process or after the other GPU tests."""
import ctypes

import pytest

from gpu_util import E, H, I, log

pytestmark = pytest.mark.gpu


def noalloc(gpu):
    L = gpu.lib()
    fn = L.moe_ffn_noalloc
    vp, i = ctypes.c_void_p, ctypes.c_int
    fn.argtypes = [vp, i, vp, vp, vp, i, vp, i, vp]
    fn.restype = ctypes.c_int
    return fn


@pytest.fixture(scope="module")
def ctx(gpu):
    c = gpu.Context(H, I, E, 1, 8, gpu.W_RENORM)
    c.bind_packed(0, gpu.gen_layer(H, I, E, gpu.seed_for(0, 0, gpu.TAG_W)))
    yield c
    c.close()


def test_noalloc_matches_moe_ffn(gpu, ctx):
    import torch
    fn = noalloc(gpu)
    stream = torch.cuda.current_stream().cuda_stream
    for M, flags in ((8, 3), (3, 2), (2, 1), (1, 0), (1, 3)):
        log(f"moe_ffn_noalloc M={M} flags={flags}")
        x = gpu.gen_normal(M * H, 5000 + M).view(M, H)
        ids, w = ctx.router_topk(gpu.gen_logits(M, E, 5100 + M))
        y0 = gpu.gen_normal(M * H, 5200 + M).view(M, H)
        want = y0.clone()
        ctx.ffn(0, x, ids, w, y=want, accumulate=bool(flags & 1), rmsnorm=bool(flags & 2))
        got = y0.clone()
        st = fn(ctx.handle, 0, x.data_ptr(), ids.data_ptr(), w.data_ptr(), M, got.data_ptr(), flags, stream)
        assert st == gpu.MOE_OK, gpu.lib().moe_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))
        assert ctx.device_flags() == 0


def test_noalloc_rejects_sizes_beyond_its_scratch(gpu, ctx):
    import torch
    fn = noalloc(gpu)
    x = torch.zeros((9, H), device="cuda")
    ids = torch.zeros((9, 9), dtype=torch.uint16, device="cuda")
    w = torch.zeros((9, 9), device="cuda")
    st = fn(ctx.handle, 0, x.data_ptr(), ids.data_ptr(), w.data_ptr(), 9, x.data_ptr(), 0, None)
    assert st == gpu.MOE_EINVAL
    assert b"static scratch" in gpu.lib().moe_last_error()


def test_noalloc_allocates_nothing_and_captures(gpu, ctx):
    """Calls take no device memory (free memory unchanged around them, with every tensor they
    use allocated first), and a call captured into a HIP graph replays to the eager result
    bit for bit, with eager calls of another M between the replays."""
    import torch
    fn = noalloc(gpu)
    M = 4
    x = gpu.gen_normal(M * H, 5300).view(M, H)
    ids, w = ctx.router_topk(gpu.gen_logits(M, E, 5301))
    x2 = gpu.gen_normal(2 * H, 5302).view(2, H)
    ids2, w2 = ctx.router_topk(gpu.gen_logits(2, E, 5303))
    eager = torch.empty_like(x)
    y = torch.empty_like(x)
    y2 = torch.empty_like(x2)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        assert fn(ctx.handle, 0, x.data_ptr(), ids.data_ptr(), w.data_ptr(), M, eager.data_ptr(), 2,
                  stream) == gpu.MOE_OK
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    log("moe_ffn_noalloc under graph capture, 3 replays")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            st = fn(ctx.handle, 0, x.data_ptr(), ids.data_ptr(), w.data_ptr(), M, y.data_ptr(), 2,
                    s.cuda_stream)
    assert st == gpu.MOE_OK, gpu.lib().moe_last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), eager.view(torch.int32)), rep
        # an eager call of another M between replays (it rewrites the shared scratch)
        assert fn(ctx.handle, 0, x2.data_ptr(), ids2.data_ptr(), w2.data_ptr(), 2, y2.data_ptr(), 0,
                  stream) == gpu.MOE_OK
        torch.cuda.synchronize()
    assert ctx.device_flags() == 0
