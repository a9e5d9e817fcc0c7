"""GPU: moe_ffn_noalloc (the decode path of moe_ffn with its h scratch in a static device
array, for callers that cannot allocate) against moe_ffn on the same inputs: two calls in a
row, the second with fewer tokens, each bit-identical to moe_ffn's output (same kernels, only
the scratch differs).  Runs alone in a fresh process or after the other GPU tests."""
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
    for M, flags in ((8, 3), (3, 2)):
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
