"""GPU: router top-8 (ids exact, weights to 1e-5) and bucket fill (exact) vs the oracle."""
import numpy as np
import pytest

from gpu_util import E, log

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx(gpu):
    c = gpu.Context(2048, 512, E, 1, 4096, gpu.W_REF)
    yield c
    c.close()


@pytest.fixture(scope="module")
def ctx_renorm(gpu):
    c = gpu.Context(2048, 512, E, 1, 4096, gpu.W_RENORM)
    yield c
    c.close()


@pytest.mark.parametrize("M,kind", [(1, 0), (7, 0), (512, 1), (4096, 2)])
@pytest.mark.parametrize("mode", [0, 1])
def test_router_matches_oracle(gpu, orc, ctx, ctx_renorm, M, kind, mode):
    import torch
    log(f"router M={M} kind={kind} mode={mode}")
    logits = gpu.gen_logits(M, E, 1000 + M, kind, 1.1 if kind == 1 else 0.05, 1000.0)
    c = ctx if mode == 0 else ctx_renorm
    ids, w = c.router_topk(logits)
    torch.cuda.synchronize()
    rid, rw = orc.router_topk(logits.cpu().numpy(), mode)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-30)


def test_router_edge_cases(gpu, orc, ctx):
    import torch
    log("router edge cases")
    l = np.zeros((6, E), dtype=np.float32)
    l[1, :] = np.nan
    l[1, [5, 9]] = [1.0, 2.0]
    l[2, [3, 40]] = np.inf
    l[3, :] = -np.inf
    l[4, ::2] = -0.0
    l[5, :] = np.arange(E)[::-1] % 7
    ids, w = ctx.router_topk(torch.from_numpy(l).cuda())
    torch.cuda.synchronize()
    rid, rw = orc.router_topk(l, 0)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=0)


def test_router_empty(gpu, ctx):
    import torch
    ids, w = ctx.router_topk(torch.empty((0, E), device="cuda"))
    torch.cuda.synchronize()
    assert ids.numel() == 0


@pytest.mark.parametrize("M", [0, 1, 9, 63, 64, 65, 512, 1024, 1025, 3000, 4096])
def test_bucket_fill_matches_oracle(gpu, orc, ctx, M):
    import torch
    log(f"bucket fill M={M}")
    logits = gpu.gen_logits(max(M, 1), E, 2000 + M, 1, 1.1)[:M]
    ids, w = ctx.router_topk(logits)
    ranges, stok, sw = ctx.bucket_fill(ids, w)
    torch.cuda.synchronize()
    rr, rt, rsw, _ = orc.bucket_fill(ids.cpu().numpy(), w.cpu().numpy(), E)
    assert np.array_equal(ranges.cpu().numpy().astype(np.int64), rr.astype(np.int64))
    assert np.array_equal(stok.cpu().numpy(), rt)
    assert np.array_equal(sw.cpu().numpy().view(np.uint32), rsw.view(np.uint32))
    assert ctx.device_flags() == 0


def test_bucket_fill_flags_invalid_ids(gpu, ctx):
    import torch
    log("bucket fill invalid ids")
    M = 70
    ids = torch.from_numpy(np.tile(np.arange(9, dtype=np.uint16), (M, 1))).cuda()
    w = torch.ones((M, 9), dtype=torch.float32, device="cuda")
    ids_bad = ids.clone()
    ids_bad[3, 2] = E + 7        # out of range
    ids_bad[5, 4] = ids_bad[5, 1]  # duplicate inside one token
    ranges, stok, sw = ctx.bucket_fill(ids_bad, w)
    f = ctx.device_flags()
    assert f & gpu.DEVFLAG_BAD_ID and f & gpu.DEVFLAG_DUP_ID
    r = ranges.cpu().numpy()
    assert r[-1] == 9 * M - 2 and np.all(np.diff(r) >= 0)
    ranges, stok, sw = ctx.bucket_fill(ids, w)
    assert ctx.device_flags() == 0


# ---------------------------------------------------------------- router gate GEMV

def _router_gemv_case(gpu, orc, c, E_, H_, M, seed, rmsnorm, dense=None):
    """dense: None for an IQ4_XS gate matrix, or np.float32 / np.float16 for an unquantized one."""
    import torch
    if dense is None:
        wg = gpu.gen_iq4xs(E_ * H_ // 256, seed)
        wg_h = None
    else:
        wg_h = (np.random.default_rng(seed).standard_normal((E_, H_)) * 0.05).astype(dense)
        wg = torch.from_numpy(wg_h).cuda()
    x = gpu.gen_normal(M * H_, seed ^ 0x58, 0, 0.0, 1.0).view(M, H_)
    lg, ids, w = c.router_gemv_topk(wg, x, rmsnorm=rmsnorm)
    torch.cuda.synchronize()
    ref = orc.router_gemv(wg.cpu().numpy() if wg_h is None else wg_h, x.cpu().numpy(), E_,
                          flags=2 if rmsnorm else 0)
    got = lg.cpu().numpy()
    # f32 sums of exact weights: within 1e-5 of each row's logit scale
    scale = np.maximum(np.abs(ref).max(axis=1, keepdims=True), 1.0)
    assert np.all(np.abs(got - ref) <= 1e-5 * scale)
    # the fused top-8 is moe_router_topk of the GEMV's own logits, bit for bit
    ids2, w2 = c.router_topk(lg)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids2.cpu().numpy())
    assert np.array_equal(w.cpu().numpy().view(np.uint32), w2.cpu().numpy().view(np.uint32))
    # against the oracle's routing of the oracle's logits, on every token whose sorted top-9
    # logits are separated by more than the logits' tolerance: ids exact; weights within what
    # the logit error allows (w_i = exp(l_i - l_max) / sum: a logit error d moves w_i by at most
    # 2 max|d| relative, to first order) plus the softmax's own 1e-5
    rid, rw = orc.router_topk(ref, c.wmode)
    top9 = -np.sort(-ref, axis=1)[:, :9]
    clear = np.all(-np.diff(top9, axis=1) > 2e-5 * scale, axis=1)
    assert clear.mean() > 0.9
    gi, gw = ids.cpu().numpy(), w.cpu().numpy()
    assert np.array_equal(gi[clear], rid[clear])
    d = np.abs(got - ref).max(axis=1, keepdims=True).astype(np.float64)
    rtol = 2.5 * d + 1e-5
    err = np.abs(gw.astype(np.float64) - rw)
    assert np.all((err <= rtol * np.abs(rw) + 1e-37)[clear])
    return got


@pytest.mark.parametrize("M", [1, 5, 64, 300])
@pytest.mark.parametrize("rmsnorm", [False, True])
def test_router_gemv_matches_oracle(gpu, orc, ctx, ctx_renorm, M, rmsnorm):
    log(f"router gemv E={E} H=2048 M={M} rmsnorm={rmsnorm}")
    _router_gemv_case(gpu, orc, ctx if M % 2 else ctx_renorm, E, 2048, M, 0x52470000 + M, rmsnorm)


@pytest.mark.parametrize("M", [1, 2, 8, 9, 64])
@pytest.mark.parametrize("dense", [np.float32, np.float16])
def test_router_gemv_dense_matches_oracle(gpu, orc, ctx, ctx_renorm, M, dense):
    """Unquantized gate matrices (a GGUF ffn_gate_inp as llama.cpp leaves it), f32 and f16, at
    M from 1 to 64 (1, 2 and 4 tokens per wave)."""
    log(f"router gemv dense {np.dtype(dense).name} E={E} H=2048 M={M}")
    _router_gemv_case(gpu, orc, ctx if M % 2 else ctx_renorm, E, 2048, M, 0x52480000 + M, True, dense=dense)


@pytest.mark.parametrize("M", [1, 7])
def test_router_gemv_small_shape(gpu, orc, M):
    log(f"router gemv E=16 H=512 M={M}")
    c = gpu.Context(512, 256, 16, 1, 64, gpu.W_RENORM)
    try:
        _router_gemv_case(gpu, orc, c, 16, 512, M, 0x52471000 + M, True)
    finally:
        c.close()


def test_router_gemv_outputs_and_errors(gpu, orc, ctx):
    import torch
    log("router gemv: logits-only, ids-only, bad flags")
    wg = gpu.gen_iq4xs(E * 2048 // 256, 0x5247AAAA)
    x = gpu.gen_normal(3 * 2048, 0x5247AAAB).view(3, 2048)
    lg, ids, w = ctx.router_gemv_topk(wg, x)
    lg1, n1, n2 = ctx.router_gemv_topk(wg, x, want_ids=False)
    n3, ids1, w1 = ctx.router_gemv_topk(wg, x, want_logits=False)
    torch.cuda.synchronize()
    assert n1 is None and n2 is None and n3 is None
    assert np.array_equal(lg.cpu().numpy(), lg1.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), ids1.cpu().numpy())
    assert np.array_equal(w.cpu().numpy(), w1.cpu().numpy())
    L = gpu.lib()
    for flags in (1, 4):
        assert L.moe_router_gemv_topk(ctx._h, wg.data_ptr(), x.data_ptr(), 3, flags, lg.data_ptr(), None, None,
                                      None) == gpu.MOE_EINVAL
    assert L.moe_router_gemv_topk(ctx._h, wg.data_ptr(), x.data_ptr(), 3, 0, None, None, None, None) == gpu.MOE_EINVAL
    assert L.moe_router_gemv_topk(ctx._h, wg.data_ptr() + 4, x.data_ptr(), 3, 0, lg.data_ptr(), None, None,
                                  None) == gpu.MOE_EINVAL


def test_router_gemv_graph_replays(gpu, ctx):
    """Replays of a captured moe_router_gemv_topk (GEMV + top-8), with eager calls of another
    M in between, each give the eager result bit for bit."""
    import torch
    log("router gemv + top-8: graph capture, 4 replays")
    wg = gpu.gen_iq4xs(E * 2048 // 256, 0x5249)
    x = gpu.gen_normal(3 * 2048, 0x524A).view(3, 2048)
    x5 = gpu.gen_normal(5 * 2048, 0x524B).view(5, 2048)
    lg0, ids0, w0 = (t.clone() for t in ctx.router_gemv_topk(wg, x))
    torch.cuda.synchronize()
    lg = torch.empty_like(lg0)
    ids = torch.empty_like(ids0)
    w = torch.empty_like(w0)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ctx.router_gemv_topk(wg, x, logits=lg, ids=ids, w=w, stream=s)
    torch.cuda.synchronize()
    for rep in range(4):
        lg.fill_(float("nan"))
        ids.zero_()
        w.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(lg.view(torch.int32), lg0.view(torch.int32)), rep
        assert torch.equal(ids, ids0) and torch.equal(w.view(torch.int32), w0.view(torch.int32)), rep
        ctx.router_gemv_topk(wg, x5)        # an eager call of another M in between
        torch.cuda.synchronize()
