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
