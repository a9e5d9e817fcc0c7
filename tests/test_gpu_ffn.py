"""GPU: the expert FFN + combine vs the f64 oracle on identical seeded inputs.

Tolerances (normwise, max|y - ref| / max|ref|): decode (M <= 8, f32 arithmetic) 1e-3;
prefill (bf16 MFMA operands, f32 accumulate) 5e-3 -- the bounds BASELINE.json states.
"""
import numpy as np
import pytest

from gpu_util import E, H, I, Layer, log, normwise_err

pytestmark = pytest.mark.gpu

TOL_DECODE = 1e-3
TOL_PREFILL = 5e-3


def run_case(gpu, orc, ctx, layer, M, seed, kind=0, param=0.0, hot=0.0, flags=0, mode=0,
             subset=None):
    import torch
    hidden, E_ = ctx.hidden, ctx.n_experts
    x = gpu.gen_normal(M * hidden, seed).view(M, hidden)
    logits = gpu.gen_logits(M, E_, seed + 1, kind, param, hot)
    ids, w = ctx.router_topk(logits)
    y0 = gpu.gen_normal(M * hidden, seed + 2).view(M, hidden)
    y = y0.clone()
    ctx.ffn(0, x, ids, w, y=y, accumulate=bool(flags & 1), rmsnorm=bool(flags & 2))
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    c = 1.0 / 9 if mode == 0 else 1.0
    xs, ids_h, w_h, y0_h, y_h = (t.cpu().numpy() for t in (x, ids, w, y0, y))
    if subset is not None:
        xs, ids_h, w_h, y0_h, y_h = xs[subset], ids_h[subset], w_h[subset], y0_h[subset], y_h[subset]
    ref = orc.moe_ffn(layer.host(), xs, ids_h, w_h, c, flags, y=y0_h if flags & 1 else None)
    if flags & 1:  # compare the FFN part, not the residual
        return normwise_err(y_h - y0_h, ref - y0_h), y
    return normwise_err(y_h, ref), y


# ---------------------------------------------------------------- small shape, brute force

@pytest.fixture(scope="module")
def small(gpu, orc):
    ctx = gpu.Context(512, 256, 16, 1, 256, gpu.W_REF)
    layer = Layer(gpu, orc, 31, 512, 256, 16)
    ctx.bind_packed(0, layer.dev)
    yield ctx, layer
    ctx.close()


@pytest.mark.parametrize("M", [1, 2, 5, 8, 9, 37, 200])
@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_small_shape(gpu, orc, small, M, flags):
    ctx, layer = small
    log(f"small H=512 I=256 E=16 M={M} flags={flags}")
    err, _ = run_case(gpu, orc, ctx, layer, M, 100 + M, flags=flags)
    log(f"  normwise err {err:.3e}")
    assert err <= (TOL_DECODE if M <= 8 else TOL_PREFILL)


# ---------------------------------------------------------------- moe-680m shapes

@pytest.fixture(scope="module")
def full(gpu, orc):
    ctx = gpu.Context(H, I, E, 1, 4096, gpu.W_REF)
    layer = Layer(gpu, orc, gpu.seed_for(0, 0, gpu.TAG_W))
    ctx.bind_packed(0, layer.dev)
    yield ctx, layer
    ctx.close()


def test_config0_decode_m1(gpu, orc, full):
    ctx, layer = full
    log("config 0: decode M=1")
    err, _ = run_case(gpu, orc, ctx, layer, 1, gpu.seed_for(0, 0, gpu.TAG_X))
    log(f"  normwise err {err:.3e}")
    assert err <= TOL_DECODE


@pytest.mark.parametrize("M", [2, 4, 8])
def test_config3_decode_small_batch(gpu, orc, full, M):
    ctx, layer = full
    log(f"config 3: decode M={M}")
    err, _ = run_case(gpu, orc, ctx, layer, M, gpu.seed_for(3, 0, gpu.TAG_X) + M)
    log(f"  normwise err {err:.3e}")
    assert err <= TOL_DECODE


def test_decode_flags(gpu, orc, full):
    ctx, layer = full
    for flags in (1, 2, 3):
        log(f"decode M=3 flags={flags}")
        err, _ = run_case(gpu, orc, ctx, layer, 3, 555 + flags, flags=flags)
        assert err <= TOL_DECODE


def test_config1_prefill_m512_zipf(gpu, orc, full):
    ctx, layer = full
    log("config 1: prefill M=512, Zipf(1.1) bias")
    err, _ = run_case(gpu, orc, ctx, layer, 512, gpu.seed_for(1, 0, gpu.TAG_X), kind=1, param=1.1)
    log(f"  normwise err {err:.3e}")
    assert err <= TOL_PREFILL


def test_config4_prefill_m4096_hot(gpu, orc, full):
    ctx, layer = full
    log("config 4: prefill M=4096, 5% hot expert (96 tokens checked)")
    rng = np.random.default_rng(4)
    subset = np.sort(rng.choice(4096, 96, replace=False))
    err, _ = run_case(gpu, orc, ctx, layer, 4096, gpu.seed_for(4, 0, gpu.TAG_X), kind=2, param=0.05,
                      hot=1000.0, subset=subset)
    log(f"  normwise err {err:.3e}")
    assert err <= TOL_PREFILL


def test_prefill_flags(gpu, orc, full):
    ctx, layer = full
    for flags in (1, 2, 3):
        log(f"prefill M=40 flags={flags}")
        err, _ = run_case(gpu, orc, ctx, layer, 40, 777 + flags, flags=flags)
        assert err <= TOL_PREFILL


def test_renorm_mode(gpu, orc, full):
    import torch
    ctx_r = gpu.Context(H, I, E, 1, 64, gpu.W_RENORM)
    _, layer = full
    ctx_r.bind_packed(0, layer.dev)
    for M in (1, 33):
        log(f"RENORM mode M={M}")
        err, _ = run_case(gpu, orc, ctx_r, layer, M, 900 + M, mode=1)
        assert err <= (TOL_DECODE if M <= 8 else TOL_PREFILL)
    ctx_r.close()


def test_deterministic(gpu, full):
    import torch
    ctx, _ = full
    for M in (1, 8, 300):
        log(f"determinism M={M}")
        x = gpu.gen_normal(M * H, 11).view(M, H)
        ids, w = ctx.router_topk(gpu.gen_logits(M, E, 12, 1, 1.1))
        a = ctx.ffn(0, x, ids, w)
        b = ctx.ffn(0, x, ids, w)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_in_place_residual(gpu, full):
    import torch
    ctx, _ = full
    for M in (1, 64):
        log(f"in-place residual M={M}")
        x = gpu.gen_normal(M * H, 21).view(M, H)
        ids, w = ctx.router_topk(gpu.gen_logits(M, E, 22))
        out = x.clone()
        ctx.ffn(0, x, ids, w, y=out, accumulate=True, rmsnorm=True)
        inplace = x.clone()
        ctx.ffn(0, inplace, ids, w, y=inplace, accumulate=True, rmsnorm=True)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), inplace.view(torch.int32))


def test_api_errors_on_gpu(gpu, full):
    import torch
    ctx, _ = full
    x = torch.zeros((4, H), device="cuda")
    ids = torch.zeros((4, 9), dtype=torch.uint16, device="cuda")
    w = torch.zeros((4, 9), device="cuda")
    with pytest.raises(gpu.MoeError) as e:
        ctx.ffn(1, x, ids, w)           # layer out of range
    assert e.value.status == gpu.MOE_EINVAL
    with pytest.raises(gpu.MoeError):
        ctx.ffn(0, x[:, 1:], ids, w)     # misaligned
    big = torch.zeros((5000, H), device="cuda")
    with pytest.raises(gpu.MoeError):
        ctx.ffn(0, big, ids, w)          # M > m_max
    ctx.ffn(0, x[:0], ids[:0], w[:0])  # M = 0 is a no-op


def test_kernel_timing_hook(gpu, full):
    import torch
    ctx, _ = full
    log("timing hook")
    x = gpu.gen_normal(2 * H, 31).view(2, H)
    ids, w = ctx.router_topk(gpu.gen_logits(2, E, 32))
    ctx.timing_enable(64)
    ctx.router_topk(gpu.gen_logits(2, E, 32), ids, w)
    ctx.ffn(0, x, ids, w)
    xp = gpu.gen_normal(40 * H, 33).view(40, H)
    idp, wp = ctx.router_topk(gpu.gen_logits(40, E, 34))
    ctx.ffn(0, xp, idp, wp)
    t = ctx.timing_read()
    assert t["router_topk"][0] == 2 and t["decode_gate_up"][0] == 1 and t["decode_down"][0] == 1
    # the prefill chain: bucket fill and prep in one launch, then gate/up, down, combine
    for k in ("bucket_fill", "prefill_gate_up", "prefill_down", "prefill_combine"):
        assert t[k][0] == 1 and t[k][1] > 0
    assert "prefill_prep" not in t
    assert ctx.timing_read() == {}
    ctx.timing_enable(0)
    ctx.ffn(0, x, ids, w)
    torch.cuda.synchronize()
