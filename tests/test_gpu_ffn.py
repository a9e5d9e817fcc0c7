"""GPU: the expert FFN + combine vs the f64 oracle on identical seeded inputs.

Tolerances (normwise, max|y - ref| / max|ref|): decode (M <= 8: activations as two int8
planes per 32-element chunk, f32 accumulation) 1e-3; prefill (f16 MFMA operands after exact
power-of-two scaling, f32 accumulate) 5e-3 -- the bounds BASELINE.json states.  Beside it the
elementwise error max |y - ref| / max(|ref|, 1e-3 rms(ref)) is asserted (gpu_util.EW_DECODE,
EW_PREFILL): both paths' errors are near-uniform in absolute size over the outputs, so it is
largest on the few outputs near zero, where the 1e-3 rms floor bounds it.  BASELINE's
configs name the renormalised top-8 (MOE_W_RENORM); both conventions are run.
"""
import numpy as np
import pytest

from gpu_util import E, H, I, Layer, check_errs, log, normwise_err

pytestmark = pytest.mark.gpu

TOL_DECODE = 1e-3
TOL_PREFILL = 5e-3


def run_case(gpu, orc, ctx, layer, M, seed, kind=0, param=0.0, hot=0.0, flags=0, mode=None,
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
    if mode is None:
        mode = ctx.wmode
    c = 1.0 / 9 if mode == 0 else 1.0
    xs, ids_h, w_h, y0_h, y_h = (t.cpu().numpy() for t in (x, ids, w, y0, y))
    if subset is not None:
        xs, ids_h, w_h, y0_h, y_h = xs[subset], ids_h[subset], w_h[subset], y0_h[subset], y_h[subset]
    ref = orc.moe_ffn(layer.host(), xs, ids_h, w_h, c, flags, y=y0_h if flags & 1 else None)
    if flags & 1:  # compare the FFN part, not the residual
        got_p, ref_p = y_h - y0_h, ref - y0_h
    else:
        got_p, ref_p = y_h, ref
    # the elementwise bound of the path is asserted here; the normwise one by the caller
    err = check_errs(got_p, ref_p, M <= 8, assert_normwise=False)
    return err, y


# ---------------------------------------------------------------- small shape, brute force

@pytest.fixture(scope="module")
def small(gpu, orc):
    ctx = gpu.Context(512, 256, 16, 1, 256, gpu.W_REF)
    layer = Layer(gpu, orc, 31, 512, 256, 16)
    ctx.bind_packed(0, layer.dev)
    yield ctx, layer
    ctx.close()


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 9, 37, 200])
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


@pytest.mark.parametrize("M", [2, 3, 4, 5, 6, 7, 8])
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
    """Every one of the 4096 tokens is checked (the hot expert's ~200 tokens span full
    64-row tiles and a remainder tile; the other experts' ~128 fill 64-row tiles too)."""
    ctx, layer = full
    log("config 4: prefill M=4096, 5% hot expert, all tokens checked")
    err, _ = run_case(gpu, orc, ctx, layer, 4096, gpu.seed_for(4, 0, gpu.TAG_X), kind=2, param=0.05,
                      hot=1000.0)
    log(f"  normwise err {err:.3e}")
    assert err <= TOL_PREFILL


def test_prefill_m1024_every_token(gpu, orc, full):
    """M in 769..1024: the wide (128-column) gate/up items with the keep-in-LDS bucket fill."""
    ctx, layer = full
    for M in (800, 1024):
        log(f"prefill M={M}, Zipf(1.1), all tokens checked")
        err, _ = run_case(gpu, orc, ctx, layer, M, 4400 + M, kind=1, param=1.1)
        log(f"  normwise err {err:.3e}")
        assert err <= TOL_PREFILL


def test_prefill_flags(gpu, orc, full):
    ctx, layer = full
    for flags in (1, 2, 3):
        log(f"prefill M=40 flags={flags}")
        err, _ = run_case(gpu, orc, ctx, layer, 40, 777 + flags, flags=flags)
        assert err <= TOL_PREFILL


@pytest.fixture(scope="module")
def full_renorm(gpu, full):
    """The moe-680m layer of `full` in a context with BASELINE's weight convention."""
    ctx_r = gpu.Context(H, I, E, 1, 4096, gpu.W_RENORM)
    _, layer = full
    ctx_r.bind_packed(0, layer.dev)
    yield ctx_r, layer
    ctx_r.close()


def test_renorm_configs(gpu, orc, full_renorm):
    """BASELINE configs 0, 1, 3 and 4 under the renormalised top-8 (c = 1), all tokens."""
    ctx, layer = full_renorm
    cases = [("config 0", 1, gpu.seed_for(0, 0, gpu.TAG_X), 0, 0.0, 0.0),
             ("config 3", 2, gpu.seed_for(3, 0, gpu.TAG_X) + 2, 0, 0.0, 0.0),
             ("config 3", 4, gpu.seed_for(3, 0, gpu.TAG_X) + 4, 0, 0.0, 0.0),
             ("config 3", 8, gpu.seed_for(3, 0, gpu.TAG_X) + 8, 0, 0.0, 0.0),
             ("config 1", 512, gpu.seed_for(1, 0, gpu.TAG_X), 1, 1.1, 0.0),
             ("config 4", 4096, gpu.seed_for(4, 0, gpu.TAG_X), 2, 0.05, 1000.0)]
    for name, M, seed, kind, param, hot in cases:
        log(f"RENORM {name} M={M}")
        err, _ = run_case(gpu, orc, ctx, layer, M, seed, kind=kind, param=param, hot=hot)
        log(f"  normwise err {err:.3e}")
        assert err <= (TOL_DECODE if M <= 8 else TOL_PREFILL)


def test_renorm_flags(gpu, orc, full_renorm):
    ctx, layer = full_renorm
    for M in (1, 33):
        for flags in (1, 3):
            log(f"RENORM M={M} flags={flags}")
            err, _ = run_case(gpu, orc, ctx, layer, M, 900 + M + flags, flags=flags)
            assert err <= (TOL_DECODE if M <= 8 else TOL_PREFILL)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 8, 9, 40, 512, 1000, 1025, 4096])
def test_ffn_route_equals_router_then_ffn(gpu, full, M):
    """moe_ffn_route (routing inside the decode launches for M <= 8, a router launch before the
    prefill launches beyond) gives the router's ids and weights and the FFN's output bit for
    bit, on both bucket-fill paths (one workgroup up to M = 1024, many beyond)."""
    import torch
    ctx, _ = full
    log(f"ffn_route M={M}")
    x = gpu.gen_normal(M * H, 3100 + M).view(M, H)
    logits = gpu.gen_logits(M, E, 3200 + M)
    ids, w = ctx.router_topk(logits)
    y_ref = ctx.ffn(0, x, ids, w, rmsnorm=True).clone()
    y, ids2, w2 = ctx.ffn_route(0, x, logits, rmsnorm=True)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2)
    assert torch.equal(w.view(torch.int32), w2.view(torch.int32))
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32))
    assert ctx.device_flags() == 0


@pytest.mark.parametrize("M", [512, 1025])
def test_ffn_route_prefill_graph_replays(gpu, full, M):
    """Graph replays of the routed prefill (router launch, bucket fill, GEMMs, combine), with
    eager calls of another M in between, equal the eager result bit for bit."""
    import torch
    ctx, _ = full
    log(f"ffn_route prefill M={M}: graph capture, 3 replays")
    x = gpu.gen_normal(M * H, 3700 + M).view(M, H)
    logits = gpu.gen_logits(M, E, 3800 + M, 1, 1.1)
    y0, i0, w0 = (t.clone() for t in ctx.ffn_route(0, x, logits))
    x2 = gpu.gen_normal(64 * H, 3900).view(64, H)
    l2 = gpu.gen_logits(64, E, 3901)
    torch.cuda.synchronize()
    y = torch.empty_like(y0)
    ids = torch.empty_like(i0)
    w = torch.empty_like(w0)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            ctx.ffn_route(0, x, logits, y=y, ids=ids, w=w, stream=s)
    torch.cuda.synchronize()
    for rep in range(3):
        y.fill_(float("nan"))
        ids.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids, i0) and torch.equal(w.view(torch.int32), w0.view(torch.int32)), rep
        assert torch.equal(y.view(torch.int32), y0.view(torch.int32)), rep
        ctx.ffn_route(0, x2, l2)
        torch.cuda.synchronize()
    assert ctx.device_flags() == 0


def test_duplicate_and_bad_ids_same_at_decode_and_prefill(gpu, orc, full):
    """A token naming one expert twice, or an id above n_experts: the later / bad slot is
    dropped and flagged the same way whether the call takes the decode path (M = 1) or the
    prefill path (M = 9)."""
    import torch
    ctx, layer = full
    x = gpu.gen_normal(9 * H, 3301).view(9, H)
    ids, w = ctx.router_topk(gpu.gen_logits(9, E, 3302))
    ids_bad = ids.clone()
    ids_bad[0, 5] = ids_bad[0, 2]      # duplicate inside token 0
    ids_bad[0, 7] = E + 3              # out of range
    torch.cuda.synchronize()
    y1 = ctx.ffn(0, x[:1], ids_bad[:1], w[:1]).clone()
    f1 = ctx.device_flags()
    y9 = ctx.ffn(0, x, ids_bad, w).clone()
    f9 = ctx.device_flags()
    assert f1 == f9 == (gpu.DEVFLAG_BAD_ID | gpu.DEVFLAG_DUP_ID)
    ref = orc.moe_ffn(layer.host(), x[:1].cpu().numpy(), ids_bad[:1].cpu().numpy(), w[:1].cpu().numpy(),
                      1.0 / 9)
    check_errs(y1.cpu().numpy(), ref, True)
    check_errs(y9[:1].cpu().numpy(), ref, False)
    # the oracle drops exactly those slots: the same as zeroing their weights
    w_zero = w[:1].cpu().numpy().copy()
    w_zero[0, 5] = w_zero[0, 7] = 0.0
    ref0 = orc.moe_ffn(layer.host(), x[:1].cpu().numpy(), ids[:1].cpu().numpy(), w_zero, 1.0 / 9)
    assert normwise_err(ref, ref0) <= 1e-12


def test_prefill_dropped_slots_skip_nonfinite_row0(gpu, orc, full):
    """Prefill (M = 16): token 0 routes to expert 0 in slot 0, so its partial output is
    expert-sorted row 0, and its activations are +inf (that row is non-finite).  Token 1 names
    one expert twice and an id above n_experts: its dropped slots must add nothing -- not 0
    times row 0, which would be NaN -- so every token but token 0 still matches the oracle.
    Token 2 names no valid id (its output is 0), token 3 the shared expert in a routed slot
    (its slot 8 is the repeat that is dropped)."""
    import torch
    ctx, layer = full
    M = 16
    x = gpu.gen_normal(M * H, 3601).view(M, H)
    ids, w = ctx.router_topk(gpu.gen_logits(M, E, 3602))
    torch.cuda.synchronize()
    ids_h = ids.cpu().numpy().astype(np.int64)
    for t in range(M):          # expert 0 only where put below
        ids_h[t, :8][ids_h[t, :8] == 0] = 255 - t
    ids_h[0, 0] = 0
    ids_h[1, 4] = ids_h[1, 1]   # duplicate inside token 1
    ids_h[1, 6] = E + 5         # out of range
    ids_h[2, :] = E + 7         # token 2: no valid slot at all (not even the shared one)
    ids_h[3, 2] = E             # token 3 names the shared expert in a routed slot: slot 8 repeats it
    ids_bad = torch.from_numpy(ids_h.astype(np.uint16)).cuda()
    x[0] = float("inf")
    y = ctx.ffn(0, x, ids_bad, w).clone()
    torch.cuda.synchronize()
    assert ctx.device_flags() == (gpu.DEVFLAG_BAD_ID | gpu.DEVFLAG_DUP_ID)
    y_h = y.cpu().numpy()
    assert np.isfinite(y_h[1:]).all()
    ref = orc.moe_ffn(layer.host(), x[1:].cpu().numpy(), ids_h[1:].astype(np.uint16), w[1:].cpu().numpy(),
                      1.0 / 9)
    check_errs(y_h[1:], ref, False)


@pytest.mark.parametrize("route", [False, True])
def test_duplicate_and_bad_ids_decode_batch(gpu, orc, full, route):
    """The pair rule on the 2 <= M <= 8 decode path (its prep launch): token 0 names one expert
    twice and has an id above n_experts, token 2 repeats its shared slot's id in slot 3; the
    later / bad slots are dropped, the flags raised, and the other tokens untouched -- the
    oracle applies the same rule.  With route=True the valid routing comes from moe_ffn_route
    and must equal moe_router_topk's bit for bit."""
    import torch
    ctx, layer = full
    M = 4
    x = gpu.gen_normal(M * H, 3401).view(M, H)
    logits = gpu.gen_logits(M, E, 3402)
    ids, w = ctx.router_topk(logits)
    if route:
        y, ids2, w2 = ctx.ffn_route(0, x, logits)
        torch.cuda.synchronize()
        assert torch.equal(ids, ids2) and torch.equal(w.view(torch.int32), w2.view(torch.int32))
        assert ctx.device_flags() == 0
        ref = orc.moe_ffn(layer.host(), x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), 1.0 / 9)
        check_errs(y.cpu().numpy(), ref, True)
        return
    ids_bad = ids.clone()
    ids_bad[0, 5] = ids_bad[0, 2]       # duplicate inside token 0
    ids_bad[0, 7] = E + 3               # out of range
    ids_bad[2, 3] = E                   # token 2 names the shared expert in a routed slot ...
    torch.cuda.synchronize()
    y = ctx.ffn(0, x, ids_bad, w).clone()
    assert ctx.device_flags() == (gpu.DEVFLAG_BAD_ID | gpu.DEVFLAG_DUP_ID)
    ref = orc.moe_ffn(layer.host(), x.cpu().numpy(), ids_bad.cpu().numpy(), w.cpu().numpy(), 1.0 / 9)
    check_errs(y.cpu().numpy(), ref, True)
    # ... so its slot 8 (the shared id again) is the repeat that is dropped
    w_zero = w.cpu().numpy().copy()
    w_zero[0, 5] = w_zero[0, 7] = w_zero[2, 8] = 0.0
    ids_fix = ids.cpu().numpy().copy()
    ids_fix[2, 3] = E
    ref0 = orc.moe_ffn(layer.host(), x.cpu().numpy(), ids_fix, w_zero, 1.0 / 9)
    assert normwise_err(ref, ref0) <= 1e-12


@pytest.mark.parametrize("acc", [False, True])
def test_decode_batch_tokens_without_valid_slots(gpu, orc, full, acc):
    """2 <= M <= 8 with tokens left with few or no valid slots: token 3 names only ids above
    n_experts (every slot dropped: its output is the residual, or zero), token 5 names one
    expert in all nine slots (only slot 0 kept), token 6 has every slot valid.  The token-major
    down launch then has workgroups with no work unit and workgroups with one."""
    import torch
    ctx, layer = full
    M = 7
    x = gpu.gen_normal(M * H, 3501).view(M, H)
    ids, w = ctx.router_topk(gpu.gen_logits(M, E, 3502))
    ids_bad = ids.clone()
    ids_bad[3, :] = E + 7
    ids_bad[5, :] = ids_bad[5, 0]
    y0 = gpu.gen_normal(M * H, 3503).view(M, H)
    y = y0.clone()
    torch.cuda.synchronize()
    ctx.ffn(0, x, ids_bad, w, y=y, accumulate=acc)
    torch.cuda.synchronize()
    assert ctx.device_flags() == (gpu.DEVFLAG_BAD_ID | gpu.DEVFLAG_DUP_ID)
    y_h, y0_h = y.cpu().numpy(), y0.cpu().numpy()
    ref = orc.moe_ffn(layer.host(), x.cpu().numpy(), ids_bad.cpu().numpy(), w.cpu().numpy(), 1.0 / 9,
                      1 if acc else 0, y=y0_h if acc else None)
    if acc:
        check_errs(y_h - y0_h, ref - y0_h, True)
        assert np.array_equal(y_h[3], y0_h[3])
    else:
        check_errs(y_h, ref, True)
        assert not np.any(y_h[3])
    # the oracle keeps token 5's slot 0 alone
    w5 = np.zeros((1, 9), dtype=np.float32)
    w5[0, 0] = w[5, 0].item()
    ref5 = orc.moe_ffn(layer.host(), x[5:6].cpu().numpy(), ids_bad[5:6].cpu().numpy(), w5, 1.0 / 9)
    part5 = (y_h[5] - y0_h[5]) if acc else y_h[5]
    check_errs(part5[None], ref5, True)


def test_prefill_zero_block_small_activations(gpu, orc):
    """A 64-row block of W3 with d = 0 (h = 0 over a whole column block) and activations
    small enough that a row's max|h| is below 0.5: the prefill down kernel's rescale of that
    block must give zeros, not 0 * inf = NaN."""
    import torch
    hidden, inter, nexp = H, I, E
    ctx = gpu.Context(hidden, inter, nexp, 1, 64, gpu.W_REF)
    try:
        buf = gpu.gen_layer(hidden, inter, nexp, 3401)
        mb = gpu.matrix_bytes(hidden, inter)
        eb = 3 * mb
        rowb = hidden // 256 * 136
        # experts used below: zero d of W3 rows 64..127 of every expert (d is bytes 0-1 of a block)
        host = buf.cpu().numpy()
        for e in range(nexp + 1):
            base = e * eb + mb + 64 * rowb
            blk = host[base:base + 64 * rowb].reshape(64 * (hidden // 256), 136)
            blk[:, 0:2] = 0
        buf = torch.from_numpy(host).cuda()
        ctx.bind_packed(0, buf)
        layer = Layer(gpu, orc, None, hidden, inter, nexp, dev=buf)
        M = 40
        x = (gpu.gen_normal(M * hidden, 3402) * 1e-3).view(M, hidden)
        ids, w = ctx.router_topk(gpu.gen_logits(M, nexp, 3403))
        y = ctx.ffn(0, x, ids, w)
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        ref = orc.moe_ffn(layer.host(), x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), 1.0 / 9)
        log("zero W3 block, small x")
        check_errs(y.cpu().numpy(), ref, False)
    finally:
        ctx.close()


def test_prefill_row_scale_extremes(gpu, orc):
    """Super-block scales d that stress the prefill decode's per-row shift (weights enter the
    MFMA as dl * kv * 2^-s, s from the row's largest |d|): in rows 0..3 of every expert's W1,
    W3 and W2 -- one large d among minimum-subnormal ones, all zero, all subnormal, and mixed
    signs over five binades.  Prefill (M = 40) and decode (M = 3) against the oracle, which
    decodes the same bytes."""
    import torch
    hidden, inter, nexp = H, I, E
    ctx = gpu.Context(hidden, inter, nexp, 1, 64, gpu.W_REF)
    try:
        buf = gpu.gen_layer(hidden, inter, nexp, 3501)
        mb = gpu.matrix_bytes(hidden, inter)
        host = buf.cpu().numpy()
        f16 = lambda v: np.frombuffer(np.float16(v).tobytes(), dtype=np.uint8)
        for e in range(nexp + 1):
            for mi, k in ((0, hidden), (1, hidden), (2, inter)):  # W1, W3 ([inter][hidden]), W2 ([hidden][inter])
                nsb = k // 256
                for row in range(4):
                    base = e * 3 * mb + mi * mb + row * nsb * 136
                    for sb in range(nsb):
                        if row == 0:
                            d = 0.25 if sb == 0 else float(np.float16(2.0 ** -24)) * (sb + 1)
                        elif row == 1:
                            d = 0.0
                        elif row == 2:
                            d = float(np.float16(3 * 2.0 ** -24)) * (1 if sb % 2 else -1)
                        else:
                            d = (-0.03 if sb % 2 else 0.001) * (2.0 ** -(sb % 5))
                        host[base + sb * 136: base + sb * 136 + 2] = f16(d)
        buf = torch.from_numpy(host).cuda()
        ctx.bind_packed(0, buf)
        layer = Layer(gpu, orc, None, hidden, inter, nexp, dev=buf)
        for M, seed in ((40, 3502), (3, 3505)):
            x = gpu.gen_normal(M * hidden, seed).view(M, hidden)
            ids, w = ctx.router_topk(gpu.gen_logits(M, nexp, seed + 1))
            y = ctx.ffn(0, x, ids, w)
            torch.cuda.synchronize()
            assert torch.isfinite(y).all()
            ref = orc.moe_ffn(layer.host(), x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), 1.0 / 9)
            log(f"row scale extremes, M={M}")
            check_errs(y.cpu().numpy(), ref, M <= 8)
    finally:
        ctx.close()


def test_decode_graph_replays(gpu, full):
    """Graph replays of the decode path, with eager calls of another M in between, each equal
    the eager result bit for bit."""
    import torch
    ctx, _ = full
    for M in (1, 8):
        log(f"decode graph replays M={M}")
        x = gpu.gen_normal(M * H, 3500 + M).view(M, H)
        ids, w = ctx.router_topk(gpu.gen_logits(M, E, 3600 + M))
        eager = ctx.ffn(0, x, ids, w, rmsnorm=True).clone()
        y = torch.empty_like(x)
        xo = gpu.gen_normal(3 * H, 3700).view(3, H)
        io, wo = ctx.router_topk(gpu.gen_logits(3, E, 3701))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            ctx.ffn(0, x, ids, w, y=y, rmsnorm=True)
        for r in range(4):
            y.zero_()
            g.replay()
            ctx.ffn(0, xo, io, wo)   # another shape between replays
            torch.cuda.synchronize()
            assert torch.equal(y.view(torch.int32), eager.view(torch.int32)), f"replay {r}"
        assert ctx.device_flags() == 0


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
    # the prefill chain with ids given: the bucket count, the placement with the prep, then
    # gate/up, down, combine
    assert t["bucket_fill"][0] == 2 and t["bucket_fill"][1] > 0
    for k in ("prefill_gate_up", "prefill_down", "prefill_combine"):
        assert t[k][0] == 1 and t[k][1] > 0
    assert ctx.timing_read() == {}
    ctx.timing_enable(0)
    ctx.ffn(0, x, ids, w)
    torch.cuda.synchronize()
