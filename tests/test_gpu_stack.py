"""GPU: moe_decode_stack (one token through consecutive layers in one persistent launch)
vs the oracle applied layer by layer: x <- x + MoE_l(RMSNorm(x)), routing from seeded
per-layer logits.  Decode tolerance: normwise 1e-3, and the elementwise
error (gpu_util.EW_STACK) beside it."""
import numpy as np
import pytest

from gpu_util import E, EW_STACK, H, I, check_errs, log, normwise_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def oracle_chain(orc, pkg, layers_dev, hidden, inter, nexp, x0, logits, rmsnorm=True, mode=0):
    """Oracle chain on the host; copies only the experts each layer selects."""
    x = np.array(x0, dtype=np.float32).reshape(1, hidden)
    eb = 3 * (hidden * inter // 256 * 136)
    host = np.zeros((nexp + 1) * eb, dtype=np.uint8)
    all_ids, all_w = [], []
    for l, dev in enumerate(layers_dev):
        ids, w = orc.router_topk(logits[l:l + 1], mode)
        for e in ids[0]:
            host[int(e) * eb:(int(e) + 1) * eb] = dev[int(e) * eb:(int(e) + 1) * eb].cpu().numpy()
        L = orc.PackedLayer(host, hidden, inter, nexp)
        flags = orc.ACCUMULATE | (orc.RMSNORM if rmsnorm else 0)
        x = orc.moe_ffn(L, x, ids, w, 1.0 / 9 if mode == 0 else 1.0, flags, y=x)
        all_ids.append(ids[0])
        all_w.append(w[0])
    return x.reshape(-1), np.array(all_ids), np.array(all_w)


@pytest.fixture(scope="module")
def small(gpu):
    hidden, inter, nexp, nl = 512, 256, 16, 6
    ctx = gpu.Context(hidden, inter, nexp, nl, 16, gpu.W_REF)
    layers = []
    for l in range(nl):
        buf = gpu.gen_layer(hidden, inter, nexp, 500 + l)
        ctx.bind_packed(l, buf)
        layers.append(buf)
    yield ctx, layers, (hidden, inter, nexp)
    ctx.close()


@pytest.mark.parametrize("layer0,n", [(0, 1), (0, 2), (0, 3), (0, 6), (2, 3), (5, 1)])
def test_small_stack(gpu, orc, small, layer0, n):
    import torch
    ctx, layers, (hidden, inter, nexp) = small
    log(f"stack small H={hidden} layers {layer0}..{layer0 + n - 1}")
    x = gpu.gen_normal(hidden, 600 + n)
    logits = gpu.gen_logits(n, nexp, 700 + layer0 + n)
    ids = torch.empty((n, 9), dtype=torch.uint16, device="cuda")
    w = torch.empty((n, 9), dtype=torch.float32, device="cuda")
    y = ctx.decode_stack(layer0, x, logits, ids=ids, w=w)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    ref, rid, rw = oracle_chain(orc, gpu, layers[layer0:layer0 + n], hidden, inter, nexp,
                                x.cpu().numpy(), logits.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5)
    check_errs(y.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK)


def test_small_stack_no_norm_and_in_place(gpu, orc, small):
    import torch
    ctx, layers, (hidden, inter, nexp) = small
    n = 2  # without RMSNorm the seeded chain grows ~1e5x per layer and overflows by layer 4
    x = gpu.gen_normal(hidden, 801)
    x0 = x.cpu().numpy()
    logits = gpu.gen_logits(n, nexp, 802)
    ctx.decode_stack(0, x, logits, y=x, rmsnorm=False)   # in place
    torch.cuda.synchronize()
    ref, _, _ = oracle_chain(orc, gpu, layers[:n], hidden, inter, nexp, x0, logits.cpu().numpy(),
                             rmsnorm=False)
    check_errs(x.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK)


@pytest.fixture(scope="module")
def full(gpu):
    nl = 40
    ctx = gpu.Context(H, I, E, nl, 8, gpu.W_REF)
    layers = []
    for l in range(nl):
        buf = gpu.gen_layer(H, I, E, gpu.seed_for(2, l, gpu.TAG_W))
        ctx.bind_packed(l, buf)
        layers.append(buf)
    yield ctx, layers
    ctx.close()


def test_config2_forty_layers(gpu, orc, full):
    import torch
    ctx, layers = full
    log("config 2: 40-layer stack, M=1")
    x = gpu.gen_normal(H, gpu.seed_for(2, 0, gpu.TAG_X))
    logits = gpu.gen_logits(40, E, gpu.seed_for(2, 0, gpu.TAG_L))
    ids = torch.empty((40, 9), dtype=torch.uint16, device="cuda")
    w = torch.empty((40, 9), dtype=torch.float32, device="cuda")
    y = ctx.decode_stack(0, x, logits, ids=ids, w=w)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    ref, rid, rw = oracle_chain(orc, gpu, layers, H, I, E, x.cpu().numpy(), logits.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), rid)
    check_errs(y.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK)


def test_config2_forty_layers_renorm(gpu, orc, full):
    """Config 2 under BASELINE's renormalised top-8 (c = 1): a context in MOE_W_RENORM bound
    to the same 40 layers."""
    import torch
    _, layers = full
    ctx = gpu.Context(H, I, E, 40, 8, gpu.W_RENORM)
    try:
        for l, buf in enumerate(layers):
            ctx.bind_packed(l, buf)
        log("config 2 RENORM: 40-layer stack, M=1")
        x = gpu.gen_normal(H, gpu.seed_for(2, 0, gpu.TAG_X) + 1)
        logits = gpu.gen_logits(40, E, gpu.seed_for(2, 0, gpu.TAG_L) + 1)
        ids = torch.empty((40, 9), dtype=torch.uint16, device="cuda")
        w = torch.empty((40, 9), dtype=torch.float32, device="cuda")
        y = ctx.decode_stack(0, x, logits, ids=ids, w=w)
        torch.cuda.synchronize()
        assert ctx.device_flags() == 0
        ref, rid, rw = oracle_chain(orc, gpu, layers, H, I, E, x.cpu().numpy(), logits.cpu().numpy(), mode=1)
        assert np.array_equal(ids.cpu().numpy(), rid)
        assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5)
        assert np.allclose(w.cpu().numpy()[:, :8].sum(axis=1), 1.0, rtol=1e-5)
        check_errs(y.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK)
    finally:
        ctx.close()


def test_stack_timeout_leaves_x(gpu, full):
    """A host-forced timeout (spin limit 0: every wait not satisfied at its first look
    expires): TIMEOUT is raised, every workgroup exits, and the in-place x is untouched.
    The same context then runs normally again."""
    import torch
    ctx, _ = full
    n = 4
    x = gpu.gen_normal(H, 1101)
    logits = gpu.gen_logits(n, E, 1102)
    x0 = x.clone()
    good = ctx.decode_stack(0, x0, logits).clone()
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    ctx.stack_spin_limit(0)
    try:
        log("stack with spin limit 0 (forced timeout), in place")
        ctx.decode_stack(0, x, logits, y=x)
        torch.cuda.synchronize()
        f = ctx.device_flags()
        assert f & gpu.DEVFLAG_TIMEOUT
        assert torch.equal(x.view(torch.int32), x0.view(torch.int32))
    finally:
        ctx.stack_spin_limit(65536)
    ctx.decode_stack(0, x, logits, y=x)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    assert torch.equal(x.view(torch.int32), good.view(torch.int32))


@pytest.mark.parametrize("recover", ["sync", "async"])
def test_stack_recovers_from_first_launch_timeout(gpu, orc, recover):
    """A fresh context whose first stack launch (epoch 0) times out: the abort word then holds
    epoch 0's tag.  After the recovery (moe_device_flags, or moe_device_flags_async) the epoch
    restarts at 0, so the abort word must be cleared with it: the next launches -- the first
    again at epoch 0 -- run normally and match the oracle."""
    import torch
    hidden, inter, nexp, nl = 512, 256, 16, 3
    ctx = gpu.Context(hidden, inter, nexp, nl, 4, gpu.W_REF)
    try:
        layers = []
        for l in range(nl):
            buf = gpu.gen_layer(hidden, inter, nexp, 1500 + l)
            ctx.bind_packed(l, buf)
            layers.append(buf)
        x = gpu.gen_normal(hidden, 1510)
        logits = gpu.gen_logits(nl, nexp, 1511)
        ctx.stack_spin_limit(0)
        try:
            log(f"stack: first launch of a fresh context forced to time out, recovery {recover}")
            ctx.decode_stack(0, x, logits)
            torch.cuda.synchronize()
        finally:
            ctx.stack_spin_limit(65536)
        if recover == "sync":
            assert ctx.device_flags() & gpu.DEVFLAG_TIMEOUT
        else:
            dst = torch.zeros(1, dtype=torch.int32, device="cuda")
            ctx.device_flags_async(dst)
            torch.cuda.synchronize()
            assert int(dst[0]) & gpu.DEVFLAG_TIMEOUT
        ref, rid, _ = oracle_chain(orc, gpu, layers, hidden, inter, nexp, x.cpu().numpy(), logits.cpu().numpy())
        for rep in range(3):
            ids = torch.empty((nl, 9), dtype=torch.uint16, device="cuda")
            w = torch.empty((nl, 9), dtype=torch.float32, device="cuda")
            y = ctx.decode_stack(0, x, logits, ids=ids, w=w)
            torch.cuda.synchronize()
            assert ctx.device_flags() == 0, rep
            assert np.array_equal(ids.cpu().numpy(), rid)
            check_errs(y.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK, tag=f"rep {rep}: ")
    finally:
        ctx.close()


def test_device_flags_async(gpu, full):
    """moe_device_flags_async moves and clears the sticky flags in stream order, into device
    memory or pinned host memory, without a host synchronisation."""
    import torch
    ctx, _ = full
    dst = torch.full((1,), 0x7F, dtype=torch.int32, device="cuda")
    pinned = torch.full((1,), 0x7F, dtype=torch.int32).pin_memory()
    ctx.device_flags_async(dst)
    ctx.stack_spin_limit(0)
    try:
        ctx.decode_stack(0, gpu.gen_normal(H, 1201), gpu.gen_logits(2, E, 1202))
    finally:
        ctx.stack_spin_limit(65536)
    ctx.device_flags_async(pinned)
    ctx.device_flags_async(dst)   # cleared by the previous move
    torch.cuda.synchronize()
    assert int(pinned[0]) & gpu.DEVFLAG_TIMEOUT
    assert int(dst[0]) == 0
    assert ctx.device_flags() == 0


def test_stack_matches_per_layer_path(gpu, full):
    import torch
    ctx, _ = full
    n = 6
    log("stack vs per-layer router + ffn")
    x = gpu.gen_normal(H, 901)
    logits = gpu.gen_logits(n, E, 902)
    y = ctx.decode_stack(10, x, logits)
    xr = x.clone().view(1, H)
    for l in range(n):
        ids, w = ctx.router_topk(logits[l:l + 1])
        ctx.ffn(10 + l, xr, ids, w, y=xr, accumulate=True, rmsnorm=True)
    torch.cuda.synchronize()
    err = normwise_err(y.cpu().numpy(), xr.view(-1).cpu().numpy())
    log(f"  stack vs per-layer normwise diff {err:.3e}")
    # the stack's W1/W3 products read x as two int8 planes per 32-element chunk (error per
    # element <= 1/512 of the chunk scale, 1.6e-5 of the chunk's largest |x|); the per-layer
    # path reads f32.  Over these six layers the two differ by ~8e-5 (measured).
    assert err <= 2e-4


def test_stack_graph_replays(gpu, full):
    import torch
    ctx, _ = full
    log("stack under graph capture, 4 replays")
    x = gpu.gen_normal(H, 903)
    logits = gpu.gen_logits(8, E, 904)
    y = torch.empty_like(x)
    eager = ctx.decode_stack(0, x, logits).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.decode_stack(0, x, logits, y=y)
    for _ in range(4):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), eager.view(torch.int32))
        assert ctx.device_flags() == 0


def test_stack_errors(gpu, full):
    import torch
    ctx, _ = full
    x = torch.zeros(H, device="cuda")
    lg = torch.zeros((2, E), device="cuda")
    with pytest.raises(gpu.MoeError):
        ctx.decode_stack(39, x, lg)          # runs past the last layer
    with pytest.raises(gpu.MoeError):
        ctx.decode_stack(0, x[1:], lg)       # misaligned


def test_rebind_refreshes_copies(gpu, small):
    """Rebinding a layer rewrites the library's own copies of it (the stack's split layout,
    the prefill layout): results equal those of a fresh context bound to the new weights."""
    import torch
    ctx, layers, (hidden, inter, nexp) = small
    other = gpu.gen_layer(hidden, inter, nexp, 999)
    fresh = gpu.Context(hidden, inter, nexp, 6, 16, gpu.W_REF)
    try:
        ctx.bind_packed(0, other)
        fresh.bind_packed(0, other)
        x = gpu.gen_normal(hidden, 1001)
        logits = gpu.gen_logits(1, nexp, 1002)
        a = ctx.decode_stack(0, x, logits).clone()
        b = fresh.decode_stack(0, x, logits).clone()
        xp = gpu.gen_normal(12 * hidden, 1003).view(12, hidden)
        ids, w = ctx.router_topk(gpu.gen_logits(12, nexp, 1004))
        ya = ctx.ffn(0, xp, ids, w).clone()
        yb = fresh.ffn(0, xp, ids, w).clone()
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
        assert torch.equal(ya.view(torch.int32), yb.view(torch.int32))
        assert ctx.device_flags() == 0 and fresh.device_flags() == 0
    finally:
        ctx.bind_packed(0, layers[0])  # the module's other tests use the original layer 0
        fresh.close()


# ---------------------------------------------------------------- activation-routed stack

def plane_logit_bound(orc, W, xin):
    """Largest error the stack's int8-plane activations can put on a logit: element k of a
    32-element chunk c is off by at most max_c |xin| / (127 * 512), so logit e is off by at most
    sum_c max_c|xin| / 65024 * sum_{k in c} |W_ek|."""
    Wd = (orc.dequant(W).astype(np.float64) if W.dtype == np.uint8 else W.astype(np.float64))
    nexp = xin.shape[-1] and (Wd.size // xin.shape[-1])
    Wd = np.abs(Wd.reshape(nexp, -1))
    cmax = np.abs(xin.astype(np.float64)).reshape(-1, 32).max(axis=1) / 65024.0
    return float((Wd.reshape(nexp, -1, 32).sum(axis=2) * cmax[None, :]).sum(axis=1).max())


def oracle_chain_routed(orc, layers_dev, routers, hidden, inter, nexp, x0, gpu_ids, gpu_w, rmsnorm=True,
                        mode=0):
    """The oracle chain routed from each layer's own input: logits = orc.router_gemv(Wg_l, xin)
    (xin = RMSNorm(x) when asked), top-8 by orc.router_topk, then the FFN.  With lb the
    layer's int8-plane logit error bound (plane_logit_bound, plus f32 rounding): where the
    oracle's 8th and 9th logits are more than 2 lb apart, the GPU's ids must equal the
    oracle's and its weights agree to 2.5 lb relative (a logit error d moves a softmax weight by
    at most 2 max|d| relative, to first order); a closer pair is a near-tie that may break
    either way, and the GPU's routing is followed.  Returns (y, layers checked)."""
    x = np.array(x0, dtype=np.float32).reshape(1, hidden)
    eb = 3 * (hidden * inter // 256 * 136)
    host = np.zeros((nexp + 1) * eb, dtype=np.uint8)
    checked = 0
    for l, dev in enumerate(layers_dev):
        lg = orc.router_gemv(routers[l], x, nexp, flags=orc.RMSNORM if rmsnorm else 0)
        xin = x / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) if rmsnorm else x
        lb = plane_logit_bound(orc, routers[l], xin) + 1e-6 * np.abs(lg).max()
        rid, rw = orc.router_topk(lg, mode)
        top9 = -np.sort(-lg[0])[:9]
        if top9[7] - top9[8] > 2 * lb:
            assert np.array_equal(gpu_ids[l], rid[0]), (l, gpu_ids[l], rid[0])
            assert np.allclose(gpu_w[l], rw[0], rtol=2.5 * lb + 1e-5, atol=0), (l, lb)
            ids, w = rid, rw
            checked += 1
        else:
            # a near-tie: every expert the GPU chose is within 2 lb of the oracle's 8th logit,
            # and it chose 8 distinct routed experts and the shared one
            g = gpu_ids[l][:8].astype(np.int64)
            assert len(set(g.tolist())) == 8 and gpu_ids[l][8] == nexp, l
            assert np.all(lg[0][g] >= top9[7] - 2 * lb), (l, lg[0][g], top9[7], lb)
            ids, w = gpu_ids[l:l + 1], gpu_w[l:l + 1]
        for e in ids[0]:
            host[int(e) * eb:(int(e) + 1) * eb] = dev[int(e) * eb:(int(e) + 1) * eb].cpu().numpy()
        L = orc.PackedLayer(host, hidden, inter, nexp)
        flags = orc.ACCUMULATE | (orc.RMSNORM if rmsnorm else 0)
        x = orc.moe_ffn(L, x, ids, w, 1.0 / 9 if mode == 0 else 1.0, flags, y=x)
    return x.reshape(-1), checked


def make_routers(gpu, hidden, nexp, n, seed, kinds=("iq4", "f32", "f16")):
    """n router gate matrices [nexp][hidden], cycling through the element types: (device
    tensors, host arrays for the oracle)."""
    import torch
    rng = np.random.default_rng(seed)
    dev, host = [], []
    for l in range(n):
        kind = kinds[l % len(kinds)]
        if kind == "iq4":
            t = gpu.gen_iq4xs(nexp * hidden // 256, seed + 17 * l)
            torch.cuda.synchronize()
            h = t.cpu().numpy()
        else:
            h = (rng.standard_normal((nexp, hidden)) * 0.05).astype(np.float32 if kind == "f32" else np.float16)
            t = torch.from_numpy(h).cuda()
        dev.append(t)
        host.append(h)
    return dev, host


@pytest.mark.parametrize("layer0,n,rmsnorm", [(0, 1, True), (0, 6, True), (2, 3, True), (0, 2, False)])
def test_small_stack_routed_from_activations(gpu, orc, small, layer0, n, rmsnorm):
    """MOE_STACK_ROUTE_GEMV: every layer routed from its own input through its bound router
    (IQ4_XS, f32 and f16 matrices in turn), against the oracle chain with orc.router_gemv."""
    import torch
    ctx, layers, (hidden, inter, nexp) = small
    rdev, rhost = make_routers(gpu, hidden, nexp, 6, 7100)
    try:
        for l in range(6):
            ctx.bind_router(l, rdev[l])
        log(f"stack routed from activations, small H={hidden} layers {layer0}..{layer0 + n - 1} "
            f"rmsnorm={rmsnorm}")
        x = gpu.gen_normal(hidden, 7200 + n)
        ids = torch.empty((n, 9), dtype=torch.uint16, device="cuda")
        w = torch.empty((n, 9), dtype=torch.float32, device="cuda")
        y = ctx.decode_stack(layer0, x, ids=ids, w=w, rmsnorm=rmsnorm, n_layers=n)
        torch.cuda.synchronize()
        assert ctx.device_flags() == 0
        ref, checked = oracle_chain_routed(orc, layers[layer0:layer0 + n], rhost[layer0:layer0 + n], hidden, inter,
                                           nexp, x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(),
                                           rmsnorm=rmsnorm)
        log(f"  routing checked on {checked} of {n} layers")
        assert checked >= (n + 1) // 2
        check_errs(y.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK)
    finally:
        for l in range(6):
            ctx.bind_router(l, None)


@pytest.fixture(scope="module")
def full_routers(gpu, full):
    ctx, _ = full
    rdev, rhost = make_routers(gpu, H, E, 40, 7300)
    for l in range(40):
        ctx.bind_router(l, rdev[l])
    yield rdev, rhost
    for l in range(40):
        ctx.bind_router(l, None)


def test_config2_forty_layers_routed_from_activations(gpu, orc, full, full_routers):
    """Config 2 as a forward pass: 40 layers, each routed from its own RMSNorm'd input by its
    router (IQ4_XS, f32, f16 in turn), against the oracle chain."""
    import torch
    ctx, layers = full
    rdev, rhost = full_routers
    log("config 2 routed from activations: 40-layer stack, M=1")
    x = gpu.gen_normal(H, gpu.seed_for(2, 0, gpu.TAG_X) + 7)
    ids = torch.empty((40, 9), dtype=torch.uint16, device="cuda")
    w = torch.empty((40, 9), dtype=torch.float32, device="cuda")
    y = ctx.decode_stack(0, x, ids=ids, w=w, n_layers=40)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    ref, checked = oracle_chain_routed(orc, layers, rhost, H, I, E, x.cpu().numpy(), ids.cpu().numpy(),
                                       w.cpu().numpy())
    log(f"  routing checked on {checked} of 40 layers")
    assert checked >= 30
    check_errs(y.cpu().numpy(), ref, True, tol=TOL, ew_tol=EW_STACK)


def test_routed_stack_matches_per_layer_path(gpu, full, full_routers):
    """The activation-routed stack against the per-layer calls it replaces:
    moe_router_gemv_topk_typed (RMSNorm) then moe_ffn (RMSNorm, ACCUMULATE), layer by layer.
    The stack reads x as int8 planes where the per-layer path reads f32: ids equal on these
    layers, outputs within the stack-vs-per-layer bound."""
    import torch
    ctx, _ = full
    rdev, _ = full_routers
    n = 6
    x = gpu.gen_normal(H, 7401)
    ids = torch.empty((n, 9), dtype=torch.uint16, device="cuda")
    w = torch.empty((n, 9), dtype=torch.float32, device="cuda")
    y = ctx.decode_stack(8, x, ids=ids, w=w, n_layers=n)
    xr = x.clone().view(1, H)
    pids = []
    for l in range(n):
        _, i_l, w_l = ctx.router_gemv_topk(rdev[8 + l], xr, rmsnorm=True, want_logits=False)
        pids.append(i_l.clone())
        ctx.ffn(8 + l, xr, i_l, w_l, y=xr, accumulate=True, rmsnorm=True)
    torch.cuda.synchronize()
    assert torch.equal(ids, torch.cat(pids))
    err = normwise_err(y.cpu().numpy(), xr.view(-1).cpu().numpy())
    log(f"  routed stack vs per-layer normwise diff {err:.3e}")
    assert err <= 2e-4


def test_routed_stack_graph_replays_and_timeout(gpu, full, full_routers):
    """Graph replays of the activation-routed stack equal the eager result bit for bit; a
    host-forced timeout leaves an in-place x untouched, and the context then runs normally."""
    import torch
    ctx, _ = full
    x = gpu.gen_normal(H, 7501)
    eager = ctx.decode_stack(0, x, n_layers=8).clone()
    torch.cuda.synchronize()
    y = torch.empty_like(x)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ctx.decode_stack(0, x, y=y, n_layers=8)
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), eager.view(torch.int32))
        assert ctx.device_flags() == 0
    xi = x.clone()
    ctx.stack_spin_limit(0)
    try:
        log("routed stack with spin limit 0 (forced timeout), in place")
        ctx.decode_stack(0, xi, y=xi, n_layers=8)
        torch.cuda.synchronize()
        assert ctx.device_flags() & gpu.DEVFLAG_TIMEOUT
        assert torch.equal(xi.view(torch.int32), x.view(torch.int32))
    finally:
        ctx.stack_spin_limit(65536)
    again = ctx.decode_stack(0, x, n_layers=8)
    torch.cuda.synchronize()
    assert ctx.device_flags() == 0
    assert torch.equal(again.view(torch.int32), eager.view(torch.int32))


def test_routed_stack_errors(gpu, full):
    import torch
    ctx, _ = full
    x = torch.zeros(H, device="cuda")
    ctx.bind_router(39, None)
    with pytest.raises(gpu.MoeError, match="no bound router"):
        ctx.decode_stack(38, x, n_layers=2)
    with pytest.raises(gpu.MoeError):
        ctx.bind_router(0, torch.zeros(E * H + 1, dtype=torch.float32, device="cuda")[1:])  # misaligned
