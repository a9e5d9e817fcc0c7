"""CPU tests that pin the oracle before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the oracle (wrong nibble half, wrong
scale bit, dropped term, transposed operand, wrong tie rule, unstable fill) fails it:
golden KAT vectors, brute force, library routines (numpy/scipy), and invariants.
"""
import hashlib
import json
import math
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KV_PUBLISHED = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def bits_equal(a, b):
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return np.all((a.view(np.uint32) == b.view(np.uint32)) | nan)


# ---------------------------------------------------------------- f16

def test_f16_decode_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    assert bits_equal(got, ref)


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(1e-3),
        rng.standard_normal(2000).astype(np.float32) * np.float32(1e4),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf],
                 dtype=np.float32)])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- IQ4_XS codec

def test_dequant_golden_kat(orc):
    z = np.load(os.path.join(GOLD, "iq4xs_kat.npz"))
    got = orc.dequant(z["blocks"])
    assert bits_equal(got, z["expected"])


def test_dequant_codebook_is_published_table(orc):
    # d = 1 and ls = 33 in every sub-block (scales_h bits 10, scales_l nibble 1), so
    # dl = 1 and the outputs are the codebook itself, nibble by nibble.
    b = np.zeros(136, dtype=np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2:4] = [0xAA, 0xAA]
    b[4:8] = 0x11
    b[8:] = np.array([j | (j << 4) for j in range(16)] * 8, dtype=np.uint8)
    y = orc.dequant(b).reshape(8, 32)
    kv = np.array(KV_PUBLISHED, dtype=np.float32)
    for ib in range(8):
        assert np.array_equal(y[ib, :16], kv)
        assert np.array_equal(y[ib, 16:], kv)
    # ls = 0 (dl = -32 * d) flips and scales it
    b[2:8] = 0
    assert np.array_equal(orc.dequant(b).reshape(8, 32)[0, :16], -32 * kv)


def test_dequant_invariants(orc):
    rng = np.random.default_rng(2)
    blocks = rng.integers(0, 256, size=(32, 136), dtype=np.uint8)
    blocks[:, 1] &= 0x3B  # keep d finite and moderate
    y = orc.dequant(blocks.reshape(-1)).reshape(32, 8, 32)
    # ls = 32 -> zero sub-block
    b2 = blocks.copy()
    b2[:, 4:8] = 0x00
    b2[:, 2:4] = 0xAA  # high bits 10 -> ls = 32 for all
    assert np.all(orc.dequant(b2.reshape(-1)) == 0)
    # doubling d (exponent + 1) doubles every output exactly
    b3 = blocks.copy()
    d = b3[:, 0:2].copy().view(np.uint16).reshape(-1)
    ok = ((d >> 10) & 31) > 0
    ok &= ((d >> 10) & 31) < 30
    d2 = d + (1 << 10)
    b3[:, 0:2] = d2.view(np.uint8).reshape(-1, 2)
    y3 = orc.dequant(b3.reshape(-1)).reshape(32, 8, 32)
    assert np.array_equal(y3[ok], 2 * y[ok])
    # sub-block ib of a block depends only on its own scale bits and 16 qs bytes
    b4 = blocks.copy()
    b4[:, 8 + 16 * 3: 8 + 16 * 4] ^= 0xFF
    y4 = orc.dequant(b4.reshape(-1)).reshape(32, 8, 32)
    keep = [i for i in range(8) if i != 3]
    assert np.array_equal(y4[:, keep], y[:, keep])


# ---------------------------------------------------------------- router

def brute_topk(logits):
    key = np.where(np.isnan(logits), -np.inf, logits.astype(np.float64))
    key = np.where(key == 0, 0.0, key)
    out = []
    for row in key:
        order = np.lexsort((np.arange(row.size), -row))  # logit desc, index asc
        out.append(order[:8])
    return np.array(out)


def softmax64(l):
    from scipy.special import softmax
    return softmax(l.astype(np.float64), axis=-1)


@pytest.mark.parametrize("mode", [0, 1])
def test_router_bruteforce(orc, mode):
    rng = np.random.default_rng(3 + mode)
    logits = rng.standard_normal((128, 256)).astype(np.float32)
    ids, w = orc.router_topk(logits, mode)
    assert np.array_equal(ids[:, :8], brute_topk(logits))
    assert np.all(ids[:, 8] == 256) and np.all(w[:, 8] == 1.0)
    p = softmax64(logits)
    sel = np.take_along_axis(p, ids[:, :8].astype(np.int64), axis=1)
    if mode == 1:
        sel = sel / sel.sum(axis=1, keepdims=True)
        assert np.allclose(w[:, :8].sum(axis=1), 1.0, rtol=1e-6)
    assert np.allclose(w[:, :8], sel, rtol=1e-6, atol=0)
    assert np.all(np.diff(w[:, :8], axis=1) <= 0)


def test_router_ties_nan_inf(orc):
    E = 64
    l = np.zeros((6, E), dtype=np.float32)
    l[1, :] = np.nan
    l[1, [5, 9]] = [1.0, 2.0]                 # only two non-NaN
    l[2, [3, 40]] = np.inf                    # two +inf share the mass
    l[3, :] = -np.inf                         # all -inf: uniform
    l[4, ::2] = -0.0                          # -0 ties with +0 -> index order
    l[5, :] = np.arange(E)[::-1] % 7          # repeated values
    ids, w = orc.router_topk(l, 0)
    assert list(ids[0, :8]) == list(range(8)) and np.allclose(w[0, :8], 1 / E)
    assert list(ids[1, :2]) == [9, 5] and list(ids[1, 2:8]) == [0, 1, 2, 3, 4, 6]
    assert np.all(w[1, 2:8] == 0)
    assert list(ids[2, :2]) == [3, 40] and np.allclose(w[2, :2], 0.5) and np.all(w[2, 2:8] == 0)
    assert list(ids[3, :8]) == list(range(8)) and np.allclose(w[3, :8], 1 / E)
    assert list(ids[4, :8]) == list(range(8))
    assert np.array_equal(ids[5, :8], brute_topk(l[5:6])[0])


# ---------------------------------------------------------------- bucket fill

def test_bucket_fill_bruteforce(orc):
    rng = np.random.default_rng(5)
    E = 256
    bias = -1.1 * np.log(rng.permutation(E) + 1.0)
    logits = (rng.standard_normal((300, E)) + bias).astype(np.float32)
    ids, w = orc.router_topk(logits, 0)
    ranges, stok, sw, pos = orc.bucket_fill(ids, w, E)
    M = ids.shape[0]
    flat_e = ids.reshape(-1).astype(np.int64)
    flat_t = np.repeat(np.arange(M), 9)
    order = np.argsort(flat_e, kind="stable")        # numpy's stable sort = reference fill order
    assert np.array_equal(stok, flat_t[order])
    assert np.array_equal(sw, w.reshape(-1)[order])
    counts = np.bincount(flat_e, minlength=E + 1)
    assert np.array_equal(ranges, np.concatenate([[0], np.cumsum(counts)]))
    assert ranges[-1] == 9 * M and np.all(np.diff(ranges.astype(np.int64)) >= 0)
    assert (counts == 0).any(), "Zipf skew should leave empty buckets"
    inv = np.empty(9 * M, dtype=np.int64)
    inv[order] = np.arange(9 * M)
    assert np.array_equal(pos.reshape(-1), inv)
    for e in range(E + 1):
        seg = stok[ranges[e]:ranges[e + 1]]
        assert np.all(np.diff(seg.astype(np.int64)) > 0)


# ---------------------------------------------------------------- FFN

def spec_dequant(blocks):
    import sys
    sys.path.insert(0, GOLD)
    from make_golden import spec_decode
    return spec_decode(np.asarray(blocks, dtype=np.uint8))


def small_layer(orc, H=512, I=256, E=16, seed=7):
    from oracle import PackedLayer, SB_BYTES
    n = (E + 1) * 3 * H * I // 256
    buf = orc.gen_iq4xs(seed, 0, n)
    return PackedLayer(buf, H, I, E)


def test_expert_forward_matches_numpy(orc):
    H, I = 512, 256
    L = small_layer(orc, H, I)
    w1, w3, w2 = L.expert(3)
    W1 = spec_dequant(w1).reshape(I, H).astype(np.float64)
    W3 = spec_dequant(w3).reshape(I, H).astype(np.float64)
    W2 = spec_dequant(w2).reshape(H, I).astype(np.float64)
    x = np.random.default_rng(8).standard_normal(H).astype(np.float32)
    g, u = W1 @ x, W3 @ x
    ref = W2 @ (g / (1 + np.exp(-g)) * u)
    got = orc.expert_forward(w1, w3, w2, H, I, x)
    assert np.allclose(got, ref, rtol=1e-10, atol=1e-10 * np.abs(ref).max())


def test_expert_forward_special_cases(orc):
    H, I = 512, 256
    L = small_layer(orc, H, I)
    w1, w3, w2 = L.expert(0)
    # x = e_k picks column k: g = W1[:, k]
    W1 = spec_dequant(w1).reshape(I, H).astype(np.float64)
    W3 = spec_dequant(w3).reshape(I, H).astype(np.float64)
    W2 = spec_dequant(w2).reshape(H, I).astype(np.float64)
    k = 77
    x = np.zeros(H, dtype=np.float32)
    x[k] = 1.0
    g, u = W1[:, k], W3[:, k]
    assert np.allclose(orc.expert_forward(w1, w3, w2, H, I, x), W2 @ (g / (1 + np.exp(-g)) * u),
                       rtol=1e-12)
    # zero gate weights: silu(0) = 0 so the expert outputs exactly 0
    z1 = w1.copy().reshape(-1, 136)
    z1[:, 2:8] = [0xAA, 0xAA, 0, 0, 0, 0]  # ls = 32 in every sub-block
    y = orc.expert_forward(z1.reshape(-1), w3, w2, H, I, np.ones(H, dtype=np.float32))
    assert np.all(y == 0)


def test_moe_ffn_composition(orc):
    H, I, E = 512, 256, 16
    L = small_layer(orc, H, I, E)
    rng = np.random.default_rng(9)
    M = 5
    x = rng.standard_normal((M, H)).astype(np.float32)
    ids, w = orc.router_topk(rng.standard_normal((M, E)).astype(np.float32), 0)
    y0 = rng.standard_normal((M, H)).astype(np.float32)
    c = 1.0 / 9
    got = orc.moe_ffn(L, x, ids, w, c, 0)
    got_acc = orc.moe_ffn(L, x, ids, w, c, 1, y=y0)
    xn = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    got_norm = orc.moe_ffn(L, x, ids, w, c, 2)
    for t in range(M):
        ref = np.zeros(H)
        refn = np.zeros(H)
        for s in range(9):
            e = int(ids[t, s])
            w1, w3, w2 = L.expert(e)
            ref += w[t, s] * orc.expert_forward(w1, w3, w2, H, I, x[t])
            refn += w[t, s] * orc.expert_forward(w1, w3, w2, H, I, xn[t].astype(np.float32))
        assert np.allclose(got[t], c * ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
        assert np.allclose(got_acc[t], y0[t] + c * ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
        assert np.allclose(got_norm[t], c * refn, rtol=1e-5, atol=1e-5 * np.abs(refn).max())


def test_moe_ffn_drops_repeated_and_bad_slots(orc):
    """A slot naming an id above E, or an id its token already named in an earlier slot, adds
    nothing: the result equals the composition of single experts over the remaining slots."""
    H, I, E = 512, 256, 16
    L = small_layer(orc, H, I, E)
    rng = np.random.default_rng(19)
    x = rng.standard_normal((2, H)).astype(np.float32)
    ids, w = orc.router_topk(rng.standard_normal((2, E)).astype(np.float32), 0)
    ids[0, 6] = ids[0, 1]      # repeat of slot 1: dropped
    ids[1, 3] = E + 5          # out of range: dropped
    ids[1, 7] = ids[1, 0]      # repeat of slot 0: dropped
    got = orc.moe_ffn(L, x, ids, w, 1.0, 0)
    kept = {0: [s for s in range(9) if s != 6], 1: [s for s in range(9) if s not in (3, 7)]}
    for t in range(2):
        ref = np.zeros(H)
        for s in kept[t]:
            w1, w3, w2 = L.expert(int(ids[t, s]))
            ref += w[t, s] * orc.expert_forward(w1, w3, w2, H, I, x[t])
        assert np.allclose(got[t], ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


def test_moe_ffn_f32_port_matches_oracle(orc):
    """The f32 port timed as the CPU baseline computes the same layer as the f64 oracle (to
    f32 rounding), for every flag combination, repeated ids included."""
    H, I, E = 512, 256, 16
    L = small_layer(orc, H, I, E, seed=29)
    rng = np.random.default_rng(29)
    x = rng.standard_normal((5, H)).astype(np.float32)
    ids, w = orc.router_topk(rng.standard_normal((5, E)).astype(np.float32), 1)
    ids[2, 5] = ids[2, 0]
    y0 = rng.standard_normal((5, H)).astype(np.float32)
    for flags in (0, 1, 2, 3):
        ref = orc.moe_ffn(L, x, ids, w, 1.0, flags, y=y0)
        got = orc.moe_ffn_f32(L, x, ids, w, 1.0, flags, y=y0)
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max(), flags


# ---------------------------------------------------------------- router gate GEMV

def router_weights(orc, E, H, seed):
    return orc.gen_iq4xs(seed, 0, E * H // 256)


def test_router_gemv_matches_numpy(orc):
    """Against numpy's f64 product of the dequantised matrix (rows = experts): a transposed
    operand, a dropped sub-block or a wrong row stride would all differ by O(1)."""
    E, H = 16, 512
    wg = router_weights(orc, E, H, 0x5267)
    W = orc.dequant(wg).astype(np.float64).reshape(E, H)
    rng = np.random.default_rng(23)
    x = rng.standard_normal((6, H)).astype(np.float32)
    got = orc.router_gemv(wg, x, E)
    ref = x.astype(np.float64) @ W.T
    assert np.allclose(got, ref, rtol=2e-7, atol=1e-7 * np.abs(ref).max())
    xn = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    got_n = orc.router_gemv(wg, x, E, flags=2)
    ref_n = xn @ W.T
    assert np.allclose(got_n, ref_n, rtol=2e-7, atol=1e-7 * np.abs(ref_n).max())


def test_router_gemv_closed_forms(orc):
    """x = unit vector e_k gives column k of Wg exactly (as values: a -0 weight sums to +0);
    a constant row under RMSNorm gives the row sums times 1/sqrt(1 + 1e-6/c^2)."""
    E, H = 16, 512
    wg = router_weights(orc, E, H, 0x5268)
    W = orc.dequant(wg).reshape(E, H)
    ks = [0, 1, 31, 32, 255, 256, 511]
    x = np.zeros((len(ks), H), dtype=np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    got = orc.router_gemv(wg, x, E)
    for i, k in enumerate(ks):
        assert np.array_equal(got[i], W[:, k])
    c = 3.0
    got_c = orc.router_gemv(wg, np.full((1, H), c, dtype=np.float32), E, flags=2)
    ref_c = W.astype(np.float64).sum(axis=1) / math.sqrt(1.0 + 1e-6 / c ** 2)
    assert np.allclose(got_c[0], ref_c, rtol=1e-6, atol=1e-6 * np.abs(ref_c).max())


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_router_gemv_dense_weights(orc, dtype):
    """F32 and F16 gate matrices (llama.cpp keeps ffn_gate_inp unquantized): against numpy's
    f64 product of the matrix as given (rows = experts; f16 widened exactly), under RMSNorm
    too; a unit vector e_k picks column k exactly; a transposed [H][E] matrix differs."""
    E, H = 16, 512
    rng = np.random.default_rng(31)
    W = (rng.standard_normal((E, H)) * 0.05).astype(dtype)
    x = rng.standard_normal((5, H)).astype(np.float32)
    Wd = W.astype(np.float64)
    got = orc.router_gemv(W, x, E)
    ref = x.astype(np.float64) @ Wd.T
    assert np.allclose(got, ref, rtol=2e-7, atol=1e-7 * np.abs(ref).max())
    xn = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    got_n = orc.router_gemv(W, x, E, flags=2)
    assert np.allclose(got_n, xn @ Wd.T, rtol=2e-7, atol=1e-7 * np.abs(ref).max())
    e_k = np.zeros((3, H), dtype=np.float32)
    for i, k in enumerate((0, 77, H - 1)):
        e_k[i, k] = 1.0
    got_k = orc.router_gemv(W, e_k, E)
    for i, k in enumerate((0, 77, H - 1)):
        assert np.array_equal(got_k[i], W[:, k].astype(np.float32))
    # the [H][E] transpose of the same numbers is a different matrix (only square shapes hide it)
    got_t = orc.router_gemv(np.ascontiguousarray(W.T.reshape(E, H)), x, E)
    assert np.abs(got_t - got).max() > 1e-2


# ---------------------------------------------------------------- generator

def test_generator_math(orc):
    L = orc.lib()
    rng = np.random.default_rng(10)
    for x in np.concatenate([rng.random(2000), [1.0, 2.0 ** -53, 0.5, 0.7071067811865476, 3.0, 256.0]]):
        assert abs(L.orc_glog(float(x)) - math.log(x)) <= 4e-16 * max(1.0, abs(math.log(x)))
    for u in np.concatenate([rng.random(2000), [0.0, 0.125, 0.25, 0.375, 0.5, 0.75, 0.999999]]):
        assert abs(L.orc_gcos2pi(float(u)) - math.cos(2 * math.pi * u)) <= 2e-15


def test_generator_statistics(orc):
    from scipy import stats
    z = orc.gen_normal(42, 0, 200000).astype(np.float64)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert stats.kstest(z, "norm").pvalue > 1e-3
    blocks = orc.gen_iq4xs(43, 0, 20000).reshape(-1, 136)
    nib = np.concatenate([blocks[:, 8:] & 15, blocks[:, 8:] >> 4]).reshape(-1)
    assert stats.chisquare(np.bincount(nib, minlength=16)).pvalue > 1e-3
    sh = blocks[:, 2].astype(np.int64) | (blocks[:, 3].astype(np.int64) << 8)
    ls = np.stack([((blocks[:, 4 + ib // 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
                   for ib in range(8)]).reshape(-1)
    assert stats.chisquare(np.bincount(ls, minlength=64)).pvalue > 1e-3
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
    assert np.all(d >= 0)
    assert stats.kstest(d / 2e-3, stats.halfnorm.cdf).pvalue > 1e-4
    sub = np.mean(d < 2.0 ** -14)
    assert abs(sub - 0.0243) < 0.004  # ~2.4% subnormal d, decoded exactly


def test_generator_golden_sha(orc):
    with open(os.path.join(GOLD, "gen_sha256.json")) as fh:
        want = json.load(fh)
    got = {
        "iq4xs seed=0x6D6F65363830^0x57 first=0 n=64": orc.gen_iq4xs(0x6D6F65363830 ^ 0x57, 0, 64),
        "iq4xs seed=12345 first=1000000 n=16": orc.gen_iq4xs(12345, 1000000, 16),
        "normal seed=0x6D6F65363830^0x58 first=0 n=4096": orc.gen_normal(0x6D6F65363830 ^ 0x58, 0, 4096),
        "logits seed=99 M=8 E=256 kind=0": orc.gen_logits(99, 8, 256, 0),
        "logits seed=99 M=8 E=256 kind=1 s=1.1": orc.gen_logits(99, 8, 256, 1, 1.1),
        "logits seed=99 M=64 E=256 kind=2 p=0.05 hot=1000": orc.gen_logits(99, 64, 256, 2, 0.05, 1000.0),
    }
    for k, v in got.items():
        assert hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() == want[k], k


def test_logit_bias_kinds(orc):
    E = 256
    ranks = sorted(orc.lib().orc_zipf_rank(99, E, e) for e in range(E))
    assert ranks == list(range(1, E + 1))
    base = orc.gen_logits(99, 64, E, 0)
    zipf = orc.gen_logits(99, 64, E, 1, 1.1)
    bias = (zipf.astype(np.float64) - base).mean(axis=0)
    r = np.array([orc.lib().orc_zipf_rank(99, E, e) for e in range(E)])
    assert np.allclose(bias, -1.1 * np.log(r), atol=1e-5)
    hot = orc.gen_logits(99, 4096, E, 2, 0.05, 1000.0)
    h = orc.lib().orc_hot_expert(99, E)
    frac = np.mean(hot[:, h] == 1000.0)
    assert 0.04 < frac < 0.06
