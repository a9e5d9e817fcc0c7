"""GPU: IQ4_XS decode (bit-exact) and the seeded generators (bit-identical to the oracle)."""
import os

import numpy as np
import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits_equal(a, b):
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | nan))


def test_dequant_golden_kat(gpu):
    import torch
    z = np.load(os.path.join(GOLD, "iq4xs_kat.npz"))
    log(f"dequant KAT: {z['blocks'].size // 136} blocks")
    blocks = torch.from_numpy(z["blocks"]).cuda()
    out = gpu.dequant_iq4xs(blocks).cpu().numpy()
    assert bits_equal(out, z["expected"])


def test_dequant_generated_blocks(gpu, orc):
    import torch
    n = 65536
    log(f"dequant generated: {n} blocks")
    blocks = gpu.gen_iq4xs(n, seed=77)
    got = gpu.dequant_iq4xs(blocks).cpu().numpy()
    ref = orc.dequant(blocks.cpu().numpy())
    assert bits_equal(got, ref)
    # subnormal d values are present and decoded exactly, not flushed
    d = blocks.cpu().numpy().reshape(-1, 136)[:, 0:2].copy().view(np.uint16).reshape(-1)
    sub = ((d >> 10) & 31) == 0
    assert sub.mean() > 0.01
    assert np.any(got.reshape(-1, 256)[sub] != 0)


def test_dequant_empty_and_odd_sizes(gpu, orc):
    import torch
    for n in (0, 1, 3, 31, 33):
        log(f"dequant n={n}")
        blocks = gpu.gen_iq4xs(max(n, 1), seed=5)[: n * 136]
        out = torch.empty(max(n * 256, 4), dtype=torch.float32, device="cuda")
        gpu.dequant_iq4xs(blocks, out=out)
        torch.cuda.synchronize()
        if n:
            assert bits_equal(out[: n * 256].cpu().numpy(), orc.dequant(blocks.cpu().numpy()))


def test_generators_match_oracle(gpu, orc):
    log("generators")
    for seed, first, n in [(0x6D6F65363830 ^ 0x57, 0, 4096), (12345, 10 ** 9, 257)]:
        assert np.array_equal(gpu.gen_iq4xs(n, seed, first).cpu().numpy(), orc.gen_iq4xs(seed, first, n))
    for seed, first, n in [(0x6D6F65363830 ^ 0x58, 0, 200000), (3, 5 * 10 ** 8, 1000)]:
        g = gpu.gen_normal(n, seed, first).cpu().numpy()
        assert np.array_equal(g.view(np.uint32), orc.gen_normal(seed, first, n).view(np.uint32))
    for kind, param, hot in [(0, 0.0, 0.0), (1, 1.1, 0.0), (2, 0.05, 1000.0)]:
        g = gpu.gen_logits(512, 256, 99, kind, param, hot).cpu().numpy()
        o = orc.gen_logits(99, 512, 256, kind, param, hot)
        assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), kind
