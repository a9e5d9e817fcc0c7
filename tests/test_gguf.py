"""GGUF reader: parse, tensor mapping and error paths on the CPU; on the GPU, weights bound
from a synthetic file give bit-identical results to the same bytes bound directly.

The files are written here from the seeded generator (tests/gguf_writer.py); no model file
is fetched or read from elsewhere."""
import os

import numpy as np
import pytest

from gguf_writer import F16, IQ4_XS, T_ARRAY, T_BOOL, T_F32, T_STRING, T_U32, layer_tensors, write_gguf

H, I, E = 512, 256, 16


@pytest.fixture(scope="module")
def gg(pkg):
    import importlib
    return importlib.import_module("moe680m_amd.gguf")


def packed_layer(orc, seed):
    mb = H * I // 256 * 136
    return orc.gen_iq4xs(seed, 0, (E + 1) * 3 * mb // 136)


def router_bytes(orc, seed):
    return orc.gen_iq4xs(seed, 0, E * H // 256)


@pytest.mark.parametrize("alignment,version", [(32, 3), (64, 3), (32, 2)])
def test_parse_metadata_and_tensors(gg, orc, tmp_path, alignment, version):
    md = [("general.architecture", T_STRING, "moe680m"), ("moe680m.expert_count", T_U32, E),
          ("moe680m.rope.freq_base", T_F32, 1.5), ("general.flag", T_BOOL, True),
          ("tokenizer.tokens", T_ARRAY, (T_STRING, ["a", "bc", ""]))]
    t1 = orc.gen_iq4xs(11, 0, 3)            # 3 blocks: 408 bytes, not a multiple of 32
    t2 = orc.gen_iq4xs(12, 0, 4)
    path = tmp_path / "t.gguf"
    write_gguf(path, md, [("a.weight", [256, 3], IQ4_XS, t1), ("b.weight", [512, 2], IQ4_XS, t2)],
               alignment=alignment, version=version)
    with gg.GGUFFile(path) as g:
        assert g.version == version and g.alignment == alignment
        assert g.metadata["general.architecture"] == "moe680m"
        assert g.metadata["moe680m.expert_count"] == E
        assert g.metadata["moe680m.rope.freq_base"] == np.float32(1.5)
        assert g.metadata["general.flag"] is True
        assert g.metadata["tokenizer.tokens"] == ["a", "bc", ""]
        assert g.tensors["a.weight"].dims == (256, 3) and g.tensors["b.weight"].dims == (512, 2)
        assert np.array_equal(g.iq4xs("a.weight"), t1)
        assert np.array_equal(g.iq4xs("b.weight", (512, 2)), t2)
        assert g.data_offset % alignment == 0


@pytest.mark.parametrize("merged", [True, False])
def test_layer_mapping_matches_packed_layout(gg, orc, tmp_path, merged):
    packed = [packed_layer(orc, 100 + L) for L in range(2)]
    routers = [router_bytes(orc, 200 + L) for L in range(2)]
    tensors = []
    for L in range(2):
        tensors += layer_tensors(L, packed[L], H, I, E, router=routers[L], merged=merged)
    path = tmp_path / "m.gguf"
    write_gguf(path, [("general.architecture", T_STRING, "moe680m")], tensors)
    with gg.GGUFFile(path) as g:
        for L in range(2):
            host, wg = gg._layer_host(g, L, H, I, E)
            assert np.array_equal(host, packed[L])
            assert np.array_equal(wg, routers[L])


def test_errors(gg, orc, tmp_path):
    good = layer_tensors(0, packed_layer(orc, 300), H, I, E, router=router_bytes(orc, 301))
    p = tmp_path / "e.gguf"

    def expect(msg, **kw):
        with pytest.raises(gg.GGUFError, match=msg):
            with gg.GGUFFile(p) as g:
                gg._layer_host(g, 0, kw.get("h", H), kw.get("i", I), kw.get("e", E))

    write_gguf(p, [], good)
    p.write_bytes(b"GGUX" + p.read_bytes()[4:])
    expect("bad magic")
    write_gguf(p, [], good, version=1)
    expect("version 1")
    write_gguf(p, [], good)
    data = p.read_bytes()
    p.write_bytes(data[:-1000])
    expect("past the end")
    p.write_bytes(data[:40])
    expect("truncated")
    bad = [(n, d, F16 if "up_exps" in n else t, b) for n, d, t, b in good]
    write_gguf(p, [], bad)
    expect("expected IQ4_XS")
    write_gguf(p, [], good)
    expect("dims", i=512)
    write_gguf(p, [], good, misalign="blk.0.ffn_down_exps.weight")
    expect("not aligned")
    write_gguf(p, [], good[:-2])   # no shared down matrix (and no router)
    expect("not in")
    with pytest.raises(gg.GGUFError, match="local"):
        gg.GGUFFile("https://example.invalid/model.gguf")


@pytest.mark.gpu
def test_bound_from_file_equals_direct_binding(gpu, gg, orc, tmp_path):
    import torch
    from gpu_util import log
    log("gguf: two layers bound from a synthetic file vs the same bytes bound directly")
    packed = [gpu.gen_layer(H, I, E, 0x6767 + L) for L in range(2)]
    routers = [gpu.gen_iq4xs(E * H // 256, 0x6868 + L) for L in range(2)]
    torch.cuda.synchronize()
    tensors = []
    for L in range(2):
        tensors += layer_tensors(L, packed[L].cpu().numpy(), H, I, E, router=routers[L].cpu().numpy())
    path = tmp_path / "g.gguf"
    write_gguf(path, [("general.architecture", T_STRING, "moe680m")], tensors, alignment=64)
    a = gpu.Context(H, I, E, 2, 64, gpu.W_RENORM)
    b = gpu.Context(H, I, E, 2, 64, gpu.W_RENORM)
    try:
        got_routers = gg.load_layers(a, path, layers=[0, 1], file_layers=[1, 0])
        b.bind_packed(0, packed[1])
        b.bind_packed(1, packed[0])
        for L, FL in ((0, 1), (1, 0)):
            assert torch.equal(got_routers[L].cpu(), routers[FL].cpu())
        for M in (1, 5, 40):
            x = gpu.gen_normal(M * H, 0x6969 + M).view(M, H)
            for L in range(2):
                _, ids, w = a.router_gemv_topk(got_routers[L], x, rmsnorm=True, want_logits=False)
                ya = a.ffn(L, x, ids, w, rmsnorm=True)
                yb = b.ffn(L, x, ids, w, rmsnorm=True)
                torch.cuda.synchronize()
                assert torch.equal(ya.view(torch.int32), yb.view(torch.int32)), (M, L)
    finally:
        a.close()
        b.close()
