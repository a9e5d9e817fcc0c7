"""GGUF reader: parse, tensor mapping and error paths on the CPU (against a hand-assembled
golden file too); on the GPU, a file in llama.cpp's layout with an F32 or F16 router, opened
with open_context, routes and runs the FFN like the oracle does on the arrays written into it,
and weights bound from a file give bit-identical results to the same bytes bound directly.

The files are written here from the seeded generator (tests/gguf_writer.py); no model file
is fetched or read from elsewhere."""
import os

import numpy as np
import pytest

from gguf_writer import (F16, F32, IQ4_XS, Q8_0, T_ARRAY, T_BOOL, T_F32, T_STRING, T_U32, layer_tensors,
                         write_gguf)

H, I, E = 512, 256, 16
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny.gguf")


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


def test_golden_file_hand_assembled(gg, orc):
    """tests/golden/tiny.gguf, assembled field by field with hand-computed offsets
    (tests/golden/make_gguf_golden.py): header, metadata of four types, general.alignment 64,
    the data start at 384, tensor offsets relative to it, F32 rows read row-major as
    [ne1][ne0], F16 values and an IQ4_XS block that the oracle decodes per the GGML layout."""
    with gg.GGUFFile(GOLDEN) as g:
        assert g.version == 3 and g.alignment == 64 and g.data_offset == 384
        assert g.metadata["general.architecture"] == "moe680m"
        assert g.metadata["moe680m.expert_count"] == 2
        assert g.metadata["tokenizer.ggml.scores"] == [0.5, -1.25]
        t = g.tensors
        assert (t["blk.0.ffn_gate_inp.weight"].dims, t["blk.0.ffn_gate_inp.weight"].type) == ((4, 2), 0)
        assert (t["blk.0.ffn_up_shexp.weight"].dims, t["blk.0.ffn_up_shexp.weight"].type) == ((256, 1), 23)
        assert (t["h16"].dims, t["h16"].type, t["h16"].offset) == ((8,), 1, 256)
        raw, ty = g.tensor_bytes("blk.0.ffn_gate_inp.weight", (4, 2), types=(gg.GGML_TYPE_F32,))
        W = np.array(raw).view(np.float32).reshape(2, 4)
        assert ty == gg.GGML_TYPE_F32 and W[1, 3] == 8.0 and W[0, 1] == 2.0 and W[1, 0] == -1.0
        h16 = np.array(g.tensor_bytes("h16", types=(gg.GGML_TYPE_F16,))[0]).view(np.float16)
        assert h16.tolist() == [0.0, 1.0, -2.0, 0.5, 65504.0, 2.0 ** -24, -0.0, 3.0]
        blk = np.array(g.iq4xs("blk.0.ffn_up_shexp.weight", (256, 1)))
        assert blk.size == 136 and blk[8] == 0 and blk[135] == 127
        # d = 1.0; sub-block 0: ls = (scales_l[0] & 15) | (scales_h & 3) << 4 = 16, dl = -16;
        # qs[0] = 0 -> kvalues_iq4nl[0] = -127 for weight 0, and qs[0] >> 4 = 0 for weight 16
        y = orc.dequant(blk)
        assert y[0] == -16.0 * -127 and y[16] == -16.0 * -127
        with pytest.raises(gg.GGUFError, match=r"ggml type F16 \(1\), expected IQ4_XS \(23\)"):
            g.iq4xs("h16")


@pytest.mark.parametrize("router_type", [F32, F16])
def test_llamacpp_layout_dense_router(gg, orc, tmp_path, router_type):
    """llama.cpp's merged layout with an unquantized router (ffn_gate_inp as F32 or F16): the
    router comes back as the [n_experts][hidden] matrix in its own dtype, exactly."""
    packed = packed_layer(orc, 400)
    dt = np.float32 if router_type == F32 else np.float16
    W = (np.random.default_rng(401).standard_normal((E, H)) * 0.05).astype(dt)
    path = tmp_path / "d.gguf"
    write_gguf(path, [("general.architecture", T_STRING, "moe680m")],
               layer_tensors(0, packed, H, I, E, router=W, router_type=router_type))
    with gg.GGUFFile(path) as g:
        host, wg = gg._layer_host(g, 0, H, I, E)
    assert np.array_equal(host, packed)
    assert wg.dtype == dt and wg.shape == (E, H) and np.array_equal(wg, W)


def test_refused_types_and_gated_shared_expert(gg, orc, tmp_path):
    """A router of another ggml type and an expert matrix that is not IQ4_XS are refused with
    the tensor's name and type; so is a gated shared expert (ffn_gate_inp_shexp), whose
    output weight is not 1."""
    packed = packed_layer(orc, 410)
    p = tmp_path / "r.gguf"
    good = layer_tensors(0, packed, H, I, E, router=router_bytes(orc, 411))
    bad_router = [(n, d, Q8_0 if n.endswith("ffn_gate_inp.weight") else t, b) for n, d, t, b in good]
    write_gguf(p, [], bad_router)
    with gg.GGUFFile(p) as g:
        with pytest.raises(gg.GGUFError, match=r"blk\.0\.ffn_gate_inp\.weight: ggml type Q8_0 \(8\)"):
            gg._layer_host(g, 0, H, I, E)
    bad_exp = [(n, d, F16 if n.endswith("ffn_down_exps.weight") else t, b) for n, d, t, b in good]
    write_gguf(p, [], bad_exp)
    with gg.GGUFFile(p) as g:
        with pytest.raises(gg.GGUFError, match=r"ffn_down_exps\.weight: ggml type F16 \(1\), expected IQ4_XS"):
            gg._layer_host(g, 0, H, I, E)
    gated = good + [("blk.0.ffn_gate_inp_shexp.weight", [H], F32, np.zeros(4 * H, dtype=np.uint8))]
    write_gguf(p, [], gated)
    with gg.GGUFFile(p) as g:
        with pytest.raises(gg.GGUFError, match="gated shared expert"):
            gg._layer_host(g, 0, H, I, E)


@pytest.mark.parametrize("style", ["llamacpp", "reference"])
def test_model_config(gg, tmp_path, style):
    """The MoE shape from the metadata: llama.cpp's keys under general.architecture (with
    expert_feed_forward_length), or the reference's llama.* keys (src/gguf.rs:120-128)."""
    if style == "llamacpp":
        md = [("general.architecture", T_STRING, "qwen2moe"), ("qwen2moe.block_count", T_U32, 40),
              ("qwen2moe.embedding_length", T_U32, 2048), ("qwen2moe.feed_forward_length", T_U32, 5632),
              ("qwen2moe.expert_feed_forward_length", T_U32, 512), ("qwen2moe.expert_count", T_U32, 256),
              ("qwen2moe.expert_used_count", T_U32, 8)]
    else:
        md = [("general.architecture", T_STRING, "moe680m"), ("llama.block_count", T_U32, 40),
              ("llama.embedding_length", T_U32, 2048), ("llama.feed_forward_length", T_U32, 512),
              ("llama.expert_count", T_U32, 256), ("llama.expert_used_count", T_U32, 8)]
    p = tmp_path / "c.gguf"
    write_gguf(p, md, [])
    with gg.GGUFFile(p) as g:
        assert gg.model_config(g) == {"hidden": 2048, "inter": 512, "n_experts": 256, "n_experts_used": 8,
                                      "n_layers": 40}
    write_gguf(p, md[:-1], [])
    with gg.GGUFFile(p) as g:
        with pytest.raises(gg.GGUFError, match="expert_used_count"):
            gg.model_config(g)


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


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["small", "full"])
def test_llamacpp_file_against_oracle(gpu, gg, orc, tmp_path, shape):
    """A synthetic file in llama.cpp's layout (merged ffn_*_exps, *_shexp, an unquantized
    ffn_gate_inp: F32, or F16 on the small shape's second layer; metadata under the file's
    architecture) opened with open_context: moe_router_gemv_topk_typed on the file's router and
    moe_ffn on the file-bound layer against orc.router_gemv and orc.moe_ffn on the arrays that
    were written into the file."""
    import torch
    from gpu_util import check_errs, log
    if shape == "small":
        h, i, e, nl, Ms = 512, 256, 16, 2, (1, 5, 40)
    else:
        h, i, e, nl, Ms = 2048, 512, 256, 1, (1, 8, 24)
    rng = np.random.default_rng(0x6C6C)
    packed, routers, tensors = [], [], []
    for L in range(nl):
        dev = gpu.gen_layer(h, i, e, 0x6C00 + L)
        torch.cuda.synchronize()
        packed.append(dev.cpu().numpy())
        del dev
        rt = F16 if (shape == "small" and L == 1) else F32
        W = (rng.standard_normal((e, h)) * 0.05).astype(np.float16 if rt == F16 else np.float32)
        routers.append(W)
        tensors += layer_tensors(L, packed[L], h, i, e, router=W, router_type=rt)
    md = [("general.architecture", T_STRING, "qwen2moe"), ("qwen2moe.block_count", T_U32, nl),
          ("qwen2moe.embedding_length", T_U32, h), ("qwen2moe.feed_forward_length", T_U32, 4 * i),
          ("qwen2moe.expert_feed_forward_length", T_U32, i), ("qwen2moe.expert_count", T_U32, e),
          ("qwen2moe.expert_used_count", T_U32, 8)]
    path = tmp_path / "llamacpp.gguf"
    write_gguf(path, md, tensors)
    del tensors
    log(f"gguf llama.cpp layout {shape}: H={h} I={i} E={e}, {nl} layer(s), dense router")
    ctx, got_routers = gg.open_context(path, m_max=64, wmode=gpu.W_RENORM)
    try:
        assert (ctx.hidden, ctx.inter, ctx.n_experts, ctx.n_layers) == (h, i, e, nl)
        for L in range(nl):
            assert got_routers[L].dtype == (torch.float16 if routers[L].dtype == np.float16 else torch.float32)
            host = orc.PackedLayer(packed[L], h, i, e)
            for M in Ms:
                x = gpu.gen_normal(M * h, 0x6D00 + 16 * L + M).view(M, h)
                lg, ids, w = ctx.router_gemv_topk(got_routers[L], x, rmsnorm=True)
                y = ctx.ffn(L, x, ids, w, rmsnorm=True)
                torch.cuda.synchronize()
                assert ctx.device_flags() == 0
                xh = x.cpu().numpy()
                ref_lg = orc.router_gemv(routers[L], xh, e, flags=orc.RMSNORM)
                scale = np.maximum(np.abs(ref_lg).max(axis=1, keepdims=True), 1.0)
                assert np.all(np.abs(lg.cpu().numpy() - ref_lg) <= 1e-5 * scale), (L, M)
                rid, rw = orc.router_topk(ref_lg, orc.W_RENORM)
                top9 = -np.sort(-ref_lg, axis=1)[:, :9]
                clear = np.all(-np.diff(top9, axis=1) > 2e-5 * scale, axis=1)
                gi, gw = ids.cpu().numpy(), w.cpu().numpy()
                assert np.array_equal(gi[clear], rid[clear]), (L, M)
                assert np.allclose(gw[clear], rw[clear], rtol=1e-4), (L, M)
                ref_y = orc.moe_ffn(host, xh, gi, gw, 1.0, orc.RMSNORM)
                check_errs(y.cpu().numpy(), ref_y, M <= 8, tag=f"layer {L} M={M}: ")
    finally:
        ctx.close()
