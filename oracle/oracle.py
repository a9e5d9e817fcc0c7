"""Python view of the CPU oracle (liborc.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, as
the checker or as the timed CPU baseline.  The product package never imports it.
All arrays are numpy; see moe_oracle.h for the semantics and the reference lines each
function restates.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liborc.so")

QK, SB_BYTES, SLOTS = 256, 136, 9
W_REF, W_RENORM = 0, 1
ACCUMULATE, RMSNORM = 1, 2
KVALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                   dtype=np.int32)

_L = None


def lib():
    global _L
    if _L is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} missing: run make -C oracle")
        L = ctypes.CDLL(LIB_PATH)
        vp, i, u64, sz, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_double
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_dequant_iq4xs.argtypes = [vp, sz, vp]
        L.orc_router_topk.argtypes = [vp, i, i, i, vp, vp]
        L.orc_bucket_fill.argtypes = [vp, vp, i, i, vp, vp, vp, vp]
        L.orc_moe_ffn.argtypes = [vp, i, i, i, vp, vp, vp, i, d, i, vp]
        L.orc_expert_forward.argtypes = [vp, vp, vp, i, i, vp, vp]
        L.orc_router_gemv.argtypes = [vp, i, i, vp, i, i, vp]
        L.orc_router_gemv_f32.argtypes = [vp, i, i, vp, i, i, vp]
        L.orc_moe_ffn_f32.argtypes = [vp, i, i, i, vp, vp, vp, i, ctypes.c_float, i, vp]
        L.orc_mix64.argtypes = [u64]
        L.orc_mix64.restype = u64
        L.orc_rng.argtypes = [u64, u64]
        L.orc_rng.restype = u64
        L.orc_normal.argtypes = [u64, u64]
        L.orc_normal.restype = d
        L.orc_glog.argtypes = [d]
        L.orc_glog.restype = d
        L.orc_gcos2pi.argtypes = [d]
        L.orc_gcos2pi.restype = d
        L.orc_gen_iq4xs.argtypes = [u64, u64, sz, vp]
        L.orc_gen_normal.argtypes = [u64, u64, sz, ctypes.c_float, ctypes.c_float, vp]
        L.orc_gen_logits.argtypes = [u64, i, i, i, d, d, vp]
        L.orc_zipf_rank.argtypes = [u64, i, i]
        L.orc_zipf_rank.restype = i
        L.orc_hot_expert.argtypes = [u64, i]
        L.orc_hot_expert.restype = i
        L.orc_num_threads.restype = i
        _L = L
    return _L


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class OrcLayer(ctypes.Structure):
    _fields_ = [("w1", ctypes.c_void_p), ("w3", ctypes.c_void_p), ("w2", ctypes.c_void_p),
                ("w1_stride", ctypes.c_size_t), ("w3_stride", ctypes.c_size_t),
                ("w2_stride", ctypes.c_size_t), ("shared_w1", ctypes.c_void_p),
                ("shared_w3", ctypes.c_void_p), ("shared_w2", ctypes.c_void_p)]


def dequant(blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // SB_BYTES
    out = np.empty(n * QK, dtype=np.float32)
    lib().orc_dequant_iq4xs(_p(blocks), n, _p(out))
    return out


def router_topk(logits, mode=W_REF):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    M, E = logits.shape
    ids = np.empty((M, SLOTS), dtype=np.uint16)
    w = np.empty((M, SLOTS), dtype=np.float32)
    lib().orc_router_topk(_p(logits), M, E, mode, _p(ids), _p(w))
    return ids, w


def router_gemv(wg, x, E, flags=0):
    """logits [M][E] f32 = (x or RMSNorm(x)) . Wg^T.  wg: IQ4_XS bytes of [E][H] (uint8), or
    the matrix [E][H] as float32, or as float16 (widened exactly to float32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, H = x.shape
    out = np.empty((M, E), dtype=np.float32)
    wg = np.asarray(wg)
    if wg.dtype == np.uint8:
        wg = np.ascontiguousarray(wg)
        assert wg.size == E * H // QK * SB_BYTES
        lib().orc_router_gemv(_p(wg), H, E, _p(x), M, flags, _p(out))
    else:
        assert wg.dtype in (np.float32, np.float16) and wg.size == E * H
        W = np.ascontiguousarray(wg.reshape(E, H), dtype=np.float32)
        lib().orc_router_gemv_f32(_p(W), H, E, _p(x), M, flags, _p(out))
    return out


def bucket_fill(ids, w, E):
    ids = np.ascontiguousarray(ids, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M = ids.shape[0]
    ranges = np.empty(E + 2, dtype=np.uint32)
    stok = np.empty(SLOTS * M, dtype=np.uint16)
    sw = np.empty(SLOTS * M, dtype=np.float32)
    pos = np.empty((M, SLOTS), dtype=np.uint32)
    lib().orc_bucket_fill(_p(ids), _p(w), M, E, _p(ranges), _p(stok), _p(sw), _p(pos))
    return ranges, stok, sw, pos


class PackedLayer:
    """Host copy of one layer packed as [E+1][w1|w3|w2] (shared expert last)."""

    def __init__(self, buf, H, I, E):
        self.buf = np.ascontiguousarray(buf, dtype=np.uint8)
        self.H, self.I, self.E = H, I, E
        self.mb = H * I // QK * SB_BYTES
        self.eb = 3 * self.mb
        base = self.buf.ctypes.data
        sh = base + E * self.eb
        self.s = OrcLayer(base, base + self.mb, base + 2 * self.mb, self.eb, self.eb, self.eb,
                          sh, sh + self.mb, sh + 2 * self.mb)

    def expert(self, e):
        o = e * self.eb
        return (self.buf[o:o + self.mb], self.buf[o + self.mb:o + 2 * self.mb],
                self.buf[o + 2 * self.mb:o + 3 * self.mb])


def moe_ffn(layer, x, ids, w, c, flags=0, y=None):
    """layer: PackedLayer.  Returns y (float32 [M][H])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M = x.shape[0]
    if y is None:
        y = np.zeros_like(x)
    else:
        y = np.array(y, dtype=np.float32, copy=True)
    lib().orc_moe_ffn(ctypes.byref(layer.s), layer.H, layer.I, layer.E, _p(x), _p(ids), _p(w), M,
                      float(c), flags, _p(y))
    return y


def moe_ffn_f32(layer, x, ids, w, c, flags=0, y=None):
    """The f32, all-core port of moe_ffn used as the timed CPU baseline.  Returns y."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M = x.shape[0]
    y = np.zeros_like(x) if y is None else np.array(y, dtype=np.float32, copy=True)
    lib().orc_moe_ffn_f32(ctypes.byref(layer.s), layer.H, layer.I, layer.E, _p(x), _p(ids), _p(w), M,
                          float(c), flags, _p(y))
    return y


def expert_forward(w1, w3, w2, H, I, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(H, dtype=np.float64)
    w1 = np.ascontiguousarray(w1, dtype=np.uint8)
    w3 = np.ascontiguousarray(w3, dtype=np.uint8)
    w2 = np.ascontiguousarray(w2, dtype=np.uint8)
    lib().orc_expert_forward(_p(w1), _p(w3), _p(w2), H, I, _p(x), _p(y))
    return y


def gen_iq4xs(seed, first, n):
    out = np.empty(n * SB_BYTES, dtype=np.uint8)
    lib().orc_gen_iq4xs(seed & (2**64 - 1), first, n, _p(out))
    return out


def gen_normal(seed, first, n, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().orc_gen_normal(seed & (2**64 - 1), first, n, mean, std, _p(out))
    return out


def gen_logits(seed, M, E, kind=0, param=0.0, hot_value=0.0):
    out = np.empty((M, E), dtype=np.float32)
    lib().orc_gen_logits(seed & (2**64 - 1), M, E, kind, param, hot_value, _p(out))
    return out


def f16_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def f32_to_f16(f):
    return lib().orc_f32_to_f16(float(f))


def num_threads():
    return lib().orc_num_threads()
