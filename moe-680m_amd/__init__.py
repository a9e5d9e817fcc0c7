"""moe680m_amd -- Python binding of the MI355X-native MoE expert-FFN path.

The compute lives in ``libmoe680m.so`` (hand-written gfx950 HIP kernels behind the C ABI
declared in ``include/moe_ffn.h``).  This module only marshals torch tensors (device
memory and the current HIP stream) into that ABI; it has no compute of its own and no
CPU fallback: if the shared library is missing, importing this package raises.

The package directory is ``moe-680m_amd/`` (not an importable identifier), so callers
load it by path; see ``load()`` in ``__graft_entry__.py`` and ``tests/conftest.py``.

Reference interfaces mirrored (path:line in the reference tree):
  ``Context.router_topk``  -- router::route_single / route_cpu (src/router.rs:13-51) and
                              the GPU top-k read back by do_route (src/inference.rs:622-659)
  ``Context.bucket_fill``  -- router::build_expert_batches (src/router.rs:55-97)
  ``Context.ffn``          -- InferenceEngine::record_and_submit_moe (src/inference.rs:663-766)
  ``Context.ffn_route``    -- the RouterTopk dispatch + do_route + record_and_submit_moe of one
                              layer (src/inference.rs:608-616, 622-766)
"""
import ctypes
import os

import torch  # must precede the library load: it brings the process's HIP runtime

_HERE = os.path.dirname(os.path.abspath(__file__))
# MOE680M_TRACE=1 loads the same library built with the decode stack's per-phase timeline
# (moe_stack_trace); results are identical, launches slightly slower.
LIB_PATH = os.path.join(_HERE, "libmoe680m_trace.so" if os.environ.get("MOE680M_TRACE") == "1"
                        else "libmoe680m.so")

QK = 256
SB_BYTES = 136
SLOTS = 9
TOPK = 8
DECODE_MAX_M = 8

MOE_OK, MOE_EINVAL, MOE_ENOMEM, MOE_EHIP, MOE_EUNSUPPORTED, MOE_EDEVICE = range(6)
STATUS_NAMES = {0: "MOE_OK", 1: "MOE_EINVAL", 2: "MOE_ENOMEM", 3: "MOE_EHIP",
                4: "MOE_EUNSUPPORTED", 5: "MOE_EDEVICE"}
W_REF, W_RENORM = 0, 1
FFN_ACCUMULATE, FFN_RMSNORM, STACK_ROUTE_GEMV = 1, 2, 4
DEVFLAG_BAD_ID, DEVFLAG_DUP_ID, DEVFLAG_TIMEOUT = 1, 2, 4
# Router gate matrix element types (GGML type ids, include/moe_ffn.h MOE_WG_*).
WG_F32, WG_F16, WG_IQ4_XS = 0, 1, 23

# Every symbol include/moe_ffn.h declares (checked by the CPU test suite).
EXPORTS = (
    "moe_create", "moe_destroy", "moe_bind_layer", "moe_bind_router", "moe_router_topk", "moe_router_gemv_topk",
    "moe_router_gemv_topk_typed", "moe_bucket_fill",
    "moe_ffn", "moe_ffn_route", "moe_ffn_noalloc", "moe_decode_stack", "moe_dequant_iq4xs", "moe_device_flags",
    "moe_device_flags_async", "moe_stack_spin_limit", "moe_stack_trace", "moe_last_error",
    "moe_timing_enable", "moe_timing_read",
    "moe_gen_iq4xs", "moe_gen_normal", "moe_gen_logits",
)

KERNELS = ("router_topk", "bucket_fill", "decode_gate_up", "decode_down", "prefill_gate_up",
           "prefill_down", "prefill_combine", "decode_stack", "router_gemv", "decode_prep")


class MoeError(RuntimeError):
    def __init__(self, status, message):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


class _Config(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("n_experts", ctypes.c_int),
                ("n_layers", ctypes.c_int), ("m_max", ctypes.c_int), ("wmode", ctypes.c_int)]


class _LayerWeights(ctypes.Structure):
    _fields_ = [("w1", ctypes.c_void_p), ("w3", ctypes.c_void_p), ("w2", ctypes.c_void_p),
                ("w1_stride", ctypes.c_size_t), ("w3_stride", ctypes.c_size_t),
                ("w2_stride", ctypes.c_size_t), ("shared_w1", ctypes.c_void_p),
                ("shared_w3", ctypes.c_void_p), ("shared_w2", ctypes.c_void_p)]


_lib = None


def lib():
    """Load libmoe680m.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                          "(make -C moe-680m_amd); there is no fallback path")
    L = ctypes.CDLL(LIB_PATH)
    vp, i, u64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_size_t
    sigs = {
        "moe_create": [i, ctypes.POINTER(_Config), ctypes.POINTER(vp)],
        "moe_destroy": [vp],
        "moe_bind_layer": [vp, i, ctypes.POINTER(_LayerWeights)],
        "moe_router_topk": [vp, vp, i, vp, vp, vp],
        "moe_router_gemv_topk": [vp, vp, vp, i, i, vp, vp, vp, vp],
        "moe_router_gemv_topk_typed": [vp, vp, i, vp, i, i, vp, vp, vp, vp],
        "moe_bind_router": [vp, i, vp, i],
        "moe_bucket_fill": [vp, vp, vp, i, vp, vp, vp, vp],
        "moe_ffn": [vp, i, vp, vp, vp, i, vp, i, vp],
        "moe_ffn_route": [vp, i, vp, vp, i, vp, vp, vp, i, vp],
        "moe_ffn_noalloc": [vp, i, vp, vp, vp, i, vp, i, vp],
        "moe_decode_stack": [vp, i, i, vp, vp, vp, vp, vp, i, vp],
        "moe_dequant_iq4xs": [vp, sz, vp, vp],
        "moe_device_flags": [vp, vp, ctypes.POINTER(ctypes.c_uint32)],
        "moe_device_flags_async": [vp, vp, vp],
        "moe_stack_spin_limit": [vp, ctypes.c_uint32],
        "moe_stack_trace": [vp, vp, sz],
        "moe_gen_iq4xs": [vp, sz, u64, u64, vp],
        "moe_gen_normal": [vp, sz, u64, u64, ctypes.c_float, ctypes.c_float, vp],
        "moe_gen_logits": [vp, i, i, u64, i, ctypes.c_double, ctypes.c_double, vp],
        "moe_timing_enable": [vp, i],
        "moe_timing_read": [vp, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_double)],
    }
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    L.moe_last_error.argtypes = []
    L.moe_last_error.restype = ctypes.c_char_p
    _lib = L
    return L


def _check(status):
    if status != MOE_OK:
        raise MoeError(status, lib().moe_last_error().decode(errors="replace"))


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream=None):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def matrix_bytes(hidden, inter):
    """Bytes of one IQ4_XS [inter][hidden] (or [hidden][inter]) matrix."""
    return hidden * inter // QK * SB_BYTES


def expert_bytes(hidden, inter):
    """Bytes of one expert packed as w1 | w3 | w2."""
    return 3 * matrix_bytes(hidden, inter)


def layer_bytes(hidden, inter, n_experts):
    """Bytes of one layer packed as experts 0..n_experts-1 then the shared expert."""
    return (n_experts + 1) * expert_bytes(hidden, inter)


class Context:
    """One moe_ctx: shapes, per-layer weight tables and all workspaces."""

    def __init__(self, hidden=2048, inter=512, n_experts=256, n_layers=1, m_max=512,
                 wmode=W_REF, device=0):
        self.hidden, self.inter, self.n_experts = hidden, inter, n_experts
        self.n_layers, self.m_max, self.wmode, self.device = n_layers, m_max, wmode, device
        cfg = _Config(hidden, inter, n_experts, n_layers, m_max, wmode)
        h = ctypes.c_void_p()
        _check(lib().moe_create(device, ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h is not None and self._h.value:
            _check(lib().moe_destroy(self._h))
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bind_layer(self, layer, w1, w3, w2, w1_stride, w3_stride, w2_stride,
                   shared_w1, shared_w3, shared_w2):
        lw = _LayerWeights(_ptr(w1), _ptr(w3), _ptr(w2), w1_stride, w3_stride, w2_stride,
                           _ptr(shared_w1), _ptr(shared_w3), _ptr(shared_w2))
        _check(lib().moe_bind_layer(self._h, layer, ctypes.byref(lw)))

    def bind_packed(self, layer, buf):
        """Bind a uint8 device tensor laid out as [n_experts+1][w1|w3|w2]; the shared
        expert is the last one.  The library keeps its own copy: buf may be freed after."""
        mb = matrix_bytes(self.hidden, self.inter)
        eb = 3 * mb
        need = (self.n_experts + 1) * eb
        if buf.numel() < need:
            raise ValueError(f"layer buffer has {buf.numel()} bytes, needs {need}")
        base = buf.data_ptr()
        sh = base + self.n_experts * eb
        self.bind_layer(layer, base, base + mb, base + 2 * mb, eb, eb, eb,
                        sh, sh + mb, sh + 2 * mb)

    def router_topk(self, logits, ids=None, w=None, stream=None):
        M = logits.shape[0]
        if logits.shape[-1] != self.n_experts:
            raise ValueError("logits last dimension must be n_experts")
        if ids is None:
            ids = torch.empty((M, SLOTS), dtype=torch.uint16, device=logits.device)
        if w is None:
            w = torch.empty((M, SLOTS), dtype=torch.float32, device=logits.device)
        _check(lib().moe_router_topk(self._h, _ptr(logits), M, _ptr(ids), _ptr(w), _stream(stream)))
        return ids, w

    def router_gemv_topk(self, wg, x, rmsnorm=False, logits=None, ids=None, w=None, want_logits=True,
                         want_ids=True, stream=None):
        """Router gate GEMV + top-8 (moe_router_gemv_topk_typed): wg = the [n_experts][hidden]
        gate matrix on the device, as IQ4_XS bytes (uint8), float32 or float16 -- the element
        type follows its dtype; x [M][hidden] f32.  Returns (logits or None, ids or None,
        w or None)."""
        M = x.shape[0]
        if x.shape[-1] != self.hidden:
            raise ValueError("x last dimension must be hidden")
        if wg.dtype == torch.uint8:
            wtype, want = WG_IQ4_XS, matrix_bytes(self.hidden, self.n_experts)
        elif wg.dtype == torch.float32:
            wtype, want = WG_F32, self.n_experts * self.hidden
        elif wg.dtype == torch.float16:
            wtype, want = WG_F16, self.n_experts * self.hidden
        else:
            raise ValueError(f"gate matrix dtype {wg.dtype}: uint8 (IQ4_XS), float32 or float16")
        if wg.numel() != want or not wg.is_contiguous():
            raise ValueError("wg must hold the n_experts x hidden gate matrix, contiguous")
        dev = x.device
        if want_logits and logits is None:
            logits = torch.empty((M, self.n_experts), dtype=torch.float32, device=dev)
        if want_ids and ids is None:
            ids = torch.empty((M, SLOTS), dtype=torch.uint16, device=dev)
        if want_ids and w is None:
            w = torch.empty((M, SLOTS), dtype=torch.float32, device=dev)
        _check(lib().moe_router_gemv_topk_typed(self._h, _ptr(wg), wtype, _ptr(x), M,
                                                FFN_RMSNORM if rmsnorm else 0, _ptr(logits), _ptr(ids),
                                                _ptr(w), _stream(stream)))
        return logits, ids, w

    def bucket_fill(self, ids, w, stream=None):
        M = ids.shape[0]
        dev = ids.device
        ranges = torch.empty(self.n_experts + 2, dtype=torch.int32, device=dev)
        stok = torch.empty(max(SLOTS * M, 1), dtype=torch.uint16, device=dev)
        sw = torch.empty(max(SLOTS * M, 1), dtype=torch.float32, device=dev)
        _check(lib().moe_bucket_fill(self._h, _ptr(ids), _ptr(w), M, _ptr(ranges), _ptr(stok),
                                     _ptr(sw), _stream(stream)))
        return ranges, stok[: SLOTS * M], sw[: SLOTS * M]

    def ffn(self, layer, x, ids, w, y=None, accumulate=False, rmsnorm=False, stream=None):
        M = x.shape[0]
        if y is None:
            y = torch.empty_like(x)
        flags = (FFN_ACCUMULATE if accumulate else 0) | (FFN_RMSNORM if rmsnorm else 0)
        _check(lib().moe_ffn(self._h, layer, _ptr(x), _ptr(ids), _ptr(w), M, _ptr(y), flags,
                             _stream(stream)))
        return y

    def ffn_noalloc(self, layer, x, ids, w, y=None, accumulate=False, rmsnorm=False, stream=None):
        """moe_ffn_noalloc: the decode path (M <= 8) with the library's static scratch."""
        if y is None:
            y = torch.empty_like(x)
        flags = (FFN_ACCUMULATE if accumulate else 0) | (FFN_RMSNORM if rmsnorm else 0)
        _check(lib().moe_ffn_noalloc(self._h, layer, _ptr(x), _ptr(ids), _ptr(w), x.shape[0], _ptr(y), flags,
                                     _stream(stream)))
        return y

    def ffn_route(self, layer, x, logits, y=None, ids=None, w=None, accumulate=False, rmsnorm=False,
                  stream=None):
        """Router + expert FFN in one call (moe_ffn_route); returns (y, ids, w)."""
        M = x.shape[0]
        if y is None:
            y = torch.empty_like(x)
        if ids is None:
            ids = torch.empty((M, SLOTS), dtype=torch.uint16, device=x.device)
        if w is None:
            w = torch.empty((M, SLOTS), dtype=torch.float32, device=x.device)
        flags = (FFN_ACCUMULATE if accumulate else 0) | (FFN_RMSNORM if rmsnorm else 0)
        _check(lib().moe_ffn_route(self._h, layer, _ptr(x), _ptr(logits), M, _ptr(y), _ptr(ids), _ptr(w),
                                   flags, _stream(stream)))
        return y, ids, w

    def decode_stack(self, layer0, x, logits=None, y=None, ids=None, w=None, rmsnorm=True, n_layers=None,
                     stream=None):
        """One token through consecutive layers starting at layer0, x <- x + MoE_l(RMSNorm(x)):
        routing from logits[l] (len(logits) layers), or -- logits None -- from each layer's
        input through the routers bound with bind_router (n_layers layers).  Returns y (= x
        if y is x)."""
        flags = FFN_RMSNORM if rmsnorm else 0
        if logits is None:
            if n_layers is None:
                raise ValueError("n_layers is required when routing from the activations")
            n = n_layers
            flags |= STACK_ROUTE_GEMV
        else:
            n = logits.shape[0]
        if y is None:
            y = torch.empty_like(x)
        _check(lib().moe_decode_stack(self._h, layer0, n, _ptr(x), _ptr(logits), _ptr(y), _ptr(ids),
                                      _ptr(w), flags, _stream(stream)))
        return y

    def bind_router(self, layer, wg):
        """Bind layer's router gate matrix [n_experts][hidden] (a device tensor: uint8 IQ4_XS
        bytes, float32 or float16) for decode_stack without logits; None unbinds.  The
        library keeps the pointer: keep the tensor alive while it is bound."""
        if wg is None:
            _check(lib().moe_bind_router(self._h, layer, None, 0))
            return
        wtype = {torch.uint8: WG_IQ4_XS, torch.float32: WG_F32, torch.float16: WG_F16}.get(wg.dtype)
        if wtype is None:
            raise ValueError(f"gate matrix dtype {wg.dtype}: uint8 (IQ4_XS), float32 or float16")
        want = matrix_bytes(self.hidden, self.n_experts) if wtype == WG_IQ4_XS else self.n_experts * self.hidden
        if wg.numel() != want or not wg.is_contiguous():
            raise ValueError("wg must hold the n_experts x hidden gate matrix, contiguous")
        _check(lib().moe_bind_router(self._h, layer, _ptr(wg), wtype))

    def device_flags(self, stream=None):
        v = ctypes.c_uint32()
        _check(lib().moe_device_flags(self._h, _stream(stream), ctypes.byref(v)))
        return v.value

    def device_flags_async(self, dst, stream=None):
        """Enqueue the move of the sticky flags into dst (a 1-element int32/uint32 tensor on
        the device or in pinned host memory); no host synchronisation."""
        _check(lib().moe_device_flags_async(self._h, _ptr(dst), _stream(stream)))
        return dst

    def stack_spin_limit(self, polls):
        _check(lib().moe_stack_spin_limit(self._h, polls))

    def stack_trace(self, buf):
        """Record decode_stack's per-phase timeline into buf (a device int64 tensor of
        hidden/8 x n_layers x 16 words), or stop with None (MOE680M_TRACE=1 builds only)."""
        _check(lib().moe_stack_trace(self._h, _ptr(buf), 0 if buf is None else buf.numel()))

    def timing_enable(self, capacity=4096):
        _check(lib().moe_timing_enable(self._h, capacity))

    def timing_read(self):
        """{kernel name: (launches timed, total ms)} since the last read."""
        n = len(KERNELS)
        counts = (ctypes.c_int * n)()
        ms = (ctypes.c_double * n)()
        _check(lib().moe_timing_read(self._h, counts, ms))
        return {k: (counts[i], ms[i]) for i, k in enumerate(KERNELS) if counts[i]}


def dequant_iq4xs(blocks, out=None, stream=None):
    n = blocks.numel() // SB_BYTES
    if out is None:
        out = torch.empty(n * QK, dtype=torch.float32, device=blocks.device)
    _check(lib().moe_dequant_iq4xs(_ptr(blocks), n, _ptr(out), _stream(stream)))
    return out


def gen_iq4xs(n_sb, seed, first=0, out=None, device="cuda", stream=None):
    if out is None:
        out = torch.empty(n_sb * SB_BYTES, dtype=torch.uint8, device=device)
    _check(lib().moe_gen_iq4xs(_ptr(out), n_sb, seed & (2**64 - 1), first, _stream(stream)))
    return out


def gen_normal(n, seed, first=0, mean=0.0, std=1.0, out=None, device="cuda", stream=None):
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=device)
    _check(lib().moe_gen_normal(_ptr(out), n, seed & (2**64 - 1), first, mean, std,
                                _stream(stream)))
    return out


def gen_logits(M, E, seed, kind=0, param=0.0, hot_value=0.0, out=None, device="cuda",
               stream=None):
    if out is None:
        out = torch.empty((M, E), dtype=torch.float32, device=device)
    _check(lib().moe_gen_logits(_ptr(out), M, E, seed & (2**64 - 1), kind, param, hot_value,
                                _stream(stream)))
    return out


def gen_layer(hidden, inter, n_experts, seed, out=None, device="cuda", stream=None):
    """One layer's packed weights ([n_experts+1][w1|w3|w2]) from stream `seed`."""
    nbytes = layer_bytes(hidden, inter, n_experts)
    return gen_iq4xs(nbytes // SB_BYTES, seed, 0, out=out, device=device, stream=stream)


# Seeds: base ^ (config << 48) ^ (layer << 32) ^ tensor tag.
SEED_BASE = 0x6D6F65363830
TAG_W, TAG_X, TAG_L = 0x57, 0x58, 0x4C


def seed_for(config, layer, tag):
    return SEED_BASE ^ (config << 48) ^ (layer << 32) ^ tag
