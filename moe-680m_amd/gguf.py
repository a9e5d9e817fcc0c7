"""GGUF reader for the MoE layers' IQ4_XS weights, from a local file only.

Replaces the reference's loader for this path: the GGUF parse of src/gguf.rs:147-212 and the
per-layer tensor lookup of src/memory.rs:147-174, 236-262.  Two of the reference's choices are
not followed because they contradict the published GGUF/GGML format (the file format is the
contract): it maps IQ4_XS to type id 30 with 36-byte blocks of 32 weights (src/gguf.rs:47,55,67)
where GGML's IQ4_XS is type 23 with 136-byte blocks of 256 weights, and it ignores
general.alignment (src/gguf.rs:180).  Tensor names: llama.cpp's merged expert tensors
blk.L.ffn_{gate,up,down}_exps (one [n_expert][rows][cols] tensor each), the shared expert
blk.L.ffn_{gate,up,down}_shexp and the router blk.L.ffn_gate_inp; or the reference's own
per-expert names blk.L.experts.E.w{1,3,2}, blk.L.shared_expert.w{1,3,2} and blk.L.ffn_gate
(src/memory.rs:152-172).  The expert matrices must be IQ4_XS; the router may be IQ4_XS, F32 or
F16 (llama.cpp's quantizer leaves ffn_gate_inp unquantized).

The file is memory-mapped; a layer's bytes are copied to the GPU once and bound, after which
the library holds its own copy (moe_bind_layer) and the staging buffer is released.
"""
import mmap
import os
import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_IQ4_XS = 0, 1, 23
QK, SB_BYTES = 256, 136
DEFAULT_ALIGNMENT = 32
# ggml's type ids (ggml.h enum ggml_type), for error messages.  The reference's own table
# (src/gguf.rs:12-28) gives IQ4_XS the id 30, which is ggml's BF16.
GGML_TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1",
                   10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS",
                   17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S",
                   23: "IQ4_XS", 24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16"}
# Bytes per block and elements per block of the types this reader returns.
_TYPE_LAYOUT = {GGML_TYPE_F32: (4, 1), GGML_TYPE_F16: (2, 1), GGML_TYPE_IQ4_XS: (SB_BYTES, QK)}


def type_name(t):
    return f"{GGML_TYPE_NAMES.get(t, 'unknown')} ({t})"

# GGUF metadata value types: id -> struct format (scalars), or the special ids below.
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_T_STRING, _T_ARRAY = 8, 9


class GGUFError(ValueError):
    pass


class _Reader:
    def __init__(self, buf):
        self.buf, self.off = buf, 0

    def need(self, n):
        if self.off + n > len(self.buf):
            raise GGUFError(f"truncated file: {n} bytes needed at offset {self.off}, {len(self.buf)} present")

    def scalar(self, fmt):
        n = struct.calcsize(fmt)
        self.need(n)
        v = struct.unpack_from(fmt, self.buf, self.off)[0]
        self.off += n
        return v

    def string(self):
        n = self.scalar("<Q")
        self.need(n)
        s = bytes(self.buf[self.off:self.off + n]).decode("utf-8", errors="replace")
        self.off += n
        return s

    def value(self, vt):
        if vt in _SCALAR:
            return self.scalar(_SCALAR[vt])
        if vt == _T_STRING:
            return self.string()
        if vt == _T_ARRAY:
            et, n = self.scalar("<I"), self.scalar("<Q")
            if n > len(self.buf):
                raise GGUFError(f"array of {n} elements cannot fit the file")
            return [self.value(et) for _ in range(n)]
        raise GGUFError(f"unknown metadata value type {vt}")


class TensorInfo:
    __slots__ = ("name", "dims", "type", "offset")

    def __init__(self, name, dims, ttype, offset):
        self.name, self.dims, self.type, self.offset = name, tuple(dims), ttype, offset

    @property
    def n_elements(self):
        n = 1
        for d in self.dims:
            n *= d
        return n

    def nbytes(self, types=(GGML_TYPE_IQ4_XS,)):
        """Bytes of the tensor's data, when its type is one of `types` (else a named error)."""
        if self.type not in types:
            want = " or ".join(type_name(t) for t in types)
            raise GGUFError(f"{self.name}: ggml type {type_name(self.type)}, expected {want}")
        bb, be = _TYPE_LAYOUT[self.type]
        if self.dims[0] % be:
            raise GGUFError(f"{self.name}: row length {self.dims[0]} is not a multiple of {be}")
        return self.n_elements // be * bb


class GGUFFile:
    """Header, metadata and tensor table of a GGUF v2/v3 file; tensor bytes by name."""

    def __init__(self, path):
        if "://" in str(path):
            raise GGUFError("a local file path is required")
        self.path = os.fspath(path)
        self._f = open(self.path, "rb")
        size = os.fstat(self._f.fileno()).st_size
        if size < 24:
            self._f.close()
            raise GGUFError(f"{self.path}: {size} bytes is too short for a GGUF header")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse(memoryview(self._mm))
        except Exception:
            self.close()
            raise

    def _parse(self, buf):
        r = _Reader(buf)
        r.need(4)
        if bytes(buf[0:4]) != GGUF_MAGIC:
            raise GGUFError(f"bad magic {bytes(buf[0:4])!r}, expected {GGUF_MAGIC!r}")
        r.off = 4
        self.version = r.scalar("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"GGUF version {self.version} (2 and 3 are read)")
        n_tensors, n_kv = r.scalar("<Q"), r.scalar("<Q")
        if n_tensors > len(buf) or n_kv > len(buf):
            raise GGUFError("tensor or metadata count cannot fit the file")
        self.metadata = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.scalar("<I"))
        self.tensors = {}
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar("<I")
            if nd == 0 or nd > 4:
                raise GGUFError(f"{name}: {nd} dimensions")
            dims = [r.scalar("<Q") for _ in range(nd)]
            ttype, off = r.scalar("<I"), r.scalar("<Q")
            if name in self.tensors:
                raise GGUFError(f"tensor {name} listed twice")
            self.tensors[name] = TensorInfo(name, dims, ttype, off)
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"general.alignment {self.alignment} is not a power of two")
        self.data_offset = (r.off + self.alignment - 1) // self.alignment * self.alignment
        self._size = len(buf)

    def close(self):
        if getattr(self, "_mm", None) is not None:
            try:
                self._mm.close()
            except BufferError:  # a view from iq4xs() is still alive: the GC unmaps later
                pass
            self._mm = None
        if getattr(self, "_f", None) is not None:
            self._f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def has(self, name):
        return name in self.tensors

    def tensor_bytes(self, name, dims=None, types=(GGML_TYPE_IQ4_XS,)):
        """(read-only uint8 view of the tensor's bytes, its ggml type), valid while the file is
        open.  The type must be one of `types`; dims are checked when given, in GGUF order
        (dims[0] is the row length)."""
        ti = self.tensors.get(name)
        if ti is None:
            raise GGUFError(f"tensor {name} not in {self.path}")
        if dims is not None and ti.dims != tuple(dims):
            raise GGUFError(f"{name}: dims {list(ti.dims)}, expected {list(dims)}")
        n = ti.nbytes(types)
        start = self.data_offset + ti.offset
        if ti.offset % self.alignment:
            raise GGUFError(f"{name}: offset {ti.offset} not aligned to {self.alignment}")
        if start + n > self._size:
            raise GGUFError(f"{name}: {n} bytes at {start} run past the end of the file ({self._size})")
        return np.frombuffer(self._mm, dtype=np.uint8, count=n, offset=start), ti.type

    def iq4xs(self, name, dims=None):
        """Read-only uint8 view of an IQ4_XS tensor's bytes (tensor_bytes restricted to IQ4_XS)."""
        return self.tensor_bytes(name, dims)[0]


def model_config(g):
    """The MoE shape a GGUF file's metadata states, as the reference's ModelConfig reads it
    (src/gguf.rs:116-130, keys under "llama."), or under the file's own general.architecture
    prefix as llama.cpp writes it: {"hidden", "inter", "n_experts", "n_experts_used",
    "n_layers"}.  The expert width is <arch>.expert_feed_forward_length when present (llama.cpp
    MoE architectures), else <arch>.feed_forward_length."""
    md = g.metadata
    arch = md.get("general.architecture")
    prefixes = [p for p in (arch, "llama") if p]

    def get(key, required=True):
        for p in prefixes:
            if f"{p}.{key}" in md:
                return int(md[f"{p}.{key}"])
        if required:
            raise GGUFError(f"metadata {prefixes[0]}.{key} missing")
        return None

    inter = get("expert_feed_forward_length", required=False)
    if inter is None:
        inter = get("feed_forward_length")
    return {"hidden": get("embedding_length"), "inter": inter, "n_experts": get("expert_count"),
            "n_experts_used": get("expert_used_count"), "n_layers": get("block_count")}


_ROUTER_DTYPES = {GGML_TYPE_IQ4_XS: np.uint8, GGML_TYPE_F32: np.float32, GGML_TYPE_F16: np.float16}


def _layer_host(g, L, hidden, inter, n_experts):
    """Host bytes of layer L packed as [n_experts+1][w1|w3|w2] (the shared expert last), and
    the router matrix [n_experts][hidden] (or None when the file has none): uint8 IQ4_XS
    bytes, float32 or float16, by the tensor's type.  Every expert matrix must be IQ4_XS; any
    other type is refused with the tensor's name and type."""
    mb = hidden * inter // QK * SB_BYTES
    out = np.empty((n_experts + 1) * 3 * mb, dtype=np.uint8)
    view = out.reshape(n_experts + 1, 3, mb)
    gate_dims = (hidden, inter)   # [rows = inter][cols = hidden]
    down_dims = (inter, hidden)   # [rows = hidden][cols = inter]
    merged = f"blk.{L}.ffn_gate_exps.weight"
    if g.has(merged):
        # llama.cpp's layout: merged [n_expert][rows][cols] expert tensors, the shared expert
        # as *_shexp, the router as ffn_gate_inp
        for j, (stem, dims) in enumerate((("gate", gate_dims), ("up", gate_dims), ("down", down_dims))):
            t = g.iq4xs(f"blk.{L}.ffn_{stem}_exps.weight", dims + (n_experts,))
            view[:n_experts, j, :] = t.reshape(n_experts, mb)
            view[n_experts, j, :] = g.iq4xs(f"blk.{L}.ffn_{stem}_shexp.weight", dims)
        router = f"blk.{L}.ffn_gate_inp.weight"
        shgate = f"blk.{L}.ffn_gate_inp_shexp.weight"
        if g.has(shgate):
            raise GGUFError(f"{shgate}: a gated shared expert is not this path's model (its shared "
                            "expert has weight 1, src/router.rs:50)")
    else:
        # the reference's per-expert names (src/memory.rs:152-172)
        for j, (w, dims) in enumerate((("w1", gate_dims), ("w3", gate_dims), ("w2", down_dims))):
            for e in range(n_experts):
                view[e, j, :] = g.iq4xs(f"blk.{L}.experts.{e}.{w}.weight", dims)
            view[n_experts, j, :] = g.iq4xs(f"blk.{L}.shared_expert.{w}.weight", dims)
        router = f"blk.{L}.ffn_gate.weight"
    wg = None
    if g.has(router):
        raw, t = g.tensor_bytes(router, (hidden, n_experts), types=tuple(_ROUTER_DTYPES))
        wg = np.array(raw).view(_ROUTER_DTYPES[t])
        if t != GGML_TYPE_IQ4_XS:
            wg = wg.reshape(n_experts, hidden)
    return out, wg


def load_layers(ctx, path, layers=None, file_layers=None, device="cuda"):
    """Bind the MoE weights of the GGUF file at `path` into `ctx` (a moe680m_amd.Context).
    layers: context layer indices to fill (default all); file_layers: the file's block index
    for each (default the same).  Returns {context layer: router matrix on the device -- uint8
    IQ4_XS bytes, float32 or float16 as the file stores it, for Context.router_gemv_topk --
    or None}."""
    import torch
    layers = list(range(ctx.n_layers)) if layers is None else list(layers)
    file_layers = layers if file_layers is None else list(file_layers)
    if len(file_layers) != len(layers):
        raise GGUFError("layers and file_layers differ in length")
    routers = {}
    with GGUFFile(path) as g:
        for L, FL in zip(layers, file_layers):
            host, wg = _layer_host(g, FL, ctx.hidden, ctx.inter, ctx.n_experts)
            dev = torch.from_numpy(host).to(device)
            ctx.bind_packed(L, dev)   # the library copies; dev may go
            del dev
            routers[L] = torch.from_numpy(wg).to(device) if wg is not None else None
    return routers


def open_context(path, m_max, wmode=None, device=0):
    """A Context sized from the file's metadata (model_config) with every layer bound, and the
    routers load_layers returns: the loader role of the reference's InferenceEngine::new for
    this path (src/inference.rs:85-126 with src/gguf.rs:147-212 and src/memory.rs:227-291).
    The file must route 8 experts per token (expert_used_count), as this path does."""
    from . import W_RENORM, Context, TOPK
    with GGUFFile(path) as g:
        cfg = model_config(g)
    if cfg["n_experts_used"] != TOPK:
        raise GGUFError(f"expert_used_count {cfg['n_experts_used']}: this path routes {TOPK} experts per token")
    ctx = Context(cfg["hidden"], cfg["inter"], cfg["n_experts"], cfg["n_layers"], m_max,
                  W_RENORM if wmode is None else wmode, device=device)
    try:
        routers = load_layers(ctx, path, device=f"cuda:{device}")
    except Exception:
        ctx.close()
        raise
    return ctx, routers
