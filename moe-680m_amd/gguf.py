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
(src/memory.rs:152-172).

The file is memory-mapped; a layer's bytes are copied to the GPU once and bound, after which
the library holds its own copy (moe_bind_layer) and the staging buffer is released.
"""
import mmap
import os
import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
GGML_TYPE_IQ4_XS = 23
QK, SB_BYTES = 256, 136
DEFAULT_ALIGNMENT = 32

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

    def nbytes(self):
        if self.type != GGML_TYPE_IQ4_XS:
            raise GGUFError(f"{self.name}: ggml type {self.type}, expected IQ4_XS ({GGML_TYPE_IQ4_XS})")
        if self.dims[0] % QK:
            raise GGUFError(f"{self.name}: row length {self.dims[0]} is not a multiple of {QK}")
        return self.n_elements // QK * SB_BYTES


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

    def iq4xs(self, name, dims=None):
        """Read-only uint8 view of an IQ4_XS tensor's bytes, valid while the file is open (dims
        checked when given, in GGUF order: dims[0] is the row length)."""
        ti = self.tensors.get(name)
        if ti is None:
            raise GGUFError(f"tensor {name} not in {self.path}")
        if dims is not None and ti.dims != tuple(dims):
            raise GGUFError(f"{name}: dims {list(ti.dims)}, expected {list(dims)}")
        n = ti.nbytes()
        start = self.data_offset + ti.offset
        if ti.offset % self.alignment:
            raise GGUFError(f"{name}: offset {ti.offset} not aligned to {self.alignment}")
        if start + n > self._size:
            raise GGUFError(f"{name}: {n} bytes at {start} run past the end of the file ({self._size})")
        return np.frombuffer(self._mm, dtype=np.uint8, count=n, offset=start)


def _layer_host(g, L, hidden, inter, n_experts):
    """Host bytes of layer L packed as [n_experts+1][w1|w3|w2] (the shared expert last), and
    the router matrix (or None when the file has none)."""
    mb = hidden * inter // QK * SB_BYTES
    out = np.empty((n_experts + 1) * 3 * mb, dtype=np.uint8)
    view = out.reshape(n_experts + 1, 3, mb)
    gate_dims = (hidden, inter)   # [rows = inter][cols = hidden]
    down_dims = (inter, hidden)   # [rows = hidden][cols = inter]
    merged = f"blk.{L}.ffn_gate_exps.weight"
    if g.has(merged):
        for j, (stem, dims) in enumerate((("gate", gate_dims), ("up", gate_dims), ("down", down_dims))):
            t = g.iq4xs(f"blk.{L}.ffn_{stem}_exps.weight", dims + (n_experts,))
            view[:n_experts, j, :] = t.reshape(n_experts, mb)
            view[n_experts, j, :] = g.iq4xs(f"blk.{L}.ffn_{stem}_shexp.weight", dims)
        router = f"blk.{L}.ffn_gate_inp.weight"
    else:
        for j, (w, dims) in enumerate((("w1", gate_dims), ("w3", gate_dims), ("w2", down_dims))):
            for e in range(n_experts):
                view[e, j, :] = g.iq4xs(f"blk.{L}.experts.{e}.{w}.weight", dims)
            view[n_experts, j, :] = g.iq4xs(f"blk.{L}.shared_expert.{w}.weight", dims)
        router = f"blk.{L}.ffn_gate.weight"
    wg = np.array(g.iq4xs(router, (hidden, n_experts))) if g.has(router) else None
    return out, wg


def load_layers(ctx, path, layers=None, file_layers=None, device="cuda"):
    """Bind the MoE weights of the GGUF file at `path` into `ctx` (a moe680m_amd.Context).
    layers: context layer indices to fill (default all); file_layers: the file's block index
    for each (default the same).  Returns {context layer: router matrix as a device uint8
    tensor, or None} for moe_router_gemv_topk."""
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
