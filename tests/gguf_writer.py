"""Writer of small synthetic GGUF v2/v3 files for the loader tests (layout per the published
GGUF spec: header, metadata key/values, tensor infos, then aligned tensor data)."""
import struct

import numpy as np

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
        T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
F32, F16, Q8_0, IQ4_XS = 0, 1, 8, 23


def _string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vt, v):
    if vt == T_STRING:
        return _string(v)
    if vt == T_ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[vt], v)


def write_gguf(path, metadata, tensors, alignment=32, version=3, misalign=None):
    """metadata: [(key, type, value)] (arrays as (elem_type, [values])); tensors:
    [(name, dims, ggml_type, bytes)] with dims in GGUF order (dims[0] = row length).
    general.alignment is written when alignment != 32.  misalign: a tensor name whose
    recorded offset is shifted by 1 (for the error tests)."""
    md = list(metadata)
    if alignment != 32:
        md.append(("general.alignment", T_U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(md))
    for k, vt, v in md:
        head += _string(k) + struct.pack("<I", vt) + _value(vt, v)
    offs, off = [], 0
    for name, dims, tt, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, dims, tt, data), o in zip(tensors, offs):
        o2 = o + 1 if name == misalign else o
        head += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", tt, o2)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, dims, tt, data), o in zip(tensors, offs):
            cur = f.tell() - len(head) - pad
            f.write(b"\0" * (o - cur))
            f.write(np.asarray(data, dtype=np.uint8).tobytes())


def layer_tensors(L, packed, hidden, inter, n_experts, router=None, merged=True, router_type=IQ4_XS):
    """GGUF tensors of one layer from bytes packed as [n_experts+1][w1|w3|w2] (shared last).
    router: IQ4_XS bytes, or (router_type F32 / F16) the [n_experts][hidden] matrix."""
    mb = hidden * inter // 256 * 136
    v = np.asarray(packed, dtype=np.uint8).reshape(n_experts + 1, 3, mb)
    gate, down = [hidden, inter], [inter, hidden]
    out = []
    if merged:
        for j, (stem, dims) in enumerate((("gate", gate), ("up", gate), ("down", down))):
            out.append((f"blk.{L}.ffn_{stem}_exps.weight", dims + [n_experts], IQ4_XS, v[:n_experts, j].reshape(-1)))
            out.append((f"blk.{L}.ffn_{stem}_shexp.weight", dims, IQ4_XS, v[n_experts, j]))
        if router is not None:
            rb = np.ascontiguousarray(router).view(np.uint8).reshape(-1)
            out.append((f"blk.{L}.ffn_gate_inp.weight", [hidden, n_experts], router_type, rb))
    else:
        for j, (w, dims) in enumerate((("w1", gate), ("w3", gate), ("w2", down))):
            for e in range(n_experts):
                out.append((f"blk.{L}.experts.{e}.{w}.weight", dims, IQ4_XS, v[e, j]))
            out.append((f"blk.{L}.shared_expert.{w}.weight", dims, IQ4_XS, v[n_experts, j]))
        if router is not None:
            rb = np.ascontiguousarray(router).view(np.uint8).reshape(-1)
            out.append((f"blk.{L}.ffn_gate.weight", [hidden, n_experts], router_type, rb))
    return out
