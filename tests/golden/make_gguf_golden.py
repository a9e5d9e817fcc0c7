"""Writes tests/golden/tiny.gguf: a 656-byte GGUF v3 file assembled field by field from the
published GGUF layout -- the same field order the reference's parser walks
(src/gguf.rs:147-212: magic, u32 version, u64 tensor count, u64 metadata count, the key/values,
then per tensor u64-length name, u32 n_dims, u64 dims, u32 ggml type, u64 offset; tensor data
from the first general.alignment boundary after the tensor table) -- with every offset
computed by hand below and asserted, so that the loader test does not rest on the test-side
writer (tests/gguf_writer.py) reading the format the same way as the loader does.

Contents: 4 metadata entries (a string, general.alignment = 64, a u32, an f32 array); 3
tensors: F32 [4, 2] (a 2 x 4 matrix, rows of 4), IQ4_XS [256, 1] (one super-block), F16 [8].
Run from the repository root: python tests/golden/make_gguf_golden.py"""
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


def gstr(s):
    b = s.encode("ascii")
    return u64(len(b)) + b


# the tensor payloads (values chosen so that a transposed or offset read shows)
F32_ROWS = np.array([[1.0, 2.0, 3.0, 4.0], [-1.0, 0.5, 0.0, 8.0]], dtype="<f4")   # [ne1 = 2][ne0 = 4]
IQ4_BLOCK = bytes([0x00, 0x3C,          # d = f16 1.0
                   0x55, 0xAA,          # scales_h
                   0x10, 0x32, 0x54, 0x76]) + bytes(range(128))                   # scales_l, qs
F16_VALS = np.array([0.0, 1.0, -2.0, 0.5, 65504.0, 2.0 ** -24, -0.0, 3.0], dtype="<f2")


def build():
    b = bytearray()
    b += b"GGUF" + u32(3) + u64(3) + u64(4)
    assert len(b) == 24                                     # 4 + 4 + 8 + 8
    b += gstr("general.architecture") + u32(8) + gstr("moe680m")
    assert len(b) == 24 + (8 + 20) + 4 + (8 + 7) == 71
    b += gstr("general.alignment") + u32(4) + u32(64)
    assert len(b) == 71 + (8 + 17) + 4 + 4 == 104
    b += gstr("moe680m.expert_count") + u32(4) + u32(2)
    assert len(b) == 104 + (8 + 20) + 4 + 4 == 140
    b += gstr("tokenizer.ggml.scores") + u32(9) + u32(6) + u64(2) + struct.pack("<ff", 0.5, -1.25)
    assert len(b) == 140 + (8 + 21) + 4 + 4 + 8 + 8 == 193
    b += gstr("blk.0.ffn_gate_inp.weight") + u32(2) + u64(4) + u64(2) + u32(0) + u64(0)
    assert len(b) == 193 + (8 + 25) + 4 + 16 + 4 + 8 == 258
    b += gstr("blk.0.ffn_up_shexp.weight") + u32(2) + u64(256) + u64(1) + u32(23) + u64(64)
    assert len(b) == 258 + (8 + 25) + 4 + 16 + 4 + 8 == 323
    b += gstr("h16") + u32(1) + u64(8) + u32(1) + u64(256)
    assert len(b) == 323 + (8 + 3) + 4 + 8 + 4 + 8 == 358
    b += bytes(384 - 358)                                   # data from the next 64-byte boundary
    b += F32_ROWS.tobytes()                                 # 384 + 0, 32 bytes
    b += bytes(64 - 32)
    b += IQ4_BLOCK                                          # 384 + 64, 136 bytes
    assert len(b) == 384 + 64 + 136 == 584
    b += bytes(384 + 256 - 584)
    b += F16_VALS.tobytes()                                 # 384 + 256, 16 bytes
    assert len(b) == 656
    return bytes(b)


if __name__ == "__main__":
    with open(os.path.join(HERE, "tiny.gguf"), "wb") as f:
        f.write(build())
