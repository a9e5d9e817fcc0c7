"""Writes the committed golden fixtures under tests/golden/.

    python tests/golden/make_golden.py

iq4xs_kat.npz
    Exhaustive known-answer vectors for the GGML IQ4_XS codec: every 6-bit scale (0..63)
    against every nibble (0..15) in both nibble positions, for d in {1, 2^-14 (smallest
    normal), 2^-24 (smallest subnormal), 3*2^-20 (subnormal), 65504 (largest), -0, 2e-3},
    plus bit-placement blocks (one scale or one nibble differs from a background).
    Expected values come from this file's own numpy restatement of ggml's published
    block_iq4_xs / dequantize_row_iq4_xs definition (the reference names the format but
    ships no decoder for it, and ggml is not present), written independently of the C
    oracle: d decoded by numpy's float16, products in float32.
gen_sha256.json
    SHA-256 of small slices of the seeded generator streams (weights, activations and
    logits as used by the tests and the benchmark), so a change to the generator is
    caught.  These come from the C oracle's generator.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))

KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
              dtype=np.float32)
D_VALUES = [(0x3C00, "one"), (0x0400, "min_normal"), (0x0001, "min_subnormal"),
            (0x0003, "subnormal3"), (0x7BFF, "max"), (0x8000, "neg_zero"), (0x1819, "2e-3")]


def pack_block(d_bits, ls8, qs128):
    """ls8: 8 ints in 0..63; qs128: 128 bytes."""
    b = np.zeros(136, dtype=np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    sh = 0
    for ib, ls in enumerate(ls8):
        b[4 + ib // 2] |= (ls & 15) << (4 * (ib % 2))
        sh |= (ls >> 4) << (2 * ib)
    b[2], b[3] = sh & 0xFF, sh >> 8
    b[8:] = np.asarray(qs128, dtype=np.uint8)
    return b


def spec_decode(blocks):
    """numpy restatement of dequantize_row_iq4_xs."""
    blocks = blocks.reshape(-1, 136)
    out = np.empty((blocks.shape[0], 256), dtype=np.float32)
    for n, b in enumerate(blocks):
        d = np.frombuffer(b[0:2].tobytes(), dtype=np.float16)[0].astype(np.float32)
        sh = int(b[2]) | (int(b[3]) << 8)
        for ib in range(8):
            ls = ((int(b[4 + ib // 2]) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
            dl = np.float32(d) * np.float32(ls - 32)
            q = b[8 + 16 * ib: 8 + 16 * ib + 16]
            out[n, 32 * ib: 32 * ib + 16] = dl * KV[q & 15]
            out[n, 32 * ib + 16: 32 * ib + 32] = dl * KV[q >> 4]
    return out.reshape(-1)


def kat_blocks():
    blocks, labels = [], []
    qs_all = np.array([(j | ((15 - j) << 4)) for j in range(16)] * 8, dtype=np.uint8)
    for d_bits, name in D_VALUES:
        for g in range(8):  # 8 blocks x 8 sub-blocks cover ls 0..63
            blocks.append(pack_block(d_bits, [8 * g + i for i in range(8)], qs_all))
            labels.append(f"{name}/ls{8 * g}-{8 * g + 7}")
    # bit placement: background ls=33 (dl = d), nibble 8 (kv = 1); one field changed
    bg_q = np.full(128, 0x88, dtype=np.uint8)
    for ib in range(8):
        for ls in (0, 16, 31, 47, 63):
            ls8 = [33] * 8
            ls8[ib] = ls
            blocks.append(pack_block(0x3C00, ls8, bg_q))
            labels.append(f"place/ls ib{ib}={ls}")
    for pos in range(128):
        for val in (0x80, 0x0F, 0xF8, 0x08 | (3 << 4)):
            q = bg_q.copy()
            q[pos] = val
            blocks.append(pack_block(0x3C00, [33] * 8, q))
            labels.append(f"place/qs{pos}={val:#04x}")
    return np.stack(blocks), labels


def main():
    blocks, labels = kat_blocks()
    expected = spec_decode(blocks)
    np.savez_compressed(os.path.join(HERE, "iq4xs_kat.npz"), blocks=blocks.reshape(-1),
                        expected=expected, labels=np.array(labels))
    import oracle
    sums = {}
    specs = {
        "iq4xs seed=0x6D6F65363830^0x57 first=0 n=64":
            lambda: oracle.gen_iq4xs(0x6D6F65363830 ^ 0x57, 0, 64),
        "iq4xs seed=12345 first=1000000 n=16": lambda: oracle.gen_iq4xs(12345, 1000000, 16),
        "normal seed=0x6D6F65363830^0x58 first=0 n=4096":
            lambda: oracle.gen_normal(0x6D6F65363830 ^ 0x58, 0, 4096),
        "logits seed=99 M=8 E=256 kind=0": lambda: oracle.gen_logits(99, 8, 256, 0),
        "logits seed=99 M=8 E=256 kind=1 s=1.1": lambda: oracle.gen_logits(99, 8, 256, 1, 1.1),
        "logits seed=99 M=64 E=256 kind=2 p=0.05 hot=1000":
            lambda: oracle.gen_logits(99, 64, 256, 2, 0.05, 1000.0),
    }
    for k, f in specs.items():
        sums[k] = hashlib.sha256(np.ascontiguousarray(f()).tobytes()).hexdigest()
    with open(os.path.join(HERE, "gen_sha256.json"), "w") as fh:
        json.dump(sums, fh, indent=1, sort_keys=True)
    print(f"{len(labels)} KAT blocks, {len(sums)} generator checksums")


if __name__ == "__main__":
    main()
