"""Writes tests/golden/decode_small.npz: a small seeded decode case and the
oracle's output for it. The test that reads it also checks the stored output
against torch's scaled_dot_product_attention, so the fixture pins the oracle
independently of this script.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import paged_ref as ref  # noqa: E402


def main():
    rng = np.random.default_rng(2024)
    lengths = np.array([0, 1, 15, 16, 17, 40, 63], np.int32)
    block, heads, kv_heads, dim = 8, 4, 2, 16
    pages = int(sum(-(-n // block) for n in lengths)) + 3
    k = rng.standard_normal((pages, block, kv_heads, dim)).astype(np.float32)
    v = rng.standard_normal((pages, block, kv_heads, dim)).astype(np.float32)
    order = list(rng.permutation(pages))
    width = max(-(-int(n) // block) for n in lengths)
    tables = np.full((len(lengths), width), -1, np.int32)
    for row, n in enumerate(lengths):
        for p in range(-(-int(n) // block)):
            tables[row, p] = order.pop()
    q = rng.standard_normal((len(lengths), heads, dim)).astype(np.float32)
    out = ref.paged_attention(q, k, v, tables, lengths)
    np.savez_compressed(os.path.join(HERE, "decode_small.npz"), q=q, k=k, v=v, tables=tables,
                        lengths=lengths, out=out)


if __name__ == "__main__":
    main()
