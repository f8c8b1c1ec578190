"""Write the golden fixtures for the decode operator (tests/golden/*.npz).

The reference repository holds no golden vectors (its tests generate every
case from seeds), so these fixtures are produced here: seeded fp16 inputs
(ragged batches, shuffled physical pages, never-referenced pages and table
columns, partial last pages, empty rows, x8 keys) and their expected output
from the float64 brute force in oracle/brute.py, which is itself pinned
against torch's scaled_dot_product_attention and closed-form answers
(tests/test_oracle_pins.py).  Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import random
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.brute import decode_f64  # noqa: E402

# name: (lens, num_kv_heads, group, head_dim, page_size, key_boost, scale)
CASES = {
    "primary_gqa6_d128_ps16": ([1, 17, 40, 70], 2, 6, 128, 16, 0, None),
    "gqa1_d64_ps8": ([5, 64, 70], 2, 1, 64, 8, 0, None),
    "gqa4_d32_ps1": ([7, 40], 2, 4, 32, 1, 0, None),
    "gqa8_d128_ps32": ([5, 33, 60], 1, 8, 128, 32, 0, None),
    "zero_len_rows": ([0, 20, 0, 45], 2, 4, 64, 16, 0, None),
    "gqa16_d128_ps16": ([50], 2, 16, 128, 16, 0, None),
    "d96_ps12": ([13, 50], 2, 3, 96, 12, 0, None),
    "d256_gqa2": ([10, 40], 1, 2, 256, 16, 0, None),
    "scaled_keys_x8": ([60, 40], 2, 6, 128, 16, 3, None),
    "explicit_scale": ([33, 40], 2, 6, 128, 16, 0, 0.05),
}


def build(name, lens, hkv, group, d, ps, key_boost, scale, seed):
    rng = random.Random(seed)
    gen = np.random.default_rng(seed)
    pages = [-(-n // ps) if n > 0 else 0 for n in lens]
    width = max(max(pages), 1) + 1
    num_pages = sum(pages) + 2
    ids = list(range(num_pages))
    rng.shuffle(ids)
    bt = np.zeros((len(lens), width), dtype=np.int32)
    cur = 0
    for b, n in enumerate(pages):
        bt[b, :n] = ids[cur:cur + n]
        bt[b, n:] = ids[(cur + n) % num_pages]
        cur += n
    k = gen.standard_normal((num_pages, ps, hkv, d)).astype(np.float16)
    v = gen.standard_normal((num_pages, ps, hkv, d)).astype(np.float16)
    q = gen.standard_normal((len(lens), hkv * group, d)).astype(np.float16)
    for b, n in enumerate(lens):
        for _ in range(key_boost if n > 0 else 0):
            t = rng.randrange(n)
            k[bt[b, t // ps], t % ps] *= np.float16(8.0)
    sl = np.array(lens, dtype=np.int32)
    expected = decode_f64(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), bt, sl, scale)
    return dict(q=q, k_cache=k, v_cache=v, block_table=bt, seq_lens=sl,
                scale=np.array(np.nan if scale is None else scale, dtype=np.float64), expected=expected)


def main():
    for i, (name, spec) in enumerate(CASES.items()):
        arrays = build(name, *spec, seed=9000 + i)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
