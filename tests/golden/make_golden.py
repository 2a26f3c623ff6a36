"""Write golden vectors of the reference's own CPU paged attention.

Runs examples/run_gpt2.c:46-83 (static paged_attention), compiled from the
reference tree into oracle/_ref/libref_gpt2_attn.so by `make -C oracle ref`,
on small seeded inputs and stores inputs + outputs in gpt2_paged_attention.npz.
Run in the build container (where the reference tree exists):
    python tests/golden/make_golden.py
The fixture is data only; the tests use it to pin the oracle wherever
oracle/_ref is not built.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from xllms_amd import workloads as W  # noqa: E402

# (name, num_heads, head_dim, page_size, seq_len, num_pages, q_scale)
CASES = [
    ("h12_d64_p16_L20", 12, 64, 16, 20, 2, 1.0),
    ("h4_d64_p16_L1", 4, 64, 16, 1, 1, 1.0),
    ("h4_d32_p4_L13_perm", 4, 32, 4, 13, 6, 1.0),
    ("h2_d64_p8_L40_sharp", 2, 64, 8, 40, 5, 3.0),
]


def build_case(i, name, H, D, P, L, npages, q_scale):
    seed = 20261000 + i
    q = W.normal_values(H * D, seed * 16 + 1).reshape(H, D) * np.float32(q_scale)
    k = W.normal_values(npages * P * H * D, seed * 16 + 2).reshape(npages, P, H, D)
    v = W.normal_values(npages * P * H * D, seed * 16 + 3).reshape(npages, P, H, D)
    rng = np.random.default_rng(seed)
    pages = rng.permutation(npages)[: -(-L // P)]
    page_table = np.array([pages[t // P] for t in range(L)], dtype=np.int32)
    out = O.gpt2_paged_attention(q, k, v, page_table, L, H, D, P, use_reference=True)
    return {f"{name}/q": q.astype(np.float32), f"{name}/k": k, f"{name}/v": v,
            f"{name}/page_table": page_table, f"{name}/out": out,
            f"{name}/shape": np.array([H, D, P, L], dtype=np.int32)}


def main():
    if O.ref_lib() is None:
        O.build(ref=True)
    if O.ref_lib() is None:
        raise SystemExit("oracle/_ref not built: the reference tree is required")
    data = {}
    for i, case in enumerate(CASES):
        data.update(build_case(i, *case))
    data["cases"] = np.array([c[0] for c in CASES])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gpt2_paged_attention.npz")
    np.savez_compressed(path, **data)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
