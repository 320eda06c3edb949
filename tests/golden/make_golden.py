"""Writes tests/golden/known_answers.npz: inputs and expected outputs computed
with numpy alone (independent of oracle/lava_oracle.c), for the reference's own
known-answer cases on this path and a few small end-to-end problems.

  * int8 / uint8 16x16x16 tiles with a[l] = l % 7, b[l] = l % 5 over the 1-based
    linear index l of a column-major 16x16 tile (test/spirv/test_coopmat_int8.jl:29-40)
  * the per-element callback e * (row + 1) + col (test/spirv/test_coopmat_perelement_inline.jl:20)
  * fp32 -> fp16 narrowing of the named edge inputs (test/test_exact_narrowing.jl:50-52)
  * dot4x8 on edge words (src/vocabulary/vocabulary.jl:31-35)
  * a 48x40x24 fp16 GEMM and a causal S=32 D=16 attention, expected in float64

Run: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "known_answers.npz"


def main():
    d = {}
    # -- int8 / uint8 tiles (column-major, l = 1..256)
    l = np.arange(1, 257)
    a = (l % 7).reshape(16, 16, order="F")
    b = (l % 5).reshape(16, 16, order="F")
    d["i8_a"] = a.astype(np.int8)
    d["i8_b"] = b.astype(np.int8)
    d["i8_c"] = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    # signed extremes: every product -128 * -128
    d["i8_min_c"] = np.full((16, 16), 16 * 16384, dtype=np.int32)
    # -- per-element callback on a 16x16 and a 32x32 fp32 tile
    for t in (16, 32):
        m = (np.arange(t * t, dtype=np.float32).reshape(t, t) / np.float32(7.0) - np.float32(3.0)).astype(np.float32)
        r = np.arange(t, dtype=np.float32)[:, None]
        c = np.arange(t, dtype=np.float32)[None, :]
        d[f"pe_in_{t}"] = m
        d[f"pe_out_{t}"] = (m * (r + np.float32(1)) + c).astype(np.float32)
    # -- exact narrowing edges
    edges = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, -65520.0, np.inf, -np.inf,
                      np.float32(np.finfo(np.float16).tiny), 2.0 ** -24, 2.0 ** -25, np.nextafter(np.float32(2.0 ** -25), np.float32(1)),
                      3.0 * 2.0 ** -26, np.nextafter(np.float32(0), np.float32(1)), np.finfo(np.float32).tiny,
                      1.0 + 2.0 ** -11, 1.0 + 3.0 * 2.0 ** -11], dtype=np.float32)
    d["narrow_in"] = edges
    d["narrow_f16_bits"] = edges.astype(np.float16).view(np.uint16)
    # -- dot4x8
    words_a = np.array([0x80808080, 0x7F7F7F7F, 0x00000000, 0xFFFFFFFF, 0x01020304, 0x80FF7F01], dtype=np.uint32)
    words_b = np.array([0x80808080, 0x7F7F7F7F, 0x12345678, 0xFFFFFFFF, 0x04030201, 0x7F01FF80], dtype=np.uint32)
    ba = words_a.view(np.uint8).reshape(-1, 4).view(np.int8).astype(np.int32)
    bb = words_b.view(np.uint8).reshape(-1, 4).view(np.int8).astype(np.int32)
    d["dot_a"], d["dot_b"], d["dot_y"] = words_a, words_b, (ba * bb).sum(axis=1).astype(np.int32)
    # -- a small fp16 GEMM (A, B row-major)
    g = np.random.default_rng(20240601)
    A = g.uniform(-1, 1, size=(48, 24)).astype(np.float16)
    B = g.uniform(-1, 1, size=(24, 40)).astype(np.float16)
    d["gemm_a"], d["gemm_b"] = A, B
    d["gemm_c"] = A.astype(np.float64) @ B.astype(np.float64)
    # -- a small causal attention, (E, L, H, B) = (16, 32, 2, 1), column-major
    E, L, H = 16, 32, 2
    Q = g.standard_normal((E, L, H, 1)).astype(np.float16)
    K = g.standard_normal((E, L, H, 1)).astype(np.float16)
    V = g.standard_normal((E, L, H, 1)).astype(np.float16)
    O = np.zeros((E, L, H, 1))
    for h in range(H):
        q, k, v = (x[:, :, h, 0].T.astype(np.float64) for x in (Q, K, V))
        s = q @ k.T / np.sqrt(E)
        s[np.triu_indices(L, 1)] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        O[:, :, h, 0] = (p @ v).T
    d["attn_q"], d["attn_k"], d["attn_v"], d["attn_o"] = Q, K, V, O
    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
