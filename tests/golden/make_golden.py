"""Write the known-answer fixtures of the reference's own tests, with numpy only.

The reference's native-kernel test (tests/test_cpu_lightspark.py:80-122 in the
reference repository) draws its inputs from ``np.random.default_rng(41)`` and
checks against numpy expressions; both are reproduced here from numpy alone,
so no reference code is imported or run.  The pack and argmax goldens are the
literal arrays of tests/test_cpu_lightspark.py:36-39 and :59-64.

Output: tests/golden/litespark_kat.npz (plain arrays, no pickles).
Run:    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "litespark_kat.npz"


def main() -> None:
    # tests/test_cpu_lightspark.py:59-62 (pack golden)
    pack_w = np.array([[-7, -1, 0, 7], [6, -6, 3, -3]], dtype=np.int8)
    pack_p = np.array([[0xF9, 0x70], [0xA6, 0xD3]], dtype=np.uint8)
    # tests/test_cpu_lightspark.py:36-39 (argmax)
    argmax_logits = np.array([-1.0, 3.0, 2.0], dtype=np.float32)
    argmax_expected = np.array(1, dtype=np.int64)

    # tests/test_cpu_lightspark.py:80-88 (GEMV known answer)
    rng = np.random.default_rng(41)
    gemv_w = rng.integers(-7, 8, size=(67, 128), dtype=np.int8)
    gemv_x = rng.integers(-127, 128, size=128, dtype=np.int8)
    gemv_scales = rng.random(67, dtype=np.float32)
    gemv_act = np.float32(0.007)
    gemv_acc = gemv_w.astype(np.int32) @ gemv_x.astype(np.int32)
    gemv_expected = gemv_acc.astype(np.float32)
    gemv_expected *= gemv_scales * 0.007

    # tests/test_cpu_lightspark.py:103-122 (GQA known answer, same stream)
    kv_heads, groups, context, capacity, head_dim = 2, 3, 7, 11, 16
    query = rng.standard_normal((kv_heads * groups, head_dim), dtype=np.float32)
    keys = rng.standard_normal((capacity, kv_heads, head_dim), dtype=np.float32)
    values = rng.standard_normal((capacity, kv_heads, head_dim), dtype=np.float32)
    ref_scores = np.einsum(
        "hgd,thd->hgt", query.reshape(kv_heads, groups, head_dim), keys[:context],
        dtype=np.float32,
    ) / np.sqrt(np.float32(head_dim))
    ref_scores -= ref_scores.max(axis=-1, keepdims=True)
    ref_scores = np.exp(ref_scores)
    ref_scores /= ref_scores.sum(axis=-1, keepdims=True)
    gqa_expected = np.einsum(
        "hgt,thd->hgd", ref_scores, values[:context], dtype=np.float32,
    ).reshape(kv_heads * groups, head_dim)

    np.savez(
        OUT,
        pack_w=pack_w, pack_p=pack_p,
        argmax_logits=argmax_logits, argmax_expected=argmax_expected,
        gemv_w=gemv_w, gemv_x=gemv_x, gemv_scales=gemv_scales,
        gemv_act=np.array(gemv_act), gemv_acc=gemv_acc, gemv_expected=gemv_expected,
        gqa_shape=np.array([kv_heads, groups, context, capacity, head_dim], dtype=np.int32),
        gqa_query=query, gqa_keys=keys, gqa_values=values, gqa_expected=gqa_expected,
    )
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
