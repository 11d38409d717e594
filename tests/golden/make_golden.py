"""Writes tests/golden/seeded_small.npz: small seeded cases in the reference's
three weight layouts with the outputs of the pinned CPU oracle (oracle/,
checked against the reference's own known answers in tests/test_oracle.py).

    python tests/golden/make_golden.py

Each case <name> stores: __meta [fmt, in_dim, out_dim], __wbytes (reference
layout bytes), __ws (w_scales), __x (f32 input rows), __q / __inv (quantised
input, AVX-512 rounding), __acc (i32 dots), __y (f32 outputs)."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402


def lcg_ternary(seed, n, p0_num=None):
    r = oracle.Lcg(seed)
    return np.array([[-1, 0, 1][r.below(3)] for _ in range(n)], np.int8)


def main():
    out = {}
    cases = [("pack4_300x37", 0, 300, 37, 3), ("pack5_333x21", 1, 333, 21, 2),
             ("sparse_200x19", 2, 200, 19, 2), ("pack4_2560x16", 0, 2560, 16, 1)]
    for i, (name, fmt, K, N, M) in enumerate(cases):
        t = lcg_ternary(0x1234_5678_9abc_def0 + i, K * N).reshape(N, K)
        rng = np.random.default_rng(100 + i)
        x = rng.standard_normal((M, K)).astype(np.float32)
        x[0, :4] = [2.5, -2.5, 0.5, 10.0]
        ws = rng.uniform(0.5, 1.5, N).astype(np.float32)
        if fmt == 2:
            blob, _ = oracle.sparse_encode_tensor(t, K, N)
            wbytes = np.frombuffer(blob, np.uint8)
            masks, signs, _ = oracle.sparse_from_blob(blob, N, K)
            y, q, inv, acc = oracle.linear_forward(2, K, N, x, ws, masks=masks, signs=signs)
        else:
            pack = oracle.pack4 if fmt == 0 else oracle.pack5
            wbytes = np.concatenate([pack(t[o].astype(np.float32)) for o in range(N)])
            y, q, inv, acc = oracle.linear_forward(fmt, K, N, x, ws, wbytes=wbytes)
        out[name + "__meta"] = np.array([fmt, K, N], np.int64)
        out[name + "__wbytes"] = wbytes
        out[name + "__ws"] = ws
        out[name + "__x"] = x
        out[name + "__q"] = q
        out[name + "__inv"] = inv
        out[name + "__acc"] = acc
        out[name + "__y"] = y
    np.savez_compressed(os.path.join(HERE, "seeded_small.npz"), **out)


if __name__ == "__main__":
    main()
