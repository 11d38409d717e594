"""Activation loads of the ternary product kernels for 2-128 rows: the decode
GEMV's wave-private LDS slices (all rows at once for M <= 4 / 8; 4-row loads
staged chunk by chunk for 5-16 rows) and the prefill GEMM's 4-row loads
through an LDS slice.  Every output and i32 accumulator must equal an exact
float64 matmul of the ternary weights (layers.rs:294's epilogue on the
oracle-checked i8 rows), and the f32 forward the q forward, for ragged M,
ragged K and several row groups / chunk counts per wave."""
import numpy as np
import pytest
import torch

import xtern

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def tern(rng, N, K, p0=0.35):
    p = (1 - p0) / 2
    return rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[p, p0, p])


def bits(t):
    return t.cpu().numpy().view(np.int32)


def run_exact(w, t, ws, x):
    q, inv = xtern.quantize_i8(x)
    y, acc = xtern.linear_q(w, q, inv, acc=True)
    qn, invn = q.cpu().numpy(), inv.cpu().numpy()
    a64 = (qn.astype(np.float64) @ t.astype(np.float64).T).astype(np.int64)
    assert np.array_equal(acc.cpu().numpy(), a64), f"{int((acc.cpu().numpy() != a64).sum())} dots differ"
    y_ref = ((a64.astype(np.float32) * invn[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32)
    assert np.array_equal(bits(y), y_ref.view(np.int32))
    return q, inv, y


@pytest.mark.parametrize("fmt", [xtern.XT_PACK4, xtern.XT_XORSPARSE], ids=["pack4", "sparse"])
@pytest.mark.parametrize("K,N", [(2560, 6912), (6912, 2600), (14336, 1040), (700, 3300)])
@pytest.mark.parametrize("M", [2, 5, 8, 9, 13, 16])
def test_decode_slices(fmt, K, N, M):
    print(f"[case] slices fmt={fmt} K={K} N={N} M={M}", flush=True)
    rng = np.random.default_rng(K + 3 * N + 7 * M + fmt)
    t = tern(rng, N, K)
    if fmt == xtern.XT_PACK4:
        wb = np.concatenate([xtern.pack_ternary4(r) for r in t])
    else:
        wb = np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)
    ws = rng.uniform(0.02, 0.1, N).astype(np.float32)
    w = xtern.DeviceWeights(fmt, K, N, wb, ws)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(DEV)
    _, _, y = run_exact(w, t, ws, x)
    assert np.array_equal(bits(xtern.linear_f32(w, x)), bits(y))


@pytest.mark.parametrize("K,N,M", [(6912, 2560, 17), (6912, 2560, 23), (2560, 2560, 40),
                                   (6912, 2560, 100), (1000, 640, 31)])
def test_prefill_slice(K, N, M):
    print(f"[case] prefill slice K={K} N={N} M={M}", flush=True)
    rng = np.random.default_rng(K + N + M)
    t = tern(rng, N, K)
    wb = np.concatenate([xtern.pack_ternary4(r) for r in t])
    ws = rng.uniform(0.02, 0.1, N).astype(np.float32)
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, wb, ws)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(DEV)
    _, _, y = run_exact(w, t, ws, x)
    assert np.array_equal(bits(xtern.linear_f32(w, x)), bits(y))
