"""The streaming decode GEMV (xtern_gstream.hip), which a single product
takes for tall matrices (at least 16384 row groups, M <= 16, Pack4 or
XorSparse tiles).  Checked through the C ABI (xt_ternary_linear_q / _f32)
bit for bit: the weight matrix is `copies` copies of one small matrix
stacked along the output dimension, so every block of outputs must equal
the oracle's TernaryLinear::forward of the small matrix (layers.rs:262-345) --
a size-independent check of the full-size launch."""
import zlib

import numpy as np
import pytest
import torch

import oracle
import xtern

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[case] {msg}", flush=True)


def tern(rng, N, K, p0=0.35):
    u = rng.random((N, K))
    return np.where(u < p0, 0, np.where(rng.random((N, K)) < 0.5, -1, 1)).astype(np.int8)


CASES = [  # K, N of the small matrix, copies (N * copies >= 16384 * 16), M
    (2560, 6912, 38, 1),
    (2560, 6912, 38, 2),
    (256, 4096, 64, 5),
    (300, 1000, 263, 8),   # ragged K (padded chunk) and N (last group half full)
    (1024, 2048, 128, 16),
]


@pytest.mark.parametrize("K,N,copies,M", CASES)
@pytest.mark.parametrize("sparse", [False, True])
def test_tall_matrix_stacked_copies(K, N, copies, M, sparse):
    log(f"gstream K={K} N={N} copies={copies} M={M} sparse={sparse}")
    rng = np.random.default_rng(zlib.crc32(f"{K}-{N}-{M}-{sparse}".encode()) & 0xffff)
    t = tern(rng, N, K)
    ws = rng.uniform(0.5, 1.5, N).astype(np.float32)
    NT = N * copies
    assert (NT + 15) // 16 >= 16384
    if sparse:
        blob = np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)
        w = xtern.DeviceWeights(xtern.XT_XORSPARSE, K, NT, np.tile(blob, copies), np.tile(ws, copies))
    else:
        wb = np.concatenate([xtern.pack_ternary4(r) for r in t])
        w = xtern.DeviceWeights(xtern.XT_PACK4, K, NT, np.tile(wb.reshape(N, -1), (copies, 1)).ravel(),
                                np.tile(ws, copies))
    wb4 = np.concatenate([xtern.pack_ternary4(r) for r in t])
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    for mode in (xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR):
        y_ref, q_ref, inv_ref, acc_ref = oracle.linear_forward(0, K, N, x, ws, wbytes=wb4, quant_mode=mode)
        xd = torch.from_numpy(x).cuda()
        y = xtern.linear_f32(w, xd, mode=mode).cpu().numpy()
        assert np.array_equal(y.reshape(M, copies, N).view(np.int32),
                              np.broadcast_to(y_ref[:, None, :], (M, copies, N)).view(np.int32))
    # forward_with_quantized with the i32 accumulators
    q = torch.from_numpy(q_ref).cuda()
    inv = torch.from_numpy(inv_ref).cuda()
    y, acc = xtern.linear_q(w, q, inv, acc=True)
    assert np.array_equal(acc.cpu().numpy().reshape(M, copies, N),
                          np.broadcast_to(acc_ref[:, None, :], (M, copies, N)))
