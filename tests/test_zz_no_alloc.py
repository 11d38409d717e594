"""xt_ternary_linear_f32_noalloc (static device scratch, no allocation in the
library) against xt_ternary_linear_f32 through the C ABI: bit-identical
outputs on two calls in a row, the second with a smaller input (the scratch
keeps the first call's contents), for every kernel family that takes the
scratch; sizes beyond the scratch are refused with XT_ERR_INVALID."""
import ctypes

import numpy as np
import pytest
import torch

import xtern

pytestmark = pytest.mark.gpu

LIB = xtern.lib()


def log(msg):
    print(f"[case] {msg}", flush=True)


def tern_bytes(rng, fmt, N, K):
    t = rng.integers(-1, 2, (N, K)).astype(np.int8)
    pack = xtern.pack_ternary5 if fmt == xtern.XT_PACK5 else xtern.pack_ternary4
    return np.concatenate([pack(r) for r in t])


def call(fn, w, x, M, N, mode, stream):
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    rc = fn(w.handle, ctypes.c_void_p(x.data_ptr()), M, ctypes.c_void_p(y.data_ptr()), mode,
            ctypes.c_void_p(stream.cuda_stream))
    return rc, y


CASES = [("pack4_c1_up", xtern.XT_PACK4, 2560, 6912, (128, 40)),
         ("pack4_c1_down", xtern.XT_PACK4, 6912, 2560, (128, 17)),
         ("pack4_gemv", xtern.XT_PACK4, 2560, 640, (8, 2)),
         ("pack4_ragged", xtern.XT_PACK4, 333, 40, (33, 4)),
         ("pack5", xtern.XT_PACK5, 3200, 512, (64, 8)),
         ("int8", xtern.XT_INT8, 2560, 1000, (16, 3))]


@pytest.mark.parametrize("name,fmt,K,N,Ms", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("mode", [xtern.XT_QUANT_AVX512, xtern.XT_QUANT_SCALAR])
def test_noalloc_equals_linear_f32(name, fmt, K, N, Ms, mode):
    rng = np.random.default_rng(7)
    if fmt == xtern.XT_INT8:
        wb = rng.integers(-127, 128, N * K).astype(np.int8).view(np.uint8)
    else:
        wb = tern_bytes(rng, fmt, N, K)
    w = xtern.DeviceWeights(fmt, K, N, wb, rng.uniform(0.5, 1.5, N).astype(np.float32))
    s = torch.cuda.Stream()
    for M in Ms:  # second call smaller than the first
        log(f"noalloc {name} M={M} mode={mode}")
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32) * 3).cuda()
        torch.cuda.synchronize()
        rc0, y0 = call(LIB.xt_ternary_linear_f32, w, x, M, N, mode, s)
        rc1, y1 = call(LIB.xt_ternary_linear_f32_noalloc, w, x, M, N, mode, s)
        s.synchronize()
        assert rc0 == 0 and rc1 == 0, (rc0, rc1, xtern.lib().xt_last_error())
        a, b = y0.cpu().numpy(), y1.cpu().numpy()
        assert np.array_equal(a.view(np.int32), b.view(np.int32)), f"{int((a != b).sum())} differ"


def test_noalloc_refuses_beyond_scratch():
    log("noalloc size limit")
    rng = np.random.default_rng(3)
    K, N, M = 6912, 32, 1300  # 1300 * 6912 bytes > 8 MiB
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, tern_bytes(rng, xtern.XT_PACK4, N, K),
                            np.ones(N, np.float32))
    x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
    rc, _ = call(LIB.xt_ternary_linear_f32_noalloc, w, x, M, N, 0, torch.cuda.current_stream())
    assert rc == xtern.XT_ERR_INVALID
    assert b"scratch" in LIB.xt_last_error()
