"""Several host threads calling one weight handle on ONE shared stream (the
reference shares `forward(&self)` across threads through Arc<Llama>:
examples/batch_bench.rs:101-151, server/main.rs:642-644).  Every call's
output must equal the oracle's bit for bit: a workspace shared between two
concurrent callers would let one call's product read the other's quantised
rows.  The shapes take the entry points that use a workspace: M > 1 (separate
quantiser), the long-K kernel, Pack5, and the Int8 LM head."""
import threading

import numpy as np
import pytest
import torch

import oracle
import xtern

pytestmark = pytest.mark.gpu

THREADS, ROUNDS = 4, 12


def log(msg):
    print(f"[case] {msg}", flush=True)


def tern(rng, N, K, p0=0.35):
    p = (1 - p0) / 2
    return rng.choice(np.array([-1, 0, 1], np.int8), size=(N, K), p=[p, p0, p])


CASES = [("pack4", xtern.XT_PACK4, 2560, 640, 8),
         ("pack4_longk", xtern.XT_PACK4, 6912, 256, 32),
         ("pack5", xtern.XT_PACK5, 3200, 512, 8),
         ("int8_head", xtern.XT_INT8, 2560, 128256, 2)]


@pytest.mark.parametrize("name,fmt,K,N,M", CASES, ids=[c[0] for c in CASES])
def test_threads_share_one_stream(name, fmt, K, N, M):
    log(f"concurrent {name} K={K} N={N} M={M} threads={THREADS} rounds={ROUNDS}")
    rng = np.random.default_rng(99)
    if fmt == xtern.XT_INT8:
        wb, ws = oracle.int_new(8, rng.standard_normal((N, K)).astype(np.float32), N, K)
    else:
        t = tern(rng, N, K)
        pack = xtern.pack_ternary4 if fmt == xtern.XT_PACK4 else xtern.pack_ternary5
        wb = np.concatenate([pack(r) for r in t])
        ws = rng.uniform(0.5, 1.5, N).astype(np.float32)
    w = xtern.DeviceWeights(fmt, K, N, wb, ws)
    xs = [rng.standard_normal((M, K)).astype(np.float32) * (1 + i) for i in range(THREADS)]
    if fmt == xtern.XT_INT8:
        want = [oracle.int_forward(8, wb, ws, K, N, x)[0] for x in xs]
    else:
        want = [oracle.linear_forward(fmt, K, N, x, ws, wbytes=wb)[0] for x in xs]
    stream = torch.cuda.Stream()
    xd = [torch.from_numpy(x).cuda() for x in xs]
    ys = [[torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(ROUNDS)]
          for _ in range(THREADS)]
    torch.cuda.synchronize()
    go = threading.Barrier(THREADS)
    errors = []

    def body(i):
        try:
            go.wait()
            for r in range(ROUNDS):
                xtern.linear_f32(w, xd[i], out=ys[i][r], stream=stream)
        except Exception as e:  # reported below
            errors.append(e)

    th = [threading.Thread(target=body, args=(i,)) for i in range(THREADS)]
    for x in th:
        x.start()
    for x in th:
        x.join()
    assert not errors, errors
    stream.synchronize()
    bad = []
    for i in range(THREADS):
        for r in range(ROUNDS):
            y = ys[i][r].cpu().numpy()
            if not np.array_equal(y.view(np.int32), want[i].view(np.int32)):
                bad.append((i, r, int((y != want[i]).sum())))
    assert not bad, f"(thread, round, differing outputs): {bad[:8]}"


def test_short_lived_threads_one_after_another():
    """A server that starts a thread per request (server/main.rs:589-676):
    30 short-lived threads, each making calls of growing size on a shared
    stream and ending.  Every output equals the oracle's; the library hands
    an ended thread's workspace to the next thread (xtern_workspace.h)."""
    log("short-lived threads")
    rng = np.random.default_rng(7)
    K, N = 2560, 640
    t = tern(rng, N, K)
    wb = np.concatenate([xtern.pack_ternary4(r) for r in t])
    ws = rng.uniform(0.5, 1.5, N).astype(np.float32)
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, N, wb, ws)
    stream = torch.cuda.Stream()
    errors = []
    for i in range(30):
        M = 2 + (i % 7) * 5
        x = rng.standard_normal((M, K)).astype(np.float32)
        want = oracle.linear_forward(0, K, N, x, ws, wbytes=wb)[0]
        xd = torch.from_numpy(x).cuda()
        torch.cuda.synchronize()
        out = {}

        def body():
            with torch.cuda.stream(stream):
                out["y"] = xtern.linear_f32(w, xd, stream=stream)
            stream.synchronize()

        th = threading.Thread(target=body)
        th.start()
        th.join()
        got = out["y"].cpu().numpy()
        if not np.array_equal(got.view(np.int32), want.view(np.int32)):
            errors.append(i)
    assert not errors, f"threads {errors} produced wrong outputs"
