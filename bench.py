#!/usr/bin/env python3
"""Benchmark of the MI355X ternary linear path (libxtern) on one GPU.

Default workload: Pack4 ternary GEMM at prefill size,
M = 128 tokens, up projection (K=2560 -> N=6912) and down projection
(K=6912 -> N=2560).  One step = TernaryLinear::forward of both matrices
(f32 activations in HBM -> per-token absmax i8 quantisation -> ternary i8
MFMA product -> f32 outputs).  Weights rotate over distinct device copies
totalling more than 2x the 256 MB MALL, so every step streams its weights
from HBM.  `value` is whole-job int8 TOPS (2*M*N*K per matrix / step time).

Also reported, from the same process:
  configs      BASELINE configs[2..4]: Pack5 and XorSparse GEMV µs per call and
               GB/s at their M values, and the 30-layer BitNet-2B decode linear
               stack at M = 1, 8, 32
  roofline     the product kernel (mm_kernel) alone: algorithmic ops per
               launch / average launch duration from HIP events on the
               launch stream, against the 5.0 POP/s dense int8 MFMA peak
  gemv_m1      BASELINE configs[0] (Pack4 GEMV, M=1, K=2560, N=6912): GB/s of
               algorithmic bytes against the 8 TB/s HBM peak
  cpu_baseline the oracle's restatement of the reference CPU path (AVX-512
               VNNI dot, min(nproc, 8) threads, per-token tasks) on a bounded
               sample of the same workload

    python bench.py [--steps K] [--warmup W] [--workload c1|c0|c0s|c2s|c3|c4]
                    [--no-cpu] [--copy-calibration]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "xor-net_amd"))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def tern_bytes(np, rng, N, K, fmt, p0=0.35):
    import xtern
    p = (1 - p0) / 2
    u = rng.random((N, K), dtype=np.float32)
    t = np.where(u < p, -1, np.where(u < p + p0, 0, 1)).astype(np.int8)
    if fmt == xtern.XT_PACK4:
        codes = np.where(t < 0, 0, np.where(t > 0, 2, 1)).astype(np.uint8)
        pad = (-K) % 4
        if pad:
            codes = np.concatenate([codes, np.ones((N, pad), np.uint8)], axis=1)
        g = codes.reshape(N, -1, 4)
        return (g[..., 0] | (g[..., 1] << 2) | (g[..., 2] << 4) | (g[..., 3] << 6)).astype(np.uint8).ravel(), t
    if fmt == xtern.XT_PACK5:
        return np.concatenate([xtern.pack_ternary5(r) for r in t]), t
    return np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8), t


def make_copies(np, xtern, fmt, K, N, wb, ws, min_total):
    """Distinct device copies of one matrix, >= min_total bytes together."""
    first = xtern.DeviceWeights(fmt, K, N, wb, ws)
    one = first.device_bytes()
    n = max(1, -(-min_total // one))
    return [first] + [xtern.DeviceWeights(fmt, K, N, wb, ws) for _ in range(n - 1)]


def workload_c1(np, torch, xtern, rng):
    M = 128
    mats = [("up", 2560, 6912), ("down", 6912, 2560)]
    per = max(2 * MALL_BYTES // len(mats), 1)
    sets = []
    for name, K, N in mats:
        wb, _ = tern_bytes(np, rng, N, K, xtern.XT_PACK4)
        ws = np.full(N, 0.8, np.float32)
        copies = make_copies(np, xtern, xtern.XT_PACK4, K, N, wb, ws, per)
        x = rng.standard_normal((M, K)).astype(np.float32)
        x[rng.random((M, K)) < 0.01] *= 20          # 1% outliers x20
        xd = torch.from_numpy(x).cuda()
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        sets.append(dict(name=name, K=K, N=N, copies=copies, x=xd, y=y, xh=x, wb=wb, ws=ws))
    ops_per_step = sum(2 * M * s["N"] * s["K"] for s in sets)
    return dict(M=M, sets=sets, ops=ops_per_step, fmt=xtern.XT_PACK4,
                config={"workload": "c1_pack4_gemm_m128", "M": M,
                        "matrices": [[s["K"], s["N"]] for s in sets],
                        "weight_copies": [len(s["copies"]) for s in sets]})


def run_steps(xtern, wl, steps, start_idx=0):
    for i in range(steps):
        for s in wl["sets"]:
            w = s["copies"][(start_idx + i) % len(s["copies"])]
            xtern.linear_f32(w, s["x"], out=s["y"])


class Graph:
    """A HIP graph of `fn(i)` for i in range(n), captured on its own stream
    after one eager warm-up pass on that stream (workspaces are allocated
    outside capture).  Replays launch the recorded kernels back to back."""

    def __init__(self, torch, fn, n):
        self.torch = torch
        self.stream = torch.cuda.Stream()
        with torch.cuda.stream(self.stream):
            for i in range(n):
                fn(i)
        self.stream.synchronize()
        self.g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.g, stream=self.stream):
            for i in range(n):
                fn(i)
        self.n = n

    def time_ms_median(self, replays):
        """Median, min and max ms per captured call over `replays` replays,
        each replay timed on its own (HIP events on the replay stream); one
        untimed replay first."""
        torch = self.torch
        per = []
        with torch.cuda.stream(self.stream):
            self.g.replay()
            for _ in range(replays):
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record()
                self.g.replay()
                b.record()
                b.synchronize()
                per.append(a.elapsed_time(b) / self.n)
        per.sort()
        return per[len(per) // 2], per[0], per[-1]

    def time_ms(self, replays):
        """Average ms per captured call over `replays` replays (HIP events on
        the replay stream)."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            self.g.replay()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(replays):
                self.g.replay()
            b.record()
        b.synchronize()
        return a.elapsed_time(b) / (replays * self.n)


def flush_mall(torch):
    """Write 1 GiB (4x the 256 MB MALL) so no weights stay cached in it."""
    t = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    t.fill_(1)
    torch.cuda.synchronize()
    del t


def time_exact_steps(torch, xtern, wl, steps, warmup):
    """`warmup` untimed steps, then exactly `steps` timed steps: one HIP graph
    holding `steps` steps (step i on weight copy i mod ncopy), replayed once
    between HIP events on its stream.  The warm-up steps run through their
    own graph on other copies; then the MALL is flushed, so the timed steps
    stream their weights from HBM even when `steps` is below the number of
    copies.  A sleep kernel queued ahead of the start event keeps the GPU
    busy while the host submits the graph, so the events bracket device
    time.  Checks the last timed step's outputs against an eager run."""
    ncopy = len(wl["sets"][0]["copies"])
    g = Graph(torch, lambda i: run_steps(xtern, wl, 1, start_idx=i), steps)
    if warmup > 0:
        gw = Graph(torch, lambda i: run_steps(xtern, wl, 1, start_idx=(steps + i) % ncopy), warmup)
        gw.g.replay()
        gw.stream.synchronize()
        del gw
    flush_mall(torch)
    with torch.cuda.stream(g.stream):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        a.record()
        g.g.replay()
        b.record()
    b.synchronize()
    ms = a.elapsed_time(b) / steps
    got = [s["y"].clone() for s in wl["sets"]]
    run_steps(xtern, wl, 1, start_idx=steps - 1)
    torch.cuda.synchronize()
    for s, y in zip(wl["sets"], got):
        if not torch.equal(s["y"], y):
            raise SystemExit("graph replay output differs from eager output")
    return ms, steps


def product_only(np, torch, xtern, wl, reps):
    """Average duration of one product launch per matrix: a HIP graph of
    back-to-back linear_q (forward_with_quantized) launches over the rotating
    copies, timed with events on the graph's stream."""
    out = []
    for s in wl["sets"]:
        q, inv = xtern.quantize_i8(s["x"])
        torch.cuda.synchronize()
        n = len(s["copies"])
        g = Graph(torch, lambda i, s=s, q=q, inv=inv:
                  xtern.linear_q(s["copies"][i], q, inv, out=s["y"]), n)
        out.append(g.time_ms(max(1, reps // n)))
    return out


def single_launch_us(np, torch, fn, n, reps=60):
    """Median us between HIP events around ONE launch, with a sleep kernel
    queued ahead of the first event so the GPU, not the host, sets the pace:
    the kernel's own duration plus its dispatch, without the launch-to-launch
    gap of back-to-back replays.  fn(i) launches on weight copy i mod n."""
    ts = []
    for r in range(reps):
        torch.cuda._sleep(200_000)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fn(r % n)
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1e3)
    return float(np.median(ts))


def gemv_m1(np, torch, xtern, rng, reps=400):
    """Pack4 GEMV M=1 (K=2560, N=6912), rotating copies
    in a HIP graph; bytes = packed weights + M*K i8 + 4*M inv + 4*N w_scales
    + 4*M*N f32 out (the product launch given q, as the metric's GEMV)."""
    K, N, M = 2560, 6912, 1
    wb, _ = tern_bytes(np, rng, N, K, xtern.XT_PACK4)
    ws = np.full(N, 0.8, np.float32)
    copies = make_copies(np, xtern, xtern.XT_PACK4, K, N, wb, ws, 2 * MALL_BYTES)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    q, inv = xtern.quantize_i8(x)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    y2 = torch.empty_like(y)
    torch.cuda.synchronize()
    n = len(copies)
    g = Graph(torch, lambda i: xtern.linear_q(copies[i], q, inv, out=y), n)
    ms = g.time_ms(max(1, reps // n))
    gf = Graph(torch, lambda i: xtern.linear_f32(copies[i], x, out=y2), n)
    fwd_ms = gf.time_ms(max(1, reps // n))
    us_one = single_launch_us(np, torch, lambda i: xtern.linear_q(copies[i], q, inv, out=y), n)
    wbytes = N * ((K + 3) // 4)
    alg = wbytes + M * K + 4 * M + 4 * N + 4 * M * N
    gbs = alg / (ms * 1e-3) / 1e9
    gbs_one = alg / (us_one * 1e-6) / 1e9
    fwd_alg = wbytes + 4 * M * K + 4 * N + 4 * M * N
    return {"workload": "c0_pack4_gemv_m1", "K": K, "N": N, "M": M,
            "us_per_call_product": round(ms * 1e3, 3),
            "us_per_call_forward_f32": round(fwd_ms * 1e3, 3),
            "forward_f32_GBs": round(fwd_alg / (fwd_ms * 1e-3) / 1e9, 1),
            "alg_bytes_per_call": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "timing": "launch to launch (HIP graph of back-to-back calls)",
                         "traffic": (recorded_traffic() or {}).get("gemv_c0")},
            "us_single_launch": round(us_one, 3),
            "roofline_single_launch": {"achieved": round(gbs_one, 1), "unit": "GB/s",
                                       "frac": round(gbs_one / HBM_PEAK_GBS, 4),
                                       "timing": "events around one launch behind a sleep "
                                                 "kernel (kernel duration + dispatch)"},
            "weight_copies": len(copies)}


def gemv_sustained(np, torch, xtern, rng, ncopies=121, reps=10):
    """north_star's "sustains >= 70 % of peak HBM bandwidth" for the C0 GEMV:
    ONE launch of the decode GEMV over `ncopies` C0 matrices (K=2560,
    N=6912 each) stacked into one weight array of ncopies * 6912 rows at
    distinct addresses (535 MB, > 2x the MALL, so every replay streams from
    HBM), M=1, i8 row given.  Every copy holds the same bytes, so each
    6912-row block of the output must equal the single-matrix output
    (checked), which is itself the C0 product."""
    K, N, M = 2560, 6912, 1
    wb, _ = tern_bytes(np, rng, N, K, xtern.XT_PACK4)
    NT = N * ncopies
    big = np.tile(wb.reshape(N, -1), (ncopies, 1)).ravel()
    w = xtern.DeviceWeights(xtern.XT_PACK4, K, NT, big, np.full(NT, 0.8, np.float32))
    w1 = xtern.DeviceWeights(xtern.XT_PACK4, K, N, wb, np.full(N, 0.8, np.float32))
    del big
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    q, inv = xtern.quantize_i8(x)
    y = torch.empty((M, NT), dtype=torch.float32, device="cuda")
    y1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    xtern.linear_q(w1, q, inv, out=y1)
    torch.cuda.synchronize()
    # eight launches back to back per graph: launch-to-launch time, as for
    # the per-call lines (a graph of one launch adds the replay's own gap:
    # 87-94 us there against 84-85 us with 8 or 16 per graph)
    g = Graph(torch, lambda i: xtern.linear_q(w, q, inv, out=y), 8)
    ms, ms_lo, ms_hi = g.time_ms_median(9)
    if not torch.equal(y.view(ncopies, N), y1.expand(ncopies, N)):
        raise SystemExit("sustained GEMV: a copy's output differs from the single-matrix output")
    alg = NT * (K // 4) + M * K + 4 * M + 4 * NT + 4 * M * NT
    gbs = alg / (ms * 1e-3) / 1e9
    del w, g
    torch.cuda.empty_cache()
    # the same work as a decode stack of ncopies independent C0 ops (distinct
    # weight buffers, one f32 input each, quantised inside the launch)
    copies = [xtern.DeviceWeights(xtern.XT_PACK4, K, N, wb, np.full(N, 0.8, np.float32))
              for _ in range(ncopies)]
    xs = [torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda() for _ in range(ncopies)]
    ys = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(ncopies)]
    st = xtern.Stack([([w_], x_, [y_], None) for w_, x_, y_ in zip(copies, xs, ys)], M)
    gs = Graph(torch, lambda _i: st.run(), 8)
    ms_st, st_lo, st_hi = gs.time_ms_median(9)
    if st.gave_up():
        raise SystemExit("sustained stack: a dependency wait gave up")
    for w_, x_, y_ in zip(copies[:4], xs[:4], ys[:4]):
        if not torch.equal(xtern.linear_f32(w_, x_), y_):
            raise SystemExit("sustained stack output differs from the per-call output")
    alg_st = ncopies * (N * (K // 4) + 4 * M * K + 4 * N + 4 * M * N)
    gbs_st = alg_st / (ms_st * 1e-3) / 1e9
    del gs, st, copies, w1
    torch.cuda.empty_cache()
    return {"workload": "c0_sustained", "K": K, "N_per_copy": N, "copies": ncopies, "M": M,
            "us_per_launch": round(ms * 1e3, 2),
            "us_per_launch_min_max": [round(ms_lo * 1e3, 2), round(ms_hi * 1e3, 2)],
            "timing": "median of 9 graph replays of 8 back-to-back launches, each replay timed",
            "alg_bytes_per_launch": alg,
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "checked": "every copy's 6912 outputs bit-equal to the single C0 product",
            "stack_us_per_launch": round(ms_st * 1e3, 2),
            "stack_us_min_max": [round(st_lo * 1e3, 2), round(st_hi * 1e3, 2)],
            "stack_GBs": round(gbs_st, 1), "stack_hbm_frac": round(gbs_st / HBM_PEAK_GBS, 4),
            "stack_form": f"{ncopies} independent C0 ops (f32 in, quantised in the launch) in one "
                          f"xt_stack launch; checked against per-call outputs"}


def sparse_tern(np, rng, N, K):
    """BASELINE configs[3] weights: ternary with a zero fraction drawn from
    U[0.3, 0.7] per 64-block."""
    nb = K // 64
    zf = rng.uniform(0.3, 0.7, (N, nb, 1)).astype(np.float32)
    u = rng.random((N, nb, 64), dtype=np.float32)
    sign = np.where(rng.random((N, nb, 64), dtype=np.float32) < 0.5, -1, 1)
    return np.where(u < zf, 0, sign).astype(np.int8).reshape(N, K)


def time_product(np, torch, xtern, copies, K, N, M, rng, reps=200):
    """Product (i8 q given) and forward (f32 x) µs per call over rotating
    weight copies, HIP graphs timed with events on the replay stream."""
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    q, inv = xtern.quantize_i8(x)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    n = len(copies)
    gq = Graph(torch, lambda i: xtern.linear_q(copies[i], q, inv, out=y), n)
    gf = Graph(torch, lambda i: xtern.linear_f32(copies[i], x, out=y), n)
    return gq.time_ms(max(1, reps // n)) * 1e3, gf.time_ms(max(1, reps // n)) * 1e3


def gemv_configs(np, torch, xtern, rng, only=None):
    """BASELINE configs[2] (Pack5) and configs[3] (XorSparse): µs per call,
    GB/s of algorithmic bytes (device weight bytes + M*K i8 + scales + f32
    out) against the 8 TB/s HBM peak; weights rotate over > 2x the MALL."""
    out = []
    cases = [("c2_pack5", xtern.XT_PACK5, 3200, 8640, (1, 8)),
             ("c2_pack5", xtern.XT_PACK5, 8640, 3200, (1, 8)),
             ("c3_xorsparse", xtern.XT_XORSPARSE, 4096, 14336, (1, 4, 16)),
             ("c3_xorsparse", xtern.XT_XORSPARSE, 14336, 4096, (1, 4, 16)),
             ("c3_xorsparse_stream", xtern.XT_XORSPARSE_STREAM, 4096, 14336, (1, 4, 16)),
             ("c3_xorsparse_stream", xtern.XT_XORSPARSE_STREAM, 14336, 4096, (1, 4, 16))]
    for name, fmt, K, N, Ms in cases:
        if only and not name.startswith(only):
            continue
        if fmt == xtern.XT_PACK5:
            wb, _ = tern_bytes(np, rng, N, K, fmt, p0=0.4)
            wbytes = N * ((K + 4) // 5)
            blob = None
        else:
            t = sparse_tern(np, rng, N, K)
            wb = np.frombuffer(xtern.encode_sparse_tensor(t, K, N)[0], np.uint8)
            wbytes = N * (K // 64) * 16  # lane-order mask/sign form, as the reference's runtime
            blob = int(wb.size)
            del t
        ws = np.full(N, 0.8, np.float32)
        copies = make_copies(np, xtern, fmt, K, N, wb, ws, 2 * MALL_BYTES)
        if fmt == xtern.XT_XORSPARSE_STREAM:  # the compact stream the kernel reads
            wbytes = copies[0].device_bytes() - 4 * N
        for M in Ms:
            us_q, us_f = time_product(np, torch, xtern, copies, K, N, M, rng)
            alg = wbytes + M * K + 4 * M + 4 * N + 4 * M * N
            gbs = alg / (us_q * 1e-6) / 1e9
            r = {"workload": name, "K": K, "N": N, "M": M, "us_product": round(us_q, 3),
                 "us_forward_f32": round(us_f, 3), "GBs": round(gbs, 1),
                 "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
            if blob:
                r["compact_blob_bytes"] = blob
                r["weight_bytes_read"] = int(wbytes)
            out.append(r)
        del copies
        torch.cuda.empty_cache()
    return out


def stack_c4(np, torch, xtern, rng, Ms=(1, 8, 32), layers=30):
    """the BitNet-2B decode-step linear stack, 30 layers
    x {q, k, v, o, gate, up, down}, f32 activations (q/k/v and gate/up share
    one quantised input, as fused_forward_qkv / _mlp).  Weights are distinct
    device buffers (521 MB, > 2x the MALL).  Four ways, same weights:
      per_call       one library call per op (120 calls), one HIP graph per stack;
      residual_only  the projection stack (xt_stack_*) with only the residual
                     dependency: layer L's q/k/v and gate/up read layer
                     L-1's down output; o and down read inputs that are
                     ready before the run (the library runs it in one launch);
      chain          the strict chain q/k/v -> o -> gate/up -> down -> next
                     layer, each op reading the previous op's raw output (no
                     norm / attention / activation in between: the library
                     runs none of those), in the plan the library picks (one
                     call per op: 120 dependency levels);
      chain_one_launch  the same chain forced into one persistent launch.
    The persistent outputs are checked bit-exact against the per-call ones."""
    shapes = {"q": (2560, 2560), "k": (2560, 640), "v": (2560, 640), "o": (2560, 2560),
              "gate": (2560, 6912), "up": (2560, 6912), "down": (6912, 2560)}
    proto = {n: tern_bytes(np, rng, N, K, xtern.XT_PACK4)[0] for n, (K, N) in shapes.items()}
    # w_scale 1 / sqrt(0.65 K) keeps the outputs at the inputs' magnitude
    # through the 120-projection chain (a fixed 0.9 overflows to inf there)
    W = [{n: xtern.DeviceWeights(xtern.XT_PACK4, K, N, proto[n],
                                 np.full(N, 1.0 / np.sqrt(0.65 * K), np.float32))
          for n, (K, N) in shapes.items()} for _ in range(layers)]
    wbytes = layers * sum(N * K // 4 for K, N in shapes.values())
    ops1 = layers * sum(2 * N * K for K, N in shapes.values())
    res = []
    for M in Ms:
        f32 = torch.float32
        xa = torch.from_numpy(rng.standard_normal((M, 2560)).astype(np.float32)).cuda()
        xd = torch.from_numpy(rng.standard_normal((M, 6912)).astype(np.float32)).cuda()
        ys = {n: torch.empty((M, N), dtype=f32, device="cuda") for n, (K, N) in shapes.items()}

        def stack(_i):
            for L in W:
                xtern.linear_multi_f32([L["q"], L["k"], L["v"]], xa,
                                       outs=[ys["q"], ys["k"], ys["v"]])
                xtern.linear_f32(L["o"], xa, out=ys["o"])
                xtern.linear_multi_f32([L["gate"], L["up"]], xa, outs=[ys["gate"], ys["up"]])
                xtern.linear_f32(L["down"], xd, out=ys["down"])
        g = Graph(torch, stack, 1)
        us = g.time_ms(10) * 1e3
        del g
        row = {"workload": "c4_bitnet2b_projection_stack", "M": M, "layers": layers,
               "us_per_stack": round(us, 1), "weight_GBs": round(wbytes / (us * 1e-6) / 1e9, 1),
               "hbm_frac": round(wbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
               "TOPS": round(ops1 * M / (us * 1e-6) / 1e12, 2)}

        # persistent, two dependency shapes over the same weights:
        #  residual_only  layer L's q/k/v and gate/up read layer L-1's down
        #                 output (written in the launch); o and down read
        #                 inputs ready before the launch, so o/down items can
        #                 run ahead of their layer;
        #  chain          the strict projection chain: q/k/v read the previous
        #                 down, o reads q, gate/up read o, down reads up --
        #                 every op waits for the one before it (the dependency
        #                 shape of a decode step, without its elementwise work).
        xo = [torch.from_numpy(rng.standard_normal((M, 2560)).astype(np.float32)).cuda()
              for _ in range(layers)]
        xdl = [torch.from_numpy(rng.standard_normal((M, 6912)).astype(np.float32)).cuda()
               for _ in range(layers)]
        outs = [{n: torch.empty((M, N), dtype=f32, device="cuda") for n, (K, N) in shapes.items()}
                for _ in range(layers)]

        def ops_residual_only():
            ops = []
            prev_h, prev_dep = xa, None
            for L in range(layers):
                w, o = W[L], outs[L]
                ops.append(([w["down"]], xdl[L], [o["down"]], None))
                dn = len(ops) - 1
                ops.append(([w["q"], w["k"], w["v"]], prev_h, [o["q"], o["k"], o["v"]], prev_dep))
                ops.append(([w["o"]], xo[L], [o["o"]], None))
                ops.append(([w["gate"], w["up"]], prev_h, [o["gate"], o["up"]], prev_dep))
                prev_h, prev_dep = o["down"], dn
            return ops

        def ops_chain():
            ops = []
            prev_h, prev_dep = xa, None
            for L in range(layers):
                w, o = W[L], outs[L]
                ops.append(([w["q"], w["k"], w["v"]], prev_h, [o["q"], o["k"], o["v"]], prev_dep))
                ops.append(([w["o"]], o["q"], [o["o"]], len(ops) - 1))
                ops.append(([w["gate"], w["up"]], o["o"], [o["gate"], o["up"]], len(ops) - 1))
                ops.append(([w["down"]], o["up"], [o["down"]], len(ops) - 1))
                prev_h, prev_dep = o["down"], len(ops) - 1
            return ops

        # plan None: the library's choice (the chain runs per op, the
        # residual-only list in one launch); chain_one_launch forces the
        # chain into one launch, to show what its dependencies cost there
        for tag, ops, plan in (("residual_only", ops_residual_only(), None), ("chain", ops_chain(), None),
                               ("chain_one_launch", ops_chain(), "one_launch")):
            st = xtern.Stack(ops, M, plan=plan)
            row[f"{tag}_plan"] = st.plan_name
            # eight runs back to back in one graph (launch to launch; the runs
            # are ordered on the graph's stream, as the stack requires)
            gs = Graph(torch, lambda _i: st.run(), 8)
            us_p = gs.time_ms_median(5)[0] * 1e3  # (median of 5 replays of 8 runs)
            if st.gave_up():
                raise SystemExit("decode stack: a dependency wait gave up")
            # bit-exact against one call per op, in list order (a chained
            # op's input is the launch's own output of the op before it)
            for ws_, x_, ys_, _d in ops:
                ref = [torch.empty_like(y) for y in ys_]
                if len(ws_) == 1:
                    xtern.linear_f32(ws_[0], x_, out=ref[0])
                else:
                    xtern.linear_multi_f32(ws_, x_, outs=ref)
                for a_, b_ in zip(ys_, ref):
                    if not torch.isfinite(a_).all():
                        raise SystemExit(f"stack ({tag}): non-finite outputs")
                    if not torch.equal(a_, b_):
                        raise SystemExit(f"stack ({tag}) output differs from the per-call output")
            row.update({f"{tag}_us_per_stack": round(us_p, 1),
                        f"{tag}_weight_GBs": round(wbytes / (us_p * 1e-6) / 1e9, 1),
                        f"{tag}_hbm_frac": round(wbytes / (us_p * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        f"{tag}_TOPS": round(ops1 * M / (us_p * 1e-6) / 1e12, 2)})
            del gs, st
        row["persistent_checked"] = "bit-exact vs per-call outputs (every dependency shape and plan)"
        res.append(row)
        del outs, xo, xdl
        torch.cuda.empty_cache()
    del W
    torch.cuda.empty_cache()
    return res


def lm_head(np, torch, xtern, rng, Ms=(1, 16)):
    """The BitNet-2B LM head (128256 x 2560) as the reference's Int8Linear /
    Int4Linear (dynamic_linear.rs:180-535): µs per call given i8 rows
    (product) and f32 rows (forward), HBM GB/s of the weight bytes; weights
    rotate over > 2x the MALL.  Not a BASELINE config."""
    N, K = 128256, 2560
    res = []
    for fmt, name, nb in ((xtern.XT_INT8, "lm_head_int8", N * K), (xtern.XT_INT4, "lm_head_int4", N * K // 2)):
        hb = rng.integers(0, 256, nb, dtype=np.uint8)
        ws = rng.uniform(0.5, 1.5, N).astype(np.float32)
        copies = make_copies(np, xtern, fmt, K, N, hb, ws, 2 * MALL_BYTES)
        for M in Ms:
            us_q, us_f = time_product(np, torch, xtern, copies, K, N, M, rng, reps=40)
            alg = nb + 4 * N + M * K + 4 * M + 4 * M * N
            gbs = alg / (us_q * 1e-6) / 1e9
            res.append({"workload": name, "K": K, "N": N, "M": M, "us_product": round(us_q, 2),
                        "us_forward_f32": round(us_f, 2), "GBs": round(gbs, 1),
                        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
        del copies
        torch.cuda.empty_cache()
    return res


def stack_c2_pack5(np, torch, xtern, rng, Ms=(1, 4, 8), layers=26):
    """The Pack5 weights of BASELINE config 2 (BitNet-3B shapes, P(0) = 0.4)
    as a decode stack: 26 layers x {q, k, v, o, gate, up, down} (548 MB of
    distinct device weights, > 2x the MALL), residual dependency only (as
    stack_c4's residual_only), one launch, against one library call per op;
    every output checked bit-exact against the per-call one.  Not a BASELINE
    metric: it shows the Pack5 format streaming through the one-launch plan."""
    shapes = {"q": (3200, 3200), "k": (3200, 320), "v": (3200, 320), "o": (3200, 3200),
              "gate": (3200, 8640), "up": (3200, 8640), "down": (8640, 3200)}
    proto = {n: tern_bytes(np, rng, N, K, xtern.XT_PACK5, p0=0.4)[0] for n, (K, N) in shapes.items()}
    W = [{n: xtern.DeviceWeights(xtern.XT_PACK5, K, N, proto[n],
                                 np.full(N, 1.0 / np.sqrt(0.6 * K), np.float32))
          for n, (K, N) in shapes.items()} for _ in range(layers)]
    wbytes = sum(w.device_bytes() for L in W for w in L.values())
    res = []
    for M in Ms:
        f32 = torch.float32
        xa = torch.from_numpy(rng.standard_normal((M, 3200)).astype(np.float32)).cuda()
        xo = [torch.from_numpy(rng.standard_normal((M, 3200)).astype(np.float32)).cuda() for _ in range(layers)]
        xd = [torch.from_numpy(rng.standard_normal((M, 8640)).astype(np.float32)).cuda() for _ in range(layers)]
        outs = [{n: torch.empty((M, N), dtype=f32, device="cuda") for n, (K, N) in shapes.items()}
                for _ in range(layers)]
        ops = []
        h, dep = xa, None
        for L in range(layers):
            w, o = W[L], outs[L]
            ops.append(([w["down"]], xd[L], [o["down"]], None))
            dn = len(ops) - 1
            ops.append(([w["q"], w["k"], w["v"]], h, [o["q"], o["k"], o["v"]], dep))
            ops.append(([w["o"]], xo[L], [o["o"]], None))
            ops.append(([w["gate"], w["up"]], h, [o["gate"], o["up"]], dep))
            h, dep = o["down"], dn

        def per_call(_i):
            for ws_, x_, ys_, _d in ops:
                if len(ws_) == 1:
                    xtern.linear_f32(ws_[0], x_, out=ys_[0])
                else:
                    xtern.linear_multi_f32(ws_, x_, outs=ys_)
        g = Graph(torch, per_call, 1)
        us_call = g.time_ms(5) * 1e3
        del g
        st = xtern.Stack(ops, M)
        gs = Graph(torch, lambda _i: st.run(), 8)
        us = gs.time_ms_median(5)[0] * 1e3
        if st.gave_up():
            raise SystemExit("pack5 stack: a dependency wait gave up")
        for ws_, x_, ys_, _d in ops:
            ref = [torch.empty_like(y) for y in ys_]
            if len(ws_) == 1:
                xtern.linear_f32(ws_[0], x_, out=ref[0])
            else:
                xtern.linear_multi_f32(ws_, x_, outs=ref)
            for a_, b_ in zip(ys_, ref):
                if not torch.isfinite(a_).all() or not torch.equal(a_, b_):
                    raise SystemExit("pack5 stack output differs from the per-call output")
        res.append({"workload": "c2_pack5_projection_stack_bitnet3b", "M": M, "layers": layers,
                    "weight_bytes": wbytes, "plan": st.plan_name,
                    "us_per_stack_per_call": round(us_call, 1),
                    "us_per_stack": round(us, 1),
                    "weight_GBs": round(wbytes / (us * 1e-6) / 1e9, 1),
                    "hbm_frac": round(wbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "checked": "bit-exact vs per-call outputs",
                    "timing": "median of 5 graph replays of 8 back-to-back runs"})
        del gs, st, outs, xo, xd
        torch.cuda.empty_cache()
    del W
    torch.cuda.empty_cache()
    return res


def mlp_block_c4(np, torch, xtern, rng, Ms=(1, 8), layers=30):
    """The BitNet-2B MLP block of the decode step as the reference's
    fused_mlp_all runs it (layers.rs:497-645): gate+up on one quantised input,
    ReLU^2(gate) * up, ffn_sub_norm (RMSNorm, exact sequential sum of
    squares), requantisation, down -- 30 layers of distinct weights (398 MB,
    > the MALL), independent inputs per layer, one HIP graph per pass.  Not a
    BASELINE config (configs[4] times the linear layers alone); reported so
    the middle stage is measured too."""
    proto = {n: tern_bytes(np, rng, N, K, xtern.XT_PACK4)[0]
             for n, (K, N) in (("gate", (2560, 6912)), ("up", (2560, 6912)), ("down", (6912, 2560)))}
    L = []
    for _ in range(layers):
        L.append({n: xtern.DeviceWeights(xtern.XT_PACK4, K, N, proto[n], np.full(N, 0.05, np.float32))
                  for n, (K, N) in (("gate", (2560, 6912)), ("up", (2560, 6912)), ("down", (6912, 2560)))})
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, 6912).astype(np.float32)).cuda()
    wbytes = layers * 3 * 6912 * 2560 // 4
    res = []
    for M in Ms:
        x = torch.from_numpy(rng.standard_normal((M, 2560)).astype(np.float32)).cuda()
        y = torch.empty((M, 2560), dtype=torch.float32, device="cuda")

        def run(_i):
            for w in L:
                xtern.mlp_f32(w["gate"], w["up"], w["down"], x, norm_w=nw, out=y)
        g = Graph(torch, run, 1)
        us = g.time_ms(10) * 1e3
        res.append({"workload": "c4_mlp_block_subnorm", "M": M, "layers": layers,
                    "us_per_mlp": round(us / layers, 2),
                    "weight_GBs": round(wbytes / (us * 1e-6) / 1e9, 1)})
    del L
    torch.cuda.empty_cache()
    return res


def host_cpu_info():
    """CPU model, logical CPUs usable by this process, physical cores (unique
    (package, core id) pairs of /proc/cpuinfo)."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    try:
        logical = len(os.sched_getaffinity(0))
    except AttributeError:
        logical = os.cpu_count() or 1
    return {"model": model, "logical": logical, "physical_cores_host": len(cores) or None}


def cpu_baseline(np, wl, rng, budget_s=6.0):
    """The oracle's restatement of the reference CPU path (TernaryLinear::forward
    with the AVX-512 VNNI dot when the host has it, else the scalar dot) on
    the host cores of the GPU box, in the same run:
      c1  16-token samples of each C1 matrix, one task per token
          (layers.rs:298-310), repeated for ~budget_s;
      c0  the M = 1 GEMV (K=2560, N=6912) with the reference's row chunks of
          max(ceil(N/T), 128) rows (layers.rs:284-296), repeated for ~budget_s/2;
    each at T = min(nproc, 8) (the reference default, lib.rs:32-42) and at
    every usable logical CPU (capped by OMP_NUM_THREADS when set)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    info = host_cpu_info()
    default_t = min(info["logical"], 8)
    all_t = info["logical"]
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        all_t = min(all_t, int(os.environ["OMP_NUM_THREADS"]))
    kernel = 1 if oracle.has_vnni() else 0
    isa = "avx512-vnni" if kernel else "scalar"

    def c1(threads):
        rows, ops, t_total, reps = 16, 0, 0.0, 0
        while t_total < budget_s:
            for s in wl["sets"]:
                t0 = time.perf_counter()
                oracle.linear_forward(0, s["K"], s["N"], s["xh"][:rows], s["ws"], wbytes=s["wb"],
                                      threads=threads, kernel=kernel)
                t_total += time.perf_counter() - t0
                ops += 2 * rows * s["N"] * s["K"]
            reps += 1
        return ops / t_total / 1e12, reps, t_total

    K, N = 2560, 6912
    wb0, _ = tern_bytes(np, rng, N, K, 0)
    ws0 = np.full(N, 0.8, np.float32)
    x0 = rng.standard_normal((1, K)).astype(np.float32)
    alg0 = N * K // 4 + 4 * K + 4 * N + 4 * N

    def c0(threads):
        times = []
        t_total = 0.0
        while t_total < budget_s / 2 or len(times) < 50:
            t0 = time.perf_counter()
            oracle.linear_forward(0, K, N, x0, ws0, wbytes=wb0, threads=threads, kernel=kernel)
            dt = time.perf_counter() - t0
            times.append(dt)
            t_total += dt
        med = float(np.median(times))
        return med * 1e6, alg0 / med / 1e9, len(times)

    variants = []
    for T in sorted({default_t, all_t}):
        tops, reps, tt = c1(T)
        us0, gbs0, n0 = c0(T)
        variants.append({"threads": T, "c1_TOPS": round(tops, 5),
                         "c1_sample": f"{reps} passes x 16 tokens of each c1 matrix ({tt:.1f} s)",
                         "c0_us_per_call_median": round(us0, 1), "c0_GBs": round(gbs0, 2),
                         "c0_calls": n0})
    head = next(v for v in variants if v["threads"] == default_t)
    return {"value": head["c1_TOPS"], "unit": "TOPS (int8)", "cores": default_t, "kind": "port",
            "sample": head["c1_sample"] + f", isa={isa}", "isa": isa,
            "cpu_model": info["model"], "logical_cpus": info["logical"],
            "physical_cores_host": info["physical_cores_host"], "variants": variants}


def recorded_traffic():
    """HBM bytes per product launch (FETCH_SIZE + WRITE_SIZE, calibrated)
    from the committed rocprofv3 summary, or None."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic_c1.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                kv = dict(t.split("=") for t in line.split(":", 1)[1].split())
                return {k: int(v) for k, v in kv.items()}
    except OSError:
        pass
    return None


def copy_calibration(torch):
    """A plain device copy of known size, for scaling rocprof FETCH/WRITE_SIZE."""
    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "launches": 3}))


def peaks(torch):
    """On-box ceilings (libxtern_diag.so): a streaming read of 1 GiB (HBM
    bound, 4x the MALL), single-launch reads of 4.4 MB (the C0 weight bytes)
    over rotating buffers > 2x the MALL, launch to launch in a HIP graph, the
    i8 MFMA rate of back-to-back 32x32x32 and 16x16x64 instructions, and the
    launch-to-launch floor of an empty kernel.  HIP events on the launch
    stream; one JSON line."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "xor-net_amd", "xtern", "libxtern_diag.so"))
    vp = ctypes.c_void_p
    lib.xtd_read.argtypes = [vp, ctypes.c_size_t, ctypes.c_int, vp, vp]
    lib.xtd_mfma_i8.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
    lib.xtd_empty.argtypes = [ctypes.c_int, ctypes.c_int, vp]
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    res = {}

    def graph_ms(fn, n, replays=3):
        g = Graph(torch, fn, n)
        return g.time_ms(replays)

    def sp():
        return vp(torch.cuda.current_stream().cuda_stream)

    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(3)
    for blocks in (1024, 2048, 4096):
        ms = graph_ms(lambda i: lib.xtd_read(vp(big.data_ptr()), big.numel(), blocks,
                                             vp(sink.data_ptr()), sp()), 4)
        res[f"read_1GiB_blocks{blocks}_GBs"] = round(big.numel() / (ms * 1e-3) / 1e9, 1)
    del big
    torch.cuda.empty_cache()
    nb = 4481536  # C0's weight bytes rounded to 16
    copies = [torch.empty(nb, dtype=torch.uint8, device="cuda").fill_(i & 255)
              for i in range(-(-2 * MALL_BYTES // nb))]
    for blocks in (256, 512, 1088):
        ms = graph_ms(lambda i: lib.xtd_read(vp(copies[i].data_ptr()), nb, blocks,
                                             vp(sink.data_ptr()), sp()), len(copies))
        res[f"read_4.4MB_blocks{blocks}_us"] = round(ms * 1e3, 3)
        res[f"read_4.4MB_blocks{blocks}_GBs"] = round(nb / (ms * 1e-3) / 1e9, 1)
    del copies
    torch.cuda.empty_cache()
    for shape, ops_per in ((32, 65536), (16, 32768)):
        blocks, iters = 2048, 1000
        ms = graph_ms(lambda i: lib.xtd_mfma_i8(shape, blocks, iters, vp(sink.data_ptr()), sp()), 2)
        tops = blocks * 4 * 4 * iters * ops_per / (ms * 1e-3) / 1e12
        res[f"mfma_i8_{shape}_TOPS"] = round(tops, 1)
    for blocks in (1, 256, 1024):
        ms = graph_ms(lambda i: lib.xtd_empty(blocks, 256, sp()), 200)
        res[f"empty_kernel_grid{blocks}_us"] = round(ms * 1e3, 3)
    print(json.dumps({"peaks": res}))


def vendor_int8(np, torch, xtern, rng):
    """Reference point, not the product: the ROCm library's dense int8 GEMM
    (torch._int_mm, i8 weights -- 4x the bytes of Pack4) on the C1 and short
    prefill shapes, beside this library's Pack4 product on the same shapes;
    both over rotating weight copies (> 2x the MALL) in HIP graphs."""
    rows = []
    for M, K, N in ((128, 2560, 6912), (128, 6912, 2560), (32, 2560, 2560), (32, 2560, 6912)):
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda")
        n = max(2, -(-2 * MALL_BYTES // (K * N)))
        bs = [torch.randint(-1, 2, (N, K), dtype=torch.int8, device="cuda").t() for _ in range(n)]
        g = Graph(torch, lambda i: torch._int_mm(a, bs[i]), n)
        us_lib = g.time_ms(max(1, 100 // n)) * 1e3
        del g, bs
        torch.cuda.empty_cache()
        wb, _ = tern_bytes(np, rng, N, K, xtern.XT_PACK4)
        copies = make_copies(np, xtern, xtern.XT_PACK4, K, N, wb, np.ones(N, np.float32), 2 * MALL_BYTES)
        us_q, _ = time_product(np, torch, xtern, copies, K, N, M, rng, reps=100)
        del copies
        torch.cuda.empty_cache()
        rows.append({"M": M, "K": K, "N": N, "us_int_mm_i8": round(us_lib, 2),
                     "us_xtern_pack4": round(us_q, 2),
                     "TOPS_int_mm": round(2 * M * K * N / us_lib / 1e6, 1),
                     "TOPS_xtern": round(2 * M * K * N / us_q / 1e6, 1)})
    print(json.dumps({"vendor_int8_gemm": rows}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c1")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--peaks", action="store_true",
                    help="measure the on-box read / MFMA / launch ceilings and exit")
    ap.add_argument("--vendor-int8", action="store_true",
                    help="time the ROCm dense int8 GEMM beside the Pack4 product and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import xtern

    if args.copy_calibration:
        copy_calibration(torch)
        return
    if args.peaks:
        peaks(torch)
        return
    rng = np.random.default_rng(1234)
    if args.vendor_int8:
        vendor_int8(np, torch, xtern, rng)
        return
    if args.workload == "c0":
        print(json.dumps({"gemv_m1": gemv_m1(np, torch, xtern, rng)}))
        return
    if args.workload == "c0s":
        print(json.dumps({"c0_sustained": gemv_sustained(np, torch, xtern, rng)}))
        return
    if args.workload == "c4":
        print(json.dumps({"c4": stack_c4(np, torch, xtern, rng)}))
        return
    if args.workload == "c2s":
        print(json.dumps({"c2_stack": stack_c2_pack5(np, torch, xtern, rng)}))
        return
    if args.workload == "c3":
        print(json.dumps({"c3": gemv_configs(np, torch, xtern, rng, only="c3")}))
        return
    if args.workload != "c1":
        raise SystemExit("workloads: c1 (the headline step), c0 (the M=1 GEMV alone), c0s (the "
                         "C0 GEMV sustained over 121 matrices), c2s (the Pack5 BitNet-3B stack), "
                         "c3 (XorSparse: tiles and compact stream), c4 (stack)")
    log("setting up c1 weights (rotating copies) ...")
    wl = workload_c1(np, torch, xtern, rng)

    # eager reference outputs, then the timed graph of exactly `steps` steps
    run_steps(xtern, wl, 1)
    torch.cuda.synchronize()
    ms_step, steps_timed = time_exact_steps(torch, xtern, wl, args.steps, args.warmup)
    tops = wl["ops"] / (ms_step * 1e-3) / 1e12
    log(f"step {ms_step * 1e3:.2f} us over {steps_timed} steps")

    prod_ms = product_only(np, torch, xtern, wl, reps=max(args.steps, 50))
    prod_ops = [2 * wl["M"] * s["N"] * s["K"] for s in wl["sets"]]
    ach = sum(prod_ops) / (sum(prod_ms) * 1e-3) / 1e12
    tr = recorded_traffic()
    prod_tr = {k: v for k, v in (tr or {}).items() if k in ("gemm32s_up", "mm_down")}
    roof = {"bound": "mfma", "achieved": round(ach, 2), "peak": INT8_PEAK_TOPS,
            "unit": "TOPS", "frac": round(ach / INT8_PEAK_TOPS, 4),
            "traffic": (sum(prod_tr.values()) // len(prod_tr)) if prod_tr else None,
            "traffic_per_launch": prod_tr or None,
            "traffic_source": "profiles/pmc_traffic_c1.md (rocprofv3 --pmc FETCH_SIZE, "
                              "WRITE_SIZE of the same kernels, copy-calibrated; not measured "
                              "in this run)",
            "kernel": "product launches (gemm32s_kernel up, mm_kernel down)",
            "us_per_launch": {s["name"]: round(m * 1e3, 3) for s, m in zip(wl["sets"], prod_ms)}}

    out = {"metric": "ternary GEMM int8 TOPS at M=128 (Pack4, BitNet-2B up+down)",
           "value": round(tops, 3), "unit": "TOPS", "n_gpus": 1, "steps": steps_timed,
           "warmup": args.warmup, "ms_per_step": round(ms_step, 6), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "i8 x ternary -> i32, f32 io",
           "data": "synthetic (seeded ternary weights P(0)=0.35, N(0,1) activations, 1% x20)",
           "config": wl["config"], "roofline": roof}
    if not args.no_extra:
        log("c0 gemv ...")
        out["gemv_m1"] = gemv_m1(np, torch, xtern, rng)
        log("c0 sustained ...")
        out["gemv_m1_sustained"] = gemv_sustained(np, torch, xtern, rng)
        log("c2 / c3 gemv ...")
        out["configs"] = gemv_configs(np, torch, xtern, rng)
        log("c4 stack ...")
        out["configs"] += stack_c4(np, torch, xtern, rng)
        log("c2 pack5 stack ...")
        out["configs"] += stack_c2_pack5(np, torch, xtern, rng)
        log("c4 mlp block ...")
        out["configs"] += mlp_block_c4(np, torch, xtern, rng)
        log("lm head ...")
        out["configs"] += lm_head(np, torch, xtern, rng)
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(np, wl, rng)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
