"""Benchmark of the torch_spyre MI355X hot path (one JSON line on stdout).

Headline (BASELINE.json metric, configs[1]): fp16 GEMM C = A @ B with
M = N = K = 4096, A, B ~ U(-1, 1) from seed 0xAFFE, fp32 accumulate, on one
MI355X.  A step is one GEMM over resident HBM inputs.  Secondary figures for
the other hot-path kernels (config 1 softmax, config 2 bmm, config 3 norms and
GELU chain) are reported under "extra", each against its roofline.

Kernel durations are taken with HIP events on the stream the kernels run on;
the CPU baseline times the oracle (numpy, CPU) on a bounded slice of the same
workload on this host's cores.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "torch-spyre_amd"))
sys.path.insert(0, os.path.join(REPO, "tests"))
sys.path.insert(0, REPO)

PEAK_FP16_TFLOPS = 2516.6   # MI355X dense fp16 MFMA (256 CU x 4096 FLOP/clk x 2.4 GHz)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SEED = 0xAFFE
# Warmup launches of each secondary figure (the part's clock settles after
# ~35 ms of sustained load; 300 launches of the shortest kernel cover that
# only together with the ones before it).
SUB_WARMUP = 300
# untimed launches of the headline GEMM before its warmup (steady clock)
PRECONDITION_MS = 100.0


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _gen(k):
    import torch

    return torch.Generator().manual_seed(SEED + k)


class Timer:
    """HIP-event timing of `fn` launched `steps` times on `stream`."""

    def __init__(self, stream):
        import torch

        self.torch = torch
        self.stream = stream

    def run(self, fn, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(self.stream)
        for _ in range(steps):
            fn()
        end.record(self.stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        return start.elapsed_time(end) / steps, wall


def graph_us(launch, reps, per_graph=20):
    """Average GPU time per launch of `launch(stream_handle)` captured
    `per_graph` times into one HIP graph and replayed `reps` times (events on
    the capture stream)."""
    import torch

    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        launch(cs.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for _ in range(per_graph):
            launch(cs.cuda_stream)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(cs):  # replay() launches on the current stream
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        start.record(cs)
        for _ in range(reps):
            g.replay()
        end.record(cs)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (reps * per_graph)


# Symbols of the kernels bench.py times, by the key of their figure.  A
# traffic measurement in profiles/traffic.json counts only for the kernel it
# was taken of: entries are keyed by symbol, so a changed kernel reports no
# traffic until it is measured again.
TIMED_SYMBOLS = {
    "gemm": "_ZN3sph12_GLOBAL__N_114gemm_dl_kernelIDF16_Lb0ELi256ELb0ELi64EEEvNS0_8GemmArgsE",
    "bmm": "_ZN3sph12_GLOBAL__N_123gemm_shortk_ring_kernelIDF16_Lb0ELi2ELi2ELi2EEEvNS0_8GemmArgsE",
    "softmax": "_ZN3sph12_GLOBAL__N_112softmax_fullIDF16_DF16_Li128ELi4EEEvPKT_lPT0_llfill",
    "rmsnorm": "_ZN3sph12_GLOBAL__N_19norm_regsIDF16_DF16_Li256ELi2ELb1ELb0EEEvPKT_S4_PKT0_S7_PS2_"
               "S8_PfS9_llf",
    "layernorm": "_ZN3sph12_GLOBAL__N_19norm_regsIDF16_DF16_Li256ELi2ELb1ELb1EEEvPKT_S4_PKT0_S7_"
                 "PS2_S8_PfS9_llf",
    "gelu_rowsum": "_ZN3sph12_GLOBAL__N_116gelu_rowsum_rowsIDF16_Li512ELi1ELi2ELb1EEEvPKT_S4_S4_"
                   "ffPS2_S5_l",
}
# The calibration kernel (bench.py --kernel copy: 512 MiB read, 512 MiB written).
COPY_SYMBOL = "_ZN3sph12_GLOBAL__N_16pw_vecIDF16_EEvNS0_6PwArgsE"
COPY_BYTES = 512 * 1024 * 1024
# Algorithmic bytes per launch of each timed kernel (operands read once,
# results written once).
ALGORITHMIC_BYTES = {
    "gemm": 3 * 4096 * 4096 * 2,
    "bmm": (2 * 32 * 2048 * 128 + 32 * 2048 * 2048) * 2,
    "softmax": 2 * 512 * 4096 * 2,
    "rmsnorm": 4 * 8192 * 4096 * 2 + 4096 * 2,
    "layernorm": 4 * 8192 * 4096 * 2 + 2 * 4096 * 2,
    "gelu_rowsum": 2 * 8192 * 4096 * 2 + 2 * 4096 * 2 + 8192 * 2,
}
TRAFFIC_JSON = os.path.join(REPO, "profiles", "traffic.json")


def _traffic_for(key):
    """HBM bytes per launch of the kernel timed under `key`, measured by
    rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, each scaled by what the counter
    reads for a plain copy of known size), committed in profiles/traffic.json
    under the kernel's symbol; None when that kernel has not been measured."""
    try:
        with open(TRAFFIC_JSON) as f:
            entry = json.load(f).get("kernels", {}).get(TIMED_SYMBOLS[key])
    except (OSError, ValueError):
        return None
    return None if entry is None else entry.get("bytes_per_launch")


def summarize_traffic(root, algorithmic):
    """Reads rocprofv3 --pmc outputs under `root` (directories pmc_<part>_
    <COUNTER>/ holding p_counter_collection.csv, one counter per pass) and
    writes profiles/traffic.json: per timed kernel symbol the median
    FETCH_SIZE / WRITE_SIZE (KiB per dispatch), both scaled by the copy
    kernel's calibration."""
    import csv
    import glob
    import statistics

    vals = {}
    for d in glob.glob(os.path.join(root, "pmc_*_*_SIZE")):
        counter = "FETCH_SIZE" if d.endswith("FETCH_SIZE") else "WRITE_SIZE"
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for row in csv.DictReader(f):
                    vals.setdefault((row["Kernel_Name"], counter), []).append(
                        float(row["Counter_Value"]))

    def med(sym, counter):
        v = vals.get((sym, counter))
        return statistics.median(v) if v else None

    cf, cw = med(COPY_SYMBOL, "FETCH_SIZE"), med(COPY_SYMBOL, "WRITE_SIZE")
    if not cf or not cw:
        raise SystemExit(f"no copy calibration ({COPY_SYMBOL}) under {root}")
    ff, fw = COPY_BYTES / (cf * 1024), COPY_BYTES / (cw * 1024)
    out = {"copy_calibration": {"kernel": COPY_SYMBOL, "bytes_read": COPY_BYTES,
                                "bytes_written": COPY_BYTES, "fetch_kib_raw": cf,
                                "write_kib_raw": cw, "fetch_factor": round(ff, 5),
                                "write_factor": round(fw, 5)},
           "kernels": {}}
    for key, sym in TIMED_SYMBOLS.items():
        f, w = med(sym, "FETCH_SIZE"), med(sym, "WRITE_SIZE")
        if f is None or w is None:
            continue
        out["kernels"][sym] = {"key": key, "fetch_kib_raw": f, "write_kib_raw": w,
                               "bytes_per_launch": int(f * 1024 * ff + w * 1024 * fw),
                               "algorithmic_bytes": algorithmic.get(key)}
    with open(TRAFFIC_JSON, "w") as fh:
        json.dump(out, fh, indent=1)
        fh.write("\n")
    return out


def bench_gemm(steps, warmup, stream, capi):
    import torch

    M = N = K = 4096
    a = (torch.rand(M, K, generator=_gen(0)) * 2 - 1).half().cuda()
    b = (torch.rand(K, N, generator=_gen(1)) * 2 - 1).half().cuda()
    d = torch.empty(M, N, dtype=torch.float16, device="cuda")
    s = stream.cuda_stream
    lib = capi.lib()

    def step():
        rc = lib.sph_gemm_f16(M, N, K, a.data_ptr(), b.data_ptr(), d.data_ptr(), s)
        if rc:
            capi.check(rc, "sph_gemm_f16")

    # Preconditioning: the part lowers its clock under this MFMA + LDS load
    # (power-limited) and needs ~35 ms of it to settle; launches before that
    # measure the clock's transition, not the kernel (4096^3: 989 TFLOP/s
    # after 10 launches, 1165 after 100, 1207-1212 after 300 or 1000).  So
    # the kernel runs PRECONDITION_MS of untimed launches first; then come
    # exactly `warmup` untimed and `steps` timed launches.
    n_pre = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < PRECONDITION_MS:
        for _ in range(50):
            step()
        n_pre += 50
        torch.cuda.synchronize()
    kernel_ms, wall_ms = Timer(stream).run(step, steps, warmup)
    flop = 2.0 * M * N * K
    return {"kernel_ms": kernel_ms, "wall_ms": wall_ms, "flop": flop,
            "tflops": flop / (kernel_ms * 1e-3) / 1e12, "a": a, "b": b, "d": d,
            "precondition_launches": n_pre}


def bench_gemm_cold(steps, warmup, stream, capi, sets=8):
    """GEMMs whose operands come from HBM: `sets` operand sets used in turn
    (c2 4096^3 A @ B: 8 x 64 MiB of A and B, more than the 256 MiB MALL;
    c4's QKV projection x W^T, 2048 x 6144 x 4096: 8 x 64 MiB), so a launch
    finds none of its operands in the caches, as a projection inside a
    decoder layer does.  HIP events over launches that rotate the sets."""
    import torch

    lib = capi.lib()
    s = stream.cuda_stream
    timer = Timer(stream)
    out = {}
    for name, M, N, K, tb in (("c2_mm_4096_cold", 4096, 4096, 4096, 0),
                              ("c4_qkv_2048x6144x4096_cold", 2048, 6144, 4096, 1)):
        A = [(torch.rand(M, K, generator=_gen(20 + i)) * 2 - 1).half().cuda() for i in range(sets)]
        B = [(torch.rand((N, K) if tb else (K, N), generator=_gen(40 + i)) * 2 - 1).half().cuda()
             for i in range(sets)]
        D = [torch.empty(M, N, dtype=torch.float16, device="cuda") for _ in range(sets)]
        ldb = K if tb else N
        it = [0]

        def step():
            i = it[0] % sets
            it[0] += 1
            rc = lib.sph_gemm(capi.F16, 0, tb, M, N, K, 1.0, A[i].data_ptr(), K, B[i].data_ptr(),
                              ldb, 0.0, None, 0, 0, D[i].data_ptr(), N, 0, s)
            if rc:
                capi.check(rc, "sph_gemm")

        ms, _ = timer.run(step, max(steps, 2 * sets), max(warmup, 4 * sets))
        flop = 2.0 * M * N * K
        out[name] = {"us_per_launch": round(ms * 1e3, 2),
                     "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 1),
                     "roofline_frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
                     "bound": "mfma", "operand_sets": sets}
        del A, B, D
    return out


def bench_gemm_bf16(steps, warmup, stream, capi):
    """c2's 4096^3 A @ B (both row-major) in bf16 through sph_gemm, HIP events
    after the fp16 headline's warmup count; a sample of rows must agree with
    torch's fp32 product of the same bf16 operands within 2e-2."""
    import torch

    lib = capi.lib()
    s = stream.cuda_stream
    M = N = K = 4096
    a = (torch.rand(M, K, generator=_gen(80)) * 2 - 1).to(torch.bfloat16).cuda()
    b = (torch.rand(K, N, generator=_gen(81)) * 2 - 1).to(torch.bfloat16).cuda()
    d = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")

    def step():
        rc = lib.sph_gemm(capi.BF16, 0, 0, M, N, K, 1.0, a.data_ptr(), K, b.data_ptr(), N, 0.0,
                          None, 0, 0, d.data_ptr(), N, 0, s)
        if rc:
            capi.check(rc, "sph_gemm")

    ms, _ = Timer(stream).run(step, max(steps, 20), max(warmup, 300))
    rows = torch.arange(0, M, 256, device="cuda")
    ref = a.index_select(0, rows).float() @ b.float()
    torch.testing.assert_close(d.index_select(0, rows).float(), ref, rtol=2e-2, atol=2e-2)
    flop = 2.0 * M * N * K
    tf = flop / (ms * 1e-3) / 1e12
    return {"c2_mm_4096_bf16": {"us_per_launch": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                                "roofline_frac": round(tf / PEAK_FP16_TFLOPS, 4), "bound": "mfma",
                                "note": "bf16 operands and output, fp32 accumulate; "
                                        "dense bf16 MFMA peak = the fp16 one"}}


def bench_extra(steps, warmup, stream, capi):
    """Secondary kernels: bytes / FLOPs per launch and roofline fractions."""
    out = bench_rows(steps, warmup, stream, capi)
    out.update(bench_bmm(steps, warmup, stream, capi))
    return out


def bench_rows(steps, warmup, stream, capi):
    """c1 softmax and the c3 row kernels through the C-ABI."""
    import torch

    s = stream.cuda_stream
    lib = capi.lib()
    out = {}
    timer = Timer(stream)

    def hbm_entry(name, key, nbytes, fn):
        ms, _ = timer.run(fn, steps, warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_launch": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
                     "GB/s": round(gbs, 1), "roofline_frac": round(gbs / PEAK_HBM_GBS, 4),
                     "bound": "hbm", "traffic": _traffic_for(key)}

    # c1 softmax [512, 4096] fp16, N(0,1)*4.  Cold-cache variant rotates 80
    # input/output pairs (640 MiB > MALL) so each launch reads from HBM.
    R, C = 512, 4096
    x = (torch.randn(R, C, generator=_gen(0)) * 4).half().cuda()
    y = torch.empty_like(x)
    # launched from Python through ctypes: the host's ~4 us per call, not the
    # kernel, sets this one (the graph-replayed figure below is the GPU's)
    hbm_entry("c1_softmax_512x4096_hot_python_launches", "softmax", 2 * R * C * 2,
              lambda: lib.sph_softmax_rows_f16(x.data_ptr(), y.data_ptr(), R, C, s))
    xs = [x.clone() for _ in range(80)]
    ys = [torch.empty_like(x) for _ in range(80)]
    it = [0]

    def cold_softmax(hs):
        i = it[0] = (it[0] + 1) % 80
        lib.sph_softmax_rows_f16(xs[i].data_ptr(), ys[i].data_ptr(), R, C, hs)

    # cold: one graph of 80 launches over 80 input/output pairs (640 MiB, more
    # than the 256 MiB MALL), so each launch reads from HBM
    us = graph_us(cold_softmax, max(steps // 4, 5), per_graph=80)
    gbs = 2 * R * C * 2 / (us * 1e-6) / 1e9
    out["c1_softmax_512x4096_cold"] = {
        "us_per_launch": round(us, 2), "algorithmic_bytes": 2 * R * C * 2, "GB/s": round(gbs, 1),
        "roofline_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
        "note": "80 launches over 80 buffer pairs per HIP graph replay"}
    del xs, ys
    # The same kernel launched from a captured HIP graph (20 launches per
    # replay): per-launch GPU time without the Python/ctypes call between
    # launches, which is longer than this kernel.  The replayed output is
    # checked against an eager launch.
    ref = torch.empty_like(x)
    lib.sph_softmax_rows_f16(x.data_ptr(), ref.data_ptr(), R, C, s)
    us = graph_us(lambda hs: lib.sph_softmax_rows_f16(x.data_ptr(), y.data_ptr(), R, C, hs),
                  max(steps, 50))
    assert torch.equal(y, ref), "graph-replayed softmax differs from the eager launch"
    gbs = 2 * R * C * 2 / (us * 1e-6) / 1e9
    out["c1_softmax_512x4096_hot"] = {
        "us_per_launch": round(us, 2), "algorithmic_bytes": 2 * R * C * 2, "GB/s": round(gbs, 1),
        "roofline_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
        "traffic": _traffic_for("softmax"),
        "note": "20 launches per HIP graph replay (GPU time per launch, back to back)"}

    # c3 residual add + RMSNorm / LayerNorm, GELU chain: [8192, 4096] fp16
    R, C = 8192, 4096
    x = torch.randn(R, C, generator=_gen(0)).half().cuda()
    r = torch.randn(R, C, generator=_gen(1)).half().cuda()
    w = (torch.randn(C, generator=_gen(2)) * 0.02 + 1).half().cuda()
    bb = (torch.randn(C, generator=_gen(3)) * 0.02).half().cuda()
    yy = torch.empty_like(x)
    h = torch.empty_like(x)
    hbm_entry("c3_add_rmsnorm_8192x4096", "rmsnorm", 4 * R * C * 2 + C * 2,
              lambda: lib.sph_rmsnorm_f16(x.data_ptr(), r.data_ptr(), w.data_ptr(),
                                          yy.data_ptr(), h.data_ptr(), R, C, 1e-5, s))
    hbm_entry("c3_add_layernorm_8192x4096", "layernorm", 4 * R * C * 2 + 2 * C * 2,
              lambda: lib.sph_layernorm_f16(x.data_ptr(), r.data_ptr(), w.data_ptr(),
                                            bb.data_ptr(), yy.data_ptr(), h.data_ptr(), R, C,
                                            1e-5, s))
    rs = torch.empty(R, dtype=torch.float16, device="cuda")
    hbm_entry("c3_gelu_affine_rowsum_8192x4096", "gelu_rowsum", 2 * R * C * 2 + 2 * C * 2 + R * 2,
              lambda: lib.sph_gelu_affine_rowsum_f16(x.data_ptr(), w.data_ptr(), bb.data_ptr(),
                                                     yy.data_ptr(), rs.data_ptr(), R, C, s))
    del x, r, yy, h
    return out


def bench_attention(steps, warmup, stream, capi):
    """c4's attention as one fused kernel (sph_attention_fwd): 8 KV heads x
    4 stacked query heads x 2048 positions, head dim 128, fp16, with c4's
    additive causal mask (block pre-pass included) and without a mask.
    MFMA-bound: 4 mq sk d FLOP per batch element dense; the causal figure
    counts the visible (lower-triangle) share."""
    import math

    import torch

    s = stream.cuda_stream
    lib = capi.lib()
    B, MQ, SK, D = 8, 8192, 2048, 128
    q = torch.randn(B, MQ, D, generator=_gen(40)).half().cuda()
    k = torch.randn(B, SK, D, generator=_gen(41)).half().cuda()
    v = torch.randn(B, SK, D, generator=_gen(42)).half().cuda()
    o = torch.empty_like(q)
    mask = torch.full((SK, SK), float("-inf")).triu(1).repeat(MQ // SK, 1).half().cuda()
    nws = lib.sph_attention_workspace_bytes(B, MQ, SK, 0)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    sc = 1 / math.sqrt(D)
    timer = Timer(stream)

    def run(mp, w):
        capi.check(lib.sph_attention_fwd(capi.F16, B, MQ, SK, D, q.data_ptr(), D, MQ * D,
                                         k.data_ptr(), D, SK * D, v.data_ptr(), D, SK * D, mp,
                                         SK if mp else 0, 0, 0, 0, sc, o.data_ptr(), D, MQ * D,
                                         w, nws if w else 0, s), "sph_attention_fwd")

    dense = 4.0 * B * MQ * SK * D
    visible = dense * (SK + 1) / (2 * SK)
    out = {}
    ms, _ = timer.run(lambda: run(mask.data_ptr(), ws.data_ptr()), steps, warmup)
    out["c4_attention_causal_mask"] = {
        "us_per_launch": round(ms * 1e3, 2), "visible_flop": visible,
        "TFLOP/s": round(visible / ms / 1e9, 1),
        "roofline_frac": round(visible / ms / 1e9 / PEAK_FP16_TFLOPS, 4), "bound": "mfma"}
    ms, _ = timer.run(lambda: run(None, None), steps, warmup)
    out["c4_attention_no_mask"] = {
        "us_per_launch": round(ms * 1e3, 2), "flop": dense, "TFLOP/s": round(dense / ms / 1e9, 1),
        "roofline_frac": round(dense / ms / 1e9 / PEAK_FP16_TFLOPS, 4), "bound": "mfma"}
    return out


def bench_decode_step(reps, stream, capi):
    """c5's fused decode-step attention (sph_decode_attention_step: RoPE,
    KV-cache append and attention over keys 0..pos, plus the merge of the
    64-key partials): batch 4, 32 query / 8 KV heads, a 1152-slot cache with
    dim-major V, position 1087 (the mean of c5's 128 steps).  16 cache
    copies (302 MB, more than the 256 MB MALL) are used in turn, so K and V
    come from HBM as in the decode step, where 16 GB of weights pass between
    two visits of a layer's cache.  Algorithmic bytes: K and V of keys
    0..pos."""
    import math

    import torch

    lib = capi.lib()
    B, H, Hkv, L, D, pos, ncopy = 4, 32, 8, 1152, 128, 1087, 16
    g = _gen(60)
    ks = [torch.randn(B, Hkv, L, D, generator=g).half().cuda() for _ in range(ncopy)]
    vs = [torch.randn(B, Hkv, D, L, generator=g).half().cuda() for _ in range(ncopy)]
    ang = torch.arange(L, dtype=torch.float32)[:, None] * \
        (1e4 ** (-torch.arange(0, D, 2, dtype=torch.float32) / D))[None, :]
    ang = torch.cat([ang, ang], -1)
    cs, sn = ang.cos().half().cuda(), ang.sin().half().cuda()
    qkv = torch.randn(B, (H + 2 * Hkv) * D, generator=g).half().cuda()
    nws = lib.sph_decode_attention_step_workspace_bytes(B, H, Hkv, L)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty(B, H * D, dtype=torch.float16, device="cuda")
    pd = torch.tensor([pos], dtype=torch.int64, device="cuda")
    turn = [0]

    def launch(st):
        kc, vc = ks[turn[0] % ncopy], vs[turn[0] % ncopy]
        turn[0] += 1
        capi.check(lib.sph_decode_attention_step(
            capi.F16, B, H, Hkv, D, qkv.data_ptr(), qkv.stride(0), cs.data_ptr(), sn.data_ptr(),
            cs.stride(0), pd.data_ptr(), err.data_ptr(), kc.data_ptr(), kc.stride(0),
            kc.stride(1), kc.stride(2), vc.data_ptr(), vc.stride(0), vc.stride(1), 1,
            vc.stride(2), L, 1.0 / math.sqrt(D), out.data_ptr(), out.stride(0), ws.data_ptr(),
            nws, st), "sph_decode_attention_step")

    us = graph_us(launch, reps, per_graph=ncopy)
    torch.cuda.synchronize()
    assert int(err.cpu()[0]) == 0
    nbytes = 2 * B * Hkv * (pos + 1) * D * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"c5_decode_attention_step": {
        "us_per_call": round(us, 2), "algorithmic_bytes": nbytes, "GB/s": round(gbs, 1),
        "roofline_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
        "note": "step kernel + merge kernel back to back in a HIP graph, K/V from HBM"}}


def bench_launch_floor(reps, capi):
    """What a small kernel costs back to back in one HIP graph (GPU time per
    launch): torch's fill of one element (the dispatch floor), torch's copy
    of 4 MiB into 4 MiB (the 8 MiB that c1's softmax reads and writes, at
    the same launch count) and the c1 softmax itself through the C-ABI.  A
    softmax near the copy's time is at the floor that launch latency and
    first-byte latency set for this many bytes, whatever its arithmetic."""
    import torch

    lib = capi.lib()
    R, C = 512, 4096
    one = torch.empty(1, dtype=torch.float16, device="cuda")
    src = torch.randn(R, C, generator=_gen(0)).half().cuda()
    dst = torch.empty_like(src)
    x = (torch.randn(R, C, generator=_gen(0)) * 4).half().cuda()
    y = torch.empty_like(x)
    out = {}
    for name, fn in (
            ("fill_1_element_torch", lambda st: one.fill_(1.0)),
            ("copy_4MiB_torch", lambda st: dst.copy_(src)),
            ("c1_softmax_512x4096", lambda st: capi.check(
                lib.sph_softmax_rows_f16(x.data_ptr(), y.data_ptr(), R, C, st),
                "sph_softmax_rows_f16"))):
        out[name] = {"us_per_launch": round(graph_us(fn, reps, per_graph=50), 2)}
    nbytes = 2 * R * C * 2
    for k in ("copy_4MiB_torch", "c1_softmax_512x4096"):
        out[k]["GB/s"] = round(nbytes / (out[k]["us_per_launch"] * 1e-6) / 1e9, 1)
    return {"launch_floor": out}


# (name, M, N, K, B layout[, split-K workspace]): "nn" = B [K, N] row-major
# (A @ B), "nt" = B given as a weight [N, K] (A @ W^T, nn.Linear); the
# workspace is passed unless the entry says False (then a shape whose
# 256-wide tiles leave CUs idle runs 256 x 128 tiles)
YARDSTICK_SHAPES = [
    ("c2 4096^3 A@B", 4096, 4096, 4096, "nn"),
    ("4096^3 A@W^T", 4096, 4096, 4096, "nt"),
    ("8192^3 A@B", 8192, 8192, 8192, "nn"),
    ("c4 QKV 2048x6144x4096", 2048, 6144, 4096, "nt"),
    ("c4 O 2048x4096x4096", 2048, 4096, 4096, "nt"),
    ("c4 O 2048x4096x4096 without workspace", 2048, 4096, 4096, "nt", False),
    ("c4 gate/up 2048x25600x4096", 2048, 25600, 4096, "nt"),
    ("c4 down 2048x4096x12800", 2048, 4096, 12800, "nt"),
    ("c5 prefill gate/up 4096x25600x4096", 4096, 25600, 4096, "nt"),
    ("c5 prefill down 4096x4096x12800", 4096, 4096, 12800, "nt"),
]


def bench_gemm_yardstick(stream, capi, settle_ms=60.0, time_ms=40.0):
    """This build's GEMM (sph_gemm_ex with its split-K workspace, as the
    ATen mm / linear ops call it) next to torch's ROCm BLAS with hipBLASLt
    selected, on the same fp16 operands (U(-1, 1)), at the c2 / c4 / c5
    shapes and 8192^3.  Each side runs ~settle_ms of untimed launches (the
    part's steady clock) and then ~time_ms of timed ones (HIP events on one
    stream); a sample of rows of both results must agree within 1e-2, so
    both do the same work."""
    import torch

    torch.backends.cuda.preferred_blas_library("cublaslt")  # hipBLASLt on ROCm
    lib = capi.lib()
    s = stream.cuda_stream
    timer = Timer(stream)
    out = {}
    for name, M, N, K, lay, *opt in YARDSTICK_SHAPES:
        A = (torch.rand(M, K, generator=_gen(70)) * 2 - 1).half().cuda()
        Bm = (torch.rand(*((N, K) if lay == "nt" else (K, N)), generator=_gen(71)) * 2 - 1)
        Bm = Bm.half().cuda()
        D = torch.empty(M, N, dtype=torch.float16, device="cuda")
        nws = lib.sph_gemm_workspace_bytes(1, M, N, K) if not opt or opt[0] else 0
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
        tb = 1 if lay == "nt" else 0
        ldb = K if lay == "nt" else N

        def ours():
            capi.check(lib.sph_gemm_ex(capi.F16, 0, tb, 1, M, N, K, 1.0, A.data_ptr(), K, 0,
                                       Bm.data_ptr(), ldb, 0, 0.0, None, 0, 0, 0, D.data_ptr(),
                                       N, 0, 0, ws.data_ptr() if nws else None, nws, s),
                       "sph_gemm_ex")

        def theirs():
            return torch.mm(A, Bm.t() if lay == "nt" else Bm)

        flop = 2.0 * M * N * K
        est_ms = flop / 1.2e15 * 1e3
        warm = max(5, int(settle_ms / est_ms))
        reps = max(5, int(time_ms / est_ms))
        ms_o, _ = timer.run(ours, reps, warm)
        with torch.cuda.stream(stream):
            ms_t, _ = timer.run(theirs, reps, warm)
            ref = theirs()
        torch.cuda.synchronize()
        rows = torch.arange(0, M, max(1, M // 16), device="cuda")
        torch.testing.assert_close(D.index_select(0, rows).float(),
                                   ref.index_select(0, rows).float(), rtol=1e-2, atol=1e-2)
        out[name] = {"M": M, "N": N, "K": K, "B": lay,
                     "spyre_TFLOP/s": round(flop / ms_o / 1e9, 1),
                     "hipblaslt_TFLOP/s": round(flop / ms_t / 1e9, 1),
                     "spyre_frac": round(flop / ms_o / 1e9 / PEAK_FP16_TFLOPS, 4)}
        del A, Bm, D, ws, ref
    return {"gemm_yardstick": out}


def bench_bmm(steps, warmup, stream, capi):
    """c2 bmm 32 x [2048,128] x [128,2048]: HBM-bound (AI 113.8 < ridge 314.6)."""
    import torch

    s = stream.cuda_stream
    lib = capi.lib()
    out = {}
    timer = Timer(stream)
    Bt, M, N, K = 32, 2048, 2048, 128
    A = (torch.rand(Bt, M, K, generator=_gen(0)) * 2 - 1).half().cuda()
    Bm = (torch.rand(Bt, K, N, generator=_gen(1)) * 2 - 1).half().cuda()
    D = torch.empty(Bt, M, N, dtype=torch.float16, device="cuda")
    ms, _ = timer.run(lambda: lib.sph_bmm_f16(Bt, M, N, K, A.data_ptr(), Bm.data_ptr(),
                                              D.data_ptr(), s), steps, warmup)
    nbytes = (Bt * M * K + Bt * K * N + Bt * M * N) * 2
    flop = 2.0 * Bt * M * N * K
    gbs = nbytes / (ms * 1e-3) / 1e9
    out["c2_bmm_32x2048x2048x128"] = {
        "us_per_launch": round(ms * 1e3, 2), "algorithmic_bytes": nbytes,
        "GB/s": round(gbs, 1), "roofline_frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
        "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 1), "traffic": _traffic_for("bmm")}
    return out


def bench_copy(steps, warmup, stream, capi):
    """Plain device copy of a known size (512 MiB read + 512 MiB written):
    the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = 256 * 1024 * 1024  # fp16 elements = 512 MiB
    src = torch.empty(n, dtype=torch.float16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    ops = (capi.Operand * 2)(capi.operand(dst.data_ptr(), capi.F16, [1]),
                             capi.operand(src.data_ptr(), capi.F16, [1]))
    sizes = capi.i64_array([n])
    lib = capi.lib()
    s = stream.cuda_stream

    def step():
        capi.check(lib.sph_pointwise(0, 1, ops, 1, sizes, 0.0, 0.0, s), "sph_pointwise copy")

    ms, _ = Timer(stream).run(step, steps, warmup)
    return {"us_per_launch": round(ms * 1e3, 2), "bytes": 2 * n * 2,
            "GB/s": round(2 * n * 2 / (ms * 1e-3) / 1e9, 1)}


def _spyre_timer():
    """Timer on the spyre stream (HIP events recorded on that stream)."""
    import torch

    from torch_spyre import _C

    return Timer(torch.cuda.ExternalStream(_C._stream_handle(0)))


def bench_spyre_paths(steps, warmup):
    """The drop-in paths on "spyre" tensors: eager ATen kernels and
    torch.compile-generated kernels for the c1 / c3 workloads."""
    import torch
    import torch.nn.functional as F

    import torch_spyre  # noqa: F401

    timer = _spyre_timer()
    out = {}

    def entry(name, nbytes, fn):
        fn()
        torch.spyre.synchronize()
        ms, _ = timer.run(fn, steps, warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_call": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                     "roofline_frac": round(gbs / PEAK_HBM_GBS, 4)}

    R, C = 512, 4096
    x = (torch.randn(R, C, generator=_gen(0)) * 4).half().to("spyre")
    sm = torch.compile(lambda a: torch.softmax(a, dim=-1))
    entry("c1_softmax_eager_spyre", 2 * R * C * 2, lambda: torch.softmax(x, -1))
    entry("c1_softmax_compiled_spyre", 2 * R * C * 2, lambda: sm(x))
    # The same compiled function with its host path taken away: 20 calls
    # captured in one HIP graph of the spyre stream, replayed (GPU time per
    # call).  The gap to the entry above is torch.compile's per-call host
    # path, not the generated kernel.
    per_graph = 20
    g = torch.spyre.SpyreGraph()
    with torch.spyre.graph(g):
        for _ in range(per_graph):
            sm(x)
    ms, _ = timer.run(g.replay, max(steps // 4, 5), 3)
    us = ms * 1e3 / per_graph
    gbs = 2 * R * C * 2 / (us * 1e-6) / 1e9
    out["c1_softmax_compiled_spyre_graph"] = {
        "us_per_call": round(us, 2), "GB/s": round(gbs, 1),
        "roofline_frac": round(gbs / PEAK_HBM_GBS, 4),
        "note": f"{per_graph} compiled calls per HIP graph replay"}
    g.reset()
    R, C = 8192, 4096
    x = torch.randn(R, C, generator=_gen(0)).half().to("spyre")
    r = torch.randn(R, C, generator=_gen(1)).half().to("spyre")
    w = (torch.randn(C, generator=_gen(2)) * 0.02 + 1).half().to("spyre")
    b = (torch.randn(C, generator=_gen(3)) * 0.02).half().to("spyre")
    rms = torch.compile(lambda a, c, g: (lambda s: (s, torch.rms_norm(s, [C], g, 1e-5)))(a + c))
    ln = torch.compile(lambda a, c, g, e: (lambda s: (s, F.layer_norm(s, [C], g, e, 1e-5)))(a + c))
    gl = torch.compile(lambda a, s, c: (lambda t: (t, t.sum(-1)))(F.gelu(a * s + c)))
    entry("c3_add_rmsnorm_compiled_spyre", 4 * R * C * 2 + C * 2, lambda: rms(x, r, w))
    entry("c3_add_layernorm_compiled_spyre", 4 * R * C * 2 + 2 * C * 2, lambda: ln(x, r, w, b))
    entry("c3_gelu_rowsum_compiled_spyre", 2 * R * C * 2 + 2 * C * 2 + R * 2, lambda: gl(x, w, b))
    entry("c3_rms_norm_eager_spyre", 2 * R * C * 2 + C * 2,
          lambda: torch.rms_norm(x, [C], w, 1e-5))
    return out


def bench_host_copies(reps=5, mib=256):
    """Host<->device copy throughput of spyre tensors (GB/s, median of
    `reps`), pageable and pinned, next to torch-ROCm's own copies of the
    same bytes as a yardstick.  Wall time from the call to the end of a
    device synchronise."""
    import statistics
    import time

    import torch

    n = mib << 20
    x = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=_gen(7))
    xp = x.pin_memory()
    back = torch.empty_like(x)
    backp = torch.empty_like(x).pin_memory()
    d = torch.empty(n, dtype=torch.uint8, device="spyre")
    c = torch.empty(n, dtype=torch.uint8, device="cuda")

    def rate(fn, sync):
        fn()
        sync()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            sync()
            ts.append(time.perf_counter() - t0)
        return round(n / statistics.median(ts) / 1e9, 1)

    ss, cs = torch.spyre.synchronize, torch.cuda.synchronize
    out = {"bytes": n,
           "spyre_h2d_pageable_GBs": rate(lambda: d.copy_(x), ss),
           "spyre_h2d_pinned_nonblocking_GBs": rate(lambda: d.copy_(xp, non_blocking=True), ss),
           "spyre_d2h_pageable_GBs": rate(lambda: back.copy_(d), ss),
           "spyre_d2h_pinned_nonblocking_GBs": rate(lambda: backp.copy_(d, non_blocking=True), ss),
           "torch_rocm_h2d_pageable_GBs": rate(lambda: c.copy_(x), cs),
           "torch_rocm_h2d_pinned_nonblocking_GBs": rate(lambda: c.copy_(xp, non_blocking=True), cs),
           "torch_rocm_d2h_pageable_GBs": rate(lambda: back.copy_(c), cs),
           "torch_rocm_d2h_pinned_nonblocking_GBs": rate(lambda: backp.copy_(c, non_blocking=True), cs)}
    assert torch.equal(back, x) and torch.equal(backp, x)
    return out


def bench_decoder(steps, warmup, c5_layers=40, decode_steps=128):
    """c4: one decoder layer (+ embedding) compiled, prefill of 2048 tokens;
    c5: the 40-layer model, compiled prefill of 4 x 1024 tokens into the KV
    cache, then greedy decode steps (eager), all on "spyre" tensors."""
    import torch

    import torch_spyre  # noqa: F401
    from torch_spyre.examples import decoder as D

    dev = "spyre"
    timer = _spyre_timer()
    out = {}
    # --- c4 -----------------------------------------------------------------
    cfg = D.C4
    S = 2048
    params = D.init_params(cfg, dev, seed=SEED)
    tok = torch.randint(0, cfg.vocab, (1, S), generator=_gen(0)).to(dev)
    cos, sin = D.rope_tables(cfg, S, dev)
    mask = D.causal_mask(cfg, S, dev)
    blk = torch.compile(D.block_forward)
    blk(tok, params, cos, sin, mask, cfg)
    torch.spyre.synchronize()
    # >= 20 timed calls: the host's ~140 us to reach the first launch of the
    # first call is inside the timed region and is spread over the calls
    c4_steps = max(steps, 20)
    ms, wall = timer.run(lambda: blk(tok, params, cos, sin, mask, cfg), c4_steps, max(warmup, 10))
    flop = 2 * S * (cfg.hidden * (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim
                    + cfg.n_heads * cfg.head_dim * cfg.hidden + 3 * cfg.hidden * cfg.intermediate) \
        + 4 * S * S * cfg.n_heads * cfg.head_dim
    out["c4_layer_prefill_compiled"] = {
        "ms_per_step": round(ms, 3), "wall_ms": round(wall, 3),
        "tok/s": round(S / (ms * 1e-3), 1), "TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 1),
        "mfma_frac": round(flop / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
        "flop_per_step": flop, "steps": c4_steps,
        "note": "dense attention FLOPs (no causal halving)"}
    del params, blk
    torch._dynamo.reset()
    # --- c5 -----------------------------------------------------------------
    if c5_layers <= 0:
        return out
    cfg = D.DecoderConfig(n_layers=c5_layers)
    B, S = 4, 1024
    t0 = time.perf_counter()
    params = D.init_params(cfg, dev, seed=SEED, pool_elems=1 << 26)
    torch.spyre.synchronize()
    init_s = time.perf_counter() - t0
    prompt = torch.randint(0, cfg.vocab, (B, S), generator=_gen(1)).to(dev)
    cos, sin = D.rope_tables(cfg, S + decode_steps, dev)
    mask = D.causal_mask(cfg, S, dev)
    cache = D.new_cache(cfg, B, S + decode_steps, dev)
    layer = torch.compile(D.layer_forward)

    def run_prefill():
        return D.prefill(prompt, params, cos, sin, mask, cache, cfg, layer)

    logits = run_prefill()
    torch.spyre.synchronize()
    reps = 3
    ms, wall = timer.run(run_prefill, reps, 1)
    flop = cfg.n_layers * (2 * B * S * (cfg.hidden * (cfg.n_heads + 2 * cfg.n_kv_heads)
                                        * cfg.head_dim + cfg.n_heads * cfg.head_dim * cfg.hidden
                                        + 3 * cfg.hidden * cfg.intermediate)
                           + 4 * B * S * S * cfg.n_heads * cfg.head_dim) \
        + 2 * B * cfg.hidden * cfg.vocab
    entry = {"layers": cfg.n_layers, "batch": B, "prompt": S, "init_s": round(init_s, 1),
             "prefill_ms": round(ms, 2), "prefill_wall_ms": round(wall, 2),
             "prefill_tok/s": round(B * S / (ms * 1e-3), 1),
             "prefill_TFLOP/s": round(flop / (ms * 1e-3) / 1e12, 1)}
    # greedy decode: the static decode step compiled (one graph for all 40
    # layers; position tensor advanced on the device) and captured with the
    # argmax and the position update into one HIP graph; a step is one
    # replay plus the copy of the chosen tokens into the next step's input
    import torch_spyre.graphs as graphs

    dec = torch.compile(D.decode_step_static)
    pos = torch.full((1,), S, dtype=torch.int64).to(dev)
    feed = logits.argmax(-1)
    t0 = time.perf_counter()
    for _ in range(2):  # compile + warm (rewrites cache position S each time)
        dec(feed, pos, params, cos, sin, cache, cfg)
    torch.spyre.synchronize()
    entry["decode_compile_s"] = round(time.perf_counter() - t0, 1)
    g = graphs.SpyreGraph()
    with graphs.graph(g):
        step_logits = dec(feed, pos, params, cos, sin, cache, cfg)
        step_arg = step_logits.argmax(-1)
        pos.add_(1)
    tokens = torch.empty((B, decode_steps), dtype=torch.int64, device=dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(timer.stream)
    for t in range(decode_steps):
        g.replay()
        tokens[:, t].copy_(step_arg)
        feed.copy_(step_arg)
    ev1.record(timer.stream)
    torch.spyre.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / decode_steps
    dms = ev0.elapsed_time(ev1) / decode_steps
    g.reset()
    wbytes = sum(t.numel() * t.element_size() for w in params["layers"]
                 for k, t in w.items() if k in ("attn_norm", "wqkv", "wo", "mlp_norm", "wgu", "wd")) \
        + params["lm_head"].numel() * 2
    kvbytes = sum(k.numel() * k.element_size() * 2 for k, _ in cache)
    entry.update({"decode_steps": decode_steps, "decode_ms_per_step": round(dms, 3),
                  "decode_wall_ms_per_step": round(wall, 3),
                  "decode_tok/s": round(B / (wall * 1e-3), 1),
                  "decode_weight_GB/s": round(wbytes / (wall * 1e-3) / 1e9, 1),
                  "decode_hbm_frac": round((wbytes + kvbytes) / (wall * 1e-3) / 1e9 / PEAK_HBM_GBS,
                                           4),
                  "decode_path": "torch.compile(decode_step_static) + argmax captured in one "
                                 "HIP graph per step; KV over the full cache"})
    # without the graph (the compiled step called from Python), from position
    # S again: the replays above advanced `pos` to the end of the cache
    # (at most decode_steps of them: the cache holds S + decode_steps positions)
    n_side = min(8, decode_steps)
    pos.fill_(S)
    torch.spyre.synchronize()
    t0 = time.perf_counter()
    for t in range(n_side):
        lg = dec(feed, pos, params, cos, sin, cache, cfg)
        feed = lg.argmax(-1)
    torch.spyre.synchronize()
    entry["decode_nograph_wall_ms_per_step"] = round((time.perf_counter() - t0) * 1e3 / n_side, 3)
    # the eager decode step, for comparison (a few steps)
    torch.spyre.synchronize()
    t0 = time.perf_counter()
    for t in range(n_side):
        D.decode_step(feed, S + t, params, cos, sin, cache, cfg)
    torch.spyre.synchronize()
    entry["decode_eager_wall_ms_per_step"] = round((time.perf_counter() - t0) * 1e3 / n_side, 3)
    out["c5_model"] = entry
    del params, cache
    torch._dynamo.reset()
    return out


def bench_eager_mm(steps, warmup):
    """torch.mm on "spyre" tensors: the drop-in (PrivateUse1) path to the same
    kernel, timed on the spyre stream."""
    import torch

    import torch_spyre  # noqa: F401

    a = (torch.rand(4096, 4096, generator=_gen(0)) * 2 - 1).half().to("spyre")
    b = (torch.rand(4096, 4096, generator=_gen(1)) * 2 - 1).half().to("spyre")
    for _ in range(warmup):
        torch.mm(a, b)
    torch.spyre.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        torch.mm(a, b)
    torch.spyre.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"ms_per_call": round(ms, 4), "TFLOP/s": round(2 * 4096 ** 3 / (ms * 1e-3) / 1e12, 1)}


def _cpu_setup():
    """Threads = the cores this process may run on (BASELINE's CPU protocol);
    returns (threads, CPU model name)."""
    import torch

    torch.set_num_threads(len(os.sched_getaffinity(0)))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return torch.get_num_threads(), model


CPU_BUDGET_S = 6.0  # wall time of one CPU figure's repetitions


def _median_s(fn, reps=10, warmup=3, budget_s=CPU_BUDGET_S):
    """Median wall time of up to `reps` calls after up to `warmup` calls,
    cut so that the calls fit about `budget_s` (the first call, timed, sets
    the counts; at least one timed call follows it).  Returns (median,
    times)."""
    import statistics

    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    fit = int(budget_s / max(first, 1e-6))
    for _ in range(max(0, min(warmup - 1, fit // 4))):
        fn()
    ts = []
    for _ in range(max(1, min(reps, fit))):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


def cpu_per_config():
    """The reference's CPU path for every config, timed on this host in the
    same run: the config's function run eagerly by torch on CPU tensors of
    the same shapes and dtype (fp16), as the reference's tests do
    (compare_with_cpu, tests/_inductor/utils_inductor.py:186-198).  c1-c3:
    full inputs, median of up to 10 after 3 warmups; c4: the full layer at
    seq 2048, median of up to 3, or a shorter sequence when one full call
    would take more than a few seconds on this CPU (torch's fp16 matmul is
    slow on CPUs without fp16 arithmetic); c5: one layer of the prefill and
    decode steps of a 2-layer slice, scaled to 40 layers.  Each figure is
    bounded to a few seconds, so the whole section takes well under a
    minute on any host; every sample is stated."""
    import torch
    import torch.nn.functional as F

    from torch_spyre.examples import decoder as D

    threads, model = _cpu_setup()
    out = {"threads": threads, "cpu": model}

    def hbm(name, nbytes, fn, sample):
        _log(f"cpu {name}")
        t, ts = _median_s(fn)
        out[name] = {"GB/s": round(nbytes / t / 1e9, 2), "ms": round(t * 1e3, 3),
                     "reps": len(ts), "sample": sample}

    R, C = 512, 4096
    x = (torch.randn(R, C, generator=_gen(0)) * 4).half()
    hbm("c1_softmax_512x4096", 2 * R * C * 2, lambda: torch.softmax(x, dim=-1),
        "torch.softmax(x, -1), fp16 CPU, full input")
    R, C = 8192, 4096
    x = torch.randn(R, C, generator=_gen(0)).half()
    r = torch.randn(R, C, generator=_gen(1)).half()
    w = (torch.randn(C, generator=_gen(2)) * 0.02 + 1).half()
    b = (torch.randn(C, generator=_gen(3)) * 0.02).half()
    hbm("c3_add_rmsnorm", 4 * R * C * 2 + C * 2,
        lambda: (lambda h: (h, torch.rms_norm(h, [C], w, 1e-5)))(x + r),
        "h = x + res; rms_norm(h) * w, fp16 CPU, full input")
    hbm("c3_add_layernorm", 4 * R * C * 2 + 2 * C * 2,
        lambda: (lambda h: (h, F.layer_norm(h, [C], w, b, 1e-5)))(x + r),
        "h = x + res; layer_norm(h, w, b), fp16 CPU, full input")
    hbm("c3_gelu_rowsum", 2 * R * C * 2 + 2 * C * 2 + R * 2,
        lambda: (lambda y: (y, y.sum(-1)))(F.gelu(x * w + b)),
        "y = gelu(x * s + b); y.sum(-1), fp16 CPU, full input")
    del x, r
    _log("cpu c2 bmm")
    A = (torch.rand(32, 2048, 128, generator=_gen(0)) * 2 - 1).half()
    Bm = (torch.rand(32, 128, 2048, generator=_gen(1)) * 2 - 1).half()
    # batches are independent: time the first nb of them when all 32 would
    # not fit the budget (one probe batch sets nb)
    t0 = time.perf_counter()
    torch.bmm(A[:1], Bm[:1])
    one = time.perf_counter() - t0
    nb = 32 if one * 32 <= 2.0 else max(1, min(32, int(2.0 / max(one, 1e-6))))
    As, Bs = A[:nb], Bm[:nb]
    t, ts = _median_s(lambda: torch.bmm(As, Bs))
    out["c2_bmm_32x2048x2048x128"] = {
        "TFLOP/s": round(2 * nb * 2048 * 2048 * 128 / t / 1e12, 4), "ms": round(t * 1e3, 2),
        "reps": len(ts),
        "sample": "torch.bmm, fp16 CPU, " + ("full input" if nb == 32 else
                                             f"batches 0..{nb} of 32")}
    # c4: embedding + one layer, fp16; the sequence length is cut when a
    # full-length call would not fit the budget
    cfg = D.C4
    params = D.init_params(cfg, "cpu", pool_elems=1 << 24)
    with torch.no_grad():
        S = 2048
        for S in (256, 512, 1024, 2048):
            cos, sin = D.rope_tables(cfg, S, "cpu")
            mask = D.causal_mask(cfg, S, "cpu")
            tok = torch.randint(0, cfg.vocab, (1, S), generator=_gen(0))
            _log(f"cpu c4 layer, seq {S}")
            t0 = time.perf_counter()
            D.block_forward(tok, params, cos, sin, mask, cfg)
            if S == 2048 or (time.perf_counter() - t0) * 2.5 > 2.0:
                break
        t, ts = _median_s(lambda: D.block_forward(tok, params, cos, sin, mask, cfg), reps=3,
                          warmup=1)
    out["c4_layer_prefill"] = {"tok/s": round(S / t, 1), "ms": round(t * 1e3, 1),
                               "reps": len(ts),
                               "sample": f"decoder.block_forward (embedding + 1 layer), seq {S}"
                                         f"{'' if S == 2048 else ' of 2048'}, fp16 CPU"}
    del params
    # c5: one layer of the prefill at batch 4 (or fewer rows), and decode
    # steps of a 2-layer slice; per-layer times x 40 + the LM head
    B, S, T = 4, 1024, 128
    sl = D.DecoderConfig(n_layers=2)
    params = D.init_params(sl, "cpu", pool_elems=1 << 24)
    cos, sin = D.rope_tables(sl, S + T, "cpu")
    mask = D.causal_mask(sl, S, "cpu")
    w0 = params["layers"][0]
    with torch.no_grad():
        # one layer over the first Sp prompt positions of one sequence
        # (causal: the same work as a prompt of length Sp), Sp doubled from
        # 128 while the next call fits the budget; time per token is scaled
        # to 4 x 1024, which undercounts attention's quadratic part, so the
        # CPU figure is an upper bound of the CPU's throughput
        Sp, one = 128, None
        for sp in (128, 256, 512, 1024):
            if one is not None and one * 2.2 > 3.0:
                break
            Sp = sp
            h = torch.randn(1, Sp, sl.hidden, generator=_gen(2)).half()
            _log(f"cpu c5 prefill layer (1 x {Sp})")
            t0 = time.perf_counter()
            D.layer_forward(h, w0, cos[:Sp], sin[:Sp], D.causal_mask(sl, Sp, "cpu"), sl)
            one = time.perf_counter() - t0
        hl = torch.randn(1, sl.hidden, generator=_gen(3)).half()
        t_head, _ = _median_s(lambda: D.lm_logits(hl, params, sl), reps=3, warmup=1, budget_s=3.0)
        pre40 = (one * 40 + t_head) * (B * S / Sp)
        _log("cpu c5 decode steps (2-layer slice)")
        cache = D.new_cache(sl, B, S + T, "cpu")
        feed = torch.randint(0, sl.vocab, (B,), generator=_gen(4))
        D.decode_step(feed, S, params, cos, sin, cache, sl)
        t0 = time.perf_counter()
        steps = 2
        for i in range(steps):
            D.decode_step(feed, S + 1 + i, params, cos, sin, cache, sl)
        t_dec = (time.perf_counter() - t0) / steps
        h4 = torch.randn(B, sl.hidden, generator=_gen(5)).half()
        t_head4, _ = _median_s(lambda: D.lm_logits(h4, params, sl), reps=3, warmup=1,
                               budget_s=3.0)
    dec40 = (t_dec - t_head4) / sl.n_layers * 40 + t_head4
    out["c5_prefill_extrapolated"] = {
        "tok/s": round(B * S / pre40, 1), "s": round(pre40, 2),
        "sample": f"one decoder layer over 1 x {Sp} prompt positions, fp16 CPU, one call; "
                  "x 40 layers + the LM head, scaled by tokens to 4 x 1024 (extrapolated)"}
    out["c5_decode_extrapolated"] = {
        "tok/s": round(B / dec40, 2), "ms_per_step": round(dec40 * 1e3, 1),
        "sample": f"decoder.decode_step of a 2-layer slice, batch 4, {steps} steps, fp16 CPU; "
                  "per-layer time x 40 + the LM head (extrapolated)"}
    return out


def cpu_baseline_gemm(a, b):
    """The CPU baseline of the headline: the reference's CPU path
    fn(*cpu_args) = torch.mm eager on the same fp16 tensors on this host's
    CPU (what compare_with_cpu runs, tests/_inductor/utils_inductor.py:190),
    median of up to 10 after 3 warmups.  Full 4096^3 when a call takes at
    most ~1.5 s here; otherwise the first rows of A (a GEMM's time is linear
    in its rows: a 16-row probe sets how many rows fill about 4 s), stated in
    `sample`."""
    import torch

    threads, model = _cpu_setup()
    ac, bc = a.cpu(), b.cpu()
    t0 = time.perf_counter()
    torch.mm(ac[:16], bc)
    est = (time.perf_counter() - t0) * (ac.shape[0] / 16)
    rows = ac.shape[0]
    if est > 1.5:
        rows = max(16, int(ac.shape[0] * 4.0 / est) // 16 * 16)
    a_s = ac[:rows]
    t, ts = _median_s(lambda: torch.mm(a_s, bc), budget_s=12.0)
    flop = 2.0 * rows * ac.shape[1] * bc.shape[1]
    what = "full 4096^3" if rows == ac.shape[0] else f"rows 0..{rows} of A (4096 x 4096 B)"
    return {"value": round(flop / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "reference",
            "sample": f"torch.mm eager on the same fp16 A, B on the CPU ({model}), {what}, "
                      f"median of {len(ts)} ({min(ts) * 1e3:.0f}-{max(ts) * 1e3:.0f} ms)"}


def cpu_oracle_gemm(a, b, seconds=3.0):
    """The oracle's numpy fp32 GEMM (BLAS) on 512 rows of the same problem:
    a second CPU figure, the restatement the parity tests check against."""
    from oracle import ops as O

    rows = 512
    an = a[:rows].float().cpu().numpy()
    bn = b.float().cpu().numpy()
    O.gemm(an[:64], bn)
    reps, t0 = 0, time.perf_counter()
    while True:
        O.gemm(an, bn)
        reps += 1
        el = time.perf_counter() - t0
        if el > seconds:
            break
    return {"TFLOP/s": round(2.0 * rows * b.shape[0] * b.shape[1] * reps / el / 1e12, 4),
            "sample": f"oracle.ops.gemm (numpy fp32) on rows 0..{rows}, {reps} reps"}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The part needs ~30-40 ms of sustained load to reach its steady clock:
    # 4096^3 measured 989 TFLOP/s after 10 warmup launches, 1165 after 100,
    # 1210-1212 after 300 or 1000.  300 launches (~35 ms) reach steady state.
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decoder", action="store_true")
    ap.add_argument("--c5-layers", type=int, default=40)
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--kernel", choices=["all", "gemm", "copy", "decoder", "bmm", "h2d",
                                         "attention", "spyre", "rows", "decode_step", "floor",
                                         "yardstick", "gemm_cold"],
                    default="all",
                    help="gemm / copy / decoder / bmm / h2d / attention / decode_step / floor / "
                         "yardstick (the GEMM next to hipBLASLt) / gemm_cold (operands from "
                         "HBM) / "
                         "rows (c1 softmax and "
                         "the c3 row kernels) / spyre (the eager and compiled paths on spyre "
                         "tensors): run only that part (for rocprofv3 passes)")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="summarise rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes under DIR "
                         "(pmc_<part>_<COUNTER>/) into profiles/traffic.json and exit")
    args = ap.parse_args(argv)
    if args.decode_steps < 1 or args.c5_layers < 1:
        ap.error("--decode-steps and --c5-layers must be at least 1")
    if args.traffic_from:
        print(json.dumps(summarize_traffic(args.traffic_from, ALGORITHMIC_BYTES), indent=1))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one MI355X; runs on more than one GPU are not "
              "part of it (see DESIGN.md, 'How the path would shard').", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    # A function that hits dynamo's recompile limit would run eagerly from
    # then on: a figure labelled compiled must come from the compiled program.
    torch._dynamo.config.fail_on_recompile_limit_hit = True
    from torch_spyre import _capi

    stream = torch.cuda.current_stream()
    if args.kernel == "copy":
        print(json.dumps({"kernel": "copy", **bench_copy(args.steps, args.warmup, stream, _capi)}))
        return 0
    if args.kernel == "bmm":
        print(json.dumps({"kernel": "bmm", **bench_bmm(args.steps, args.warmup, stream, _capi)}))
        return 0
    if args.kernel == "rows":
        print(json.dumps({"kernel": "rows", **bench_rows(args.steps, args.warmup, stream, _capi)}))
        return 0
    if args.kernel == "attention":
        print(json.dumps({"kernel": "attention",
                          **bench_attention(args.steps, args.warmup, stream, _capi)}))
        return 0
    if args.kernel == "yardstick":
        print(json.dumps({"kernel": "yardstick", **bench_gemm_yardstick(stream, _capi)}))
        return 0
    if args.kernel == "gemm_cold":
        print(json.dumps({"kernel": "gemm_cold",
                          **bench_gemm_cold(args.steps, args.warmup, stream, _capi),
                          **bench_gemm_bf16(args.steps, args.warmup, stream, _capi)}))
        return 0
    if args.kernel == "floor":
        print(json.dumps({"kernel": "floor", **bench_launch_floor(max(20, args.steps), _capi)}))
        return 0
    if args.kernel == "decode_step":
        print(json.dumps({"kernel": "decode_step",
                          **bench_decode_step(max(20, args.steps), stream, _capi)}))
        return 0
    if args.kernel == "h2d":
        print(json.dumps({"kernel": "h2d", **bench_host_copies()}))
        return 0
    if args.kernel == "spyre":
        print(json.dumps({"kernel": "spyre", **bench_spyre_paths(args.steps, args.warmup)}))
        return 0
    if args.kernel == "decoder":
        print(json.dumps({"kernel": "decoder",
                          **bench_decoder(5, 2, args.c5_layers, args.decode_steps)}))
        return 0
    if args.kernel == "gemm":
        args.no_extra = args.no_cpu = True
    # The secondary kernels run first, each with its own warmup (at least
    # SUB_WARMUP launches: their figures are per-kernel and need the part's
    # steady clock, which it reaches after ~35 ms of sustained load).  The
    # headline GEMM then runs exactly `--warmup` untimed and `--steps` timed
    # launches on a part that has been working, as it would inside a model.
    extra = {}
    sub_w = max(args.warmup, SUB_WARMUP)
    if not args.no_extra:
        _log("extra kernels")
        extra = bench_extra(max(10, args.steps), sub_w, stream, _capi)
        _log("fused attention (c4 shape)")
        extra.update(bench_attention(max(10, args.steps), sub_w, stream, _capi))
        _log("decode-step attention (c5 shape)")
        extra.update(bench_decode_step(max(20, args.steps), stream, _capi))
        _log("GEMMs with operands from HBM")
        extra.update(bench_gemm_cold(max(10, args.steps), sub_w, stream, _capi))
        _log("bf16 gemm 4096^3")
        extra.update(bench_gemm_bf16(max(10, args.steps), sub_w, stream, _capi))
    _log("gemm 4096^3")
    g = bench_gemm(args.steps, args.warmup, stream, _capi)
    if not args.no_extra:
        _log("eager torch.mm on spyre tensors")
        extra["c2_mm_4096_spyre_device_eager"] = bench_eager_mm(max(10, args.steps), sub_w)
        _log("spyre device paths (eager + torch.compile)")
        extra["spyre_device"] = bench_spyre_paths(max(10, args.steps), sub_w)
        _log("host<->device copies")
        extra["host_device_copy"] = bench_host_copies()
        if not args.no_decoder:
            _log("decoder workloads (c4 layer, c5 model)")
            extra["decoder"] = bench_decoder(5, 2, args.c5_layers, args.decode_steps)
    cpu = None
    if not args.no_cpu:
        _log("cpu baseline")
        cpu = cpu_baseline_gemm(g["a"], g["b"])
        extra["cpu_oracle_gemm_numpy"] = cpu_oracle_gemm(g["a"], g["b"])
        if not args.no_extra:
            _log("cpu side of every config")
            extra["cpu_per_config"] = cpu_per_config()
    tflops = g["tflops"]
    line = {
        "metric": "fp16 GEMM TFLOP/s (M=N=K=4096, fp32 accumulate)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (U(-1,1), seed 0xAFFE)",
        "config": {"workload": "c2: fp16 mm C = A @ B, M=N=K=4096 (BASELINE configs[1])",
                   "M": 4096, "N": 4096, "K": 4096, "path": "C-ABI sph_gemm_f16"},
        "precondition": {"launches": g["precondition_launches"], "ms": PRECONDITION_MS,
                         "why": "untimed launches before the warmup so the timed steps run at "
                                "the part's steady clock under this load"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": _traffic_for("gemm")},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
