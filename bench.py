#!/usr/bin/env python3
"""bench.py -- headline benchmark of the gfx950 attention core on one MI355X.

Metric: "attn TFLOP/s (causal fwd S=4096 D=128) + decode HBM
GB/s, 1 MI355X".

  value      causal prefill forward, config C3: B=4 H=32 S=4096 D=128, fp32
             Q/K/V in HBM, fp32 O and LSE out, bf16 MFMA with fp32 accumulate.
             A step is one gonn_hip_attn_fwd call (pack kernel + attention
             kernel). FLOP per step = 4*B*H*S^2*D*0.5 (the reference's
             convention, benchmark/flashattn/main.go:138-142).
  decode     config C4: B=64 H=32 D=128, bf16 cache of 8192 positions,
             lengths ~ U[512, 8192]; bytes per step = valid K+V rows + q + o.
  mha        config C1: nn.MultiHeadAttention forward, B=2 S=128 E=256 H=4,
             causal, fp64 host data: projections on the host with the fused
             core, the resident layer (weights in HBM; one upload and one
             download per call), and the resident layer on device buffers.
  roofline   the dominant kernel of each workload, timed live with HIP events
             recorded by the library on the stream the kernel runs on.
  cpu_baseline  the fp64 oracle (a C restatement of GoNN's CPU attention op
             sequence; GoNN's Go path cannot run here) on a bounded sample of
             the same workload: whole (b,h) slices, scaled to TFLOP/s with
             the same FLOP convention.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "attn TFLOP/s (causal fwd S=4096 D=128) + decode HBM GB/s, 1 MI355X"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def load_traffic(key: str):
    """HBM bytes per launch of `kernel:workload` measured by rocprofv3 --pmc
    (FETCH_SIZE and WRITE_SIZE passes, scaled by the 1 GiB copy calibration,
    profiles/README.md); None if absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t.get(key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def _prime_queue(torch, ms=20.0):
    """Queue a bounded spin kernel (~ms at 2 GHz) ahead of a timed loop, so the
    host enqueues the loop's calls while the GPU spins and the calls then run
    back to back: a step shorter than its host-side call (C2, decode) is timed
    as device work rather than as the gaps of a starved queue. The timed span
    starts after the spin."""
    torch.cuda._sleep(int(ms * 2e6))


def _run_steps(torch, run, steps):
    """Time `steps` back-to-back calls on the current stream with an event
    before each call and one after the last: (mean ms, median ms, wall s).
    The mean is the span of the whole run over `steps`."""
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    # No garbage-collector pause inside the timed span (host-side only: the
    # device work is unchanged).
    gc.collect()
    gc.disable()
    try:
        _prime_queue(torch)
        t0 = time.perf_counter()
        for i in range(steps):
            ev[i].record()
            run()
        ev[steps].record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    finally:
        gc.enable()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return ev[0].elapsed_time(ev[steps]) / steps, statistics.median(per), wall


def bench_prefill(torch, hip, steps, warmup):
    B, H, S, D = 4, 32, 4096, 128
    flop = 4.0 * B * H * S * S * D * 0.5
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    q = torch.randn((B * H, S, D), generator=g, device="cuda")
    k = torch.randn((B * H, S, D), generator=g, device="cuda")
    v = torch.randn((B * H, S, D), generator=g, device="cuda")
    o = torch.empty_like(q)
    run = lambda: hip.attn_fwd(q, k, v, causal=True, mode="bf16", out=o)  # noqa: E731
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    ms, med, wall = _run_steps(torch, run, steps)
    # per-kernel pass (events recorded by the library around each stage)
    hip.profile_reset()
    hip.profile_enable(True)
    _prime_queue(torch)
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    hip.profile_enable(False)
    kt, kn = hip.profile_read("fwd_bf16")
    pt, pn = hip.profile_read("pack_kv")
    hip.profile_reset()
    # Shader clock over the same run of steps: a one-wave probe on a side
    # stream starts when the spin ahead of the steps ends and reads the
    # clock for 90% of their measured span.
    side = torch.cuda.Stream()
    _prime_queue(torch)
    start = torch.cuda.Event()
    start.record()
    side.wait_event(start)
    hip.calib_clock_start(0.9 * ms * steps, stream=side)
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    sclk = hip.calib_clock_read()
    # Per-launch time of each stage and the launches per step (one pack and
    # one attention kernel per gonn_hip_attn_fwd call).
    return dict(B=B, H=H, S=S, D=D, flop=flop, ms=ms, median_ms=med, wall_s=wall,
                kernel_ms=kt / max(kn, 1), pack_ms=pt / max(pn, 1),
                launches=max(kn, 1) / steps, sclk_ghz=sclk, q=q, k=k, v=v)


def calibration(torch, hip, sclk_ghz):
    """Figures of the box itself, measured in the same process, so a slow box
    can be told from a slow kernel: the rate and clock of a fixed MFMA loop on
    constant operands and on random ones (real data's switching, under which
    the power limit lowers the clock: the rate no bf16 MFMA kernel can pass
    on this box), the bandwidth of a 1 GiB device copy (bytes read + written
    per second), and the shader clock during the C3 steps (nominal 2.4 GHz)."""
    mfma, mfma_ghz = hip.calib_mfma(False)
    mfma_r, mfma_r_ghz = hip.calib_mfma(True)
    n = 1 << 28
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    for _ in range(2):
        y.copy_(x)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 5 * 2 * 4 * n / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del x, y
    return {"mfma_const_TFLOPs": round(mfma, 1),
            "mfma_const_frac": round(mfma / PEAK_BF16_TFLOPS, 4),
            "mfma_const_GHz": round(mfma_ghz, 3),
            "mfma_random_TFLOPs": round(mfma_r, 1),
            "mfma_random_frac": round(mfma_r / PEAK_BF16_TFLOPS, 4),
            "mfma_random_GHz": round(mfma_r_ghz, 3),
            "copy_1GiB_GBps": round(copy_gbs, 1),
            "copy_frac": round(copy_gbs / PEAK_HBM_GBS, 4),
            "sclk_GHz_during_c3": round(sclk_ghz, 3),
            "note": "mfma_const / mfma_random: v_mfma_f32_32x32x16_bf16 loop on constant / "
                    "uniform random operands, two waves per SIMD, clock over the loop; copy: "
                    "torch copy_ of 2^28 floats, read + write bytes; "
                    "sclk: s_memtime against the 100 MHz s_memrealtime over the C3 steps"}


def bench_decode(torch, hip, steps, warmup):
    import numpy as np
    B, H, Lmax, D = 64, 32, 8192, 128
    lens = np.random.default_rng(4).integers(512, Lmax + 1, B).astype(np.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(44)
    q = torch.randn((B, H, D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn((B, H, Lmax, D), generator=g, device="cuda", dtype=torch.bfloat16)
    vc = torch.randn((B, H, Lmax, D), generator=g, device="cuda", dtype=torch.bfloat16)
    kl = torch.from_numpy(lens).cuda()
    o = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
    nbytes = int(2 * H * D * 2 * int(lens.sum()) + B * H * D * 2 + B * H * D * 4)
    run = lambda: hip.attn_decode(q, kc, vc, kl, out=o)  # noqa: E731
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    ms, med, _ = _run_steps(torch, run, steps)
    hip.profile_reset()
    hip.profile_enable(True)
    _prime_queue(torch)
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    hip.profile_enable(False)
    st, sn = hip.profile_read("decode_split")
    ct, cn = hip.profile_read("decode_combine")
    hip.profile_reset()
    del kc, vc
    return dict(B=B, H=H, Lmax=Lmax, D=D, mean_len=float(lens.mean()), bytes=nbytes, ms=ms,
                median_ms=med, split_ms=st / max(sn, 1), combine_ms=ct / max(cn, 1))


def bench_incremental(torch, hip, steps, warmup, Ts=(1, 4)):
    """Device-resident incremental decoding through one MHA layer at the C4
    cache shape: B=64 sequences, H=32 heads of D=128 (E=4096), a bf16 cache
    of 8192 positions holding ~U[512, 7900] per sequence. One step appends T
    new positions of every sequence (gonn_hip_mha_forward_incremental_dev:
    fp64 q/k/v projection, append, causal multi-token attend, merge, output
    projection, one host synchronisation). Weights and inputs are seeded
    N(0,1) (weights scaled by 1/sqrt(E))."""
    import numpy as np
    B, H, D, Lmax = 64, 32, 128, 8192
    E = H * D
    lens = np.random.default_rng(5).integers(512, 7900, B).astype(np.int32)
    g = torch.Generator(device="cuda")
    g.manual_seed(55)
    W = [(torch.randn((E, E), generator=g, device="cuda", dtype=torch.float64) / math.sqrt(E))
         .cpu().numpy() for _ in range(4)]
    bs = [np.zeros(E) for _ in range(4)]
    dev = hip.DeviceMHA(E, H, W[0], bs[0], W[1], bs[1], W[2], bs[2], W[3], bs[3])
    del W
    cache = hip.KVCache(B, H, Lmax, D)
    chunk = 1024
    for c0 in range(0, int(lens.max()), chunk):
        cnt = np.clip(lens - c0, 0, chunk).astype(np.int32)
        k = torch.randn((B, H, chunk, D), generator=g, device="cuda", dtype=torch.bfloat16)
        v = torch.randn((B, H, chunk, D), generator=g, device="cuda", dtype=torch.bfloat16)
        cache.append(k, v, counts=cnt)
        del k, v
    torch.cuda.synchronize()
    res = {"config": {"workload": "resident MHA incremental decoding over a bf16 KV cache",
                      "B": B, "H": H, "E": E, "D": D, "Lmax": Lmax,
                      "mean_len_at_start": float(lens.mean())}}
    for T in Ts:
        x = torch.randn((B, T, E), generator=g, device="cuda", dtype=torch.float64)
        out = torch.empty_like(x)
        ws = torch.empty(dev.incremental_workspace_bytes(cache, T), dtype=torch.uint8,
                         device="cuda")
        run = lambda: dev.forward_incremental_dev(x, cache, out=out, ws=ws)  # noqa: E731
        for _ in range(warmup):
            run()
        torch.cuda.synchronize()
        len0 = cache.lengths().astype(np.int64)
        ms, med, _ = _run_steps(torch, run, steps)
        hip.profile_reset()
        hip.profile_enable(True)
        _prime_queue(torch)
        for _ in range(steps):
            run()
        torch.cuda.synchronize()
        hip.profile_enable(False)
        st, sn = hip.profile_read("decode_causal_split")
        ct, cn = hip.profile_read("decode_causal_combine")
        hip.profile_reset()
        # attend bytes: every valid K and V row once per group of queries, at
        # the mean cache length of the profiled pass
        groups = -(-T // 4)
        mean_len = float((len0 + steps * T + steps * T / 2).mean())
        abytes = groups * 2 * H * D * 2 * mean_len * B
        split_ms = st / max(sn, 1)
        res[f"T{T}"] = {"ms_per_step": round(ms, 5), "median_ms_per_step": round(med, 5),
                        "tokens_per_s": round(B * T / (ms * 1e-3), 1),
                        "attend_split_ms": round(split_ms, 5),
                        "attend_combine_ms": round(ct / max(cn, 1), 5),
                        "attend_GBps": round(abytes / (split_ms * 1e-3) / 1e9, 2),
                        "attend_frac": round(abytes / (split_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        del x, out, ws
    cache.close()
    dev.close()
    return res


def _timed(torch, hip, run, steps, warmup, stages):
    """Mean ms per step over `steps` launches bracketed by events on the current
    stream, then a second pass with the library's per-stage event profiler;
    returns (ms_per_step, {stage: mean ms per launch})."""
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    ms, med, _ = _run_steps(torch, run, steps)
    hip.profile_reset()
    hip.profile_enable(True)
    _prime_queue(torch)
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    hip.profile_enable(False)
    per, launches = {}, {}
    for st in stages:
        t, n = hip.profile_read(st)
        per[st] = t / max(n, 1)
        launches[st] = max(n, 1) / steps
    hip.profile_reset()
    return (ms, med), per, launches


def bench_fwd_bwd(torch, hip, steps, warmup):
    """C5: causal flash forward + backward, B=2 H=16 S=8192 D=128, bf16 MFMA."""
    B, H, S, D = 2, 16, 8192, 128
    fwd_flop = 4.0 * B * H * S * S * D * 0.5
    bwd_flop = 2.5 * fwd_flop
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    q, k, v, do = (torch.randn((B * H, S, D), generator=g, device="cuda") for _ in range(4))
    o, lse = hip.attn_fwd(q, k, v, causal=True, mode="bf16")
    grads = tuple(torch.empty_like(q) for _ in range(3))

    def run():
        hip.attn_fwd(q, k, v, causal=True, mode="bf16", out=o, lse_out=lse)
        hip.attn_bwd(q, k, v, o, lse, do, causal=True, mode="bf16", out=grads)
    stages = ("pack_kv", "fwd_bf16", "bwd_prep", "bwd_pack", "bwd_dkdv", "bwd_dq")
    (ms, med), per, nl = _timed(torch, hip, run, steps, warmup, stages)
    # stage times per step (a stage may be several launches)
    per = {k: v * nl[k] for k, v in per.items()}
    # The other dQ path (S and dP formed again instead of the stored dS),
    # timed in the same run so the measuring box shows which default wins.
    prev = os.environ.get("GONN_HIP_BWD_DQ")
    os.environ["GONN_HIP_BWD_DQ"] = "recompute"
    try:
        (ms_rc, _), per_rc, nl_rc = _timed(torch, hip, run, steps, max(warmup // 2, 1), stages)
    finally:
        if prev is None:
            del os.environ["GONN_HIP_BWD_DQ"]
        else:
            os.environ["GONN_HIP_BWD_DQ"] = prev
    per_rc = {k: v * nl_rc[k] for k, v in per_rc.items()}
    return dict(B=B, H=H, S=S, D=D, fwd_flop=fwd_flop, bwd_flop=bwd_flop, ms=ms, median_ms=med,
                per=per, ms_recompute=ms_rc, per_recompute=per_rc)


def bench_encoder(torch, hip, steps, warmup, mode):
    """C2: non-causal encoder attention, B=8 H=12 S=1024 D=64, fp32 in/out."""
    B, H, S, D = 8, 12, 1024, 64
    flop = 4.0 * B * H * S * S * D
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    q, k, v = (torch.randn((B * H, S, D), generator=g, device="cuda") for _ in range(3))
    o = torch.empty_like(q)
    run = lambda: hip.attn_fwd(q, k, v, causal=False, mode=mode, out=o)  # noqa: E731
    kname = "fwd_bf16" if mode == "bf16" else "fwd_f32"
    (ms, med), per, nl = _timed(torch, hip, run, steps, warmup, ("pack_kv", kname))
    return dict(B=B, H=H, S=S, D=D, flop=flop, ms=ms, median_ms=med, kernel_ms=per[kname],
                pack_ms=per["pack_kv"], launches=nl[kname])


def bench_wide_gate(torch, hip, steps, warmup, kind):
    """The wider fused gate in bf16-MFMA mode, forward + backward:
    masked: C2's shape (B=8 H=12 S=1024 D=64, non-causal) with an additive
            (B, S, S) mask (WithAttnMask; N(0,1) bias, a blocked key band of
            -1e30), forward and backward read it;
    cross:  decoder cross-attention Forward(x, memory, memory, false),
            B=4 H=16 Sq=1024 Sk=4096 D=128."""
    if kind == "masked":
        B, H, Sq, Sk, D = 8, 12, 1024, 1024, 64
    else:
        B, H, Sq, Sk, D = 4, 16, 1024, 4096, 128
    fwd_flop = 4.0 * B * H * Sq * Sk * D
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    q, do = (torch.randn((B, H, Sq, D), generator=g, device="cuda") for _ in range(2))
    k, v = (torch.randn((B, H, Sk, D), generator=g, device="cuda") for _ in range(2))
    m = None
    if kind == "masked":
        m = torch.randn((B, Sq, Sk), generator=g, device="cuda")
        m[:, :, 100:140] = -1e30
    o, lse = hip.attn_fwd(q, k, v, mode="bf16", attn_mask=m)
    grads = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v))

    def run():
        hip.attn_fwd(q, k, v, mode="bf16", out=o, lse_out=lse, attn_mask=m)
        hip.attn_bwd(q, k, v, o, lse, do, mode="bf16", out=grads, attn_mask=m)
    (ms, med), per, nl = _timed(torch, hip, run, steps, warmup,
                                ("pack_kv", "fwd_bf16", "bwd_prep", "bwd_pack", "bwd_dkdv",
                                 "bwd_dq"))
    per = {k: v * nl[k] for k, v in per.items()}
    tot = 3.5 * fwd_flop
    return {"metric": "fwd+bwd TFLOP/s", "value": round(tot / (ms * 1e-3) / 1e12, 3),
            "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "median_ms_per_step": round(med, 4),
            "config": {"workload": f"{kind}: " + ("C2 shape + (B,S,S) additive mask"
                                                  if kind == "masked" else
                                                  "decoder cross-attention, Sq != Sk"),
                       "B": B, "H": H, "Sq": Sq, "Sk": Sk, "D": D, "causal": False,
                       "mode": "bf16", "fwd_flop": fwd_flop, "bwd_flop": 2.5 * fwd_flop},
            "fwd_TFLOPs": round(fwd_flop / (per["fwd_bf16"] * 1e-3) / 1e12, 3),
            "bwd_TFLOPs": round(2.5 * fwd_flop / ((per["bwd_dkdv"] + per["bwd_dq"]) * 1e-3)
                                / 1e12, 3),
            "stage_ms": {k: round(v, 5) for k, v in per.items()}}


def bench_mha(torch, hip, steps, warmup):
    """C1: MHA forward, three routes, ms per forward."""
    import numpy as np
    from gonn_amd import nn
    B, S, E, H = 2, 128, 256, 4
    rng = np.random.default_rng(20)
    s = 1.0 / math.sqrt(E)
    W = [rng.standard_normal((E, E)) * s for _ in range(4)]
    b = [rng.standard_normal(E) * s for _ in range(4)]
    x = rng.standard_normal((B, S, E)) * s
    mha = nn.MultiHeadAttention(E, H, W[0], b[0], W[1], b[1], W[2], b[2], W[3], b[3])
    hip.SetAttnMode("fp32")

    def wall(fn):
        for _ in range(warmup):
            fn()
        t = []
        for _ in range(steps):
            t0 = time.perf_counter()
            fn()
            t.append((time.perf_counter() - t0) * 1e3)
        return statistics.mean(t), statistics.median(t)

    host = wall(lambda: mha.forward_fused(x, x, x, True))
    res = mha.to_device()
    resident = wall(lambda: res.forward(x, x, x, True))
    xd = torch.from_numpy(x).cuda()
    ws = torch.empty(res.dev.workspace_bytes(B, S, S), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(xd)
    run = lambda: res.dev.forward_dev(xd, xd, xd, out=out, causal=True, ws=ws)  # noqa: E731
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    dev_ms, dev_med, _ = _run_steps(torch, run, steps)
    res.close()
    r = lambda v: round(v, 4)  # noqa: E731
    return {"config": {"workload": "C1 MHA forward, fp64 host data, fp32-MFMA core",
                       "B": B, "S": S, "E": E, "H": H, "causal": True},
            "unit": "ms per forward",
            "host_projections_fused_core": {"ms": r(host[0]), "median_ms": r(host[1])},
            "resident_host_data": {"ms": r(resident[0]), "median_ms": r(resident[1])},
            "resident_device_buffers": {"ms": r(dev_ms), "median_ms": r(dev_med)}}


# GoNN's published fused-forward numbers (fp64, head_dim 64, RTX 3060,
# benchmark/results/gonn_flash.json:7-82): GFLOP/s by (BH, S, causal).
REF_F64_GFLOPS = {(64, 512, False): 85.06, (32, 1024, False): 86.13, (16, 2048, False): 85.64,
                  (64, 512, True): 77.78, (32, 1024, True): 80.31, (16, 2048, True): 80.10}
PEAK_FP64_TFLOPS = 78.6  # MI355X dense fp64 (vector and matrix)


def bench_f64_reference(hip, iters=30):
    """The reference-named BenchFlashAttnF64 entry (gonn_cuda.cu:532-560's
    protocol: zero-filled device inputs, 5 warm-ups, one event pair around
    `iters` launches, mean ms) at the shapes GoNN publishes, d = 64, in the
    f64 entries' exact fp64 mode and in their default fp32-MFMA mode; FLOP
    by the reference's convention (4 BH S^2 d, halved when causal)."""
    prev = hip.AttnMode()
    rows = []
    try:
        for mode, peak in (("f64", PEAK_FP64_TFLOPS), ("fp32", PEAK_FP32_TFLOPS)):
            hip.SetAttnMode(mode)
            for (BH, S, causal), ref in REF_F64_GFLOPS.items():
                ms = hip.BenchFlashAttnF64(BH, S, 64, iters, causal)
                flop = 4.0 * BH * S * S * 64 * (0.5 if causal else 1.0)
                gf = flop / (ms * 1e-3) / 1e9
                rows.append({"mode": mode, "BH": BH, "S": S, "d": 64, "causal": causal,
                             "ms": round(ms, 5), "GFLOPs": round(gf, 1),
                             "frac": round(gf / 1e3 / peak, 4),
                             "reference_GFLOPs": ref, "vs_reference": round(gf / ref, 1)})
        # The exact-mode backward at the same shapes (no reference figure:
        # GoNN publishes no backward timing). FLOP: the five S^2 d products
        # (S, dP, dV, dK, dQ), 10 BH S^2 d, halved when causal.
        hip.SetAttnMode("f64")
        bwd = []
        for (BH, S, causal) in REF_F64_GFLOPS:
            ms = hip.BenchFlashAttnF64Bwd(BH, S, 64, iters, causal)
            gf = 10.0 * BH * S * S * 64 * (0.5 if causal else 1.0) / (ms * 1e-3) / 1e9
            bwd.append({"mode": "f64", "BH": BH, "S": S, "d": 64, "causal": causal,
                        "ms": round(ms, 5), "GFLOPs": round(gf, 1),
                        "frac": round(gf / 1e3 / PEAK_FP64_TFLOPS, 4)})
    finally:
        hip.SetAttnMode(prev)
    return {"metric": "fused forward GFLOP/s at GoNN's published shapes",
            "unit": "GFLOP/s",
            "note": "reference: GoNN's fp64 CUDA kernel on an RTX 3060 "
                    "(benchmark/results/gonn_flash.json); frac against the MI355X peak of the "
                    "mode (fp64 78.6 TFLOP/s, fp32 MFMA 157.3 TFLOP/s)",
            "rows": rows, "bwd_rows": bwd}


def cpu_baseline(pre, seconds):
    """Time GoNN's CPU attention core on a bounded sample of the prefill
    workload (whole (b,h) slices), two ways:

    * the returned line: the oracle's restatement of GoNN's own pass structure
      (oracle.attn_fwd_goflow: every tensor op a whole-tensor pass into a new
      buffer, broadcasts materialised, elementwise loops and reductions on one
      thread, GEMMs threaded across the host cores, as gonum's Dgemm is);
    * "threaded": the fused oracle (oracle.attn_fwd), whose score rows,
      softmax and P.V rows are all threaded -- faster than GoNN's CPU path,
      kept as an upper bound for a CPU port.
    """
    import numpy as np
    import oracle
    S, D, BH = pre["S"], pre["D"], pre["B"] * pre["H"]
    threads = oracle.get_threads()
    flop1 = 4.0 * S * S * D * 0.5

    def sl(a, i, j):
        return a[i:j].double().cpu().numpy()

    def timed(fn, chunk):
        t0 = time.perf_counter()
        fn(sl(pre["q"], 0, 1), sl(pre["k"], 0, 1), sl(pre["v"], 0, 1))
        t1 = time.perf_counter() - t0
        n = max(1, min(int(seconds / max(t1, 1e-3)), BH))
        dt = 0.0
        for i in range(0, n, chunk):
            j = min(n, i + chunk)
            q, k, v = sl(pre["q"], i, j), sl(pre["k"], i, j), sl(pre["v"], i, j)
            t0 = time.perf_counter()
            fn(q, k, v)
            dt += time.perf_counter() - t0
        return n, dt

    host = f"{cpu_model()} (nproc {os.cpu_count()})"
    n, dt = timed(lambda q, k, v: oracle.attn_fwd_goflow(q, k, v, causal=True), 2)
    n2, dt2 = timed(lambda q, k, v: oracle.attn_fwd(q, k, v, causal=True), BH)
    return {"value": flop1 * n / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{n} of {BH} (b,h) slices of C3 (S={S}, D={D}, causal), extrapolated to "
                      f"the whole workload (every slice does equal work), fp64, GoNN's "
                      f"op sequence and pass structure (MatMul, MulScalar, Add mask, Softmax as "
                      f"MaxAxis/Sub/Exp/SumAxis/Div, MatMul; broadcasts materialised), the two "
                      f"GEMMs threaded over {threads} threads, the elementwise passes and "
                      f"reductions on 1 thread; {dt:.1f} s on {host}, 2 slices per call; "
                      f"same FLOP convention as value",
            "seconds": dt,
            "threaded": {"value": flop1 * n2 / dt2 / 1e12, "cores": threads,
                         "sample": f"{n2} slices (extrapolated), fused per-row oracle with "
                                   f"scores, softmax and "
                                   f"P.V rows all threaded ({dt2:.1f} s); faster than GoNN's "
                                   f"CPU path"}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-bwd", action="store_true")
    ap.add_argument("--no-encoder", action="store_true")
    ap.add_argument("--no-mha", action="store_true")
    ap.add_argument("--no-incremental", action="store_true",
                    help="skip the resident incremental-decoding leg")
    ap.add_argument("--no-wide", action="store_true", help="skip the masked / cross legs")
    ap.add_argument("--no-f64", action="store_true",
                    help="skip the f64 entries at the reference's published shapes")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the headline leg (profiling runs of the other legs only)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run one device copy of 1 GiB, the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this attention core is measured on one GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE {world}) is not run. The (b,h) slices shard with no exchange; "
              "see the sharding paragraph of the design notes.", file=sys.stderr)
        sys.exit(2)

    import torch
    from gonn_amd import hip
    if not hip.Available():
        print("bench.py: no gfx950 device visible to libgonn_hip.so", file=sys.stderr)
        sys.exit(1)

    if args.copy_calib:
        n = 1 << 28  # 2^28 floats = 1 GiB read + 1 GiB written
        x = torch.ones(n, device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        y.copy_(x)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {4 * n} bytes read, {4 * n} bytes written")
        del x, y
    if args.no_prefill:
        if not args.no_decode:
            log("[bench] decode C4")
            bench_decode(torch, hip, args.steps, args.warmup)
        if not args.no_bwd:
            log("[bench] fwd+bwd C5")
            bench_fwd_bwd(torch, hip, args.steps, args.warmup)
        if not args.no_encoder:
            for mode in ("bf16", "fp32"):
                log(f"[bench] encoder C2 {mode}")
                bench_encoder(torch, hip, args.steps, args.warmup, mode)
        if not args.no_wide:
            for kind in ("masked", "cross"):
                log(f"[bench] wide gate {kind}")
                bench_wide_gate(torch, hip, max(args.steps // 5, 3), max(args.warmup // 2, 1),
                                kind)
        if not args.no_incremental:
            log("[bench] resident incremental decoding")
            bench_incremental(torch, hip, max(args.steps // 5, 5), max(args.warmup // 2, 2))
        return
    log("[bench] prefill C3")
    pre = bench_prefill(torch, hip, args.steps, args.warmup)
    tflops = pre["flop"] / (pre["ms"] * 1e-3) / 1e12
    ach = pre["flop"] / pre["launches"] / (pre["kernel_ms"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms"], 5),
        "median_ms_per_step": round(pre["median_ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) fp32 Q/K/V (torch cuda generator)",
        "config": {"workload": "C3 causal prefill forward, fp32 in/out, bf16 MFMA",
                   "B": pre["B"], "H": pre["H"], "S": pre["S"], "D": pre["D"], "causal": True,
                   "flop_per_step": pre["flop"], "wall_s": round(pre["wall_s"], 4)},
        "roofline": {"bound": "mfma", "achieved": round(ach, 3), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4),
                     "traffic": load_traffic("fwd_bf16:C3"), "kernel": "fwd_bf16_pipe_kernel",
                     "kernel_ms": round(pre["kernel_ms"], 5),
                     "launches_per_step": pre["launches"],
                     "pack_kv_ms": round(pre["pack_ms"], 5)},
    }
    log("[bench] calibration")
    line["calibration"] = calibration(torch, hip, pre["sclk_ghz"])
    # The kernel against the MFMA rate this box sustains on random operands.
    rnd = line["calibration"]["mfma_random_TFLOPs"]
    line["roofline"]["frac_of_mfma_random"] = round(ach / rnd, 4) if rnd > 0 else None
    if not args.no_decode:
        log("[bench] decode C4")
        dec = bench_decode(torch, hip, args.steps, args.warmup)
        gbs = dec["bytes"] / (dec["ms"] * 1e-3) / 1e9
        kgbs = dec["bytes"] / (dec["split_ms"] * 1e-3) / 1e9
        line["decode"] = {
            "metric": "decode HBM GB/s", "value": round(gbs, 2), "unit": "GB/s",
            "ms_per_step": round(dec["ms"], 5), "median_ms_per_step": round(dec["median_ms"], 5),
            "bytes_per_step": dec["bytes"],
            "config": {"workload": "C4 split-KV decode, bf16 cache", "B": dec["B"],
                       "H": dec["H"], "Lmax": dec["Lmax"], "D": dec["D"],
                       "mean_len": dec["mean_len"]},
            "roofline": {"bound": "hbm", "achieved": round(kgbs, 2), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(kgbs / PEAK_HBM_GBS, 4),
                         "traffic": load_traffic("decode_split:C4"),
                         "kernel": "decode_split_kernel",
                         "kernel_ms": round(dec["split_ms"], 5),
                         "combine_ms": round(dec["combine_ms"], 5)},
        }
    if not args.no_bwd:
        log("[bench] fwd+bwd C5")
        fb = bench_fwd_bwd(torch, hip, max(args.steps // 5, 3), max(args.warmup // 2, 1))
        per = fb["per"]
        bwd_ms = sum(per[k] for k in ("bwd_prep", "bwd_pack", "bwd_dkdv", "bwd_dq"))
        tot = fb["fwd_flop"] + fb["bwd_flop"]
        line["fwd_bwd"] = {
            "metric": "causal fwd+bwd TFLOP/s", "value": round(tot / (fb["ms"] * 1e-3) / 1e12, 3),
            "unit": "TFLOP/s", "ms_per_step": round(fb["ms"], 4),
            "median_ms_per_step": round(fb["median_ms"], 4),
            "config": {"workload": "C5 causal flash fwd+bwd, fp32 in/out, bf16 MFMA",
                       "B": fb["B"], "H": fb["H"], "S": fb["S"], "D": fb["D"],
                       "fwd_flop": fb["fwd_flop"], "bwd_flop": fb["bwd_flop"]},
            "bwd_TFLOPs": round(fb["bwd_flop"] / (bwd_ms * 1e-3) / 1e12, 3),
            "stage_ms": {k: round(v, 5) for k, v in per.items()},
            "dq_paths": {
                "default": "stored dS (one GEMM)", "stored_ds_dq_ms": round(per["bwd_dq"], 5),
                "stored_ds_dkdv_ms": round(per["bwd_dkdv"], 5),
                "recompute_dq_ms": round(fb["per_recompute"]["bwd_dq"], 5),
                "recompute_dkdv_ms": round(fb["per_recompute"]["bwd_dkdv"], 5),
                "recompute_step_ms": round(fb["ms_recompute"], 4),
                "note": "GONN_HIP_BWD_DQ=recompute: dK/dV stores no dS and the dQ kernel forms "
                        "S and dP again; both paths timed in this run"},
            "roofline": {"bound": "mfma", "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "kernel": "bwd_dkdv + bwd_dq",
                         "traffic": (load_traffic("bwd_dkdv:C5") or 0) + (load_traffic("bwd_dq:C5") or 0)
                         or None,
                         "achieved": round(fb["bwd_flop"] / ((per["bwd_dkdv"] + per["bwd_dq"])
                                                             * 1e-3) / 1e12, 3),
                         "frac": round(fb["bwd_flop"] / ((per["bwd_dkdv"] + per["bwd_dq"]) * 1e-3)
                                       / 1e12 / PEAK_BF16_TFLOPS, 4)},
        }
    if not args.no_encoder:
        line["encoder"] = {}
        for mode, peak in (("bf16", PEAK_BF16_TFLOPS), ("fp32", PEAK_FP32_TFLOPS)):
            log(f"[bench] encoder C2 {mode}")
            en = bench_encoder(torch, hip, args.steps, args.warmup, mode)
            ach = en["flop"] / en["launches"] / (en["kernel_ms"] * 1e-3) / 1e12
            line["encoder"][mode] = {
                "value": round(en["flop"] / (en["ms"] * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
                "ms_per_step": round(en["ms"], 5), "median_ms_per_step": round(en["median_ms"], 5),
                "config": {"workload": f"C2 encoder non-causal, fp32 in/out, {mode} MFMA",
                           "B": en["B"], "H": en["H"], "S": en["S"], "D": en["D"]},
                "roofline": {"bound": "mfma", "achieved": round(ach, 3), "peak": peak,
                             "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                             "kernel_ms": round(en["kernel_ms"], 5),
                             "launches_per_step": en["launches"],
                             "pack_kv_ms": round(en["pack_ms"], 5)}}
    if not args.no_wide:
        line["wide_gate"] = {}
        for kind in ("masked", "cross"):
            log(f"[bench] wide gate {kind}")
            line["wide_gate"][kind] = bench_wide_gate(torch, hip, max(args.steps // 5, 3),
                                                      max(args.warmup // 2, 1), kind)
    if not args.no_f64:
        log("[bench] f64 entries at the reference's shapes")
        line["f64_reference_shapes"] = bench_f64_reference(hip)
    if not args.no_mha:
        log("[bench] MHA C1")
        line["mha"] = bench_mha(torch, hip, args.steps, args.warmup)
    if not args.no_incremental:
        log("[bench] resident incremental decoding")
        line["kv_incremental"] = bench_incremental(torch, hip, max(args.steps // 5, 5),
                                                   max(args.warmup // 2, 2))
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline(pre, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
