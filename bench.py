#!/usr/bin/env python3
"""Benchmark of the gfx950 numeric backend on BASELINE.json's headline metric.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--only fa,fa_cases,fd,i8,mlp,llama,mv,cmp,regions]
                  (also: copy = counter calibration, vendor = ROCm library kernels for context)

One step = one launch of the hot path over one batch of synthetic, seeded
input already resident in HBM.  The headline (`value`) is the FA prefill
config (bf16 Q,K,V [1,16,2048,128], causal) in TFLOP/s of
algorithmic (causal, visible-pair) work; FD decode (config 2), the int8 GEMM
(config 3), the fp32 MLP block (config 0) and the decoder layer (config 4)
are reported in `secondary`,
each with its own roofline fraction and CPU baseline; so are the movement
commands, the comparator, and the elementwise command with the fused regions
at HBM scale (`regions`).  Timing: W untimed
launches, then exactly K launches captured into one HIP graph, replayed
untimed for SETTLE_S seconds so the GPU clocks settle, and replayed once
between two HIP events on the stream the kernels run on (the backend binds
torch's current stream at each call, the capture stream during capture).

cpu_baseline: the CPU oracle (oracle/, a C restatement of the Reference
backend's semantics, test infrastructure) timed on this host's cores over a
bounded sample of the same workload, scaled to the metric's unit.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK = {"bf16": 2500.0, "i8": 5000.0, "f32": 157.3, "hbm": 8000.0}  # TFLOP/s, TOP/s, GB/s

FA_SHAPE = (1, 16, 2048, 128)
FA_FLOPS = 4 * 16 * 128 * (2048 * 2049 // 2)           # 17,188,257,792
FA_BYTES = 4 * 1 * 16 * 2048 * 128 * 2                  # Q, K, V, O
FD_B, FD_HQ, FD_HKV, FD_L, FD_D, FD_CHUNKS = 32, 32, 8, 8192, 128, 16
FD_BYTES = 2 * FD_B * FD_HKV * FD_L * FD_D * 2 + 2 * FD_B * FD_HQ * FD_D * 2  # 1,074,266,112
FD_FLOPS = 4 * FD_B * FD_HQ * FD_L * FD_D
I8_N = 4096
I8_OPS = 2 * I8_N ** 3
MLP_FLOPS = 2 * 128 * 512 * 2048 * 2
SEED = 20260803
COPY_BYTES = 1 << 30


def cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


TRAFFIC_SOURCE = ("read from profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this kernel, "
                  "calibrated on a copy kernel, measured offline (not in this run)")


def traffic_for(kernel: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), if committed.  The bench
    itself does not run the counters (they need their own profiler pass);
    the roofline carries TRAFFIC_SOURCE next to the figure."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get(kernel, {}).get("bytes_per_launch")
    except (ValueError, OSError):
        return None


def cpu_time(fn):
    """Wall seconds of one call of fn (the CPU oracle over a bounded sample)."""
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0


def cpu_gbs(nbytes, dt, sample, cores_used=1):
    """cpu_baseline record for an HBM-class leg: algorithmic bytes of the
    sample / wall time."""
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": cores_used, "kind": "port",
            "sample": f"{sample}, {dt:.3f} s wall"}


SETTLE_S = 0.3  # untimed replays before the timed one: the GPU's clocks
                # take tens of milliseconds of sustained load to settle


def timed(torch, fn, steps: int, warmup: int) -> float:
    """Average milliseconds per step over exactly `steps` steps.

    The W warmup steps run eagerly (they also size the backend's workspace).
    The K timed steps are captured once into a HIP graph; the graph is
    replayed untimed for at least SETTLE_S seconds (the clocks of an idle
    GPU ramp up over tens of milliseconds of load; a short warmup times the
    ramp, not the kernel), then one replay is timed between two HIP events
    on the replay stream, so the figure is the GPU's time for K back-to-back
    steps, free of the Python binding's per-call host cost (a C++ caller of
    the C ABI does not pay it)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for _ in range(steps):
                fn()
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()  # untimed: first replay uploads the graph
    torch.cuda.synchronize()
    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        graph.replay()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def rnd_bf16(torch, gen, shape):
    return torch.randn(shape, device="cuda", generator=gen).to(torch.bfloat16)


# ---------------------------------------------------------------- workloads
def bench_fa(torch, hip, steps, warmup, with_cpu=True):
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    q, k, v = (rnd_bf16(torch, gen, FA_SHAPE) for _ in range(3))
    o = torch.empty(FA_SHAPE, dtype=torch.bfloat16, device="cuda")
    scale = 1.0 / math.sqrt(FA_SHAPE[3])
    ms = timed(torch, lambda: hip.attention_prefill(q, k, v, o, scale, causal=True), steps, warmup)
    achieved = FA_FLOPS / (ms * 1e-3) / 1e12
    res = {
        "ms": ms, "value": achieved,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK["bf16"], "unit": "TFLOP/s",
                     "frac": achieved / PEAK["bf16"], "traffic": traffic_for("fa_prefill"), "traffic_source": TRAFFIC_SOURCE},
    }
    if with_cpu:
        from oracle import oracle as orc
        heads = 4
        qs, ks, vs = (t[:, :heads].contiguous().cpu().view(torch.int16).numpy().view("uint16") for t in (q, k, v))
        t0 = time.perf_counter()
        orc.attention_prefill(qs, ks, vs, scale, causal=True, block_k=64, nthreads=cores())
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": (FA_FLOPS * heads / 16) / dt / 1e12, "unit": "TFLOP/s", "cores": cores(),
                               "kind": "port",
                               "sample": f"{heads} of 16 heads of the same causal [2048,128] bf16 prefill "
                                         f"(block_k 64), {dt:.2f} s wall"}
    return res


def causal_flops(heads, s, d):
    """Algorithmic FLOPs of causal attention: 4*d per visible (q, k) pair."""
    return 4 * heads * d * (s * (s + 1) // 2)


TX81_28x2048_MS = 3.649  # docs/attention-optimization-retrospective.md:9 (TX81, 16 tiles)


def bench_fa_cases(torch, hip, steps, warmup, with_cpu=True):
    """FA on the shapes and formats the reference's own attention cases use:
    config 1 in F16 through the plain entry (the dedicated head_dim-128
    kernel), config 1 through the masked entry in F16 and BF16 (the fa_fwd
    kernels, which serve every masked / windowed / valid-prefix case),
    attention-prefill at the cases' default head_dim 64 (q = kv = 1024, one
    head, causal; wafer_pytorch_board_cases.py:34, 1058-1070), and the
    TX81 retrospective's [1,28,2048,128] bf16 causal shape, next to its
    published 3.649 ms."""
    from vibe_compiler_amd.backend import BF16, F16

    gen = torch.Generator(device="cuda").manual_seed(SEED)
    legs = []

    def leg(name, kernel, shape, fmt, masked, ref_ms=None):
        dt = torch.bfloat16 if fmt == BF16 else torch.float16
        q, k, v = (torch.randn(shape, device="cuda", generator=gen).to(dt) for _ in range(3))
        o = torch.empty(shape, dtype=dt, device="cuda")
        scale = 1.0 / math.sqrt(shape[3])
        if masked:
            fn = lambda: hip.attention_prefill_masked(q, k, v, o, scale, causal=True, fmt=fmt)  # noqa: E731
        else:
            fn = lambda: hip.attention_prefill(q, k, v, o, scale, causal=True, fmt=fmt)  # noqa: E731
        ms = timed(torch, fn, steps, warmup)
        fl = causal_flops(shape[0] * shape[1], shape[2], shape[3])
        tf = fl / (ms * 1e-3) / 1e12
        e = {"name": name, "kernel": kernel, "workload": f"{'F16' if fmt == F16 else 'BF16'} Q,K,V {list(shape)} causal",
             "ms": ms, "value": tf, "unit": "TFLOP/s", "algorithmic_flops": fl,
             "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK["bf16"], "unit": "TFLOP/s",
                          "frac": tf / PEAK["bf16"], "traffic": None}}
        if ref_ms is not None:
            e["reference_published_ms"] = ref_ms
            e["speedup_vs_reference_published"] = ref_ms / ms
        if with_cpu:
            # the oracle of the same entry (masked: the masked-attention
            # restatement) on a bounded sample of the heads
            from oracle import oracle as orc
            heads = min(shape[1], 4)
            qs, ks, vs = (t[:, :heads].contiguous().cpu().view(torch.int16).numpy().view("uint16") for t in (q, k, v))
            t0 = time.perf_counter()
            if masked:
                orc.attention_prefill_ex(qs, ks, vs, scale, causal=True, fmt=fmt, nthreads=cores())
            else:
                orc.attention_prefill(qs, ks, vs, scale, causal=True, block_k=64, fmt=fmt, nthreads=cores())
            cdt = time.perf_counter() - t0
            e["cpu_baseline"] = {"value": fl * heads / shape[1] / cdt / 1e12, "unit": "TFLOP/s", "cores": cores(),
                                 "kind": "port",
                                 "sample": f"{heads} of {shape[1]} heads of the same shape, {cdt:.2f} s wall"}
        legs.append(e)

    leg("fa_prefill_f16_config1", "fa_prefill_d128<_Float16, true, false>", FA_SHAPE, F16, False)
    leg("fa_fwd_bf16_config1", "fa_fwd<__bf16, 128, MASK_CAUSAL>", FA_SHAPE, BF16, True)
    leg("fa_fwd_f16_config1", "fa_fwd<_Float16, 128, MASK_CAUSAL>", FA_SHAPE, F16, True)
    leg("attention_prefill_d64_1024_f16", "fa_fwd<_Float16, 64, MASK_CAUSAL>", (1, 1, 1024, 64), F16, False)
    leg("attention_prefill_d64_1024_bf16", "fa_fwd<__bf16, 64, MASK_CAUSAL>", (1, 1, 1024, 64), BF16, False)
    leg("tx81_28x2048_bf16", "fa_prefill_d128<__bf16, true, false>", (1, 28, 2048, 128), BF16, False,
        ref_ms=TX81_28x2048_MS)
    return {"workload": "FA prefill on the reference's attention-case shapes and formats", "legs": legs}


def bench_fd(torch, hip, steps, warmup, with_cpu=True):
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    q = rnd_bf16(torch, gen, (FD_B, FD_HQ, 1, FD_D))
    k = rnd_bf16(torch, gen, (FD_B, FD_HKV, FD_L, FD_D))
    v = rnd_bf16(torch, gen, (FD_B, FD_HKV, FD_L, FD_D))
    o = torch.empty((FD_B, FD_HQ, 1, FD_D), dtype=torch.bfloat16, device="cuda")
    scale = 1.0 / math.sqrt(FD_D)
    ms = timed(torch, lambda: hip.attention_decode(q, k, v, o, scale, chunks=FD_CHUNKS), steps, warmup)
    gbs = FD_BYTES / (ms * 1e-3) / 1e9
    res = {
        "workload": "FD decode bf16 Q[32,32,1,128] KV[32,8,8192,128] GQA 32/8, 16 chunks, LSE fold",
        "metric": "HBM GB/s", "ms": ms, "value": gbs, "unit": "GB/s", "tflops": FD_FLOPS / (ms * 1e-3) / 1e12,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK["hbm"], "unit": "GB/s",
                     "frac": gbs / PEAK["hbm"], "traffic": traffic_for("fd_decode"), "traffic_source": TRAFFIC_SOURCE},
    }
    if with_cpu:
        from oracle import oracle as orc
        nb = 8
        qs, ks, vs = (t[:nb].contiguous().cpu().view(torch.int16).numpy().view("uint16") for t in (q, k, v))
        t0 = time.perf_counter()
        orc.attention_decode(qs, ks, vs, scale, chunks=FD_CHUNKS, block_k=64, nthreads=cores())
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": (FD_BYTES * nb / FD_B) / dt / 1e9, "unit": "GB/s", "cores": cores(),
                               "kind": "port",
                               "sample": f"{nb} of 32 sequences of the same decode, {dt:.2f} s wall"}
    return res


def bench_i8(torch, hip, steps, warmup, with_cpu=True):
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    n = I8_N
    a = torch.randint(-127, 128, (n, n), device="cuda", generator=gen, dtype=torch.int8)
    b = torch.randint(-127, 128, (n, n), device="cuda", generator=gen, dtype=torch.int8)
    scale = torch.rand(n, device="cuda", generator=gen) * 0.009 + 0.001
    y = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
    ms = timed(torch, lambda: hip.gemm_i8(a, b, scale, y, n, n, n), steps, warmup)
    tops = I8_OPS / (ms * 1e-3) / 1e12
    res = {
        "workload": "int8 GEMM 4096^3 (rhs [K,N]), exact int32 accumulate, per-column f32 dequant, bf16 out",
        "metric": "TOP/s", "ms": ms, "value": tops, "unit": "TOP/s",
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK["i8"], "unit": "TOP/s",
                     "frac": tops / PEAK["i8"], "traffic": traffic_for("gemm_i8"), "traffic_source": TRAFFIC_SOURCE},
    }
    if with_cpu:
        from oracle import oracle as orc
        rows = 256
        an, bn, sn = a[:rows].cpu().numpy(), b.cpu().numpy(), scale.cpu().numpy()
        t0 = time.perf_counter()
        orc.gemm_i8(an, bn, sn, rows, n, n, nthreads=cores(), want_acc=False)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": (2 * rows * n * n) / dt / 1e12, "unit": "TOP/s", "cores": cores(),
                               "kind": "port", "sample": f"{rows} of 4096 output rows, {dt:.2f} s wall"}
    return res


def bench_mlp(torch, hip, B, steps, warmup, with_cpu=True, lane="mfma"):
    """BASELINE config 0.  lane "mfma": two wafer_hip_gemm_f32_mfma calls with
    the bias (+ tanh-GELU) regions in their epilogues (tolerance class, C1's
    1e-4 relative); lane "formal": the bit-exact formal GEMM order with
    separate bias_add / gelu_tanh region launches."""
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    x = torch.randn((128, 512), device="cuda", generator=gen)
    w1 = torch.randn((512, 2048), device="cuda", generator=gen) / math.sqrt(512)
    b1 = torch.randn(2048, device="cuda", generator=gen) * 0.02
    w2 = torch.randn((2048, 512), device="cuda", generator=gen) / math.sqrt(2048)
    b2 = torch.randn(512, device="cuda", generator=gen) * 0.02
    hbuf = torch.empty((128, 2048), device="cuda")
    y = torch.empty((128, 512), device="cuda")

    def step_formal():
        hip.gemm(x, w1, hbuf, 128, 512, 2048)
        hip.bias_add(hbuf, b1, hbuf, fmt=B.F32)
        hip.gelu_tanh(hbuf, hbuf, fmt=B.F32)
        hip.gemm(hbuf, w2, y, 128, 2048, 512)
        hip.bias_add(y, b2, y, fmt=B.F32)

    def step_mfma():
        hip.gemm_f32_mfma(x, w1, hbuf, 128, 512, 2048, bias=b1, epilogue=B.EPILOGUE_BIAS_GELU_TANH)
        hip.gemm_f32_mfma(hbuf, w2, y, 128, 2048, 512, bias=b2, epilogue=B.EPILOGUE_BIAS)

    if lane == "mfma":
        step_mfma()  # grows the split-k partial area before any graph capture
        torch.cuda.synchronize()
    ms = timed(torch, step_mfma if lane == "mfma" else step_formal, steps, warmup)
    tf = MLP_FLOPS / (ms * 1e-3) / 1e12
    res = {
        "workload": ("fp32 MLP block x[128,512] W1[512,2048] W2[2048,512] tanh-GELU, "
                     + ("f32 MFMA GEMMs with fused bias/GELU epilogues (tolerance class)" if lane == "mfma"
                        else "formal (bit-exact) GEMM order")),
        "metric": "TFLOP/s", "ms": ms, "value": tf, "unit": "TFLOP/s",
        "roofline": {"bound": "mfma" if lane == "mfma" else "valu-f32", "achieved": tf, "peak": PEAK["f32"],
                     "unit": "TFLOP/s", "frac": tf / PEAK["f32"], "traffic": None},
    }
    if with_cpu:
        from oracle import oracle as orc
        xn, w1n, w2n, b1n, b2n = (t.cpu().numpy() for t in (x, w1, w2, b1, b2))
        t0 = time.perf_counter()
        h1 = orc.gemm_formal(5, 5, xn, w1n, 128, 512, 2048, nthreads=cores()).reshape(128, 2048)
        h1 = orc.gelu_tanh(orc.bias_add(h1, b1n), fmt=5)
        orc.bias_add(orc.gemm_formal(5, 5, h1, w2n, 128, 2048, 512, nthreads=cores()).reshape(128, 512), b2n)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": MLP_FLOPS / dt / 1e12, "unit": "TFLOP/s", "cores": cores(),
                               "kind": "port", "sample": f"the whole block, {dt:.2f} s wall"}
    return res


def bench_llama(torch, hip, steps, warmup, with_cpu=True):
    """one Llama-style decoder layer forward, [1,1024,4096]
    bf16, GQA 32/8, FFN 14336, through vibe_compiler_amd.decoder_layer."""
    from vibe_compiler_amd import decoder_layer as DL

    gen = torch.Generator(device="cuda").manual_seed(SEED)
    W = DL.random_weights(torch, gen)
    x = torch.randn((1024, 4096), device="cuda", generator=gen).to(torch.bfloat16)
    y = torch.empty_like(x)
    layer = DL.DecoderLayer(hip, W, 1024)
    ms = timed(torch, lambda: layer.forward(x, y), steps, warmup)
    fl = DL.flops()
    tf = fl / (ms * 1e-3) / 1e12
    res = {
        "workload": "Llama-style decoder layer x[1,1024,4096] bf16, GQA 32/8 (head_dim 128), FFN 14336, "
                    "RMSNorm eps 1e-5, RoPE theta 1e4, causal; weights ~N(0,0.02) bf16",
        "metric": "TFLOP/s", "ms": ms, "value": tf, "unit": "TFLOP/s",
        "roofline": {"bound": "mfma", "achieved": tf, "peak": PEAK["bf16"], "unit": "TFLOP/s",
                     "frac": tf / PEAK["bf16"], "traffic": None},
    }
    if with_cpu:
        from oracle import oracle as orc
        rows = 16
        h = x[:rows].contiguous().cpu().view(torch.int16).numpy().view("uint16")
        mats = [W[n].cpu().view(torch.int16).numpy().view("uint16") for n in ("wqkv", "wo", "wgate", "wup")]
        wd = W["wdown"].cpu().view(torch.int16).numpy().view("uint16")
        act = np.zeros((rows, 14336), dtype=np.uint16)
        t0 = time.perf_counter()
        for w in mats:
            orc.gemm_formal(3, 3, h, w, rows, 4096, w.shape[0], rhs_t=True, nthreads=cores())
        orc.gemm_formal(3, 3, act, wd, rows, 14336, 4096, rhs_t=True, nthreads=cores())
        dt = time.perf_counter() - t0
        sample = 2 * rows * 218_103_808
        res["cpu_baseline"] = {"value": sample / dt / 1e12, "unit": "TFLOP/s", "cores": cores(), "kind": "port",
                               "sample": f"the seven projection GEMMs (97% of the layer's FLOPs) for {rows} of "
                                         f"1024 tokens on the formal-order lane, {dt:.2f} s wall"}
    return res


def bench_mv(torch, hip, steps, warmup, with_cpu=True):
    """Movement commands: a strided tile gather (RDMA shape: 131072 rows of
    4 KiB out of an 8 KiB-pitch matrix into a dense tile, 512 MiB payload,
    working set above the 256 MB last-level cache) and
    a 2-byte-element transpose of a 16384 x 16384 bf16 matrix (gather-scatter,
    512 MiB payload).  Algorithmic bytes = payload read + payload written."""
    rows, pitch, inner = 131072, 8192, 4096
    src = torch.randint(0, 256, (rows * pitch,), dtype=torch.uint8, device="cuda")
    tile = torch.empty(rows * inner, dtype=torch.uint8, device="cuda")
    ms = timed(torch, lambda: hip.strided_copy(src, tile, inner, [pitch, 0, 0], [rows, 1, 1], [inner, 0, 0],
                                               [rows, 1, 1]), steps, warmup)
    gbs = 2 * rows * inner / (ms * 1e-3) / 1e9
    n = 16384
    x = torch.randint(-32768, 32767, (n, n), dtype=torch.int16, device="cuda")
    t = torch.empty_like(x)
    ms_t = timed(torch, lambda: hip.strided_copy(x, t, 2, [2, 2 * n, 0], [n, n, 1], [2 * n, 2, 0], [n, n, 1]),
                 steps, warmup)
    gbs_t = 2 * n * n * 2 / (ms_t * 1e-3) / 1e9
    cpu = None
    if with_cpu:
        from oracle import oracle as orc
        rs = 16384  # 16384 rows of the gather (64 MiB payload)
        src_s = src[: rs * pitch].cpu().numpy()
        dst_s = np.zeros(rs * inner, np.uint8)
        dt = cpu_time(lambda: orc.strided_copy(src_s, dst_s, inner, [pitch, 0, 0], [rs, 1, 1], [inner, 0, 0],
                                               [rs, 1, 1]))
        cpu = cpu_gbs(2 * rs * inner, dt, f"{rs} of {rows} rows of the same gather (scalar C oracle)")
        nt = 4096  # a 4096 x 4096 corner of the transpose
        xs = x[:nt, :nt].contiguous().cpu().numpy().view(np.uint8).reshape(-1)
        dt_t = cpu_time(lambda: orc.strided_copy(xs, np.zeros_like(xs), 2, [2, 2 * nt, 0], [nt, nt, 1],
                                                 [2 * nt, 2, 0], [nt, nt, 1]))
        cpu_t = cpu_gbs(2 * nt * nt * 2, dt_t, f"a {nt} x {nt} bf16 transpose (scalar C oracle)")
    return {
        "workload": "strided tile gather 131072 x 4 KiB segments at 8 KiB pitch -> dense (512 MiB payload)",
        "metric": "GB/s", "ms": ms, "value": gbs, "unit": "GB/s",
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK["hbm"], "unit": "GB/s",
                     "frac": gbs / PEAK["hbm"], "traffic": None},
        "cpu_baseline": cpu,
        "transpose": {"workload": "bf16 16384 x 16384 transpose, 2-byte segments (512 MiB payload)", "ms": ms_t,
                      "value": gbs_t, "unit": "GB/s", "frac": gbs_t / PEAK["hbm"],
                      "cpu_baseline": cpu_t if with_cpu else None},
    }


def bench_cmp(torch, hip, steps, warmup, with_cpu=True):
    """Program-boundary comparator on a 256M-element bf16 pair (512 MiB each,
    above the 256 MB last-level cache): the output gate (one statistics pass)
    and the full error statistics (that pass plus the radix-selection passes
    for the p99/p999 quantiles).  Both entries end with a host
    synchronisation, so they are timed per call, host time included."""
    n = 256 << 20
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    x = torch.randn(n, device="cuda", generator=gen)
    y = (x * (1 + 1e-3 * torch.randn(n, device="cuda", generator=gen))).to(torch.bfloat16)
    x = x.to(torch.bfloat16)
    a, e = (10, y.view(torch.uint8), (n,)), (10, x.view(torch.uint8), (n,))

    def per_call(fn):
        for _ in range(max(1, warmup // 5)):
            fn()
        torch.cuda.synchronize()
        k = max(1, steps // 5)
        t0 = time.perf_counter()
        for _ in range(k):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / k

    ms_gate = per_call(lambda: hip.compare_expected(a, e, 0.008, 0.006, (0.9999, 0.01)))
    ms_elem = per_call(lambda: hip.compare_expected(a, e, 0.008, 0.006))
    ms_stats = per_call(lambda: hip.compare_statistics(a, e, 0.008, 0.006))
    gbs = 2 * n * 2 / (ms_gate * 1e-3) / 1e9
    cpu = cpu_s = None
    if with_cpu:
        from oracle import oracle as orc
        ns = 16 << 20  # 16M-element sample of the same pair
        ya, xe = y[:ns].cpu().view(torch.uint8).numpy(), x[:ns].cpu().view(torch.uint8).numpy()
        dt = cpu_time(lambda: orc.compare_expected((10, (ns,), ya), (10, (ns,), xe), 0.008, 0.006, (0.9999, 0.01)))
        cpu = cpu_gbs(2 * ns * 2, dt, f"{ns} of {n} elements of the same bf16 pair (scalar C oracle)")
        nq = 4 << 20  # the statistics' quantile selection is the slow part: a 4M-element sample
        dt_s = cpu_time(lambda: orc.compare_statistics((10, (nq,), ya[:2 * nq]), (10, (nq,), xe[:2 * nq]), 0.008,
                                                       0.006))
        cpu_s = {"elements_per_s": nq / dt_s, "cores": 1, "kind": "port",
                 "sample": f"{nq} elements of the same pair, {dt_s:.3f} s wall"}
    return {
        "workload": "comparator gate (similarity policy) on a bf16 pair of 268,435,456 elements",
        "metric": "GB/s", "ms": ms_gate, "value": gbs, "unit": "GB/s",
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK["hbm"], "unit": "GB/s",
                     "frac": gbs / PEAK["hbm"], "traffic": None},
        "cpu_baseline": cpu,
        "elementwise_gate": {"ms": ms_elem, "value": 2 * n * 2 / (ms_elem * 1e-3) / 1e9, "unit": "GB/s"},
        "statistics": {"workload": "full statistics incl. nearest-rank p99/p999 of |error| and ULP",
                       "ms": ms_stats, "elements_per_s": n / (ms_stats * 1e-3), "cpu_baseline": cpu_s},
    }


def bench_vendor(torch, hip, steps, warmup):
    """ROCm's own kernels on the same shapes, timed the same way, as context
    for the roofline fractions (not part of the headline): torch SDPA
    restricted to its flash / memory-efficient backends (never the math path)
    for config 1, hipBLASLt through torch.matmul for a bf16 4096^3 GEMM next
    to this backend's MFMA GEMM, and torch._int_mm for the int8 4096^3
    product (int32 out, no dequant) next to this backend's int8 GEMM with the
    rhs already in [N,K] form."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import torch.nn.functional as F
    from vibe_compiler_amd.backend import BF16

    gen = torch.Generator(device="cuda").manual_seed(SEED)
    out = {}

    def record(name, fn, work, unit):
        try:
            ms = timed(torch, fn, steps, warmup)
            out[name] = {"ms": ms, "value": work / (ms * 1e-3) / 1e12, "unit": unit}
        except Exception as e:  # a backend the installed torch does not offer
            out[name] = {"error": f"{type(e).__name__}: {str(e)[:160]}"}

    q, k, v = (rnd_bf16(torch, gen, FA_SHAPE) for _ in range(3))
    scale = 1.0 / math.sqrt(FA_SHAPE[3])
    for name, be in (("sdpa_flash", SDPBackend.FLASH_ATTENTION), ("sdpa_efficient", SDPBackend.EFFICIENT_ATTENTION)):
        def fa_fn(be=be):
            with sdpa_kernel([be]):
                F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
        record(name, fa_fn, FA_FLOPS, "TFLOP/s")
    del q, k, v
    n = I8_N
    a = rnd_bf16(torch, gen, (n, n))
    b = rnd_bf16(torch, gen, (n, n))
    bt = b.t().contiguous()
    y = torch.empty((n, n), dtype=torch.bfloat16, device="cuda")
    record("hipblaslt_bf16_mm", lambda: torch.matmul(a, b), I8_OPS, "TFLOP/s")
    record("wafer_bf16_mfma_nt", lambda: hip.gemm_mfma(a, bt, y, n, n, n, in_fmt=BF16, out_fmt=BF16, rhs_t=True),
           I8_OPS, "TFLOP/s")
    ai = torch.randint(-127, 128, (n, n), device="cuda", generator=gen, dtype=torch.int8)
    bi = torch.randint(-127, 128, (n, n), device="cuda", generator=gen, dtype=torch.int8)
    bit = bi.t().contiguous()
    sc = torch.rand(n, device="cuda", generator=gen) * 0.009 + 0.001
    record("torch_int_mm", lambda: torch._int_mm(ai, bi), I8_OPS, "TOP/s")
    record("wafer_i8_nt", lambda: hip.gemm_i8(ai, bit, sc, y, n, n, n, rhs_t=True), I8_OPS, "TOP/s")
    return {"workload": "ROCm library kernels on config 1 and 4096^3 GEMM shapes (context only)", **out}


REGION_ROWS, REGION_COLS = 65536, 4096  # 256M elements: 512 MiB per bf16 tensor, twice the 256 MB last-level cache


def bench_regions(torch, hip, steps, warmup, with_cpu=True):
    """The managed elementwise command and the fused regions at HBM scale:
    every tensor is 256M elements (512 MiB in bf16, 1 GiB in f32), twice the
    256 MB last-level cache, so each launch streams from HBM.  Algorithmic
    bytes = one read of every input element plus one write of every output
    element (RMSNorm's weight, RoPE's positions and the bias row are a few
    KiB).  Each entry carries its HBM roofline fraction and, when
    profiles/traffic.json has it, the rocprofv3-measured bytes per launch."""
    gen = torch.Generator(device="cuda").manual_seed(SEED)
    R, C = REGION_ROWS, REGION_COLS
    n = R * C
    out = []

    SR = 4096  # CPU sample: 4096 of the rows (16M elements)

    def leg(name, kernel, workload, fn, nbytes, cpu_fn=None):
        ms = timed(torch, fn, steps, warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        e = {"name": name, "kernel": kernel, "workload": workload, "ms": ms, "value": gbs, "unit": "GB/s",
             "algorithmic_bytes": nbytes,
             "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK["hbm"], "unit": "GB/s",
                          "frac": gbs / PEAK["hbm"], "traffic": traffic_for(name), "traffic_source": TRAFFIC_SOURCE}}
        if with_cpu and cpu_fn is not None:
            dt = cpu_time(cpu_fn)
            e["cpu_baseline"] = cpu_gbs(nbytes * SR // R, dt, f"{SR} of {R} rows of the same tensors (scalar C oracle)")
        out.append(e)

    from oracle import oracle as orc
    h16 = lambda t: t[:SR].contiguous().cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731

    B = 2  # bytes per bf16 element
    x = rnd_bf16(torch, gen, (R, C))
    y = torch.empty_like(x)
    z = rnd_bf16(torch, gen, (R, C))
    from vibe_compiler_amd.backend import BF16, F32
    xs, zs = h16(x), h16(z)
    leg("ew_add", "ew_kernel (Add)", f"managed elementwise Add, bf16, {n} elements",
        lambda: hip.elementwise("Add", BF16, x, y, z), 3 * n * B, lambda: orc.elementwise(8, orc.BF16, xs, zs))
    leg("silu_mul", "silu_mul", f"silu(gate) * up, bf16, {n} elements", lambda: hip.silu_mul(x, z, y), 3 * n * B,
        lambda: orc.silu_mul(xs, zs))
    leg("gelu_tanh", "gelu_tanh", f"tanh-GELU, bf16, {n} elements", lambda: hip.gelu_tanh(x, y), 2 * n * B,
        lambda: orc.gelu_tanh(xs))
    w = rnd_bf16(torch, gen, (C,))
    ws = w.cpu().view(torch.int16).numpy().view(np.uint16)
    leg("rmsnorm", "rmsnorm", f"RMSNorm rows of {C}, bf16, {R} rows", lambda: hip.rmsnorm(x, w, y, 1e-5),
        2 * n * B + C * B, lambda: orc.rmsnorm(xs, ws, 1e-5))
    leg("softmax", "softmax", f"row softmax over {C} columns, bf16, {R} rows", lambda: hip.softmax(x, y),
        2 * n * B, lambda: orc.softmax(xs))
    xr, yr = x.view(R, 32, C // 32), y.view(R, 32, C // 32)
    pos = torch.arange(R, dtype=torch.int32, device="cuda")
    xrs, ps = xs.reshape(SR, 32, C // 32), np.arange(SR, dtype=np.int32)
    leg("rope", "rope", f"RoPE (rotate-half, theta 1e4), bf16 [{R}, 32, {C // 32}]",
        lambda: hip.rope(xr, yr, pos, 1e4), 2 * n * B + R * 4, lambda: orc.rope(xrs, ps, 1e4))
    del x, y, z, xr, yr
    torch.cuda.empty_cache()
    xf = torch.randn((R, C), device="cuda", generator=gen)
    yf = torch.empty_like(xf)
    bias = torch.randn((C,), device="cuda", generator=gen)
    xfs, bs = xf[:SR].cpu().numpy(), bias.cpu().numpy()
    leg("bias_add", "bias_add", f"row bias add, f32 [{R}, {C}]", lambda: hip.bias_add(xf, bias, yf, fmt=F32),
        2 * n * 4 + C * 4, lambda: orc.bias_add(xfs, bs))
    del xf, yf
    torch.cuda.empty_cache()
    return out


def bench_copy(torch, steps, warmup):
    """A plain device copy of known size: the calibration kernel for the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters (reads and writes COPY_BYTES)."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").fill_(7)
    dst = torch.empty_like(src)
    ms = timed(torch, lambda: dst.copy_(src), steps, warmup)
    return {"workload": f"device copy of {COPY_BYTES} bytes (counter calibration)", "metric": "GB/s",
            "ms": ms, "value": 2 * COPY_BYTES / (ms * 1e-3) / 1e9, "unit": "GB/s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="fa,fa_cases,fd,i8,mlp,llama,mv,cmp,regions",
                    help="comma list of fa, fa_cases, fd, i8, mlp, llama, mv, cmp, regions, copy, vendor")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this backend runs on one GPU; --gpus {args.gpus} is not a configuration it "
              "measures (the multi-GPU sharding is a design note only)", file=sys.stderr)
        return 2

    import torch
    from vibe_compiler_amd import backend as B

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    hip = B.Context(0)
    only = set(args.only.split(","))
    with_cpu = not args.no_cpu
    secondary = []
    fa = None
    if "fa" in only:
        fa = bench_fa(torch, hip, args.steps, args.warmup, with_cpu)
    if "fa_cases" in only:
        secondary.append(dict(name="fa_cases", **bench_fa_cases(torch, hip, args.steps, args.warmup, with_cpu)))
    if "fd" in only:
        secondary.append(dict(name="fd_decode", **bench_fd(torch, hip, args.steps, args.warmup, with_cpu)))
    if "i8" in only:
        secondary.append(dict(name="gemm_i8", **bench_i8(torch, hip, args.steps, args.warmup, with_cpu)))
    if "mlp" in only:
        secondary.append(dict(name="mlp_fp32", **bench_mlp(torch, hip, B, args.steps, args.warmup, with_cpu)))
        secondary.append(dict(name="mlp_fp32_formal", **bench_mlp(torch, hip, B, args.steps, args.warmup, with_cpu,
                                                                  lane="formal")))
    if "llama" in only:
        secondary.append(dict(name="llama_layer", **bench_llama(torch, hip, args.steps, args.warmup, with_cpu)))
    if "mv" in only:
        secondary.append(dict(name="movement", **bench_mv(torch, hip, args.steps, args.warmup, with_cpu)))
    if "cmp" in only:
        secondary.append(dict(name="comparator", **bench_cmp(torch, hip, args.steps, args.warmup, with_cpu)))
    if "regions" in only:
        secondary.append({"name": "regions", "legs": bench_regions(torch, hip, args.steps, args.warmup, with_cpu)})
    if "copy" in only:
        secondary.append(dict(name="copy", **bench_copy(torch, args.steps, args.warmup)))
    if "vendor" in only:
        secondary.append(dict(name="vendor", **bench_vendor(torch, hip, args.steps, args.warmup)))
    hip.close()

    line = {
        "metric": "FA prefill TFLOP/s + FD decode HBM GB/s (% of roofline), 1\u00d7MI355X",
        "value": fa["value"] if fa else None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": fa["ms"] if fa else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 inputs resident in HBM)",
        "config": {"workload": "FA prefill bf16 Q,K,V [1,16,2048,128] causal, scale 1/sqrt(128), "
                               "fp32 online softmax, bf16 out",
                   "batch": 1, "heads": 16, "seq_len": 2048, "head_dim": 128, "causal": True},
        "roofline": fa["roofline"] if fa else None,
        "cpu_baseline": fa.get("cpu_baseline") if fa else None,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
