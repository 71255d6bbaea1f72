#!/usr/bin/env python3
"""Benchmark of the routed-expert MoE hot path on one MI355X; prints one JSON line.

Workload (the decode configuration the metric is quoted on): one synthetic MoE layer, hidden
2048, 256 routed experts, top-8 with softmax-renormalised weights, SwiGLU experts with F 512,
TQ2_T packed trellis weights; batch-1 decode of `--steps` tokens with fresh seeded N(0, 1)
activations, every input resident in HBM before the timed region. A step is one token's pass
through the layer (router and rotation, routed gate/up, SwiGLU and down rotation, down and
combine). Twelve byte-identical copies of the layer (2.57 GB of experts) are cycled, so that under
uniform routing less than a tenth of a token's expert reads can find their lines still in the
256 MB Infinity Cache. Parity is checked on at least 1000 tokens of the configuration (the timed
tokens first) whatever --steps is.

Reported beside the throughput:
  roofline      the dominant kernel (moe_decode_gu: the routed gate/up dequant-GEMV, 8 experts x
                2 x 278,528 packed bytes per launch) timed by its own dispatch start and end
                (gd_dispatch_timed) over a second timed pass; beside it the kernel-trace average
                of the committed rocprofv3 summary, HBM traffic per launch from the committed
                counter summary, and a second roof: the codebook-gather ceiling of the decode,
                measured in the same run by decode_gather_probe (moe_decode_gu's block dot on
                register-resident blocks, LDS codebook gathers only): the time the launch's
                131,072 blocks take at the chip's measured block rate.
  mixed, stack, coder
                the mixed-quant layer, the 48-layer stack and the real model's expert shape (see
                --mixed, --stack and --coder below), as objects of the same line unless
                --no-mixed / --no-stack / --no-coder.
  cpu_baseline  the CPU oracle (a C restatement of src/engine.zig ffn and its thread pool) on a
                bounded sample of the same tokens, on this host's cores.
  parity        rel-RMS and cosine of the GPU outputs against that CPU sample.
  --stack       (its own JSON line) the residual stack x <- x + MoE_l(RMSNorm_l(x)) of 48 distinct
                seeded layers resident in HBM: batch 1, 8 (decode path), 32, 64 (prefill path) and
                a 4096-token prefill, each with tok/s and the fraction of its binding roofline
                (HBM: measured distinct experts' packed bytes plus the router matrices per step;
                MFMA: routed-expert FLOPs), and the CPU oracle on a sample of 8 tokens.
  --mixed       (its own JSON line) the mixed-quant layer: routed experts' projections assigned
                by seed across the eight Gyro types, plus the always-on bf16 shared SwiGLU expert of
                width 1024; batch-1 decode and a 512-token prefill, with
                packed-byte and FLOP rooflines, and the CPU oracle on a sample. Decode runs the
                decode path's type-generic kernels, prefill the prefill path's type-generic
                grouped GEMMs (one persistent launch) and shared-expert GEMMs.
  --coder       (its own JSON line) the real model's routed-expert shape, hidden 2560, 256
                experts, top-10, F 640, in TQ2_T and in GGUF 148: batch-1 decode over cycled layer
                copies and a 1024-token prefill, with rooflines, and decode parity with the oracle
                on 16 tokens.
  prefill       1024-token prefill of the same layer with a Zipf(1.1) router bias (cycled
                copies, distinct bf16 N(0, 1) token batches): tok/s, per-kernel dispatch times,
                and routed-expert FLOPs (51,539,607,552 per call) against the 2.5 PFLOP/s dense
                16-bit MFMA peak, for the grouped GEMMs alone and for the whole layer; the CPU
                oracle times one of the calls and checks its outputs.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "gyro-dx_amd"))

METRIC = "MoE-layer decode tok/s + % HBM peak; prefill grouped-GEMM % bf16 MFMA peak"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0
E, F, N_EXPERT, TOP_K = 2048, 512, 256, 8
PROJ_BYTES = F * (E // 128) * 34  # 278,528 packed bytes per expert projection
EXPERT_BYTES_PER_TOKEN = TOP_K * 3 * PROJ_BYTES  # 6,684,672
GU_BYTES_PER_LAUNCH = TOP_K * 2 * PROJ_BYTES  # 4,456,448
ROUTER_BYTES = N_EXPERT * E * 4  # fp32 router matrix read per layer and step
TRAFFIC_FILE = ROOT / "profiles" / "moe_decode_gu_traffic.md"
TRACE_FILE = ROOT / "profiles" / "moe_decode_kernels_b1.md"
GU_BLOCKS_PER_LAUNCH = TOP_K * 2 * F * (E // 128)  # 131,072 TQ2_T blocks of 128 weights
BLOCKS_PER_EXPERT = 2 * F * (E // 128) + E * (F // 128)  # 24,576: an expert's gate, up and down blocks
CUS = 256
PARITY_TOKENS = 1000
GEMM_COUNTERS_FILE = ROOT / "profiles" / "moe_prefill_gemm_counters.md"
# How the synthetic expert blocks are drawn (gyrodx.synth.random_blocks): trellis stream bytes
# uniform; block scales binary16 with a random sign, exponent field 7..11 and a uniform mantissa.
BLOCK_SCALES = "binary16, random sign, exponent field 7..11 (|scale| in [2^-8, 2^-3)), uniform mantissa"
PREFILL_TOKENS = 1024
# Routed-expert FLOPs of one prefill call: tokens x top-8 x (gate, up, down) x 2 x E x F.
PREFILL_GU_FLOPS = PREFILL_TOKENS * TOP_K * 2 * 2 * E * F       # 34,359,738,368
PREFILL_DOWN_FLOPS = PREFILL_TOKENS * TOP_K * 2 * E * F         # 17,179,869,184
PREFILL_FLOPS = PREFILL_GU_FLOPS + PREFILL_DOWN_FLOPS           # 51,539,607,552
BUNDLE_BYTES = 3 * PROJ_BYTES                                   # 835,584 per expert
COPY_WORDS = 8 << 20  # calibration copy of the traffic probe: 32 MiB read, 32 MiB written


def read_traffic():
    """HBM bytes per moe_decode_gu launch from the committed counter summary (its
    `bytes_per_launch:` line), or None when no summary is present."""
    if not TRAFFIC_FILE.exists():
        return None
    m = re.search(r"^bytes_per_launch:\s*(\d+)", TRAFFIC_FILE.read_text(), re.M)
    return int(m.group(1)) if m else None


def read_trace_us(kernel: str):
    """Average kernel-trace duration (us) of `kernel` from the committed rocprofv3 summary of the
    decode bench (its table row `| kernel | calls | avg us | ...`), or None when absent."""
    if not TRACE_FILE.exists():
        return None
    m = re.search(rf"^\|\s*{re.escape(kernel)}\s*\|\s*\d+\s*\|\s*([0-9.]+)\s*\|", TRACE_FILE.read_text(), re.M)
    return float(m.group(1)) if m else None


def gather_probe(groups: int = CUS, iters: int = 256):
    """The chip's rate of moe_decode_gu's block dot with every operand on chip (decode_gather_probe,
    one group of 512 threads per compute unit, `iters` blocks per thread): decoded blocks per
    second over the span from the first group's start to the last group's end (100 MHz counter),
    the shader clock (shader-clock cycles over real-time ticks, median over groups) and blocks
    per clock per compute unit. The second launch of two is the one measured."""
    import ctypes as C
    from gyrodx import CODEBOOK, KERNEL_DIR, native
    L = native.lib()
    opts = native.Options(0, 0, 0, 32 << 20, 1024)
    ctx = C.c_void_p()
    native.check(L.gd_create(C.byref(opts), C.byref(ctx)), "gd_create")
    code = (KERNEL_DIR / "decode_gather_probe.co").read_bytes()
    pipe = C.c_void_p()
    native.check(L.gd_create_pipeline(ctx, code, len(code), C.byref(pipe)), "gd_create_pipeline")
    g = np.random.default_rng(5)
    blocks = g.integers(0, 1 << 32, (512, 9), dtype=np.uint64).astype(np.uint32)
    blocks[:, 0] = (blocks[:, 0] & 0xFFFF0000) | 0x2800  # even blocks: scale 2^-5
    blocks[:, 0] = (blocks[:, 0] & 0x0000FFFF) | (0x2800 << 16)  # odd blocks: the same
    data = {"blocks": blocks.tobytes(), "book": Path(CODEBOOK).read_bytes(),
            "x": g.standard_normal(8 * 128).astype(np.float32).tobytes(),
            "out": bytes(8 * 4 * groups), "sums": bytes(512 * 4 * groups)}
    bufs = {}
    for name, raw in data.items():
        h, info = C.c_void_p(), native.BufferInfo()
        native.check(L.gd_create_resource(ctx, len(raw), 1, C.byref(h), C.byref(info)), "gd_create_resource")
        C.memmove(info.mapped, raw, len(raw))
        bufs[name] = (h, info)
    cst = (C.c_uint32 * 6)(bufs["blocks"][1].srv_index, bufs["book"][1].srv_index, bufs["x"][1].srv_index,
                           bufs["out"][1].uav_index, bufs["sums"][1].uav_index, iters)
    ticket = C.c_uint64()
    for _ in range(2):
        native.check(L.gd_begin(ctx, 60000), "gd_begin")
        native.check(L.gd_dispatch(ctx, pipe, cst, 6, groups, 1, 1), "gd_dispatch")
        native.check(L.gd_submit(ctx, C.byref(ticket)), "gd_submit")
        native.check(L.gd_wait_compute(ctx, ticket, 60000), "gd_wait_compute")
    out = np.frombuffer(C.string_at(bufs["out"][1].mapped, 8 * 4 * groups), np.uint32).reshape(groups, 8)
    sums = np.frombuffer(C.string_at(bufs["sums"][1].mapped, 512 * 4 * groups), np.float32)
    for h, _ in bufs.values():
        native.check(L.gd_release_buffer(ctx, h, 60000), "gd_release_buffer")
    native.check(L.gd_release_pipeline(ctx, pipe, 60000), "gd_release_pipeline")
    native.check(L.gd_destroy(ctx, 60000), "gd_destroy")
    w = out.astype(np.uint64)
    r0, r1, c0, c1 = (w[:, 0] | w[:, 1] << 32), (w[:, 2] | w[:, 3] << 32), (w[:, 4] | w[:, 5] << 32), (w[:, 6] | w[:, 7] << 32)
    span_s = float(r1.max() - r0.min()) / 1e8
    ghz = float(np.median((c1 - c0).astype(np.float64) / (r1 - r0).astype(np.float64))) * 0.1
    blocks_per_s = groups * 512.0 * iters / span_s
    return {"blocks_per_s": blocks_per_s, "clock_ghz": round(ghz, 3),
            "blocks_per_clk_per_cu": round(blocks_per_s / (CUS * ghz * 1e9), 4),
            "finite": bool(np.isfinite(sums).all())}


def gather_roof(kernel_us: float, probe):
    """The codebook-gather ceiling of moe_decode_gu: its launch's 131,072 blocks at the probe's
    chip-wide block rate, and the fraction of the measured launch time that ceiling accounts for."""
    ceiling_us = GU_BLOCKS_PER_LAUNCH / probe["blocks_per_s"] * 1e6
    return {"bound": "lds codebook gathers", "blocks_per_launch": GU_BLOCKS_PER_LAUNCH,
            "blocks_per_clk_per_cu": probe["blocks_per_clk_per_cu"], "clock_ghz": probe["clock_ghz"],
            "ceiling_us": round(ceiling_us, 3), "frac": round(ceiling_us / kernel_us, 4),
            "probe": "decode_gather_probe: moe_decode_gu's block dot, register-resident blocks and "
                     "activations, LDS codebook gathers; one group of 512 threads per compute unit"}


def read_gemm_counters():
    """MFMA-busy and useful fractions of the prefill GEMMs from the committed counter summary
    (its `mfma_busy_<kernel>:` and `mfma_useful_<kernel>:` lines), or None when absent."""
    if not GEMM_COUNTERS_FILE.exists():
        return None
    text = GEMM_COUNTERS_FILE.read_text()
    got = {k: float(v) for k, v in re.findall(r"^(mfma_(?:busy|useful)_moe_prefill_\w+):\s*([0-9.]+)", text, re.M)}
    return {"source": str(GEMM_COUNTERS_FILE.relative_to(ROOT)), **got} if got else None


def copy_calibration(reps: int) -> None:
    """Launches the bit-exact 32-bit copy (ew op 5) over COPY_WORDS words `reps` times, device to
    device, so that a counter pass sees FETCH_SIZE and WRITE_SIZE of a kernel of known traffic."""
    import ctypes as C
    from gyrodx import KERNEL_DIR, native
    L = native.lib()
    opts = native.Options(0, 0, 0, 32 << 20, 1024)
    ctx = C.c_void_p()
    native.check(L.gd_create(C.byref(opts), C.byref(ctx)), "gd_create")
    code = (KERNEL_DIR / "ew.co").read_bytes()
    pipe = C.c_void_p()
    native.check(L.gd_create_pipeline(ctx, code, len(code), C.byref(pipe)), "gd_create_pipeline")
    bufs = []
    for _ in range(2):
        h, info = C.c_void_p(), native.BufferInfo()
        native.check(L.gd_create_resource(ctx, COPY_WORDS * 4, 0, C.byref(h), C.byref(info)), "gd_create_resource")
        bufs.append((h, info))
    (_, src), (_, dst) = bufs
    cst = (C.c_uint32 * 12)(src.uav_index, 0, 0, src.uav_index, 0, 0, dst.uav_index, 0, 0, COPY_WORDS, 1, 5)
    native.check(L.gd_begin(ctx, 60000), "gd_begin")
    for _ in range(reps):
        native.check(L.gd_dispatch(ctx, pipe, cst, 12, COPY_WORDS // 256, 1, 1), "gd_dispatch")
    ticket = C.c_uint64()
    native.check(L.gd_submit(ctx, C.byref(ticket)), "gd_submit")
    native.check(L.gd_wait_compute(ctx, ticket, 60000), "gd_wait_compute")
    for h, _ in bufs:
        native.check(L.gd_release_buffer(ctx, h, 60000), "gd_release_buffer")
    native.check(L.gd_release_pipeline(ctx, pipe, 60000), "gd_release_pipeline")
    native.check(L.gd_destroy(ctx, 60000), "gd_destroy")


def cpu_threads() -> int:
    n = os.cpu_count() or 1
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


def cpu_baseline(layer, tokens, gpu_out, budget_s: float, seed: int):
    """Times the CPU oracle on batch-1 tokens one at a time until the budget is spent: the timed
    run's tokens first (their outputs are the parity check), then further seeded N(0, 1) tokens
    of the same workload, so that the sample does not shrink with --steps."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from gyrodx import synth
    threads = cpu_threads()
    ol = oracle.OracleLayer(layer)
    ol.forward(tokens[:1], threads=threads)  # thread pool start-up outside the timing
    outs = []
    n, extra, t0 = 0, 0, time.perf_counter()
    batch = tokens
    while time.perf_counter() - t0 <= budget_s:
        for i in range(len(batch)):
            y = ol.forward(batch[i:i + 1], threads=threads)[0]
            if batch is tokens:
                outs.append(y)
            else:
                extra += 1
            n += 1
            if time.perf_counter() - t0 > budget_s:
                break
        batch = synth.make_tokens(seed + 1000 + n, 256, layer.E)
    dt = time.perf_counter() - t0
    ref = np.stack(outs)
    m = len(outs)
    parity = {"tokens": m, "rel_rms": oracle.rel_rms(ref, gpu_out[:m]), "cosine": oracle.cosine(ref, gpu_out[:m]),
              "bar": {"rel_rms": 2e-3, "cosine": 0.9999}}
    base = {"value": n / dt, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} batch-1 decode tokens of the same layer ({m} of the timed run, {extra} further seeded "
                      f"tokens), {dt:.1f} s on {threads} threads"}
    return base, parity


def prefill_bench(eng, layer, args):
    """1024-token prefill of the layer with a Zipf(1.1) router bias over the cycled copies;
    `args.prefill_calls` timed calls on distinct bf16 token batches already in HBM."""
    import dataclasses
    from gyrodx import synth
    from gyrodx.engine import PATH_PREFILL
    zl = dataclasses.replace(layer, router_bias=synth.zipf_bias(args.seed, N_EXPERT, 1.1))
    layers = [eng.add_layer(zl) for _ in range(args.copies)]
    batches = args.prefill_calls
    x = synth.make_tokens(args.seed + 3, PREFILL_TOKENS * batches, bf16=True)
    eng.set_tokens(x)
    eng.run(PATH_PREFILL, PREFILL_TOKENS, min(batches, 4), layers, first=0)  # warm-up
    dev_ms, wall_ms, _ = eng.run(PATH_PREFILL, PREFILL_TOKENS, batches, layers, first=0)
    # The engine runs both GEMMs as one persistent launch (bracket 2) unless created with
    # GYRO_PREFILL_FUSED=0 (then moe_prefill_gu, bracket 2, and moe_prefill_down, bracket 3).
    fused = os.environ.get("GYRO_PREFILL_FUSED", "1") != "0"
    gemms = (("moe_prefill_gemm", 2),) if fused else (("moe_prefill_gu", 2), ("moe_prefill_down", 3))
    us = {}
    for name, br in (("moe_prefill_router", 1), ("moe_prefill_topk", 4), ("moe_prefill_sort", 5), *gemms,
                     ("moe_prefill_combine", 6)):
        us[name] = round(eng.run(PATH_PREFILL, PREFILL_TOKENS, batches, layers, bracket=br, first=0)[2], 3)
    out0 = eng.read_outputs(PREFILL_TOKENS)
    # Distinct experts of the first batch (product path routes, read back after a forward).
    eng.forward(layers[0], x[:PREFILL_TOKENS], PATH_PREFILL)
    ids, _ = eng.last_routes(PREFILL_TOKENS)
    distinct = int(np.unique(ids).size)
    n_tiles = int(eng.last_tiles().shape[0])
    # The GEMMs' decode-gather ceiling: each tile decodes all of its expert's blocks once.
    gather_s = n_tiles * BLOCKS_PER_EXPERT / gather_probe()["blocks_per_s"]
    t_call = wall_ms / batches * 1e-3
    t_dev = dev_ms / batches * 1e-3
    gemm_s = sum(us[name] for name, _ in gemms) * 1e-6
    res = {
        "workload": "single MoE layer, 1024-token prefill, Zipf(1.1) router bias, bf16 N(0,1) tokens",
        "tokens_per_call": PREFILL_TOKENS, "calls": batches, "layer_copies": args.copies,
        "tok_s": round(PREFILL_TOKENS / t_call, 1),
        "us_per_call": round(t_call * 1e6, 2), "device_us_per_call": round(t_dev * 1e6, 2),
        "kernel_us": us,
        "flops_per_call": PREFILL_FLOPS,
        "mfma_peak_tflops": MFMA_PEAK_TFLOPS, "mfma_dtype": "fp16 (same dense peak as bf16)",
        "layer_tflops": round(PREFILL_FLOPS / t_dev / 1e12, 1),
        "layer_frac_of_peak": round(PREFILL_FLOPS / t_dev / 1e12 / MFMA_PEAK_TFLOPS, 4),
        "grouped_gemm_tflops": round(PREFILL_FLOPS / gemm_s / 1e12, 1),
        "grouped_gemm_frac_of_peak": round(PREFILL_FLOPS / gemm_s / 1e12 / MFMA_PEAK_TFLOPS, 4),
        "distinct_experts": distinct, "expert_bytes": distinct * BUNDLE_BYTES,
        "gather_roof": {"bound": "lds codebook gathers", "kernel": " + ".join(name for name, _ in gemms),
                        "tiles": n_tiles, "decoded_blocks": n_tiles * BLOCKS_PER_EXPERT,
                        "ceiling_us": round(gather_s * 1e6, 2), "frac": round(gather_s / gemm_s, 4)},
        "block_scales": BLOCK_SCALES,
        # The grouped GEMMs' roofline: routed-expert FLOPs over the GEMM launch's dispatch time
        # (measured above); the counter pass's MFMA-busy and useful-work fractions of the
        # gate/up and down units beside it.
        "roofline": {"bound": "mfma", "kernel": " + ".join(name for name, _ in gemms),
                     "achieved": round(PREFILL_FLOPS / gemm_s / 1e12, 1), "peak": MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(PREFILL_FLOPS / gemm_s / 1e12 / MFMA_PEAK_TFLOPS, 4),
                     "traffic": None, "counters": read_gemm_counters()},
    }
    if fused:
        res["two_launch_gemms"] = prefill_two_launch(zl, x, args)
    return res, x[:PREFILL_TOKENS], out0, zl


def prefill_two_launch(zl, x, args):
    """The same timed calls on an engine that runs the GEMMs as two launches (moe_prefill_gu,
    moe_prefill_down): device time per call and the two kernels' dispatch times."""
    from gyrodx.engine import PATH_PREFILL, Engine
    saved = os.environ.get("GYRO_PREFILL_FUSED")
    os.environ["GYRO_PREFILL_FUSED"] = "0"
    try:
        eng = Engine(max_tok=PREFILL_TOKENS)
    finally:
        if saved is None:
            os.environ.pop("GYRO_PREFILL_FUSED", None)
        else:
            os.environ["GYRO_PREFILL_FUSED"] = saved
    layers = [eng.add_layer(zl) for _ in range(args.copies)]
    eng.set_tokens(x)
    batches = args.prefill_calls
    eng.run(PATH_PREFILL, PREFILL_TOKENS, min(batches, 4), layers, first=0)
    dev_ms, _, _ = eng.run(PATH_PREFILL, PREFILL_TOKENS, batches, layers, first=0)
    us = {name: round(eng.run(PATH_PREFILL, PREFILL_TOKENS, batches, layers, bracket=br, first=0)[2], 3)
          for name, br in (("moe_prefill_gu", 2), ("moe_prefill_down", 3))}
    eng.close()
    return {"device_us_per_call": round(dev_ms / batches * 1e3, 2), "kernel_us": us}


def prefill_cpu(layer, x, gpu_out, budget_s: float = 8.0):
    """The CPU oracle on the first timed batch (the parity check), then on further calls of the
    same batch until about `budget_s` seconds are spent."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    threads = cpu_threads()
    ol = oracle.OracleLayer(layer)
    t0 = time.perf_counter()
    ref = ol.forward(x, threads=threads)
    calls = 1
    while (time.perf_counter() - t0) * (calls + 1) / calls <= budget_s:  # the next call fits the budget
        ol.forward(x, threads=threads)
        calls += 1
    dt = time.perf_counter() - t0
    return ({"value": round(calls * x.shape[0] / dt, 1), "unit": "tok/s", "cores": threads, "kind": "port",
             "sample": f"{calls} calls of the first timed {x.shape[0]}-token batch, {dt:.1f} s on {threads} threads"},
            {"rel_rms": oracle.rel_rms(ref, gpu_out), "cosine": oracle.cosine(ref, gpu_out)})


LAYER_FLOPS_PER_TOKEN = TOP_K * 3 * 2 * E * F  # 50,331,648


def stack_bench(args):
    """The 48-layer residual stack: batch sweep and 4096-token prefill (see the module doc)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from gyrodx import synth
    from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

    n_layers = args.stack_layers
    eng = Engine(max_tok=4096)
    sample = synth.make_tokens(args.seed + 7, 8)
    xo = sample.copy()  # the oracle's own (free-running) stack
    xg = sample.copy()  # the GPU's stack after the layers so far
    threads = cpu_threads()
    cpu_s = 0.0
    ids, layer_err, excluded = [], [], 0
    t0 = time.perf_counter()
    for l in range(n_layers):
        L = synth.make_stack(args.seed + 100 + l, 1)[0]
        ids.append(eng.add_layer(L))
        ol = oracle.OracleLayer(L)
        # Teacher-forced check of layer l: the oracle's step from the GPU's own stack state
        # against the GPU's step (tokens with a near-tie at this layer's top-8 excluded).
        xg_next = eng.forward_stack(ids, sample, PATH_DECODE)
        h = oracle.rms_norm(xg, L.norm_weight, L.norm_eps)
        t1 = time.perf_counter()
        y = ol.forward(h, threads=threads)
        cpu_s += time.perf_counter() - t1
        p = ol.router_f64(h)
        p = -np.sort(-np.exp(p - p.max(axis=1, keepdims=True)), axis=1)
        sep = (p[:, TOP_K - 1] - p[:, TOP_K]) > 1e-5 * p[:, TOP_K - 1]
        excluded += int((~sep).sum())
        layer_err.append(oracle.rel_rms(y[sep], (xg_next - xg)[sep]) if sep.any() else 0.0)
        xg = xg_next
        xo = xo + ol.forward(oracle.rms_norm(xo, L.norm_weight, L.norm_eps), threads=threads)
        del L, ol
        if l % 8 == 7:
            print(f"stack: {l + 1} of {n_layers} layers resident ({time.perf_counter() - t0:.0f} s)",
                  file=sys.stderr, flush=True)
    bundle_all = n_layers * N_EXPERT * BUNDLE_BYTES
    # The trellis decode's own ceiling: every decoded 128-weight block costs the codebook gathers
    # whose chip-wide rate decode_gather_probe measures (both paths gather from the same LDS
    # codebook, two 4-byte gathers per state). Decode decodes every slot's expert blocks; prefill
    # every tile's (a tile: up to 128 sorted slots of one expert).
    probe = gather_probe()
    points = []
    sweep = ((1, PATH_DECODE, 200), (8, PATH_DECODE, 100), (32, PATH_PREFILL, 50), (64, PATH_PREFILL, 50),
             (4096, PATH_PREFILL, 4))
    wanted = {int(b) for b in args.stack_batches.split(",")}
    for batch, path, calls in (p for p in sweep if p[0] in wanted):
        x = synth.make_tokens(args.seed + 200 + batch, batch * calls, bf16=path == PATH_PREFILL)
        eng.set_tokens(x)
        eng.run_stack(path, batch, 1, ids)  # warm-up
        dev_ms, wall_ms = eng.run_stack(path, batch, calls, ids)
        # Measured distinct experts per layer on the first batch: the stack's prefix up to each
        # layer, then that layer's routes.
        distinct, tiles = [], []
        for l in range(n_layers if batch <= 64 else 1):
            eng.forward_stack(ids[:l + 1], x[:batch], path)
            r, _ = eng.last_routes(batch)
            counts = np.bincount(r.ravel(), minlength=N_EXPERT)
            distinct.append(int((counts > 0).sum()))
            tiles.append(int(((counts + 127) // 128).sum()))
        if batch > 64:  # every expert at 4096 tokens; tiles of the first layer for every layer
            distinct = [N_EXPERT] * n_layers
            tiles = tiles * n_layers
        step_s = wall_ms / calls * 1e-3
        step_bytes = sum(distinct) * BUNDLE_BYTES + n_layers * ROUTER_BYTES
        flops = batch * n_layers * LAYER_FLOPS_PER_TOKEN
        hbm_gbs = step_bytes / step_s / 1e9
        tflops = flops / step_s / 1e12
        bound = "hbm" if step_bytes / (HBM_PEAK_GBS * 1e9) > flops / (MFMA_PEAK_TFLOPS * 1e12) else "mfma"
        frac = hbm_gbs / HBM_PEAK_GBS if bound == "hbm" else tflops / MFMA_PEAK_TFLOPS
        units = batch * TOP_K * n_layers if path == PATH_DECODE else sum(tiles)
        blocks = units * BLOCKS_PER_EXPERT
        gather_ms = blocks / probe["blocks_per_s"] * 1e3
        points.append({"batch": batch, "path": "decode" if path == PATH_DECODE else "prefill", "calls": calls,
                       "tok_s": round(batch / step_s, 1), "ms_per_step": round(step_s * 1e3, 4),
                       "device_ms_per_step": round(dev_ms / calls, 4),
                       "distinct_experts_per_layer": round(sum(distinct) / n_layers, 1),
                       "bytes_per_step": step_bytes, "flops_per_step": flops,
                       "hbm_gbs": round(hbm_gbs, 1), "tflops": round(tflops, 2),
                       "roofline": {"bound": bound, "frac": round(frac, 4)},
                       "gather_roof": {"bound": "lds codebook gathers",
                                       "decoded_blocks_per_step": blocks,
                                       "decoded": "slot experts" if path == PATH_DECODE else
                                                  ("sort tiles" if batch <= 64 else "sort tiles (first layer's x layers)"),
                                       "ceiling_ms": round(gather_ms, 4), "frac": round(gather_ms / (step_s * 1e3), 4)}})
        print(f"stack: batch {batch}: {points[-1]['tok_s']} tok/s", file=sys.stderr, flush=True)
    eng.close()
    return {
        "workload": f"{n_layers}-layer residual MoE stack (RMSNorm -> MoE -> residual), hidden {E}, "
                    f"{N_EXPERT} TQ2_T experts per layer, top-{TOP_K}, F {F}",
        "layers": n_layers, "resident_expert_bytes": bundle_all,
        "hbm_peak_gbs": HBM_PEAK_GBS, "mfma_peak_tflops": MFMA_PEAK_TFLOPS,
        "gather_probe": {"blocks_per_clk_per_cu": probe["blocks_per_clk_per_cu"], "clock_ghz": probe["clock_ghz"]},
        "points": points,
        "cpu_baseline": {"value": round(8 / cpu_s, 2), "unit": "tok/s", "cores": threads, "kind": "port",
                         "sample": f"8 decode tokens through all {n_layers} layers, {cpu_s:.1f} s on {threads} threads"},
        "parity": {"teacher_forced_max_layer_rel_rms": round(max(layer_err), 7),
                   "teacher_forced_mean_layer_rel_rms": round(float(np.mean(layer_err)), 7),
                   "near_tie_token_layers_excluded": excluded,
                   "free_running_per_token_rel_rms": [round(oracle.rel_rms(xo[t], xg[t]), 6) for t in range(8)],
                   "note": "per layer: the oracle's MoE output from the GPU's stack state vs the GPU's; free "
                           "running: 48 layers each way, where one routing flip changes a token's path"},
    }


SHARED_F = 1024
SHARED_BYTES = 3 * SHARED_F * E * 2  # bf16 gate, up, down of the shared expert


def mixed_bench(args):
    """The mixed-quant layer with the shared expert (see the module doc)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from gyrodx import synth
    from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

    layer = synth.make_layer(args.seed + 50, mixed_types=True, SF=SHARED_F)
    copies = args.copies
    eng = Engine(max_tok=512)
    ids = [eng.add_layer(layer) for _ in range(copies)]
    res = {"workload": f"mixed-quant MoE layer: hidden {E}, {N_EXPERT} experts of mixed Gyro types (all 8), "
                       f"top-{TOP_K}, F {F}, bf16 shared expert of width {SHARED_F}",
           "types_present": sorted(int(t) for t in np.unique(layer.types)), "layer_copies": copies}
    # Packed bytes of the experts the decode tokens select (measured per token), shared expert and router.
    steps = args.mixed_steps
    x = synth.make_tokens(args.seed + 51, steps + 16)
    eng.set_tokens(x)
    eng.run(PATH_DECODE, 1, 16, ids, first=0)
    dev_ms, wall_ms, _ = eng.run(PATH_DECODE, 1, steps, ids, first=16)
    gpu = eng.read_outputs(steps + 16)[16:]
    expert_bytes = []
    for t in range(min(steps, 32)):
        eng.forward(ids[0], x[16 + t:17 + t], PATH_DECODE)
        r, _ = eng.last_routes(1)
        expert_bytes.append(sum(layer.expert_bytes(int(e)) for e in r[0]))
    step_s = wall_ms / steps * 1e-3
    per_tok = float(np.mean(expert_bytes)) + SHARED_BYTES + ROUTER_BYTES
    res["decode"] = {"path": "decode (moe_router, moe_decode_gu_x, shared expert, moe_decode_down_x)",
                     "tok_s": round(1.0 / step_s, 1), "us_per_token": round(step_s * 1e6, 2),
                     "bytes_per_token": int(per_tok), "hbm_gbs": round(per_tok / step_s / 1e9, 1),
                     "roofline": {"bound": "hbm", "frac": round(per_tok / step_s / 1e9 / HBM_PEAK_GBS, 4)}}
    # 512-token prefill on the prefill path (type-generic grouped GEMMs, shared expert GEMMs).
    calls = 8
    xp = synth.make_tokens(args.seed + 52, 512 * calls, bf16=True)
    eng.set_tokens(xp)
    eng.run(PATH_PREFILL, 512, 2, ids, first=0)
    dev_ms, wall_ms, _ = eng.run(PATH_PREFILL, 512, calls, ids, first=0)
    pout = eng.read_outputs(512)
    us = {}
    for name, br in (("moe_prefill_router", 1), ("moe_prefill_topk", 4), ("moe_prefill_sort", 5),
                     ("moe_prefill_gemm_x (gate/up + down, one launch)", 2), ("moe_prefill_shared gate/up", 7),
                     ("moe_prefill_shared down", 8), ("moe_prefill_combine", 6)):
        us[name] = round(eng.run(PATH_PREFILL, 512, calls, ids, bracket=br, first=0)[2], 3)
    call_s = wall_ms / calls * 1e-3
    dev_s = dev_ms / calls * 1e-3
    flops = 512 * (LAYER_FLOPS_PER_TOKEN + 3 * 2 * E * SHARED_F)
    res["prefill"] = {"path": "prefill (router, top-k, sort, moe_prefill_gemm_x, moe_prefill_shared x2, combine)",
                      "tokens": 512, "calls": calls, "tok_s": round(512 / call_s, 1),
                      "us_per_call": round(call_s * 1e6, 2), "device_us_per_call": round(dev_s * 1e6, 2),
                      "kernel_us": us, "flops_per_call": flops, "tflops": round(flops / dev_s / 1e12, 2),
                      "roofline": {"bound": "mfma", "frac": round(flops / dev_s / 1e12 / MFMA_PEAK_TFLOPS, 4)}}
    eng.close()
    if not args.no_cpu:
        threads = cpu_threads()
        ol = oracle.OracleLayer(layer)
        t0 = time.perf_counter()
        ref = ol.forward(x[16:16 + 16], threads=threads)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(16 / dt, 1), "unit": "tok/s", "cores": threads, "kind": "port",
                               "sample": f"16 batch-1 decode tokens, {dt:.2f} s on {threads} threads"}
        refp = ol.forward(xp[:64], threads=threads)
        res["parity"] = {"decode_rel_rms": oracle.rel_rms(ref, gpu[:16]), "decode_cosine": oracle.cosine(ref, gpu[:16]),
                         "prefill_rel_rms_first64": oracle.rel_rms(refp, pout[:64])}
    return res


def coder_decode_kernels(layer, ids_of, x, steps, eng, names):
    """Dispatch times of the batch-1 decode kernels (brackets 1, 2, 3) of `names` that ran."""
    from gyrodx.engine import PATH_DECODE
    return {name: round(eng.run(PATH_DECODE, 1, steps, ids_of, bracket=br, first=16)[2], 3)
            for name, br in names}


def coder_bench(args):
    """The real model's routed-expert shape (hidden 2560, 256 experts, top-10, F 640) in TQ2_T
    (batch-1 decode on moe_router / moe_decode_gu_g / moe_decode_down_g) and in a 64-step type,
    GGUF 148 (decode on moe_router /
    moe_decode_gu_xg / moe_decode_down_xg): batch-1 decode over cycled layer copies, a
    1024-token prefill, per-kernel times, and parity of 16 decode tokens with the oracle."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from gyrodx import synth
    from gyrodx.engine import PATH_DECODE, PATH_PREFILL, Engine

    cE, cF, cNE, cU = 2560, 640, 256, 10
    out = {}
    for type_id in (144, 148):
        layer = synth.make_layer(args.seed + type_id, E=cE, F=cF, n_expert=cNE, n_used=cU, type_id=type_id)
        eng = Engine(max_tok=PREFILL_TOKENS)
        ids = [eng.add_layer(layer) for _ in range(args.copies)]
        steps = args.mixed_steps
        x = synth.make_tokens(args.seed + type_id + 1, steps + 16, E=cE)
        eng.set_tokens(x)
        eng.run(PATH_DECODE, 1, 16, ids, first=0)
        dev_ms, wall_ms, _ = eng.run(PATH_DECODE, 1, steps, ids, first=16)
        gpu = eng.read_outputs(steps + 16)[16:]
        suffix = "g" if type_id == 144 else "xg"
        kus = coder_decode_kernels(layer, ids, x, steps, eng, (("moe_router", 1), (f"moe_decode_gu_{suffix}", 2),
                                                                (f"moe_decode_down_{suffix}", 3)))
        expert_bytes = []
        for t in range(32):
            eng.forward(ids[0], x[16 + t:17 + t], PATH_DECODE)
            r, _ = eng.last_routes(1)
            expert_bytes.append(sum(layer.expert_bytes(int(e)) for e in r[0]))
        step_s = wall_ms / steps * 1e-3
        per_tok = float(np.mean(expert_bytes)) + cNE * cE * 4
        rec = {"decode": {"tok_s": round(1.0 / step_s, 1), "us_per_token": round(step_s * 1e6, 2),
                          "kernel_us": kus, "bytes_per_token": int(per_tok),
                          "hbm_gbs": round(per_tok / step_s / 1e9, 1),
                          "roofline": {"bound": "hbm", "frac": round(per_tok / step_s / 1e9 / HBM_PEAK_GBS, 4)}}}
        calls = 8
        xp = synth.make_tokens(args.seed + type_id + 2, PREFILL_TOKENS * calls, E=cE, bf16=True)
        eng.set_tokens(xp)
        eng.run(PATH_PREFILL, PREFILL_TOKENS, 2, ids, first=0)
        pdev, pwall, _ = eng.run(PATH_PREFILL, PREFILL_TOKENS, calls, ids, first=0)
        flops = PREFILL_TOKENS * cU * 3 * 2 * cE * cF
        dev_s = pdev / calls * 1e-3
        pus = {}
        one = os.environ.get("GYRO_PREFILL_FUSED", "1") != "0"  # one GEMM launch (moe_prefill_gemm or _x)
        gemms = (("gate/up + down (one launch)", 2),) if one else (("gate/up", 2), ("down", 3))
        for name, br in (("router", 1), ("topk", 4), ("sort", 5), *gemms, ("combine", 6)):
            pus[name] = round(eng.run(PATH_PREFILL, PREFILL_TOKENS, calls, ids, bracket=br, first=0)[2], 3)
        rec["prefill"] = {"tokens": PREFILL_TOKENS, "calls": calls, "tok_s": round(PREFILL_TOKENS * calls / pwall * 1e3, 1),
                          "device_us_per_call": round(dev_s * 1e6, 2), "kernel_us": pus, "flops_per_call": flops,
                          "roofline": {"bound": "mfma", "frac": round(flops / dev_s / 1e12 / MFMA_PEAK_TFLOPS, 4)}}
        eng.close()
        if not args.no_cpu:
            ol = oracle.OracleLayer(layer)
            ref = ol.forward(x[16:32], threads=cpu_threads())
            rec["parity"] = {"decode_tokens": 16, "rel_rms": oracle.rel_rms(ref, gpu[:16]),
                             "cosine": oracle.cosine(ref, gpu[:16])}
        out[f"type_{type_id}"] = rec
        print(f"coder shape, type {type_id}: {json.dumps(rec)}", file=sys.stderr, flush=True)
    return {"workload": f"routed experts at hidden {cE}, {cNE} experts, top-{cU}, F {cF}; "
                        f"{args.copies} layer copies cycled", **out}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--copies", type=int, default=12, help="layer copies cycled to defeat the Infinity Cache")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-calls", type=int, default=16, help="timed 1024-token prefill calls (0: skip)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="for profiling passes: only the prefill measurement, printed as its own JSON line")
    ap.add_argument("--stack", action="store_true",
                    help="the 48-layer stack batch sweep and 4096-token prefill, printed as its own JSON line")
    ap.add_argument("--stack-layers", type=int, default=48)
    ap.add_argument("--mixed", action="store_true",
                    help="the mixed-quant layer with the shared expert, printed as its own JSON line")
    ap.add_argument("--mixed-steps", type=int, default=500)
    ap.add_argument("--coder", action="store_true",
                    help="the real model's expert shape (2560 / 640 / top-10) in TQ2_T and GGUF 148; prints its own JSON line")
    ap.add_argument("--stack-batches", default="1,8,32,64,4096", help="sweep points of --stack (of 1,8,32,64,4096)")
    ap.add_argument("--no-mixed", action="store_true", help="leave the mixed-quant object out of the default line")
    ap.add_argument("--no-stack", action="store_true", help="leave the 48-layer stack object out of the default line")
    ap.add_argument("--no-coder", action="store_true", help="leave the real-model shape object out of the default line")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for counter passes: the warm-up and timed decode steps, then 20 calibration "
                         "copies of 32 MiB; prints the probe's shape and no benchmark line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the layer is sharded by experts across GPUs only in design).", file=sys.stderr)
        return 2

    from gyrodx import synth
    from gyrodx.engine import PATH_DECODE, Engine

    if args.stack:
        print(json.dumps({"stack": stack_bench(args)}), flush=True)
        return 0
    if args.mixed:
        print(json.dumps({"mixed": mixed_bench(args)}), flush=True)
        return 0
    if args.coder:
        print(json.dumps({"coder": coder_bench(args)}), flush=True)
        return 0
    layer = synth.make_layer(args.seed)
    if args.prefill_only:
        eng = Engine(max_tok=PREFILL_TOKENS)
        pre, _, _, _ = prefill_bench(eng, layer, args)
        eng.close()
        print(json.dumps({"prefill": pre}), flush=True)
        return 0
    n_tok = args.warmup + args.steps
    n_par = max(args.steps, PARITY_TOKENS)  # parity tokens: the timed ones first
    tokens = synth.make_tokens(args.seed + 1, args.warmup + n_par)
    eng = Engine(max_tok=PREFILL_TOKENS)
    layers = [eng.add_layer(layer) for _ in range(args.copies)]
    eng.set_tokens(tokens)

    # Warm-up on the first W tokens, then exactly K timed steps on the next K tokens; gm_run
    # returns after the device finished (synchronised on both sides).
    eng.run(PATH_DECODE, 1, args.warmup, layers, first=0)
    if args.traffic_probe:
        eng.run(PATH_DECODE, 1, args.steps, layers, first=args.warmup)
        eng.close()
        copy_calibration(20)
        print(json.dumps({"probe": "traffic", "decode_tokens": n_tok, "gu_bytes_per_launch": GU_BYTES_PER_LAUNCH,
                          "copy_bytes_read": COPY_WORDS * 4, "copy_bytes_written": COPY_WORDS * 4,
                          "copy_launches": 20}), flush=True)
        return 0
    dev_ms, wall_ms, _ = eng.run(PATH_DECODE, 1, args.steps, layers, first=args.warmup)
    if n_par > args.steps:  # untimed: the parity tokens past the timed ones
        eng.run(PATH_DECODE, 1, n_par - args.steps, layers, first=n_tok)
    gpu_out = eng.read_outputs(args.warmup + n_par)[args.warmup:]
    # Roofline pass: the same steps, the dominant kernel timed by its own dispatch start and end.
    _, _, gu_us = eng.run(PATH_DECODE, 1, args.steps, layers, bracket=2, first=args.warmup)
    _, _, down_us = eng.run(PATH_DECODE, 1, args.steps, layers, bracket=3, first=args.warmup)
    _, _, router_us = eng.run(PATH_DECODE, 1, args.steps, layers, bracket=1, first=args.warmup)

    value = args.steps / (wall_ms / 1e3)
    achieved = GU_BYTES_PER_LAUNCH / (gu_us * 1e-6) / 1e9
    traffic = read_traffic()
    trace_us = read_trace_us("moe_decode_gu")
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "tq2_t weights (fp32 block scale x fp32 codebook value), fp32 activations, fp32 accumulate",
        "data": "synthetic (seeded TQ2_T bytes, N(0,0.02) router, N(0,1) tokens)",
        "config": {"workload": "single MoE layer, batch-1 decode", "hidden": E, "experts": N_EXPERT,
                   "top_k": TOP_K, "ffn": F, "expert_type": "TQ2_T (GGUF 144)", "tokens": args.steps,
                   "layer_copies": args.copies, "block_scales": BLOCK_SCALES, "parallelism": "none (1 GPU)"},
        "device_ms_per_step": round(dev_ms / args.steps, 5),
        "expert_hbm_gbs": round(EXPERT_BYTES_PER_TOKEN / (wall_ms / args.steps * 1e-3) / 1e9, 1),
        "kernel_us": {"moe_router": round(router_us, 3), "moe_decode_gu": round(gu_us, 3),
                      "moe_decode_down": round(down_us, 3)},
        "roofline": {"bound": "hbm", "kernel": "moe_decode_gu", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "bytes_per_launch": GU_BYTES_PER_LAUNCH,
                     "dispatch_us": round(gu_us, 3), "trace_us": trace_us,
                     "frac_trace": round(GU_BYTES_PER_LAUNCH / (trace_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                     if trace_us else None,
                     "second_roof": gather_roof(trace_us or gu_us, gather_probe())},
    }
    if not args.no_cpu:
        line["cpu_baseline"], line["parity"] = cpu_baseline(layer, tokens[args.warmup:], gpu_out, args.cpu_budget,
                                                            args.seed)
    if args.prefill_calls > 0:
        pre, px, pout, zl = prefill_bench(eng, layer, args)
        if not args.no_cpu:
            pre["cpu_baseline"], pre["parity"] = prefill_cpu(zl, px, pout)
        line["prefill"] = pre
    eng.close()
    if not args.no_mixed:
        line["mixed"] = mixed_bench(args)
        print("bench: mixed-quant layer done", file=sys.stderr, flush=True)
    if not args.no_stack:
        line["stack"] = stack_bench(args)
        print("bench: 48-layer stack done", file=sys.stderr, flush=True)
    if not args.no_coder:
        line["coder"] = coder_bench(args)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
