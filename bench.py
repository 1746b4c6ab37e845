#!/usr/bin/env python3
"""DA3-BASE ViT block benchmark on one MI355X.

Metric: "DA3-BASE ViT block us @504x336 (865 tok); GEMM/attn %
fp32-MFMA peak".  A step is one full encoder block over a
synthetic 865-token image already resident in HBM, as five kernels on the
runtime's stream: QKV with LayerNorm 1 folded in (row statistics from its A
slices) and RoPE; flash attention over 3 key splits, merged in split order by
the split that finishes last in each query group; out-projection+LayerScale+residual (writing the updated rows' statistics);
fc1 with LayerNorm 2 folded in and GELU; fc2+LayerScale+residual.

Timing: the block is prepared, then runs W untimed steps and K steps between
two HIP events on the runtime's stream (vh_timer_start/stop), and a second
pass of K steps with per-launch event profiling gives each kernel's average
duration, from which the roofline fractions are computed with algorithmic
FLOPs / bytes.  The GPU's clock is low when it starts from idle and settles
within about 50 ms of continuous work (measured: W = 5, K = 20 take 192 us
per block from idle and 164.5 us after 50-400 ms of blocks; half a second of
idling brings the 189 us back).  Both passes therefore run twice: from the
idle GPU right after preparation (`cold_start`), then after CLOCK_SETTLE_MS
of untimed blocks (`value`, `kernels`, `roofline`).  The secondary sections
follow (Q8_0 block, elementwise kernels, DPT head, BASELINE configs 4, 1, 2
and 5).  The CPU baselines
are the oracle's restatement of the crate's AVX-512 kernels (block, each
projection, flash attention, VNNI Q8_0 GEMM, the Q8_0 block and the 12-layer
encoder), timed on this host with 16 threads and with every core of the
affinity mask, warm-up then the median of at least 10 runs (3 for the
second-long encoder runs; examples/current_shape_bench.rs:24-40).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--calibrate]
       python bench.py --only {q8_0,elementwise,dpt,encoder,configs,block,block4}
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "vestra-kernels_amd"))

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
# Non-packed fp32 VALU lane-ops per second: 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz.
PEAK_VALU_OPS = 256 * 4 * 16 * 2.4e9

T = 865
D, H, HD, F = 768, 12, 64, 3072
FLOPS = {
    "gemm_qkv_rope": 2.0 * T * D * 3 * D,
    "gemm_proj_residual": 2.0 * T * D * D,
    "gemm_fc1_gelu": 2.0 * T * D * F,
    "gemm_fc2_residual": 2.0 * T * F * D,
    "flash_attention": 4.0 * H * T * T * HD,
}
# Q8_0 projections: int8 multiply-adds x 2 per launch.
INT8_OPS = {
    "gemm_q8_0_qkv": 2.0 * T * D * 3 * D,
    "gemm_q8_0_proj_residual": 2.0 * T * D * D,
    "gemm_q8_0_fc1_gelu": 2.0 * T * D * F,
    "gemm_q8_0_fc2_residual": 2.0 * T * F * D,
}
# Algorithmic HBM bytes per launch of the bandwidth-bound kernels.
BYTES = {"layernorm": 2.0 * T * D * 4 + 2 * D * 4}


TRAFFIC_SUMMARY = ROOT / "profiles" / "block_865_hbm_traffic.md"

# Untimed blocks before the timed passes: the clock settles within ~50 ms.
CLOCK_SETTLE_MS = 100.0


def settle_clock(rt, fn, ms: float = CLOCK_SETTLE_MS) -> int:
    """Untimed calls of fn for `ms` of wall time, synchronising every 20: the
    host work between a section's cases idles the GPU, and its clock then
    needs tens of ms of work to ramp back.  Returns the number of calls."""
    rt.synchronize()
    t0, n = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(20):
            fn()
        n += 20
        rt.synchronize()
    return n


def pct_peak(kernels: dict) -> float:
    """GEMM + attention FLOPs of one block over the summed durations of those
    launches, as a percentage of the fp32-MFMA peak."""
    names = [n for n in FLOPS if n in kernels]
    t_us = sum(kernels[n]["avg_us"] * kernels[n]["launches_per_block"] for n in names)
    return round(100.0 * sum(FLOPS[n] for n in names) / (t_us * 1e-6) / 1e12 /
                 PEAK_FP32_MFMA_TFLOPS, 2)


def measured_traffic(launch: str):
    """HBM bytes per launch of `launch` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), or
    None when the summary has no row for it."""
    try:
        text = TRAFFIC_SUMMARY.read_text()
    except OSError:
        return None
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == f"`{launch}`" and cells[2].isdigit():
            return int(cells[2])
    return None


MFMA_SUMMARY = ROOT / "profiles" / "block_865_mfma_busy.md"
TRACE_SUMMARY = ROOT / "profiles" / "block_865_kernel_trace.md"
CONFIG_TRACE_SUMMARY = ROOT / "profiles" / "configs_kernel_trace.md"


def measured_trace_us() -> dict:
    """Per-launch kernel-trace durations of one block at 865 tokens from the
    committed rocprofv3 --kernel-trace summary (median per kernel, summed over
    the kernels of a launch), keyed by launch name; {} when absent.  Unlike
    the per-launch HIP events, the trace adds no event packets around each
    launch."""
    try:
        text = TRACE_SUMMARY.read_text()
    except OSError:
        return {}
    out = {}
    in_block = False
    for line in text.splitlines():
        if line.startswith("## One f32 block"):
            in_block = True
            continue
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if in_block and len(cells) == 3 and cells[0].startswith("`"):
            try:
                out[cells[0].strip("`")] = out.get(cells[0].strip("`"), 0.0) + float(cells[2])
            except ValueError:
                pass
    return out


def measured_config_trace_us() -> dict:
    """Kernel-trace durations of the standalone config 1 and 2 cases from the
    committed rocprofv3 --kernel-trace summary (median over each case's timed
    launches), keyed by case name; {} when absent."""
    try:
        text = CONFIG_TRACE_SUMMARY.read_text()
    except OSError:
        return {}
    out = {}
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0].startswith("`"):
            try:
                out[cells[0].strip("`")] = float(cells[3])
            except ValueError:
                pass
    return out


def measured_mfma_busy() -> dict:
    """Per-launch MFMA-busy fraction of the contraction kernels from the
    committed rocprofv3 --pmc summary (SQ_VALU_MFMA_BUSY_CYCLES over the
    SIMD-cycles of the kernel), keyed by launch name; {} when absent."""
    try:
        text = MFMA_SUMMARY.read_text()
    except OSError:
        return {}
    out = {}
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 3 and cells[0].startswith("`") and cells[0].endswith("`"):
            try:
                out[cells[0].strip("`")] = float(cells[-1])
            except ValueError:
                pass
    return out


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class BlockBench:
    """One DA3-BASE block at 865 tokens (BASELINE config 3 weights and
    input), prepared once so that its timing passes have no host work
    between them and the GPU work before them."""

    def __init__(self, q8_0: bool = False, images: int = 1):
        import vestra_hip as vh
        from vestra_hip import da3, seeded

        self.q8_0 = q8_0
        self.images = images
        self.rt = vh.Runtime(0)
        self.block = self.rt.prepare_block(da3.block_weights(seed=3), q8_0=q8_0)
        self.pos = da3.positions_yx(24, 36)
        self.x = self.rt.upload_f32(seeded.normal(300, images * T * D))
        self.rt.synchronize()

    def step(self) -> None:
        self.rt.vit_block_run(self.block, self.x, self.images, T, self.pos)

    def timed_ms(self, steps: int, warmup: int) -> float:
        """W untimed steps, then K steps between two HIP events; ms per step."""
        for _ in range(warmup):
            self.step()
        self.rt.synchronize()
        self.rt.timer_start()
        for _ in range(steps):
            self.step()
        return self.rt.timer_stop() / steps

    def run(self, steps: int, warmup: int) -> dict:
        rt = self.rt
        ms = self.timed_ms(steps, warmup)
        log(f"timed {steps} {'Q8_0 ' if self.q8_0 else ''}blocks: {ms * steps:.3f} ms")
        rt.profile_reset()
        rt.profile_enable(True)
        for _ in range(steps):
            self.step()
        prof = rt.profile_report()
        rt.profile_enable(False)
        kernels = {}
        for name, (count, ms_tot) in prof.items():
            per_block = count / steps
            avg_us = 1e3 * ms_tot / count
            entry = {"launches_per_block": per_block, "avg_us": round(avg_us, 3)}
            if name in FLOPS:
                tf = FLOPS[name] / (avg_us * 1e-6) / 1e12
                entry.update(tflops=round(tf, 2), frac_fp32_mfma=round(tf / PEAK_FP32_MFMA_TFLOPS, 4))
            if name in INT8_OPS:
                entry.update(top_s=round(INT8_OPS[name] / (avg_us * 1e-6) / 1e12, 2))
            if name in BYTES:
                gbs = BYTES[name] / (avg_us * 1e-6) / 1e9
                entry.update(gbs=round(gbs, 1), frac_hbm=round(gbs / PEAK_HBM_GBS, 4))
            kernels[name] = entry
            log(f"  {name:22s} x{per_block:.0f}/block avg {avg_us:9.2f} us " +
                (f"{entry.get('tflops', 0):7.2f} TF/s" if 'tflops' in entry else
                 f"{entry.get('top_s', 0):7.2f} TOP/s" if 'top_s' in entry else
                 f"{entry.get('gbs', 0):7.1f} GB/s" if 'gbs' in entry else ""))
        return {"ms_per_step": ms, "kernels": kernels}

    def settle(self, ms: float) -> int:
        """Untimed blocks for `ms` of wall time, synchronising every 20 so the
        queue stays short: the GPU clock ramps over about 50 ms of continuous
        work from idle.  Returns the number of blocks run."""
        self.rt.synchronize()
        t0, n = time.perf_counter(), 0
        while (time.perf_counter() - t0) * 1e3 < ms:
            for _ in range(20):
                self.step()
            n += 20
            self.rt.synchronize()
        return n

    def steady(self, steps: int, warmup: int = 0) -> dict:
        """The timed and profiled passes of run() after CLOCK_SETTLE_MS of
        untimed blocks."""
        blocks = self.settle(CLOCK_SETTLE_MS)
        out = self.run(steps, warmup)
        out["clock_settle"] = {"ms": CLOCK_SETTLE_MS, "blocks": blocks}
        return out


# BASELINE config 5 (4 x 865 tokens, one 3457-token image) and the north
# star's own target, one 504 x 336 image (865 tokens).
ENCODER_CASES = (("encoder_12x_4x865", 4, 24, 36), ("encoder_12x_1x3457", 1, 48, 72),
                 ("encoder_12x_1x865", 1, 24, 36))
ENCODER_LAYERS = 12


def encoder_flops(images: int, tokens: int) -> float:
    """Algorithmic FLOPs of the 12-layer encoder: per layer the four
    projections (2 M N K each, M = images x tokens) and the attention
    (4 H T^2 64 per image)."""
    m = images * tokens
    gemm = 2.0 * m * D * (3 * D + D + F) + 2.0 * m * F * D
    attn = 4.0 * H * tokens * tokens * HD * images
    return ENCODER_LAYERS * (gemm + attn)


def encoder_inputs(images: int, tokens: int):
    """Seeded weights of the 12 layers and the input rows of a case."""
    from vestra_hip import da3

    return ([da3.block_weights(seed=50, layer=l) for l in range(ENCODER_LAYERS)],
            encoder_x(images, tokens))


def encoder_x(images: int, tokens: int):
    """The seeded input rows of a case (without regenerating the weights)."""
    from vestra_hip import seeded

    return seeded.normal(51, images * tokens * D)


# Timed encoder passes per case: at least this many, and at least ENCODER_MIN_MS
# of GPU work.
ENCODER_REPS = 5
ENCODER_MIN_MS = 20.0


def gpu_encoder() -> dict:
    """the 12-layer DA3-BASE encoder (independent seeded
    layers) at 4 images x 865 tokens and at one 1008 x 672 image (3457
    tokens), and the north star's one 504 x 336 image (865 tokens), whole
    encoder between two HIP events, with its algorithmic FLOPs as a
    fraction of the fp32-MFMA peak.  Each case first runs untimed passes
    for CLOCK_SETTLE_MS, as the block does: the host work between cases
    idles the GPU, and a 2 ms case timed right after would run on a
    ramping clock."""
    import vestra_hip as vh
    from vestra_hip import da3

    rt = vh.Runtime(0)
    weights, _ = encoder_inputs(1, T)
    blocks = [rt.prepare_block(w) for w in weights]
    out = {}
    for name, images, gh, gw in ENCODER_CASES:
        tokens = gh * gw + 1
        pos = da3.positions_yx(gh, gw)
        x = rt.upload_f32(encoder_x(images, tokens))
        rt.synchronize()
        # The first pass after the host work, on the clock the idle gap
        # left (for the first case of a size it also grows the runtime's
        # workspaces).
        t0 = time.perf_counter()
        rt.timer_start()
        rt.encoder_run(blocks, x, images, tokens, pos)
        first_ms = rt.timer_stop()
        passes = 1
        while (time.perf_counter() - t0) * 1e3 < CLOCK_SETTLE_MS:
            rt.encoder_run(blocks, x, images, tokens, pos)
            rt.synchronize()
            passes += 1
        settle_ms = (time.perf_counter() - t0) * 1e3
        reps = max(ENCODER_REPS, math.ceil(ENCODER_MIN_MS * passes / settle_ms))
        rt.timer_start()
        for _ in range(reps):
            rt.encoder_run(blocks, x, images, tokens, pos)
        ms = rt.timer_stop() / reps
        flops = encoder_flops(images, tokens)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"images": images, "tokens": tokens, "layers": ENCODER_LAYERS,
                     "ms": round(ms, 3), "us_per_layer": round(ms * 1e3 / ENCODER_LAYERS, 1),
                     "tokens_per_s": round(images * tokens / (ms * 1e-3), 1),
                     "gflop": round(flops / 1e9, 2), "tflops": round(tf, 2),
                     "frac_fp32_mfma": round(tf / PEAK_FP32_MFMA_TFLOPS, 4),
                     "timed_passes": reps, "first_pass_ms": round(first_ms, 3),
                     "clock_settle": {"ms": CLOCK_SETTLE_MS, "passes": passes}}
        log(f"  {name}: {ms:.3f} ms ({tf:.1f} TF/s, {reps} passes after {passes} untimed; "
            f"first pass {first_ms:.3f} ms)")
    return out


def gpu_q8_0(steps: int) -> dict:
    """fc1-shaped Q8_0 path.  X [865, 768] ~ N(0,1)
    quantised on the device each step, W [768, 3072] ~ N(0, 0.02^2)
    quantised along K at load time, C = X_q . W_q [865, 3072] f32."""
    import vestra_hip as vh
    from vestra_hip import seeded

    rt = vh.Runtime(0)
    m, k, n = T, D, F
    x = rt.upload_f32(seeded.normal(11, m * k))
    w = seeded.normal(12, k * n, 0.02).reshape(k, n)
    wq = rt.quantize_q8_0(rt.upload_f32(np.ascontiguousarray(w.T).reshape(-1)), n, k)
    settle_clock(rt, lambda: rt.gemm_q8_0(rt.quantize_q8_0(x, m, k), wq, m, n, k))
    rt.profile_reset()
    rt.profile_enable(True)
    keep = []  # outputs stay alive: no stream-ordered frees between the timed launches
    for _ in range(steps):
        aq = rt.quantize_q8_0(x, m, k)
        keep.append((aq, rt.gemm_q8_0(aq, wq, m, n, k)))
    prof = rt.profile_report()
    rt.profile_enable(False)
    del keep
    q_us = 1e3 * prof["quantize_q8_0"][1] / prof["quantize_q8_0"][0]
    g_event = 1e3 * prof["gemm_q8_0"][1] / prof["gemm_q8_0"][0]
    # A burst of back-to-back GEMMs into one preallocated output
    # (Kernels::gemm_q8_0's own c argument) between two events, reported
    # beside gemm_us (the per-launch events above, each carrying the events'
    # own ~1-2 us): the burst reruns the same operands into the same output,
    # so its caches stay warm, and it is not the headline figure.
    aq = rt.quantize_q8_0(x, m, k)
    c = rt.upload_f32(np.zeros(m * n, np.float32))
    settle_clock(rt, lambda: rt.gemm_q8_0_into(aq, wq, m, n, k, c), CLOCK_SETTLE_MS / 4)
    rt.timer_start()
    for _ in range(steps):
        rt.gemm_q8_0_into(aq, wq, m, n, k, c)
    g_burst = 1e3 * rt.timer_stop() / steps
    g_us = g_event
    gemm_bytes = m * k + m * (k // 32) * 2 + n * k + n * (k // 32) * 2 + m * n * 4
    quant_bytes = m * k * 4 + m * k + m * (k // 32) * 2
    gbs = gemm_bytes / (g_us * 1e-6) / 1e9
    # The bit-exact fold acc + (da * db) * isum is four VALU ops per output
    # and 32-wide block (int-to-float conversion, two multiplies, add): a
    # floor the HBM roofline does not see.
    fold_ops = m * n * (k // 32) * 4
    valu_us = fold_ops / PEAK_VALU_OPS * 1e6
    log(f"  q8_0 quantize {q_us:.2f} us, gemm {g_us:.2f} us per-launch events (burst on the same "
        f"operands {g_burst:.2f}; {gbs:.0f} GB/s algorithmic, fold VALU floor {valu_us:.2f} us)")
    return {"workload": "q8_0_fc1_865", "quantize_us": round(q_us, 3), "gemm_us": round(g_us, 3),
            "gemm_us_source": "per-launch HIP events",
            "gemm_us_burst_same_operands": round(g_burst, 3),
            "gemm_top_s": round(2.0 * m * n * k / (g_us * 1e-6) / 1e12, 1),
            "gemm_algorithmic_bytes": gemm_bytes, "gemm_gbs": round(gbs, 1),
            "gemm_frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "gemm_fold_valu_ops": fold_ops, "gemm_valu_floor_us": round(valu_us, 3),
            "gemm_frac_valu": round(valu_us / g_us, 4), "quantize_algorithmic_bytes": quant_bytes,
            "quantize_gbs": round(quant_bytes / (q_us * 1e-6) / 1e9, 1)}


def gpu_elementwise(reps: int = 20) -> dict:
    """The bandwidth-bound kernels; bytes = the algorithmic reads plus writes.
    Two size classes: the encoder's own shapes (LayerNorm and quantisation
    over 4 x 865 tokens, GELU over the batched fc1 output), and sizes where
    HBM bandwidth decides: working sets of 384-768 MiB, past the 256 MiB
    Infinity Cache that would otherwise serve repeated launches.  A device
    copy of 256 MiB (hipMemcpyAsync) at the same scale gives the bandwidth a
    streaming kernel can reach (`frac_copy`).  Each case is timed twice: a burst of `reps` back-to-back
    launches between two HIP events (`us_burst`, which can include host issue
    time for kernels shorter than one call's host cost) and per-launch event
    pairs (`us_event`, each carrying the events' own ~1-2 us).  Both are upper
    bounds on the kernel's duration; `us` is the smaller.  Each case first
    runs for CLOCK_SETTLE_MS untimed, so that the clock has settled."""
    import vestra_hip as vh
    from vestra_hip import da3, seeded

    rt = vh.Runtime(0)
    g = rt.upload_f32(np.ones(D, np.float32))
    b = rt.upload_f32(np.zeros(D, np.float32))
    cases = []

    def big(seed, n):
        # Large inputs tile one seeded block of 8 Mi values.
        base = seeded.normal(seed, min(n, 8 << 20))
        return np.tile(base, (n + base.size - 1) // base.size)[:n]

    def ln_case(rows):
        x = rt.upload_f32(big(31, rows * D))
        return (f"layernorm {rows}x{D}", lambda: rt.layernorm_f32(x, g, b, rows, D, 1e-6),
                2 * rows * D * 4 + 2 * D * 4, "layernorm")

    def gelu_case(n):
        f = rt.upload_f32(big(32, n))
        return (f"gelu {n}", lambda: rt.gelu_f32_in_place(f), 2 * n * 4, "gelu")

    def add_case(n):
        a1, a2 = rt.upload_f32(np.ones(n, np.float32)), rt.upload_f32(np.ones(n, np.float32))
        return (f"add {n}", lambda: rt.add_f32_in_place(a1, a2), 3 * n * 4, "add")

    def q8_case(rows):
        # Into one preallocated Q8_0 tensor (quantize_row_q8_0(x, out)): an
        # allocating call per launch makes the burst host-bound at this size.
        x = rt.upload_f32(big(33, rows * D))
        out = rt.quantize_q8_0(x, rows, D)
        return (f"quantize_q8_0 {rows}x{D}", lambda: rt.quantize_q8_0_into(x, rows, D, out),
                rows * D * 4 + rows * D + rows * D // 16, "quantize_q8_0")

    def rope_case(heads, grid_h, grid_w):
        n = grid_h * grid_w + 1
        x = rt.upload_f32(big(34, heads * n * HD))
        pos = da3.positions_yx(grid_h, grid_w)
        return (f"rope2d {heads}x{n}x{HD}",
                lambda: rt.rope2d_f32_in_place(x, heads, n, HD, pos, da3.ROPE_FREQ),
                2 * heads * n * HD * 4, "rope2d")

    block_shapes = [ln_case(4 * T), gelu_case(4 * T * F), q8_case(4 * T), rope_case(2 * 4 * H, 24, 36)]
    def copy_case(n):
        src, dst = rt.upload_f32(np.ones(n, np.float32)), rt.upload_f32(np.zeros(n, np.float32))
        return (f"copy {n}", lambda: rt.copy_segment_into_f32(dst, 0, src, 0, n), 2 * n * 4,
                "copy_segment_into")

    at_scale = [copy_case(64 << 20), ln_case(131072), gelu_case(96 << 20), add_case(64 << 20),
                q8_case(131072), rope_case(40 * H, 72, 48)]
    out = {}
    copy_gbs = None  # set by the first bandwidth case, the copy
    for label, cases in (("block_shapes", block_shapes), ("bandwidth_sizes", at_scale)):
        res = {}
        for name, fn, nbytes, prof_name in cases:
            settle_clock(rt, fn)
            rt.timer_start()
            for _ in range(reps):
                fn()  # an output dropped here is recycled by the stream-ordered pool
            us_burst = 1e3 * rt.timer_stop() / reps
            rt.profile_reset()
            rt.profile_enable(True)
            keep = [fn() for _ in range(reps)]
            prof = rt.profile_report()
            rt.profile_enable(False)
            del keep
            us_event = 1e3 * prof[prof_name][1] / prof[prof_name][0]
            us = min(us_burst, us_event)
            gbs = nbytes / (us * 1e-6) / 1e9
            res[name] = {"us": round(us, 2), "us_burst": round(us_burst, 2),
                         "us_event": round(us_event, 2), "gbs": round(gbs, 1),
                         "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": nbytes}
            if label == "bandwidth_sizes":
                if prof_name == "copy_segment_into":
                    copy_gbs = gbs
                res[name]["frac_copy"] = round(gbs / copy_gbs, 4)
            log(f"  {name:28s} {us:8.2f} us {gbs:8.1f} GB/s "
                f"(burst {us_burst:.2f}, per-launch events {us_event:.2f})")
        out[label] = res
    return out


def dpt_values(seed: int, n: int) -> np.ndarray:
    """Seeded uniform [-1, 1) inputs of the DPT cases (GPU and CPU legs)."""
    from vestra_hip import seeded

    return (seeded.uniform01(seed, n) * 2.0 - 1.0).astype(np.float32)


def gpu_dpt(reps: int = 20) -> dict:
    """DPT-head operations at DA3-BASE fusion shapes: a 3x3 convolution
    128 -> 128 over the 144 x 96 map (a residual conv unit), the k4s4
    transposed convolution 96 -> 96 from the 24 x 36 patch grid, the
    align-corners 2x upsample of 128 channels from 72 x 48, and the 3x3
    768 -> 128 convolution of the 12 x 18 level (timed on its own).  Per-launch HIP
    event timing; conv FLOPs are 2 * pixels * out_c * in_c * 9."""
    import vestra_hip as vh

    rt = vh.Runtime(0)
    c, h, w = 128, 96, 144
    x = rt.upload_f32(dpt_values(1, c * h * w))
    wt = dpt_values(2, c * c * 9) * np.float32(1.0 / 34.0)
    conv = rt.prepare_conv2d_f32(c, c, 3, 3, 1, 1, wt, dpt_values(3, c))
    tc, th, tw = 96, 24, 36
    xt = rt.upload_f32(dpt_values(4, tc * th * tw))
    ct = rt.prepare_conv_transpose2d_f32(tc, tc, 4, 4, 4, dpt_values(5, tc * tc * 16),
                                         dpt_values(6, tc))
    rh, rw = 48, 72
    xr = rt.upload_f32(dpt_values(7, c * rh * rw))
    def step():
        conv.run(x, h, w)
        ct.run(xt, th, tw)
        rt.bilinear_resize_align_corners_f32(xr, c, rh, rw, 2 * rh, 2 * rw)

    settle_clock(rt, step)
    rt.profile_reset()
    rt.profile_enable(True)
    keep = []
    for _ in range(reps):
        keep.append(conv.run(x, h, w))
        keep.append(ct.run(xt, th, tw))
        keep.append(rt.bilinear_resize_align_corners_f32(xr, c, rh, rw, 2 * rh, 2 * rw))
    prof = rt.profile_report()
    rt.profile_enable(False)
    del keep
    # The layer_rn convolution of the 12 x 18 level (768 -> 128, 3x3): 8
    # output tiles of K = 6912, whose K the direct route splits 27 ways.
    sc, sh, sw = 768, 12, 18
    xs = rt.upload_f32(dpt_values(8, sc * sh * sw))
    convs = rt.prepare_conv2d_f32(sc, c, 3, 3, 1, 1,
                                  dpt_values(9, c * sc * 9) * np.float32(1.0 / np.sqrt(sc * 9)),
                                  dpt_values(10, c))
    for _ in range(20):
        convs.run(xs, sh, sw)
    rt.synchronize()
    rt.profile_reset()
    rt.profile_enable(True)
    keep = [convs.run(xs, sh, sw) for _ in range(reps)]
    prof_small = rt.profile_report()
    rt.profile_enable(False)
    del keep
    small_us = sum(1e3 * ms / n for n, ms in prof_small.values())
    small_flops = 2.0 * sh * sw * c * sc * 9

    def us(name, per=1):
        n, ms = prof[name]
        return 1e3 * ms / n * per

    flops = 2.0 * h * w * c * c * 9
    conv_parts = {k: us(k) for k in ("conv_to_padded_hwc", "conv_to_hwc", "im2col", "conv_gemm",
                                     "conv_to_chw") if k in prof}
    conv_us = sum(conv_parts.values())
    t_flops = 2.0 * th * tw * tc * tc * 16
    t_parts = {label: us(k) for label, k in (("to_hwc", "conv_transpose_to_hwc"),
                                             ("gemm", "conv_transpose_gemm"),
                                             ("scatter", "patch_scatter")) if k in prof}
    t_us = sum(t_parts.values())
    r_us = us("bilinear_align_corners")
    r_bytes = 4.0 * c * (rh * rw + 4 * rh * rw)
    out = {
        "conv3x3_128_144x96": {
            "us": round(conv_us, 2), "parts_us": {k: round(v, 2) for k, v in conv_parts.items()},
            "tflops": round(flops / (conv_us * 1e-6) / 1e12, 2),
            "gemm_tflops": round(flops / (conv_parts["conv_gemm"] * 1e-6) / 1e12, 2),
            "frac_fp32_mfma": round(flops / (conv_us * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)},
        "conv_transpose_k4s4_96_24x36": {
            "us": round(t_us, 2), "parts_us": {k: round(v, 2) for k, v in t_parts.items()},
            "tflops": round(t_flops / (t_us * 1e-6) / 1e12, 2)},
        "conv3x3_768_128_12x18": {
            "us": round(small_us, 2), "launches": sorted(prof_small),
            "tflops": round(small_flops / (small_us * 1e-6) / 1e12, 2)},
        "resize_align_corners_128_48x72_to_96x144": {
            "us": round(r_us, 2), "gbs": round(r_bytes / (r_us * 1e-6) / 1e9, 1),
            "frac_hbm": round(r_bytes / (r_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)},
    }
    log(f"  dpt conv3x3 {conv_us:.2f} us ({out['conv3x3_128_144x96']['tflops']} TF/s), "
        f"transposed conv {t_us:.2f} us, resize {r_us:.2f} us, "
        f"conv3x3 768->128 on 12x18 {small_us:.2f} us")
    return out


# BASELINE config 2 shapes (K, N) per launch, and the config-1 attention.
PROJ_SHAPES = {"gemm_qkv_rope": (D, 3 * D), "gemm_proj_residual": (D, D),
               "gemm_fc1_gelu": (D, F), "gemm_fc2_residual": (F, D)}


def config2_weights(name: str):
    """BASELINE config 2 inputs of one projection: X ~ N(0,1) [T, K],
    W ~ N(0, 0.02^2) [K, N] row-major, b ~ N(0, 0.01^2) [N]."""
    from vestra_hip import seeded

    k, n = PROJ_SHAPES[name]
    tid = list(PROJ_SHAPES).index(name)
    return (seeded.normal(11 + 10 * tid, T * k), seeded.normal(12 + 10 * tid, k * n, 0.02),
            seeded.normal(13 + 10 * tid, n, 0.01))


def config1_qkv():
    """BASELINE config 1 inputs: Q, K, V ~ N(0,1), [12, 865, 64] each."""
    from vestra_hip import seeded

    return tuple(seeded.normal(1 + i, H * T * HD) for i in range(3))


def gpu_configs(reps: int = 20) -> dict:
    """BASELINE configs 1 and 2 standalone, each on its own stated inputs:
    the config-1 attention (token-major output [865, 768]) and the four
    config-2 projections with bias (vh_linear_run: one GEMM launch with the
    bias epilogue).  Each case first runs for CLOCK_SETTLE_MS untimed (the
    preparation between cases idles the GPU and its clock drops), then
    `reps` launches each between its own pair of HIP events (`us`, the
    analogue of the reference's per-call timing, examples/
    current_shape_bench.rs:24-40; events add 1-2.5 us per launch) and a burst
    of `reps` back-to-back launches between two events (`us_burst`)."""
    import vestra_hip as vh

    rt = vh.Runtime(0)
    q, k, v = (rt.upload_f32(a) for a in config1_qkv())
    cases = [("attention_config1", lambda: rt.flash_attention_f32_da3_base(q, k, v, H, T, True),
              "flash_attention", FLOPS["flash_attention"])]
    keep_alive = []
    for name in PROJ_SHAPES:
        x, w, b = config2_weights(name)
        kk, nn = PROJ_SHAPES[name]
        lin = rt.prepare_linear_f32(kk, nn, w, b)
        xt = rt.upload_f32(x)
        keep_alive.append((lin, xt))
        cases.append((f"{name.split('_')[1]}_config2_{T}x{kk}x{nn}",
                      (lambda lin=lin, xt=xt: lin.run(xt, T)), "gemm_bias_scale",
                      2.0 * T * kk * nn))
    out = {}
    traced = measured_config_trace_us()
    for label, fn, prof_name, flops in cases:
        settle = settle_clock(rt, fn)
        rt.timer_start()
        for _ in range(reps):
            fn()
        us_burst = 1e3 * rt.timer_stop() / reps
        rt.profile_reset()
        rt.profile_enable(True)
        keep = [fn() for _ in range(reps)]
        prof = rt.profile_report()
        rt.profile_enable(False)
        del keep
        us = 1e3 * prof[prof_name][1] / prof[prof_name][0]
        tf = flops / (us * 1e-6) / 1e12
        tf_burst = flops / (us_burst * 1e-6) / 1e12
        out[label] = {"us": round(us, 2), "us_source": "per-launch HIP events",
                      "tflops": round(tf, 2), "frac_fp32_mfma": round(tf / PEAK_FP32_MFMA_TFLOPS, 4),
                      "us_burst": round(us_burst, 2),
                      "frac_fp32_mfma_burst": round(tf_burst / PEAK_FP32_MFMA_TFLOPS, 4),
                      "clock_settle": {"ms": CLOCK_SETTLE_MS, "launches": settle}}
        if label in traced:
            out[label]["trace_us"] = traced[label]
            out[label]["frac_fp32_mfma_trace"] = round(
                flops / (traced[label] * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)
        log(f"  {label:34s} {us:8.2f} us {tf:7.2f} TF/s per-launch events (burst {us_burst:.2f})")
    if traced:
        out["trace_source"] = ("profiles/configs_kernel_trace.md: committed rocprofv3 --kernel-trace "
                               "summary (median over each case's timed launches), not measured in "
                               "this run")
    return out


def cpu_thread_counts() -> list:
    """The CPU timing configurations: 16 threads (the reference's protocol,
    BENCHMARKING.md:16-20) and every core of this process's affinity mask."""
    return [("16_threads", 16), ("affinity_cores", len(os.sched_getaffinity(0)))]


def cpu_median_us(fn, min_runs: int = 10, budget_s: float = 2.0, max_runs: int = 50) -> tuple:
    """Warm-up, then the median of at least min_runs timed runs
    (examples/current_shape_bench.rs:24-40)."""
    fn()
    times = []
    start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - start < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e6, len(times)


def cpu_kernels() -> dict:
    """Per-kernel CPU baselines: the oracle's restatements of the crate's
    AVX-512 kernels on BASELINE config 1/2/4 inputs -- qkv_avx512_column_split
    (36 panels), linear_bias_scale_avx512_rows<6> for out-proj and fc2 (145
    row tiles), linear_avx512_column_split_rows<6> for fc1 (48 panels), the
    QT8 flash attention (12 x 109 query tiles), each at 16 threads and at
    every affinity core; and Kernels::gemm_q8_0 (VNNI), which the crate runs
    on one thread."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from vestra_hip import seeded

    avx = oracle.has_avx512()
    ins = {name: config2_weights(name) for name in PROJ_SHAPES}
    ones = np.ones(F, np.float32)
    q, k, v = config1_qkv()
    work = {
        "gemm_qkv_rope": lambda: oracle.qkv(*ins["gemm_qkv_rope"], T),
        "gemm_proj_residual": lambda: oracle.linear_bias_scale(
            ins["gemm_proj_residual"][0], ins["gemm_proj_residual"][1],
            ins["gemm_proj_residual"][2], ones[:D], T, D, D),
        "gemm_fc1_gelu": lambda: oracle.linear(ins["gemm_fc1_gelu"][0], ins["gemm_fc1_gelu"][1],
                                               T, F, D),
        "gemm_fc2_residual": lambda: oracle.linear_bias_scale(
            ins["gemm_fc2_residual"][0], ins["gemm_fc2_residual"][1],
            ins["gemm_fc2_residual"][2], ones[:D], T, D, F),
        "flash_attention": lambda: oracle.flash_attention_avx512(q, k, v, H, T),
    }
    names = {"gemm_qkv_rope": "qkv_f32_da3_base 865x768x2304",
             "gemm_proj_residual": "linear_bias_scale_f32_da3_base 865x768x768",
             "gemm_fc1_gelu": "linear_f32_da3_base 865x768x3072",
             "gemm_fc2_residual": "linear_bias_scale_f32_da3_base 865x3072x768",
             "flash_attention": "flash_attention_f32_da3_base 12x865x64"}
    out = {}
    for name, fn in work.items():
        entry = {"unit": "us", "kind": "port", "isa": "AVX-512" if avx else "scalar"}
        for label, threads in cpu_thread_counts():
            oracle.set_threads(threads)
            us, runs = cpu_median_us(fn)
            entry[label] = {"value": round(us, 1), "cores": threads, "runs": runs}
        entry.update(value=entry["16_threads"]["value"], cores=16,
                     sample=f"{names[name]}, median of >=10 warm runs per thread count")
        out[name] = entry
        log(f"  cpu {name:22s} 16 threads {entry['16_threads']['value']:9.1f} us, "
            f"{entry['affinity_cores']['cores']} cores {entry['affinity_cores']['value']:9.1f} us")
    oracle.set_threads(0)
    x = seeded.normal(11, T * D)
    w = seeded.normal(12, D * F, 0.02).reshape(D, F)
    aq = oracle.quantize_rows_q8_0(x, T, D)
    bq = oracle.quantize_rows_q8_0(np.ascontiguousarray(w.T).reshape(-1), F, D)
    us, runs = cpu_median_us(lambda: oracle.gemm_q8_0(aq, bq, T, F, D, impl="kernels"),
                             budget_s=0.0)
    out["gemm_q8_0"] = {"value": round(us, 1), "unit": "us", "cores": 1, "kind": "port",
                        "isa": "AVX-512 VNNI" if avx else "scalar", "runs": runs,
                        "sample": "Kernels::gemm_q8_0 865x3072x768 (single-threaded in the "
                                  "crate), median of 10 warm runs"}
    log(f"  cpu gemm_q8_0 (1 thread) {us:9.1f} us")
    return out


def cpu_dpt_conv(budget_s: float) -> dict:
    """The crate's CPU route for the bench's 3x3 convolution: Winograd
    F(2x2, 3x3) with the AVX-512 product (conv::conv3x3_winograd_f2_prepared,
    src/conv.rs:282-302 and 681-829; src/specialized.rs:597-633), the filter
    prepared once as the DPT head prepares it, at 16 threads (`value`) and at
    every core of the affinity mask, median of >= 10 warm runs.  The direct
    conv2d_naive (the definition the crate tests against) is timed beside it
    at 16 threads."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    c, h, w = 128, 96, 144
    x = dpt_values(1, c * h * w)
    wt = dpt_values(2, c * c * 9) * np.float32(1.0 / 34.0)
    b = dpt_values(3, c)
    u = oracle.winograd_f2_filter(wt, c, c)
    isa = "AVX-512" if oracle.has_avx512() else "scalar"
    out = {"unit": "us", "kind": "port", "isa": isa}
    for label, threads in cpu_thread_counts():
        oracle.set_threads(threads)
        us, runs = cpu_median_us(lambda: oracle.conv3x3_winograd_f2(x, c, h, w, None, c, b, u=u),
                                 budget_s=budget_s)
        out[label] = {"value": round(us, 1), "cores": threads, "runs": runs}
    oracle.set_threads(16)
    us, runs = cpu_median_us(lambda: oracle.conv2d_naive(x, c, h, w, wt, c, 3, 3, 1, 1, b),
                             min_runs=5, budget_s=budget_s, max_runs=20)
    oracle.set_threads(0)
    out["conv2d_naive_16_threads"] = {"value": round(us, 1), "cores": 16, "runs": runs}
    out.update(value=out["16_threads"]["value"], cores=16,
               sample=(f"Winograd F(2x2,3x3) 128->128 3x3 at 144x96, prepared filter (median of "
                       f"{out['16_threads']['runs']} warm runs at 16 threads, "
                       f"{out['affinity_cores']['runs']} at {out['affinity_cores']['cores']} "
                       f"affinity cores), C restatement of the crate's {isa} path"))
    return out


def cpu_block(budget_s: float, q8_0: bool = False) -> dict:
    """The oracle's DA3-BASE block (the crate's AVX-512 kernels composed as
    the engine composes them; with q8_0, Kernels::gemm_q8_0 for the four
    projections, single-threaded in the crate), median over a bounded sample
    of blocks, at 16 threads (`value`) and at every core of the affinity
    mask."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from vestra_hip import da3, seeded

    w = da3.block_weights(seed=3)
    x0 = seeded.normal(300, T * D)
    pos = da3.positions_yx(24, 36)
    out = {"unit": "us", "kind": "port"}
    for label, threads in cpu_thread_counts():
        oracle.set_threads(threads)
        state = {"x": x0}

        def step():
            state["x"] = oracle.vit_block(state["x"], w, 1, T, pos, q8_0=q8_0)

        us, runs = cpu_median_us(step, min_runs=3 if q8_0 else 10, budget_s=budget_s, max_runs=200)
        out[label] = {"value": round(us, 1), "cores": threads, "runs": runs}
    oracle.set_threads(0)
    isa = ("AVX-512" if oracle.has_avx512() else "scalar") + (" (VNNI Q8_0 GEMMs)" if q8_0 else "")
    kind = "Q8_0-projection " if q8_0 else ""
    out.update(value=out["16_threads"]["value"], cores=16,
               sample=(f"DA3-BASE {kind}blocks at 865 tokens (median of {out['16_threads']['runs']} "
                       f"warm runs at 16 threads, {out['affinity_cores']['runs']} at "
                       f"{out['affinity_cores']['cores']} affinity cores), C restatement of the "
                       f"crate's {isa} path, {os.cpu_count()} visible CPUs"))
    return out


def cpu_encoder() -> dict:
    """The oracle's 12-layer encoder on each config-5 case (the GPU leg's
    weights and inputs): one warm-up run, then the median of 3 runs, at 16
    threads (`value`) and at every core of the affinity mask."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from vestra_hip import da3

    isa = "AVX-512" if oracle.has_avx512() else "scalar"
    out = {}
    for name, images, gh, gw in ENCODER_CASES:
        tokens = gh * gw + 1
        pos = da3.positions_yx(gh, gw)
        weights, x = encoder_inputs(images, tokens)
        entry = {"unit": "ms", "kind": "port"}
        for label, threads in cpu_thread_counts():
            oracle.set_threads(threads)
            us, runs = cpu_median_us(lambda: oracle.encoder(x, weights, images, tokens, pos),
                                     min_runs=3, budget_s=0.0)
            entry[label] = {"value": round(us * 1e-3, 1), "cores": threads, "runs": runs}
        entry.update(value=entry["16_threads"]["value"], cores=16,
                     sample=(f"12-layer DA3-BASE encoder, {images} x {tokens} tokens (median of 3 "
                             f"warm runs per thread count), C restatement of the crate's {isa} path"))
        out[name] = entry
        log(f"  cpu {name}: 16 threads {entry['16_threads']['value']:.1f} ms, "
            f"{entry['affinity_cores']['cores']} cores {entry['affinity_cores']['value']:.1f} ms")
    oracle.set_threads(0)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # ~17 ms of blocks: the first blocks from an idle GPU run on a ramping clock.
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run 5 residual-add kernels over 16M floats (reads 128 MiB, "
                         "writes 64 MiB each) to scale PMC byte counters")
    ap.add_argument("--only", choices=["q8_0", "elementwise", "dpt", "encoder", "configs", "block",
                                       "block4", "q8_0_block"],
                    help="run one secondary section alone and print its JSON (for profiling "
                         "runs; not the benchmark line)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the DA3 block is sharded by image across GPUs; see the design notes).",
              file=sys.stderr)
        return 2

    if args.only:
        section = {"q8_0": lambda: gpu_q8_0(max(10, min(args.steps, 100))),
                   "elementwise": gpu_elementwise, "dpt": gpu_dpt,
                   "encoder": gpu_encoder, "configs": gpu_configs,
                   "block": lambda: BlockBench().steady(args.steps),
                   "block4": lambda: BlockBench(images=4).steady(args.steps),
                   "q8_0_block": lambda: BlockBench(q8_0=True).steady(args.steps)}[args.only]
        print(json.dumps({args.only: section()}), flush=True)
        return 0

    # cold_start: W warm-up and K timed blocks right after preparation, from
    # an idle GPU whose clock is still low.  value: the same W and K after
    # CLOCK_SETTLE_MS of untimed blocks.  Both blocks are prepared first, so
    # no host work separates the settle from the timed passes.
    f32_block, q8_block_bench = BlockBench(), BlockBench(q8_0=True)
    cold = f32_block.run(args.steps, args.warmup)
    log(f"cold start: {cold['ms_per_step'] * 1e3:.2f} us/block")
    gpu = f32_block.steady(args.steps, args.warmup)
    log(f"after {CLOCK_SETTLE_MS:.0f} ms of untimed blocks: {gpu['ms_per_step'] * 1e3:.2f} us/block")
    q8_block = q8_block_bench.run(max(10, min(args.steps, 100)), args.warmup)
    elementwise = gpu_elementwise()
    dpt = gpu_dpt()
    q8 = gpu_q8_0(max(10, min(args.steps, 100)))
    configs = gpu_configs()
    encoder = gpu_encoder()
    if args.calibrate:
        import vestra_hip as vh

        rt = vh.Runtime(0)
        n = 16 * 1024 * 1024
        a, b = rt.upload_f32(np.ones(n, np.float32)), rt.upload_f32(np.ones(n, np.float32))
        for _ in range(5):
            rt.add_f32_in_place(a, b)
        rt.synchronize()
        log("calibration: 5 x add_kernel over 16M floats (128 MiB read, 64 MiB written)")
    ker = gpu["kernels"]
    gemm_attn = [n for n in FLOPS if n in ker]
    dominant = max(gemm_attn, key=lambda n: ker[n]["avg_us"])
    d = ker[dominant]
    result = {
        "metric": "DA3-BASE ViT block us @504x336 (865 tok); GEMM/attn % fp32-MFMA peak",
        "value": round(gpu["ms_per_step"] * 1e3, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) input, N(0,0.02^2) weights, LayerScale 1e-5)",
        "config": {"workload": "vit_block_865", "images": 1, "tokens": T, "dim": D, "heads": H,
                   "mlp": F, "rope": "2-D axial, theta 100, 24x36 grid"},
        "gemm_attn_pct_fp32_mfma_peak": pct_peak(ker),
        "roofline": {
            "kernel": dominant,
            "bound": "mfma",
            "achieved": d["tflops"],
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": d["frac_fp32_mfma"],
            "traffic": measured_traffic(dominant),
            "traffic_unit": "bytes per launch",
            "traffic_source": ("profiles/block_865_hbm_traffic.md: committed rocprofv3 --pmc "
                               "FETCH_SIZE / WRITE_SIZE summary of this block, not measured "
                               "in this run"),
        },
        "timing": (f"W warm-up then K timed blocks after {CLOCK_SETTLE_MS:.0f} ms of untimed blocks "
                   "(clock_settle), which bring the GPU clock from its idle level to steady; "
                   "cold_start is the same W and K right after preparation from the idle GPU"),
        "clock_settle": gpu["clock_settle"],
        "cold_start": {"us_per_block": round(cold["ms_per_step"] * 1e3, 2),
                       "gemm_attn_pct_fp32_mfma_peak": pct_peak(cold["kernels"]),
                       "kernels": cold["kernels"]},
        "kernels": ker,
        "config1_2_standalone": configs,
        "q8_0": q8,
        "q8_0_block": {"workload": "vit_block_865_q8_0_projections",
                       "us_per_block": round(q8_block["ms_per_step"] * 1e3, 2),
                       "kernels": q8_block["kernels"]},
        "elementwise_at_scale": elementwise,
        "dpt": dpt,
        "encoder": encoder,
    }
    mfma = measured_mfma_busy()
    for name, frac in mfma.items():
        if name in ker:
            ker[name]["mfma_busy_frac"] = frac
    if mfma:
        result["mfma_busy_source"] = ("profiles/block_865_mfma_busy.md: committed rocprofv3 "
                                      "--pmc summary, not measured in this run")
    trace = measured_trace_us()
    for name, us in trace.items():
        if name in ker and name in FLOPS:
            ker[name]["trace_us"] = round(us, 2)
            ker[name]["frac_fp32_mfma_trace"] = round(FLOPS[name] / (us * 1e-6) / 1e12 /
                                                     PEAK_FP32_MFMA_TFLOPS, 4)
    if trace:
        result["trace_source"] = ("profiles/block_865_kernel_trace.md: committed rocprofv3 "
                                  "--kernel-trace summary (medians over its block launches), not "
                                  "measured in this run; avg_us and frac_fp32_mfma are this run's "
                                  "per-launch HIP events, which add 1-2.5 us per launch")
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_block(args.cpu_seconds)
        cpu_k = cpu_kernels()
        for name, entry in cpu_k.items():
            if name in ker:
                ker[name]["cpu_baseline"] = entry
        configs["attention_config1"]["cpu_baseline"] = cpu_k["flash_attention"]
        for label in configs:
            for name in PROJ_SHAPES:
                if label.startswith(name.split("_")[1] + "_config2"):
                    configs[label]["cpu_baseline"] = cpu_k[name]
        q8["gemm_cpu_baseline"] = cpu_k["gemm_q8_0"]
        result["q8_0_block"]["cpu_baseline"] = cpu_block(2.0, q8_0=True)
        for name, entry in cpu_encoder().items():
            encoder[name]["cpu_baseline"] = entry
        dpt["conv3x3_128_144x96"]["cpu_baseline"] = cpu_dpt_conv(5.0)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
