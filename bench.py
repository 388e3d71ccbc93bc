"""Benchmark of the affine 4-bit quantized linear path on one MI355X.

Prints ONE JSON line.  The headline ("value") is the qGEMM throughput in
TFLOP/s at M=4608, K=3072, N=18432 (the DiT MLP-in projection at 1024^2,
bf16 activations, 4-bit group-64 weights); one "step" is one qGEMM launch
over that synthetic batch, inputs resident in HBM.  The same line carries:

* roofline   -- the qGEMM against the dense bf16 MFMA peak (2.5 PFLOP/s, quoted
                at a 2400 MHz engine clock), and against that peak scaled to
                the engine clock the GPU held while the headline ran;
* device     -- engine / memory clock, board power, power cap and junction
                temperature from the GPU's sysfs node: idle, averaged over the
                loaded headline, and after it;
* dense_bf16_reference -- the vendor dense GEMM (hipBLASLt via torch.matmul)
                on the headline shape with the weights already bf16, same box,
                with the clock and power it ran at (a reference point only);
* qgemv      -- M=1/4/16 on the text-encoder MLP shapes [9728x2560] and
                [2560x9728], GB/s of algorithmic bytes against 8 TB/s, with the
                weights rotated over enough copies to miss the 256 MB MALL
                (a captured graph of 48 launches), and one launch alone after
                a 512 MiB read that evicts every cache (single_us);
* qgemv_f32  -- the conditioner's M=1 f32 qmm ([18432x3072], [3072x256]), GB/s;
* dequant    -- the two projections of a DiT single-stream block, GB/s;
* prescale   -- the f16 sandwich's pre-scale cast (x / 16 to f16) on [4608x3072] float32, GB/s;
* qgemm_shapes -- the other qGEMM shapes (PR1 1024x9216x3072, single-block
                pair);
* qmm_small_m -- text-encoder shapes at M = 32, 128, 512 through the regime
                dispatcher (K split when the output tiles are too few);
* dit_single_block -- one DiT single-stream block's projections at 1024^2
                (f16): to_qkv_mlp_proj with the SwiGLU fused into its epilogue,
                to_out with the gated residual add fused;
* dit_step     -- a whole DiT step's quantized linear layers (5 double + 20
                single blocks, l_img 4096 + l_txt 512, f16, random-init packed
                weights of the model's shapes) replayed as one HIP graph;
* upload       -- the loader's host -> device path (pinned double buffer, each
                chunk filled by four host threads) in GB/s;
* cpu_baseline -- the C oracle's f32-accumulating CPU quantized matmul
                (MLX is not available) on a bounded sample of the same problem.

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 100] [--no-cpu-baseline]

Before its W warmup steps the headline runs untimed launches for 1 s, so
the clock and power state have settled whatever W is: under a sustained dense
MFMA load the board reaches its power cap and the engine clock settles well
below its 2400 MHz maximum within about 0.7 s.
"""

from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "4-bit qGEMM TFLOP/s (% MFMA peak) at M=4608; qGEMV GB/s (% HBM) at M=1"
PREWARM_S = 1.0  # untimed launches before the warmup steps of the headline
STEADY_S = 0.5   # the clock / power readings averaged: the pre-warm's last STEADY_S + the timed steps
MAX_SCLK_MHZ = 2400.0  # the engine clock the dense MFMA peak is quoted at
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
TARGET = (4608, 18432, 3072)  # M, N, K
# Text-encoder prefill and splice rows, and the reference's published qmm shape
# (M = 512, K = 2560, N = 4096), through the regime dispatcher.
MID_M_SHAPES = ((32, 9728, 2560), (128, 9728, 2560), (512, 9728, 2560), (512, 2560, 9728),
                (512, 4096, 2560))


def qmm_bytes(m: int, n: int, k: int) -> int:
    """Algorithmic bytes of one call: bf16 x and y, packed W, bf16 scales+biases."""
    return 2 * m * k + n * k // 2 + 4 * n * k // 64 + 2 * m * n


def dequant_bytes(n: int, k: int) -> int:
    return n * k // 2 + 4 * n * k // 64 + 2 * n * k


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


@contextlib.contextmanager
def no_gc(collect: bool = False):
    """Python's cyclic collector off inside a timed region: a full collection
    of this process's objects takes 20-40 ms, and inside a host-bound timed
    loop (the conditioning chain's one-timestep calls) it would be timed as
    the library's (20 calls of 45 us read as 2 ms each when one landed there).
    collect: run one first -- only where a pre-warm follows, since the GPU
    idles through it and its clock drops (timed right after one, the tile
    kernel's shapes ran 15-18% slower)."""
    was = gc.isenabled()
    if collect and was:
        gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def time_events(fn, reps: int) -> float:
    """Average milliseconds per fn() over reps back-to-back calls (HIP events on
    torch's current stream, the stream the library launches on)."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with no_gc():
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


class GpuState:
    """The GPU's engine clock, memory clock, board power, power cap and
    temperatures, read from its amdgpu sysfs node (found by the PCI address
    torch reports).  The power and clock readings are the firmware's running
    averages, refreshed every few ms; a reading that fails is left out."""

    def __init__(self, torch):
        props = torch.cuda.get_device_properties(0)
        self.dev = (f"/sys/bus/pci/devices/{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:"
                    f"{props.pci_device_id:02x}.0")
        hw = os.path.join(self.dev, "hwmon")
        names = sorted(os.listdir(hw)) if os.path.isdir(hw) else []
        self.hwmon = os.path.join(hw, names[0]) if names else None

    @staticmethod
    def _read(path):
        try:
            with open(path) as f:
                return f.read()
        except OSError:
            return None

    def _level(self, name):
        """MHz of the current level of pp_dpm_<name> (the line marked '*')."""
        txt = self._read(os.path.join(self.dev, name))
        for line in (txt or "").splitlines():
            if line.rstrip().endswith("*"):
                try:
                    return int(line.split(":")[1].strip().lower().split("mhz")[0])
                except (IndexError, ValueError):
                    return None
        return None

    def _hw(self, name, scale):
        if not self.hwmon:
            return None
        txt = self._read(os.path.join(self.hwmon, name))
        try:
            return round(int(txt) / scale, 1) if txt else None
        except ValueError:
            return None

    def snapshot(self) -> dict:
        snap = {"sclk_mhz": self._level("pp_dpm_sclk"), "mclk_mhz": self._level("pp_dpm_mclk"),
                "power_w": self._hw("power1_input", 1e6) or self._hw("power1_average", 1e6),
                "power_cap_w": self._hw("power1_cap", 1e6),
                "temp_junction_c": self._hw("temp2_input", 1e3),
                "temp_mem_c": self._hw("temp3_input", 1e3)}
        return {k: v for k, v in snap.items() if v is not None}


class StateSampler:
    """Samples GpuState every ~20 ms on a host thread while work runs;
    summary(since) averages the samples taken after `since` seconds."""

    def __init__(self, state: GpuState):
        import threading

        self.state = state
        self.samples = []
        self._stop = threading.Event()
        self._t0 = time.perf_counter()
        self._th = threading.Thread(target=self._run, daemon=True)

    def _run(self):
        while not self._stop.is_set():
            self.samples.append((time.perf_counter() - self._t0, self.state.snapshot()))
            self._stop.wait(0.02)

    def __enter__(self):
        self._th.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._th.join()

    def elapsed(self) -> float:
        return time.perf_counter() - self._t0

    def summary(self, since: float = 0.0) -> dict:
        rows = [snap for t, snap in self.samples if t >= since]
        out = {"samples": len(rows)}

        def vals(key):
            return [r[key] for r in rows if key in r]

        if v := vals("sclk_mhz"):
            out.update(sclk_mhz=round(sum(v) / len(v), 1), sclk_min_mhz=min(v),
                       sclk_max_mhz=max(v))
        if v := vals("power_w"):
            out.update(power_w=round(sum(v) / len(v), 1), power_max_w=max(v))
        if v := vals("temp_junction_c"):
            out.update(temp_junction_max_c=max(v))
        return out


def time_single(fn_list, flush, reps: int = 24) -> float:
    """Median milliseconds of ONE launch: before each, `flush` overwrites a
    buffer larger than the 256 MB MALL (so the launch reads its operands from
    HBM), then HIP events on torch's current stream bracket fn_list[i] alone."""
    import torch

    times = []
    with no_gc():
        for r in range(reps):
            flush()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            fn_list[r % len(fn_list)]()
            end.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(end))
    times.sort()
    return times[len(times) // 2]


def mall_flush(torch):
    """A function that reads 512 MiB (twice the MALL) and so leaves no
    operand of the next launch in any cache."""
    buf = torch.ones(128 << 20, dtype=torch.int32, device="cuda")
    return lambda: buf.amax()


def time_graph(launches, replays: int = 5) -> float:
    """Average milliseconds per launch of a captured back-to-back sequence.
    The warm-up and the capture share one stream, so a split-K workspace the
    warm-up grew is the one the graph uses."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in launches:
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for f in launches:
            f()
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with no_gc():
        start.record()
        for _ in range(replays):
            g.replay()
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * len(launches))


def bench_qgemv(imq, synth, torch, copies: int = 48, ms_list=(1, 4, 16),
                few_rows=(4, 8, 16)) -> dict:
    """The qGEMV at M in ms_list, and the regime dispatcher at M in few_rows (the
    weight-streaming matrix-core kernel), weights rotated over `copies` copies."""
    out = {}
    flush = mall_flush(torch)
    for (n, k) in ((9728, 2560), (2560, 9728)):
        p = synth.make_problem(16, n, k, seed=0)
        x, w, s, b = synth.to_device(p)
        ws = [w.clone() for _ in range(copies)]
        ss = [s.clone() for _ in range(copies)]
        bs = [b.clone() for _ in range(copies)]
        del w, s, b
        for m, fn, tag in ([(m, imq.qgemv, "qgemv") for m in ms_list]
                           + [(m, imq.quantized_matmul, "qmm_t") for m in few_rows]):
            xm = x[:m].contiguous()
            ys = [torch.empty((m, n), dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
            launches = [(lambda i=i, fn=fn: fn(xm, ws[i], ss[i], bs[i], out=ys[i]))
                        for i in range(copies)]
            ms = time_graph(launches)
            one = time_single(launches, flush)
            byts = qmm_bytes(m, n, k)
            gbs = byts / (ms * 1e-3) / 1e9
            key = f"M{m}_N{n}_K{k}" if tag == "qgemv" else f"qmm_t_M{m}_N{n}_K{k}"
            out[key] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                        "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": byts,
                        "single_us": round(one * 1e3, 3),
                        "single_GB/s": round(byts / (one * 1e-3) / 1e9, 1)}
            log(f"{tag} M={m} N={n} K={k}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s "
                f"(one cold launch: {one * 1e3:.2f} us)")
        del ws, ss, bs
        # The floor one launch of this size reaches: a device copy moving the
        # M=1 call's bytes (half read, half written), rotated the same way.
        byts = qmm_bytes(1, n, k)
        words = byts // 8
        src = [torch.empty(words, dtype=torch.int32, device="cuda") for _ in range(copies)]
        dst = [torch.empty(words, dtype=torch.int32, device="cuda") for _ in range(copies)]
        launches = [(lambda i=i: dst[i].copy_(src[i])) for i in range(copies)]
        ms = time_graph(launches)
        one = time_single(launches, flush)
        gbs = 8 * words / (ms * 1e-3) / 1e9
        qg = out[f"M1_N{n}_K{k}"] if 1 in ms_list else None
        out[f"copy_floor_N{n}_K{k}"] = {
            "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "bytes": 8 * words,
            "single_us": round(one * 1e3, 3),
            "qgemv_M1_vs_copy": round(ms * 1e3 / qg["us"], 3) if qg else None,
            "qgemv_M1_vs_copy_single": round(one * 1e3 / qg["single_us"], 3) if qg else None}
        log(f"device copy of the M=1 bytes ({8 * words} B moved): {ms * 1e3:.2f} us  "
            f"{gbs:.0f} GB/s, one cold launch {one * 1e3:.2f} us"
            + (f"  (qGEMV M=1 at {ms * 1e3 / qg['us']:.2f} of its rate, "
               f"{one * 1e3 / qg['single_us']:.2f} single)" if qg else ""))
        del src, dst
        torch.cuda.empty_cache()
    return out


def bench_fused_decode(imq, synth, torch, copies: int = 48) -> dict:
    """Projections that share x at decode sizes as one launch: the text
    encoder's gate and up ([9728 x 2560] each, rows concatenated) with the
    SiLU-mul stage (qmm_swiglu; the qGEMV's pair mode at M <= 4), and q/k/v
    ([4096 + 1024 + 1024 rows x 2560], one plain call), beside the single
    [9728 x 2560] launch; weights rotated over `copies` copies (from HBM)."""
    out = {}
    k, inter = 2560, 9728
    for tag, n_rows in (("gate_up_swiglu", 2 * inter), ("qkv", 6144)):
        p = synth.make_problem(4, n_rows, k, seed=7)
        x, w, s, b = synth.to_device(p)
        ws = [w.clone() for _ in range(copies)]
        ss = [s.clone() for _ in range(copies)]
        bs = [b.clone() for _ in range(copies)]
        del w, s, b
        for m in (1, 4):
            xm = x[:m].contiguous()
            width = inter if tag == "gate_up_swiglu" else n_rows
            ys = [torch.empty((m, width), dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
            if tag == "gate_up_swiglu":
                launches = [(lambda i=i: imq.qmm_swiglu(xm, ws[i], ss[i], bs[i], inter, 0, inter,
                                                        out=ys[i])) for i in range(copies)]
            else:
                launches = [(lambda i=i: imq.quantized_matmul(xm, ws[i], ss[i], bs[i], out=ys[i]))
                            for i in range(copies)]
            ms = time_graph(launches)
            byts = 2 * m * k + n_rows * k // 2 + 4 * n_rows * k // 64 + 2 * m * width
            gbs = byts / (ms * 1e-3) / 1e9
            out[f"{tag}_M{m}_N{n_rows}_K{k}"] = {
                "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": byts}
            log(f"{tag} M={m} N={n_rows} K={k}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s")
        del ws, ss, bs
        torch.cuda.empty_cache()
    return out


def bench_qgemv_f32(imq, synth, torch, copies: int = 24) -> dict:
    """The conditioner's M=1 qmm with f32 x, scales, biases and y
    (DirectConditioner.swift:48,75-84): its largest projection [18432x3072]
    and a [3072x256] one, weights rotated over enough copies to miss the MALL."""
    out = {}
    for (n, k) in ((18432, 3072), (3072, 256)):
        p = synth.make_problem(1, n, k, seed=5)
        x, w, s, b = synth.to_device(p)
        x, s, b = x.float(), s.float(), b.float()
        reps = copies if n * k >= (1 << 24) else 4
        ws = [w.clone() for _ in range(reps)]
        ss = [s.clone() for _ in range(reps)]
        bs = [b.clone() for _ in range(reps)]
        ys = [torch.empty((1, n), dtype=torch.float32, device="cuda") for _ in range(reps)]
        launches = [(lambda i=i: imq.quantized_matmul(x, ws[i], ss[i], bs[i], out=ys[i]))
                    for i in range(reps)]
        ms = time_graph(launches)
        byts = 4 * k + n * k // 2 + 2 * 4 * n * (k // 64) + 4 * n
        gbs = byts / (ms * 1e-3) / 1e9
        out[f"M1_N{n}_K{k}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": byts}
        log(f"qgemv f32 M=1 N={n} K={k}: {ms * 1e3:.2f} us  {gbs:.0f} GB/s")
        del ws, ss, bs, ys
        torch.cuda.empty_cache()
    return out


def bench_cond_chain(torch) -> dict:
    """The DiT's conditioning chain (DirectConditioner.stepConditioning) at FLUX.2
    klein sizes: dim 3072, sin_dim 256, the four modulation heads concatenated
    (52224 rows), f32 parameters; all timesteps of a call in one pass (the
    reference runs six M = 1 dispatches with a blocking wait each per timestep).
    Device time per call from HIP events, host sinusoid and copy included."""
    from aestrix_amd.cond import Conditioner, random_conditioner

    l1, l2, heads = random_conditioner(3072, 256, seed=3)
    cond = Conditioner(l1, l2, heads)
    byts = sum(q.n * q.k // 2 + 2 * 4 * q.n * (q.k // 64) for q in (l1, l2, heads))
    out = {"weight_bytes": byts}
    for count in (1, 4):
        t = [1000.0 * (i + 1) / count for i in range(count)]
        temb = torch.empty((count, 3072), device="cuda")
        hd = torch.empty((count, heads.n), device="cuda")
        for _ in range(3):
            cond.run(t, temb, hd)
        ms = time_events(lambda: cond.run(t, temb, hd), 20)
        gbs = byts / (ms * 1e-3) / 1e9
        out[f"timesteps{count}"] = {"us": round(ms * 1e3, 2), "GB/s_weights": round(gbs, 1),
                                    "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"conditioning chain, {count} timesteps: {ms * 1e3:.1f} us ({gbs:.0f} GB/s of weights)")
    cond.close()
    return out


def bench_te_layer(torch, rows_list=(512, 30, 16, 8, 4, 1)) -> dict:
    """One Qwen3 4B text-encoder layer's quantized-linear work (imq_te: RMSNorm +
    q/k/v; o_proj + dq_add, RMSNorm, gate/up + dq_silu_mul, down_proj + dq_add)
    at the padded window L = 512, the splice regime L = 30 and a few shorter
    windows (DirectTEEncoder.swift:249-412), bf16, graph-timed over 27 layers."""
    from aestrix_amd.te import TextEncoderLayers, random_te_layers

    layers = random_te_layers(27, dtype=torch.bfloat16, seed=4)
    te = TextEncoderLayers(layers, max_rows=512)
    out = {}
    flop_per_row = 2.0 * (6144 * 2560 + 2560 * 4096 + 2 * 9728 * 2560 + 2560 * 9728)
    for rows in rows_list:
        x = torch.randn((rows, 2560), device="cuda").bfloat16()
        attn = torch.randn((rows, 4096), device="cuda").bfloat16()
        qkv = torch.empty((rows, 6144), dtype=torch.bfloat16, device="cuda")
        h = [torch.empty_like(x) for _ in range(2)]
        launches = []
        for i in range(27):
            src = x if i == 0 else h[(i - 1) % 2]
            launches.append(lambda i=i, src=src: te.attn_in(i, src, qkv))
            launches.append(lambda i=i, src=src: te.attn_out_mlp(i, src, attn, h[i % 2]))
        ms = time_graph(launches) * len(launches) / 27
        tf = flop_per_row * rows / (ms * 1e-3) / 1e12
        out[f"L{rows}"] = {"us_per_layer": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1)}
        log(f"TE layer L={rows}: {ms * 1e3:.1f} us per layer  {tf:.1f} TFLOP/s")
    te.close()
    del layers
    torch.cuda.empty_cache()
    return out


def bench_dequant(imq, synth, torch, copies: int = 6) -> dict:
    out = {}
    flush = mall_flush(torch)
    for (n, k) in ((27648, 3072), (3072, 12288)):
        p = synth.make_problem(0, n, k, seed=1)
        _, w, s, b = synth.to_device(p)
        ws = [w.clone() for _ in range(copies)]
        ss = [s.clone() for _ in range(copies)]
        bs = [b.clone() for _ in range(copies)]
        os_ = [torch.empty((n, k), dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
        launches = [(lambda i=i: imq.dequantize(ws[i], ss[i], bs[i], out=os_[i]))
                    for i in range(copies)]
        ms = time_graph(launches, replays=4)
        one = time_single(launches, flush, reps=12)
        byts = dequant_bytes(n, k)
        gbs = byts / (ms * 1e-3) / 1e9
        out[f"N{n}_K{k}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                             "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": byts,
                             "single_us": round(one * 1e3, 2),
                             "single_GB/s": round(byts / (one * 1e-3) / 1e9, 1)}
        log(f"dequant N={n} K={k}: {ms * 1e3:.1f} us  {gbs:.0f} GB/s "
            f"(one cold launch: {one * 1e3:.1f} us)")
        del ws, ss, bs, os_
        torch.cuda.empty_cache()
    return out


def bench_prescale(imq, torch, copies: int = 4) -> dict:
    """The f16 sandwich's pre-scale cast (x / 16 to f16) on the single block's input
    [4608 x 3072] float32: 6 bytes per element, buffers rotated past the MALL."""
    m, k = 4608, 3072
    xs = [torch.randn((m, k), device="cuda") for _ in range(copies)]
    ys = [torch.empty((m, k), dtype=torch.float16, device="cuda") for _ in range(copies)]
    launches = [(lambda i=i: imq.cast_prescale(xs[i], 16.0, torch.float16, out=ys[i]))
                for i in range(copies)]
    ms = time_graph(launches, replays=4)
    byts = m * k * 6
    gbs = byts / (ms * 1e-3) / 1e9
    log(f"prescale [{m}x{k}] f32 -> f16: {ms * 1e3:.1f} us  {gbs:.0f} GB/s")
    del xs, ys
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": byts}


def bench_rmsnorm(imq, torch, copies: int = 4) -> dict:
    """RMSNorm into a qmm input: the DiT's fp32 residual [4608 x 3072] to f16
    (6 bytes per element) and the text encoder's bf16 stream [512 x 2560] to bf16
    (4 bytes per element), buffers rotated past the MALL for the first."""
    out = {}
    for tag, (m, k), xdt, ydt, per in (("dit_f32_to_f16", (4608, 3072), torch.float32, torch.float16, 6),
                                        ("te_bf16", (512, 2560), torch.bfloat16, torch.bfloat16, 4)):
        xs = [torch.randn((m, k), device="cuda").to(xdt) for _ in range(copies)]
        ys = [torch.empty((m, k), dtype=ydt, device="cuda") for _ in range(copies)]
        w = torch.ones(k, device="cuda")
        # 32 launches per graph: a graph of a few microsecond-long kernels
        # would otherwise be timed by its own launch latency.
        launches = [(lambda i=i: imq.rmsnorm(xs[i % copies], w, 1e-5, out_dtype=ydt,
                                             out=ys[i % copies])) for i in range(32)]
        ms = time_graph(launches, replays=4)
        byts = m * k * per + 4 * k
        gbs = byts / (ms * 1e-3) / 1e9
        out[tag] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                    "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "bytes": byts}
        log(f"rmsnorm {tag} [{m}x{k}]: {ms * 1e3:.1f} us  {gbs:.0f} GB/s")
        del xs, ys
    torch.cuda.empty_cache()
    return out


def bench_x_embedder(imq, synth, torch) -> dict:
    """The DiT's x_embedder sandwich at 1024^2 (latents [4096 x 128] f32 / 16 to f16,
    the qmm with K = 128 -- the register-staged tile kernel, K % 256 != 0 -- and
    the x16 post-scale into f32 [4096 x 3072])."""
    m, n, k = 4096, 3072, 128
    p = synth.make_problem(1, n, k, seed=6)
    _, w, s, b = synth.to_device(p)
    lin = imq.QuantizedLinear(w, s.half(), b.half())
    lat = torch.randn((m, k), device="cuda")
    y = torch.empty((m, n), device="cuda")
    x16 = torch.empty((m, k), dtype=torch.float16, device="cuda")
    # Six sandwiches per captured graph (one launch pair per graph would time
    # the graph launch more than the kernels).
    launches = [lambda: imq.cast_prescale(lat, 16.0, torch.float16, out=x16),
                lambda: imq.qmm_postscale(x16, lin.weight, lin.scales, lin.biases, 16.0, out=y)]
    ms = time_graph(launches * 6, replays=10) * 2
    qmm_ms = time_graph(launches[1:] * 12, replays=10)
    tf = 2.0 * m * n * k / (qmm_ms * 1e-3) / 1e12
    byts = m * n * 4 + m * k * 2 + n * k // 2
    log(f"x_embedder sandwich M={m} N={n} K={k}: {ms * 1e3:.1f} us (qmm + post-scale "
        f"{qmm_ms * 1e3:.1f} us, {tf:.1f} TFLOP/s, {byts / (qmm_ms * 1e-3) / 1e9:.0f} GB/s)")
    return {"us": round(ms * 1e3, 2), "qmm_postscale_us": round(qmm_ms * 1e3, 2),
            "TFLOP/s": round(tf, 1), "GB/s": round(byts / (qmm_ms * 1e-3) / 1e9, 1)}


def bench_dense_bf16(torch, imq, x, w, s, b, gpu: GpuState, steps: int = 20) -> dict:
    """A reference point on the same box, not part of the product: the vendor
    dense GEMM (hipBLASLt through torch.matmul) on the headline shape with the
    weights already dequantized to bf16 (4x the weight bytes, no dequant work),
    timed like the headline, with the clock and power it runs at."""
    m, k = x.shape
    n = w.shape[0]
    wt = imq.dequantize(w, s, b).t().contiguous()  # [K, N] bf16
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    with StateSampler(gpu) as smp, no_gc(collect=True):
        t_pre = time.perf_counter()
        while time.perf_counter() - t_pre < PREWARM_S:
            for _ in range(20):
                torch.matmul(x, wt, out=y)
            torch.cuda.synchronize()
        steady_from = smp.elapsed() - STEADY_S
        ms = time_events(lambda: torch.matmul(x, wt, out=y), steps)
    loaded = smp.summary(since=steady_from)
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    log(f"dense bf16 reference (torch.matmul, hipBLASLt) M={m} N={n} K={k}: {ms:.4f} ms  "
        f"{tf:.1f} TFLOP/s  loaded: {loaded}")
    del wt, y
    out = {"what": "torch.matmul (hipBLASLt) on the dequantized bf16 weights, same shape and box",
           "ms": round(ms, 5), "TFLOP/s": round(tf, 1),
           "frac_mfma": round(tf / PEAK_BF16_TFLOPS, 4), "loaded": loaded}
    if sclk := loaded.get("sclk_mhz"):
        out["frac_at_loaded_clock"] = round(tf / (PEAK_BF16_TFLOPS * sclk / MAX_SCLK_MHZ), 4)
    return out


def bench_qgemm_shape(imq, synth, torch, m, n, k, reps=10, dispatcher=False) -> dict:
    """One qGEMM shape: imq_qgemm (the tile kernel), or with dispatcher=True
    imq_qmm_t (which may split K for shapes with few output tiles)."""
    p = synth.make_problem(m, n, k, seed=0)
    x, w, s, b = synth.to_device(p)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    fn = imq.quantized_matmul if dispatcher else imq.qgemm
    # Warm up for about 60 ms of MFMA work (past the clock transient).
    warm = max(2, min(2000, int(60e-3 * 1e15 / (2.0 * m * n * k))))
    for _ in range(warm):
        fn(x, w, s, b, out=y)
    if dispatcher:  # microseconds per call: a captured graph keeps host launches out
        ms = time_graph([lambda: fn(x, w, s, b, out=y)] * 20)
    else:
        ms = time_events(lambda: fn(x, w, s, b, out=y), max(reps, 20))
    tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    log(f"{'qmm_t' if dispatcher else 'qgemm'} M={m} N={n} K={k}: {ms:.3f} ms  {tf:.1f} TFLOP/s")
    return {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / PEAK_BF16_TFLOPS, 4)}


def cpu_baseline(synth, seconds: float = 10.0) -> dict:
    """The C oracle's f32-accumulating CPU quantized matmul on rows of the
    target problem, repeated for about `seconds` (MLX is not available)."""
    import numpy as np

    from oracle import cref

    m, n, k = TARGET
    rows = 32
    p = synth.make_problem(rows, n, k, seed=0)
    threads = cref.max_threads()
    cref.qmm_t_f32acc(p.x[:2], p.w[:256], p.scales[:256], p.biases[:256])  # warm
    calls = 0
    t0 = time.perf_counter()
    while True:
        cref.qmm_t_f32acc(p.x, p.w, p.scales, p.biases)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    flop = 2.0 * rows * n * k * calls
    del np
    return {"value": round(flop / el / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"MLX-equivalent CPU qmm (MLX unavailable): C oracle, on-the-fly bf16 dequant, "
                      f"f32 accumulate, bf16 out; {rows} rows x N={n} x K={k} of the seed-0 "
                      f"target problem, {calls} calls in {el:.1f} s on {threads} OpenMP threads"}


def floors(torch) -> int:
    """Reference kernels for reading kernel durations under rocprofv3: a
    one-element fill (the launch floor) and device-to-device copies of
    6225920 bytes between 48 distinct buffer pairs (12.45 MB of HBM traffic
    per launch, the qGEMV weight size, past the 256 MB MALL)."""
    t = torch.empty(1, dtype=torch.float32, device="cuda")
    for _ in range(200):
        t.zero_()
    words = 9728 * 2560 // 16
    src = [torch.ones(words, dtype=torch.int32, device="cuda") for _ in range(48)]
    dst = [torch.empty(words, dtype=torch.int32, device="cuda") for _ in range(48)]
    for _ in range(5):
        for a, b in zip(src, dst):
            b.copy_(a)
    torch.cuda.synchronize()
    log(f"floors: 200 one-element fills; 240 copies of {words * 4} bytes")
    return 0


def bench_dit_single_block(imq, torch) -> dict:
    """Single-stream block projections at J=4608 (f16): QKV part of
    to_qkv_mlp_proj (9216 rows), its MLP part with SwiGLU fused (2 x 9216 rows
    -> 9216 outputs), to_out (K=12288) with the gated residual fused."""
    from aestrix_amd.step import random_projections, DitDims
    d = DitDims(n_double=0, n_single=1)
    proj, out_w = random_projections(d, torch.float16, seed=3)
    J, dim, ffi = d.joint, d.dim, d.ff_inner
    nx = torch.randn((J, dim), device="cuda").half()
    qkv = torch.empty((J, 3 * dim), dtype=torch.float16, device="cuda")
    concat = torch.zeros((J, dim + ffi), dtype=torch.float16, device="cuda")
    x = torch.randn((J, dim), device="cuda")
    gate = torch.ones(dim, device="cuda")
    w3, s3, b3 = proj.w[:3 * dim], proj.s[:3 * dim], proj.b[:3 * dim]

    def block():
        imq.quantized_matmul(nx, w3, s3, b3, out=qkv)
        imq.qmm_swiglu(nx, proj.w, proj.s, proj.b, ffi, 3 * dim, 3 * dim + ffi,
                       out=concat[:, dim:])
        imq.qmm_gate_add(concat, out_w.w, out_w.s, out_w.b, x, gate, 1.0, out=x)

    for _ in range(5):
        block()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with no_gc():
        e0.record()
        for _ in range(20):
            block()
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 20
    flop = 2.0 * J * dim * (3 * dim + 2 * ffi) + 2.0 * J * (dim + ffi) * dim
    log(f"dit single block (f16, fused SwiGLU + gated residual): {ms:.3f} ms "
        f"{flop / ms / 1e9:.1f} TFLOP/s")
    return {"ms": round(ms, 4), "TFLOP/s": round(flop / ms / 1e9, 1),
            "frac_mfma": round(flop / ms / 1e9 / PEAK_BF16_TFLOPS, 4), "gflop": round(flop / 1e9, 2)}


def bench_dit_step(torch) -> dict:
    """A whole step (5 double + 20 single blocks) as one graph launch."""
    from aestrix_amd.step import DitDims, DitStep, random_projections
    d = DitDims()
    projs = random_projections(d, torch.float16, seed=4)
    step = DitStep(d, projs)
    h = torch.randn((d.l_img, d.dim), device="cuda")
    e = torch.randn((d.l_txt, d.dim), device="cuda")
    out = torch.empty((d.joint, d.dim), device="cuda")
    with no_gc(collect=True):
        t_pre = time.perf_counter()
        while time.perf_counter() - t_pre < PREWARM_S:
            step.run(h, e, out)
            torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            step.run(h, e, out)
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    finite = bool(torch.isfinite(out).all().item())
    flop = d.step_flops()
    wbytes = sum(q.w.numel() * 4 + 2 * q.s.numel() * 2 for q in projs)
    log(f"dit step (graph, {step.launches} launches): {ms:.2f} ms {flop / ms / 1e9:.1f} TFLOP/s")
    res = {"ms": round(ms, 3), "TFLOP/s": round(flop / ms / 1e9, 1),
           "frac_mfma": round(flop / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
           "tflop_per_step": round(flop / 1e12, 3), "launches": step.launches,
           "output_finite": finite,
           "packed_weight_bytes": wbytes,
           "config": "5 double + 20 single blocks, l_img 4096 + l_txt 512, dim 3072, "
                     "ff_inner 9216, f16, RMSNorm before each block's projections"}
    step.close()
    del projs
    torch.cuda.empty_cache()
    return res


def bench_upload(torch) -> dict:
    """Loader path: host -> device through the library's pinned double buffer
    (imq_upload, what the safetensors loader uses for mapped shards) from a
    pageable 1 GiB host buffer, beside a plain pageable torch copy."""
    import ctypes

    import numpy as np

    from aestrix_amd import _lib, ops

    n = 1 << 30
    host = np.ones(n, dtype=np.uint8)
    dev = torch.empty(n, dtype=torch.uint8, device="cuda")
    L = _lib.load()
    ctx = ops.context()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def staged():
        _lib.check(L.imq_upload(ctx, ctypes.c_void_p(dev.data_ptr()),
                                host.ctypes.data_as(ctypes.c_void_p), n, st), ctx)

    staged()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        staged()
    torch.cuda.synchronize()
    staged_s = (time.perf_counter() - t0) / 3
    src = torch.from_numpy(host)
    dev.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        dev.copy_(src)
    torch.cuda.synchronize()
    plain_s = (time.perf_counter() - t0) / 3
    log(f"upload 1 GiB: staged {n / staged_s / 1e9:.1f} GB/s, plain pageable copy "
        f"{n / plain_s / 1e9:.1f} GB/s")
    return {"bytes": n, "staged_GB/s": round(n / staged_s / 1e9, 2),
            "pageable_copy_GB/s": round(n / plain_s / 1e9, 2)}


def traffic_from_profiles():
    path = os.path.join(ROOT, "profiles", "qgemm_target_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-target", action="store_true",
                    help="time the headline qGEMM only (for profiling runs)")
    ap.add_argument("--only-hbm", action="store_true",
                    help="run the HBM-bound and few-row kernels only (M=1 qGEMV, few-row M=4/8/16, "
                         "dequantize, pre-scale, RMSNorm, the K=128 x_embedder) and a calibration "
                         "copy (for counter runs)")
    ap.add_argument("--floors", action="store_true",
                    help="run the launch and streaming-read floor kernels only (for profiling runs)")
    ap.add_argument("--only-step", action="store_true",
                    help="run the whole DiT step benchmark only (for profiling runs)")
    ap.add_argument("--only-te", action="store_true",
                    help="run the text-encoder layer benchmark only (for profiling runs)")
    ap.add_argument("--only-midm", action="store_true",
                    help="run the mid-M shapes only (M = 32, 128, 512 through the dispatcher, the "
                         "text-encoder layer at L = 512) and a calibration copy (for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} requested, but this path runs on one GPU "
              "(no sharding, no collectives); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import aestrix_amd as imq
    from aestrix_amd import synth

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.floors:
        return floors(torch)
    imq._lib.load()
    props = torch.cuda.get_device_properties(0)
    if args.only_step:
        bench_dit_step(torch)
        return 0
    if args.only_te:
        bench_te_layer(torch)
        return 0
    if args.only_midm:
        for (m, n, k) in MID_M_SHAPES:
            bench_qgemm_shape(imq, synth, torch, m, n, k, dispatcher=True)
        bench_te_layer(torch, rows_list=(512,))
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 268435456 bytes read and written")
        return 0
    if args.only_hbm:
        bench_qgemv(imq, synth, torch, ms_list=(1,), few_rows=(4, 8, 16))
        bench_dequant(imq, synth, torch)
        bench_prescale(imq, torch)
        bench_rmsnorm(imq, torch)
        bench_x_embedder(imq, synth, torch)
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 268435456 bytes read and written")
        return 0

    m, n, k = TARGET
    log(f"target qgemm M={m} N={n} K={k}")
    p = synth.make_problem(m, n, k, seed=0)
    x, w, s, b = synth.to_device(p)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    gpu = GpuState(torch)
    idle = gpu.snapshot()
    with StateSampler(gpu) as smp:
        # Untimed pre-warm until PREWARM_S of wall time has passed (the GPU
        # leaves its idle clock and settles at its loaded clock and power),
        # then the W warmup steps.  The collector is off from before the
        # pre-warm (a collection after it would idle the GPU for tens of ms
        # and let the clock rise again before the timed steps).
        with no_gc(collect=True):
            t_pre = time.perf_counter()
            while time.perf_counter() - t_pre < PREWARM_S:
                for _ in range(20):
                    imq.quantized_matmul(x, w, s, b, out=y)
                torch.cuda.synchronize()
            steady_from = smp.elapsed() - STEADY_S
            for _ in range(args.warmup):
                imq.quantized_matmul(x, w, s, b, out=y)
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            start.record()
            for _ in range(args.steps):
                imq.quantized_matmul(x, w, s, b, out=y)
            end.record()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
    loaded = smp.summary(since=steady_from)
    after = gpu.snapshot()
    ms = start.elapsed_time(end) / args.steps
    flop = 2.0 * m * n * k
    tflops = flop / (ms * 1e-3) / 1e12
    log(f"target qgemm: {ms:.4f} ms/step  {tflops:.1f} TFLOP/s  (host wall {wall:.3f} s); "
        f"loaded: {loaded}")
    dense = None
    if not args.only_target:
        dense = bench_dense_bf16(torch, imq, x, w, s, b, gpu)
    del x, w, s, b, y
    torch.cuda.empty_cache()
    if args.only_target:
        # Counter calibration for profiling runs: one device copy of a known
        # size (256 MiB read + 256 MiB written) in the same process.
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 268435456 bytes read and written")
        del src, dst

    extra = {}
    if not args.only_target:
        extra["qgemv"] = bench_qgemv(imq, synth, torch)
        extra["fused_decode"] = bench_fused_decode(imq, synth, torch)
        extra["qgemv_f32"] = bench_qgemv_f32(imq, synth, torch)
        extra["cond_chain"] = bench_cond_chain(torch)
        extra["te_layer"] = bench_te_layer(torch)
        extra["dequant"] = bench_dequant(imq, synth, torch)
        extra["prescale"] = bench_prescale(imq, torch)
        extra["rmsnorm"] = bench_rmsnorm(imq, torch)
        extra["x_embedder"] = bench_x_embedder(imq, synth, torch)
        extra["qgemm_shapes"] = {
            "M1024_N9216_K3072": bench_qgemm_shape(imq, synth, torch, 1024, 9216, 3072,
                                                   dispatcher=True),
            "M4608_N27648_K3072": bench_qgemm_shape(imq, synth, torch, 4608, 27648, 3072),
            "M4608_N3072_K9216": bench_qgemm_shape(imq, synth, torch, 4608, 3072, 9216),
        }
        # Text-encoder prefill and splice rows through the dispatcher (K split
        # when the output tiles are too few to fill the GPU).
        extra["qmm_small_m"] = {
            f"M{m}_N{n}_K{k}": bench_qgemm_shape(imq, synth, torch, m, n, k, dispatcher=True)
            for (m, n, k) in MID_M_SHAPES
        }
        extra["dit_single_block"] = bench_dit_single_block(imq, torch)
        extra["dit_step"] = bench_dit_step(torch)
        extra["upload"] = bench_upload(torch)

    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded PCG64: x~N(0,1) bf16, uniform 4-bit codes, "
                "s=|N(0,0.02)|, b=-8s+N(0,0.002), group 64)",
        "config": {"workload": "qgemm: y[4608x18432] = x[4608x3072] . deq(W[18432x3072])^T, "
                               "affine 4-bit group 64, bf16 in/out, fp32 accumulate",
                   "m": m, "n": n, "k": k, "group_size": 64, "bits": 4},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profiles(),
                     "traffic_source": "profiles/qgemm_target_traffic.md: rocprofv3 --pmc "
                                       "FETCH_SIZE / WRITE_SIZE of this kernel and shape, scaled "
                                       "by a 256 MiB copy in the same process (not this run)"},
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "hip": torch.version.hip, "idle": idle, "headline_loaded": loaded,
                   "after_headline": after},
    }
    if sclk := loaded.get("sclk_mhz"):
        # The peak is quoted at MAX_SCLK_MHZ; under the board's power cap the
        # engine clock of a sustained dense MFMA load settles lower.
        peak_at_clock = PEAK_BF16_TFLOPS * sclk / MAX_SCLK_MHZ
        result["roofline"]["loaded_sclk_mhz"] = sclk
        result["roofline"]["peak_at_loaded_clock"] = round(peak_at_clock, 1)
        result["roofline"]["frac_at_loaded_clock"] = round(tflops / peak_at_clock, 4)
    if dense:
        result["dense_bf16_reference"] = dense
    result.update(extra)
    if qgemv := extra.get("qgemv"):
        result["qgemv_headline"] = {"shape": "M=1 [9728x2560]",
                                    **qgemv["M1_N9728_K2560"]}
        if floor := qgemv.get("copy_floor_N9728_K2560"):
            # A device copy moving the same bytes in one launch, same run.
            result["qgemv_headline"]["copy_floor_GB/s"] = floor["GB/s"]
            result["qgemv_headline"]["frac_of_copy_floor"] = floor["qgemv_M1_vs_copy"]
            result["qgemv_headline"]["copy_floor_single_us"] = floor["single_us"]
            result["qgemv_headline"]["single_frac_of_copy_floor"] = floor["qgemv_M1_vs_copy_single"]
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(synth)
        log(f"cpu baseline: {result['cpu_baseline']['value']} TFLOP/s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
