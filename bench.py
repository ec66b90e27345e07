#!/usr/bin/env python3
"""Benchmark of the BDH strict-tril attention hot path on one MI355X.

Headline (``value``): the cold tril-attention + RoPE prefill forward at the
BASELINE shape B=8, nh=4, T=512, N=8192, D=256 in bf16, RoPE fused into the
HIP kernels (``kernels.bdh_attn_rope(impl="hip")``), inputs resident in HBM.
One step = one call over the whole batch.  Throughput is the algorithmic
F = B*nh*(N+D)*T*(T-1) flops per step (strict lower triangle; RoPE's
elementwise work is not counted) divided by the measured step time.  The step
first runs untimed, back to back, until two consecutive windows of about 0.1 s
agree within 1 % (at least 1 s, at most 4 s: the shader clock keeps rising for
about a second of sustained work), then W warmup steps, then exactly K timed
steps (defaults K = 200, W = 100), synchronised on both sides.

The JSON line also carries:
  * ``roofline``: the dominant kernel (``k_sy_scores``, the score tiles QR QR^T)
    timed over K more steps run right after the timed ones: each launch
    carries HIP start/stop events that the runtime stamps at the kernel's own
    start and end (hipExtLaunchKernelGGL on the launch stream, no extra
    stream work); achieved = its algorithmic flops B*nh*N*T*(T-1) / mean
    duration, against the 2.5 PFLOP/s bf16 dense MFMA peak.  The events leave
    kernel durations as they are but make each launch wait for the previous
    one to end, so they stay out of the K timed steps; ``ms_per_step_observed``
    is the step time with them.  ``kernels_us_isolated`` and
    ``frac_isolated`` repeat the measurement with a synchronisation after
    every step (no kernel overlapping the previous one's tail, as under a
    profiler's kernel trace).  ``traffic`` is the HBM
    bytes per launch from the committed rocprofv3 counter runs (read requests
    by size, 128 x TCC_EA0_RDREQ_128B + 64 x ..._64B + 32 x ..._32B, plus
    WRITE_SIZE; profiles/<kernel>_c1_bf16_pmc.txt) when present, else null;
    ``traffic_source`` names that file, the SHA-1 of the kernel source it
    was measured on and whether the source built here is the same.
  * ``device``: CU count, architecture, the shader clock amd-smi reports while
    the step runs back to back, and how the settle phase ended.
  * ``cpu_baseline``: the CPU oracle (numpy restatement of the reference CPU
    path, fp32, BLAS threads as reported) on bounded samples: C1 (the
    headline's unit), the C2 model, C3 decode attention (integrated over a
    generate), the C4 training op and the C5 attention op; ``gpu_beside_cpu``
    puts each GPU figure of the line next to its CPU sample.
  * ``extra``: other hot-path legs (C1 in fp32 against the fp32 MFMA peak,
    the C5 attention op, decode step GB/s at C3, training op fwd+bwd TFLOP/s
    at C4, the unfused path and torch eager on the GPU).
  * ``models``: the model harness (``bdh_harness.BDH``, random N(0, 0.02^2)
    weights, uniform byte tokens) at C2 and C5 (prefill tok/s, bf16 autocast),
    a C2 training step (AMP forward, backward, AdamW), and C3 (``generate``
    tok/s with a bf16 packed cache), HIP attention beside the same model with
    eager attention.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--no-models]
       python bench.py --model c2|c5|c3     (one model leg, HIP path only)
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "bdh-gpu-fast_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "tril-attn TFLOP/s & %MFMA peak; BDH prefill tok/s; decode tok/s + HBM GB/s"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3
C1 = dict(B=8, nh=4, T=512, N=8192, D=256)
C3 = dict(B=64, nh=4, N=8192, D=256, S=(256, 384, 511))
C4 = dict(B=16, nh=4, T=1024, N=8192, D=256)
C2 = dict(n_layer=6, D=256, nh=4, mult=128, B=32, T=512)
C5 = dict(n_layer=8, D=512, nh=8, mult=128, B=4, T=2048)
C3_GEN = dict(n_layer=6, D=256, nh=4, mult=128, B=64, prompt=256, new=256, top_k=3, seed=5)
CALIB_BYTES = 1 << 29  # reference elementwise pass that scales the HBM byte counters
MARK_ELEMS = 1 << 16  # the section marker multiply of --pmc-targets (a grid no other target has)
# the library kernels of the layer's gated product (alone, or chained into the decoder)
GATED_KERNELS = ("k_gated_gemm", "k_gated_enc", "k_relu_mul", "k_gated_dec", "k_head_sum")
# the library kernels of the layer's encoder with its ReLU
ENCODER_KERNELS = ("k_relu_enc", "k_relu_gemm")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def attn_flops(B, nh, T, N, D) -> float:
    return float(B * nh * (N + D) * T * (T - 1))


def settle(fn, window_s: float = 0.1, tol: float = 0.01, max_s: float = 4.0, min_s: float = 1.0) -> dict:
    """Run the step untimed until its rate has settled: back-to-back windows
    of about ``window_s`` seconds each (HIP events), until two in a row agree
    within ``tol``, after at least ``min_s`` seconds and at most ``max_s``.
    Two effects make a cold start slow.  The first ~100 steps of a process
    run up to 10 % slower (queues and caches settling).  The shader clock then
    keeps rising for about a second of back-to-back work: on MI355X amd-smi
    read 2.06 GHz early in a run and 2.25 GHz after 1.5 s, and the C1 score
    kernel went from 99.6 to 88.0 us.  Windows of a few milliseconds agree
    with each other long before the clock has risen, so the windows here are
    sized in time.  Returns the window times (ms per step) and whether they
    converged."""
    import torch

    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(8):  # warm calls size the window
        fn()
    torch.cuda.synchronize()
    per_step = max((time.perf_counter() - t1) / 8, 1e-6)
    window = max(3, int(window_s / per_step))
    t_end = t0 + max_s
    t_min = t0 + min_s
    hist: list = []
    converged = False
    while time.perf_counter() < t_end:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(window):
            fn()
        e1.record()
        torch.cuda.synchronize()
        hist.append(e0.elapsed_time(e1) / window)
        if len(hist) >= 2 and time.perf_counter() >= t_min and abs(hist[-1] - hist[-2]) <= tol * hist[-2]:
            converged = True
            break
    return {"windows": len(hist), "steps_per_window": window, "seconds": round(time.perf_counter() - t0, 2),
            "last_ms": hist[-2:], "converged": converged}


def sample_sclk(fn, seconds: float = 1.5, n_samples: int = 6) -> dict:
    """Shader clock while ``fn`` runs back to back: amd-smi's per-XCD gfx
    clocks (MHz, averaged over the XCDs), sampled ``n_samples`` times from a
    thread during a busy window.  One amd-smi reading is an instantaneous
    value and can land in a momentary idle dip, so the line reports the
    median and every sample.  Best effort: None fields when amd-smi is not
    available."""
    import subprocess
    import threading

    import torch

    samples: list = []

    def poll():
        for _ in range(n_samples):
            try:
                r = subprocess.run(["amd-smi", "metric", "-g", "0", "--clock", "--json"], capture_output=True,
                                   text=True, timeout=10)
                data = json.loads(r.stdout)
                clk = data["gpu_data"][0]["clock"] if isinstance(data, dict) else data[0]["clock"]
                vals = [v["clk"]["value"] for k, v in clk.items() if k.startswith("gfx_") and isinstance(v, dict)]
                vals = [float(x) for x in vals if isinstance(x, (int, float))]
                if vals:
                    samples.append(sum(vals) / len(vals))
            except Exception:  # pragma: no cover - informational only
                return

    th = threading.Thread(target=poll, daemon=True)
    t_end = time.perf_counter() + seconds
    th.start()
    while time.perf_counter() < t_end or th.is_alive():
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
        if time.perf_counter() > t_end + 30:
            break
    th.join(timeout=1)
    props = torch.cuda.get_device_properties(0)
    return {
        "sclk_mhz_busy": round(statistics.median(samples), 1) if samples else None,
        "sclk_samples_mhz": [round(x, 1) for x in samples],
        "cus": int(props.multi_processor_count),
        "arch": str(getattr(props, "gcnArchName", "")),
        "device": str(props.name),
    }


def time_steps(fn, steps: int, warmup: int, settle_s: float = 0.5) -> float:
    """ms per step over exactly ``steps`` calls, synchronised on both sides,
    after a settle (at least ``settle_s`` seconds of back-to-back steps, until
    two windows of about 0.1 s agree within 1 %) and ``warmup`` untimed calls."""
    import torch

    if settle_s > 0:
        settle(fn, max_s=max(2 * settle_s, 2.0), min_s=settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def kernel_means(fn, steps: int, isolated: bool = False) -> dict:
    """Mean per-kernel duration (ms) from the library's HIP events: each launch
    carries start/stop events the runtime stamps when the kernel itself starts
    and ends (hipExtLaunchKernelGGL).  ``isolated``: a synchronisation after
    every step, so no kernel overlaps the previous one's tail."""
    import torch
    import bdh_hip_ext as ext

    torch.cuda.synchronize()
    ext.profile_enable(True)
    try:
        for _ in range(steps):
            fn()
            if isolated:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        recs = ext.profile_collect()
    finally:
        ext.profile_enable(False)
    return _agg(recs, steps)


def _agg(recs, steps: int) -> dict:
    agg: dict = {}
    for name, ms in recs:
        agg.setdefault(name, []).append(ms)
    return {k: (sum(v) / len(v), len(v) // steps) for k, v in agg.items()}


KERNEL_SOURCE = ROOT / "bdh-gpu-fast_amd" / "csrc" / "syrk.hip"


def source_sha1(path: Path = KERNEL_SOURCE) -> str:
    import hashlib

    return hashlib.sha1(path.read_bytes()).hexdigest()


def pmc_traffic(kernel: str, workload_tag: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 summary
    and where they come from: (bytes or None, source dict).  rocprofv3's
    counter runs profile a process of their own, so the figure is the
    committed one; the summary records the SHA-1 of the kernel source it was
    measured on, and the source dict says whether that is the source built
    here (``matches_current_source``)."""
    path = ROOT / "profiles" / f"{kernel}_{workload_tag}_pmc.txt"
    if not path.exists():
        return None, None
    text = path.read_text()
    m = re.search(r"hbm_bytes_per_launch\s*[:=]\s*([0-9.eE+]+)", text)
    h = re.search(r"kernel_source_sha1\s*[:=]\s*([0-9a-f]{40})", text)
    src = {
        "file": str(path.relative_to(ROOT)),
        "kernel_source_sha1": h.group(1) if h else None,
        "matches_current_source": bool(h) and h.group(1) == source_sha1(),
    }
    return (float(m.group(1)) if m else None), src


def cpu_baseline(reps: int = 3) -> dict:
    """Oracle (numpy, fp32) timing of a bounded sample of C1 on the host cores."""
    import numpy as np

    import oracle as O

    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"), default=1)
    except Exception:  # pragma: no cover - informational only
        threads = os.cpu_count() or 1
    Bs = 1
    nh, T, N, D = C1["nh"], C1["T"], C1["N"], C1["D"]
    rng = np.random.default_rng(0)
    x = np.maximum(rng.standard_normal((Bs, nh, T, N), dtype=np.float32) * np.float32(0.32), 0)
    v = rng.standard_normal((Bs, 1, T, D), dtype=np.float32)
    f = O.get_freqs(N)
    O.tril_rope_score_v(x, v, f, 0)  # warmup
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        O.tril_rope_score_v(x, v, f, 0)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    F = attn_flops(Bs, nh, T, N, D)

    # Model harness counterpart (C2 shape, fp32): the numpy model oracle on one sequence.
    from oracle import bdh_model_oracle as M

    c = C2
    Nl = c["mult"] * c["D"] // c["nh"]
    p = M.init_params(c["n_layer"], c["D"], c["nh"], Nl, 256, seed=0)
    idx = rng.integers(0, 256, (1, c["T"]))
    M.bdh_forward(p, idx)  # warmup
    mt = []
    for _ in range(reps):
        t = time.perf_counter()
        M.bdh_forward(p, idx)
        mt.append(time.perf_counter() - t)
    mmed = statistics.median(mt)

    # C4 (training op): forward + analytic merged backward on one of 16 batch
    # elements, fp32 (the reference's CPU path: tril_attn_cpu.cpp forward,
    # attention_bwd.py blocked backward).
    n4, T4, N4, D4 = C4["nh"], C4["T"], C4["N"], C4["D"]
    x4 = np.maximum(rng.standard_normal((1, n4, T4, N4), dtype=np.float32) * np.float32(0.32), 0)
    v4 = rng.standard_normal((1, 1, T4, D4), dtype=np.float32)
    d4 = rng.standard_normal((1, n4, T4, D4), dtype=np.float32)

    def c4():
        O.tril_score_v_cpu(x4, x4, v4)
        O.self_attn_backward(x4, v4, d4)

    c4()
    t4 = []
    for _ in range(2):
        t = time.perf_counter()
        c4()
        t4.append(time.perf_counter() - t)
    m4 = statistics.median(t4)
    F4 = 3 * attn_flops(1, n4, T4, N4, D4)
    del x4, v4, d4

    # C5 (long prefill): the fused RoPE attention op on one of 4 batch
    # elements at the C5 width (nh=8, T=2048, N=8192, D=512).
    n5, T5, D5 = C5["nh"], C5["T"], C5["D"]
    N5 = C5["mult"] * D5 // n5
    x5 = np.maximum(rng.standard_normal((1, n5, T5, N5), dtype=np.float32) * np.float32(0.32), 0)
    v5 = rng.standard_normal((1, 1, T5, D5), dtype=np.float32)
    f5 = O.get_freqs(N5)
    O.tril_rope_score_v(x5, v5, f5, 0)
    t5 = []
    for _ in range(2):
        t = time.perf_counter()
        O.tril_rope_score_v(x5, v5, f5, 0)
        t5.append(time.perf_counter() - t)
    m5 = statistics.median(t5)
    F5 = attn_flops(1, n5, T5, N5, D5)
    del x5, v5

    # C3 (decode): one layer step of the decode attention at S = 256, 384,
    # 511 on 8 of the 64 sequences (scaled by 8), a straight line through the
    # three fitted by least squares, summed over the 256 generated tokens
    # (S = 256 .. 511) and the 6 layers: the attention seconds of one C3
    # generate on the CPU.
    Bs3, n3, N3, D3 = 8, C3["nh"], C3["N"], C3["D"]
    Smax = max(C3["S"])
    k3 = np.maximum(rng.standard_normal((Bs3, n3, Smax, N3), dtype=np.float32) * np.float32(0.32), 0)
    v3 = rng.standard_normal((Bs3, 1, Smax, D3), dtype=np.float32)
    q3 = np.maximum(rng.standard_normal((Bs3, n3, 1, N3), dtype=np.float32) * np.float32(0.32), 0)
    per_s = {}
    for S in C3["S"]:
        kp, vp = k3[:, :, :S], v3[:, :, :S]
        O.tril_decode_cpu(q3, kp, vp)
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            O.tril_decode_cpu(q3, kp, vp)
            ts.append(time.perf_counter() - t)
        per_s[S] = statistics.median(ts) * (C3["B"] // Bs3)
    Ss = np.array(list(per_s), dtype=np.float64)
    ys = np.array([per_s[S] for S in per_s])
    b1, b0 = np.polyfit(Ss, ys, 1)
    steps = np.arange(C3_GEN["prompt"], C3_GEN["prompt"] + C3_GEN["new"], dtype=np.float64)
    total3 = float(np.sum(b0 + b1 * steps)) * C3_GEN["n_layer"]
    by3 = sum(4 * (C3["B"] * n3 * S * N3 + C3["B"] * S * D3) for S in range(C3_GEN["prompt"], C3_GEN["prompt"] + C3_GEN["new"]))
    by3 *= C3_GEN["n_layer"]
    del k3, v3
    return {
        "value": F / med / 1e12,
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"C1 fp32 with B={Bs} of 8 (nh=4 T=512 N=8192 D=256): numpy RoPE + tiled strict-tril "
        f"score x V (oracle/tril_attn_oracle.py), median of {reps} after 1 warmup, {med * 1e3:.0f} ms per call",
        "ms_per_call": med * 1e3,
        "models": {
            "c2_prefill": {
                "tok_s": c["T"] / mmed,
                "sample": f"C2 model (L=6 D=256 nh=4 N=8192) fp32 forward of B=1 of 32 sequences, T=512 "
                f"(oracle/bdh_model_oracle.py), median of {reps} after 1 warmup, {mmed * 1e3:.0f} ms per sequence",
            }
        },
        "configs": {
            "c3_decode_attention": {
                "value": C3_GEN["B"] * C3_GEN["new"] / total3,
                "unit": "tok/s (decode attention only)",
                "seconds_per_generate": total3,
                "gbs_fp32_cache": by3 / total3 / 1e9,
                "per_layer_step_ms": {str(S): t * 1e3 for S, t in per_s.items()},
                "sample": f"C3 decode attention, fp32 (oracle tril_decode_cpu): one layer step at S = 256/384/511 on 8 "
                f"of 64 sequences, times 8, median of {reps} after 1 warmup; a line through the three, summed over "
                f"S = 256..511 and 6 layers",
            },
            "c4_train_op": {
                "value": F4 / m4 / 1e12,
                "unit": "TFLOP/s",
                "ms_per_call": m4 * 1e3,
                "sample": f"C4 fp32 forward + analytic merged backward (oracle tril_score_v_cpu + self_attn_backward) "
                f"on B=1 of 16 (nh=4 T=1024 N=8192 D=256), median of 2 after 1 warmup, {m4:.2f} s per call",
            },
            "c5_attention_op": {
                "value": F5 / m5 / 1e12,
                "unit": "TFLOP/s",
                "ms_per_call": m5 * 1e3,
                "sample": f"C5 fp32 RoPE + strict-tril attention (oracle tril_rope_score_v) on B=1 of 4 (nh=8 T=2048 "
                f"N=8192 D=512), median of 2 after 1 warmup, {m5:.2f} s per call",
            },
        },
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the decode / backward / comparison legs")
    ap.add_argument("--no-models", action="store_true", help="skip the model-harness legs (C2, C3, C5)")
    ap.add_argument("--model", choices=("c2", "c5", "c3"), default=None,
                    help="run only this model-harness leg on the HIP path (for profiling) and print its JSON")
    ap.add_argument(
        "--pmc-targets",
        action="store_true",
        help="run only the profiled kernels a few times each (for rocprofv3 counter passes): the C1 fused "
        "forward in bf16 and in fp32, the C5 attention op, the C4 training op, one C2 layer's gated GEMM, one C2 layer's RoPE attention backward "
        "on both routes (recomputed tiles; kept tiles, as the training step runs it), the C3 decode step at "
        "S=511, and the calibration multiply",
    )
    ap.add_argument(
        "--calibrate",
        action="store_true",
        help="also run one elementwise multiply over CALIB_BYTES (the reference point that scales "
        "the rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)",
    )
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one GPU only: the strict-tril attention hot path is benchmarked on a single "
            "MI355X (per-GPU work at its real shape); multi-GPU runs are not part of this build.",
            file=sys.stderr,
        )
        return 2

    import torch

    import bdh_hip_ext as ext
    import kernels

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.model is not None:
        print(json.dumps(run_models(torch, ext, dev, only=args.model)), flush=True)
        return 0
    if args.pmc_targets:
        run_pmc_targets(torch, ext, kernels, dev)
        return 0

    B, nh, T, N, D = (C1[k] for k in ("B", "nh", "T", "N", "D"))
    gq = torch.Generator(device=dev).manual_seed(0)
    gv = torch.Generator(device=dev).manual_seed(1)
    x = torch.relu(0.32 * torch.randn(B, nh, T, N, generator=gq, device=dev)).to(torch.bfloat16)
    v = torch.randn(B, 1, T, D, generator=gv, device=dev).to(torch.bfloat16)
    freqs = kernels.get_freqs(N).to(dev)

    def step():
        return kernels.bdh_attn_rope(x, v, freqs, 0, impl="hip")

    if args.calibrate:
        # Reference kernel of known traffic for the HBM byte counters: one
        # full-grid elementwise multiply (torch's vectorized_elementwise_kernel)
        # reading and writing CALIB_BYTES, like the kernels it scales.
        src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        log(f"[bench] calibration multiply: {CALIB_BYTES} bytes read, {CALIB_BYTES} bytes written")
        del src, dst

    settled = settle(step)
    log(f"[bench] settle: {settled}")
    launches0 = ext.launch_count()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms = time_steps(step, args.steps, 0, settle_s=0)
    # The per-kernel events ride on the launches of the next K steps, run
    # right after the timed ones (stamped by the runtime at kernel start and
    # end).  They do not change a kernel's duration, but the runtime starts
    # each evented launch only after the previous one has ended (median gap
    # 7.8 us in a kernel trace, 0 without events), which would slow the
    # timed steps themselves; ms_per_step_observed shows that cost.
    ext.profile_enable(True)
    try:
        ms_obs = time_steps(step, args.steps, 0, settle_s=0)
        live = _agg(ext.profile_collect(), args.steps)
    finally:
        ext.profile_enable(False)
    assert ext.launch_count() - launches0 == 2 * args.steps + args.warmup, "HIP library calls missing"
    F = attn_flops(B, nh, T, N, D)
    value = F / (ms * 1e-3) / 1e12
    log(f"[bench] fused RoPE tril-attn fwd C1 bf16: {ms * 1e3:.1f} us/step, {value:.1f} TFLOP/s")

    means = live
    isolated = kernel_means(step, args.steps, isolated=True)
    kname = max(means, key=lambda k: means[k][0] * means[k][1])  # dominant kernel of the step
    k_ms = means[kname][0]
    # the score tiles R R^T over the strict lower triangle: B*nh*N*T*(T-1) flops
    F_scores = float(B * nh * N * T * (T - 1))
    achieved = F_scores / (k_ms * 1e-3) / 1e12
    traffic, traffic_src = pmc_traffic(kname, "c1_bf16")
    roofline = {
        "bound": "mfma",
        "kernel": kname,
        "achieved": achieved,
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": achieved / PEAK_BF16_TFLOPS,
        "traffic": traffic,
        "traffic_source": traffic_src,
        "kernel_us": k_ms * 1e3,
        "ms_per_step_observed": ms_obs,
        "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in means.items()},
        "kernels_us_isolated": {k: round(v[0] * 1e3, 2) for k, v in isolated.items()},
        "frac_isolated": F_scores / (isolated[kname][0] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "algorithmic_flops_per_launch": F_scores,
    }
    log(f"[bench] kernels: {roofline['kernels_us']} -> {kname} {achieved:.1f} TFLOP/s")
    device = sample_sclk(step)
    device["settle"] = settled
    log(f"[bench] device: {device}")

    extra: dict = {}
    if not args.no_extra:
        extra = run_extra(torch, ext, kernels, dev, max(3, args.steps // 5), max(2, args.warmup // 5), x, v)

    models: dict = {}
    if not args.no_models:
        models = run_models(torch, ext, dev)

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle on host cores)...")
        cpu = cpu_baseline()
        log(f"[bench] cpu baseline: {cpu['value']:.4f} TFLOP/s on {cpu['cores']} threads; "
            f"C2 model {cpu['models']['c2_prefill']['tok_s']:.0f} tok/s")

    if cpu is not None:
        # the GPU figure of each config beside its CPU sample (same unit)
        side = {"c1": {"unit": "TFLOP/s", "gpu_bf16": value, "cpu_fp32": cpu["value"]}}
        cc = cpu["configs"]
        if "c1_fp32_fused_rope" in extra:
            side["c1"]["gpu_fp32"] = extra["c1_fp32_fused_rope"]["tflops"]
        if "c4_train_op_fwd_bwd" in extra:
            side["c4"] = {"unit": "TFLOP/s", "gpu_bf16": extra["c4_train_op_fwd_bwd"]["tflops"],
                          "cpu_fp32": cc["c4_train_op"]["value"]}
        if "c5_attention_op" in extra:
            side["c5"] = {"unit": "TFLOP/s", "gpu_bf16": extra["c5_attention_op"]["tflops"],
                          "cpu_fp32": cc["c5_attention_op"]["value"]}
        c3g = models.get("c3_generate", {}).get("hip", {})
        if c3g.get("decode_attention_ms"):
            side["c3"] = {"unit": "tok/s (decode attention only)",
                          "gpu_bf16_cache": C3_GEN["B"] * C3_GEN["new"] / (c3g["decode_attention_ms"] * 1e-3),
                          "cpu_fp32": cc["c3_decode_attention"]["value"]}
        if "c2_prefill" in models:
            side["c2"] = {"unit": "tok/s", "gpu_bf16": models["c2_prefill"]["hip"]["tok_s"],
                          "cpu_fp32": cpu["models"]["c2_prefill"]["tok_s"]}
        cpu["gpu_beside_cpu"] = side

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C1 tril-attention + RoPE prefill forward (fused RoPE), bf16 in / fp32 accumulate",
            "B": B,
            "nh": nh,
            "T": T,
            "N": N,
            "D": D,
            "rope_theta": 65536,
            "frac_of_bf16_peak": value / PEAK_BF16_TFLOPS,
        },
        "roofline": roofline,
        "device": device,
        "cpu_baseline": cpu,
        "extra": extra,
        "models": models,
    }
    print(json.dumps(line), flush=True)
    return 0


def run_extra(torch, ext, kernels, dev, steps, warmup, x, v) -> dict:
    out: dict = {}
    B, nh, T, N, D = (C1[k] for k in ("B", "nh", "T", "N", "D"))
    F = attn_flops(B, nh, T, N, D)
    freqs = kernels.get_freqs(N).to(dev)
    qr = torch.empty_like(x)
    kernels.bdh_attn_rope(x, v, freqs, 0, out_kr=qr, impl="hip")
    ms = time_steps(lambda: kernels.bdh_attn(qr, qr, v, impl="hip"), steps, warmup)
    out["c1_unfused_tril_score_v_on_qr"] = {"us": ms * 1e3, "tflops": F / ms / 1e9}
    cos, sin = kernels.rope_cos_sin(T, 0, freqs)
    ms_r = time_steps(lambda: kernels.bdh_rope_rotate(x, cos, sin, out=qr, impl="hip"), steps, warmup)
    out["c1_rope_apply_hip"] = {"us": ms_r * 1e3, "gbs": 2 * x.numel() * 2 / ms_r / 1e6}

    # The unchanged caller's cold prefill (bdh.py:405-412): RoPE into a fresh
    # QR, then bdh_attn(QR, QR, V), both on the HIP kernels.
    def bdh_py_route():
        q = kernels.bdh_rope_rotate(x, cos, sin, impl="hip")
        return kernels.bdh_attn(q, q, v, impl="hip")

    ms_b = time_steps(bdh_py_route, steps, warmup)
    out["c1_bdh_py_route"] = {"us": ms_b * 1e3, "tflops": F / ms_b / 1e9,
                              "frac_bf16_peak": F / ms_b / 1e9 / PEAK_BF16_TFLOPS}
    log(f"[bench] bdh.py route (RoPE pass + bdh_attn): {ms_b * 1e3:.1f} us, {F / ms_b / 1e9:.1f} TFLOP/s")

    def eager():
        s = qr @ qr.mT.contiguous()
        s.tril_(-1)
        return s @ v

    ms_e = time_steps(eager, steps, warmup)
    out["c1_torch_eager_gpu_on_qr"] = {"us": ms_e * 1e3, "tflops": F / ms_e / 1e9}
    log(f"[bench] unfused {ms * 1e3:.1f} us, rope {ms_r * 1e3:.1f} us, torch eager {ms_e * 1e3:.1f} us")

    # C1 as BASELINE.json states it: fp32 in and out (the fp32 HIP path),
    # against the fp32 MFMA peak.
    x32, v32 = x.float(), v.float()
    ms_32 = time_steps(lambda: kernels.bdh_attn_rope(x32, v32, freqs, 0, impl="hip"), max(3, steps // 2), 2)
    out["c1_fp32_fused_rope"] = {"us": ms_32 * 1e3, "tflops": F / ms_32 / 1e9,
                                 "frac_fp32_peak": F / ms_32 / 1e9 / PEAK_FP32_TFLOPS}
    log(f"[bench] C1 fp32: {ms_32 * 1e3:.1f} us, {F / ms_32 / 1e9:.1f} TFLOP/s")
    del x32, v32

    # C5 attention op alone at its full width (B=4 nh=8 T=2048 N=8192 D=512,
    # bf16, fused RoPE): the attention of one C5 layer.
    B5, n5, T5, D5 = C5["B"], C5["nh"], C5["T"], C5["D"]
    N5 = C5["mult"] * D5 // n5
    g5 = torch.Generator(device=dev).manual_seed(0)
    x5 = torch.relu(0.32 * torch.randn(B5, n5, T5, N5, generator=g5, device=dev)).to(torch.bfloat16)
    v5 = torch.randn(B5, 1, T5, D5, generator=g5, device=dev).to(torch.bfloat16)
    f5 = kernels.get_freqs(N5).to(dev)
    F5 = attn_flops(B5, n5, T5, N5, D5)
    ms_5 = time_steps(lambda: kernels.bdh_attn_rope(x5, v5, f5, 0, impl="hip"), max(3, steps // 4), 2)
    out["c5_attention_op"] = {"us": ms_5 * 1e3, "tflops": F5 / ms_5 / 1e9,
                              "frac_bf16_peak": F5 / ms_5 / 1e9 / PEAK_BF16_TFLOPS}
    log(f"[bench] C5 attention op: {ms_5 * 1e3:.1f} us, {F5 / ms_5 / 1e9:.1f} TFLOP/s")
    del x5, v5

    out.update(run_decode(torch, kernels, dev, steps, warmup))

    # Training op (C4): fwd + merged-gradient bwd, bf16.
    B4, nh4, T4, N4, D4 = (C4[k] for k in ("B", "nh", "T", "N", "D"))
    g4 = torch.Generator(device=dev).manual_seed(0)
    q4 = torch.relu(0.32 * torch.randn(B4, nh4, T4, N4, generator=g4, device=dev)).to(torch.bfloat16)
    v4 = torch.randn(B4, 1, T4, D4, generator=g4, device=dev).to(torch.bfloat16)
    d4 = torch.randn(B4, nh4, T4, D4, generator=g4, device=dev).to(torch.bfloat16)

    # The forward keeps its bf16 score tiles (84 MB) for the backward, as the
    # hip autograd function does (the reference's default autograd keeps S);
    # the recompute variant is reported beside it.
    def train_op():
        _, sc = ext.tril_score_v_save(q4, v4)
        ext.tril_score_v_bwd_saved(q4, v4, d4, sc)

    def train_op_recompute():
        ext.tril_score_v(q4, q4, v4)
        ext.tril_score_v_bwd(q4, None, v4, d4)

    F4 = 3 * attn_flops(B4, nh4, T4, N4, D4)
    for key, fn in (("c4_train_op_fwd_bwd", train_op), ("c4_train_op_fwd_bwd_recompute", train_op_recompute)):
        ms_t = time_steps(fn, max(2, steps // 2), 1)
        out[key] = {"us": ms_t * 1e3, "tflops": F4 / ms_t / 1e9, "frac_bf16_peak": F4 / ms_t / 1e9 / PEAK_BF16_TFLOPS}
        log(f"[bench] {key}: {ms_t * 1e3:.1f} us, {F4 / ms_t / 1e9:.1f} TFLOP/s")
    return out


def run_decode(torch, kernels, dev, steps, warmup) -> dict:
    """C3 decode-step legs: the bf16 cache read in place at each C3 past, and the
    routes of the reference generate's caches at the longest past."""
    out: dict = {}
    # Decode step (C3): B=64 nh=4 N=8192 D=256, bf16 cache read in place.
    Bd, nhd, Nd, Dd = (C3[k] for k in ("B", "nh", "N", "D"))
    cap = max(C3["S"]) + 1
    g = torch.Generator(device=dev).manual_seed(5)
    kcache = torch.relu(0.32 * torch.randn(Bd, nhd, cap, Nd, generator=g, device=dev)).to(torch.bfloat16)
    vcache = torch.randn(Bd, 1, cap, Dd, generator=g, device=dev).to(torch.bfloat16)
    q = torch.relu(0.32 * torch.randn(Bd, nhd, 1, Nd, generator=g, device=dev)).to(torch.bfloat16)
    dec = {}
    for S in C3["S"]:
        kp, vp = kcache.narrow(2, 0, S), vcache.narrow(2, 0, S)
        ms_d = time_steps(lambda: kernels.bdh_attn_decode(q, kp, vp, impl="hip"), steps * 4, warmup)
        by = 2 * (Bd * nhd * S * Nd + Bd * S * Dd + Bd * nhd * Nd + Bd * nhd * Dd)
        dec[str(S)] = {"us": ms_d * 1e3, "gbs": by / ms_d / 1e6, "frac_hbm": by / ms_d / 1e6 / PEAK_HBM_GBS}
    out["c3_decode_step_per_layer"] = dec
    log(f"[bench] decode: {json.dumps(dec)}")

    # The caches the reference's generate builds (compute fp32, bdh.py:1115-1123),
    # at the longest C3 past:
    #  * fp32_cache: cache_dtype=None, fp32 q and past (k_decode_f32q);
    #  * bf16_cache_reference_cast: bf16 storage, the past cast up to fp32 by
    #    the reference CacheManager.get_past (bdh_cache.py:238-243) on every
    #    layer step, timed with the decode it feeds (bf16 q, fp32 past);
    #  * bf16_cache_storage_views: the package's CacheManager hands the bf16
    #    views to the HIP decode (no cast).
    S = max(C3["S"])
    kp, vp = kcache.narrow(2, 0, S), vcache.narrow(2, 0, S)
    k32, v32 = kcache.float(), vcache.float()
    q32 = q.float()
    elems = Bd * nhd * S * Nd + Bd * S * Dd + Bd * nhd * Nd + Bd * nhd * Dd
    routes = {
        "fp32_cache": (lambda: kernels.bdh_attn_decode(q32, k32.narrow(2, 0, S), v32.narrow(2, 0, S), impl="hip"), 4),
        "bf16_cache_reference_cast": (lambda: kernels.bdh_attn_decode(q, kp.to(torch.float32), vp.to(torch.float32),
                                                                      impl="hip"), 2),
        "bf16_cache_storage_views": (lambda: kernels.bdh_attn_decode(q, kp, vp, impl="hip"), 2),
    }
    rt = {}
    for name, (fn, width) in routes.items():
        ms_d = time_steps(fn, steps * 2, warmup)
        rt[name] = {"S": S, "us": ms_d * 1e3, "cache_bytes_per_elem": width,
                    "gbs_cache_bytes": width * elems / ms_d / 1e6}
    rt["views_speedup_over_cast"] = rt["bf16_cache_reference_cast"]["us"] / rt["bf16_cache_storage_views"]["us"]
    out["c3_decode_reference_cache_routes"] = rt
    log(f"[bench] decode routes: {json.dumps(rt)}")
    del kcache, vcache, k32, v32

    return out


def run_models(torch, ext, dev, only=None) -> dict:
    """Model harness legs: prefill tok/s (C2, C5) and generate tok/s (C3).
    ``only`` ("c2", "c5" or "c3") runs that leg alone, HIP path only."""
    import bdh_harness as H

    out: dict = {}

    def build(c):
        torch.manual_seed(0)
        cfg = H.BDHConfig(n_layer=c["n_layer"], n_embd=c["D"], n_head=c["nh"], mlp_internal_dim_multiplier=c["mult"])
        return H.BDH(cfg).to(dev)

    impls = ("hip",) if only else ("hip", "eager")
    for name, c in (("c2_prefill", C2), ("c5_long_prefill", C5)):
        if only is not None and not name.startswith(only):
            continue
        m = build(c)
        g = torch.Generator(device=dev).manual_seed(1)
        idx = torch.randint(0, 256, (c["B"], c["T"]), generator=g, device=dev)
        leg = {"B": c["B"], "T": c["T"], "n_layer": c["n_layer"], "D": c["D"], "nh": c["nh"]}
        for impl in impls:
            log(f"[bench] {name} {impl} ...")

            def fwd():
                with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                    return m(idx, impl=impl)[0]
            ms = time_steps(fwd, 3, 1)
            leg[impl] = {"ms": ms, "tok_s": c["B"] * c["T"] / (ms * 1e-3)}
        ext.profile_enable(True)
        fwd_hip = lambda: m(idx, impl="hip")  # noqa: E731
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            fwd_hip()
        rec = ext.profile_collect()
        ext.profile_enable(False)
        mlp = GATED_KERNELS
        leg["hip"]["attention_kernels_ms"] = sum(t for n, t in rec if n not in mlp + ENCODER_KERNELS)
        leg["hip"]["gated_product_kernels_ms"] = sum(t for n, t in rec if n in mlp)
        leg["hip"]["encoder_kernels_ms"] = sum(t for n, t in rec if n in ENCODER_KERNELS)
        out[name] = leg
        log(f"[bench] {name}: hip {leg['hip']['tok_s']:.0f} tok/s ({leg['hip']['ms']:.2f} ms, attention kernels "
            f"{leg['hip']['attention_kernels_ms']:.2f} ms, gated product {leg['hip']['gated_product_kernels_ms']:.2f} ms, "
            f"encoder {leg['hip']['encoder_kernels_ms']:.2f} ms)"
            + (f", eager {leg['eager']['tok_s']:.0f} tok/s" if "eager" in leg else ""))
        del m, idx
        torch.cuda.empty_cache()

    if only is None or only == "c2":
        out["c2_train_step"] = run_train_step(torch, ext, dev, build)
    if only is not None and only != "c3":
        return out
    c = C3_GEN
    m = build(c)
    g = torch.Generator(device=dev).manual_seed(2)
    prompt = torch.randint(0, 256, (c["B"], c["prompt"]), generator=g, device=dev)
    leg = {"B": c["B"], "prompt": c["prompt"], "new_tokens": c["new"], "top_k": c["top_k"], "cache": "bf16"}
    # hip: the harness's own cache; hip_cache_manager: bdh_cache.CacheManager in
    # bdh.py's call order, storage-dtype views to the decode;
    # hip_cache_manager_reference_cast: the same with the reference's get_past
    # casts (bf16 past copied up to fp32 on every layer step)
    variants = [("hip", {}), ("hip_cache_manager", {"cache_manager": True}),
                ("hip_cache_manager_reference_cast", {"cache_manager": True, "decode_views": False})]
    if "eager" in impls:
        variants.append(("eager", {}))
    for key, kw in variants:
        impl = "eager" if key == "eager" else "hip"
        log(f"[bench] c3_generate {key} ...")

        def gen():
            return m.generate(prompt, c["new"], top_k=c["top_k"], cache_dtype=torch.bfloat16,
                              amp_dtype=torch.bfloat16, impl=impl,
                              generator=torch.Generator(device=dev).manual_seed(c["seed"]), **kw)
        gen()  # warm-up (allocator, library)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        gen()
        torch.cuda.synchronize()
        s = time.perf_counter() - t0
        leg[key] = {"s": s, "tok_s": c["B"] * c["new"] / s}
        if key == "hip":
            ext.profile_enable(True)
            gen()
            rec = ext.profile_collect()
            ext.profile_enable(False)
            dec = [t for n, t in rec if n.startswith("k_decode")]
            Nl = c["mult"] * c["D"] // c["nh"]
            by = sum(2 * (c["B"] * c["nh"] * S * Nl + c["B"] * S * c["D"] + c["B"] * c["nh"] * Nl + c["B"] * c["nh"] * c["D"])
                     for S in range(c["prompt"], c["prompt"] + c["new"])) * c["n_layer"]
            leg[impl]["decode_attention_ms"] = sum(dec)
            leg[impl]["decode_attention_gbs"] = by / (sum(dec) * 1e-3) / 1e9 if dec else None
            leg[impl]["library_kernels_ms"] = sum(t for _, t in rec)
    out["c3_generate"] = leg
    log(f"[bench] c3_generate: hip {leg['hip']['tok_s']:.0f} tok/s ({leg['hip']['s']:.3f} s; decode attention "
        f"{leg['hip']['decode_attention_ms']:.1f} ms, {leg['hip']['decode_attention_gbs']:.0f} GB/s); "
        f"CacheManager {leg['hip_cache_manager']['tok_s']:.0f} tok/s, with the reference's casts "
        f"{leg['hip_cache_manager_reference_cast']['tok_s']:.0f} tok/s"
        + (f", eager {leg['eager']['tok_s']:.0f} tok/s" if "eager" in leg else ""))
    del m
    torch.cuda.empty_cache()
    return out


def run_pmc_targets(torch, ext, kernels, dev, reps: int = 3) -> None:
    """The kernels the committed counter tables cover, ``reps`` calls each on
    synthetic inputs of their configuration (rocprofv3 --pmc runs this with
    --kernel-include-regex to pick them), then one calibration multiply over
    CALIB_BYTES (the reference point that scales FETCH_SIZE / WRITE_SIZE).
    Each section ends with a small elementwise multiply (MARK_ELEMS floats), a
    marker in the dispatch order: some kernels run in two sections with the
    same grid (the C1 and C2 score passes, C4's and C2's S x V and dV), and a
    counter table tells them apart by the markers before them."""
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    mark = torch.ones(MARK_ELEMS, dtype=torch.float32, device=dev)

    def section_end():
        torch.cuda.synchronize()
        torch.mul(mark, 1.0, out=mark)
        torch.cuda.synchronize()

    # C1 fused forward (k_sy_scores, k_sy_sv)
    B, nh, T, N, D = (C1[k] for k in ("B", "nh", "T", "N", "D"))
    x = torch.relu(0.32 * torch.randn(B, nh, T, N, generator=g, device=dev)).to(bf)
    v = torch.randn(B, 1, T, D, generator=g, device=dev).to(bf)
    f = kernels.get_freqs(N).to(dev)
    for _ in range(reps):
        kernels.bdh_attn_rope(x, v, f, 0, impl="hip")
    section_end()
    # C1 as BASELINE.json states it, fp32 operands (the generic MFMA kernels
    # k_scores, k_score_v)
    x32, v32 = x.float(), v.float()
    del x, v
    for _ in range(reps):
        kernels.bdh_attn_rope(x32, v32, f, 0, impl="hip")
    del x32, v32
    section_end()
    # C5 attention op (B=4 nh=8 T=2048 N=8192 D=512, fused RoPE, one split)
    N5 = C5["mult"] * C5["D"] // C5["nh"]
    x5 = torch.relu(0.32 * torch.randn(C5["B"], C5["nh"], C5["T"], N5, generator=g, device=dev)).to(bf)
    v5 = torch.randn(C5["B"], 1, C5["T"], C5["D"], generator=g, device=dev).to(bf)
    f5 = kernels.get_freqs(N5).to(dev)
    for _ in range(reps):
        kernels.bdh_attn_rope(x5, v5, f5, 0, impl="hip")
    del x5, v5
    section_end()
    # C4 training op (k_sy_scores, k_sy_sv, k_dv_dma, G, k_dq_sy)
    B4, n4, T4, N4, D4 = (C4[k] for k in ("B", "nh", "T", "N", "D"))
    q4 = torch.relu(0.32 * torch.randn(B4, n4, T4, N4, generator=g, device=dev)).to(bf)
    v4 = torch.randn(B4, 1, T4, D4, generator=g, device=dev).to(bf)
    d4 = torch.randn(B4, n4, T4, D4, generator=g, device=dev).to(bf)
    for _ in range(reps):
        _, sc = ext.tril_score_v_save(q4, v4)
        ext.tril_score_v_bwd_saved(q4, v4, d4, sc)
    del q4, v4, d4, sc
    section_end()
    # one C2 layer's gated product (k_gated_gemm): y (B, nh, T, D), encoder_v^T (nh, N, D), x (B, T, nh, N);
    # then the same product chained into the decoder (k_gated_dec, k_head_sum), dec (nh*N, D),
    # then the encoder with its ReLU (k_relu_enc) on rows shared by the heads
    c = C2
    N2 = c["mult"] * c["D"] // c["nh"]
    y = torch.randn(c["B"], c["nh"], c["T"], c["D"], generator=g, device=dev).to(bf)
    wt = (0.02 * torch.randn(c["nh"], N2, c["D"], generator=g, device=dev)).to(bf)
    xb = torch.relu(torch.randn(c["B"], c["T"], c["nh"], N2, generator=g, device=dev)).to(bf)
    dec = (0.02 * torch.randn(c["nh"] * N2, c["D"], generator=g, device=dev)).to(bf)
    for _ in range(reps):
        kernels.gated_gemm(y, wt, xb)
    for _ in range(reps):
        kernels.gated_decoder(y, wt, xb, dec)
    ye = y[:, :1].expand(-1, c["nh"], -1, -1)  # the encoder: one row set shared by the heads
    for _ in range(reps):
        kernels.relu_gemm(ye, wt)
    del y, wt, xb, dec, ye
    section_end()
    # one C2 layer's fused RoPE attention backward, bf16, x_sparse as the
    # model's permuted (B, T, nh, N) view: the route that recomputes the score
    # tiles, then the training step's route (the forward keeps its tiles, the
    # backward recomputes none)
    x2 = torch.relu(0.32 * torch.randn(c["B"], c["T"], c["nh"], N2, generator=g, device=dev)).to(bf).permute(0, 2, 1, 3)
    v2 = torch.randn(c["B"], 1, c["T"], c["D"], generator=g, device=dev).to(bf)
    d2 = torch.randn(c["B"], c["nh"], c["T"], c["D"], generator=g, device=dev).to(bf)
    f2 = kernels.get_freqs(N2).to(dev)
    for _ in range(reps):
        ext.tril_rope_score_v_bwd(x2, v2, d2, f2, 0)
    section_end()
    for _ in range(reps):
        _, sc2 = ext.tril_rope_score_v_save(x2, v2, f2, 0)
        ext.tril_rope_score_v_bwd_saved(x2, v2, d2, f2, 0, sc2)
    del x2, v2, d2, sc2
    section_end()
    # C3 decode step at the longest past (k_decode_bf16)
    Bd, nhd, Nd, Dd = (C3[k] for k in ("B", "nh", "N", "D"))
    S = max(C3["S"])
    kc = torch.relu(0.32 * torch.randn(Bd, nhd, S + 1, Nd, generator=g, device=dev)).to(bf)
    vc = torch.randn(Bd, 1, S + 1, Dd, generator=g, device=dev).to(bf)
    qd = torch.relu(0.32 * torch.randn(Bd, nhd, 1, Nd, generator=g, device=dev)).to(bf)
    for _ in range(reps):
        kernels.bdh_attn_decode(qd, kc.narrow(2, 0, S), vc.narrow(2, 0, S), impl="hip")
    del kc, vc, qd
    torch.cuda.synchronize()
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.mul(src, 2.0, out=dst)
    torch.cuda.synchronize()
    log(f"[bench] pmc targets done ({reps} calls each; calibration multiply over {CALIB_BYTES} bytes)")


def run_train_step(torch, ext, dev, build) -> dict:
    """Model-level training step at the C2 configuration (L=6 D=256 nh=4
    N=8192, B=32 T=512) under bf16 autocast: forward with cross entropy,
    backward through the HIP attention autograd functions, one AdamW step
    (the work of train.py's train_step, reference train.py:997-1034)."""
    c = C2
    m = build(c)
    opt = torch.optim.AdamW(m.parameters(), lr=1e-4, foreach=True)
    g = torch.Generator(device=dev).manual_seed(3)
    idx = torch.randint(0, 256, (c["B"], c["T"]), generator=g, device=dev)
    tgt = torch.randint(0, 256, (c["B"], c["T"]), generator=g, device=dev)

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = m(idx, tgt, impl="hip")
        loss.backward()
        opt.step()

    log("[bench] c2_train_step hip ...")
    launches0 = ext.launch_count()
    ms = time_steps(step, 3, 1, settle_s=0)
    assert ext.launch_count() > launches0, "HIP library calls missing in the training step"
    leg = {"B": c["B"], "T": c["T"], "n_layer": c["n_layer"], "amp": "bf16", "optimizer": "AdamW",
           "ms": ms, "tok_s": c["B"] * c["T"] / (ms * 1e-3)}
    ext.profile_enable(True)
    step()
    rec = ext.profile_collect()
    ext.profile_enable(False)
    leg["attention_kernels_ms"] = sum(t for n, t in rec if n not in GATED_KERNELS + ENCODER_KERNELS)
    log(f"[bench] c2_train_step: {ms:.1f} ms, {leg['tok_s']:.0f} tok/s (attention kernels {leg['attention_kernels_ms']:.2f} ms)")
    del m, opt
    torch.cuda.empty_cache()
    return leg


if __name__ == "__main__":
    sys.exit(main())
