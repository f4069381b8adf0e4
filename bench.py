#!/usr/bin/env python3
"""Benchmark of the fused RoFormer layer kernels on one MI355X.

One "step" is one forward + backward pass of every fused layer of the kernel
microbench, bf16, with all inputs resident in HBM:

* band split: ``x[4, 258, 4100]`` (62 BS-RoFormer bands) -> ``[4, 258, 62, 192]``,
  saved-input backward;
* q/k RMSNorm over the head dim + rotary (theta 10000): two ``[248, 258, 8, 64]`` tensors;
* mask estimator final layer: per band hidden 768 -> 2 * I_b, bias, GLU.

``value`` is the algorithmic HBM bytes of all kernels in a step divided by the
step time (GB/s).  Per-op average durations come from HIP events recorded on
the launch stream inside the timed region; ``roofline`` reports the op with
the largest share of the step.  ``cpu_baseline`` times the numpy oracle
(``oracle/``) on a bounded sample of the same workload on the host.

``train`` reports the second half of the metric: BS-RoFormer train
samples/s with the stock modules and with the HIP kernels patched in.

Usage: ``python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu-baseline]
[--train-steps 20] [--train-warmup 3]``.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "fused-layer fwd+bwd HBM GB/s (% peak) + BSR train samples/s, 1 MI355X"
# ops of the step that are a single kernel, launched n times per op call
SINGLE_KERNEL_OPS = {
    "band_split_fwd": ("bs_fwd_kernel", 1),
    "qk_norm_rotary_fwd": ("norm_rot_fwd_kernel", 2),
    "mask_final_fwd": ("me_fwd_dma_kernel", 1),
}
# measured HBM bytes per launch, by kernel: rocprofv3 FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 (KiB per
# dispatch x 1024).  The factors are what the same counters read for a 1 GiB bf16 copy (torch.mul) in
# the same runs: FETCH_SIZE 524310 KiB for 1048576 KiB read, WRITE_SIZE 1048576 KiB for 1048576 written.
TRAFFIC_PER_LAUNCH: dict = {
    "me_fwd_dma_kernel": (57624 * 2 + 26676) * 1024,
    "norm_rot_fwd_kernel": (32278 * 2 + 65984) * 1024,
    "bs_fwd_kernel": (14253 * 2 + 26452) * 1024,
}
BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])


def _args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--train-steps", type=int, default=20, help="timed BS-RoFormer train steps per backend (0: skip)")
    ap.add_argument("--train-warmup", type=int, default=3)
    ap.add_argument("--train-impl", choices=("both", "fused", "stock"), default="both",
                    help="which train-step legs to run (profiling one implementation at a time)")
    ap.add_argument("--train-workload", default="bsr_train",
                    help="training configuration of the train leg (pymsst_amd.workloads.WORKLOADS key; "
                         "bsr_train = configs[2])")
    return ap.parse_args(argv)


class Workload:
    """Seeded synthetic inputs of configs[1] (fixed seeds, so every run times the same data)."""

    def __init__(self, torch, ext, dtype):
        import numpy as np

        self.torch, self.ext, self.dtype = torch, ext, dtype
        dev = torch.device("cuda:0")
        self.dims = BSR_WIDTHS
        self.B, self.T, self.dim, self.hidden = 4, 258, 192, 768
        self.M = self.B * self.T
        self.F = sum(self.dims)
        self.NB = len(self.dims)
        g = lambda s: torch.Generator().manual_seed(s)  # noqa: E731
        lap = torch.distributions.Laplace(0.0, 0.05)
        torch.manual_seed(0)
        self.x = lap.sample((self.M, self.F)).to(dev, dtype)
        self.qk_shape = (self.B * self.NB, self.T, 8, 64)
        self.q = torch.randn(self.qk_shape, generator=g(1)).to(dev, dtype)
        self.k = torch.randn(self.qk_shape, generator=g(2)).to(dev, dtype)
        self.h = torch.randn(self.M, self.NB, self.hidden, generator=g(3)).to(dev, dtype)
        pg = g(4)
        self.gamma_bs = (1 + 0.1 * torch.randn(self.F, generator=pg)).to(dev, dtype)
        self.w_bs = torch.cat([(torch.randn(self.dim, d, generator=pg) / d**0.5).reshape(-1) for d in self.dims])
        self.w_bs = self.w_bs.to(dev, dtype)
        self.b_bs = (0.1 * torch.randn(self.NB * self.dim, generator=pg)).to(dev, dtype)
        self.gamma_q = (1 + 0.1 * torch.randn(64, generator=pg)).to(dev)
        self.gamma_k = (1 + 0.1 * torch.randn(64, generator=pg)).to(dev)
        self.w_me = torch.cat(
            [(torch.randn(2 * d, self.hidden, generator=pg) / self.hidden**0.5).reshape(-1) for d in self.dims]
        ).to(dev, dtype)
        self.b_me = (0.1 * torch.randn(2 * self.F, generator=pg)).to(dev, dtype)
        from pymsst_amd.core.transformer import RotaryEmbedding

        cos, sin = RotaryEmbedding(64, 10000.0).tables(self.T, dev, dtype)
        self.cos, self.sin = cos[..., ::2], sin[..., ::2]  # [1, T, 1, 32] strided views
        gg = g(5)
        self.g_bs = torch.randn(self.M, self.NB, self.dim, generator=gg).to(dev, dtype)
        self.g_q = torch.randn(self.qk_shape, generator=gg).to(dev, dtype)
        self.g_k = torch.randn(self.qk_shape, generator=gg).to(dev, dtype)
        self.g_me = torch.randn(self.M, self.F, generator=gg).to(dev, dtype)
        del np

    # --------------------------------------------------------------- ops (name, callable)
    def ops(self):
        e, w = self.ext, self
        state = {}

        def bs_fwd():
            state["bs"] = e.band_split_ragged_forward_packed(w.x, w.gamma_bs, w.w_bs, w.b_bs, w.dims, write_normed=False)

        def bs_bwd():
            e.band_split_ragged_backward_packed(w.g_bs, w.x, True, state["bs"][2], w.gamma_bs, w.w_bs, w.dims, True)

        def qk_fwd():
            state["q"] = e.rms_norm_rotary_forward(w.q, w.gamma_q, w.cos, w.sin)
            state["k"] = e.rms_norm_rotary_forward(w.k, w.gamma_k, w.cos, w.sin)

        def qk_bwd():
            e.rms_norm_rotary_backward(w.g_q, w.q, state["q"][1], w.gamma_q, w.cos, w.sin)
            e.rms_norm_rotary_backward(w.g_k, w.k, state["k"][1], w.gamma_k, w.cos, w.sin)

        def me_fwd():
            state["me"] = e.mask_estimator_final_forward_packed(w.h, w.w_me, w.b_me, w.dims)

        def me_bwd():
            e.mask_estimator_final_backward_packed(w.g_me, w.h, state["me"][1], w.w_me, w.dims)

        return [("band_split_fwd", bs_fwd), ("band_split_bwd", bs_bwd), ("qk_norm_rotary_fwd", qk_fwd),
                ("qk_norm_rotary_bwd", qk_bwd), ("mask_final_fwd", me_fwd), ("mask_final_bwd", me_bwd)]

    # --------------------------------------------------------------- algorithmic bytes / flops per op
    def traffic(self):
        s = 2 if self.dtype != self.torch.float32 else 4
        M, F, NB, O, H = self.M, self.F, self.NB, self.dim, self.hidden
        R = self.qk_shape[0] * self.qk_shape[1] * self.qk_shape[2]
        D = 64
        return {
            # read x, gamma, W, bias; write out, inv
            "band_split_fwd": (M * F * s + F * s + F * O * s + NB * O * s + M * NB * O * s + 4 * M * NB,
                               2 * M * F * O),
            # algorithmic (the op's own inputs and outputs): read dy, x, inv, gamma, W; write dx, dgamma,
            # dW, dbias.  The kernels also read the forward output for the per-row dots; that read is
            # this implementation's choice and is not counted.
            "band_split_bwd": (M * NB * O * s + 2 * M * F * s + 4 * M * NB + 2 * F * s + 2 * F * O * s + NB * O * s,
                               4 * M * F * O),
            # per tensor: read x, write out, write inv (x2 tensors)
            "qk_norm_rotary_fwd": (2 * (2 * R * D * s + 4 * R), 0),
            # per tensor: read dy, x, inv; write dx (x2)
            "qk_norm_rotary_bwd": (2 * (3 * R * D * s + 4 * R), 0),
            # read x, W, bias; write pre, out
            "mask_final_fwd": (M * NB * H * s + 2 * F * H * s + 2 * F * s + 2 * M * F * s + M * F * s,
                               2 * M * 2 * F * H),
            # read g, pre, x, W; write dx, dW, dbias
            "mask_final_bwd": (M * F * s + 2 * M * F * s + 2 * M * NB * H * s + 4 * F * H * s + 2 * F * s,
                               2 * 2 * M * 2 * F * H),
        }


def _cpu_baseline(budget_s: float):
    """Time the numpy oracle (float32 arithmetic) on row slices of the same workload.

    Each op runs on ``rows`` rows (a bounded sample of the M=1032 / R=511,872 rows of the
    GPU step) and its algorithmic bytes are scaled by the same fraction; the result is
    the oracle's GB/s over one full step's bytes, extrapolated from the sample.
    """
    import numpy as np

    import oracle

    try:
        from threadpoolctl import threadpool_info

        cores = max([int(p.get("num_threads", 1)) for p in threadpool_info()] + [1])
    except Exception:  # pragma: no cover
        cores = os.cpu_count() or 1
    rng = np.random.default_rng(0)
    dims, O, H = BSR_WIDTHS, 192, 768
    F, NB = sum(dims), len(dims)
    m = 64  # rows per band-split / mask sample (of 1032)
    rq = 32 * 64 * 8  # rows per q/k sample (of 511,872), one tensor [32, 64, 8, 64]
    acc = np.float32
    x = (rng.laplace(0, 0.05, (m, F))).astype(acc)
    gam = [np.ones(d, acc) for d in dims]
    ws = [rng.standard_normal((O, d)).astype(acc) for d in dims]
    bs = [np.zeros(O, acc) for d in dims]
    dy = rng.standard_normal((m, NB, O)).astype(acc)
    q = rng.standard_normal((32, 64, 8, 64)).astype(acc)
    cos, sin = oracle.rotary_tables(64, 64)
    gq = np.ones(64, acc)
    h = rng.standard_normal((m, NB, H)).astype(acc)
    w2 = [rng.standard_normal((2 * d, H)).astype(acc) for d in dims]
    b2 = np.zeros(2 * F, acc)
    g2 = rng.standard_normal((m, F)).astype(acc)
    s = 4
    sample_bytes = (
        (m * F + F + F * O + NB * O + m * NB * O) * s + 4 * m * NB  # band split fwd
        + (m * NB * O + 2 * m * F + 2 * F + 2 * F * O + NB * O) * s + 4 * m * NB  # band split bwd
        + (2 * rq * 64 * s + 4 * rq) + (3 * rq * 64 * s + 4 * rq)  # one q/k tensor fwd + bwd
        + (m * NB * H + 2 * F * H + 2 * F + 3 * m * F) * s  # mask fwd
        + (3 * m * F + 2 * m * NB * H + 4 * F * H + 2 * F) * s  # mask bwd
    )

    def one():
        o, n, inv = oracle.band_split_ragged_forward(x, gam, ws, bs, dims, "f32", acc)
        oracle.band_split_ragged_backward_lean(dy, x, inv, gam, ws, dims, "f32", acc)
        oq, iq = oracle.rms_norm_rotary_forward(q, gq, cos, sin, "f32", acc)
        oracle.rms_norm_rotary_backward(q, q, iq, gq, cos, sin, "f32", "f32", acc)
        out, pre = oracle.mask_estimator_final_forward(h, w2, b2, dims, "f32", acc)
        oracle.mask_estimator_final_backward(g2, h, pre, w2, dims, "f32", acc)

    one()
    reps, t0 = 0, time.perf_counter()
    while True:
        one()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    gbs = sample_bytes * reps / el / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": int(cores),
        "kind": "port",
        "sample": f"numpy oracle (fp32) on {m} of 1032 rows for band split and mask final, "
                  f"{rq} of 511872 q/k rows (one tensor); {reps} reps in {el:.1f}s",
    }


_TRAIN_DESCRIPTIONS = {
    "bsr_train": "configs[2] BS-RoFormer dim 192, depth 6, 8x64 heads, 4 stems, batch 4 x 131584 stereo "
                 "(258 frames), bf16 autocast, multi-res STFT L1, AdamW 5e-4",
    "bsr_large": "configs[4] BS-RoFormer dim 512, depth 12, 8x64 heads, 1 stem, batch 2 x 485100 stereo "
                 "(948 frames), activation checkpointing per axial block, bf16 autocast, L1, AdamW 5e-4",
    "mbr_train": "configs[3] Mel-band RoFormer dim 192, depth 8, 8x64 heads, 4 stems, 60 mel bands, batch 4 x "
                 "352800 stereo (690 frames), bf16 autocast, L1, AdamW 5e-4",
}


def _train_leg(torch, steps: int, warmup: int, impls=("stock", "fused"), workload: str = "bsr_train") -> dict:
    """Default configs[2]: BS-RoFormer dim 192, depth 6, 4 stems, batch 4 x 131584 stereo samples,
    bf16 autocast, multi-resolution STFT loss, AdamW 5e-4.  One step = forward, backward and
    optimizer step; train samples/s = batch / median step time, for the stock modules and for
    the model patched onto the HIP kernels (same seed, same batch)."""
    import statistics

    from pymsst_amd import fused_roformer as fr
    from pymsst_amd.workloads import WORKLOADS, workload_batch

    wl = WORKLOADS[workload]
    dev = torch.device("cuda:0")
    target, mixture = workload_batch(wl, seed=0, device=dev)
    out = {}
    for impl in impls:
        fr.restore_stock_implementations()
        model = wl.build_model(dev, seed=4)
        model.train()
        status = None
        if impl == "fused":
            for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
                os.environ[key] = value
            status = fr.apply_roformer_fused_training_backend(model, "hip", rms_norm_mode="fast")
            if status.active == "off":
                raise RuntimeError(f"fused backend inactive: {status.reason}")
        else:
            os.environ[fr.CORE_GROUPED_TRAIN_ENV] = "1"
        opt = torch.optim.AdamW(model.parameters(), lr=wl.lr)
        times, losses = [], []
        for i in range(warmup + steps):
            print(f"[train] {workload} {impl} step {i}", file=sys.stderr, flush=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with torch.autocast("cuda", dtype=wl.amp_dtype or torch.float32, enabled=wl.amp_dtype is not None):
                loss = model(mixture, target)
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
            torch.cuda.synchronize()
            if i >= warmup:
                times.append(time.perf_counter() - t0)
                losses.append(float(loss.detach()))
        med = statistics.median(times)
        out[impl] = {"ms_median": round(med * 1e3, 2), "samples_per_s": round(wl.batch / med, 3),
                     "first_loss": round(losses[0], 6), "last_loss": round(losses[-1], 6)}
        fr.restore_stock_implementations(model)
        del model, opt
        torch.cuda.empty_cache()
    res = {
        "workload": _TRAIN_DESCRIPTIONS.get(workload, workload),
        "steps": steps,
        "warmup": warmup,
        "detail": out,
    }
    for impl in impls:
        res[f"{impl}_samples_per_s"] = out[impl]["samples_per_s"]
    if "fused" in out and "stock" in out:
        res["speedup"] = round(out["fused"]["samples_per_s"] / out["stock"]["samples_per_s"], 3)
    return res


def main(argv=None) -> int:
    args = _args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (multi-GPU runs are out of scope)"}))
        return 2
    import torch

    from pymsst_amd.fused_extension import load_fused_band_split_extension

    ext = load_fused_band_split_extension()
    dtype = torch.bfloat16
    w = Workload(torch, ext, dtype)
    ops = w.ops()
    traffic = w.traffic()
    stream = torch.cuda.current_stream()

    def step():
        for _, fn in ops:
            fn()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # whole-step timing
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = t_start.elapsed_time(t_end) / args.steps

    # per-op timing with events bracketing each op on the launch stream
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in ops]
          for _ in range(args.steps)]
    for i in range(args.steps):
        for j, (_, fn) in enumerate(ops):
            ev[i][j][0].record(stream)
            fn()
            ev[i][j][1].record(stream)
    torch.cuda.synchronize()
    per_op = {}
    for j, (name, _) in enumerate(ops):
        ms = sum(ev[i][j][0].elapsed_time(ev[i][j][1]) for i in range(args.steps)) / args.steps
        nbytes, flops = traffic[name]
        per_op[name] = {
            "ms": round(ms, 5),
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2) if flops else None,
        }
    total_bytes = sum(b for b, _ in traffic.values())
    value = total_bytes / (ms_per_step * 1e-3) / 1e9
    # roofline of the dominant single kernel: ops that are one kernel launched `n` times
    single = {name: per_op[name]["ms"] / n for name, (_, n) in SINGLE_KERNEL_OPS.items()}
    dom = max(single, key=single.get)
    kname, nlaunch = SINGLE_KERNEL_OPS[dom]
    launch_ms = single[dom]
    launch_bytes = traffic[dom][0] / nlaunch
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    roofline = {
        "kernel": kname,
        "op": dom,
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": TRAFFIC_PER_LAUNCH.get(kname),
        "bytes_per_launch": int(launch_bytes),
        "avg_ms": round(launch_ms, 5),
    }
    # achievable streaming rate on this GPU: a plain elementwise copy of 1 GiB (read + write)
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(10):
        torch.mul(src, 1.0, out=dst)
    c1.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * src.element_size() * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del src, dst
    impls = ("stock", "fused") if args.train_impl == "both" else (args.train_impl,)
    train = (_train_leg(torch, args.train_steps, args.train_warmup, impls, args.train_workload)
             if args.train_steps > 0 else None)
    cpu = None if args.no_cpu_baseline else _cpu_baseline(args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "configs[1] kernel microbench: band split [4,258,4100]->192 (62 bands), "
                        "q/k RMSNorm+rotary [248,258,8,64]x2, mask-estimator final 768->2*I_b+GLU; fwd+bwd",
            "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
            "hbm_copy_GBps_measured": round(copy_gbs, 1),
            "wall_s_timed": round(wall, 3),
        },
        "per_op": per_op,
        "train": train,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
