#!/usr/bin/env python3
"""Benchmark of the fused RoFormer layer kernels on one MI355X (plus the
train-step configs).

One microbench "step" is one forward + backward pass of every fused layer of configs[1], with all
inputs resident in HBM:

* band split: ``x[4, 258, 4100]`` (62 BS-RoFormer bands) -> ``[4, 258, 62, 192]``;
* q/k RMSNorm over the head dim + rotary (theta 10000): two ``[248, 258, 8, 64]`` tensors;
* mask estimator: per band dim 192 -> hidden 768 + tanh -> 2 * I_b + GLU (both projections).

``value`` is the algorithmic HBM bytes of the step divided by the bf16 step time (GB/s); the same
step in fp32 is reported as ``fp32_step``.  Per-op durations come from HIP events recorded on the
launch stream inside the timed region, with the achieved TFLOP/s and MFMA utilisation of each
grouped projection.  ``roofline`` reports the op with the largest share of the step that is a single
kernel; its ``traffic`` is measured in the same run by two child ``rocprofv3 --pmc`` passes
(FETCH_SIZE, WRITE_SIZE) over that op and a plain copy of known size that calibrates the counters.

``train`` reports samples/s of full training steps with the stock modules and with the HIP kernels
patched in, for configs[2] (the headline) and configs[0], [3] and [4] (fewer steps).
``cpu_baseline`` times the restated stock PyTorch modules in fp32 on the host cores: the configs[1]
step at full shapes, and the configs[0] training step.

Usage: ``python bench.py [--gpus 1] [--steps 30] [--warmup 10] [--no-cpu-baseline] [--no-traffic]
[--train-steps 20] [--train-warmup 3] [--train-configs 0,2,3,4]``.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "fused-layer fwd+bwd HBM GB/s (% peak) + BSR train samples/s, 1 MI355X"
BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])
# ops of the step that are one kernel launched n times per op call: the roofline candidates
SINGLE_KERNEL_OPS = {
    "band_split_fwd": ("bs_fwd_kernel", 1),
    "qk_norm_rotary_fwd": ("norm_rot_fwd_kernel", 1),
    "mask_hidden_fwd": ("bs_fwd_kernel", 1),
    "mask_final_fwd": ("me_fwd_dma_kernel", 1),
    "mask_mlp_fwd": ("mlp_fwd_kernel", 1),
}
# roofline bound per op: the mask estimator's grouped projections are MFMA work, the rest HBM streams
OP_BOUND = {"mask_mlp_fwd": "mfma", "mask_hidden_fwd": "mfma", "mask_final_fwd": "mfma"}
# bytes a 16-bit copy of this many elements reads (and writes): the counter calibration
CALIB_ELEMS = 1 << 27


def _args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the configs[1] CPU sample")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 traffic passes")
    ap.add_argument("--traffic-probe", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--train-steps", type=int, default=20, help="timed configs[2] train steps per backend (0: skip)")
    ap.add_argument("--train-warmup", type=int, default=3)
    ap.add_argument("--train-configs", default="0,2,3,4", help="train configs to time (BASELINE.json indices)")
    ap.add_argument("--train-impl", choices=("both", "fused", "stock"), default="both",
                    help="which train-step legs to run (profiling one implementation at a time)")
    return ap.parse_args(argv)


class Workload:
    """Seeded synthetic inputs of configs[1] in one dtype (fixed seeds: every run times the same data)."""

    def __init__(self, torch, ext, dtype):
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
        self.h = torch.randn(self.M, self.NB, self.dim, generator=g(3)).to(dev, dtype)
        pg = g(4)
        self.gamma_bs = (1 + 0.1 * torch.randn(self.F, generator=pg)).to(dev, dtype)
        self.w_bs = torch.cat([(torch.randn(self.dim, d, generator=pg) / d**0.5).reshape(-1) for d in self.dims])
        self.w_bs = self.w_bs.to(dev, dtype)
        self.b_bs = (0.1 * torch.randn(self.NB * self.dim, generator=pg)).to(dev, dtype)
        self.gamma_q = (1 + 0.1 * torch.randn(64, generator=pg)).to(dev)
        self.gamma_k = (1 + 0.1 * torch.randn(64, generator=pg)).to(dev)
        self.w1 = (torch.randn(self.NB, self.hidden, self.dim, generator=pg) / self.dim**0.5).to(dev, dtype)
        self.b1 = (0.1 * torch.randn(self.NB, self.hidden, generator=pg)).to(dev, dtype)
        self.w2 = torch.cat(
            [(torch.randn(2 * d, self.hidden, generator=pg) / self.hidden**0.5).reshape(-1) for d in self.dims]
        ).to(dev, dtype)
        self.b2 = (0.1 * torch.randn(2 * self.F, generator=pg)).to(dev, dtype)
        from pymsst_amd.core.transformer import RotaryEmbedding

        cos, sin = RotaryEmbedding(64, 10000.0).tables(self.T, dev, dtype)
        self.cos, self.sin = cos[..., ::2], sin[..., ::2]  # [1, T, 1, 32] strided views
        gg = g(5)
        self.g_bs = torch.randn(self.M, self.NB, self.dim, generator=gg).to(dev, dtype)
        self.g_q = torch.randn(self.qk_shape, generator=gg).to(dev, dtype)
        self.g_k = torch.randn(self.qk_shape, generator=gg).to(dev, dtype)
        self.g_me = torch.randn(self.M, self.F, generator=gg).to(dev, dtype)
        # 16-bit: the whole mask MLP forward is the one-pass kernel; fp32: hidden layer + final layer
        self.one_pass = (hasattr(ext, "mask_mlp_forward") and dtype != torch.float32
                         and ext.mask_mlp_supported(self.dim, self.hidden, self.dims, dtype))

    def op_names(self):
        """The ops one step runs, in order (the mask forward is one op or two, see ``one_pass``)."""
        mask_fwd = ["mask_mlp_fwd"] if self.one_pass else ["mask_hidden_fwd", "mask_final_fwd"]
        return ["band_split_fwd", "band_split_bwd", "qk_norm_rotary_fwd", "qk_norm_rotary_bwd", *mask_fwd,
                "mask_final_bwd", "mask_hidden_bwd"]

    def fused_mask_bytes(self):
        """Algorithmic bytes of the fused mask-estimator forward as a pure forward (read x, W1, b1, W2, b2;
        write the mask): ``M*NB*D*s + NB*H*D*s + 2F*H*s + (NB*H + 2F)*s + M*F*s``.  The training op also
        writes ``pre`` and the hidden layer for its backward; ``traffic()`` counts those."""
        s = 2 if self.dtype != self.torch.float32 else 4
        M, F, NB, O, H = self.M, self.F, self.NB, self.dim, self.hidden
        return M * NB * O * s + NB * H * O * s + 2 * F * H * s + (NB * H + 2 * F) * s + M * F * s

    def step_bytes(self):
        """Algorithmic bytes of one step: the sum over the ops the step runs (and only those)."""
        traffic = self.traffic()
        return sum(traffic[name][0] for name in self.op_names())

    # --------------------------------------------------------------- ops (name, callable)
    def ops(self):
        e, w = self.ext, self
        st = {}

        def bs_fwd():
            st["bs"] = e.band_split_ragged_forward_packed(w.x, w.gamma_bs, w.w_bs, w.b_bs, w.dims, write_normed=False)

        def bs_bwd():
            e.band_split_ragged_backward_packed(w.g_bs, w.x, True, st["bs"][2], w.gamma_bs, w.w_bs, w.dims, True)

        def qk_fwd():  # q and k in one launch
            st["qk"] = e.rms_norm_rotary_pair_forward(w.q, w.k, w.gamma_q, w.gamma_k, w.cos, w.sin)

        def qk_bwd():
            e.rms_norm_rotary_pair_backward(w.g_q, w.g_k, w.q, w.k, st["qk"][2], st["qk"][3], w.gamma_q, w.gamma_k,
                                            w.cos, w.sin)

        def hid_fwd():
            st["hid"] = e.grouped_linear_forward_act(w.h, w.w1, w.b1, activation="tanh")

        def fin_fwd():
            st["fin"] = e.mask_estimator_final_forward_packed(st["hid"], w.w2, w.b2, w.dims)

        def mlp_fwd():  # one pass; the hidden layer is written for the backward, as in training
            out, pre, st["hid"] = e.mask_mlp_forward(w.h, w.w1, w.b1, w.w2, w.b2, w.dims, save_hidden=True)
            st["fin"] = (out, pre)

        def fin_bwd():
            st["dz"] = e.mask_estimator_final_backward_packed(w.g_me, st["hid"], st["fin"][1], w.w2, w.dims,
                                                              input_activation="tanh")[0]

        def hid_bwd():
            e.grouped_linear_backward(st["dz"], w.h, w.w1, has_bias=True)

        fns = {"band_split_fwd": bs_fwd, "band_split_bwd": bs_bwd, "qk_norm_rotary_fwd": qk_fwd,
               "qk_norm_rotary_bwd": qk_bwd, "mask_hidden_fwd": hid_fwd, "mask_final_fwd": fin_fwd,
               "mask_mlp_fwd": mlp_fwd, "mask_final_bwd": fin_bwd, "mask_hidden_bwd": hid_bwd}
        return [(name, fns[name]) for name in self.op_names()]

    # --------------------------------------------------------------- algorithmic bytes / flops per op
    def traffic(self):
        """``{op: (bytes, flops)}``: each op's own inputs read and outputs written, once each."""
        s = 2 if self.dtype != self.torch.float32 else 4
        M, F, NB, O, H = self.M, self.F, self.NB, self.dim, self.hidden
        R = self.qk_shape[0] * self.qk_shape[1] * self.qk_shape[2]
        D = 64
        return {
            # read x, gamma, W, bias; write out, inv
            "band_split_fwd": (M * F * s + F * s + F * O * s + NB * O * s + M * NB * O * s + 4 * M * NB,
                               2 * M * F * O),
            # read dy, x, inv, gamma, W; write dx, dgamma, dW, dbias
            "band_split_bwd": (M * NB * O * s + 2 * M * F * s + 4 * M * NB + 2 * F * s + 2 * F * O * s + NB * O * s,
                               4 * M * F * O),
            # per tensor: read x, write out, write inv (x2 tensors)
            "qk_norm_rotary_fwd": (2 * (2 * R * D * s + 4 * R), 0),
            # per tensor: read dy, x, inv; write dx (x2)
            "qk_norm_rotary_bwd": (2 * (3 * R * D * s + 4 * R), 0),
            # read x, W1, b1; write h
            "mask_hidden_fwd": (M * NB * O * s + NB * H * O * s + NB * H * s + M * NB * H * s, 2 * M * NB * O * H),
            # read h, W2, b2; write pre, out
            "mask_final_fwd": (M * NB * H * s + 2 * F * H * s + 2 * F * s + 2 * M * F * s + M * F * s,
                               2 * M * 2 * F * H),
            # read x, W1, b1, W2, b2; write pre, out and (for the backward) h
            "mask_mlp_fwd": (M * NB * O * s + NB * H * O * s + NB * H * s + 2 * F * H * s + 2 * F * s
                             + 2 * M * F * s + M * F * s + M * NB * H * s, 2 * M * NB * O * H + 2 * M * 2 * F * H),
            # read g, pre, h, W2; write dz, dW2, db2
            "mask_final_bwd": (M * F * s + 2 * M * F * s + 2 * M * NB * H * s + 4 * F * H * s + 2 * F * s,
                               2 * 2 * M * 2 * F * H),
            # read dz, x, W1; write dx, dW1, db1
            "mask_hidden_bwd": (M * NB * H * s + 2 * M * NB * O * s + 2 * NB * H * O * s + NB * H * s,
                                2 * 2 * M * NB * O * H),
        }


def _time_step(torch, w, steps, warmup):
    """Whole-step time and per-op averages (HIP events on the launch stream) of one workload."""
    ops = w.ops()
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        for _, fn in ops:
            fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record(stream)
    for _ in range(steps):
        for _, fn in ops:
            fn()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = t0.elapsed_time(t1) / steps
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in ops]
          for _ in range(steps)]
    for i in range(steps):
        for j, (_, fn) in enumerate(ops):
            ev[i][j][0].record(stream)
            fn()
            ev[i][j][1].record(stream)
    torch.cuda.synchronize()
    traffic = w.traffic()
    peak_tf = BF16_PEAK_TFLOPS if w.dtype != torch.float32 else FP32_PEAK_TFLOPS
    per_op = {}
    for j, (name, _) in enumerate(ops):
        ms = sum(ev[i][j][0].elapsed_time(ev[i][j][1]) for i in range(steps)) / steps
        nbytes, flops = traffic[name]
        tf = flops / (ms * 1e-3) / 1e12 if flops else None
        per_op[name] = {
            "bytes": int(nbytes),
            "ms": round(ms, 5),
            "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "TFLOP/s": round(tf, 2) if tf else None,
            "mfma_util": round(tf / peak_tf, 4) if tf else None,
        }
    return ms_step, wall, per_op, w.step_bytes() / (ms_step * 1e-3) / 1e9


# ------------------------------------------------------------------------------ counters


def _traffic_probe(op: str) -> int:
    """Child of the traffic passes: runs ``op`` (with the forward ops it depends on) a few times, then the
    calibration copy; rocprofv3 records the counters of both."""
    import torch

    from pymsst_amd.fused_extension import load_fused_band_split_extension

    w = Workload(torch, load_fused_band_split_extension(), torch.bfloat16)
    ops = dict(w.ops())
    deps = {"mask_final_fwd": ["mask_hidden_fwd"]}
    for _ in range(3):
        for d in deps.get(op, []):
            ops[d]()
        ops[op]()
    src = torch.empty(CALIB_ELEMS, dtype=torch.bfloat16, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print("probe done", flush=True)
    return 0


def _counter_means(path: Path, kernel: str) -> tuple[float | None, float | None]:
    """Mean counter value per dispatch of ``kernel`` and of the calibration copy in a counter CSV."""
    k, c = [], []
    with path.open(newline="") as fh:
        for row in csv.DictReader(fh):
            name = row.get("Kernel_Name", "")
            val = float(row.get("Counter_Value", "nan"))
            if kernel in name:
                k.append(val)
            elif "MulFunctor" in name:  # the probe's only multiply is the calibration copy
                c.append(val)
    return (sum(k) / len(k) if k else None), (sum(c) / len(c) if c else None)


def _measure_traffic(op: str, kernel: str, nlaunch: int) -> dict:
    """HBM bytes per launch of ``kernel`` from FETCH_SIZE and WRITE_SIZE passes, each scaled by what the same
    counter reads for a copy of 2^27 bf16 elements (256 MiB read, 256 MiB written)."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        return {"traffic": None, "reason": "rocprofv3 not found"}
    out: dict = {}
    calib_bytes = CALIB_ELEMS * 2
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory() as tmp:
            cmd = [prof, "--pmc", counter, "-f", "csv", "-d", tmp, "-o", "run", "--", sys.executable, "-u",
                   str(Path(__file__).resolve()), "--traffic-probe", op]
            try:
                proc = subprocess.run(cmd, capture_output=True, text=True, timeout=240, cwd=str(REPO),
                                      env={**os.environ, "TMPDIR": tmp})
            except subprocess.TimeoutExpired:
                return {"traffic": None, "reason": f"{counter} pass timed out"}
            files = list(Path(tmp).rglob("*counter_collection.csv"))
            if proc.returncode != 0 and not files:
                return {"traffic": None, "reason": f"{counter} pass failed: {proc.stderr[-300:]}"}
            if not files:
                return {"traffic": None, "reason": f"{counter} pass wrote no counter file"}
            kv, cv = _counter_means(files[0], kernel)
            if kv is None or not cv:
                return {"traffic": None, "reason": f"{counter}: kernel or calibration copy not found"}
            scale = calib_bytes / (cv * 1024)
            out[counter] = {"KiB_per_dispatch": round(kv, 1), "calib_KiB": round(cv, 1), "scale": round(scale, 4),
                            "bytes": kv * 1024 * scale}
    traffic = (out["FETCH_SIZE"]["bytes"] + out["WRITE_SIZE"]["bytes"])
    return {"traffic": int(traffic), "counters": out,
            "method": f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over {op} ({nlaunch} launch(es) per op call, "
                      "mean per dispatch), each scaled by the same counter's reading for a 256 MiB bf16 copy"}


# ------------------------------------------------------------------------------ CPU baseline


def _cpu_baseline(budget_s: float) -> dict:
    """The restated stock PyTorch modules (``pymsst_amd.core``) in fp32 on the host: whole configs[1] steps
    at full shapes (band split, q/k RMSNorm + rotary, mask estimator MLP; forward + backward) for about
    ``budget_s`` seconds, scaled to GB/s with the GPU step's algorithmic bytes; and configs[0] train steps
    (BS-RoFormer tiny, fp32) as samples/s."""
    import statistics

    import torch

    from pymsst_amd.core.bands import BandSplit, MaskEstimator
    from pymsst_amd.core.transformer import RMSNorm, RotaryEmbedding, apply_rotary_emb_fast
    from pymsst_amd.workloads import WORKLOADS, workload_batch

    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    B, T, NB, O, H = 4, 258, len(BSR_WIDTHS), 192, 768
    F = sum(BSR_WIDTHS)
    torch.manual_seed(4)
    bs = BandSplit(O, BSR_WIDTHS)
    me = MaskEstimator(O, BSR_WIDTHS, depth=2, mlp_expansion_factor=4)
    nq, nk = RMSNorm(64), RMSNorm(64)
    x = torch.distributions.Laplace(0.0, 0.05).sample((B, T, F)).requires_grad_()
    h = torch.randn(B, T, NB, O, generator=g).requires_grad_()
    q = torch.randn(B * NB, T, 8, 64, generator=g).requires_grad_()
    k = torch.randn(B * NB, T, 8, 64, generator=g).requires_grad_()
    cos, sin = RotaryEmbedding(64, 10000.0).tables(T, torch.device("cpu"), torch.float32)
    grads = {}

    def step():
        for name, fn in (("bs", lambda: bs(x)), ("me", lambda: me(h)), ("q", lambda: apply_rotary_emb_fast(cos, sin, nq(q))),
                         ("k", lambda: apply_rotary_emb_fast(cos, sin, nk(k)))):
            y = fn()
            if name not in grads:
                grads[name] = torch.randn(y.shape, generator=g)
            y.backward(grads[name])

    step()
    times = []
    t_all = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all >= budget_s:
            break
    # the GPU step's algorithmic bytes at fp32 (s = 4)
    M, R, D, s = B * T, B * NB * T * 8, 64, 4
    step_bytes = (
        (M * F + F + F * O + NB * O + M * NB * O) * s + 4 * M * NB
        + (M * NB * O + 2 * M * F + 2 * F + 2 * F * O + NB * O) * s + 4 * M * NB
        + 2 * (2 * R * D * s + 4 * R) + 2 * (3 * R * D * s + 4 * R)
        + (M * NB * O + NB * H * O + NB * H + M * NB * H) * s
        + (M * NB * H + 2 * F * H + 2 * F + 3 * M * F) * s
        + (3 * M * F + 2 * M * NB * H + 4 * F * H + 2 * F) * s
        + (M * NB * H + 2 * M * NB * O + 2 * NB * H * O + NB * H) * s
    )
    med = statistics.median(times)
    # whole BS-RoFormer tiny training steps on the CPU
    wl = WORKLOADS["bsr_tiny"]
    model = wl.build_model(None, seed=4)
    model.train()
    opt = torch.optim.AdamW(model.parameters(), lr=wl.lr)
    target, mixture = workload_batch(wl, seed=0)
    ctimes = []
    for i in range(4):
        t0 = time.perf_counter()
        loss = model(mixture, target)
        loss.backward()
        opt.step()
        opt.zero_grad(set_to_none=True)
        if i >= 1:
            ctimes.append(time.perf_counter() - t0)
    c0 = statistics.median(ctimes)
    return {
        "value": round(step_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"restated stock PyTorch modules (pymsst_amd.core), fp32, {len(times)} whole configs[1] steps at "
                  f"full shapes (band split, q/k RMSNorm+rotary, mask-estimator MLP; fwd+bwd), median "
                  f"{med:.3f} s per step; os.cpu_count()={os.cpu_count()}, torch.get_num_threads()={threads}",
        "ms_per_step": round(med * 1e3, 1),
        "configs0_train": {"samples_per_s": round(wl.batch / c0, 3), "ms_median": round(c0 * 1e3, 1), "steps": 3,
                           "workload": "configs[0] BS-RoFormer tiny, fp32, batch 2 x 32768 stereo, spectrogram L1, "
                                       "AdamW"},
    }


# ------------------------------------------------------------------------------ train leg


_TRAIN = {
    0: ("bsr_tiny", "configs[0] BS-RoFormer tiny dim 64, depth 1, 4x32 heads, 1 stem, batch 2 x 32768 stereo, fp32, "
                    "spectrogram L1, AdamW"),
    2: ("bsr_train", "configs[2] BS-RoFormer dim 192, depth 6, 8x64 heads, 4 stems, batch 4 x 131584 stereo "
                     "(258 frames), bf16 autocast, multi-res STFT L1, AdamW 5e-4"),
    3: ("mbr_train", "configs[3] Mel-band RoFormer dim 192, depth 8, 8x64 heads, 4 stems, 60 mel bands, batch 4 x "
                     "352800 stereo (690 frames), bf16 autocast, L1, AdamW 5e-4"),
    4: ("bsr_large", "configs[4] BS-RoFormer dim 512, depth 12, 8x64 heads, 1 stem, batch 2 x 485100 stereo "
                     "(948 frames), activation checkpointing per axial block, bf16 autocast, L1, AdamW 5e-4"),
}


def _device_work_per_step(torch, train_step, nsteps: int) -> dict:
    """Device copies, fills and kernel launches per steady-state train step (torch.profiler over ``nsteps``
    untimed steps after the timed ones)."""
    from torch.profiler import ProfilerActivity, profile

    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        for _ in range(nsteps):
            train_step()
        torch.cuda.synchronize()
    rows = {r.key: r for r in prof.key_averages()}

    def per(key):
        r = rows.get(key)
        return {"count": round(r.count / nsteps, 1), "ms": round(r.device_time_total / nsteps / 1e3, 3)} if r else \
            {"count": 0, "ms": 0.0}

    launch_apis = ("hipLaunchKernel", "hipExtModuleLaunchKernel", "hipModuleLaunchKernel")
    return {
        "memcpy_dtod": per("Memcpy DtoD (Device -> Device)"),
        "memcpy_htod": per("Memcpy HtoD (Host -> Device)"),
        "memcpy_dtoh": per("Memcpy DtoH (Device -> Host)"),
        "memset": per("Memset (Device)"),
        "kernel_launches": round(sum(rows[k].count for k in launch_apis if k in rows) / nsteps, 1),
        "method": f"torch.profiler over {nsteps} steady-state steps after the timed ones",
    }


def _train_leg(torch, cfg: int, steps: int, warmup: int, impls=("stock", "fused"), profile_steps: int = 0) -> dict:
    """Samples/s of full training steps (forward, backward, AdamW step) = batch / median step time, for the
    stock modules and for the model patched onto the HIP kernels (same seed, same batch); the median time
    the host takes to enqueue a step; with ``profile_steps`` the device copies and launches per step."""
    import statistics

    from pymsst_amd import fused_roformer as fr
    from pymsst_amd.workloads import WORKLOADS, workload_batch

    key, desc = _TRAIN[cfg]
    wl = WORKLOADS[key]
    dev = torch.device("cuda:0")
    target, mixture = workload_batch(wl, seed=0, device=dev)
    out = {}
    for impl in impls:
        fr.restore_stock_implementations()
        model = wl.build_model(dev, seed=4)
        model.train()
        if impl == "fused":
            for k, v in fr.RUNTIME_PRESETS["hip_full"].items():
                os.environ[k] = v
            status = fr.apply_roformer_fused_training_backend(model, "hip", rms_norm_mode="fast")
            if status.active == "off":
                raise RuntimeError(f"fused backend inactive: {status.reason}")
        else:
            os.environ[fr.CORE_GROUPED_TRAIN_ENV] = "1"
        opt = torch.optim.AdamW(model.parameters(), lr=wl.lr)

        def train_step():
            with torch.autocast("cuda", dtype=wl.amp_dtype or torch.float32, enabled=wl.amp_dtype is not None):
                loss = model(mixture, target)
            loss.backward()
            opt.step()
            opt.zero_grad(set_to_none=True)
            return loss

        times, enqueue, losses = [], [], []
        for i in range(warmup + steps):
            print(f"[train] configs[{cfg}] {impl} step {i}", file=sys.stderr, flush=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            loss = train_step()
            t_enq = time.perf_counter()
            torch.cuda.synchronize()
            if i >= warmup:
                times.append(time.perf_counter() - t0)
                enqueue.append(t_enq - t0)
                losses.append(float(loss.detach()))
        med = statistics.median(times)
        out[impl] = {"ms_median": round(med * 1e3, 2), "samples_per_s": round(wl.batch / med, 3),
                     "host_enqueue_ms_median": round(statistics.median(enqueue) * 1e3, 2),
                     "first_loss": round(losses[0], 6), "last_loss": round(losses[-1], 6)}
        if profile_steps > 0:
            out[impl]["per_step_device_work"] = _device_work_per_step(torch, train_step, profile_steps)
        fr.restore_stock_implementations(model)
        del model, opt
        torch.cuda.empty_cache()
    res = {"workload": desc, "steps": steps, "warmup": warmup, "detail": out}
    for impl in impls:
        res[f"{impl}_samples_per_s"] = out[impl]["samples_per_s"]
    if "fused" in out and "stock" in out:
        res["speedup"] = round(out["fused"]["samples_per_s"] / out["stock"]["samples_per_s"], 3)
    return res


# ------------------------------------------------------------------------------ main


def main(argv=None) -> int:
    args = _args(argv)
    if args.traffic_probe:
        return _traffic_probe(args.traffic_probe)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (multi-GPU runs are out of scope)"}))
        return 2
    import torch

    from pymsst_amd.fused_extension import load_fused_band_split_extension

    ext = load_fused_band_split_extension()
    w = Workload(torch, ext, torch.bfloat16)
    ms_per_step, wall, per_op, value = _time_step(torch, w, args.steps, args.warmup)
    traffic = w.traffic()
    fused_mask_bytes = w.fused_mask_bytes()
    step_bytes = w.step_bytes()
    del w
    w32 = Workload(torch, ext, torch.float32)
    ms32, _, per_op32, value32 = _time_step(torch, w32, max(args.steps // 3, 3), 3)
    step_bytes32 = w32.step_bytes()
    del w32
    torch.cuda.empty_cache()

    # roofline of the dominant single kernel
    single = {name: per_op[name]["ms"] / n for name, (_, n) in SINGLE_KERNEL_OPS.items() if name in per_op}
    dom = max(single, key=single.get)
    kname, nlaunch = SINGLE_KERNEL_OPS[dom]
    launch_ms = single[dom]
    launch_bytes = traffic[dom][0] / nlaunch
    launch_flops = traffic[dom][1] / nlaunch
    # the bound of each op class is fixed by the scope table, not by the bytes this build chooses to save:
    # the grouped projections of the mask estimator are MFMA-bound (fused AI ~498 FLOP/B), the norms,
    # rotary and band split HBM-bound
    bound = OP_BOUND.get(dom, "hbm")
    if bound == "mfma":
        achieved, peak, unit = launch_flops / (launch_ms * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved, peak, unit = launch_bytes / (launch_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
    meas = {"traffic": None, "reason": "skipped (--no-traffic)"} if args.no_traffic else \
        _measure_traffic(dom, kname, nlaunch)
    roofline = {
        "kernel": kname, "op": dom, "bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
        "frac": round(achieved / peak, 4), "traffic": meas.get("traffic"), "bytes_per_launch": int(launch_bytes),
        "flops_per_launch": int(launch_flops), "avg_ms": round(launch_ms, 5),
        "hbm_view": {
            "bytes_per_launch": int(launch_bytes),
            "GB/s": round(launch_bytes / (launch_ms * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(launch_bytes / (launch_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "pure_forward_bytes": int(fused_mask_bytes) if dom == "mask_mlp_fwd" else None,
            "note": "bytes_per_launch counts what the training op reads and writes, including the tensors it "
                    "saves for the backward; pure_forward_bytes is the fused forward alone (x, W1, b1, W2, b2 "
                    "read, mask written)",
        },
        "traffic_detail": {k: v for k, v in meas.items() if k != "traffic"},
    }

    # achievable streaming rate on this GPU: a plain elementwise copy of 1 GiB (read + write)
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device="cuda").uniform_()
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    stream = torch.cuda.current_stream()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(10):
        torch.mul(src, 1.0, out=dst)
    c1.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 2 * src.numel() * src.element_size() * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del src, dst

    impls = ("stock", "fused") if args.train_impl == "both" else (args.train_impl,)
    train = None
    if args.train_steps > 0:
        cfgs = [int(c) for c in args.train_configs.split(",") if c.strip()]
        head = 2 if 2 in cfgs else cfgs[0]
        train = _train_leg(torch, head, args.train_steps, args.train_warmup, impls, profile_steps=2)
        others = {}
        for cfg in cfgs:
            if cfg != head:
                others[f"configs[{cfg}]"] = _train_leg(torch, cfg, max(args.train_steps // 3, 4), 2, impls)
        if others:
            train["other_configs"] = others
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
            "workload": "configs[1] kernel microbench, fwd+bwd: band split [4,258,4100]->192 (62 bands), q/k "
                        "RMSNorm+rotary [248,258,8,64]x2, mask estimator per band 192 -> 768 + tanh -> 2*I_b + GLU",
            "bytes_per_step": int(step_bytes),
            "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
            "hbm_copy_GBps_measured": round(copy_gbs, 1),
            "wall_s_timed": round(wall, 3),
        },
        "per_op": per_op,
        "fp32_step": {"ms_per_step": round(ms32, 4), "GB/s": round(value32, 2), "bytes_per_step": int(step_bytes32),
                      "per_op": per_op32},
        "train": train,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
