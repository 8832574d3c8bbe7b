"""Benchmark of the mHC layer forward+backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload static]

Prints ONE JSON line (rank 0): tokens/s of the whole fwd+bwd step, the
achieved HBM GB/s from algorithmic bytes, the roofline of the dominant
kernel (HIP-event timing of its launches inside the timed region), and a
CPU baseline (the PyTorch oracle on the host cores, bounded sample).

Workloads (the metric is quoted at n=4, C=4096):
  static  - C3: MHCLayer static-H, x fp32 [8192, 4, 4096]      (default)
Inputs are synthetic (seeded N(0,1)) and already resident in HBM; each
step uses the next of three rotating input sets (3 x ~1 GB > the 256 MB
MALL) so no step reads the previous step's data from cache.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E, AMD public spec
ROOT = os.path.dirname(os.path.abspath(__file__))


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (calibrated FETCH_SIZE + WRITE_SIZE), or None if not measured."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.md")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1]), os.path.relpath(path, ROOT)
    return None, None


def _die(msg: str, code: int = 2):
    print(msg, file=sys.stderr, flush=True)
    sys.exit(code)


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------

class StaticWorkload:
    """C3: static-H MHCLayer fwd+bwd, x fp32 [8192, 4, 4096]."""

    name = "static"
    B, n, C = 8192, 4, 4096
    dtype = "f32"
    kernel = "layer_bwd"

    def __init__(self, torch, mhc, device, sets=3):
        self.torch = torch
        B, n, C = self.B, self.n, self.C
        g = torch.Generator(device=device).manual_seed(0)
        self.xs = [torch.randn(B, n, C, device=device, generator=g).requires_grad_(True) for _ in range(sets)]
        self.gs = [torch.randn(B, n, C, device=device, generator=g) for _ in range(sets)]
        torch.manual_seed(0)
        self.layer = mhc.MHCLayer(C, n, use_dynamic_h=False).to(device)
        with torch.no_grad():
            self.layer.H_pre.normal_()
            self.layer.H_post.normal_()
            self.layer.H_res.normal_()
        self.params = list(self.layer.parameters())
        self.i = 0

    def step(self):
        x = self.xs[self.i % len(self.xs)]
        g = self.gs[self.i % len(self.gs)]
        self.i += 1
        out = self.layer(x)
        return self.torch.autograd.grad(out, [x] + self.params, g)

    @property
    def E(self):
        return self.B * self.n * self.C

    def step_bytes(self):
        # fwd: read x (4E) + write out (4E); bwd: read g (4E) + x (4E) + write dx (4E)
        return 20 * self.E

    def kernel_bytes(self):
        # dominant kernel layer_bwd: read g + x, write dx (fp32)
        return 12 * self.E

    def config(self):
        return {"workload": "C3 MHCLayer static-H fwd+bwd", "tokens": self.B, "n": self.n, "C": self.C,
                "x_dtype": "f32", "sinkhorn_iters": 20}

    def cpu_baseline(self, torch, R, seconds):
        """The oracle (PyTorch, fp32) fwd+bwd on a token sample of the same
        layer; returns tokens/s and the sample description."""
        sample = 256
        d = R.static_layer_inputs(sample, self.n, self.C, seed=1, weight_ones=True)
        x = d["x"].requires_grad_(True)
        ps = [d[k].float().requires_grad_(True) for k in ("weight", "H_pre", "H_post", "H_res")]

        def run():
            out = R.mhc_layer_static(x, *ps, 20, 1e-8, 1e-5, dtype=torch.float32)
            torch.autograd.grad(out, [x] + ps, d["grad"])

        for _ in range(2):
            run()
        times = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        return sample / med, (f"oracle.reference.mhc_layer_static fp32 fwd+bwd (autograd) on {sample} of "
                              f"{self.B} tokens, n={self.n}, C={self.C}; median of {len(times)} runs")


WORKLOADS = {"static": StaticWorkload}


# ---------------------------------------------------------------------------

def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="static")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bounded CPU-baseline sample time (0 disables)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a plain 1 GiB device copy (known bytes) for PMC counter calibration")
    a = ap.parse_args(argv)

    if a.gpus != 1:
        _die(f"bench.py: this build runs on ONE GPU; --gpus {a.gpus} is not supported (the layer shards over "
             "tokens with one all-reduce of parameter gradients; see DESIGN.md).")

    import torch

    if not torch.cuda.is_available():
        _die("bench.py: no HIP device visible")
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import mhc_ascend_amd as mhc
    from mhc_ascend_amd import _lib

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    wl = WORKLOADS[a.workload](torch, mhc, device)

    print(f"[bench] workload={wl.name} warmup={a.warmup} steps={a.steps}", file=sys.stderr, flush=True)
    for _ in range(a.warmup):
        wl.step()
    torch.cuda.synchronize()

    if a.copy_calib:
        src = torch.empty(1 << 28, dtype=torch.float32, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    _lib.timing_reset()
    _lib.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        wl.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.timing_enable(False)
    k_ms, k_n = _lib.timing_query(wl.kernel)
    print(f"[bench] timed {a.steps} steps in {t1 - t0:.4f} s", file=sys.stderr, flush=True)

    ms_per_step = (t1 - t0) * 1e3 / a.steps
    tokens_per_s = wl.B / (ms_per_step / 1e3)
    step_gbps = wl.step_bytes() / (ms_per_step / 1e3) / 1e9
    k_avg_ms = k_ms / max(k_n, 1)
    k_gbps = wl.kernel_bytes() / (k_avg_ms / 1e3) / 1e9 if k_n else None
    traffic, traffic_src = measured_traffic(wl.kernel, wl.name)

    cpu = None
    if a.cpu_seconds > 0:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import reference as R
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        print(f"[bench] CPU baseline on {cores} cores for ~{a.cpu_seconds:.0f} s", file=sys.stderr, flush=True)
        v, sample = wl.cpu_baseline(torch, R, a.cpu_seconds)
        cpu = {"value": v, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port", "sample": sample}

    rec = {
        "metric": "mHC layer fwd+bwd tokens/sec + achieved HBM GB/s (n=4, C=4096)",
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic N(0,1), seeded, resident in HBM (3 rotating input sets)",
        "config": wl.config(),
        "hbm_gbps": step_gbps,
        "roofline": {
            "kernel": wl.kernel,
            "bound": "hbm",
            "achieved": k_gbps,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": (k_gbps / PEAK_HBM_GBPS) if k_gbps else None,
            "traffic": traffic,
            "traffic_source": traffic_src,
            "avg_launch_ms": k_avg_ms,
            "launches": k_n,
            "algorithmic_bytes": wl.kernel_bytes(),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
