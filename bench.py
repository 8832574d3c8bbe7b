"""Benchmark of the mHC layer forward+backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload static|dynamic|infer|infer_bf16|wrapper|wrapper8|ops] [--paper-configs]

Prints ONE JSON line: tokens/s of the whole fwd+bwd step (K steps timed on
the host clock with nothing else in the timed region), the achieved HBM GB/s
from algorithmic bytes, the reference's timing protocol (median and 10%
trimmed mean of >= 100 event-timed steps, benchmark.py:175-269), the
roofline of the dominant kernel (HIP events around each of its launches on
the stream the library launches on, in a separate pass after the timed
region), and a CPU baseline (the PyTorch oracle on the host cores, on a
bounded token sample).  The default static workload (C3, the metric's
configuration) also carries sub-records of the dynamic-H workload (C4, the
reference layer's default path), the wrapper (C5), the standalone operators
(C2), the forward-only entry at the C4 shape and the wrapper at n = 8 (with
the unfused path timed beside it), each measured the same way.

Workloads (the metric is quoted at n=4, C=4096):
  static  - C3: MHCLayer static-H, x fp32 [8192, 4, 4096]          (default)
  dynamic - C4: MHCLayer dynamic-H, x bf16 [8192, 4, 4096], phi [16384, 24]
  infer   - C4 shape forward only (eval, no_grad, parameters packed once),
            fp32 output as the reference; infer_bf16 the same with bf16 output
  wrapper - C5: MHCResidualWrapper, residual/branch bf16 [65536, 4, 7168]
  wrapper8 - the wrapper at n = 8 on [16384, 4, 7168] (run-time-n kernels),
            with the unfused path timed beside it (not a BASELINE config)
  ops     - C2: standalone sinkhorn_knopp / rmsnorm / stream_aggregate fwd+bwd
            (value = the step's achieved HBM GB/s)
--paper-configs runs the reference's 9-configuration sweep (benchmark.py:
299-311) instead, static and dynamic H, and prints per-configuration ms.
Inputs are synthetic (seeded N(0,1)) and already resident in HBM; each step
uses the next of several rotating input sets (together well above the
256 MB MALL) so no step reads the previous step's data from cache.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E, AMD public spec
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "mHC layer fwd+bwd tokens/sec + achieved HBM GB/s (n=4, C=4096)"


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


def _timed_cpu(run, seconds):
    """Median wall time of `run` over ~`seconds` (at least 3 runs, 1 warmup)."""
    run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------

class StaticWorkload:
    """C3: static-H MHCLayer fwd+bwd, x fp32 [8192, 4, 4096]."""

    name = "static"
    B, n, C = 8192, 4, 4096
    dtype = "f32"
    sets = 3

    def __init__(self, torch, mhc, device):
        self.torch = torch
        B, n, C = self.B, self.n, self.C
        g = torch.Generator(device=device).manual_seed(0)
        self.xs = [torch.randn(B, n, C, device=device, generator=g).requires_grad_(True) for _ in range(self.sets)]
        self.gs = [torch.randn(B, n, C, device=device, generator=g) for _ in range(self.sets)]
        torch.manual_seed(0)
        self.layer = mhc.MHCLayer(C, n, use_dynamic_h=False).to(device)
        with torch.no_grad():
            self.layer.H_pre.normal_()
            self.layer.H_post.normal_()
            self.layer.H_res.normal_()
        self.params = list(self.layer.parameters())
        self.i = 0

    def step(self):
        x = self.xs[self.i % self.sets]
        g = self.gs[self.i % self.sets]
        self.i += 1
        out = self.layer(x)
        return self.torch.autograd.grad(out, [x] + self.params, g)

    @property
    def tokens(self):
        return self.B

    @property
    def E(self):
        return self.B * self.n * self.C

    def step_bytes(self):
        # fwd: read x (4E) + write out (4E); bwd: read g (4E) + x (4E) + write dx (4E)
        return 20 * self.E

    def kernel_bytes(self):
        E = self.E
        return {"layer_fwd": 8 * E, "layer_bwd": 12 * E}

    def flops(self):
        return {}

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

        med, runs = _timed_cpu(run, seconds)
        return sample / med, (f"oracle.reference.mhc_layer_static fp32 fwd+bwd (autograd) on {sample} of "
                              f"{self.B} tokens, n={self.n}, C={self.C}; median of {runs} runs")


class DynamicWorkload:
    """C4: dynamic-H MHCLayer fwd+bwd, x bf16 [8192, 4, 4096], phi fp32
    0.02 N(0,1) [16384, 24] split into pre / post / res, alpha 0.01, b 0."""

    name = "dynamic"
    B, n, C = 8192, 4, 4096
    dtype = "f32"
    sets = 3

    def __init__(self, torch, mhc, device):
        self.torch = torch
        B, n, C = self.B, self.n, self.C
        nC = n * C
        g = torch.Generator(device=device).manual_seed(0)
        self.xs = [torch.randn(B, n, C, device=device, generator=g).bfloat16().requires_grad_(True)
                   for _ in range(self.sets)]
        self.gs = [torch.randn(B, n, C, device=device, generator=g) for _ in range(self.sets)]
        torch.manual_seed(0)
        self.layer = mhc.MHCLayer(C, n, use_dynamic_h=True).to(device)
        phi = 0.02 * torch.randn(nC, 2 * n + n * n, device=device, generator=g)
        with torch.no_grad():
            self.layer.phi_pre.copy_(phi[:, :n].t())
            self.layer.phi_post.copy_(phi[:, n:2 * n].t())
            self.layer.phi_res.copy_(phi[:, 2 * n:].t())
        self.params = list(self.layer.parameters())
        self.i = 0

    def step(self):
        x = self.xs[self.i % self.sets]
        g = self.gs[self.i % self.sets]
        self.i += 1
        out = self.layer(x)
        return self.torch.autograd.grad(out, [x] + self.params, g)

    @property
    def tokens(self):
        return self.B

    @property
    def E(self):
        return self.B * self.n * self.C

    def phi_bytes(self):
        return (2 * self.n + self.n * self.n) * self.n * self.C * 4

    def step_bytes(self):
        # fwd: read x bf16 (2E) + write out fp32 (4E); bwd: read g fp32 (4E) +
        # x (2E) + write dx bf16 (2E); Phi read in fwd and bwd, dPhi written
        return 14 * self.E + 3 * self.phi_bytes()

    def kernel_bytes(self):
        E = self.E
        # proj: x bf16 + Phi as three bf16 planes; layer_fwd: x + fp32 out;
        # layer_bwd_reduce: g fp32 + x, writes the stream part of dx (bf16);
        # proj_bwd: x + dx read, dx written, Phi read
        return {"proj": 2 * E + self.phi_bytes() * 3 // 2, "layer_fwd": 6 * E, "layer_bwd_reduce": 8 * E,
                "proj_bwd": 6 * E + self.phi_bytes()}

    def flops(self):
        # projection x_flat [B, nC] . Phi^T [nC, 2n+n^2]; its backward forms
        # dx_flat = dP . Phi and dPhi = dP^T . x_flat (twice the forward)
        f = 2 * self.B * self.n * self.C * (2 * self.n + self.n * self.n)
        return {"proj": f, "proj_bwd": 2 * f}

    def projection_ab(self, lib, reps):
        """A/B of the projection's arithmetic at this workload's shape (inside
        the timed build): the library's bf16-MFMA projection
        (fused_rmsnorm_matmul_fwd, kernel "proj") against the benchmark
        build's fp32-VALU one (kernel "proj_valu"), on x of the first input set
        and Phi = [phi_pre; phi_post; phi_res]; both checked against float64
        on 64 tokens."""
        torch = self.torch
        B, K, npr = self.B, self.n * self.C, 2 * self.n + self.n * self.n
        x = self.xs[0].detach().reshape(B, K)
        phi = torch.cat([self.layer.phi_pre, self.layer.phi_post, self.layer.phi_res]).detach().float().contiguous()
        stream = lib.stream_of(x)
        runs = {}
        for kind, fn in (("mfma", "mhc_fused_rmsnorm_matmul_fwd"), ("valu", "mhc_timing_proj_valu")):
            ws = torch.empty(getattr(lib.load(), fn + "_workspace_size")(B, K, npr), dtype=torch.uint8, device=x.device)
            out = torch.empty(B, npr, device=x.device)
            args = (x.data_ptr(), lib.BF16, phi.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), B, K, npr, stream)
            runs[kind] = (fn, args, out, ws)
        for fn, args, _, _ in runs.values():  # first launches load the code objects
            lib.call(fn, *args)
        torch.cuda.synchronize()
        lib.timing_reset()
        lib.timing_enable(True)
        for _ in range(reps):
            for fn, args, _, _ in runs.values():
                lib.call(fn, *args)
        torch.cuda.synchronize()
        lib.timing_enable(False)
        mfma_ms, mfma_n = lib.timing_query("proj")
        valu_ms, valu_n = lib.timing_query("proj_valu")
        ref = x[:64].double().cpu() @ phi.double().cpu().t()
        scale = ref.abs().max().item()
        err = {k: (runs[k][2][:64].double().cpu() - ref).abs().max().item() / scale for k in runs}
        flops = 2 * B * K * npr
        mfma_avg, valu_avg = mfma_ms / max(mfma_n, 1), valu_ms / max(valu_n, 1)
        return {"shape": {"tokens": B, "k": K, "outputs": npr, "x_dtype": "bf16"},
                "mfma": {"kernel": "proj_mfma_kernel (bf16 MFMA 16x16x32 on hi/mid/lo Phi planes)",
                         "avg_ms": mfma_avg, "launches": mfma_n, "tflops": flops / (mfma_avg / 1e3) / 1e12,
                         "gbps": 2 * B * K / (mfma_avg / 1e3) / 1e9, "max_rel_err_vs_fp64": err["mfma"]},
                "valu": {"kernel": "proj_valu_kernel (fp32 FMA, one token per lane, Phi rows by scalar loads)",
                         "avg_ms": valu_avg, "launches": valu_n, "tflops": flops / (valu_avg / 1e3) / 1e12,
                         "gbps": 2 * B * K / (valu_avg / 1e3) / 1e9, "max_rel_err_vs_fp64": err["valu"]},
                "valu_over_mfma": valu_avg / mfma_avg,
                # np + 1 FMAs per element of x (the products and x^2) at the
                # fp32 FMA issue rate without packed-FP32 forms: MI355X's
                # published 157.3 TFLOP/s vector fp32 counts 2 FMAs per lane
                # per cycle, so one FMA per lane per cycle is 39.3 T FMA/s
                "valu_fma_issue_floor_ms": B * K * (npr + 1) / 39.3e12 * 1e3,
                "timing": "HIP events around each kernel on its stream (timed build), after the workload's passes"}

    def config(self):
        return {"workload": "C4 MHCLayer dynamic-H fwd+bwd", "tokens": self.B, "n": self.n, "C": self.C,
                "x_dtype": "bf16", "phi": [self.n * self.C, 2 * self.n + self.n * self.n], "sinkhorn_iters": 20}

    def cpu_baseline(self, torch, R, seconds):
        sample = 128
        d = R.dynamic_layer_inputs(sample, self.n, self.C, seed=1)
        x = d["x"].requires_grad_(True)
        names = ("weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre",
                 "b_post", "b_res")
        ps = [d[k].float().requires_grad_(True) for k in names]

        def run():
            out = R.mhc_layer_dynamic(x, *ps, 20, 1e-8, 1e-5, dtype=torch.float32)
            torch.autograd.grad(out, [x] + ps, d["grad"])

        med, runs = _timed_cpu(run, seconds)
        return sample / med, (f"oracle.reference.mhc_layer_dynamic fp32 fwd+bwd (autograd) on {sample} of "
                              f"{self.B} tokens, n={self.n}, C={self.C}; median of {runs} runs")


class InferWorkload(DynamicWorkload):
    """C4 shape, forward only: the dynamic-H MHCLayer in eval mode under
    no_grad (the inference path of ops.py:337-380), its weight and
    projections packed once (MHCLayer.prepare_inference), output fp32 as the
    reference (workload infer) or bf16 (workload infer_bf16)."""

    name = "infer"
    metric = "mHC dynamic-H layer forward-only (inference) tokens/sec (C4 shape, n=4, C=4096)"
    out_dtype = "f32"

    def __init__(self, torch, mhc, device):
        super().__init__(torch, mhc, device)
        self.xs = [x.detach() for x in self.xs]
        self.gs = []
        self.layer.eval()
        self.odt = torch.bfloat16 if self.out_dtype == "bf16" else torch.float32
        self.mhc = mhc
        self.layer.prepare_inference()

    def step(self):
        x = self.xs[self.i % self.sets]
        self.i += 1
        L = self.layer
        with self.torch.no_grad():
            return self.mhc.mhc_layer_fused_dynamic_inference(
                x, L.rmsnorm_weight, L.phi_pre, L.phi_post, L.phi_res, L.alpha_pre, L.alpha_post, L.alpha_res,
                L.b_pre, L.b_post, L.b_res, L.num_sinkhorn_iters, L.sinkhorn_eps, L.rmsnorm_eps,
                out_dtype=self.odt, packed=L._packed())

    def out_bytes(self):
        return (2 if self.out_dtype == "bf16" else 4) * self.E

    def step_bytes(self):
        # read x bf16 (2E), write out (4E fp32 / 2E bf16), Phi planes read once
        return 2 * self.E + self.out_bytes() + self.phi_bytes() * 3 // 2

    def kernel_bytes(self):
        return {"proj": 2 * self.E + self.phi_bytes() * 3 // 2, "layer_fwd": 2 * self.E + self.out_bytes()}

    def config(self):
        return {"workload": "C4 MHCLayer dynamic-H forward-only (eval, no_grad)", "tokens": self.B, "n": self.n,
                "C": self.C, "x_dtype": "bf16", "out_dtype": self.out_dtype,
                "phi": [self.n * self.C, 2 * self.n + self.n * self.n], "sinkhorn_iters": 20}

    def cpu_baseline(self, torch, R, seconds):
        sample = 256
        d = R.dynamic_layer_inputs(sample, self.n, self.C, seed=1)
        names = ("weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre",
                 "b_post", "b_res")
        ps = [d[k].float() for k in names]

        def run():
            with torch.no_grad():
                R.mhc_layer_dynamic(d["x"], *ps, 20, 1e-8, 1e-5, dtype=torch.float32)

        med, runs = _timed_cpu(run, seconds)
        return sample / med, (f"oracle.reference.mhc_layer_dynamic fp32 forward (no_grad) on {sample} of "
                              f"{self.B} tokens, n={self.n}, C={self.C}; median of {runs} runs")


class InferBF16Workload(InferWorkload):
    """The forward-only C4 workload with its output written in bf16."""

    name = "infer_bf16"
    metric = "mHC dynamic-H layer forward-only (inference, bf16 output) tokens/sec (C4 shape, n=4, C=4096)"
    out_dtype = "bf16"


class WrapperWorkload:
    """C5: MHCResidualWrapper (dynamic H, 'decay') fwd+bwd at DeepSeek-V3
    width: residual, branch bf16 [65536, 4, 7168] (262,144 tokens)."""

    name = "wrapper"
    Bo, T, n, C = 65536, 4, 4, 7168
    dtype = "f32"
    sets = 2

    def __init__(self, torch, mhc, device):
        self.torch = torch
        self.mhc = mhc
        Bo, T, n, C = self.Bo, self.T, self.n, self.C
        nC = n * C
        g = torch.Generator(device=device).manual_seed(0)
        self.rs = [torch.randn(Bo, T, C, device=device, generator=g).bfloat16().requires_grad_(True)
                   for _ in range(self.sets)]
        self.bs = [torch.randn(Bo, T, C, device=device, generator=g).bfloat16().requires_grad_(True)
                   for _ in range(self.sets)]
        self.gs = [torch.randn(Bo, T, C, device=device, generator=g) for _ in range(self.sets)]
        torch.manual_seed(0)
        self.wrapper = mhc.MHCResidualWrapper(C, n).to(device)
        layer = self.wrapper.mhc
        phi = 0.02 * torch.randn(nC, 2 * n + n * n, device=device, generator=g)
        with torch.no_grad():
            layer.phi_pre.copy_(phi[:, :n].t())
            layer.phi_post.copy_(phi[:, n:2 * n].t())
            layer.phi_res.copy_(phi[:, 2 * n:].t())
        self.params = list(self.wrapper.parameters())
        self.i = 0

    def step(self):
        k = self.i % self.sets
        self.i += 1
        r, b, g = self.rs[k], self.bs[k], self.gs[k]
        out = self.wrapper(r, b)
        return self.torch.autograd.grad(out, [r, b] + self.params, g)

    @property
    def tokens(self):
        return self.Bo * self.T

    @property
    def F(self):
        return self.tokens * self.C

    def phi_bytes(self):
        return (2 * self.n + self.n * self.n) * self.n * self.C * 4

    def step_bytes(self):
        # fwd: read r, b bf16 (4F) + write fp32 mean (4F); bwd: read g fp32
        # (4F) + r, b (4F) + write dr, db bf16 (4F); Phi twice, dPhi once
        return 20 * self.F + 3 * self.phi_bytes()

    def kernel_bytes(self):
        F = self.F
        # wrap_bwd_reduce reads g fp32 and r, b; wrap_proj_bwd reads them again
        # and writes d r, d b
        return {"wrap_proj": 4 * F, "wrap_fwd": 8 * F, "wrap_bwd_reduce": 8 * F, "wrap_proj_bwd": 12 * F}

    def flops(self):
        f = 2 * self.tokens * self.n * self.C * (2 * self.n + self.n * self.n)
        return {"wrap_proj": f, "wrap_proj_bwd": 2 * f}

    def config(self):
        return {"workload": "C5 MHCResidualWrapper dynamic-H fwd+bwd", "tokens": self.tokens, "batch": self.Bo,
                "seq_len": self.T, "n": self.n, "C": self.C, "x_dtype": "bf16", "residual_mode": "decay",
                "sinkhorn_iters": 20}

    def cpu_baseline(self, torch, R, seconds):
        sample_b, sample_t = 32, 4
        d = R.wrapper_inputs(sample_b, sample_t, self.C, self.n, seed=1)
        r = d["residual"].requires_grad_(True)
        b = d["branch"].requires_grad_(True)
        names = ("weight", "phi_pre", "phi_post", "phi_res", "alpha_pre", "alpha_post", "alpha_res", "b_pre",
                 "b_post", "b_res")
        ps = [d[k].float().requires_grad_(True) for k in names]

        def layer_fn(X):
            return R.mhc_layer_dynamic(X, *ps, 20, 1e-8, 1e-5, dtype=torch.float32)

        def run():
            out = R.mhc_residual_wrapper(r, b, layer_fn, self.n, "decay")
            torch.autograd.grad(out, [r, b] + ps, d["grad"])

        med, runs = _timed_cpu(run, seconds)
        tok = sample_b * sample_t
        return tok / med, (f"oracle.reference.mhc_residual_wrapper over mhc_layer_dynamic fp32 fwd+bwd (autograd) "
                           f"on {tok} of {self.tokens} tokens, n={self.n}, C={self.C}; median of {runs} runs")


class Wrapper8Workload(WrapperWorkload):
    """MHCResidualWrapper at expansion rate 8 (dynamic H, 'decay'), the C5
    width on a quarter of its tokens: residual, branch bf16 [16384, 4, 7168]
    (65,536 tokens).  Runs the run-time-n wrapper kernels; the record also
    times the same step through the unfused path (the streams built with
    device tensor ops, as layer.py:299-310, and the layer run on them), the
    static-H step both ways, and n = 16 and 32 both ways (static H on
    [8192, 4096], dynamic H on [8192, 1024])."""

    name = "wrapper8"
    Bo, T, n, C = 16384, 4, 8, 7168
    metric = "mHC MHCResidualWrapper n=8 dynamic-H fwd+bwd tokens/sec (C5 width, 65,536 tokens)"

    def step_bytes(self):
        # as C5's count (r, b, g and d r, d b once each; Phi twice, dPhi once)
        return 20 * self.F + 3 * self.phi_bytes()

    def kernel_bytes(self):
        F = self.F
        # wrap_fwd reads r, b (bf16) and writes the fp32 mean; the backward's
        # row sums read g and r, b; wrap_proj_bwd (d r, d b with dP . Phi
        # folded in) reads g, r, b and writes d r, d b; proj_bwd_dphi (dPhi of
        # the pre / post rows from the rebuilt streams) reads r, b
        return {"wrap_fwd": 8 * F, "wrap_bwd_reduce": 8 * F, "wrap_proj_bwd": 12 * F, "proj_bwd_dphi": 4 * F}

    def flops(self):
        return {}

    def config(self):
        c = super().config()
        c["workload"] = "MHCResidualWrapper n=8 dynamic-H fwd+bwd (C5 width)"
        return c

    def unfused_ab(self, steps):
        """ms per step of the unfused path on the same inputs and parameters."""
        torch = self.torch
        layer = self.wrapper.mhc

        def step():
            k = self.i % self.sets
            self.i += 1
            r, b, g = self.rs[k], self.bs[k], self.gs[k]
            rr, bb = r.reshape(-1, self.C), b.reshape(-1, self.C)
            X = torch.zeros(rr.shape[0], self.n, self.C, device=rr.device, dtype=rr.dtype)
            X[:, 0] = rr
            X[:, 1] = bb
            for i in range(2, self.n):
                X[:, i] = rr * (0.1 ** (i - 1))
            out = layer(X).mean(dim=1).view(r.shape)
            return torch.autograd.grad(out, [r, b] + self.params, g)

        for _ in range(2):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        rec = {"ms_per_step": (time.perf_counter() - t0) * 1e3 / steps, "steps": steps,
               "path": "torch.zeros + slice copies + decay products (layer.py:299-310), MHCLayer on [tokens, 8, C], "
                       "mean over streams; fwd+bwd through autograd"}
        rec["static_h"] = self.static_ab(steps)
        rec["static_wide_n"] = [self.wide_ab(n, steps, False, C=4096) for n in (16, 32)]
        rec["dynamic_wide_n"] = [self.wide_ab(n, steps, True, C=1024) for n in (16, 32)]
        return rec

    def wide_ab(self, n, steps, dynamic, tokens=8192, C=4096):
        """n = 16 / 32 (the run-time-n kernels' 16- and 32-stream capacities)
        on bf16 [tokens, C] residual / branch, 'decay', static or dynamic H:
        the fused wrapper against the tensor-op streams through the layer, ms
        per fwd+bwd step, inputs and parameters shared by both paths."""
        torch, mhc = self.torch, self.mhc
        dev = self.rs[0].device
        g = torch.Generator(device=dev).manual_seed(n)
        rs = [torch.randn(tokens, C, device=dev, generator=g).bfloat16().requires_grad_(True) for _ in range(2)]
        bs = [torch.randn(tokens, C, device=dev, generator=g).bfloat16().requires_grad_(True) for _ in range(2)]
        gs = [torch.randn(tokens, C, device=dev, generator=g) for _ in range(2)]
        torch.manual_seed(n)
        wrap = mhc.MHCResidualWrapper(C, n, use_dynamic_h=dynamic).to(dev)
        layer = wrap.mhc
        params = list(wrap.parameters())

        def fused(k):
            return torch.autograd.grad(wrap(rs[k], bs[k]), [rs[k], bs[k]] + params, gs[k])

        def unfused(k):
            r, b = rs[k], bs[k]
            X = torch.zeros(tokens, n, C, device=dev, dtype=r.dtype)
            X[:, 0] = r
            X[:, 1] = b
            for i in range(2, n):
                X[:, i] = r * (0.1 ** (i - 1))
            return torch.autograd.grad(layer(X).mean(dim=1), [r, b] + params, gs[k])

        res = {"n": n, "tokens": tokens, "hidden": C, "dynamic_h": dynamic}
        for name, fn in (("fused_ms_per_step", fused), ("unfused_ms_per_step", unfused)):
            for i in range(2):
                fn(i % 2)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(steps):
                fn(i % 2)
            torch.cuda.synchronize()
            res[name] = (time.perf_counter() - t0) * 1e3 / steps
        del rs, bs, gs, wrap
        torch.cuda.empty_cache()
        return res

    def static_ab(self, steps):
        """The same A/B with static H (use_dynamic_h=False): the fused
        run-time-n wrapper against the tensor-op streams through the layer,
        ms per fwd+bwd step on the same inputs."""
        torch, mhc = self.torch, self.mhc
        torch.manual_seed(0)
        wrap = mhc.MHCResidualWrapper(self.C, self.n, use_dynamic_h=False).to(self.rs[0].device)
        layer = wrap.mhc
        params = list(wrap.parameters())

        def fused(k):
            out = wrap(self.rs[k], self.bs[k])
            return torch.autograd.grad(out, [self.rs[k], self.bs[k]] + params, self.gs[k])

        def unfused(k):
            r, b = self.rs[k].reshape(-1, self.C), self.bs[k].reshape(-1, self.C)
            X = torch.zeros(r.shape[0], self.n, self.C, device=r.device, dtype=r.dtype)
            X[:, 0] = r
            X[:, 1] = b
            for i in range(2, self.n):
                X[:, i] = r * (0.1 ** (i - 1))
            out = layer(X).mean(dim=1).view(self.rs[k].shape)
            return torch.autograd.grad(out, [self.rs[k], self.bs[k]] + params, self.gs[k])

        res = {}
        for name, fn in (("fused_ms_per_step", fused), ("unfused_ms_per_step", unfused)):
            for i in range(2):
                fn(i % self.sets)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(steps):
                fn(i % self.sets)
            torch.cuda.synchronize()
            res[name] = (time.perf_counter() - t0) * 1e3 / steps
        return res


class OpsWorkload:
    """C2: the standalone operators, fp32, forward + backward through autograd:
    sinkhorn_knopp [65536, 4, 4] ~U(0,1) (20 iterations, eps 1e-8), rmsnorm
    [16384, 4096] with weight ~N(1, 0.1) (eps 1e-5), stream_aggregate
    [16384, 4, 4096] with H_pre ~N(0,1) [16384, 4].  The reported value is the
    step's achieved HBM GB/s over the algorithmic bytes of all six kernels."""

    name = "ops"
    S, R, n, C = 65536, 16384, 4, 4096
    dtype = "f32"
    sets = 2
    metric = "mHC standalone ops (sinkhorn, rmsnorm, stream_aggregate) fwd+bwd achieved HBM GB/s (C2)"
    unit = "GB/s"

    def __init__(self, torch, mhc, device):
        self.torch, self.mhc = torch, mhc
        S, R, n, C = self.S, self.R, self.n, self.C
        g = torch.Generator(device=device).manual_seed(0)
        rnd = lambda *shape: torch.randn(*shape, device=device, generator=g)
        self.sk = [torch.rand(S, n, n, device=device, generator=g).requires_grad_(True) for _ in range(self.sets)]
        self.gsk = [rnd(S, n, n) for _ in range(self.sets)]
        self.rx = [rnd(R, C).requires_grad_(True) for _ in range(self.sets)]
        self.rw = (1.0 + 0.1 * rnd(C)).requires_grad_(True)
        self.gr = [rnd(R, C) for _ in range(self.sets)]
        self.ax = [rnd(R, n, C).requires_grad_(True) for _ in range(self.sets)]
        self.ah = [rnd(R, n).requires_grad_(True) for _ in range(self.sets)]
        self.ga = [rnd(R, C) for _ in range(self.sets)]
        self.i = 0

    def step(self):
        k = self.i % self.sets
        self.i += 1
        ag = self.torch.autograd.grad
        m = self.mhc
        o1 = m.sinkhorn_knopp(self.sk[k], 20, 1e-8)
        r1 = ag(o1, [self.sk[k]], self.gsk[k])
        o2 = m.rmsnorm(self.rx[k], self.rw, 1e-5)
        r2 = ag(o2, [self.rx[k], self.rw], self.gr[k])
        o3 = m.stream_aggregate(self.ax[k], self.ah[k])
        r3 = ag(o3, [self.ax[k], self.ah[k]], self.ga[k])
        return r1, r2, r3

    @property
    def tokens(self):
        return self.R

    def kernel_bytes(self):
        S, R, n, C = self.S, self.R, self.n, self.C
        sk = S * n * n * 4
        row = R * C * 4
        return {
            "sinkhorn_fwd": 2 * sk,                               # read inp, write out
            "sinkhorn_bwd": 3 * sk,                               # read grad, inp; write grad_inp
            "rmsnorm_fwd": 2 * row + C * 4 + R * 4,               # read x, w; write y, rms
            "rmsnorm_bwd": 3 * row + C * 4 + R * 4 + C * 4,       # read g, x, w, rms; write dx, dw
            "aggregate_fwd": n * row + row + R * n * 4 * 2,       # read x, H; write out, H_act
            "aggregate_bwd": row + 2 * n * row + R * n * 4 * 2,   # read g, x, H_act; write dx, dH
        }

    def step_bytes(self):
        return sum(self.kernel_bytes().values())

    def flops(self):
        return {}

    def config(self):
        return {"workload": "C2 standalone ops fwd+bwd", "sinkhorn": [self.S, self.n, self.n], "sinkhorn_iters": 20,
                "rmsnorm": [self.R, self.C], "stream_aggregate": [self.R, self.n, self.C], "x_dtype": "f32"}

    def cpu_baseline(self, torch, R, seconds):
        """The oracle's three ops fwd+bwd (autograd) on a row sample; returns
        the achieved GB/s of the same algorithmic bytes, scaled to the sample."""
        rows, mats = 256, 1024
        g = torch.Generator().manual_seed(1)
        sk = torch.rand(mats, self.n, self.n, generator=g).requires_grad_(True)
        x = torch.randn(rows, self.C, generator=g).requires_grad_(True)
        w = (1.0 + 0.1 * torch.randn(self.C, generator=g)).requires_grad_(True)
        ax = torch.randn(rows, self.n, self.C, generator=g).requires_grad_(True)
        ah = torch.randn(rows, self.n, generator=g).requires_grad_(True)

        def run():
            R.sinkhorn_knopp(sk, 20, 1e-8).sum().backward()
            R.rmsnorm(x, w, 1e-5)[0].sum().backward()
            R.stream_aggregate(ax, ah)[0].sum().backward()

        med, runs = _timed_cpu(run, seconds)
        kb = self.kernel_bytes()
        sample_bytes = (kb["sinkhorn_fwd"] + kb["sinkhorn_bwd"]) * mats / self.S + \
            (kb["rmsnorm_fwd"] + kb["rmsnorm_bwd"] + kb["aggregate_fwd"] + kb["aggregate_bwd"]) * rows / self.R
        return sample_bytes / med / 1e9, (f"oracle.reference sinkhorn_knopp ({mats} matrices), rmsnorm and "
                                          f"stream_aggregate ({rows} rows) fp32 fwd+bwd (autograd); GB/s of the "
                                          f"same algorithmic bytes scaled to the sample; median of {runs} runs")


WORKLOADS = {"static": StaticWorkload, "dynamic": DynamicWorkload, "infer": InferWorkload,
             "infer_bf16": InferBF16Workload, "wrapper": WrapperWorkload, "wrapper8": Wrapper8Workload,
             "ops": OpsWorkload}
KERNELS = ("layer_fwd", "layer_bwd", "layer_bwd_reduce", "proj", "proj_bwd", "proj_bwd_dphi", "wrap_proj",
           "wrap_synth", "wrap_fwd", "wrap_bwd", "wrap_bwd_reduce", "wrap_proj_bwd", "sinkhorn_fwd", "sinkhorn_bwd",
           "rmsnorm_fwd", "rmsnorm_bwd", "aggregate_fwd", "aggregate_bwd")


# ---------------------------------------------------------------------------
# The reference's configuration sweep (benchmark.py:299-311, protocol of
# benchmark.py:175-269): per (B, C, n), static and dynamic H, the forward in
# eval mode under no_grad and forward + backward of out.sum() in train mode,
# fp32 x drawn fresh per run, caches flushed before each run, events around
# the call, 10% trimmed mean.  A third column replays the same forward +
# backward library calls from a HIP graph (no host overhead).
# ---------------------------------------------------------------------------
PAPER_CONFIGS = [(320, 1280, 4), (512, 1920, 4), (1280, 2560, 4), (2560, 1280, 4), (128, 1280, 8), (256, 1280, 8),
                 (32, 1280, 32), (64, 1280, 32), (128, 1280, 32)]


def paper_sweep(torch, mhc, device, warmup=10, runs=100, only=None):
    flush = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=device)

    def timed(fn, B, n, C, train):
        times = []
        for it in range(warmup + runs):
            x = torch.randn(B, n, C, device=device, requires_grad=train)
            flush.zero_()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            fn(x)
            t1.record()
            torch.cuda.synchronize()
            if it >= warmup:
                times.append(t0.elapsed_time(t1))
        times.sort()
        trim = runs // 10
        times = times[trim:len(times) - trim] if trim else times
        return sum(times) / len(times)

    from mhc_ascend_amd import native

    def graph_ms(layer, B, n, C, dynamic):
        """The same fwd + bwd through the library entries, captured once in a
        HIP graph and replayed: the kernels' time without host overhead."""
        x = torch.randn(B, n, C, device=device)
        g = torch.ones(B, n, C, device=device)
        L = layer
        if dynamic:
            ps = [L.rmsnorm_weight, L.phi_pre, L.phi_post, L.phi_res, L.alpha_pre, L.alpha_post, L.alpha_res,
                  L.b_pre, L.b_post, L.b_res]
            ps = [p.detach() for p in ps]

            def step():
                out, saved = native.mhc_layer_dynamic_fwd(x, *ps, 20, 1e-8, 1e-5)
                native.mhc_layer_dynamic_bwd(g, x, ps[0], saved, *ps[1:], 20, 1e-8, 1e-5)
        else:
            ps = [p.detach() for p in (L.rmsnorm_weight, L.H_pre, L.H_post, L.H_res)]

            def step():
                out, rms, saved = native.mhc_layer_static_fwd(x, *ps, 20, 1e-8, 1e-5)
                native.mhc_layer_static_bwd(g, x, *ps, saved, 20, 1e-8, 1e-5)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        times = []
        for it in range(warmup + runs):
            flush.zero_()
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            graph.replay()
            t1.record()
            torch.cuda.synchronize()
            if it >= warmup:
                times.append(t0.elapsed_time(t1))
        times.sort()
        trim = runs // 10
        times = times[trim:len(times) - trim] if trim else times
        return sum(times) / len(times)

    rows = []
    for dynamic in (False, True):
        for B, C, n in PAPER_CONFIGS:
            if only and (B, C, n) not in only:
                continue
            torch.manual_seed(0)
            layer = mhc.MHCLayer(C, n, use_dynamic_h=dynamic).to(device)

            def fwd(x):
                with torch.no_grad():
                    layer(x)

            def fwd_bwd(x):
                layer(x).sum().backward()

            layer.eval()
            f_ms = timed(fwd, B, n, C, False)
            layer.train()
            fb_ms = timed(fwd_bwd, B, n, C, True)
            gr_ms = graph_ms(layer, B, n, C, dynamic)
            rows.append({"dynamic_h": dynamic, "B": B, "C": C, "n": n, "fwd_ms": f_ms, "fwd_bwd_ms": fb_ms,
                         "graph_fwd_bwd_ms": gr_ms})
            print(f"[bench] paper {'dynamic' if dynamic else 'static '} B={B:5d} C={C:5d} n={n:3d} "
                  f"fwd {f_ms:8.4f} ms  fwd+bwd {fb_ms:8.4f} ms  graph fwd+bwd {gr_ms:8.4f} ms",
                  file=sys.stderr, flush=True)
            del layer
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 50; 10 for wrapper)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="static")
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bounded CPU-baseline sample time (0 disables)")
    ap.add_argument("--paper-configs", action="store_true",
                    help="instead of a workload: the reference's 9-configuration sweep (benchmark.py:299-311), "
                         "static and dynamic H, forward and forward+backward ms per configuration")
    ap.add_argument("--paper-filter", action="append", default=[], metavar="B,C,n",
                    help="with --paper-configs: run only these configurations (repeatable)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a plain 1 GiB device copy (known bytes) for PMC counter calibration")
    ap.add_argument("--protocol-runs", type=int, default=100,
                    help="runs of the reference's timing protocol (median, 10%% trimmed mean)")
    ap.add_argument("--kernel-steps", type=int, default=10, help="steps of the per-kernel timing pass")
    ap.add_argument("--extra", action="append", default=None, choices=sorted(WORKLOADS),
                    help="with the default static workload: also measure these workloads as sub-records "
                         "(default: dynamic, the reference layer's default path; wrapper; ops; infer; wrapper8)")
    ap.add_argument("--no-extra", action="store_true", help="no sub-records")
    ap.add_argument("--extra-steps", type=int, default=50,
                    help="timed steps of each sub-record (enough that the first launch and the final drain, "
                         "timed once per run, do not inflate the per-step figure)")
    a = ap.parse_args(argv)

    if a.gpus != 1:
        _die(f"bench.py: this build runs on ONE GPU; --gpus {a.gpus} is not supported (the layer shards over "
             "tokens with one all-reduce of the parameter gradients; see DESIGN.md).")
    steps = a.steps if a.steps is not None else (10 if a.workload == "wrapper" else 50)
    if a.no_extra:
        a.extra = []
    elif a.extra is None:
        a.extra = ["dynamic", "wrapper", "ops", "infer", "wrapper8"]

    import torch

    if not torch.cuda.is_available():
        _die("bench.py: no HIP device visible")
    sys.path.insert(0, ROOT)
    import mhc_ascend_amd as mhc
    from mhc_ascend_amd import _lib

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if a.paper_configs:
        only = None
        if a.paper_filter:
            only = set()
            for f in a.paper_filter:
                cfg = tuple(int(v) for v in f.split(","))
                if cfg not in PAPER_CONFIGS:
                    _die(f"bench.py: --paper-filter {f} is not one of the configurations {PAPER_CONFIGS}")
                only.add(cfg)
        rows = paper_sweep(torch, mhc, device, only=only)
        geo = 1.0
        for r in rows:
            geo *= r["fwd_bwd_ms"]
        geo **= 1.0 / len(rows)
        print(json.dumps({"metric": "mHC layer ms per paper configuration (benchmark.py:301-311 protocol)",
                          "value": geo, "unit": "ms (geometric mean of fwd+bwd over the 18 rows)", "n_gpus": 1,
                          "higher_is_better": False, "vs_baseline": None, "dtype": "f32",
                          "data": "synthetic N(0,1) fp32 x, fresh per run; 512 MB cache flush before each run",
                          "config": {"workload": "paper configuration sweep", "warmup": 10, "runs": 100,
                                     "trimmed": "10% each end"},
                          "rows": rows}), flush=True)
        return 0
    rec = measure_workload(a.workload, torch, mhc, _lib, device, steps, a.warmup, a.protocol_runs, a.kernel_steps,
                           a.cpu_seconds, a.copy_calib)
    if a.workload == "static" and a.extra:
        # the reference layer's default path (use_dynamic_h=True, layer.py:48)
        # at the same n and C, and the other BASELINE configurations,
        # measured the same way
        sub = {}
        for name in a.extra:
            sub[name] = measure_workload(name, torch, mhc, _lib, device, a.extra_steps, a.warmup, a.protocol_runs,
                                         a.kernel_steps, a.cpu_seconds, False)
        rec["workloads"] = sub
    print(json.dumps(rec), flush=True)
    return 0


def measure_workload(name, torch, mhc, _lib, device, steps, warmup, protocol_runs, kernel_steps, cpu_seconds,
                     copy_calib):
    """One workload: W warmup steps; K timed steps (host clock, synchronised
    on both sides, no per-kernel events); the reference's protocol
    (benchmark.py:175-269: >= 100 runs, median and 10% trimmed mean) from
    HIP events recorded between consecutive steps; then a separate pass with
    the library's per-kernel event timing for the kernel table and the
    roofline; then the CPU baseline."""
    wl = WORKLOADS[name](torch, mhc, device)
    print(f"[bench] workload={wl.name} warmup={warmup} steps={steps}", file=sys.stderr, flush=True)
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()

    if copy_calib:
        src = torch.empty(1 << 28, dtype=torch.float32, device=device).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # the timed region: K steps, nothing else on the GPU
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        wl.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    print(f"[bench] timed {steps} steps in {t1 - t0:.4f} s", file=sys.stderr, flush=True)
    ms_per_step = (t1 - t0) * 1e3 / steps
    tokens_per_s = wl.tokens / (ms_per_step / 1e3)
    step_gbps = wl.step_bytes() / (ms_per_step / 1e3) / 1e9

    # the reference's protocol: per-step durations between consecutive events
    runs = max(protocol_runs, 1)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(runs + 1)]
    evs[0].record()
    for r in range(runs):
        wl.step()
        evs[r + 1].record()
    torch.cuda.synchronize()
    per = sorted(evs[r].elapsed_time(evs[r + 1]) for r in range(runs))
    trim = runs // 10
    kept = per[trim:runs - trim] if trim else per
    protocol = {"runs": runs, "median_ms": statistics.median(per), "trimmed_mean_ms": sum(kept) / len(kept),
                "mean_ms": sum(per) / runs, "min_ms": per[0], "max_ms": per[-1],
                "method": "HIP events between consecutive steps (no host synchronisation inside the loop); "
                          "10% trimmed each end as benchmark.py:208-215"}

    # per-kernel pass, after the timed region, on the library's benchmark
    # build (same sources plus HIP events around each kernel on its stream)
    timings = {}
    with _lib.timed_build():
        for _ in range(max(warmup, 2)):  # the timed build's code objects load on first use
            wl.step()
        torch.cuda.synchronize()
        _lib.timing_reset()
        _lib.timing_enable(True)
        for _ in range(kernel_steps):
            wl.step()
        torch.cuda.synchronize()
        _lib.timing_enable(False)
        for kname in KERNELS:
            timings[kname] = _lib.timing_query(kname)
        proj_ab = wl.projection_ab(_lib, kernel_steps) if wl.name == "dynamic" else None
    unfused = wl.unfused_ab(steps) if hasattr(wl, "unfused_ab") else None
    kbytes = wl.kernel_bytes()
    kflops = wl.flops()
    kernels = {}
    for kname in KERNELS:
        ms, cnt = timings[kname]
        if cnt == 0:
            continue
        avg = ms / cnt
        krec = {"avg_ms": avg, "launches": cnt, "share_of_step": avg * cnt / (ms_per_step * kernel_steps)}
        if kname in kbytes:
            krec["algorithmic_bytes"] = kbytes[kname]
            krec["gbps"] = kbytes[kname] / (avg / 1e3) / 1e9
        if kname in kflops:
            krec["tflops"] = kflops[kname] / (avg / 1e3) / 1e12
            krec["mfma_util_bf16_dense"] = krec["tflops"] / PEAK_BF16_TFLOPS
        kernels[kname] = krec
    # dominant kernel = the largest share of the step among those with known bytes
    dom = max((k for k in kernels if "gbps" in kernels[k]), key=lambda k: kernels[k]["share_of_step"], default=None)
    roof = None
    if dom is not None:
        traffic, traffic_src = measured_traffic(dom, wl.name)
        roof = {"kernel": dom, "bound": "hbm", "achieved": kernels[dom]["gbps"], "peak": PEAK_HBM_GBPS,
                "unit": "GB/s", "frac": kernels[dom]["gbps"] / PEAK_HBM_GBPS, "traffic": traffic,
                "traffic_source": traffic_src, "avg_launch_ms": kernels[dom]["avg_ms"],
                "launches": kernels[dom]["launches"], "algorithmic_bytes": kbytes[dom],
                "timing": f"HIP events around each launch on its stream (the library's timed build, "
                          f"libmhc_hip_timed.so), {kernel_steps} steps after the timed region"}

    cpu = None
    if cpu_seconds > 0:
        from oracle import reference as R
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        print(f"[bench] CPU baseline on {cores} cores for ~{cpu_seconds:.0f} s", file=sys.stderr, flush=True)
        v, sample = wl.cpu_baseline(torch, R, cpu_seconds)
        cpu = {"value": v, "unit": getattr(wl, "unit", "tokens/s"), "cores": torch.get_num_threads(), "kind": "port",
               "sample": sample}

    ops = getattr(wl, "unit", "tokens/s") == "GB/s"
    rec = {
        "metric": getattr(wl, "metric", METRIC),
        "value": step_gbps if ops else tokens_per_s,
        "unit": getattr(wl, "unit", "tokens/s"),
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": f"synthetic N(0,1), seeded, resident in HBM ({wl.sets} rotating input sets)",
        "config": wl.config(),
        "hbm_gbps": step_gbps,
        "hbm_frac": step_gbps / PEAK_HBM_GBPS,
        "step_algorithmic_bytes": wl.step_bytes(),
        "protocol": protocol,
        "roofline": roof,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    if proj_ab is not None:
        rec["projection_ab"] = proj_ab
    if unfused is not None:
        rec["unfused_ab"] = unfused
    del wl
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return rec


if __name__ == "__main__":
    sys.exit(main())
