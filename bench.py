"""Benchmark: one FLUX.1-dev-shaped 1024^2 denoise step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kinds bf16,fp8] [--no-cpu]
                    [--calibrate-copy]

Workload: the full FLUX transformer forward of one denoise step, batch 1, 4096 image tokens
(64 x 64 patch grid) + 512 text tokens, 19 double + 38 single blocks, hidden 3072, 24 x 128
heads, random-init N(0, 0.02) weights drawn on the device, latents / text / pooled N(0, 1),
guidance 3.5. `value` is the bf16 step time; the fp8 step (every block linear per-channel e4m3
with per-token activations) is reported beside it.

Each step starts with its inputs resident in HBM. W untimed warmup steps, then K steps
bracketed by torch.cuda.synchronize(); per-step times from HIP events on the step stream.

roofline: the dominant kernel is the single-block input GEMM (M 4608, N 7 x 3072, K 3072, GELU on
the MLP columns; 2 M N K = 608.8 GFLOP per launch, 38 launches per step). Its average duration
comes from HIP events recorded around each of its launches inside the timed steps.
attn_gemm: one extra probed step times every GEMM and attention launch; the fraction is the
roofline time of their algorithmic FLOPs at MFMA peak over their summed measured time.
cpu_baseline: the oracle (fp32 torch restatement of the reference's CPU path) on one double and
one single block at the real shape, on this host's cores, extrapolated to 19 + 38 blocks.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

METRIC = ("FLUX 1024² denoise step ms (bf16, fp8) at 1 GPU; attn+GEMM % of MFMA peak")
PEAK = {"bf16": 2.5e15, "fp8": 5.0e15, "mx": 5.0e15}  # dense MFMA, MI355X
HBM_PEAK = 8.0e12
IMG_HW = (64, 64)
TXT = 512
SEED = 0
COPY_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--kinds", default="bf16,fp8")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain 256 MiB bf16 elementwise copy (torch.neg) three "
                         "times, as the known-size reference for HBM byte counters")
    return ap.parse_args()


def flops_per_step(cfg, st, si):
    """Algorithmic FLOPs: GEMMs 2 M N K, attention 4 H S^2 d (QK^T and PV)."""
    d, f, s = cfg.hidden, cfg.mlp, st + si
    dbl = 2 * s * d * 3 * d + 2 * s * d * d + 2 * (2 * s * d * f)
    sgl = 2 * s * d * (3 * d + f) + 2 * s * (d + f) * d
    attn = 4 * cfg.heads * s * s * cfg.head_dim
    gemm = cfg.n_double * dbl + cfg.n_single * sgl
    emb = 2 * si * cfg.in_channels * d + 2 * st * cfg.txt_dim * d + 2 * si * d * cfg.out_channels
    return gemm, attn * (cfg.n_double + cfg.n_single), emb


class Probe:
    """Records HIP event pairs on torch's current stream around named launches."""

    def __init__(self, only=None):
        import torch

        self.torch = torch
        self.only = only
        self.events: dict[str, list] = {}

    def __call__(self, name):
        probe = self

        class _Ctx:
            def __enter__(self_):
                if probe.only is not None and name not in probe.only:
                    self_.pair = None
                    return
                s = probe.torch.cuda.Event(enable_timing=True)
                e = probe.torch.cuda.Event(enable_timing=True)
                s.record()
                self_.pair = (s, e)

            def __exit__(self_, *exc):
                if self_.pair is not None:
                    self_.pair[1].record()
                    probe.events.setdefault(name, []).append(self_.pair)

        return _Ctx()

    def times_ms(self):
        return {k: [s.elapsed_time(e) for s, e in v] for k, v in self.events.items()}


def gemm_flops_by_name(cfg, st, si):
    d, f, s = cfg.hidden, cfg.mlp, st + si
    return {
        "gemm.double.qkv": 2 * s * d * 3 * d,
        "gemm.double.out": 2 * s * d * d,
        "gemm.double.ff1": 2 * s * d * f,
        "gemm.double.ff2": 2 * s * f * d,
        "gemm.single.w1": 2 * s * d * (3 * d + f),
        "gemm.single.w2": 2 * s * (d + f) * d,
        "attn": 4 * cfg.heads * s * s * cfg.head_dim,
    }


def run_kind(kind, steps, warmup, torch, log):
    from difflet_amd.dit.flux import FluxConfig, FluxDiT, random_param_source

    dev = torch.device("cuda", 0)
    cfg = FluxConfig()
    t0 = time.time()
    model = FluxDiT(cfg, random_param_source(cfg, SEED, dev), kind=kind, device=dev)
    torch.cuda.synchronize()
    log(f"[{kind}] model built in {time.time() - t0:.1f} s, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated")
    g = torch.Generator(device=dev).manual_seed(SEED + 1)
    si = IMG_HW[0] * IMG_HW[1]
    latents = torch.randn(1, si, cfg.in_channels, generator=g, device=dev)
    text = torch.randn(1, TXT, cfg.txt_dim, generator=g, device=dev)
    pooled = torch.randn(1, cfg.pooled_dim, generator=g, device=dev)
    t = torch.rand(1, generator=g, device=dev)
    guid = torch.full((1,), 3.5, device=dev)

    def step():
        return model.forward(latents, text, pooled, t, guid, IMG_HW)

    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    if not torch.isfinite(out.float()).all():
        raise RuntimeError(f"[{kind}] non-finite output")
    log(f"[{kind}] warmup done")

    probe = Probe(only={"gemm.single.w1"})
    model.probe = probe
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    for s, e in evs:
        s.record()
        step()
        e.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t_wall) * 1e3 / steps
    model.probe = None
    per_step = sorted(s.elapsed_time(e) for s, e in evs)
    dom = probe.times_ms()["gemm.single.w1"]
    log(f"[{kind}] {steps} steps: mean {sum(per_step) / steps:.2f} ms, wall {wall_ms:.2f} ms")

    # one more step with every GEMM / attention launch probed
    full = Probe()
    model.probe = full
    step()
    torch.cuda.synchronize()
    model.probe = None
    by_name = full.times_ms()
    del model
    torch.cuda.empty_cache()
    return {"per_step": per_step, "wall_ms": wall_ms, "dominant_ms": dom, "by_name": by_name,
            "cfg": cfg, "si": si}


def cpu_baseline(log):
    """The oracle's fp32 CPU path on one double + one single block at the real shape."""
    import torch

    from oracle import flux as oflux
    from oracle import ops

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    shape = oflux.FluxShape()
    g = torch.Generator().manual_seed(SEED)
    si = IMG_HW[0] * IMG_HW[1]
    hidden = torch.randn(1, si, shape.hidden, generator=g)
    context = torch.randn(1, TXT, shape.hidden, generator=g)
    temb = torch.randn(1, shape.hidden, generator=g)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(TXT, *IMG_HW))
    dw = oflux.double_block_weights(shape, SEED, 0)
    sw = oflux.single_block_weights(shape, SEED, 0)
    # warm the thread pool and allocator on a small slice
    oflux.double_block(dw, hidden[:, :64], context[:, :64], temb, cos[: 128], sin[: 128], shape)
    t0 = time.perf_counter()
    oflux.double_block(dw, hidden, context, temb, cos, sin, shape)
    t_d = time.perf_counter() - t0
    x = torch.cat([context, hidden], dim=1)
    t0 = time.perf_counter()
    oflux.single_block(sw, x, temb, cos, sin, shape)
    t_s = time.perf_counter() - t0
    step_ms = (shape.n_double * t_d + shape.n_single * t_s) * 1e3
    log(f"[cpu] double block {t_d:.2f} s, single block {t_s:.2f} s on {threads} threads")
    return {"value": round(step_ms, 1), "unit": "ms/step (extrapolated)", "cores": threads,
            "kind": "port",
            "sample": (f"fp32 oracle, 1 double ({t_d:.2f} s) + 1 single ({t_s:.2f} s) block at "
                       f"{TXT}+{si} tokens, extrapolated x{shape.n_double} + x{shape.n_single}")}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the step's sharding across GPUs is a design in DESIGN.md, not measured)",
              file=sys.stderr)
        return 2
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    log = lambda m: print(m, file=sys.stderr, flush=True)  # noqa: E731
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    from difflet_amd import _lib

    _lib.load()
    kinds = [k for k in args.kinds.split(",") if k]
    if args.calibrate_copy:
        src = torch.randn(COPY_BYTES // 2, device="cuda").bfloat16()
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    res = {k: run_kind(k, args.steps, args.warmup, torch, log) for k in kinds}

    out = {}
    for k, r in res.items():
        cfg, si = r["cfg"], r["si"]
        gemm_f, attn_f, emb_f = flops_per_step(cfg, TXT, si)
        mean_ms = sum(r["per_step"]) / len(r["per_step"])
        fl = gemm_flops_by_name(cfg, TXT, si)
        # attn+GEMM: roofline time of their FLOPs at MFMA peak / their measured kernel time
        t_meas = sum(sum(v) for n, v in r["by_name"].items()) * 1e-3
        t_roof = sum(fl[n] * len(v) / (PEAK["bf16"] if n == "attn" else PEAK[k])
                     for n, v in r["by_name"].items())
        dom = r["dominant_ms"]
        dom_avg = sum(dom) / len(dom)
        dom_flops = fl["gemm.single.w1"]
        achieved = dom_flops / (dom_avg * 1e-3) / 1e12
        per_kernel = {n: {"launches": len(v), "avg_ms": round(sum(v) / len(v), 4),
                          "tflops": round(fl[n] / (sum(v) / len(v) * 1e-3) / 1e12, 1)}
                      for n, v in sorted(r["by_name"].items())}
        out[k] = {
            "ms_per_step": round(mean_ms, 3),
            "median_ms": round(r["per_step"][len(r["per_step"]) // 2], 3),
            "p90_ms": round(r["per_step"][int(0.9 * (len(r["per_step"]) - 1))], 3),
            "wall_ms_per_step": round(r["wall_ms"], 3),
            "tflops_step": round((gemm_f + attn_f + emb_f) / (mean_ms * 1e-3) / 1e12, 1),
            "attn_gemm_frac_of_mfma_peak": round(t_roof / t_meas, 4),
            "attn_gemm_kernel_ms": round(t_meas * 1e3, 3),
            "roofline": {"bound": "mfma", "achieved": round(achieved, 1),
                         "peak": PEAK[k] / 1e12, "unit": "TFLOP/s",
                         "frac": round(achieved * 1e12 / PEAK[k], 4), "traffic": None,
                         "kernel": "single-block input GEMM (4608 x 21504 x 3072, GELU epilogue)",
                         "avg_ms": round(dom_avg, 4), "launches_timed": len(dom)},
            "kernels": per_kernel,
        }
    head = kinds[0]
    line = {
        "metric": METRIC,
        "value": out[head]["ms_per_step"],
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": out[head]["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head,
        "data": "synthetic: random-init N(0, 0.02) weights drawn on the device; latents, text, "
                "pooled N(0, 1); timestep U[0, 1); guidance 3.5",
        "config": {"workload": "FLUX.1-dev-shaped DiT denoise step, 1024x1024 image "
                               "(64x64 patches = 4096 tokens) + 512 text tokens, 19 double + "
                               "38 single blocks, hidden 3072, 24 x 128 heads",
                   "global_batch": 1, "seq_len": TXT + IMG_HW[0] * IMG_HW[1],
                   "parallelism": "single GPU"},
        "roofline": out[head]["roofline"],
        "attn_gemm_frac_of_mfma_peak": out[head]["attn_gemm_frac_of_mfma_peak"],
        "steps_by_dtype": out,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(log)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
