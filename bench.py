"""Benchmark: one DiT denoise step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload flux|qwen|wan|weights|compile|t5|umt5|vae|wanvae|qwenvae]
                    [--kinds bf16,fp8] [--no-cpu] [--calibrate-copy]

flux (default): the full FLUX.1-dev-shaped transformer forward of one denoise step, batch 1,
4096 image tokens (64 x 64 patch grid) + 512 text tokens, 19 double + 38 single blocks, hidden
3072, 24 x 128 heads, guidance 3.5. `value` is the bf16 step time; the fp8 step (every block
linear per-channel e4m3 with per-token activations) is reported beside it.
qwen: the Qwen-Image-shaped step, 60 joint blocks, 83 x 83 = 6889 image tokens (1328^2) + 256
text tokens (3584-wide encoder states), hidden 3072, 24 x 128 heads, MLP 12288; kinds "mx"
(MXFP8 on the QWEN_IMAGE_TARGETS linears) and "bf16".
wan: the Wan-2.2-14B-shaped text-to-video step, 40 blocks, latent 21 x 60 x 104 with patch
(1, 2, 2) = 32760 video tokens + 512 text tokens (4096-wide), hidden 5120, 40 x 128 heads, FFN
13824; kinds "bf16" and "mx" (MXFP8 on the cross-attention q/k/v and FFN linears, the
reference's Wan targets).
weights: the quantized-checkpoint writer's device work, every FLUX block linear (19 double x
12 + 38 single x 5 = 418 weights, 8.61 G values) quantized from bf16 to e4m3 codes and scales,
per-channel fp8 and MXFP8; `value` is the summed quantizer time in ms, K timed calls per shape.
compile: one FLUX single block (4608 tokens, hidden 3072, 24 x 128 heads, MLP 12288) written
with the op modules, one HIP kernel per op, run eagerly and under torch.compile(fullgraph=True);
`value` is the compiled block's ms.
t5 / umt5: the text encoder before the denoise loop, FLUX's T5-XXL / Wan's UMT5-XXL (24 blocks,
4096 wide, 64 x 64 heads, gated FFN 10240) on one 512-token prompt (UMT5: 300 real tokens, the
rest padding under the mask), bf16 and fp32; `value` is the bf16 encode in ms.
vae: FLUX's VAE decoder after the loop, a 128 x 128 x 16 latent to a 1024 x 1024 image, bf16
and fp32; `value` is the bf16 decode in ms.
wanvae: Wan 2.2's 3D causal VAE decoder after the loop, a 21 x 60 x 104 x 16 latent to 81
frames of 480 x 832, bf16 and fp32; `value` is the bf16 decode in ms.
qwenvae: the same decoder on Qwen-Image's one latent frame, 166 x 166 x 16 to one 1328 x 1328
image, bf16 and fp32; `value` is the bf16 decode in ms.
Weights are random N(0, 0.02) drawn on the device (norm weights ones); inputs N(0, 1); the
encoders and the decoder draw their weights with their initializations' scales.

Each step starts with its inputs resident in HBM. W untimed warmup steps, then K steps
bracketed by torch.cuda.synchronize(); per-step times from HIP events on the step stream.

roofline: the dominant kernel of each kind's step, the attention or GEMM launch name with the
largest summed time in a fully probed step run before the timed ones (flux bf16: the single-block
input GEMM, M 4608, N 7 x 3072, K 3072, 2 M N K = 608.8 GFLOP per launch, 38 per step; flux fp8:
the joint attention, 24 heads x 4608^2 keys x 128, 4 H S^2 d = 260.9 GFLOP per launch, 57 per
step; qwen: the joint attention, 24 heads x 7145^2 keys x 128, 627.3 GFLOP per launch, 60 per
step). Its average duration comes from HIP events recorded around each of its launches inside
the timed steps, on the stream it runs on. traffic: bytes per launch of that kernel between L2
and the memory fabric from rocprofv3 read / write request counters (null when not measured for
that kernel, kind and shape).
attn_gemm: one extra probed step times every GEMM and attention launch; the fraction is the
roofline time of their algorithmic FLOPs at MFMA peak over their summed measured time.
cpu_baseline (flux, N = 1): the oracle (fp32 torch restatement of the reference's CPU path) on
one double and one single block at the real shape, on this host's cores, extrapolated to the
19 + 38 blocks.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

METRIC = ("FLUX 1024² denoise step ms (bf16, fp8) at 1 GPU; attn+GEMM % of MFMA peak")
PEAK = {"bf16": 2.5e15, "fp8": 5.0e15, "mx": 5.0e15}  # dense MFMA, MI355X
SEED = 0
COPY_BYTES = 256 << 20

# Bytes per launch of the dominant kernel between L2 and the memory fabric (read + write), from
# two rocprofv3 --pmc runs of this script: TCC_EA0_RDREQ_{32B,64B,128B} and TCC_EA0_WRREQ{,_64B}
# request counts times their sizes (the same counters read exactly 256 MiB each way for the
# --calibrate-copy 256 MiB copy). MALL hits are counted too, so this bounds HBM bytes from above.
# Keyed by (workload, probe name, kind); absent -> null.
TRAFFIC: dict = {
    # 4608 x 21504 x 3072 GEMM (GELU, fused q/k norm): 1186.5 MB read (A + W = 160 MB once, plus
    # the RoPE tables) + 198.2 MB written (C)
    ("flux", "gemm.single.w1", "bf16"): 1_384_700_000,
    # the joint attention, 24 heads x 4608 x 4608 x 128 bf16 on the split schedule (the same
    # kernel in both steps; cut tiles in lockstep sets of 16 workgroups): 190.8 MB read (q, k, v
    # 84.9 MB once) + 84.6 MB written (the output 28.3 MB and the cut query tiles' fp32 partials)
    ("flux", "attn", "fp8"): 275_400_000,
    ("flux", "attn", "bf16"): 275_400_000,
    # Qwen-Image's joint attention, 24 heads x 7145 x 7145 x 128: 266.2 MB read + 95.8 written
    ("qwen", "attn", "mx"): 362_000_000,
    ("qwen", "attn", "bf16"): 362_000_000,
    # Wan's self-attention, 40 heads x 32760 x 32760 x 128 (one query tile per workgroup, 20
    # waves of workgroups): 3019.7 MB read + 335.5 MB written
    ("wan", "attn.self", "bf16"): 3_355_200_000,
    ("wan", "attn.self", "mx"): 3_355_200_000,
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="flux",
                    choices=("flux", "qwen", "wan", "weights", "compile", "t5", "umt5", "vae",
                             "wanvae", "qwenvae"))
    ap.add_argument("--kinds", default=None,
                    help="comma list (flux: bf16,fp8 by default; qwen: mx,bf16)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a plain 256 MiB bf16 elementwise copy (torch.neg) three "
                         "times, as the known-size reference for HBM byte counters")
    return ap.parse_args()


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


# ----------------------------------------------------------------------------------- workloads
class Flux:
    name = "flux"
    kinds = ("bf16", "fp8")
    img_hw, txt = (64, 64), 512
    desc = {"gemm.single.w1": "single-block input GEMM (4608 x 21504 x 3072; bf16: GELU epilogue)",
            "gemm.single.w2": "single-block output GEMM (4608 x 3072 x 15360, gated residual)",
            "attn": "joint attention (24 heads x 4608 queries x 4608 keys x 128, bf16)"}
    config = {"workload": "FLUX.1-dev-shaped DiT denoise step, 1024x1024 image (64x64 patches "
                          "= 4096 tokens) + 512 text tokens, 19 double + 38 single blocks, "
                          "hidden 3072, 24 x 128 heads",
              "global_batch": 1, "seq_len": 4608, "parallelism": "single GPU"}
    data = ("synthetic: random-init N(0, 0.02) weights drawn on the device; latents, text, pooled "
            "N(0, 1); timestep U[0, 1); guidance 3.5")

    def __init__(self):
        from difflet_amd.dit.flux import FluxConfig

        self.cfg = FluxConfig()
        self.si = self.img_hw[0] * self.img_hw[1]

    def build(self, kind, torch, dev):
        from difflet_amd.dit.flux import FluxDiT, random_param_source

        model = FluxDiT(self.cfg, random_param_source(self.cfg, SEED, dev), kind=kind, device=dev)
        g = torch.Generator(device=dev).manual_seed(SEED + 1)
        c = self.cfg
        lat = torch.randn(1, self.si, c.in_channels, generator=g, device=dev)
        text = torch.randn(1, self.txt, c.txt_dim, generator=g, device=dev)
        pooled = torch.randn(1, c.pooled_dim, generator=g, device=dev)
        t = torch.rand(1, generator=g, device=dev)
        guid = torch.full((1,), 3.5, device=dev)
        return model, lambda: model.forward(lat, text, pooled, t, guid, self.img_hw)

    def flops(self):
        """Algorithmic FLOPs per launch by probe name: GEMM 2 M N K, attention 4 H S^2 d."""
        c, s = self.cfg, self.txt + self.si
        d, f = c.hidden, c.mlp
        return {"gemm.double.qkv": 2 * s * d * 3 * d, "gemm.double.out": 2 * s * d * d,
                "gemm.double.ff1": 2 * s * d * f, "gemm.double.ff2": 2 * s * f * d,
                "gemm.single.w1": 2 * s * d * (3 * d + f), "gemm.single.w2": 2 * s * (d + f) * d,
                "attn": 4 * c.heads * s * s * c.head_dim}

    def step_flops(self):
        c, fl = self.cfg, self.flops()
        blocks = c.n_double * sum(fl[k] for k in fl if k.startswith("gemm.double")) + \
            c.n_single * sum(fl[k] for k in fl if k.startswith("gemm.single")) + \
            (c.n_double + c.n_single) * fl["attn"]
        emb = 2 * self.si * c.in_channels * c.hidden + 2 * self.txt * c.txt_dim * c.hidden + \
            2 * self.si * c.hidden * c.out_channels
        return blocks + emb

    def peak(self, name, kind):
        return PEAK["bf16"] if name == "attn" else PEAK[kind]


class Qwen:
    name = "qwen"
    kinds = ("mx", "bf16")
    img_hw, txt = (83, 83), 256
    desc = {"attn": "joint attention (24 heads x 7145 queries x 7145 keys x 128, bf16)"}
    config = {"workload": "Qwen-Image-shaped MMDiT denoise step, 1328x1328 image (83x83 patches "
                          "= 6889 tokens) + 256 text tokens, 60 joint blocks, hidden 3072, "
                          "24 x 128 heads, MLP 12288",
              "global_batch": 1, "seq_len": 7145, "parallelism": "single GPU"}
    data = ("synthetic: random-init N(0, 0.02) weights drawn on the device; latents and text "
            "encoder states N(0, 1); timestep U[0, 1)")

    def __init__(self):
        from difflet_amd.dit.qwen import QwenConfig

        self.cfg = QwenConfig()
        self.si = self.img_hw[0] * self.img_hw[1]

    def build(self, kind, torch, dev):
        from difflet_amd.dit.qwen import QwenImageDiT, random_param_source

        model = QwenImageDiT(self.cfg, random_param_source(self.cfg, SEED, dev), kind=kind,
                             device=dev)
        g = torch.Generator(device=dev).manual_seed(SEED + 1)
        c = self.cfg
        lat = torch.randn(1, self.si, c.in_channels, generator=g, device=dev)
        text = torch.randn(1, self.txt, c.txt_dim, generator=g, device=dev)
        t = torch.rand(1, generator=g, device=dev)
        return model, lambda: model.forward(lat, text, t, self.img_hw)

    def flops(self):
        c, s = self.cfg, self.txt + self.si
        d, f = c.hidden, c.mlp
        return {"gemm.joint.qkv": 2 * s * d * 3 * d, "gemm.joint.out": 2 * s * d * d,
                "gemm.joint.ff1": 2 * s * d * f, "gemm.joint.ff2": 2 * s * f * d,
                "attn": 4 * c.heads * s * s * c.head_dim}

    def step_flops(self):
        c, fl = self.cfg, self.flops()
        emb = 2 * self.si * c.in_channels * c.hidden + 2 * self.txt * c.txt_dim * c.hidden + \
            2 * self.si * c.hidden * c.out_channels
        return c.n_blocks * sum(fl.values()) + emb

    def peak(self, name, kind):
        # the output projections are not MXFP8 targets: bf16 peak for them and attention
        return PEAK["bf16"] if name in ("attn", "gemm.joint.out") else PEAK[kind]


class Wan:
    name = "wan"
    kinds = ("bf16", "mx")
    latent_fhw, txt = (21, 60, 104), 512
    desc = {"attn.self": "self-attention (40 heads x 32760 queries x 32760 keys x 128, bf16)"}
    config = {"workload": "Wan-2.2-14B-shaped video DiT denoise step, 480x832x81 frames -> "
                          "latent 21x60x104, patch (1, 2, 2) = 32760 video tokens + 512 text "
                          "tokens, 40 blocks, hidden 5120, 40 x 128 heads, FFN 13824",
              "global_batch": 1, "seq_len": 32760, "parallelism": "single GPU"}
    data = ("synthetic: random-init N(0, 0.02) weights drawn on the device; latents and text "
            "encoder states N(0, 1); timestep U[0, 1000)")

    def __init__(self):
        from difflet_amd.dit.wan import WanConfig

        self.cfg = WanConfig()
        f, h, w = self.latent_fhw
        self.s = f * (h // 2) * (w // 2)

    def build(self, kind, torch, dev):
        from difflet_amd.dit.wan import WanDiT, random_param_source

        model = WanDiT(self.cfg, random_param_source(self.cfg, SEED, dev), device=dev, kind=kind)
        g = torch.Generator(device=dev).manual_seed(SEED + 1)
        c = self.cfg
        lat = torch.randn(1, c.in_channels, *self.latent_fhw, generator=g, device=dev)
        text = torch.randn(1, self.txt, c.text_dim, generator=g, device=dev)
        t = torch.rand(1, generator=g, device=dev) * 1000.0
        return model, lambda: model.forward(lat, t, text)

    def flops(self):
        c, s, st = self.cfg, self.s, self.txt
        d, f = c.hidden, c.ffn
        return {"gemm.qkv": 2 * s * d * 3 * d, "gemm.out1": 2 * s * d * d,
                "gemm.q2": 2 * s * d * d, "gemm.kv2": 2 * st * d * 2 * d,
                "gemm.out2": 2 * s * d * d, "gemm.ffn_in": 2 * s * d * f,
                "gemm.ffn_out": 2 * s * f * d,
                "attn.self": 4 * c.heads * s * s * c.head_dim,
                "attn.cross": 4 * c.heads * s * st * c.head_dim}

    def step_flops(self):
        c = self.cfg
        emb = 2 * self.s * 64 * c.hidden + 2 * self.txt * (c.text_dim + c.hidden) * c.hidden + \
            2 * self.s * c.hidden * 64
        return c.n_blocks * sum(self.flops().values()) + emb

    def peak(self, name, kind):
        # MXFP8 on the reference's Wan targets: cross-attention q / k, v and both FFN linears
        mx = kind == "mx" and name in ("gemm.q2", "gemm.kv2", "gemm.ffn_in", "gemm.ffn_out")
        return PEAK["mx" if mx else "bf16"]


WORKLOADS = {"flux": Flux, "qwen": Qwen, "wan": Wan}


# ----------------------------------------------------------------------------------- runs
def run_kind(wl, kind, steps, warmup, torch, log):
    dev = torch.device("cuda", 0)
    t0 = time.time()
    model, step = wl.build(kind, torch, dev)
    torch.cuda.synchronize()
    log(f"[{wl.name}/{kind}] model built in {time.time() - t0:.1f} s, "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated")
    out = None
    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    if out is not None and not torch.isfinite(out.float()).all():
        raise RuntimeError(f"[{wl.name}/{kind}] non-finite output")
    log(f"[{wl.name}/{kind}] warmup done")

    # one step with every GEMM / attention launch probed: per-kernel times (attn_gemm) and the
    # dominant kernel, the launch name with the largest summed time
    full = Probe()
    model.probe = full
    step()
    torch.cuda.synchronize()
    model.probe = None
    by_name = full.times_ms()
    dominant = max(by_name, key=lambda n: sum(by_name[n]))

    probe = Probe(only={dominant})
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
    dom = probe.times_ms()[dominant]
    log(f"[{wl.name}/{kind}] {steps} steps: mean {sum(per_step) / steps:.2f} ms, "
        f"wall {wall_ms:.2f} ms; dominant kernel {dominant}")
    del model
    torch.cuda.empty_cache()
    return {"per_step": per_step, "wall_ms": wall_ms, "dominant": dominant, "dominant_ms": dom,
            "by_name": by_name}


def summarize(wl, kind, r):
    fl = wl.flops()
    mean_ms = sum(r["per_step"]) / len(r["per_step"])
    # attn+GEMM: roofline time of their FLOPs at MFMA peak / their measured kernel time
    t_meas = sum(sum(v) for v in r["by_name"].values()) * 1e-3
    t_roof = sum(fl[n] * len(v) / wl.peak(n, kind) for n, v in r["by_name"].items())
    dom, dname = r["dominant_ms"], r["dominant"]
    dom_avg = sum(dom) / len(dom)
    peak = wl.peak(dname, kind)
    achieved = fl[dname] / (dom_avg * 1e-3) / 1e12
    per_kernel = {n: {"launches": len(v), "avg_ms": round(sum(v) / len(v), 4),
                      "tflops": round(fl[n] / (sum(v) / len(v) * 1e-3) / 1e12, 1)}
                  for n, v in sorted(r["by_name"].items())}
    return {
        "ms_per_step": round(mean_ms, 3),
        "median_ms": round(r["per_step"][len(r["per_step"]) // 2], 3),
        "p90_ms": round(r["per_step"][int(0.9 * (len(r["per_step"]) - 1))], 3),
        "wall_ms_per_step": round(r["wall_ms"], 3),
        "tflops_step": round(wl.step_flops() / (mean_ms * 1e-3) / 1e12, 1),
        "attn_gemm_frac_of_mfma_peak": round(t_roof / t_meas, 4),
        "attn_gemm_kernel_ms": round(t_meas * 1e3, 3),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved * 1e12 / peak, 4),
                     "traffic": TRAFFIC.get((wl.name, dname, kind)),
                     "kernel": wl.desc.get(dname, dname),
                     "avg_ms": round(dom_avg, 4), "launches_timed": len(dom)},
        "kernels": per_kernel,
    }


def cpu_baseline(wl, log, runs: int = 3):
    """The oracle's fp32 CPU path on one double and one single block at the real FLUX shape:
    one full-shape warm-up of each, then the median of `runs` timed runs of each, extrapolated
    to the 19 + 38 blocks of the step."""
    import statistics

    import torch

    from oracle import flux as oflux
    from oracle import ops

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    torch.set_num_threads(threads)
    shape = oflux.FluxShape()
    g = torch.Generator().manual_seed(SEED)
    h, w = wl.img_hw
    si, st = h * w, wl.txt
    hidden = torch.randn(1, si, shape.hidden, generator=g)
    context = torch.randn(1, st, shape.hidden, generator=g)
    temb = torch.randn(1, shape.hidden, generator=g)
    cos, sin = ops.flux_pos_embed(ops.flux_ids(st, h, w))
    dw = oflux.double_block_weights(shape, SEED, 0)
    sw = oflux.single_block_weights(shape, SEED, 0)
    x = torch.cat([context, hidden], dim=1)
    blocks = {"double": lambda: oflux.double_block(dw, hidden, context, temb, cos, sin, shape),
              "single": lambda: oflux.single_block(sw, x, temb, cos, sin, shape)}
    med, spread = {}, {}
    for name, fn in blocks.items():
        fn()  # warm-up at the full shape: thread pool, allocator, first-touch of the buffers
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        med[name], spread[name] = statistics.median(times), (min(times), max(times))
        log(f"[cpu] {name} block: median {med[name]:.2f} s of {runs} "
            f"({min(times):.2f}-{max(times):.2f} s) on {threads} threads")
    step_ms = (shape.n_double * med["double"] + shape.n_single * med["single"]) * 1e3
    return {"value": round(step_ms, 1), "unit": "ms/step (extrapolated)", "cores": threads,
            "kind": "port",
            "sample": (f"fp32 oracle on {threads} threads, one double and one single block at "
                       f"{st}+{si} tokens: one full-shape warm-up each, then the median of "
                       f"{runs} runs (double {med['double']:.2f} s, single {med['single']:.2f} s), "
                       f"extrapolated x{shape.n_double} + x{shape.n_single}")}


# FLUX block linears by shape [N, K] -> count over 19 double + 38 single blocks
FLUX_BLOCK_LINEARS = {(3072, 3072): 19 * 8 + 38 * 3, (12288, 3072): 19 * 2 + 38,
                      (3072, 12288): 19 * 2, (3072, 15360): 38}


def weights_bytes(fmt, n, k):
    """Algorithmic HBM bytes of one quantizer call: bf16 read, e4m3 codes and scales written."""
    return n * k * 3 + (n * 4 if fmt == "fp8_rowwise" else n * k // 32)


def run_weights(args, torch, log):
    """Times the quantized-checkpoint writer's kernels over FLUX's block linears."""
    from difflet_amd import kernels

    fmts = {"fp8_rowwise": kernels.quantize_fp8_rowwise,
            "mxfp8": lambda w: kernels.quantize_mxfp8(w, swizzled=False)}
    res = {}
    for fmt, fn in fmts.items():
        total_ms, total_bytes, shapes = 0.0, 0, {}
        for (n, k), count in FLUX_BLOCK_LINEARS.items():
            g = torch.Generator(device="cuda").manual_seed(SEED + n + k)
            w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
            for _ in range(max(args.warmup, 1)):
                fn(w)
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                fn(w)
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / args.steps
            b = weights_bytes(fmt, n, k)
            shapes[f"{n}x{k}"] = {"count": count, "us": round(ms * 1e3, 2),
                                  "GB_per_s": round(b / (ms * 1e-3) / 1e9, 1)}
            total_ms += count * ms
            total_bytes += count * b
            log(f"[weights] {fmt} {n}x{k}: {ms * 1e3:.1f} us, {b / (ms * 1e-3) / 1e9:.0f} GB/s")
            del w
        res[fmt] = {"ms": round(total_ms, 3), "bytes": total_bytes,
                    "GB_per_s": round(total_bytes / (total_ms * 1e-3) / 1e9, 1), "shapes": shapes}
    head = res["fp8_rowwise"]
    big = head["shapes"]["3072x15360"]
    line = {
        "metric": "FLUX block linears quantized to fp8 (checkpoint writer device time, ms)",
        "value": head["ms"], "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms"], "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16->e4m3", "data": "synthetic",
        "config": {"workload": "FLUX.1 block linears, 418 weights, 8.61 G values",
                   "formats": list(res)},
        "roofline": {"bound": "hbm", "achieved": big["GB_per_s"], "peak": 8000.0,
                     "unit": "GB/s", "frac": round(big["GB_per_s"] / 8000.0, 3),
                     "traffic": None,
                     "kernel": "quantize_fp8_rowwise on 3072 x 15360 (proj_out)"},
        "by_format": res,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = weights_cpu_baseline(log)
    print(json.dumps(line), flush=True)
    return 0


def weights_cpu_baseline(log):
    """The oracle's per-channel quantizer (numpy, one thread) on one 3072 x 3072 weight,
    extrapolated to the 8.61 G values of FLUX's block linears."""
    import numpy as np

    from oracle import fp8 as ofp8

    w = (np.random.default_rng(SEED).standard_normal((3072, 3072), dtype=np.float32) * 0.02)
    ofp8.quantize_rowwise(w[:64])
    t0 = time.perf_counter()
    ofp8.quantize_rowwise(w)
    dt = time.perf_counter() - t0
    values = sum(n * k * c for (n, k), c in FLUX_BLOCK_LINEARS.items())
    log(f"[cpu] quantize_rowwise 3072x3072: {dt:.2f} s")
    return {"value": round(dt * values / w.size * 1e3, 1), "unit": "ms (extrapolated)",
            "cores": 1, "kind": "port",
            "sample": f"numpy oracle quantize_rowwise on one 3072 x 3072 weight ({dt:.2f} s), "
                      f"x {values / w.size:.0f}"}


def run_compile(args, torch, log):
    """A FLUX single block on the op modules, eager against torch.compile(fullgraph=True)."""
    import math

    import torch.nn as nn
    import torch.nn.functional as F

    from difflet_amd.backends.rocm.ops_impl.attention import attention
    from difflet_amd.backends.rocm.ops_impl.embeddings import apply_rotary_emb
    from difflet_amd.backends.rocm.ops_impl.linear import ColumnParallelLinear, RowParallelLinear
    from difflet_amd.backends.rocm.ops_impl.norm import LayerNorm, RMSNorm

    d, heads, s, dev = 3072, 24, 4608, torch.device("cuda")

    class Single(nn.Module):
        """difflet/models/flux/modeling_flux.py single block: adaLN, [q|k|v] and MLP-up from one
        normed input, q/k RMSNorm + RoPE, attention, proj_out over [attn | gelu(mlp)], gated
        residual."""

        def __init__(self):
            super().__init__()
            bf = dict(dtype=torch.bfloat16, device=dev)
            self.norm = LayerNorm(d, eps=1e-6, elementwise_affine=False)
            self.qkv = ColumnParallelLinear(d, 3 * d, **bf)
            self.mlp = ColumnParallelLinear(d, 4 * d, **bf)
            self.out = RowParallelLinear(5 * d, d, **bf)
            self.norm_q, self.norm_k = RMSNorm(128).to(dev), RMSNorm(128).to(dev)
            for m in (self.qkv, self.mlp, self.out):
                nn.init.normal_(m.weight, std=0.02)
                nn.init.zeros_(m.bias)

        def forward(self, x, shift, scale, gate, cos, sin):
            h = self.norm(x) * (1 + scale) + shift
            q, k, v = self.qkv(h).view(1, s, 3, heads, 128).permute(2, 0, 3, 1, 4).unbind(0)
            q = apply_rotary_emb(self.norm_q(q), cos, sin)
            k = apply_rotary_emb(self.norm_k(k), cos, sin)
            o = attention(q, k, v, scale=1.0 / math.sqrt(128)).transpose(1, 2).reshape(1, s, d)
            m = F.gelu(self.mlp(h), approximate="tanh")
            return x + gate * self.out(torch.cat([o, m], dim=-1))

    torch.manual_seed(SEED)
    blk = Single().eval()
    x = torch.randn(1, s, d, device=dev).to(torch.bfloat16)
    shift, scale, gate = (0.1 * torch.randn(1, 1, d, device=dev).to(torch.bfloat16) for _ in range(3))
    ang = torch.arange(s, device=dev)[:, None] * torch.exp(-torch.arange(64, device=dev) / 8.0)
    cos = torch.cos(ang).repeat_interleave(2, -1)
    sin = torch.sin(ang).repeat_interleave(2, -1)
    inputs = (x, shift, scale, gate, cos, sin)

    def timed(fn):
        with torch.no_grad():
            for _ in range(max(args.warmup, 1)):
                fn(*inputs)
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                y = fn(*inputs)
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps, y

    eager_ms, y0 = timed(blk)
    t0 = time.perf_counter()
    compiled = torch.compile(blk, fullgraph=True, mode="default")
    with torch.no_grad():
        compiled(*inputs)
    compile_s = time.perf_counter() - t0
    comp_ms, y1 = timed(compiled)
    rel = ((y1.float() - y0.float()).norm() / y0.float().norm()).item()
    flops = 2 * s * d * (3 * d + 4 * d + 5 * d) + 4 * heads * s * s * 128
    log(f"[compile] eager {eager_ms:.3f} ms, compiled {comp_ms:.3f} ms, first call "
        f"{compile_s:.1f} s, rel L2 {rel:.2e}")
    line = {
        "metric": "FLUX single block on the op modules, torch.compile(fullgraph=True) ms",
        "value": round(comp_ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(comp_ms, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "FLUX.1 single block, 4608 tokens, hidden 3072, 24 x 128 heads",
                   "compile_mode": "default"},
        "eager_ms": round(eager_ms, 3), "compiled_vs_eager_rel_l2": rel,
        "first_call_s": round(compile_s, 1),
        "block_tflops": round(flops / (comp_ms * 1e-3) / 1e12, 1),
    }
    print(json.dumps(line), flush=True)
    return 0


def t5_flops(cfg, s):
    """Matrix FLOPs of one encode of s tokens: q/k/v/o, the gated FFN, scores and P V."""
    d, inner, f = cfg.d_model, cfg.inner_dim, cfg.d_ff
    per_layer = 2 * s * (4 * d * inner + 3 * d * f) + 4 * s * s * inner
    return cfg.num_layers * per_layer


def vae_flops(cfg, h, w):
    """Matrix FLOPs of one decode of an h x w latent: every convolution (9 taps, or 1 for the
    shortcuts) at its resolution, the mid-block attention's projections, scores and P V."""
    from difflet_amd.vae import decoder as dvae

    shapes = dvae.param_shapes(cfg)
    top = cfg.block_out_channels[-1]
    px = h * w
    total = 2 * px * 9 * cfg.latent_channels * top  # conv_in
    total += 2 * px * (4 * top * top) + 4 * px * px * top  # attention
    res = {"mid_block": px}
    scale = 1
    for i, j, cin, cout, up in dvae._plan(cfg):
        res[f"up_blocks.{i}"] = px * scale * scale
        if up:
            scale *= 2
    for name, shp in shapes.items():
        if not name.endswith(".weight") or len(shp) != 4 or name.startswith("decoder.conv_in"):
            continue
        blk = next((k for k in res if f"decoder.{k}." in name), None)
        pix = res[blk] if blk else px * scale * scale  # conv_out at the full resolution
        if ".upsamplers." in name:
            pix *= 4
        total += 2 * pix * shp[0] * shp[1] * shp[2] * shp[3]
    return total


def wan_vae_flops(cfg, t, h, w):
    """Matrix FLOPs of one decode of a t x h x w latent by Wan's causal decoder: every
    convolution at its resolution over the frames it runs on (the time convolutions skip the
    first latent frame), the mid-block attention's projections, scores and P V per frame."""
    from difflet_amd.vae import wan as dwan

    dims, z = cfg.dims, cfg.z_dim
    px, frames = h * w, t
    total = 2 * t * px * z * z + 2 * t * px * 27 * z * dims[0]  # post_quant_conv, conv_in
    c0 = dims[0]
    total += 2 * 2 * (2 * t * px * 27 * c0 * c0)                 # mid-block resnets
    total += t * (2 * px * c0 * 4 * c0 + 4 * px * px * c0)         # attention
    for _, cin, cout, mode in dwan.plan(cfg):
        c = cin
        for _ in range(cfg.num_res_blocks + 1):
            total += 2 * frames * px * 27 * (c * cout + cout * cout)
            if c != cout:
                total += 2 * frames * px * c * cout
            c = cout
        if mode == "upsample3d":
            total += 2 * (frames - 1) * px * 3 * cout * 2 * cout
            frames = 1 + 2 * (frames - 1)
        if mode is not None:
            px *= 4
            total += 2 * frames * px * 9 * cout * (cout // 2)
    total += 2 * frames * px * 27 * dims[-1] * cfg.out_channels
    return total


def _time(fn, steps, warmup, torch):
    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    times = []
    for _ in range(steps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    return sum(times) / len(times), sorted(times)[len(times) // 2]


def run_stage(args, torch, log):
    """The steps either side of the denoise loop: the T5 / UMT5 encoders and the VAE decoder,
    bf16 and fp32, whole-stage time and its matrix FLOP rate against the MFMA peak."""
    dev = torch.device("cuda")
    res = {}
    if args.workload in ("t5", "umt5"):
        from difflet_amd.text.t5 import T5_XXL, UMT5_XXL, T5Encoder, random_param_source

        cfg = T5_XXL if args.workload == "t5" else UMT5_XXL
        s = 512
        ids = torch.randint(0, cfg.vocab_size, (1, s), generator=torch.Generator().manual_seed(SEED)).to(dev)
        mask = None
        if cfg.per_layer_bias:
            mask = torch.ones(1, s, dtype=torch.long, device=dev)
            mask[:, 300:] = 0
        flops = t5_flops(cfg, s)
        name = "T5-XXL" if args.workload == "t5" else "UMT5-XXL"
        workload = f"{name} text encoder, 24 blocks, d_model 4096, 64 x 64 heads, d_ff 10240, 512 tokens"
        for dt in (torch.bfloat16, torch.float32):
            enc = T5Encoder(cfg, random_param_source(cfg, SEED, dev, torch.float32), dtype=dt, device=dev)
            ms, med = _time(lambda: enc(ids, mask), args.steps, args.warmup, torch)
            res[str(dt).split(".")[1]] = {"ms": round(ms, 3), "median_ms": round(med, 3),
                                          "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
            log(f"[{args.workload}] {dt}: {ms:.2f} ms")
            del enc
            torch.cuda.empty_cache()
    elif args.workload in ("wanvae", "qwenvae"):
        from difflet_amd.vae import wan as dwan

        cfg = dwan.WAN_VAE
        lat = (21, 60, 104) if args.workload == "wanvae" else (1, 166, 166)
        z = torch.randn(1, 16, *lat, generator=torch.Generator().manual_seed(SEED)).to(dev)
        flops = wan_vae_flops(cfg, *lat)
        workload = ("Wan 2.2 VAE decoder (3D causal), 21 x 60 x 104 x 16 latent -> 81 frames of "
                    "480 x 832 RGB" if args.workload == "wanvae" else
                    "Qwen-Image VAE decoder (Wan's 3D causal decoder on one frame), 166 x 166 x "
                    "16 latent -> 1328 x 1328 RGB")
        for dt in (torch.bfloat16, torch.float32):
            dec = dwan.WanVaeDecoder(cfg, dwan.random_param_source(cfg, SEED, dev), dtype=dt,
                                     device=dev)
            ms, med = _time(lambda: dec.decode(z), args.steps, args.warmup, torch)
            res[str(dt).split(".")[1]] = {"ms": round(ms, 3), "median_ms": round(med, 3),
                                          "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
            log(f"[{args.workload}] {dt}: {ms:.2f} ms")
            del dec
            torch.cuda.empty_cache()
    else:
        from difflet_amd.vae import decoder as dvae

        cfg = dvae.FLUX_VAE
        z = torch.randn(1, 16, 128, 128, generator=torch.Generator().manual_seed(SEED)).to(dev)
        flops = vae_flops(cfg, 128, 128)
        workload = "FLUX.1 VAE decoder, 128 x 128 x 16 latent -> 1024 x 1024 RGB"
        for dt in (torch.bfloat16, torch.float32):
            dec = dvae.VaeDecoder(cfg, dvae.random_param_source(cfg, SEED, dev), dtype=dt, device=dev)
            ms, med = _time(lambda: dec.decode(z), args.steps, args.warmup, torch)
            res[str(dt).split(".")[1]] = {"ms": round(ms, 3), "median_ms": round(med, 3),
                                          "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
            log(f"[vae] {dt}: {ms:.2f} ms")
            del dec
            torch.cuda.empty_cache()
    head = res["bfloat16"]
    line = {
        "metric": f"{args.workload} stage ms (bf16, fp32) at 1 GPU",
        "value": head["ms"], "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms"], "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init weights drawn on the device, random token ids / latents",
        "config": {"workload": workload, "matrix_gflop": round(flops / 1e9, 1)},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(head["tflops"] / 2500.0, 4),
                     "traffic": None, "kernel": "whole stage (matrix FLOPs / stage time)"},
        "by_dtype": res,
    }
    if "float32" in res:
        line["by_dtype"]["float32"]["frac_of_fp32_peak"] = round(res["float32"]["tflops"] / 157.3, 4)
    print(json.dumps(line), flush=True)
    return 0


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(sharding the step across GPUs is designed, not built)", file=sys.stderr)
        return 2
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    log = lambda m: print(m, file=sys.stderr, flush=True)  # noqa: E731
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    from difflet_amd import _lib

    _lib.load()
    if args.workload == "weights":
        return run_weights(args, torch, log)
    if args.workload == "compile":
        return run_compile(args, torch, log)
    if args.workload in ("t5", "umt5", "vae", "wanvae", "qwenvae"):
        return run_stage(args, torch, log)
    wl = WORKLOADS[args.workload]()
    kinds = [k for k in (args.kinds or ",".join(wl.kinds)).split(",") if k]
    if args.calibrate_copy:
        src = torch.randn(COPY_BYTES // 2, device="cuda").bfloat16()
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    out = {k: summarize(wl, k, run_kind(wl, k, args.steps, args.warmup, torch, log))
           for k in kinds}
    head = kinds[0]
    metric = {"flux": METRIC,
              "qwen": "Qwen-Image 1328² denoise step ms (MXFP8, bf16) at 1 GPU; attn+GEMM % of "
                      "MFMA peak",
              "wan": "Wan-2.2 480x832x81 denoise step ms (bf16, MXFP8) at 1 GPU; attn+GEMM % of "
                     "MFMA peak"}[wl.name]
    line = {
        "metric": metric,
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
        "data": wl.data,
        "config": wl.config,
        "roofline": out[head]["roofline"],
        "attn_gemm_frac_of_mfma_peak": out[head]["attn_gemm_frac_of_mfma_peak"],
        "steps_by_dtype": out,
    }
    if not args.no_cpu and wl.name == "flux":
        line["cpu_baseline"] = cpu_baseline(wl, log)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
