#!/usr/bin/env python3
"""Benchmark: MoE-layer tokens/s of the packed W4A16 expert path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4|c3|c2|c1]

A *step* is one quantized MoE layer over one batch -- one ``lq_moe_layer``
call on one stream: the router (softmax top-k from logits), the expert plan
(stable permutation and row blocks; for T*k <= 2048 every GEMM workgroup
derives its own block instead), the streaming GEMM1 (W1 gate and up tiles,
bf16 pre-activations), the streaming GEMM2 (SwiGLU applied while staging,
W2, routed weight) and the top-k combine.  Inputs are resident in HBM before
the timed region; weights rotate over several independently quantized
copies so every step streams its weights from HBM rather than from the
256 MB MALL.

Default workload (the north-star target): C4 of BASELINE.json -- 64 experts,
hidden 2048, intermediate 1024, INT4 group 128 with MSE scales (grid 16),
64 tokens ~N(0,1), top-8 routing with Zipf(1.1)-skewed router logits.

One JSON line is printed.  Besides the contract fields it carries
``roofline`` for the dominant kernel (GEMM1: HBM-bound at C4/C2,
MFMA-bound at C3), timed with fence-free HIP events the library records on
its own stream in a second pass over the same calls (the headline ``value``
comes from a pass without markers); ``roofline.traffic`` is the HBM bytes
per GEMM1 launch that ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE``
measured for this configuration (the committed summary under profiles/,
scaled by a device copy of known size), or null when no summary exists.
Also per-stage times, the other weight form's timing (``folded_scales`` or
``exact_weights``), ``cpu_baseline`` (the reference's dequantize-then-matmul
path on the host CPU, torch, bounded sample) and ``gpu_dequant_then_gemm``
(the same layer as dequantize-to-BF16 with the HIP dequant kernel, then
torch BF16 batched GEMMs on the same GPU).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

MI355X_HBM_GBPS = 8000.0
MI355X_BF16_TFLOPS = 2500.0

CONFIGS = {
    "c4": dict(name="C4", tokens=64, bits=4, search="mse", skew=True, renorm=False, bound="hbm"),
    "c3": dict(name="C3", tokens=4096, bits=4, search="mse", skew=False, renorm=False, bound="mfma"),
    "c2": dict(name="C2", tokens=512, bits=8, search="amax", skew=False, renorm=False, bound="hbm"),
    "c1": dict(name="C1", tokens=256, bits=4, search="amax", skew=False, renorm=True, bound="hbm",
               experts=16, hidden=1024, inter=512, top_k=2),
}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--config", choices=sorted(CONFIGS) + ["c5", "linear"], default="c4")
    p.add_argument("--layers", type=int, default=16, help="c5: layers in the stack")
    p.add_argument("--copies", type=int, default=0, help="weight copies to rotate (0: enough to exceed 3x the MALL)")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="bound on the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-c3", action="store_true",
                   help="c4: skip the large-token (C3) leg reported under the 'c3' key")
    p.add_argument("--no-gpu-baseline", action="store_true", help="skip the dequantize-then-GEMM leg")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--kernel", choices=("auto", "stream", "fused", "general", "wide"), default="auto",
                   help="GEMM family (auto: the library's own choice for the shape; fused: the streaming family "
                        "as one launch, the fused layer kernel)")
    p.add_argument("--tokens", type=int, default=0, help="override the configuration's token count")
    p.add_argument("--folded", action="store_true",
                   help="time the LQ_MOE_FOLDED_SCALES form (integer codes, fp32 group scale) as the headline")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB five times (the known-size kernel that scales "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE readings into bytes) and exit")
    return p.parse_args()


def copy_calibration(mib):
    """Five launches of torch's device copy of `mib` MiB: reads and writes exactly mib MiB each."""
    import torch

    n = mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": n, "launches": 5}), flush=True)


def pmc_traffic(config, form, kernel="gemm1"):
    """HBM bytes per launch of `kernel` from profiles/moe_gemm_<config>_pmc_traffic.txt, or None.

    The summary holds lines ``traffic_bytes <kernel> <form> <bytes>``: FETCH_SIZE and WRITE_SIZE
    per dispatch from two rocprofv3 --pmc runs of this bench, each scaled by what the counter
    reads for a device copy of known size (the commands are in the file).
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"moe_gemm_{config}_pmc_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 4 and parts[0] == "traffic_bytes" and parts[1] == kernel and parts[2] == form:
                    return int(parts[3])
    except OSError:
        return None
    return None


KERNEL_NAMES = {
    "fused": "moe_fused_kernel (route + plan + GEMM1 + GEMM2 + combine in one launch, W1/W2 streamed per CU)",
    "wide": "moe_wide_kernel<G1> (blocks of <= 128 rows, 2 weight tiles x 8 row tiles per wave, SwiGLU epilogue)",
    "stream": "moe_stream_kernel<G1> (W1 gate and up tiles streamed per CU)",
    "general": "moe_gemm_kernel<G1> (W1 gate+up, SwiGLU epilogue; persistent)",
}


def kernel_family(cfg, folded, forced):
    """The GEMM family lq_moe_layer runs for this shape (the library's rule), or the forced one."""
    if forced != "auto":
        return forced
    E, H, I, k, T = cfg["experts"], cfg["hidden"], cfg["inter"], cfg["top_k"], cfg["tokens"]
    if not folded and H % 256 == 0 and I % 256 == 0 and T * k >= 32 * E:
        return "wide"
    step = 512 if cfg["bits"] == 4 else 256
    return "stream" if H % step == 0 and I % step == 0 else "general"


def zipf_logits(torch, T, E, seed, s=1.1):
    """Router logits ~N(0,1) plus a per-expert bias making expert popularity Zipf(s)."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(E, generator=g)
    p = torch.arange(1, E + 1, dtype=torch.float64) ** (-s)
    bias = torch.log(p / p.sum())[perm].float()
    return torch.randn(T, E, generator=g) + bias


class Hip:
    """The few HIP runtime calls the bench needs (events), from torch's HIP runtime."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]

    # timing-only events: no system-scope fence (no L2 writeback / invalidate
    # when recorded), so a marker between two kernels costs next to nothing
    DISABLE_SYSTEM_FENCE = 0x20000000

    def event(self, light=False):
        ev = ctypes.c_void_p()
        if light:
            rc = self.lib.hipEventCreateWithFlags(ctypes.byref(ev), self.DISABLE_SYSTEM_FENCE)
        else:
            rc = self.lib.hipEventCreate(ctypes.byref(ev))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed ({rc})")
        return ev

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        rc = self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def destroy(self, ev):
        self.lib.hipEventDestroy(ev)


def build_workload(torch, cfg, copies, seed, dev):
    from llada_quant_amd.algorithms.symmetric import quantize_tensor

    E, H, I, k = cfg["experts"], cfg["hidden"], cfg["inter"], cfg["top_k"]
    layers = []
    for c in range(copies):
        g = torch.Generator(device=dev).manual_seed(seed * 1000 + c)
        w1 = (torch.randn(E, 2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        w2 = (torch.randn(E, H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q1 = quantize_tensor(w1, bits=cfg["bits"], group_size=128, scale_search=cfg["search"], search_grid=16)
        q2 = quantize_tensor(w2, bits=cfg["bits"], group_size=128, scale_search=cfg["search"], search_grid=16)
        layers.append((q1, q2))
        del w1, w2
    g = torch.Generator().manual_seed(seed + 7)
    T = cfg["tokens"]
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = (zipf_logits(torch, T, E, seed + 11) if cfg["skew"] else torch.randn(T, E, generator=g)).to(dev)
    return layers, x, logits


def layer_bytes(cfg, n_active):
    """Algorithmic HBM bytes (compulsory traffic, each byte once) of the layer and of its two GEMM kernels.

    GEMM1: packed w1 + its fp32 scales of every active expert, plus x [T, H]
    bf16.  GEMM2: packed w2 + scales, plus the routing weights [T, k] fp32.
    Layer: both, plus out [T, H] bf16, the router logits [T, E] fp32 and the
    ids [T, k] int32.  Intermediates (act, slot outputs) are excluded.
    """
    E, H, I, k, T = cfg["experts"], cfg["hidden"], cfg["inter"], cfg["top_k"], cfg["tokens"]
    vb = 0.5 if cfg["bits"] == 4 else 1.0
    w1 = 2 * I * H * vb + 2 * I * (H // 128) * 4
    w2 = H * I * vb + H * (I // 128) * 4
    g1 = n_active * w1 + T * H * 2
    g2 = n_active * w2 + T * k * 4
    layer = g1 + g2 + T * H * 2 + T * E * 4 + T * k * 4
    return int(layer), int(g1), int(g2)


def gpu_dequant_then_gemm(torch, cfg, layers, x, logits, steps, warmup):
    """Same-GPU baseline: dequantize both weights to BF16 (HIP kernel), then torch BF16 bmm."""
    from llada_quant_amd.algorithms.symmetric import dequantize_tensor
    import torch.nn.functional as F

    E, H, I, k, T = cfg["experts"], cfg["hidden"], cfg["inter"], cfg["top_k"], cfg["tokens"]

    def step(q1, q2):
        w1 = dequantize_tensor(q1.q, q1.scale, q1.bits, q1.group_size, torch.bfloat16, packed=q1.packed)
        w2 = dequantize_tensor(q2.q, q2.scale, q2.bits, q2.group_size, torch.bfloat16, packed=q2.packed)
        probs = torch.softmax(logits, -1, dtype=torch.float32)
        wts, ids = probs.topk(k, dim=-1)
        flat = ids.reshape(-1)
        order = torch.argsort(flat, stable=True)
        counts = torch.bincount(flat, minlength=E)
        mmax = int(counts.max())  # one host sync, like moe_align_block_size's padding
        offs = torch.cumsum(counts, 0) - counts
        pos = torch.arange(N, device=x.device) - offs[flat[order]]
        tok = order // k
        xt = torch.zeros(E, H, mmax, dtype=torch.bfloat16, device=x.device)
        xt[flat[order], :, pos] = x[tok]
        h = torch.bmm(w1, xt)  # [E, 2I, M]; right operand contiguous
        act = (F.silu(h[:, :I].float()).to(torch.bfloat16).float() * h[:, I:].float()).to(torch.bfloat16)
        y = torch.bmm(w2, act.contiguous())  # [E, H, M]
        yt = y[flat[order], :, pos].float() * wts.reshape(-1)[order].unsqueeze(1)
        out = torch.zeros(T, H, dtype=torch.float32, device=x.device)
        out.index_add_(0, tok, yt)
        return out.to(torch.bfloat16)

    N = T * k
    for i in range(warmup):
        step(*layers[i % len(layers)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(*layers[i % len(layers)])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    return {"value": round(T * steps / dt, 1), "unit": "tokens/s", "ms_per_step": round(dt / steps * 1e3, 4),
            "what": "HIP dequant of full w1/w2 to BF16 + torch BF16 bmm over all experts (padded to the "
                    "max tokens per expert) + SwiGLU + weighted index_add"}


def cpu_baseline(torch, cfg, layers, x, logits, budget_s):
    """The reference's PACKED layer (dequantize-then-matmul) on the host CPU, bounded sample."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import torch_ref

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    q1, q2 = layers[0]
    args = [t.cpu() for t in (x, logits.float(), q1.q, q1.scale, q2.q, q2.scale)]
    torch_ref.packed_layer(*args, cfg["bits"], 128, cfg["top_k"], cfg["renorm"])  # warm
    steps, t0 = 0, time.perf_counter()
    while True:
        torch_ref.packed_layer(*args, cfg["bits"], 128, cfg["top_k"], cfg["renorm"])
        steps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s or steps >= 50:
            break
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(cfg["tokens"] * steps / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{steps} full {cfg['name']} layer steps ({cfg['tokens']} tokens each, whole-tensor "
                      f"dequantize per access as the reference property does), torch CPU, {cpu_model}",
            "seconds": round(dt, 2)}


def bench_linear(args, torch):
    """QuantLinear (W8A16, group 128) on the reference's own benchmark shape: a 64 MiB weight
    (8192 x 8192 INT8), M = 16 / 64 / 128 / 256 rows (runtime/kernels/w8a16_gemm.py:1-11),
    against torch's BF16 GEMM on the already-dequantized weight on the same GPU.  Six weight
    copies (384 MiB of codes) rotate so the codes stream from HBM."""
    from llada_quant_amd.algorithms.symmetric import quantize_tensor
    from llada_quant_amd.runtime.linear import quant_linear

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    N = K = 8192
    copies = 6
    qs, wd = [], []
    for c in range(copies):
        g = torch.Generator(device=dev).manual_seed(args.seed * 100 + c)
        w = (torch.randn(N, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        q = quantize_tensor(w, bits=8, group_size=128)
        qs.append(q)
        wd.append(q.dequantize(torch.bfloat16).t().contiguous())  # [K, N] for x @ w
        del w
    steps = max(10, min(args.steps, 1000))
    warm = max(3, min(args.warmup, 200))  # past the clock ramp, for both legs alike
    rows = []
    for M in (16, 64, 128, 256):
        x = torch.randn(M, K, device=dev).to(torch.bfloat16)

        def timed(fn):
            for i in range(warm):
                fn(i)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            for i in range(steps):
                fn(i)
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / steps

        ms = timed(lambda i: quant_linear(x, qs[i % copies].q, qs[i % copies].scale, 8, 128))
        ms_bf16 = timed(lambda i: x @ wd[i % copies])
        algo = N * K + N * (K // 128) * 4 + M * K * 2 + M * N * 2
        rows.append({"M": M, "ms": round(ms, 5), "gbps": round(algo / (ms / 1e3) / 1e9, 1),
                     "hbm_frac": round(algo / (ms / 1e3) / 1e9 / MI355X_HBM_GBPS, 4),
                     "bf16_dequantized_ms": round(ms_bf16, 5), "speedup_vs_bf16": round(ms_bf16 / ms, 3)})
    r0 = rows[0]
    result = {
        "metric": "QuantLinear W8A16 rows/s, 64 MiB weight; % HBM roofline",
        "value": round(16 / (r0["ms"] / 1e3), 1), "unit": "rows/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": r0["ms"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "QuantLinear W8A16: x [M, 8192] bf16 . W^T, W 8192 x 8192 INT8 g128 amax, M = 16",
                   "sweep": rows},
        "roofline": {"kernel": "lq_quant_linear at M = 16 (linear_small_kernel, one launch)", "bound": "hbm",
                     "achieved": r0["gbps"], "peak": MI355X_HBM_GBPS, "unit": "GB/s", "frac": r0["hbm_frac"],
                     "traffic": None, "avg_ms": r0["ms"]},
    }
    print(json.dumps(result), flush=True)


def bench_c5(args, torch):
    """C5: a 16-layer INT4 MoE stack (E64, H2048, I1024, top-8) over 32 x 1024 tokens, timed
    end to end together with the GPU quantize+pack (MSE scale search, 16 clip ratios in
    [0.5, 1.0], group 128) of every layer's BF16 weights.  Each layer is
    h <- h + moe_layer(h) (a residual keeps the activations at unit scale through the
    stack; the add is inside the timed region).  Each layer is one library call over all
    32768 tokens (262144 assignments)."""
    from llada_quant_amd.algorithms.symmetric import quantize_tensor
    from llada_quant_amd.runtime.fused_moe import _chunks, max_tokens_per_call, moe_layer
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as O

    E, H, I, k = 64, 2048, 1024, 8
    L = args.layers
    T = args.tokens or 32768
    steps, warmup = max(1, min(args.steps, 5)), min(args.warmup, 1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w1s, w2s, logits = [], [], []
    for layer in range(L):
        g = torch.Generator(device=dev).manual_seed(args.seed * 1000 + layer)
        w1s.append((torch.randn(E, 2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16))
        w2s.append((torch.randn(E, H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16))
        logits.append(torch.randn(T, E, generator=g, device=dev))
    g = torch.Generator(device=dev).manual_seed(args.seed + 7)
    x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)

    def quantize_all():
        return [(quantize_tensor(w1, bits=4, group_size=128, scale_search="mse", search_grid=16),
                 quantize_tensor(w2, bits=4, group_size=128, scale_search="mse", search_grid=16))
                for w1, w2 in zip(w1s, w2s)]

    def stack(layers):
        h = x
        for (q1, q2), lg in zip(layers, logits):
            out, _ = moe_layer(h, lg, q1, q2, top_k=k)
            h = h + out
        return h

    for _ in range(warmup):
        stack(quantize_all())
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        layers = quantize_all()
        ev[i][1].record()
        h = stack(layers)
        ev[i][2].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    quant_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / steps
    stack_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / steps
    total_ms = quant_ms + stack_ms
    # the GPU quantizer against the oracle's restatement of the reference quantizer,
    # bit for bit, on a sample of rows of layer 0 (w2: 128 rows, w1: 16 rows)
    exact = True
    for w, q, rows in ((w2s[0], layers[0][1], 128), (w1s[0], layers[0][0], 16)):
        wr = w.reshape(-1, w.shape[-1])[:rows].contiguous().cpu()
        oq, os_, _ = O.quantize(wr.view(torch.int16).numpy().view("uint16"), bits=4, group_size=128,
                                scale_search="mse", grid=16, w_dtype=O.BF16)
        gq = q.q.reshape(-1, q.q.shape[-1])[:rows].cpu().numpy()
        gs = q.scale.reshape(-1, q.scale.shape[-1])[:rows].cpu().numpy()
        exact = exact and bool((gq == oq).all() and (gs == os_).all())
    flops = L * 2.0 * T * k * 3 * I * H
    weights_bf16 = L * E * 3 * I * H * 2
    packed = L * E * 3 * I * H // 2 + L * E * 3 * I * (H // 128) * 4  # codes + scales (w1: 2I x H/128, w2: H x I/128)
    stack_tflops = flops / (stack_ms / 1e3) / 1e12
    result = {
        "metric": "MoE-layer tokens/s W4A16 64E top-8 H2048; % HBM/MFMA roofline",
        "value": round(T / (total_ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(total_ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {
            "workload": f"C5: {L}-layer INT4 MoE stack (64 experts, hidden 2048, intermediate 1024, top-8, "
                        f"residual add) over {T} tokens, timed with the GPU MSE quantize+pack (grid 16) of all layers",
            "experts": E, "hidden": H, "intermediate": I, "top_k": k, "tokens": T, "layers": L, "bits": 4,
            "group_size": 128, "calls_per_layer": len(_chunks(T, max_tokens_per_call(H, I, k))),
            "quantize_ms": round(quant_ms, 3), "stack_ms": round(stack_ms, 3),
            "layer_ms": round(stack_ms / L, 4), "wall_ms_per_step": round(wall * 1e3, 3),
            "quantizer": {"bf16_bytes_read": weights_bf16, "packed_bytes_written": packed,
                          "gbps": round((weights_bf16 + packed) / (quant_ms / 1e3) / 1e9, 1),
                          "sampled_rows_bitexact_vs_oracle": exact},
        },
        "roofline": {"kernel": "MoE stack (wide GEMMs), all layers", "bound": "mfma",
                     "achieved": round(stack_tflops, 1), "peak": MI355X_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(stack_tflops / MI355X_BF16_TFLOPS, 4), "traffic": None,
                     "algorithmic_flops": flops, "avg_ms": round(stack_ms, 3)},
    }
    if not args.no_cpu:
        cfg = dict(experts=E, hidden=H, inter=I, top_k=k, tokens=256, bits=4, renorm=False, name="C5 sample")
        base = cpu_baseline(torch, cfg, layers[:1], x[:256], logits[0][:256], args.cpu_seconds)
        per_layer = base["value"]
        base["value"] = round(per_layer / L, 2)
        base["sample"] = (f"projection: one layer on 256 tokens ({base['sample']}) at {per_layer} tokens/s, "
                          f"divided by {L} layers; quantizer not included")
        result["cpu_baseline"] = base
    del h
    print(json.dumps(result), flush=True)


def main():
    args = parse_args()
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (got --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the path would shard by expert, and one GPU's share is what runs here",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.config == "c5":
        bench_c5(args, torch)
        return
    if args.config == "linear":
        bench_linear(args, torch)
        return
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from llada_quant_amd.runtime import _lib
    from llada_quant_amd.runtime.fused_moe import _check_weights, workspace_bytes

    cfg = dict(experts=64, hidden=2048, inter=1024, top_k=8)
    cfg.update(CONFIGS[args.config])
    if args.tokens:
        cfg["tokens"] = args.tokens
    E, H, I, k, T = cfg["experts"], cfg["hidden"], cfg["inter"], cfg["top_k"], cfg["tokens"]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    vb = 0.5 if cfg["bits"] == 4 else 1.0
    per_copy = E * 3 * I * H * vb * (1 + 8 / 128 / vb)
    copies = args.copies or max(3, int(3 * 256e6 // per_copy) + 1)
    layers, x, logits = build_workload(torch, cfg, copies, args.seed, dev)

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    ws_bytes = workspace_bytes(T, H, I, E, k)
    workspace = _lib.moe_workspace(ws_bytes, dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)

    def calls_for(xx, lg, renorm, ws, oo, ii, flags):
        """lq_moe_layer argument tuples, one per weight copy, for tokens xx / logits lg."""
        calls = []
        for q1, q2 in layers:
            g1, g2, _ = _check_weights(xx, q1, q2)
            calls.append((
                _lib.ptr(xx), _lib.ptr(lg), _lib.LQ_F32, xx.shape[0], H, I, E, k, int(renorm), _lib.ptr(q1.q),
                _lib.ptr(q1.scale), _lib.ptr(q2.q), _lib.ptr(q2.scale), cfg["bits"], g1, g2, flags,
                _lib.ptr(ws), ws.numel(), _lib.ptr(oo), _lib.ptr(ii), ctypes.c_void_p(stream.cuda_stream),
            ))
        return calls

    def make_calls(flags):
        return calls_for(x, logits, cfg["renorm"], workspace, out, ids, flags)

    hip = Hip()
    hip.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip_stream = ctypes.c_void_p(stream.cuda_stream)
    # stage boundaries of one lq_moe_layer call: 0 start, 1 route, 2 plan, 3 GEMM1, 4 GEMM2
    # (+SwiGLU, routed weight), 5 combine.  The fused layer kernel is one launch: its time is the
    # GEMM1 stage, the others record no kernel (route and plan too when it routes in-kernel)
    n_marks = 6

    def timed(calls, steps, warmup):
        """ms per step of `steps` layer calls, no markers inside the timed region."""
        for i in range(warmup):
            rc = lib.lq_moe_layer(*calls[i % len(calls)])
            if rc:
                _lib.check(rc, "moe_layer")
        t_start, t_end = hip.event(), hip.event()
        torch.cuda.synchronize()  # barrier (one rank) + sync on both sides of the timed region
        hip.lib.hipEventRecord(t_start, hip_stream)
        for i in range(steps):
            rc = lib.lq_moe_layer(*calls[i % len(calls)])
            if rc:
                _lib.check(rc, "moe_layer")
        hip.lib.hipEventRecord(t_end, hip_stream)
        torch.cuda.synchronize()
        total_ms = hip.elapsed_ms(t_start, t_end)
        hip.destroy(t_start)
        hip.destroy(t_end)
        return total_ms / steps

    def staged(calls, steps):
        """Mean ms per stage [route, plan, gemm1, gemm2, combine] over `steps` layer calls, from
        fence-free HIP events the library records on its stream at the kernel boundaries."""
        marks = [[hip.event(light=True) for _ in range(n_marks)] for _ in range(steps)]
        arrays = [(ctypes.c_void_p * n_marks)(*[m.value for m in row]) for row in marks]
        torch.cuda.synchronize()
        for i in range(steps):
            lib.lq_moe_profile_events(ctypes.cast(arrays[i], ctypes.c_void_p), n_marks)
            rc = lib.lq_moe_layer(*calls[i % len(calls)])
            if rc:
                _lib.check(rc, "moe_layer")
        torch.cuda.synchronize()
        stage_ms = [sum(hip.elapsed_ms(row[j], row[j + 1]) for row in marks) / steps for j in range(n_marks - 1)]
        for row in marks:
            for m in row:
                hip.destroy(m)
        return stage_ms

    family = kernel_family(cfg, args.folded, args.kernel)
    kflag = {"wide": _lib.LQ_MOE_WIDE_KERNEL, "general": _lib.LQ_MOE_GENERAL_KERNEL,
             "stream": _lib.LQ_MOE_STREAM_KERNEL,
             "fused": _lib.LQ_MOE_STREAM_KERNEL | _lib.LQ_MOE_FUSED_LAYER}.get(args.kernel, 0)
    calls = make_calls((_lib.LQ_MOE_FOLDED_SCALES if args.folded else 0) | kflag)
    wall0 = time.perf_counter()
    ms_per_step = timed(calls, args.steps, args.warmup)
    wall = time.perf_counter() - wall0
    stage_ms = staged(calls, args.steps)
    value = T / (ms_per_step / 1e3)
    n_active = int((torch.bincount(ids.reshape(-1).long(), minlength=E) > 0).sum())
    layer_b, g1_b, g2_b = layer_bytes(cfg, n_active)
    gemm1_ms = stage_ms[2]
    kname = KERNEL_NAMES[family]
    traffic = pmc_traffic(args.config, "folded" if args.folded else "exact",
                          "fused" if family == "fused" else "gemm1")
    if cfg["bound"] == "hbm":
        # the dominant kernel: GEMM1, or the fused kernel, which is the whole layer
        kb = layer_b if family == "fused" else g1_b
        achieved = kb / (gemm1_ms / 1e3) / 1e9
        roofline = {"kernel": kname, "bound": "hbm", "achieved": round(achieved, 1), "peak": MI355X_HBM_GBPS,
                    "unit": "GB/s", "frac": round(achieved / MI355X_HBM_GBPS, 4), "traffic": traffic,
                    "algorithmic_bytes": kb, "avg_ms": round(gemm1_ms, 5)}
    else:
        flops = 2.0 * T * k * 2 * I * H
        achieved = flops / (gemm1_ms / 1e3) / 1e12
        roofline = {"kernel": kname, "bound": "mfma", "achieved": round(achieved, 1), "peak": MI355X_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / MI355X_BF16_TFLOPS, 4), "traffic": traffic,
                    "algorithmic_flops": flops, "avg_ms": round(gemm1_ms, 5)}
    stages = {name: round(v, 5) for name, v in zip(("route", "plan", "gemm1", "gemm2", "combine"), stage_ms)}
    if family != "fused":
        stages["gemm2_gbps"] = round(g2_b / (stage_ms[3] / 1e3) / 1e9, 1)
    # the other weight form (the wide kernels take exact weights only)
    other_calls = make_calls(0 | kflag if args.folded else
                             _lib.LQ_MOE_FOLDED_SCALES | (kflag if args.kernel in ("general", "stream") else 0))
    other_ms = timed(other_calls, max(10, args.steps // 4), 3)
    other_stage = staged(other_calls, max(10, args.steps // 4))
    # the whole layer as one launch (the fused layer kernel), where it applies
    fused_extra = None
    if family == "stream" and not args.folded and E <= 64 and T * k <= 2048:
        fcalls = make_calls(_lib.LQ_MOE_FUSED_LAYER | kflag)
        f_ms = timed(fcalls, max(10, args.steps // 2), 5)
        fused_extra = {"ms_per_step": round(f_ms, 5), "value": round(T / (f_ms / 1e3), 1), "unit": "tokens/s",
                       "kernel": "moe_fused_kernel (route + plan + GEMM1 + GEMM2 + combine, one launch)",
                       "layer_gbps": round(layer_b / (f_ms / 1e3) / 1e9, 1)}

    result = {
        "metric": "MoE-layer tokens/s W4A16 64E top-8 H2048; % HBM/MFMA roofline",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{cfg['name']}: one MoE layer, {E} experts, hidden {H}, intermediate {I}, "
                        f"INT{cfg['bits']} g128 {cfg['search']} scales, {T} tokens, top-{k}"
                        + (", Zipf(1.1) router bias" if cfg["skew"] else ""),
            "experts": E, "hidden": H, "intermediate": I, "top_k": k, "tokens": T, "bits": cfg["bits"],
            "group_size": 128, "active_experts": n_active, "weight_copies": copies,
            "weights_in_mfma": "folded: exact codes, fp32 group scale" if args.folded else "exact bf16(fp32(q)*s)",
            "gemm_family": family,
            "layer_algorithmic_bytes": layer_b,
            "layer_gbps": round(layer_b / (ms_per_step / 1e3) / 1e9, 1),
            "wall_ms_per_step": round(wall / (args.steps + args.warmup) * 1e3, 5),
            "stage_ms": stages,
        },
        "roofline": roofline,
        ("exact_weights" if args.folded else "folded_scales"): {
            "ms_per_step": round(other_ms, 5), "gemm1_ms": round(other_stage[2], 5),
            "gemm2_ms": round(other_stage[3], 5), "value": round(T / (other_ms / 1e3), 1), "unit": "tokens/s"},
    }
    if fused_extra is not None:
        result["fused_layer"] = fused_extra
    if args.config == "c4" and not args.no_c3:
        # the large-token regime on the same weights (C3 uses C4's INT4 MSE layer): 4096 tokens,
        # unskewed routing, the wide (matrix-core) GEMMs; roofline of GEMM1 in TFLOP/s
        c3 = CONFIGS["c3"]
        T3 = c3["tokens"]
        g3 = torch.Generator().manual_seed(args.seed + 13)
        x3 = torch.randn(T3, H, generator=g3).to(torch.bfloat16).to(dev)
        lg3 = torch.randn(T3, E, generator=g3).to(dev)
        ws3 = _lib.moe_workspace(workspace_bytes(T3, H, I, E, k), dev)
        out3 = torch.empty(T3, H, dtype=torch.bfloat16, device=dev)
        ids3 = torch.empty(T3, k, dtype=torch.int32, device=dev)
        calls3 = calls_for(x3, lg3, c3["renorm"], ws3, out3, ids3, 0)
        ms3 = timed(calls3, max(10, args.steps // 4), max(10, args.warmup))  # after the C4 legs: warm to the MFMA load
        st3 = staged(calls3, max(10, args.steps // 4))
        flops1 = 2.0 * T3 * k * 2 * I * H
        tf1 = flops1 / (st3[2] / 1e3) / 1e12
        result["c3"] = {
            "workload": f"C3: the same layer over {T3} tokens, top-{k}, unskewed routing",
            "ms_per_step": round(ms3, 5), "value": round(T3 / (ms3 / 1e3), 1), "unit": "tokens/s",
            "gemm_family": kernel_family(dict(cfg, tokens=T3, skew=False), False, "auto"),
            "stage_ms": {name: round(v, 5) for name, v in zip(("route", "plan", "gemm1", "gemm2", "combine"), st3)},
            "layer_tflops": round(2.0 * T3 * k * 3 * I * H / (ms3 / 1e3) / 1e12, 1),
            "roofline": {"kernel": KERNEL_NAMES["wide"], "bound": "mfma", "achieved": round(tf1, 1),
                         "peak": MI355X_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tf1 / MI355X_BF16_TFLOPS, 4),
                         "algorithmic_flops": flops1, "avg_ms": round(st3[2], 5)},
        }
        del ws3, x3, out3
    if not args.no_gpu_baseline:
        result["gpu_dequant_then_gemm"] = gpu_dequant_then_gemm(torch, cfg, layers, x, logits,
                                                                max(5, args.steps // 10), 3)
    if not args.no_cpu:
        base = cpu_baseline(torch, cfg, layers, x, logits, args.cpu_seconds)
        # the two paths agree: one GPU step on weight copy 0 against the CPU reference output
        _lib.check(lib.lq_moe_layer(*calls[0]), "moe_layer")
        torch.cuda.synchronize()
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import torch_ref
        q1, q2 = layers[0]
        ref, _ = torch_ref.packed_layer(*[t.cpu() for t in (x, logits.float(), q1.q, q1.scale, q2.q, q2.scale)],
                                        cfg["bits"], 128, k, cfg["renorm"])
        diff = (out.float().cpu() - ref.float()).abs()
        base["gpu_vs_cpu_max_abs"] = float(diff.max())
        base["gpu_vs_cpu_mean_rel"] = float(diff.sum() / ref.float().abs().sum())
        result["cpu_baseline"] = base
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
