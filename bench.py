#!/usr/bin/env python3
"""Benchmark: ms per 832x1216 int8 DiT pass + joint-attention TFLOP/s on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-dit] [--no-gemma] [--no-vendor] [--no-lora]

Prints one JSON line. Legs, in order:

1. DiT pass (the metric, `value`): the Node host (nanosaur2-web_amd/js/run_dit.js) runs one full
   pass of the 18-block Nanosaur2 DiT at 832x1216 (latent 76 rows x 52 cols = 3952 image tokens,
   256 text tokens, batch 1) on seeded random-init weights of the real architecture (int8 ConvRot
   block linears, bf16 elsewhere). W untimed passes, then K timed passes issued back to back with
   the latent tokens resident in device memory, bracketed by stream events and a device sync:
   `value` is the device time from the first pass's start to the last pass's end, divided by K
   (`pass_ms_single` is the median of K passes run one at a time, each followed by a sync).
   The region runs from the resident latent tokens to the resident x0
   tokens and includes condition() and the text refine; `pass_ms_host_to_host` adds the latent
   upload, the two device transposes and the x0 readback.
   The dominant kernel is the tiled int8 ConvRot GEMM (qkv, proj, w12, w3, kv_y of every block):
   a profiled run of the same pass times every launch with stream events on the library's
   stream, and `roofline` is its algorithmic 2*M*N*K flops summed over the pass / its summed
   launch time, against the 2516.6 TFLOP/s dense fp16 MFMA peak.
   `dit_lora` times the same pass with a synthetic rank-32 LoRA file on all 81 block linears
   (the LoRA side path), beside it.
2. Gemma3-270M text encoder (17 of 18 layers + final norm, 256 token ids, random-init bf16 weights
   of the real architecture) through the Node host (run_gemma.js), eager and replayed as a graph.
3. Through the C ABI (ctypes), each after 1 s of back-to-back warm-up calls, timed with stream
   events and the library's per-kernel profiler:
   - joint attention at 832x1216 (3952 queries x 4208 keys, 16 heads x 96, batch 2, 2-D RoPE on
     image rows, log-weight bias on text keys): `roofline_attention` (flash kernel) and the
     whole op (pack + flash);
   - joint attention at 768x768 (2304 queries x 2432 keys, batch 1);
   - the int8 ConvRot linear at M = 2432 on fp32 activations for N x K = 4608x1536, 1536x1536,
     6144x1536 and 1536x6144: the rotation into the tiled fp16 operand plus the tiled GEMM.
4. Vendor libraries at the same shapes, for scale (`vendor_reference`): hipBLASLt fp16 GEMMs at the
   four block-linear shapes (3952 rows) and torch SDPA at the joint-attention shape.
5. CPU baselines: the oracle (a PyTorch-CPU restatement of tools/reference.py, fp32) on this
   host's cores for the same workloads -- the DiT pass on a bounded sample (one joint and one
   image-only block at 3952 tokens, scaled to 18 blocks), the two attention shapes, the four
   linears and the text encoder -- 1 warm-up and up to 3 timed repetitions each (median).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "nanosaur2-web_amd")
RUN_DIT = os.path.join(PKG, "js", "run_dit.js")
RUN_GEMMA = os.path.join(PKG, "js", "run_gemma.js")
GEMMA_TOKENS, GEMMA_LAYERS = 256, 17
METRIC = "ms per 832x1216 DiT pass (int8) + joint-attention TFLOP/s, 1 MI355X"
PUBLISHED_PASS_MS = 1730.0   # README.md:86-88 of the reference (WebGPU, laptop GPU)
FP16_PEAK_TFLOPS = 2516.6    # MI355X dense fp16 MFMA
HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
H_IMG, W_IMG, T_TXT, D, HEADS, HD, I_MLP, BLOCKS = 76, 52, 256, 1536, 16, 96, 4096, 18
CFG1_M = 2432
CFG1_SHAPES = (("qkv", 4608, 1536), ("proj", 1536, 1536), ("up", 6144, 1536), ("down", 1536, 6144))
# Bytes per launch that leave the L2s (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, each scaled by
# what the counter reads for a copy kernel of known size: FETCH_SIZE x 2.0, WRITE_SIZE x 1.0), beside
# the algorithmic bytes of the same launches: the mean over one pass's 73 tiled-GEMM launches on the
# 3952 image rows (18 each of qkv and w12+GLU, 36 of proj and w3, the stacked kv_y), and one flash
# launch at 3952x4208 batch 2. The source files hold the per-kernel tables and the commands.
GEMM_TRAFFIC_BYTES_PER_LAUNCH = 123.2e6
GEMM_ALGORITHMIC_BYTES_PER_LAUNCH = 71.9e6   # N*K int8 W + 2*M*K fp16 A + output (+ old output for +=)
GEMM_TRAFFIC_SOURCE = "profiles/dit_pass_832x1216_int8.md"
ATTN_TRAFFIC_BYTES_PER_LAUNCH = 170.0e6
ATTN_ALGORITHMIC_BYTES_PER_LAUNCH = 149.1e6  # fp32 Q (read in the kernel's prologue), fp16 K, V^T, fp32 O
ATTN_TRAFFIC_SOURCE = "profiles/attn_flash_joint_3952x4208_b2.md"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads():
    """Threads for the CPU baselines: this process's CPU share (affinity, OMP_NUM_THREADS)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def pass_flops(L=H_IMG * W_IMG, T=T_TXT):
    """Algorithmic FLOPs of one DiT pass: GEMMs 2MNK, attention 4*Lq*Lk*D*H
    (app/gpu/ops.js:30, 207)."""
    g = lambda M, N, K: 2 * M * N * K  # noqa: E731
    blk = g(L, 3 * D, D) + g(L, D, D) + g(L, 2 * I_MLP, D) + g(L, D, I_MLP)
    total = BLOCKS * blk
    total += (BLOCKS // 2) * (g(T, 2 * D, D) + 4 * L * (L + T) * HD * HEADS)   # joint blocks
    total += (BLOCKS // 2) * 4 * L * L * HD * HEADS                              # image-only blocks
    txt = g(T, 3 * D, D) + g(T, D, D) + g(T, 2 * I_MLP, D) + g(T, D, I_MLP) + 4 * T * T * HD * HEADS + g(1, 6 * D, D)
    total += 2 * txt
    total += g(L, D, 64) + g(L, D, D) + g(L, 64, D)                              # s_embed, sprint, final
    # t_embedder (two), y_pool, the shared and final adaLN projections; the y_embedder projection
    # of the prompt (prepareText) runs outside the timed pass and is not counted
    total += g(1, D, 256) + g(1, D, D) * 2 + g(1, 6 * D, D) + g(1, 2 * D, D)
    return total


# ------------------------------------------------------------------------------ Node legs

def run_node(script, args, what, timeout=900):
    cmd = ["node", script] + args
    log(" ".join(cmd))
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if p.returncode != 0:
        sys.stderr.write(p.stderr[-3000:])
        raise SystemExit(f"{what} failed with {p.returncode}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def run_dit(steps, warmup):
    return run_node(RUN_DIT, ["--synthetic", "3", "--shape", f"{H_IMG},{W_IMG},{T_TXT}",
                              "--warmup", str(warmup), "--reps", str(steps)], "run_dit.js")


def write_lora(path, rank=32, seed=11):
    """A synthetic LoRA file of the reference's PEFT format: rank `rank` on every block linear of
    the pass (qkv_x, proj, w12 and w3 of the 18 blocks, kv_y of the 9 joint blocks: 81 modules),
    bf16 A/B with std 0.05, alpha = rank / 2."""
    import numpy as np
    import torch
    from safetensors.torch import save_file

    rng = np.random.default_rng(seed)
    mods = []
    for b in range(BLOCKS):
        mods += [(f"blocks.{b}.attn.qkv_x", 3 * D, D), (f"blocks.{b}.attn.proj", D, D),
                 (f"blocks.{b}.mlp.w12", 2 * I_MLP, D), (f"blocks.{b}.mlp.w3", D, I_MLP)]
        if b % 2 == 0:
            mods.append((f"blocks.{b}.attn.kv_y", 2 * D, D))
    out = {}
    for name, n_out, n_in in mods:
        base = "diffusion_model." + name
        out[base + ".lora_A.weight"] = torch.from_numpy(
            rng.standard_normal((rank, n_in), dtype=np.float32) * np.float32(0.05)).to(torch.bfloat16)
        out[base + ".lora_B.weight"] = torch.from_numpy(
            rng.standard_normal((n_out, rank), dtype=np.float32) * np.float32(0.05)).to(torch.bfloat16)
        out[base + ".alpha"] = torch.tensor(rank / 2.0, dtype=torch.float32)
    save_file(out, path)
    return len(mods)


def run_dit_lora(steps, warmup):
    """The same pass with a rank-32 LoRA on all 81 block linears (the side path of
    app/gpu/ops.js:70-87, attached as the pipeline attaches LoRA files)."""
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "lora_r32.safetensors")
        n = write_lora(path)
        r = run_node(RUN_DIT, ["--synthetic", "3", "--shape", f"{H_IMG},{W_IMG},{T_TXT}", "--warmup", str(warmup),
                               "--reps", str(steps), "--lora", path], "run_dit.js --lora")
    matched = sum(l["matched"] for l in r.get("loras", []))
    if matched != n:
        raise SystemExit(f"LoRA leg: {matched} of {n} modules matched")
    return {"workload": f"the pass with a rank-32 LoRA (PEFT names, strength 1) on all {n} block linears",
            "ms": r["ms_device_queued_per_pass"], "ms_single": r["ms_device_median"], "modules": n}


def run_dit_profile():
    r = run_node(RUN_DIT, ["--synthetic", "3", "--shape", f"{H_IMG},{W_IMG},{T_TXT}",
                           "--warmup", "1", "--reps", "2", "--profile"], "run_dit.js --profile")
    return r.get("profile", [])


def gemma_flops(L=GEMMA_TOKENS):
    """Algorithmic FLOPs of the 17-layer Gemma3-270M stack (app/models/gemma3.js:62-92):
    per layer q/k/v (1536 x 640), o (640 x 1024), gate/up (4096 x 640), down (640 x 2048), and
    4*L*L*256*4 for the attention (the causal mask not subtracted)."""
    per_layer = 2 * L * 640 * (1536 + 1024 + 4096 + 2048) + 4 * L * L * 256 * 4
    return GEMMA_LAYERS * per_layer


def run_gemma(steps, warmup, graph=False):
    r = run_node(RUN_GEMMA, ["--synthetic", "3", "--tokens", f"{GEMMA_TOKENS},1", "--warmup", str(warmup),
                             "--reps", str(steps)] + (["--graph"] if graph else []), "run_gemma.js", timeout=600)
    ms = r["ms_device_median"]
    fl = gemma_flops()
    return {"workload": f"Gemma3-270M text encoder, {GEMMA_LAYERS} layers + final norm, {GEMMA_TOKENS} tokens, "
                        "bf16 weights (fp16 matrix-core products, fp32 accumulation)",
            "ms": ms, "ms_wall": r["ms_wall_median"], "gflop": fl / 1e9,
            "tflops": fl / (ms / 1e3) / 1e12, "frac": fl / (ms / 1e3) / 1e12 / FP16_PEAK_TFLOPS,
            "ms_device": r["ms_device"]}


# int8 ConvRot linears of the pass (tiled GEMM launches), by the op names the DiT driver uses
GEMM_OPS = ("dit.qkv", "dit.proj", "dit.mlp.w12", "dit.mlp.w3", "dit.kv_y", "dit.text.qkv", "dit.text.proj")


def gemm_roofline(kernels):
    """Pass aggregate of the int8 GEMM launches: per-op rows and sum(2MNK) / sum(time)."""
    rows = [r for r in kernels if r["name"] in GEMM_OPS and r.get("tflops")]
    flop = sum(r["tflops"] * r["ms"] * 1e9 for r in rows)
    ms = sum(r["ms"] for r in rows)
    return {
        "ops": [{"name": r["name"], "launches_per_pass": r["count"], "ms_per_pass": r["ms"],
                 "tflops": r["tflops"]} for r in rows],
        "gflop_per_pass": flop / 1e9, "ms_per_pass": ms,
        "launches_per_pass": sum(r["count"] for r in rows),
        "tflops": flop / (ms / 1e3) / 1e12 if ms else None,
    }


# ------------------------------------------------------------------------------ C ABI legs

def timed(lib, call, reps, warmup):
    """Mean ms per call three ways, after at least `warmup` calls and one second of untimed calls
    (the clocks a busy GPU settles at): `graph_ms`, `reps` calls recorded as one HIP graph and
    replayed (the device time of the op without the host's launch gaps); `eager_ms`, `reps`
    back-to-back calls from Python (stream events around them); and the library profiler's mean
    ms per launch of each kernel, from a third run with the profiler's events around every
    launch. Returns (graph_ms, eager_ms, per-kernel profile)."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < 1.0:
        call()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    a, b = lib.event(), lib.event()
    lib.record(a)
    for _ in range(reps):
        call()
    lib.record(b)
    torch.cuda.synchronize()
    eager_ms = lib.elapsed_ms(a, b) / reps
    lib.graph_begin()
    for _ in range(reps):
        call()
    g = lib.graph_end()
    lib.graph_launch(g)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        lib.record(a)
        lib.graph_launch(g)
        lib.record(b)
        torch.cuda.synchronize()
        best = min(best, lib.elapsed_ms(a, b) / reps)
    lib.graph_destroy(g)
    lib.profile_reset()
    lib.profile(True)
    for _ in range(reps):
        call()
    torch.cuda.synchronize()
    prof = {k: {"count": v["count"], "ms": v["ms"] / max(1, v["count"])} for k, v in lib.profile_report().items()}
    lib.profile(False)
    return best, eager_ms, prof


def rope_table(h, w):
    """cos|sin table of the centred 2-D RoPE (app/models/common.js:28-43 layout)."""
    import math

    import torch

    half = HD // 2
    f = torch.tensor([float(torch.tensor(1.0 / math.pow(10000.0, float(torch.tensor(2.0 * i / half, dtype=torch.float32))),
                                         dtype=torch.float32)) for i in range(half // 2)], dtype=torch.float64)
    ys = torch.arange(h, dtype=torch.float64) - (h - 1) / 2
    xs = torch.arange(w, dtype=torch.float64) - (w - 1) / 2
    yy, xx = torch.meshgrid(ys, xs, indexing="ij")
    ang = torch.cat([torch.outer(xx.flatten(), f), torch.outer(yy.flatten(), f)], dim=-1).float().double()
    return torch.cat([ang.cos().reshape(-1), ang.sin().reshape(-1)]).float()


def attention_inputs(h, w, T, B, seed, device):
    import torch

    L = h * w
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, L, D, device=device, generator=g)
    k = torch.randn(B, L + T, D, device=device, generator=g)
    v = torch.randn(B, L + T, D, device=device, generator=g)
    bias = torch.log(torch.rand(B, T, device=device, generator=g) + 0.5)
    return q, k, v, bias


def bench_attention(lib, h, w, T, B, reps, warmup):
    """Joint attention (image + text keys) through ns2_attention: flash kernel and whole op."""
    import torch

    L = h * w
    Lk = L + T
    q, k, v, bias = attention_inputs(h, w, T, B, 2, "cuda")
    o = torch.empty(B, L, D, device="cuda")
    cs = rope_table(h, w).to("cuda")

    def call():
        lib.attention(q, k, v, o, Lq=L, Lk=Lk, H=HEADS, D=HD, ldq=D, ldk=D, ldv=D, ldo=D, batch=B,
                      qBatch=L * D, kBatch=Lk * D, vBatch=Lk * D, oBatch=L * D, key_bias=bias,
                      biasStart=L, biasBatch=T, rope_cs=cs, sin_off=L * HD // 2, rope_rows=L)

    total_ms, eager_ms, prof = timed(lib, call, reps, warmup)
    flops = 4 * L * Lk * HD * HEADS * B
    flash_ms = prof["attn_flash"]["ms"]
    pack_ms = prof["attn_pack"]["ms"]
    tf = lambda ms: flops / (ms / 1e3) / 1e12  # noqa: E731
    return {
        "config": f"{L} queries x {Lk} keys ({h}x{w} image + {T} text), {HEADS} heads x {HD}, batch {B}, "
                  "2-D RoPE on image rows, log-weight bias on text keys, fp32 in/out",
        "gflop": flops / 1e9,
        "ms": total_ms, "tflops": tf(total_ms), "frac": tf(total_ms) / FP16_PEAK_TFLOPS,
        "ms_eager": eager_ms, "ms_region": "ms: pack + flash, calls replayed as a HIP graph; ms_eager: "
                                           "the same calls launched from Python",
        "flash_ms": flash_ms, "flash_tflops": tf(flash_ms), "flash_frac": tf(flash_ms) / FP16_PEAK_TFLOPS,
        "pack_ms": pack_ms, "flops_per_launch": flops,
    }


def bench_linear_cfg1(lib, reps, warmup):
    """The int8 ConvRot linear at M = 2432 on fp32 activations: rotation into the tiled fp16
    operand (ns2_rotate_f16) + the tiled GEMM (ns2_linear_i8_tiled) on a weight re-tiled once."""
    import torch

    M = CFG1_M
    out = []
    g = torch.Generator(device="cuda").manual_seed(1)
    for name, N, K in CFG1_SHAPES:
        x = torch.randn(M, K, device="cuda", generator=g)
        q = torch.randint(-127, 128, (N, K), device="cuda", generator=g, dtype=torch.int32).to(torch.int8)
        s = torch.rand(N, device="cuda", generator=g) * 9e-3 + 1e-3
        wt = torch.empty(N * K, dtype=torch.int8, device="cuda")
        lib.tile_i8_weight(q, wt, N, K)
        at = torch.empty((M + 63) // 64 * 64, K, dtype=torch.int16, device="cuda")
        y = torch.empty(M, N, device="cuda")

        def call():
            lib.rotate_f16(x, K, at, K, M, K, tiled=True)
            lib.linear_i8_tiled(at, wt, s, y, M, N, K)

        total_ms, eager_ms, prof = timed(lib, call, reps, warmup)
        flops = 2 * M * N * K
        nbytes = N * K + 4 * N + 4 * M * K + 4 * M * N   # int8 W, scales, fp32 x in, fp32 y out
        gemm_ms, rot_ms = prof["gemm_i8_tiled"]["ms"], prof["rotate_f16"]["ms"]
        tf = lambda ms: flops / (ms / 1e3) / 1e12  # noqa: E731
        out.append({
            "shape": f"{name}: M {M} x N {N} x K {K}", "gflop": flops / 1e9, "algorithmic_mb": nbytes / 1e6,
            "ms": total_ms, "tflops": tf(total_ms), "frac": tf(total_ms) / FP16_PEAK_TFLOPS,
            "gbs": nbytes / (total_ms / 1e3) / 1e9, "ms_eager": eager_ms,
            "gemm_ms": gemm_ms, "gemm_tflops": tf(gemm_ms), "gemm_frac": tf(gemm_ms) / FP16_PEAK_TFLOPS,
            "rotate_ms": rot_ms, "rotate_gbs": M * K * 6 / (rot_ms / 1e3) / 1e9,
        })
        del x, q, s, wt, at, y
    return out


def bench_vendor(reps=20):
    """The vendor libraries at the same shapes, for scale: torch.matmul in fp16 (hipBLASLt) on the
    four block-linear shapes of the pass at 3952 rows (a plain GEMM on fp16 weights, without the
    int8 decode, rotation or epilogue of the DiT's linears), and torch's scaled_dot_product_attention
    (flash and memory-efficient backends) at the joint-attention shape in fp16 (no RoPE or key
    bias). Best of 5 runs of `reps` calls, timed with torch events."""
    import torch
    import torch.nn.functional as F

    def best_ms(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                fn()
            b.record()
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) / reps)
        return best

    M = H_IMG * W_IMG
    gemms = []
    for name, N, K in (("qkv", 3 * D, D), ("proj", D, D), ("w12", 2 * I_MLP, D), ("w3", D, I_MLP)):
        a = torch.randn(M, K, device="cuda", dtype=torch.float16)
        w = torch.randn(N, K, device="cuda", dtype=torch.float16)
        ms = best_ms(lambda: a @ w.t())
        gemms.append({"shape": f"{name}: M {M} x N {N} x K {K}", "ms": ms, "tflops": 2 * M * N * K / (ms / 1e3) / 1e12})
    B, Lq, Lk = 2, M, M + T_TXT
    q = torch.randn(B, HEADS, Lq, HD, device="cuda", dtype=torch.float16)
    k = torch.randn(B, HEADS, Lk, HD, device="cuda", dtype=torch.float16)
    v = torch.randn(B, HEADS, Lk, HD, device="cuda", dtype=torch.float16)
    sdpa = {}
    from torch.nn.attention import SDPBackend, sdpa_kernel

    for be in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel([be]):
                ms = best_ms(lambda: F.scaled_dot_product_attention(q, k, v))
            sdpa[be.name.lower()] = {"ms": ms, "tflops": 4 * B * HEADS * Lq * Lk * HD / (ms / 1e3) / 1e12}
        except RuntimeError as e:  # backend not built into this torch
            sdpa[be.name.lower()] = {"unavailable": str(e)[:200]}
    return {"hipblaslt_fp16_matmul": gemms,
            "torch_sdpa_fp16": dict(sdpa, config=f"{Lq} queries x {Lk} keys, {HEADS} heads x {HD}, batch {B}")}


def copy_calibration(lib, n=64 << 20, reps=3):
    """ns2_elementwise copy of n fp32 values: 4n bytes read + 4n bytes written per launch,
    the known-size kernel that HBM byte counters are scaled against."""
    import torch

    a = torch.ones(n, device="cuda")
    b = torch.empty(n, device="cuda")
    for _ in range(reps):
        lib.elementwise("copy", a, None, b, n)
    torch.cuda.synchronize()
    return {"kernel": "elementwise_kernel (copy)", "bytes_read": 4 * n, "bytes_written": 4 * n, "launches": reps}


# ------------------------------------------------------------------------------ CPU legs

def cpu_time(fn, max_reps=3, long_s=3.0):
    """1 untimed warm-up call, then up to max_reps timed calls (1 when a call takes longer than
    long_s); returns the median in ms and the repetitions."""
    fn()
    times = []
    for _ in range(max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if times[0] > long_s:
            break
    return statistics.median(times) * 1e3, len(times)


def cpu_attention(h, w, T, B):
    import torch

    import oracle.nanosaur2_oracle as O

    L = h * w
    q, k, v, bias = attention_inputs(h, w, T, B, 2, "cpu")
    cos, sin = O.rope_2d(h, w)

    def run():
        with torch.no_grad():
            for b in range(B):
                O.joint_attention_op(q[b], k[b], v[b], L, cos, sin, key_bias=bias[b], bias_start=L)

    ms, n = cpu_time(run)
    flops = 4 * L * (L + T) * HD * HEADS * B
    return {"value": ms, "unit": "ms per call", "tflops": flops / (ms / 1e3) / 1e12, "reps": n,
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"the whole op (RoPE, bias, softmax(QK^T/sqrt(96))V), fp32 PyTorch CPU, batch {B}"}


def cpu_linear_cfg1():
    import torch

    import oracle.nanosaur2_oracle as O

    g = torch.Generator().manual_seed(1)
    rows = []
    for name, N, K in CFG1_SHAPES:
        x = torch.randn(CFG1_M, K, generator=g)
        q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int32).to(torch.int8)
        s = torch.rand(N, 1, generator=g) * 9e-3 + 1e-3
        with torch.no_grad():
            ms, n = cpu_time(lambda: O.linear_i8(x, q, s))
        rows.append({"shape": name, "ms": ms, "tflops": 2 * CFG1_M * N * K / (ms / 1e3) / 1e12, "reps": n})
    return {"rows": rows, "unit": "ms per linear", "cores": torch.get_num_threads(), "kind": "port",
            "sample": "ops.linear on the int8 weight: rotation of x per 256-group, x_r q^T, row scale; fp32 PyTorch CPU"}


def cpu_gemma():
    """The oracle's Gemma3 encode of 256 tokens on seeded weights of the real architecture; the
    embedding table holds 4096 rows (the gather is a negligible share of the work)."""
    import torch

    import oracle.nanosaur2_oracle as O

    g = torch.Generator().manual_seed(4)
    t = {"model.embed_tokens.weight": torch.randn(4096, 640, generator=g).to(torch.bfloat16)}
    shapes = {"self_attn.q_proj.weight": (1024, 640), "self_attn.k_proj.weight": (256, 640),
              "self_attn.v_proj.weight": (256, 640), "self_attn.o_proj.weight": (640, 1024),
              "mlp.gate_proj.weight": (2048, 640), "mlp.up_proj.weight": (2048, 640),
              "mlp.down_proj.weight": (640, 2048)}
    for i in range(GEMMA_LAYERS):
        p = f"model.layers.{i}."
        for n, shp in shapes.items():
            t[p + n] = (torch.randn(*shp, generator=g) * 0.02).to(torch.bfloat16)
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                  "post_feedforward_layernorm"):
            t[p + n + ".weight"] = (torch.randn(640, generator=g) * 0.1).to(torch.bfloat16)
        t[p + "self_attn.q_norm.weight"] = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16)
        t[p + "self_attn.k_norm.weight"] = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16)
    t["model.norm.weight"] = (torch.randn(640, generator=g) * 0.1).to(torch.bfloat16)
    W = O.TensorWeights(t)
    ids = torch.randint(0, 4096, (GEMMA_TOKENS,), generator=g).tolist()
    with torch.no_grad():
        ms, n = cpu_time(lambda: O.gemma_encode(W, ids))
    return {"value": ms, "unit": "ms per encode", "tflops": gemma_flops() / (ms / 1e3) / 1e12, "reps": n,
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{GEMMA_LAYERS} layers + final norm, {GEMMA_TOKENS} tokens, fp32 PyTorch CPU"}


def cpu_dit_pass():
    """Oracle (PyTorch CPU, fp32) on one joint and one image-only block at full size."""
    import torch

    import oracle.nanosaur2_oracle as O

    L, T = H_IMG * W_IMG, T_TXT
    gen = torch.Generator().manual_seed(5)
    t = {}

    def i8(name, N, K):
        t[name + ".weight"] = torch.randint(-127, 128, (N, K), generator=gen, dtype=torch.int32).to(torch.int8)
        t[name + ".weight_scale"] = torch.rand(N, 1, generator=gen) * 9e-3 + 1e-3

    def vec(name, n):
        t[name] = (torch.randn(n, generator=gen) * 0.02).to(torch.bfloat16)

    for i in (0, 1):
        p = f"blocks.{i}."
        vec(f"encoder_adaLN_offsets.{i}", 6 * D)
        vec(p + "norm1.weight", D)
        vec(p + "norm2.weight", D)
        i8(p + "attn.qkv_x", 3 * D, D)
        if i == 0:
            i8(p + "attn.kv_y", 2 * D, D)
        vec(p + "attn.q_norm.weight", HD)
        vec(p + "attn.k_norm.weight", HD)
        i8(p + "attn.proj", D, D)
        i8(p + "mlp.w12", 2 * I_MLP, D)
        i8(p + "mlp.w3", D, I_MLP)
    W = O.TensorWeights(t)
    dit = O.DiT(W)
    x = torch.randn(L, D, generator=gen)
    txt = torch.randn(T, D, generator=gen)
    mod = torch.randn(1, 6 * D, generator=gen) * 0.02
    tb = torch.log(torch.rand(T, generator=gen) + 0.5)
    cos, sin = O.rope_2d(H_IMG, W_IMG)
    with torch.no_grad():
        for name in list(t):
            if name.endswith(".weight"):
                W(name)  # dequantize once (weights are loaded before the pass in the reference too)
        times = []
        for i in (0, 1):
            dit.block(i, x, txt, cos, sin, mod, tb)  # untimed: thread-pool and allocator warmup
            t0 = time.perf_counter()
            dit.block(i, x, txt, cos, sin, mod, tb)
            times.append(time.perf_counter() - t0)
    per_pass_ms = (BLOCKS // 2) * (times[0] + times[1]) * 1e3
    return {
        "value": per_pass_ms,
        "unit": "ms per DiT pass",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle block 0 (joint, {L}+{T} keys: {times[0]*1e3:.0f} ms) and block 1 (image-only: "
                  f"{times[1]*1e3:.0f} ms) at 3952 tokens, fp32 PyTorch CPU, x9 each for 18 blocks "
                  "(conditioning, embeddings and final layer, <1% of the FLOPs, not included)",
        "cpu": cpu_model(),
    }


# ------------------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-dit", action="store_true", help="skip the DiT pass (kernels and CPU legs only)")
    ap.add_argument("--no-gemma", action="store_true", help="skip the text-encoder measurement")
    ap.add_argument("--no-vendor", action="store_true", help="skip the hipBLASLt / SDPA reference timings")
    ap.add_argument("--no-lora", action="store_true", help="skip the pass with a rank-32 LoRA on every block linear")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 256 MiB -> 256 MiB copy kernel (reference point for HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    flops = pass_flops()
    dit, kernels, gemm = None, None, None
    if not args.no_dit:
        # the Node runs come first, before this process initialises the GPU
        dit = run_dit(args.steps, args.warmup)
        kernels = run_dit_profile()
        gemm = gemm_roofline(kernels)
        log(f"DiT pass {dit['ms_device_queued_per_pass']:.3f} ms ({args.steps} passes back to back; one at a "
            f"time {dit['ms_device_median']:.3f} ms); int8 GEMMs {gemm['ms_per_pass']:.3f} ms/pass, "
            f"{gemm['tflops']:.1f} TFLOP/s")
    dit_lora = None
    if not args.no_dit and not args.no_lora:
        dit_lora = run_dit_lora(args.steps, args.warmup)
        # both legs timed the same way (back-to-back passes, whole run / K)
        dit_lora["overhead_ms"] = dit_lora["ms"] - dit["ms_device_queued_per_pass"]
        log(f"DiT pass with LoRA {dit_lora['ms']:.3f} ms (+{dit_lora['overhead_ms']:.3f} ms)")
    gemma = None
    if not args.no_gemma:
        gemma = run_gemma(max(10, args.steps), max(3, args.warmup))
        # the same encode recorded once as a HIP graph and replayed (GPU.capture)
        replay = run_gemma(max(10, args.steps), max(3, args.warmup), graph=True)
        gemma["ms_graph"], gemma["ms_graph_wall"] = replay["ms"], replay["ms_wall"]
        log(f"text encoder: {gemma['ms']:.3f} ms per {GEMMA_TOKENS}-token encode, {gemma['tflops']:.1f} TFLOP/s "
            f"(graph replay {gemma['ms_graph']:.3f} ms)")

    import torch

    sys.path.insert(0, PKG)
    import ns2

    # the legs run on a stream of their own (default priority): a HIP graph cannot record the
    # null stream; torch's allocations and fills of the legs go to the same stream
    leg_stream = torch.cuda.Stream()
    torch.cuda.set_stream(leg_stream)
    lib = ns2.load(0, leg_stream.cuda_stream)
    reps = max(10, args.steps)
    attn = bench_attention(lib, H_IMG, W_IMG, T_TXT, 2, reps, max(2, args.warmup))
    log(f"attention 3952x4208 b2: {attn['ms']:.3f} ms/call, flash {attn['flash_ms']:.3f} ms "
        f"({attn['flash_tflops']:.1f} TFLOP/s)")
    attn0 = bench_attention(lib, 48, 48, 128, 1, reps, max(2, args.warmup))
    log(f"attention 2304x2432: {attn0['ms']:.3f} ms/call, flash {attn0['flash_tflops']:.1f} TFLOP/s")
    lin1 = bench_linear_cfg1(lib, reps, max(2, args.warmup))
    for r in lin1:
        log(f"linear {r['shape']}: {r['ms'] * 1e3:.1f} us ({r['tflops']:.0f} TFLOP/s with rotation, "
            f"GEMM {r['gemm_tflops']:.0f})")
    if args.copy_calibration:
        attn["copy_calibration"] = copy_calibration(lib)
    vendor = None
    if not args.no_vendor:
        vendor = bench_vendor()
        log("vendor: hipBLASLt fp16 " + ", ".join(f"{g['shape'].split(':')[0]} {g['tflops']:.0f}"
                                                   for g in vendor["hipblaslt_fp16_matmul"]) + " TFLOP/s; SDPA "
            + ", ".join(f"{k} {v['ms'] * 1e3:.0f} us" for k, v in vendor["torch_sdpa_fp16"].items() if "ms" in v))

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, ROOT)
        torch.set_num_threads(cpu_threads())
        log(f"CPU baselines on {torch.get_num_threads()} threads ({cpu_model()})")
        cpu = cpu_dit_pass()
        attn["cpu_baseline"] = cpu_attention(H_IMG, W_IMG, T_TXT, 2)
        attn0["cpu_baseline"] = cpu_attention(48, 48, 128, 1)
        lin1_cpu = cpu_linear_cfg1()
        for r, c in zip(lin1, lin1_cpu["rows"]):
            r["cpu_ms"], r["cpu_tflops"] = c["ms"], c["tflops"]
        lin1_meta = {k: v for k, v in lin1_cpu.items() if k != "rows"}
        if gemma:
            gemma["cpu_baseline"] = cpu_gemma()
    else:
        lin1_meta = None

    ms = dit["ms_device_queued_per_pass"] if dit else None
    out = {
        "metric": METRIC,
        "value": ms,
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": (ms / PUBLISHED_PASS_MS) if ms else None,
        "dtype": "fp16",
        "data": "synthetic (seeded random-init weights of the real architecture; N(0,1) latent/context)",
        "config": {
            "workload": "one Nanosaur2 DiT pass at 832x1216: 76x52 latent = 3952 image tokens + 256 text tokens, "
                        "18 blocks (9 joint, 9 image-only), dim 1536, 16 heads x 96, MLP 4096, int8 ConvRot "
                        "block linears, batch 1",
            "tokens": H_IMG * W_IMG, "text_tokens": T_TXT, "blocks": BLOCKS, "parallelism": "none (1 GPU)",
        },
        "value_region": "K passes issued back to back on one stream after W warm-up passes, timed with stream "
                        "events from the first pass's start to the last pass's end and divided by K; each pass "
                        "runs from the latent tokens resident in HBM to the x0 tokens in HBM, including "
                        "condition() and the text refine; the reference's pass time also includes the latent "
                        "upload and x0 readback, reported here as pass_ms_host_to_host",
        "pass_tflop": flops / 1e12,
        "pass_tflops": (flops / (ms / 1e3) / 1e12) if ms else None,
        "pass_ms_wall": dit["ms_wall_median"] if dit else None,
        # one pass at a time, each bracketed by events and followed by a device sync (the median):
        # each pass then starts on an idle device and pays the host's launch latency
        "pass_ms_single": dit["ms_device_median"] if dit else None,
        # the median of the back-to-back passes' own event pairs
        "pass_ms_queued_median": dit.get("ms_device_queued_median") if dit else None,
        "pass_ms_host_to_host": dit["ms_host_to_host_median"] if dit else None,
        "weight_bytes": dit.get("weight_bytes") if dit else None,
        "dit_lora": dit_lora,
        "joint_attention": attn,
        "joint_attention_768": attn0,
        "linear_int8_m2432": {"rows": lin1, "cpu_baseline": lin1_meta},
        "text_encoder": gemma,
        "gemm_i8": gemm,
        "roofline": {
            "kernel": "gemm_tiled_kernel (int8 ConvRot block linears of one pass: qkv, proj, w12, w3, kv_y)",
            "bound": "mfma",
            "achieved": gemm["tflops"] if gemm else None,
            "peak": FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm["tflops"] / FP16_PEAK_TFLOPS if gemm and gemm["tflops"] else None,
            "traffic": GEMM_TRAFFIC_BYTES_PER_LAUNCH,
            "traffic_algorithmic": GEMM_ALGORITHMIC_BYTES_PER_LAUNCH,
            "traffic_source": GEMM_TRAFFIC_SOURCE,
        },
        "roofline_attention": {
            "kernel": "flash_wide_kernel (joint attention, 3952x4208, batch 2: 512-query blocks)",
            "bound": "mfma",
            "achieved": attn["flash_tflops"],
            "peak": FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": attn["flash_frac"],
            "whole_op_frac": attn["frac"],
            "traffic": ATTN_TRAFFIC_BYTES_PER_LAUNCH,
            "traffic_algorithmic": ATTN_ALGORITHMIC_BYTES_PER_LAUNCH,
            "traffic_source": ATTN_TRAFFIC_SOURCE,
        },
        "cpu_baseline": cpu,
        "vendor_reference": vendor,
        "kernels": kernels,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
