#!/usr/bin/env python3
"""Benchmark: ms per 832x1216 int8 DiT pass + joint-attention TFLOP/s on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-dit]

1. DiT pass (the metric): the Node host (nanosaur2-web_amd/js/run_dit.js) runs one full pass
   of the 18-block Nanosaur2 DiT at 832x1216 (latent 76 rows x 52 cols = 3952 image tokens,
   256 text tokens, batch 1) on seeded random-init weights of the real architecture (int8
   ConvRot block linears, bf16 elsewhere). W untimed passes, then K timed passes with the
   latent tokens resident in device memory, bracketed by stream events and a device sync.
   `value` is the median device time per pass in ms.
   The dominant kernel of the pass is the tiled int8 ConvRot GEMM (qkv, proj, w12, w3, kv_y of
   every block): a profiled run of the same pass times every launch with stream events on the
   library's stream, and `roofline` is its algorithmic 2*M*N*K flops summed over the pass /
   its summed launch time, against the 2516.6 TFLOP/s dense fp16 MFMA peak.
2. Joint attention at the production shape (3952 queries x 4208 keys, 16 heads x 96, batch 2,
   2-D RoPE on image rows, log-weight bias on the text keys) through the C ABI (ctypes);
   the library's kernel profiler times each launch of the flash kernel with stream events,
   which gives `roofline_attention` (algorithmic 4*Lq*Lk*D*H*B flops per launch / mean launch
   time).
3. Gemma3-270M text encoder (17 of 18 layers + final norm, 256 token ids, random-init bf16
   weights of the real architecture) through the Node host (run_gemma.js): median device time
   per encode, with the algorithmic flops of its linears (2*M*N*K) and attention (4*L*L*256*4);
   `ms_graph` is the same encode recorded once as a HIP graph and replayed.
4. CPU baseline: the oracle (a PyTorch-CPU restatement of tools/reference.py) on a bounded
   sample -- one joint block and one image-only block at the full 3952-token shape -- scaled
   to 18 blocks, on this host's cores.
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
H_IMG, W_IMG, T_TXT, D, HEADS, HD, I_MLP, BLOCKS = 76, 52, 256, 1536, 16, 96, 4096, 18
# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, each scaled by what the
# counter reads for a copy kernel of known size (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0), measured on
# the current kernels (profiles/): the mean over the pass's 89 tiled-GEMM launches, and one flash
# launch at the joint shape. Beside each, the algorithmic bytes of the same launches.
GEMM_TRAFFIC_BYTES_PER_LAUNCH = 148.2e6
GEMM_ALGORITHMIC_BYTES_PER_LAUNCH = 67.5e6   # N*K int8 W + 2*M*K fp16 A + output (+ old output for +=)
ATTN_TRAFFIC_BYTES_PER_LAUNCH = 173.9e6
ATTN_ALGORITHMIC_BYTES_PER_LAUNCH = 149.1e6  # fp32 Q (read in the kernel's prologue), fp16 K, V^T, fp32 O


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


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
    total += g(T, D, 640) + g(1, D, 256) + g(1, D, D) * 2 + g(1, 6 * D, D) + g(1, 2 * D, D)
    return total


def run_dit(steps, warmup):
    cmd = ["node", RUN_DIT, "--synthetic", "3", "--shape", f"{H_IMG},{W_IMG},{T_TXT}",
           "--warmup", str(warmup), "--reps", str(steps)]
    log(" ".join(cmd))
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    sys.stderr.write(p.stderr[-3000:])
    if p.returncode != 0:
        raise SystemExit(f"run_dit.js failed with {p.returncode}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def run_dit_profile():
    cmd = ["node", RUN_DIT, "--synthetic", "3", "--shape", f"{H_IMG},{W_IMG},{T_TXT}",
           "--warmup", "1", "--reps", "2", "--profile"]
    log(" ".join(cmd))
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if p.returncode != 0:
        sys.stderr.write(p.stderr[-3000:])
        raise SystemExit(f"run_dit.js --profile failed with {p.returncode}")
    return json.loads(p.stdout.strip().splitlines()[-1]).get("profile", [])


def gemma_flops(L=GEMMA_TOKENS):
    """Algorithmic FLOPs of the 17-layer Gemma3-270M stack (app/models/gemma3.js:62-92):
    per layer q/k/v (1536 x 640), o (640 x 1024), gate/up (4096 x 640), down (640 x 2048), and
    4*L*L*256*4 for the attention (the causal mask not subtracted)."""
    per_layer = 2 * L * 640 * (1536 + 1024 + 4096 + 2048) + 4 * L * L * 256 * 4
    return GEMMA_LAYERS * per_layer


def run_gemma(steps, warmup, graph=False):
    cmd = ["node", RUN_GEMMA, "--synthetic", "3", "--tokens", f"{GEMMA_TOKENS},1",
           "--warmup", str(warmup), "--reps", str(steps)] + (["--graph"] if graph else [])
    log(" ".join(cmd))
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if p.returncode != 0:
        sys.stderr.write(p.stderr[-3000:])
        raise SystemExit(f"run_gemma.js failed with {p.returncode}")
    r = json.loads(p.stdout.strip().splitlines()[-1])
    ms = r["ms_device_median"]
    fl = gemma_flops()
    return {"workload": f"Gemma3-270M text encoder, {GEMMA_LAYERS} layers + final norm, {GEMMA_TOKENS} tokens, "
                        "bf16 weights (fp16 matrix-core products, fp32 accumulation)",
            "ms": ms, "ms_wall": r["ms_wall_median"], "gflop": fl / 1e9,
            "tflops": fl / (ms / 1e3) / 1e12, "ms_device": r["ms_device"]}


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


def bench_attention(reps, warmup):
    """Joint attention at the production shape, batch 2 (cond + uncond)."""
    import torch

    sys.path.insert(0, PKG)
    import ns2

    lib = ns2.load(0, torch.cuda.current_stream().cuda_stream)
    dev = "cuda"
    L, B = H_IMG * W_IMG, 2
    Lk = L + T_TXT
    g = torch.Generator(device=dev).manual_seed(2)
    q = torch.randn(B, L, D, device=dev, generator=g)
    k = torch.randn(B, Lk, D, device=dev, generator=g)
    v = torch.randn(B, Lk, D, device=dev, generator=g)
    bias = torch.log(torch.rand(B, T_TXT, device=dev, generator=g) + 0.5)
    o = torch.empty(B, L, D, device=dev)
    cs = rope_table(H_IMG, W_IMG).to(dev)
    sin_off = L * HD // 2

    def call():
        lib.attention(q, k, v, o, Lq=L, Lk=Lk, H=HEADS, D=HD, ldq=D, ldk=D, ldv=D, ldo=D, batch=B,
                      qBatch=L * D, kBatch=Lk * D, vBatch=Lk * D, oBatch=L * D, key_bias=bias,
                      biasStart=L, biasBatch=T_TXT, rope_cs=cs, sin_off=sin_off, rope_rows=L)

    # untimed warmup: at least `warmup` calls and one second of back-to-back launches, so the
    # timed calls run at the clocks a busy GPU settles at (this leg starts in a fresh process
    # after the GPU has idled)
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < 1.0:
        call()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    lib.profile_reset()
    lib.profile(True)
    a, b = lib.event(), lib.event()
    lib.record(a)
    for _ in range(reps):
        call()
    lib.record(b)
    torch.cuda.synchronize()
    total_ms = lib.elapsed_ms(a, b) / reps
    prof = lib.profile_report()
    lib.profile(False)
    flops = 4 * L * Lk * HD * HEADS * B
    flash = prof.get("attn_flash", {"count": 0, "ms": 0})
    pack = prof.get("attn_pack", {"count": 0, "ms": 0})
    flash_ms = flash["ms"] / max(1, flash["count"])
    pack_ms = pack["ms"] / max(1, pack["count"])
    return {
        "config": f"{L} queries x {Lk} keys ({L} image + {T_TXT} text), {HEADS} heads x {HD}, batch {B}, "
                  "2-D RoPE on image rows, log-weight bias on text keys, fp32 in/out",
        "gflop": flops / 1e9,
        "ms": total_ms,
        "tflops": flops / (total_ms / 1e3) / 1e12,
        "flash_ms": flash_ms,
        "flash_tflops": flops / (flash_ms / 1e3) / 1e12 if flash_ms else None,
        "pack_ms": pack_ms,
        "launches": flash["count"],
        "flops_per_launch": flops,
    }


def copy_calibration(n=64 << 20, reps=3):
    """ns2_elementwise copy of n fp32 values: 4n bytes read + 4n bytes written per launch,
    the known-size kernel that HBM byte counters are scaled against."""
    import torch

    import ns2

    lib = ns2.load(0)
    a = torch.ones(n, device="cuda")
    b = torch.empty(n, device="cuda")
    for _ in range(reps):
        lib.elementwise("copy", a, None, b, n)
    torch.cuda.synchronize()
    return {"kernel": "elementwise_kernel (copy)", "bytes_read": 4 * n, "bytes_written": 4 * n, "launches": reps}


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


def cpu_baseline():
    """Oracle (PyTorch CPU, fp32) on one joint and one image-only block at full size."""
    import torch

    sys.path.insert(0, ROOT)
    import oracle.nanosaur2_oracle as O

    torch.manual_seed(0)
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
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


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-dit", action="store_true", help="only the joint-attention measurement")
    ap.add_argument("--no-gemma", action="store_true", help="skip the text-encoder measurement")
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
        log(f"int8 GEMMs: {gemm['ms_per_pass']:.3f} ms/pass, {gemm['tflops']:.1f} TFLOP/s")
    gemma = None
    if not args.no_gemma:
        gemma = run_gemma(max(10, args.steps), max(3, args.warmup))
        # the same encode recorded once as a HIP graph and replayed (GPU.capture)
        replay = run_gemma(max(10, args.steps), max(3, args.warmup), graph=True)
        gemma["ms_graph"], gemma["ms_graph_wall"] = replay["ms"], replay["ms_wall"]
        log(f"text encoder: {gemma['ms']:.3f} ms per {GEMMA_TOKENS}-token encode, {gemma['tflops']:.1f} TFLOP/s "
            f"(graph replay {gemma['ms_graph']:.3f} ms)")
    attn = bench_attention(reps=max(10, args.steps), warmup=max(2, args.warmup))
    if args.copy_calibration:
        attn["copy_calibration"] = copy_calibration()
    log(f"attention: {attn['ms']:.3f} ms/call, flash {attn['flash_ms']:.3f} ms ({attn['flash_tflops']:.1f} TFLOP/s)")
    cpu = None if args.no_cpu else cpu_baseline()

    ms = dit["ms_device_median"] if dit else None
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
        "pass_tflop": flops / 1e12,
        "pass_tflops": (flops / (ms / 1e3) / 1e12) if ms else None,
        "pass_ms_wall": dit["ms_wall_median"] if dit else None,
        "pass_ms_host_to_host": dit["ms_host_to_host_median"] if dit else None,
        "joint_attention": attn,
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
        },
        "roofline_attention": {
            "kernel": "flash_kernel (joint attention, 3952x4208, batch 2)",
            "bound": "mfma",
            "achieved": attn["flash_tflops"],
            "peak": FP16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": attn["flash_tflops"] / FP16_PEAK_TFLOPS if attn["flash_tflops"] else None,
            "traffic": ATTN_TRAFFIC_BYTES_PER_LAUNCH,
            "traffic_algorithmic": ATTN_ALGORITHMIC_BYTES_PER_LAUNCH,
        },
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
