"""Seeded DiT weights and inputs for full-pass tests, and a runner for the Node host.

Weights follow the real Nanosaur2 DiT architecture (D=1536, 18 blocks, 2 text-refine blocks,
MLP width I) and the reference's int8 file layout (tools/build_assets.py:35-56,
tools/quant.py:43-56): ConvRot linears as `weight` I8 [N,K] + `weight_scale` F32 [N,1] +
`comfy_quant` U8 JSON; every other tensor bf16. Values: int8 ~ U{-127..127}, scales ~
U[1e-3, 1e-2], bf16 tensors ~ N(0, 0.02), from numpy's PCG64 with a fixed seed.
"""

from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUN_DIT = os.path.join(ROOT, "nanosaur2-web_amd", "js", "run_dit.js")
D = 1536


def dit_spec(I=4096, blocks=18, text_blocks=2, ctx=640):
    """name -> (shape, kind) with kind in {"i8", "bf16"} (vectors are bf16 too)."""
    s = {}
    s["s_embedder.proj.weight"] = ((D, 64), "bf16")
    s["t_embedder.mlp.0.weight"] = ((D, 256), "bf16")
    s["t_embedder.mlp.2.weight"] = ((D, D), "bf16")
    s["y_embedder.proj.weight"] = ((D, ctx), "bf16")
    s["y_embedder.norm.weight"] = ((D,), "bf16")
    s["y_pool_proj.weight"] = ((D, D), "bf16")
    s["shared_encoder_adaLN.0.weight"] = ((6 * D, D), "bf16")
    s["sprint_out_proj.weight"] = ((D, D), "bf16")
    for i in range(text_blocks):
        p = f"text_refine_blocks.{i}."
        s[p + "adaLN_modulation.0.weight"] = ((6 * D, D), "bf16")
        s[p + "norm1.weight"] = ((D,), "bf16")
        s[p + "norm2.weight"] = ((D,), "bf16")
        s[p + "attn.qkv.weight"] = ((3 * D, D), "i8")
        s[p + "attn.q_norm.weight"] = ((96,), "bf16")
        s[p + "attn.k_norm.weight"] = ((96,), "bf16")
        s[p + "attn.proj.weight"] = ((D, D), "i8")
        s[p + "mlp.w12.weight"] = ((2 * I, D), "i8")
        s[p + "mlp.w3.weight"] = ((D, I), "i8")
    for i in range(blocks):
        p = f"blocks.{i}."
        s[f"encoder_adaLN_offsets.{i}"] = ((6 * D,), "bf16")
        s[p + "norm1.weight"] = ((D,), "bf16")
        s[p + "norm2.weight"] = ((D,), "bf16")
        s[p + "attn.qkv_x.weight"] = ((3 * D, D), "i8")
        if i % 2 == 0:
            s[p + "attn.kv_y.weight"] = ((2 * D, D), "i8")
        s[p + "attn.q_norm.weight"] = ((96,), "bf16")
        s[p + "attn.k_norm.weight"] = ((96,), "bf16")
        s[p + "attn.proj.weight"] = ((D, D), "i8")
        s[p + "mlp.w12.weight"] = ((2 * I, D), "i8")
        s[p + "mlp.w3.weight"] = ((D, I), "i8")
    s["final_layer.adaLN_modulation.weight"] = ((2 * D, D), "bf16")
    s["final_layer.linear.weight"] = ((64, D), "bf16")
    return s


COMFY_QUANT = json.dumps({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 256}).encode()


def make_weights(seed=3, **spec_kw):
    """name -> torch tensor in the on-disk layout (int8 / float32 scale / uint8 meta / bf16)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, (shape, kind) in dit_spec(**spec_kw).items():
        if kind == "i8":
            base = name[: -len("weight")]
            out[name] = torch.from_numpy(rng.integers(-127, 128, size=shape, dtype=np.int8))
            out[base + "weight_scale"] = torch.from_numpy(rng.uniform(1e-3, 1e-2, size=(shape[0], 1)).astype(np.float32))
            out[base + "comfy_quant"] = torch.tensor(list(COMFY_QUANT), dtype=torch.uint8)
        else:
            v = rng.standard_normal(size=shape, dtype=np.float32) * np.float32(0.02)
            out[name] = torch.from_numpy(v).to(torch.bfloat16)
    return out


def save_weights(tensors, path):
    from safetensors.torch import save_file

    save_file(tensors, path, metadata={"quant": "int8"})


def make_inputs(h, w, T, seed=7, zero_weight_tokens=()):
    rng = np.random.default_rng(seed)
    latent = rng.standard_normal((64, h, w), dtype=np.float32)
    context = rng.standard_normal((T, 640), dtype=np.float32)
    weights = rng.uniform(0.5, 1.5, size=T).astype(np.float32)
    for i in zero_weight_tokens:
        weights[i] = 0.0
    sigma = float(rng.uniform(0.0, 1.0))
    return {"h": h, "w": w, "T": T, "sigma": sigma, "latent": latent, "context": context, "weights": weights}


def write_inputs(inp, d):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "inputs.json"), "w") as f:
        json.dump({k: inp[k] for k in ("h", "w", "T", "sigma")}, f)
    inp["latent"].astype(np.float32).tofile(os.path.join(d, "latent.f32"))
    inp["context"].astype(np.float32).tofile(os.path.join(d, "context.f32"))
    inp["weights"].astype(np.float32).tofile(os.path.join(d, "weights.f32"))


def lora_targets(I=4096):
    """LoRA test targets: (module, out features, in features, rank, naming). They cover every
    kind of linear launch of the pass: int8 tiled (qkv_x, kv_y, proj, w3), the fused w12 + GLU +
    rotation launch, an int8 text-refine linear, and bf16 GEMV / GEMM linears; one module uses
    kohya naming, the others PEFT naming."""
    return [
        ("blocks.0.attn.qkv_x", 3 * D, D, 8, "peft"),
        ("blocks.0.attn.kv_y", 2 * D, D, 4, "peft"),
        ("blocks.1.mlp.w12", 2 * I, D, 16, "peft"),
        ("blocks.2.attn.proj", D, D, 4, "peft"),
        ("blocks.3.mlp.w3", D, I, 8, "kohya"),
        ("text_refine_blocks.0.attn.qkv", 3 * D, D, 8, "peft"),
        ("t_embedder.mlp.0", D, 256, 4, "peft"),
        ("final_layer.linear", 64, D, 4, "peft"),
    ]


def joint_kv_targets(r=32, blocks=18):
    """A rank-r LoRA on the text k|v projection (kv_y) of every joint block (the even blocks)."""
    return [(f"blocks.{i}.attn.kv_y", 2 * D, D, r, "peft") for i in range(0, blocks, 2)]


def make_lora(seed=9, I=4096, a_std=0.05, b_std=0.05, targets=None):
    """A LoRA file's tensors (bf16 A/B, fp32 alpha = rank / 2) for targets (lora_targets(I) by
    default), seeded."""
    rng = np.random.default_rng(seed)
    out = {}
    for module, n_out, n_in, r, naming in (targets or lora_targets(I)):
        A = torch.from_numpy(rng.standard_normal((r, n_in), dtype=np.float32) * np.float32(a_std)).to(torch.bfloat16)
        B = torch.from_numpy(rng.standard_normal((n_out, r), dtype=np.float32) * np.float32(b_std)).to(torch.bfloat16)
        alpha = torch.tensor(r / 2.0, dtype=torch.float32)
        if naming == "peft":
            base = "diffusion_model." + module
            out[base + ".lora_A.weight"], out[base + ".lora_B.weight"], out[base + ".alpha"] = A, B, alpha
        else:
            base = "lora_unet_" + module.replace(".", "_")
            out[base + ".lora_down.weight"], out[base + ".lora_up.weight"], out[base + ".alpha"] = A, B, alpha
    return out


def run_node(args, timeout=600):
    """Run the Node host's run_dit.js; returns its JSON report. Fails loudly on error."""
    cmd = ["node", RUN_DIT, *args]
    print("[node]", " ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if p.returncode != 0:
        raise RuntimeError(f"run_dit.js failed ({p.returncode}):\n{p.stderr[-4000:]}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def oracle_forward(tensors, inp, path_drop=False, dtype=torch.float32, loras=()):
    """x0 [64, h, w] from the oracle's restatement of tools/reference.py DiT.forward; loras:
    (LoRA tensor dict, strength) pairs merged into the weights."""
    import oracle.nanosaur2_oracle as O

    W = O.TensorWeights(tensors, dtype, loras)
    dit = O.DiT(W)
    with torch.no_grad():
        return dit.forward(torch.from_numpy(inp["latent"]).to(dtype), inp["sigma"],
                           torch.from_numpy(inp["context"]).to(dtype), torch.from_numpy(inp["weights"]),
                           path_drop=path_drop)
