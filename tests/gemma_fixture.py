"""Seeded Gemma3-270M text-encoder weights for tests, and a runner for the Node host.

The real architecture (app/models/gemma3.js:13; tools/reference.py:176-200): 17 layers run of
18, hidden 640, 4 query heads and 1 K/V head of 256, MLP 2048, norm weights stored as w - 1.
Linears and norms are bf16 (the file layout of the real checkpoint), values ~ N(0, 0.02) for
linears and N(0, 0.1) for the stored norm offsets, from numpy's PCG64 with a fixed seed. The
embedding table keeps only `vocab` rows (token ids below it), enough for the test sequences.
"""

from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUN_GEMMA = os.path.join(ROOT, "nanosaur2-web_amd", "js", "run_gemma.js")


def gemma_spec(layers=17, vocab=64):
    s = {"model.embed_tokens.weight": (vocab, 640)}
    for i in range(layers):
        p = f"model.layers.{i}."
        for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm"):
            s[p + n + ".weight"] = (640,)
        s[p + "self_attn.q_norm.weight"] = (256,)
        s[p + "self_attn.k_norm.weight"] = (256,)
        s[p + "self_attn.q_proj.weight"] = (1024, 640)
        s[p + "self_attn.k_proj.weight"] = (256, 640)
        s[p + "self_attn.v_proj.weight"] = (256, 640)
        s[p + "self_attn.o_proj.weight"] = (640, 1024)
        s[p + "mlp.gate_proj.weight"] = (2048, 640)
        s[p + "mlp.up_proj.weight"] = (2048, 640)
        s[p + "mlp.down_proj.weight"] = (640, 2048)
    s["model.norm.weight"] = (640,)
    return s


def make_weights(seed=5, **spec_kw):
    """name -> bf16 torch tensor."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in gemma_spec(**spec_kw).items():
        std = 1.0 if "embed" in name else (0.1 if len(shape) == 1 else 0.02)
        v = rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)
        out[name] = torch.from_numpy(v).to(torch.bfloat16)
    return out


def save_weights(tensors, path):
    from safetensors.torch import save_file

    save_file(tensors, path)


def te_lora_targets():
    """(module, out, in, rank): a LoRA on a slice of the stacked q/k/v weight (k_proj), on a
    slice of the stacked gate/up weight (up_proj) and on a whole weight (o_proj)."""
    return [("layers.1.self_attn.k_proj", 256, 640, 8), ("layers.6.mlp.up_proj", 2048, 640, 16),
            ("layers.16.self_attn.o_proj", 640, 1024, 4)]


def make_te_lora(seed=12, a_std=0.05, b_std=0.05):
    """A text-encoder LoRA file's tensors with PEFT names under "text_encoder.model." (the
    prefix both loaders strip, tools/reference.py:74, app/lora.js:18), bf16 A/B and fp32
    alpha = rank."""
    rng = np.random.default_rng(seed)
    out = {}
    for module, n_out, n_in, r in te_lora_targets():
        base = "text_encoder.model." + module
        out[base + ".lora_A.weight"] = torch.from_numpy(
            rng.standard_normal((r, n_in), dtype=np.float32) * np.float32(a_std)).to(torch.bfloat16)
        out[base + ".lora_B.weight"] = torch.from_numpy(
            rng.standard_normal((n_out, r), dtype=np.float32) * np.float32(b_std)).to(torch.bfloat16)
        out[base + ".alpha"] = torch.tensor(float(r), dtype=torch.float32)
    return out


def make_ids(n, vocab=64, seed=11):
    return [int(x) for x in np.random.default_rng(seed).integers(0, vocab, size=n)]


def run_node(args, timeout=600):
    """Run the Node host's run_gemma.js; returns its JSON report. Fails loudly on error."""
    cmd = ["node", RUN_GEMMA, *args]
    print("[node]", " ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if p.returncode != 0:
        raise RuntimeError(f"run_gemma.js failed ({p.returncode}):\n{p.stderr[-4000:]}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def oracle_encode(tensors, ids, dtype=torch.float32):
    import oracle.nanosaur2_oracle as O

    W = O.TensorWeights(tensors, dtype)
    with torch.no_grad():
        return O.gemma_encode(W, ids, dtype)
