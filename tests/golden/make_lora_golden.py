"""Writes tests/golden/lora_composition.npz from the reference implementation itself.

Run in the build container, where the reference is mounted read-only:
    python tests/golden/make_lora_golden.py [/root/reference]

It saves the seeded DiT weights of tests/dit_fixture.py (MLP width 256) and a seeded LoRA file
(tests/dit_fixture.py make_lora: int8 block linears, the GLU linear, a text-refine linear and
bf16 linears; PEFT and kohya naming) to temporary safetensors files, loads them with the
reference's own Weights class and LoRA loader (tools/reference.py Weights(path, loras),
lora_deltas), and stores DiT.forward's x0 with the LoRA at strength 0.8. The same for the
Gemma3 text encoder (tests/gemma_fixture.py weights and make_te_lora: a LoRA on k_proj, up_proj
and o_proj of three layers) through gemma_encode. Only data is written;
nothing from the reference's sources is copied.
"""

import json
import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import dit_fixture as F  # noqa: E402
import gemma_fixture as G  # noqa: E402

WEIGHT_SEED, MLP_I, LORA_SEED, STRENGTH = 3, 256, 9, 0.8
CASE = ("joint", 4, 6, 10, 21, (2,))  # name, h, w, T, input seed, zero-weight tokens
TE_SEED, TE_LORA_SEED, TE_STRENGTH, TE_IDS = 5, 12, 4.0, (17, 34)  # ids: length, seed


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "tools"))
    import reference as R
    from safetensors.torch import save_file

    torch.set_grad_enabled(False)
    out, meta = {}, {"weight_seed": WEIGHT_SEED, "mlp_width": MLP_I, "lora_seed": LORA_SEED, "strength": STRENGTH}
    with tempfile.TemporaryDirectory() as d:
        wpath, lpath = os.path.join(d, "dit.safetensors"), os.path.join(d, "lora.safetensors")
        F.save_weights(F.make_weights(seed=WEIGHT_SEED, I=MLP_I), wpath)
        save_file(F.make_lora(seed=LORA_SEED, I=MLP_I), lpath)
        name, h, w, T, seed, zero = CASE
        inp = F.make_inputs(h, w, T, seed=seed, zero_weight_tokens=zero)
        args = (torch.from_numpy(inp["latent"]), inp["sigma"], torch.from_numpy(inp["context"]),
                torch.from_numpy(inp["weights"]))
        x_plain = R.DiT(R.Weights(wpath)).forward(*args)
        x_lora = R.DiT(R.Weights(wpath, loras=[(lpath, STRENGTH)])).forward(*args)
        out["dit.x0"] = x_lora.numpy()
        rel = float((x_lora - x_plain).norm() / x_plain.norm())
        meta["dit_case"] = {"name": name, "h": h, "w": w, "T": T, "input_seed": seed, "zero_weight_tokens": list(zero),
                            "sigma": inp["sigma"], "rel_change": rel}
        print(f"DiT: |x0| {float(x_lora.norm()):.4f}, LoRA changes x0 by {100 * rel:.1f} %", flush=True)

        tpath, tlpath = os.path.join(d, "te.safetensors"), os.path.join(d, "te_lora.safetensors")
        G.save_weights(G.make_weights(seed=TE_SEED), tpath)
        save_file(G.make_te_lora(seed=TE_LORA_SEED), tlpath)
        ids = G.make_ids(TE_IDS[0], seed=TE_IDS[1])
        y_plain = R.gemma_encode(R.Weights(tpath), ids)
        y_lora = R.gemma_encode(R.Weights(tpath, loras=[(tlpath, TE_STRENGTH)]), ids)
        out["te.ids"] = np.asarray(ids, dtype=np.int32)
        out["te.out"] = y_lora.float().numpy()
        rel = float((y_lora - y_plain).norm() / y_plain.norm())
        meta["te"] = {"weight_seed": TE_SEED, "lora_seed": TE_LORA_SEED, "strength": TE_STRENGTH,
                      "ids": list(TE_IDS), "rel_change": rel}
        print(f"Gemma3: |y| {float(y_lora.norm()):.4f}, LoRA changes the encoding by {100 * rel:.1f} %", flush=True)
    out["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    path = os.path.join(HERE, "lora_composition.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
