"""Writes tests/golden/dit_composition.npz from the reference implementation itself.

Run in the build container, where the reference is mounted read-only:
    python tests/golden/make_golden.py [/root/reference]

It imports the reference's PyTorch model (tools/reference.py: DiT.forward / text_refine /
block, with its own dump hooks) and quantizer (tools/quant.py: dequantize,
quantize_int8_convrot), drives them with seeded weights from tests/dit_fixture.py (MLP width
256 to keep the file small; D = 1536, 18 blocks and 2 text-refine blocks are fixed by the
reference), and stores inputs-by-seed, weight checksums and the reference's outputs:
x0 for a normal and a path-drop pass, the dumped intermediates (txt_refined, cond, block1),
and the int8 ConvRot quantization of a small seeded matrix. Only data is written; nothing
from the reference's sources is copied.
"""

import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import dit_fixture as F  # noqa: E402

WEIGHT_SEED, MLP_I = 3, 256
CASES = [  # name, h, w, T, input seed, zero-weight tokens, path_drop
    ("joint", 4, 6, 10, 21, (2,), False),
    ("pathdrop", 3, 5, 7, 22, (), True),
]


def checksums(tensors):
    i8 = sum(int(t.to(torch.int64).sum()) for n, t in tensors.items() if t.dtype == torch.int8)
    bf = sum(float(t.double().sum()) for n, t in tensors.items() if t.dtype == torch.bfloat16)
    sc = sum(float(t.double().sum()) for n, t in tensors.items() if n.endswith("weight_scale"))
    return {"int8_sum": i8, "bf16_sum": bf, "scale_sum": sc, "count": len(tensors)}


def main(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "tools"))
    import quant as Q
    import reference as R

    torch.set_grad_enabled(False)
    tensors = F.make_weights(seed=WEIGHT_SEED, I=MLP_I)

    class Weights:
        """Duck-typed tools/reference.py Weights over in-memory tensors (int8 layers are
        dequantized on access by the reference's own quant.dequantize)."""

        def has(self, name):
            return name in tensors

        def __call__(self, name):
            base = name[: -len("weight")] if name.endswith("weight") else None
            if base is not None and base + "comfy_quant" in tensors:
                return Q.dequantize({s: tensors[base + s] for s in ("weight", "weight_scale", "comfy_quant")})
            return tensors[name].float()

    dit = R.DiT(Weights())
    out = {}
    meta = {"weight_seed": WEIGHT_SEED, "mlp_width": MLP_I, "checksums": checksums(tensors), "cases": []}
    for name, h, w, T, seed, zero, path_drop in CASES:
        inp = F.make_inputs(h, w, T, seed=seed, zero_weight_tokens=zero)
        dump = {}
        x0 = dit.forward(torch.from_numpy(inp["latent"]), inp["sigma"], torch.from_numpy(inp["context"]),
                         torch.from_numpy(inp["weights"]), path_drop=path_drop, dump=dump)
        out[f"{name}.x0"] = x0.numpy()
        for k in ("txt_refined", "cond", "block1"):
            out[f"{name}.{k}"] = dump[k].numpy()
        meta["cases"].append({"name": name, "h": h, "w": w, "T": T, "input_seed": seed, "zero_weight_tokens": list(zero),
                              "path_drop": path_drop, "sigma": inp["sigma"]})
        print(f"{name}: x0 {tuple(x0.shape)} |x0| {float(x0.norm()):.4f}", flush=True)

    g = torch.Generator().manual_seed(17)
    wq = torch.randn(8, 512, generator=g) * 0.05
    qd = Q.quantize_int8_convrot(wq)
    out["quant.w"] = wq.numpy()
    out["quant.q"] = qd["weight"].numpy()
    out["quant.scale"] = qd["weight_scale"].numpy()
    out["quant.meta"] = np.frombuffer(bytes(qd["comfy_quant"].tolist()), dtype=np.uint8)
    out["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    path = os.path.join(HERE, "dit_composition.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path) / 1024:.0f} KiB)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
