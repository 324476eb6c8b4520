"""CPU checks of the Node host's LoRA module (nanosaur2-web_amd/js/lora.js, the behaviour of
app/lora.js): the fp16 rounding of the stacked operands against numpy, the stacked side path
against the oracle's pack_lora, key inspection, and the loader's name matching (PEFT and kohya
names, DiT and text-encoder prefixes, slices of stacked weights) with fake models. The rotation
of int8 targets' down-projections runs on the device (the activation rotation kernel); the GPU
LoRA tests cover it against the reference's own LoRA outputs."""

import json
import os
import subprocess

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import dit_fixture as F
import gemma_fixture as G
import oracle.nanosaur2_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECKS = os.path.join(ROOT, "tests", "js", "lora_checks.mjs")


@pytest.fixture(scope="module")
def host(tmp_path_factory):
    d = tmp_path_factory.mktemp("lora")
    g = torch.Generator().manual_seed(8)
    f16 = [0.0, -0.0, 1.0, 65504.0, 65520.0, 1e6, -1e6, 6.1e-5, 5.96e-8, 2.98e-8, 1e-9, 0.1, 1 / 3,
           1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, -2.5e-6, float(np.float32(np.pi))]
    f16 += torch.randn(200, generator=g).mul(30).tolist()
    N, K = 48, 256
    ents = [(torch.randn(3, K, generator=g), torch.randn(N, 3, generator=g), 0.5, 0, N),
            (torch.randn(5, K, generator=g), torch.randn(16, 5, generator=g), -2.0, 20, 16)]
    lora_dit = F.make_lora(seed=9, I=256)
    dit_file = str(d / "dit_lora.safetensors")
    save_file(lora_dit, dit_file)
    te_lora = G.make_te_lora(seed=12)
    te_file = str(d / "te_lora.safetensors")
    save_file(te_lora, te_file)
    # kohya text-encoder names without "model." (the loader retries with "model_")
    kohya_te = {"lora_te_layers_1_self_attn_k_proj.lora_down.weight": te_lora["text_encoder.model.layers.1.self_attn.k_proj.lora_A.weight"],
                "lora_te_layers_1_self_attn_k_proj.lora_up.weight": te_lora["text_encoder.model.layers.1.self_attn.k_proj.lora_B.weight"],
                "lora_te_layers_1_self_attn_k_proj.hada_w1_a": torch.zeros(2)}
    kohya_file = str(d / "te_kohya.safetensors")
    save_file(kohya_te, kohya_file)
    dit_linears = [{"name": m, "kind": "i8" if (m.startswith("blocks") or m.startswith("text_refine")) else "bf16",
                    "N": n_out, "K": n_in} for m, n_out, n_in, r, nm in F.lora_targets(I=256)]
    dit_linears.append({"name": "blocks.9.attn.proj", "kind": "i8", "N": 1536, "K": 1536})
    qkv = {"kind": "bf16", "N": 1536, "K": 640, "parts": [
        {"name": "model.layers.1.self_attn.q_proj", "off": 0, "n": 1024},
        {"name": "model.layers.1.self_attn.k_proj", "off": 1024, "n": 256},
        {"name": "model.layers.1.self_attn.v_proj", "off": 1280, "n": 256}]}
    gu = {"kind": "bf16", "N": 4096, "K": 640, "parts": [
        {"name": "model.layers.6.mlp.gate_proj", "off": 0, "n": 2048},
        {"name": "model.layers.6.mlp.up_proj", "off": 2048, "n": 2048}]}
    o = {"name": "model.layers.16.self_attn.o_proj", "kind": "bf16", "N": 640, "K": 1024}
    # nine stacked parts with a rank-32 LoRA each (the DiT's kv_y of the 9 joint blocks, scaled
    # down): 288 > 256, so the side paths split into windows of whole parts
    SN, SK, SP = 16, 32, 9
    stacked = [(torch.randn(32, SK, generator=g), torch.randn(SN, 32, generator=g), 0.25 * (i + 1), SN * i, SN)
               for i in range(SP)]
    job = {
        "stacked": {"N": SN * SP, "K": SK,
                    "parts": [{"name": f"blocks.{2 * i}.attn.kv_y", "off": SN * i, "n": SN} for i in range(SP)],
                    "entries": [{"A": A.reshape(-1).tolist(), "B": B.reshape(-1).tolist(), "r": 32, "scale": s,
                                 "off": off, "n": n} for A, B, s, off, n in stacked]},
        "f16": f16, "N": N, "K": K,
        "entries": [{"A": A.reshape(-1).tolist(), "B": B.reshape(-1).tolist(), "r": A.shape[0], "scale": s, "off": off, "n": n}
                    for A, B, s, off, n in ents],
        "keys": [list(lora_dit), ["x.lokr_w1", "diffusion_model.blocks.0.attn.proj.lora_A.weight",
                                  "diffusion_model.blocks.0.attn.proj.lora_B.weight", "other_model.fc.lora_A.weight"]],
        "loads": [{"file": dit_file, "linears": dit_linears},
                  {"file": te_file, "te": True, "linears": [qkv, gu, o]},
                  {"file": kohya_file, "te": True, "linears": [qkv, gu, o]}],
    }
    jf = str(d / "job.json")
    with open(jf, "w") as f:
        json.dump(job, f)
    p = subprocess.run(["node", CHECKS, jf], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    return json.loads(p.stdout), stacked, f16, ents, lora_dit, te_lora


def test_f16_rounding_matches_numpy(host):
    out, _, f16, *_ = host
    with np.errstate(over="ignore"):  # 65520 and 1e6 overflow to infinity, as in the host code
        ref = np.asarray(f16, dtype=np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(np.asarray(out["f16"], dtype=np.uint16), ref)


def test_stacked_side_path(host):
    out, _, _, ents, *_ = host
    la, lb, R = O.pack_lora(ents, 48, 256)
    assert out["stack"]["R"] == R == 32
    assert np.allclose(np.asarray(out["stack"]["a"]).reshape(R, 256), la.numpy(), atol=1e-6)
    assert np.allclose(np.asarray(out["stack"]["b"]).reshape(48, R), lb.numpy(), atol=1e-5)


def test_stacked_parts_split_into_windows(host):
    """Nine rank-32 LoRAs on the nine parts of a stacked weight: the first eight parts share one
    side path (rank 256), the ninth gets its own; each window's operands equal the oracle's
    pack_lora over the window's entries, and the output rows of all windows together equal one
    unlimited stacked side path (no LoRA lost or doubled)."""
    out, stacked, *_ = host
    SN, SK = 16, 32
    wins = out["windows"]
    assert [(w["off"], w["n"], w["R"]) for w in wins] == [(0, 8 * SN, 256), (8 * SN, SN, 32)]
    for w, ents in ((wins[0], stacked[:8]), (wins[1], stacked[8:])):
        la, lb, R = O.pack_lora([(A, B, s, off - w["off"], n) for A, B, s, off, n in ents], w["n"], SK)
        assert np.allclose(np.asarray(w["a"]).reshape(R, SK), la.numpy(), atol=1e-6)
        assert np.allclose(np.asarray(w["b"]).reshape(w["n"], R), lb.numpy(), atol=1e-5)
    x = torch.randn(5, SK, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    la, lb, _ = O.pack_lora(stacked, SN * 9, SK)
    whole = (x @ la.T) @ lb.T
    parts = torch.cat([(x @ torch.tensor(w["a"], dtype=torch.float64).reshape(w["R"], SK).T)
                       @ torch.tensor(w["b"], dtype=torch.float64).reshape(w["n"], w["R"]).T for w in wins], 1)
    assert torch.allclose(parts, whole, rtol=1e-5, atol=1e-4)
    assert "blocks.0.attn.kv_y" in out["rankError"] and "260" in out["rankError"]


def test_inspect_keys(host):
    out = host[0]
    assert out["inspect"][0] == {"lora": True, "modules": 8, "fits": 8, "unsupported": 0}
    assert out["inspect"][1] == {"lora": True, "modules": 2, "fits": 1, "unsupported": 1}


def test_loader_matches_modules(host):
    out, _, _, _, lora_dit, te_lora = host
    dit, te, kohya = out["loads"]
    assert (dit["matched"], dit["total"], dit["skipped"]) == (8, 8, 0)
    by_w = {m["W"]: m for m in dit["modules"]}
    for mname, n_out, n_in, r, naming in F.lora_targets(I=256):
        m = by_w[mname]
        assert (m["off"], m["n"], m["r"]) == (0, n_out, r) and m["alphaScale"] == 0.5
        key = ("diffusion_model." + mname + ".lora_A.weight") if naming == "peft" else \
              ("lora_unet_" + mname.replace(".", "_") + ".lora_down.weight")
        A = lora_dit[key].float().double()
        got = torch.tensor(m["A"], dtype=torch.float64)
        assert torch.allclose(got, A.reshape(-1)[:got.numel()], atol=1e-6), mname
    assert te["matched"] == 3
    windows = sorted((m["off"], m["n"], m["r"]) for m in te["modules"])
    assert windows == [(0, 640, 4), (1024, 256, 8), (2048, 2048, 16)]
    assert (kohya["matched"], kohya["unsupported"]) == (1, 1)
    assert (kohya["modules"][0]["off"], kohya["modules"][0]["n"]) == (1024, 256)
