"""CPU checks of the drop-in boundary: the C ABI library loads and exports every entry point
declared in include/ns2.h, the ctypes binding and the N-API addon cover them, errors come back
as messages (no device in this container), and the Node host's pure-JS parts (rotary tables,
timestep embedding, safetensors reader) agree with the oracle."""

import json
import math
import os
import re
import subprocess

import numpy as np
import pytest
import torch

import ns2
import oracle.nanosaur2_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ns2.h")
HOST_CHECKS = os.path.join(ROOT, "tests", "js", "host_checks.mjs")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|void\*|size_t)\s+(ns2_\w+)\(", text, re.M)))


def test_header_symbols_exported():
    names = declared()
    assert len(names) >= 30
    lib = ns2.Lib()
    missing = [n for n in names if not hasattr(lib.dll, n)]
    assert not missing, missing
    assert sorted(ns2.SIGNATURES) == names, "ctypes binding and header disagree"


def test_symbols_visible_in_dynamic_table():
    out = subprocess.run(["nm", "-D", "--defined-only", ns2.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (ns2_\w+)", out))
    assert set(declared()) <= exported


def test_errors_without_device():
    lib = ns2.Lib()
    assert lib.dll.ns2_linear_i8(None, 0, 256, None, None, None, None, None, 1, 1, 256, 1, 0, 1.0, 0, 0, None, 0) == 4
    assert "ns2_init" in lib.error()
    rc = lib.dll.ns2_init(0)
    assert rc != 0 and lib.error()
    assert lib.dll.ns2_pool_round(257) == 512


def _pool_round_reference(b):
    """app/gpu/device.js:33-39."""
    b = max(256, b)
    p = 2 ** math.floor(math.log2(b))
    step = max(256, p // 8)
    return -(-b // step) * step


@pytest.fixture(scope="module")
def host(tmp_path_factory):
    from safetensors.torch import save_file

    d = tmp_path_factory.mktemp("st")
    g = torch.Generator().manual_seed(4)
    q = torch.randint(-127, 128, (6, 256), generator=g, dtype=torch.int32).to(torch.int8)
    meta = json.dumps({"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 256}).encode()
    bad = json.dumps({"format": "float8_e4m3fn"}).encode()
    t = {
        "blk.qkv.weight": q, "blk.qkv.weight_scale": torch.rand(6, 1, generator=g),
        "blk.qkv.comfy_quant": torch.tensor(list(meta), dtype=torch.uint8),
        "emb.weight": torch.randn(4, 64, generator=g).to(torch.bfloat16),
        "norm.weight": torch.randn(16, generator=g).to(torch.bfloat16),
        "bad.weight": q.clone(), "bad.comfy_quant": torch.tensor(list(bad), dtype=torch.uint8),
    }
    path = str(d / "w.safetensors")
    save_file(t, path)
    p = subprocess.run(["node", HOST_CHECKS, path], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stderr
    return json.loads(p.stdout), t


def test_addon_exports_and_errors(host):
    out, _ = host
    want = {"init", "malloc", "free", "h2d", "d2h", "sync", "poolGet", "poolPut", "poolTrim", "poolRound",
            "linearI8", "linearBf16", "attention", "headNorm", "normMod", "normModRotateF16", "glu",
            "gluRotateF16", "hadamard256", "rotateF16", "elementwise", "accumulate", "rowSum", "rmsnorm",
            "addRows", "attentionRows", "addRmsnorm", "transpose",
            "eventCreate", "eventRecord", "eventElapsed", "profileEnable", "profileReport",
            "graphBegin", "graphEnd", "graphLaunch", "graphDestroy", "linearBf16AddRmsnorm", "headNorm2", "linearBf16Glu"}
    assert want <= set(out["addonExports"])
    assert out["initError"] and "device" in out["initError"]
    assert "ns2_init" in out["callError"]
    assert "BigInt" in out["typeError"]
    for b, got in zip([1, 256, 257, 1000, 4096, 5000, 1 << 20, (1 << 20) + 1], out["poolRound"]):
        assert got == _pool_round_reference(b)


def test_js_rope_tables_match_oracle(host):
    out, _ = host
    cs, sin_off = O.rope2d_table(5, 7)
    assert out["rope2d"]["sinOff"] == sin_off
    assert np.allclose(out["rope2d"]["values"], cs.numpy(), atol=1e-7)
    cos, sin = O.rope_2d(5, 7, dtype=torch.float64)
    js = np.array(out["rope2d"]["values"])
    assert np.allclose(js[:sin_off].reshape(35, 48), cos.numpy(), atol=2e-6)
    # 1-D table: angle l * f_i, f_i = 1 / 10000^(2i/8)
    v = np.array(out["rope1d"]["values"])
    assert out["rope1d"]["sinOff"] == 16
    ang = np.outer(np.arange(4), [1 / 10000 ** (2 * i / 8) for i in range(4)]).reshape(-1)
    assert np.allclose(v[:16], np.cos(ang), atol=1e-6) and np.allclose(v[16:], np.sin(ang), atol=1e-6)


def test_js_timestep_embedding_matches_oracle(host):
    out, _ = host
    ref = O.timestep_embedding(0.37 * 1000.0, dtype=torch.float64)[0].numpy()
    assert np.allclose(out["temb"], ref, atol=1e-4)


def test_js_safetensors_reader(host):
    out, t = host
    st = out["st"]
    assert st["i8"]["kind"] == "i8" and st["i8"]["N"] == 6 and st["i8"]["K"] == 256
    assert st["i8"]["first"] == t["blk.qkv.weight"].reshape(-1)[:8].tolist()
    assert st["i8"]["scaleLen"] == 6
    assert st["bf16"] == {"kind": "bf16", "N": 4, "K": 64}
    assert np.allclose(st["vec"], t["norm.weight"].float().numpy())
    assert st["badError"] and "unsupported quantization" in st["badError"]


def test_js_copy_bounds(host):
    """GPU.write / fromArray / read refuse copies that leave the device buffer or tensor."""
    b = host[0]["bounds"]
    assert "overrun" in b["writeOverrun"] and "overrun" in b["writeOffset"]
    assert "released" in b["writeReleased"]
    assert "do not fit shape" in b["fromArrayShape"]
    assert "requested from a tensor of 6" in b["readCount"]


def _bench_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_refuses_several_gpus():
    p = subprocess.run(["python3", os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr


def test_bench_lora_file(tmp_path):
    """The LoRA file of bench.py's dit_lora leg: PEFT names of every block linear (qkv_x, proj,
    w12, w3 of the 18 blocks, kv_y of the 9 joint blocks), rank 32, alpha 16, bf16 A/B of the
    modules' shapes."""
    from safetensors.torch import load_file

    b = _bench_module()
    path = str(tmp_path / "lora.safetensors")
    n = b.write_lora(path)
    assert n == 81
    t = load_file(path)
    assert len(t) == 3 * 81
    D, I = b.D, b.I_MLP
    shapes = {"attn.qkv_x": (3 * D, D), "attn.proj": (D, D), "mlp.w12": (2 * I, D), "mlp.w3": (D, I), "attn.kv_y": (2 * D, D)}
    seen = set()
    for key, v in t.items():
        m = re.fullmatch(r"diffusion_model\.blocks\.(\d+)\.(attn\.\w+|mlp\.\w+)\.(lora_A\.weight|lora_B\.weight|alpha)", key)
        assert m, key
        blk, mod, part = int(m.group(1)), m.group(2), m.group(3)
        assert 0 <= blk < b.BLOCKS and (mod != "attn.kv_y" or blk % 2 == 0), key
        n_out, n_in = shapes[mod]
        if part == "alpha":
            assert v.dtype == torch.float32 and float(v) == 16.0
        else:
            assert v.dtype == torch.bfloat16
            assert tuple(v.shape) == ((32, n_in) if part == "lora_A.weight" else (n_out, 32)), key
        seen.add((blk, mod))
    assert len(seen) == 81
