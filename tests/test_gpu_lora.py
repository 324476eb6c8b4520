"""LoRA side path (app/gpu/ops.js:50-87 loraDelta, app/lora.js) through the *_lora entry points
of the C ABI, against the oracle's linear with the materialized delta added after the bias
(gemm.js:159-164): int8 ConvRot weights (row-major and tiled operands, the fused GLU + rotation
launch) and bf16 weights (GEMV, split-K and 128x128 tile paths). Each case stacks two LoRAs,
one over all output columns and one over a column window (a slice of a stacked q/k/v weight),
ranks 8 and 20 (stacked to 28, padded to 32). Tolerance 2e-3 as for the plain GEMMs (fp16
operands of the low-rank products, fp32 accumulation)."""

import json
import os

import numpy as np
import pytest
import torch

import dit_fixture as F
import gemma_fixture as G
import oracle.nanosaur2_oracle as O
from conftest import assert_close, rel_errors
from test_gpu_ops import TOL, dev, f16_as_float, gen, int8_weight, tiled_operand, untile_a

pytestmark = pytest.mark.gpu


def _entries(N, K, g, scale=(0.7, -1.3), b_std=0.3):
    """A full-width LoRA (rank 8) and one on output columns [N/4, N/4 + N/2) (rank 20); with
    b_std 0.3 the low-rank term is ~10 % of the int8 products, so an error in it shows."""
    e1 = (torch.randn(8, K, generator=g) * 0.05, torch.randn(N, 8, generator=g) * b_std, scale[0], 0, N)
    n2 = N // 2
    e2 = (torch.randn(20, K, generator=g) * 0.05, torch.randn(n2, 20, generator=g) * b_std, scale[1], N // 4, n2)
    return [e1, e2]


def _packed(entries, N, K, rotate_a):
    la, lb, R = O.pack_lora(entries, N, K, rotate_a)
    return la.half().to(dev), lb.half().to(dev), R


@pytest.mark.parametrize("M,N,K", [(97, 320, 512), (1, 256, 256), (300, 1536, 1536)])
def test_linear_i8_lora(ns2lib, M, N, K):
    g = gen(M + N + K + 1)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    bias = torch.randn(N, generator=g) * 0.1
    ents = _entries(N, K, g)
    la, lb, R = _packed(ents, N, K, rotate_a=True)
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_i8(x.to(dev), 0, K, q.to(dev), s.reshape(-1).to(dev), out, M, N, K, bias=bias.to(dev),
                     alpha=0.5, act="silu", lora=(la, lb, R))
    torch.cuda.synchronize()
    xd = x.double()
    ref = O.linear_i8(xd, q, s.double(), alpha=0.5, bias=bias.double(), add=O.lora_delta(xd, ents, N), act="silu")
    assert_close(out.cpu(), ref, TOL, f"linear_i8_lora {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(300, 384, 768), (3952, 1536, 1536), (256, 3072, 1536), (200, 1536, 1536)])
def test_linear_i8_tiled_lora(ns2lib, M, N, K):
    """(256, 3072) and (200, 1536) split K (fewer 64x64 tiles than CUs): the LoRA term is added
    by the tile-wise reduce, 200 rows ending inside a 32-row tile."""
    g = gen(M + N + K + 2)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    ents = _entries(N, K, g)
    la, lb, R = _packed(ents, N, K, rotate_a=True)
    xd, qd, sd = x.to(dev), q.to(dev), s.reshape(-1).to(dev)
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(qd, wt, N, K)
    at = tiled_operand(M, K)
    ns2lib.rotate_f16(xd, K, at, K, M, K, tiled=True)
    # gated += into a column window of a wider output (the proj / w3 launches)
    ldc, cOff = N + 64, 32
    base = torch.randn(M * ldc, generator=g)
    gate = torch.randn(N + 16, generator=g)
    outd = base.to(dev)
    ns2lib.linear_i8_tiled(at, wt, sd, outd, M, N, K, ldc=ldc, cOff=cOff, resid=True, gate=gate.to(dev), gOff=16,
                           lora=(la, lb, R))
    torch.cuda.synchronize()
    xr = x.double()
    ref = O.linear_i8(xr, q, s.double(), add=O.lora_delta(xr, ents, N), out=base.double().clone(), resid=True,
                      gate=gate.double(), gOff=16, ldc=ldc, cOff=cOff)
    assert_close(outd.cpu(), ref, TOL, f"linear_i8_tiled_lora {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,act", [(130, 1024, 512, "silu"), (3952, 8192, 1536, "silu")])
def test_linear_i8_glu_rot_tiled_lora(ns2lib, M, N, K, act):
    """The fused w12 + GLU + rotation launch: lora_b in the weight's original row order, the
    kernel follows the GLU interleave of the tiles."""
    g = gen(M + N + K + 3)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    bias = torch.randn(N, generator=g) * 0.1
    ents = _entries(N, K, g)
    la, lb, R = _packed(ents, N, K, rotate_a=True)
    I = N // 2
    xd, qd, sd = x.to(dev), q.to(dev), s.reshape(-1).to(dev)
    at = tiled_operand(M, K)
    ns2lib.rotate_f16(xd, K, at, K, M, K, tiled=True)
    wglu = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight_glu(qd, wglu, N, K)
    y = tiled_operand(M, I)
    ns2lib.linear_i8_glu_rot_tiled(at, wglu, sd, y, M, N, K, bias=bias.to(dev), act=act, lora=(la, lb, R))
    torch.cuda.synchronize()
    xr = x.double()
    h = O.linear_i8(xr, q, s.double(), bias=bias.double(), add=O.lora_delta(xr, ents, N))
    ref = O.rotate(O.glu(h, act))
    assert_close(f16_as_float(untile_a(y.cpu(), M, I)), ref, TOL, f"glu_rot_lora {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(1, 9216, 1536), (5, 1536, 256), (256, 640, 2048), (256, 1536, 640),
                                   (3952, 1536, 1536), (17, 256, 80)])
def test_linear_bf16_lora(ns2lib, M, N, K):
    """bf16 linears: GEMV (M <= 8), 64x64 tiles with K split over blocks (the LoRA term goes
    into the first split only), 128x128 tiles."""
    g = gen(M + N + K + 4)
    x = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    ents = _entries(N, K, g, scale=(1.0, 0.4))
    la, lb, R = _packed(ents, N, K, rotate_a=False)
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16(x.to(dev), K, w.view(torch.int16).to(dev), out, M, N, K, bias=bias.to(dev), alpha=2.0,
                       lora=(la, lb, R))
    torch.cuda.synchronize()
    xd = x.double()
    ref = O.linear_bf16(xd, w, alpha=2.0, bias=bias.double(), add=O.lora_delta(xd, ents, N))
    assert_close(out.cpu(), ref, TOL, f"linear_bf16_lora {M}x{N}x{K}")


@pytest.mark.parametrize("M,ranks", [(3952, (24, 40)), (250, (64, 100, 92))])
def test_linear_i8_tiled_lora_ranks(ns2lib, M, ranks):
    """Stacked ranks of 64 (3952 rows: 247 down-projection blocks of 16 rows, two 32-column slices
    of t; the 64x128 launch with three stages) and 256 (250 rows: the rank split over eight
    slices, rows ending inside a block; split K, the term added by the tile-wise reduce)."""
    N, K = 768, 1536
    g = gen(M + sum(ranks))
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    ents = []
    for i, r in enumerate(ranks):
        n0, n = (0, N) if i == 0 else ((i * 128) % (N // 2), N // 2)
        ents.append((torch.randn(r, K, generator=g) * 0.05, torch.randn(n, r, generator=g) * 0.3, 0.5 + 0.25 * i, n0, n))
    la, lb, R = _packed(ents, N, K, rotate_a=True)
    assert R == (64 if sum(ranks) <= 64 else 256)
    xd, qd, sd = x.to(dev), q.to(dev), s.reshape(-1).to(dev)
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(qd, wt, N, K)
    at = tiled_operand(M, K)
    ns2lib.rotate_f16(xd, K, at, K, M, K, tiled=True)
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_i8_tiled(at, wt, sd, out, M, N, K, lora=(la, lb, R))
    torch.cuda.synchronize()
    xr = x.double()
    ref = O.linear_i8(xr, q, s.double(), add=O.lora_delta(xr, ents, N))
    assert_close(out.cpu(), ref, TOL, f"linear_i8_tiled_lora ranks {ranks} at {M} rows")


def test_lora_rank_errors(ns2lib):
    import ns2

    x = torch.zeros(4, 256, device=dev)
    w = torch.zeros(64, 256, dtype=torch.int16, device=dev)
    out = torch.empty(4, 64, device=dev)
    la = torch.zeros(24, 256, dtype=torch.float16, device=dev)
    lb = torch.zeros(64, 24, dtype=torch.float16, device=dev)
    with pytest.raises(ns2.NS2Error, match="multiple of 32"):
        ns2lib.linear_bf16(x, 256, w, out, 4, 64, 256, lora=(la, lb, 24))


@pytest.mark.parametrize("path", ["tiled", "rows", "bf16"])
def test_lora_term_alone(ns2lib, path):
    """With an all-zero base weight the output is bias + the low-rank term: pins the side path
    (stacking, windows, strengths, the rotation of A for int8 weights) on its own."""
    M, N, K = 150, 256, 512
    g = gen(77)
    x = torch.randn(M, K, generator=g)
    bias = torch.randn(N, generator=g) * 0.1
    ents = _entries(N, K, g)
    xd = x.double()
    ref = bias.double()[None, :] + O.lora_delta(xd, ents, N)
    out = torch.empty(M, N, device=dev)
    if path == "bf16":
        la, lb, R = _packed(ents, N, K, rotate_a=False)
        w = torch.zeros(N, K, dtype=torch.int16, device=dev)
        ns2lib.linear_bf16(x.to(dev), K, w, out, M, N, K, bias=bias.to(dev), lora=(la, lb, R))
    else:
        la, lb, R = _packed(ents, N, K, rotate_a=True)
        q = torch.zeros(N, K, dtype=torch.int8, device=dev)
        s = (torch.rand(N, generator=g) * 9e-3 + 1e-3).to(dev)
        if path == "rows":
            ns2lib.linear_i8(x.to(dev), 0, K, q, s, out, M, N, K, bias=bias.to(dev), lora=(la, lb, R))
        else:
            wt = torch.empty(N * K, dtype=torch.int8, device=dev)
            ns2lib.tile_i8_weight(q, wt, N, K)
            at = tiled_operand(M, K)
            ns2lib.rotate_f16(x.to(dev), K, at, K, M, K, tiled=True)
            ns2lib.linear_i8_tiled(at, wt, s, out, M, N, K, bias=bias.to(dev), lora=(la, lb, R))
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, TOL, f"LoRA term alone ({path})")


# ------------------------------------------------------------------ whole models through Node

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "lora_composition.npz")
TOL_PASS = 1e-2


@pytest.fixture(scope="module")
def lora_golden(tmp_path_factory):
    from safetensors.torch import save_file

    z = np.load(GOLDEN, allow_pickle=False)
    return z, json.loads(bytes(z["meta"]).decode()), tmp_path_factory.mktemp("lora_models"), save_file


@pytest.mark.parametrize("reference_ops", [False, True])
def test_dit_pass_with_lora(lora_golden, reference_ops):
    """run_dit.js --lora against the reference's own x0 with the LoRA (fused path: tiled and
    GLU-fused int8 launches; reference op sequence: row-major int8 launches)."""
    z, meta, d, save_file = lora_golden
    wpath, lpath = str(d / "dit.safetensors"), str(d / "lora.safetensors")
    if not os.path.exists(wpath):
        F.save_weights(F.make_weights(seed=meta["weight_seed"], I=meta["mlp_width"]), wpath)
        save_file(F.make_lora(seed=meta["lora_seed"], I=meta["mlp_width"]), lpath)
    c = meta["dit_case"]
    inp = F.make_inputs(c["h"], c["w"], c["T"], seed=c["input_seed"], zero_weight_tokens=tuple(c["zero_weight_tokens"]))
    idir = str(d / f"in_{reference_ops}")
    F.write_inputs(inp, idir)
    out = str(d / f"x0_{reference_ops}.f32")
    args = ["--weights", wpath, "--inputs", idir, "--out", out, "--lora", f"{lpath}:{meta['strength']}"]
    if reference_ops:
        args.append("--reference-ops")
    rep = F.run_node(args)
    assert rep["loras"][0]["matched"] == 8 and rep["loras"][0]["skipped"] == 0
    got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(64, c["h"], c["w"]))
    assert_close(got, torch.from_numpy(z["dit.x0"]), TOL_PASS, f"DiT pass with LoRA (reference ops {reference_ops})")


def test_gemma_encode_with_lora(lora_golden):
    """run_gemma.js --lora against the reference's own encoding with the LoRA (slices of the
    stacked q/k/v and gate/up weights, a whole o_proj)."""
    z, meta, d, save_file = lora_golden
    t = meta["te"]
    wpath, lpath = str(d / "te.safetensors"), str(d / "te_lora.safetensors")
    G.save_weights(G.make_weights(seed=t["weight_seed"]), wpath)
    save_file(G.make_te_lora(seed=t["lora_seed"]), lpath)
    idf = str(d / "ids.json")
    ids = [int(i) for i in z["te.ids"]]
    with open(idf, "w") as f:
        json.dump(ids, f)
    out = str(d / "te.f32")
    rep = G.run_node(["--weights", wpath, "--ids", idf, "--out", out, "--lora", f"{lpath}:{t['strength']}"])
    assert rep["loras"][0]["matched"] == 3
    got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(len(ids), 640))
    assert_close(got, torch.from_numpy(z["te.out"]), TOL_PASS, "Gemma3 encoding with LoRA")


# LoRAs on the linears the fused pass stacks or re-tiles: the two adaLN projections of the
# conditioning vector (one stacked GEMV), a text block's adaLN projection (stacked with the
# other block's), and the bf16 linears that take tiled fp16 operands
STACKED_TARGETS = [
    ("shared_encoder_adaLN.0", 6 * F.D, F.D, 8, "peft"),
    ("final_layer.adaLN_modulation", 2 * F.D, F.D, 8, "kohya"),
    ("text_refine_blocks.1.adaLN_modulation.0", 6 * F.D, F.D, 8, "peft"),
    ("sprint_out_proj", F.D, F.D, 8, "peft"),
    ("s_embedder.proj", F.D, 64, 8, "peft"),
]


@pytest.mark.parametrize("reference_ops", [False, True])
def test_dit_pass_lora_on_every_joint_kv(tmp_path, reference_ops):
    """A rank-32 LoRA on the kv_y of all 9 joint blocks (288 summed ranks), plus LoRAs on the
    stacked adaLN projections and the re-tiled bf16 linears. The fused pass runs the 9 kv_y
    projections as one stacked weight, whose side paths then split into two row windows (8
    parts at rank 256, 1 at rank 32) and two launches; the reference op sequence runs each kv_y
    with its own side path. Both against the oracle with the LoRA merged into the weights
    (tools/reference.py:48-95), and closer to it than to the pass without the LoRA."""
    from safetensors.torch import save_file

    I = 256
    tensors = F.make_weights(seed=5, I=I)
    lora = F.make_lora(seed=14, I=I, b_std=0.3, targets=F.joint_kv_targets(32) + STACKED_TARGETS)
    wpath, lpath = str(tmp_path / "dit.safetensors"), str(tmp_path / "kv_lora.safetensors")
    F.save_weights(tensors, wpath)
    save_file(lora, lpath)
    inp = F.make_inputs(5, 6, 24, seed=15)
    idir = str(tmp_path / "in")
    F.write_inputs(inp, idir)
    out = str(tmp_path / "x0.f32")
    args = ["--weights", wpath, "--inputs", idir, "--out", out, "--lora", f"{lpath}:0.8"]
    if reference_ops:
        args.append("--reference-ops")
    rep = F.run_node(args)
    assert rep["loras"][0]["matched"] == 9 + len(STACKED_TARGETS) and rep["loras"][0]["skipped"] == 0
    got = torch.from_numpy(np.fromfile(out, dtype=np.float32).reshape(64, 5, 6))
    ref = F.oracle_forward(tensors, inp, loras=[(lora, 0.8)])
    assert_close(got, ref, TOL_PASS, f"DiT pass, rank-32 LoRA on all joint kv_y (reference ops {reference_ops})")
    _, without = rel_errors(F.oracle_forward(tensors, inp), ref)
    _, err = rel_errors(got, ref)
    assert err < 0.1 * without, f"the LoRA's effect (rel-L2 {without:.3e}) is not resolved: error {err:.3e}"
