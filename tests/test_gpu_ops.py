"""Parity of every HIP op against the CPU oracle, called through the C ABI (ctypes).

Tolerances: 2e-3 (max|d|/max|ref| and rel-L2) for GEMM/attention outputs computed on fp16
MFMA operands; 1e-5 for the fp32-only row kernels.
"""

import math

import pytest
import torch

import oracle.nanosaur2_oracle as O
from conftest import assert_close

pytestmark = pytest.mark.gpu
dev = "cuda"
TOL = 2e-3        # parity tolerance for attention / GEMM outputs (max-abs / max|ref|, rel-L2)
TOL_F32 = 1e-5    # kernels that compute in fp32 end to end
TOL_F16_OUT = 2e-3  # fp32 math, fp16-rounded output
TOL_ROWS = 1e-4  # fp32 attention with the hardware exp (v_exp_f32)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def int8_weight(N, K, g):
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int32).to(torch.int8)
    s = torch.rand(N, 1, generator=g) * 9e-3 + 1e-3
    return q, s


def f16_as_float(t):
    return t.view(torch.float16).float()


def untile_a(t, M, K):
    """Tiled fp16 operand [ceil(M/64)][K/64][8][64][8] -> row-major [M, K]."""
    Mb = (M + 63) // 64
    return t.reshape(Mb, K // 64, 8, 64, 8).permute(0, 3, 1, 2, 4).reshape(Mb * 64, K)[:M]


def untile_w(t, N, K):
    """Tiled weight [N/64][K/64][8][64][8] of biased bytes (w + 128) -> row-major int8 [N, K]."""
    u = t.view(torch.uint8).reshape(N // 64, K // 64, 8, 64, 8).permute(0, 3, 1, 2, 4).reshape(N, K)
    return (u.to(torch.int16) - 128).to(torch.int8)


def tiled_operand(M, K):
    return torch.empty((M + 63) // 64 * 64, K, dtype=torch.int16, device=dev)


# ----------------------------------------------------------------------------- rotation

@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 1536), (2432, 1536), (300, 4096)])
def test_hadamard256(ns2lib, rows, cols):
    g = gen(rows + cols)
    x = torch.randn(rows, cols, generator=g)
    xd = x.to(dev)
    y = torch.empty_like(xd)
    ns2lib.hadamard256(xd, y, rows * cols // 256)
    torch.cuda.synchronize()
    assert_close(y.cpu(), O.rotate(x.double()), TOL_F32, f"hadamard256 {rows}x{cols}")


def test_hadamard256_in_place(ns2lib):
    x = torch.randn(64, 512, generator=gen(3))
    xd = x.to(dev)
    ns2lib.hadamard256(xd, xd, 128)
    torch.cuda.synchronize()
    assert_close(xd.cpu(), O.rotate(x.double()), TOL_F32, "hadamard256 in place")


def test_rotate_f16_strided(ns2lib):
    x = torch.randn(100, 1024, generator=gen(4))
    xd = x.to(dev)
    y = torch.zeros(100, 640, dtype=torch.int16, device=dev)
    # columns [256, 768) of x into columns [0, 512) of a wider fp16 buffer
    ns2lib.rotate_f16(xd.data_ptr() + 256 * 4, 1024, y, 640, 100, 512)
    torch.cuda.synchronize()
    got = f16_as_float(y.cpu())[:, :512]
    assert_close(got, O.rotate(x[:, 256:768].double()), TOL_F16_OUT, "rotate_f16 strided")
    assert (f16_as_float(y.cpu())[:, 512:] == 0).all()


# ----------------------------------------------------------------------------- int8 ConvRot linear

@pytest.mark.parametrize("M,N,K", [
    (2432, 4608, 1536),   # fused QKV
    (2432, 1536, 1536),   # out projection
    (2432, 6144, 1536),   # MLP up
    (2432, 1536, 6144),   # MLP down
    (3952, 8192, 1536),   # real-model w12
    (97, 300, 512),       # ragged tails
    (1, 1536, 1536),      # GEMV path
    (5, 3072, 1536),
])
def test_linear_i8_shapes(ns2lib, M, N, K):
    g = gen(M * 7 + N + K)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    ref = O.linear_i8(x.double(), q, s.double())
    # equals x @ W_deq^T (tools/quant.py:59-64)
    if M * N * K <= 2e9:
        assert_close(ref, x.double() @ O.dequantize(q, s, torch.float64).T, 1e-9, "oracle identity")
    xd, qd, sd = x.to(dev), q.to(dev), s.reshape(-1).to(dev)
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_i8(xd, 0, K, qd, sd, out, M, N, K)
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, TOL, f"linear_i8 a_fmt=0 {M}x{N}x{K}")
    # pre-rotated fp16 input (ops.linear with opts.xr)
    xr = torch.empty(M, K, dtype=torch.int16, device=dev)
    ns2lib.rotate_f16(xd, K, xr, K, M, K)
    out2 = torch.empty(M, N, device=dev)
    ns2lib.linear_i8(xr, 1, K, qd, sd, out2, M, N, K)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out2.cpu())


def test_linear_i8_epilogues(ns2lib):
    M, N, K = 300, 384, 768
    g = gen(11)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    bias = torch.randn(N, generator=g)
    add = torch.randn(M, N, generator=g)
    gate = torch.randn(4 * N, generator=g)
    base = torch.randn(M, N, generator=g)
    xd, qd, sd = x.to(dev), q.to(dev), s.reshape(-1).to(dev)

    # bias + add + silu + alpha
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_i8(xd, 0, K, qd, sd, out, M, N, K, bias=bias.to(dev), add=add.to(dev), alpha=0.5, act="silu")
    ref = O.linear_i8(x.double(), q, s.double(), alpha=0.5, bias=bias.double(), add=add.double(), act="silu")
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, TOL, "bias+add+silu+alpha")

    # residual
    outd = base.to(dev)
    ns2lib.linear_i8(xd, 0, K, qd, sd, outd, M, N, K, resid=True)
    ref = O.linear_i8(x.double(), q, s.double(), out=base.double().clone(), resid=True)
    torch.cuda.synchronize()
    assert_close(outd.cpu(), ref, TOL, "resid")

    # gated residual (gate at an offset, app/models/nanosaur2.js:210)
    outd = base.to(dev)
    ns2lib.linear_i8(xd, 0, K, qd, sd, outd, M, N, K, resid=True, gate=gate.to(dev), gOff=2 * N)
    ref = O.linear_i8(x.double(), q, s.double(), out=base.double().clone(), resid=True, gate=gate.double(), gOff=2 * N)
    torch.cuda.synchronize()
    assert_close(outd.cpu(), ref, TOL, "gated resid")


def test_linear_i8_column_window(ns2lib):
    """kv_y writes rows [L, L+T), cols [D, 3D) of the packed qkv (app/models/nanosaur2.js:202)."""
    L, T, Dm = 40, 24, 256
    g = gen(12)
    txt = torch.randn(T, Dm, generator=g)
    q, s = int8_weight(2 * Dm, Dm, g)
    qkv = torch.randn(L + T, 3 * Dm, generator=g)
    qkvd = qkv.to(dev)
    ns2lib.linear_i8(txt.to(dev), 0, Dm, q.to(dev), s.reshape(-1).to(dev), qkvd, T, 2 * Dm, Dm,
                     ldc=3 * Dm, cOff=L * 3 * Dm + Dm)
    ref = qkv.double().clone()
    O.linear_i8(txt.double(), q, s.double(), out=ref, ldc=3 * Dm, cOff=L * 3 * Dm + Dm)
    torch.cuda.synchronize()
    got = qkvd.cpu()
    assert torch.equal(got[:L], qkv[:L]) and torch.equal(got[L:, :Dm], qkv[L:, :Dm])
    assert_close(got, ref, TOL, "kv_y column window")


# ----------------------------------------------------------------------------- tiled int8 linear

def test_tile_i8_weight(ns2lib):
    N, K = 320, 768
    q, _ = int8_weight(N, K, gen(13))
    qd = q.to(dev)
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(qd, wt, N, K)
    torch.cuda.synchronize()
    assert torch.equal(untile_w(wt.cpu(), N, K), q)


@pytest.mark.parametrize("rows", [1, 7, 100, 517])
def test_tiled_producers(ns2lib, rows):
    """The tiled forms of the three producers: the oracle's values in the tiled layout, and
    exactly the row-major results."""
    g = gen(14 + rows)
    cols, I = 1536, 4096
    xh = torch.randn(rows, cols, generator=g)
    modh = torch.randn(6 * cols, generator=g) * 0.1
    wh = torch.randn(cols, generator=g) * 0.02
    hh = torch.randn(rows, 2 * I, generator=g) * 2
    x, mod, w, h = xh.to(dev), modh.to(dev), wh.to(dev), hh.to(dev)
    refs = {
        "rotate_f16": O.rotate(xh.double()),
        "norm_mod_rotate_f16": O.rotate(O.norm_mod(xh.double(), modh.double(), 0, cols, wh.double())),
        "glu_rotate_f16": O.rotate(O.glu(hh.double(), "silu")),
    }
    for name, call, K in [
        ("rotate_f16", lambda y, t: ns2lib.rotate_f16(x, cols, y, cols, rows, cols, tiled=t), cols),
        ("norm_mod_rotate_f16",
         lambda y, t: ns2lib.norm_mod_rotate_f16(x, mod, 0, cols, rows, cols, w, y, tiled=t), cols),
        ("glu_rotate_f16", lambda y, t: ns2lib.glu_rotate_f16(h, y, rows, I, "silu", tiled=t), I),
    ]:
        flat = torch.empty(rows, K, dtype=torch.int16, device=dev)
        call(flat, False)
        til = tiled_operand(rows, K)
        call(til, True)
        torch.cuda.synchronize()
        got = untile_a(til.cpu(), rows, K)
        assert_close(f16_as_float(got), refs[name], TOL_F16_OUT, f"{name} tiled rows={rows}")
        assert torch.equal(got, flat.cpu()), name


@pytest.mark.parametrize("rows,cols", [(9, 5120), (100, 6144), (2432, 6144)])
def test_rotate_f16_wide_rows(ns2lib, rows, cols):
    """The rotation producer on rows of 20 and 24 groups (the widest block-linear input, 6144):
    the oracle's values, tiled and row-major, and both forms equal."""
    g = gen(rows + cols)
    xh = torch.randn(rows, cols, generator=g)
    x = xh.to(dev)
    flat = torch.empty(rows, cols, dtype=torch.int16, device=dev)
    ns2lib.rotate_f16(x, cols, flat, cols, rows, cols)
    til = tiled_operand(rows, cols)
    ns2lib.rotate_f16(x, cols, til, cols, rows, cols, tiled=True)
    torch.cuda.synchronize()
    got = untile_a(til.cpu(), rows, cols)
    assert_close(f16_as_float(got), O.rotate(xh.double()), TOL_F16_OUT, f"rotate_f16 {rows}x{cols}")
    assert torch.equal(got, flat.cpu())


def _tiled_linear_inputs(M, N, K, seed):
    g = gen(seed)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    return g, x, q, s, x.to(dev), q.to(dev), tiled_operand(M, K)


@pytest.mark.parametrize("M,N,K", [
    (3952, 4608, 1536),   # fused QKV, 832x1216 image + text rows
    (3952, 1536, 1536),   # out projection
    (3952, 8192, 1536),   # MLP w12
    (3952, 1536, 4096),   # MLP w3
    (256, 3072, 1536),    # kv_y on the text rows
    (256, 27648, 1536),   # the 9 joint blocks' kv_y stacked: one launch per pass
    (2432, 4608, 1536),   # the 2432-row linears on fp32 activations: fused QKV,
    (2432, 1536, 1536),   # out projection,
    (2432, 6144, 1536),   # MLP up,
    (2432, 1536, 6144),   # MLP down (24 k-tiles)
    (1100, 576, 768),     # a ragged last row tile at more than 1024 rows
    (97, 320, 512),       # ragged rows, N not a multiple of 128
    (1, 64, 256),
])
def test_linear_i8_tiled_shapes(ns2lib, M, N, K):
    g, x, q, s, xd, qd, at = _tiled_linear_inputs(M, N, K, M * 3 + N + K)
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(qd, wt, N, K)
    ns2lib.rotate_f16(xd, K, at, K, M, K, tiled=True)
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_i8_tiled(at, wt, s.reshape(-1).to(dev), out, M, N, K)
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.linear_i8(x.double(), q, s.double()), TOL, f"linear_i8_tiled {M}x{N}x{K}")


def test_linear_i8_tiled_epilogues(ns2lib):
    M, N, K = 300, 384, 768
    g, x, q, s, xd, qd, at = _tiled_linear_inputs(M, N, K, 15)
    bias = torch.randn(N, generator=g)
    gate = torch.randn(4 * N, generator=g)
    base = torch.randn(M, N, generator=g)
    sd = s.reshape(-1).to(dev)
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(qd, wt, N, K)
    ns2lib.rotate_f16(xd, K, at, K, M, K, tiled=True)

    out = torch.empty(M, N, device=dev)
    ns2lib.linear_i8_tiled(at, wt, sd, out, M, N, K, bias=bias.to(dev), alpha=0.5, act="silu")
    ref = O.linear_i8(x.double(), q, s.double(), alpha=0.5, bias=bias.double(), act="silu")
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, TOL, "tiled bias+silu+alpha")

    outd = base.to(dev)
    ns2lib.linear_i8_tiled(at, wt, sd, outd, M, N, K, resid=True, gate=gate.to(dev), gOff=2 * N)
    ref = O.linear_i8(x.double(), q, s.double(), out=base.double().clone(), resid=True, gate=gate.double(), gOff=2 * N)
    torch.cuda.synchronize()
    assert_close(outd.cpu(), ref, TOL, "tiled gated resid")

    # column window of a wider output (kv_y into the packed qkv)
    L = 40
    qkv = torch.randn(L + M, 3 * N, generator=g)
    qkvd = qkv.to(dev)
    ns2lib.linear_i8_tiled(at, wt, sd, qkvd, M, N, K, ldc=3 * N, cOff=L * 3 * N + N)
    ref = qkv.double().clone()
    O.linear_i8(x.double(), q, s.double(), out=ref, ldc=3 * N, cOff=L * 3 * N + N)
    torch.cuda.synchronize()
    got = qkvd.cpu()
    assert torch.equal(got[:L], qkv[:L]) and torch.equal(got[L:, :N], qkv[L:, :N])
    assert torch.equal(got[L:, 2 * N:], qkv[L:, 2 * N:])
    assert_close(got, ref, TOL, "tiled column window")


def test_tile_i8_weight_glu(ns2lib):
    N, K = 1024, 256
    q, _ = int8_weight(N, K, gen(16))
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight_glu(q.to(dev), wt, N, K)
    torch.cuda.synchronize()
    got = untile_w(wt.cpu(), N, K)
    c = torch.arange(N)
    src = torch.where(c % 64 < 32, 32 * (c // 64) + c % 64, N // 2 + 32 * (c // 64) + c % 64 - 32)
    assert torch.equal(got, q[src])
    assert sorted(src.tolist()) == list(range(N))


@pytest.mark.parametrize("M,N,K,act", [
    (3952, 8192, 1536, "silu"),   # the DiT MLP
    (256, 8192, 1536, "silu"),    # text refine blocks
    (97, 1024, 512, "gelu_tanh"),
    (1, 512, 256, "silu"),
])
def test_linear_i8_glu_rot_tiled(ns2lib, M, N, K, act):
    """w12 GEMM + GLU + rotation in one kernel: against the three separate ops (rounding-level
    differences in a few elements: the kernels may contract the scale-and-bias multiply-adds
    differently, and the rotation spreads a group's rounding over its outputs), and against
    the oracle."""
    g = gen(M + N + K)
    x = torch.randn(M, K, generator=g)
    q, s = int8_weight(N, K, g)
    bias = torch.randn(N, generator=g) * 0.1
    I = N // 2
    xd, qd, sd, bd = x.to(dev), q.to(dev), s.reshape(-1).to(dev), bias.to(dev)
    at = tiled_operand(M, K)
    ns2lib.rotate_f16(xd, K, at, K, M, K, tiled=True)
    wglu = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight_glu(qd, wglu, N, K)
    y = tiled_operand(M, I)
    ns2lib.linear_i8_glu_rot_tiled(at, wglu, sd, y, M, N, K, bias=bd, alpha=0.75, act=act)
    # the unfused sequence
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(qd, wt, N, K)
    h = torch.empty(M, N, device=dev)
    ns2lib.linear_i8_tiled(at, wt, sd, h, M, N, K, bias=bd, alpha=0.75)
    y2 = tiled_operand(M, I)
    ns2lib.glu_rotate_f16(h, y2, M, I, act, tiled=True)
    torch.cuda.synchronize()
    got = untile_a(y.cpu(), M, I)
    a, b = f16_as_float(got), f16_as_float(untile_a(y2.cpu(), M, I))
    assert (a - b).abs().max() <= 2.0 ** -10 * b.abs().max()
    assert (a != b).float().mean() < 0.01
    ref = O.rotate(O.glu(O.linear_i8(x.double(), q, s.double(), alpha=0.75, bias=bias.double()), act))
    assert_close(a, ref, TOL, f"glu_rot {M}x{N}x{K} {act}")


def test_linear_i8_tiled_errors(ns2lib):
    at = torch.empty(64, 256, dtype=torch.int16, device=dev)
    wt = torch.empty(96 * 256, dtype=torch.int8, device=dev)
    sc = torch.ones(96, device=dev)
    out = torch.empty(64, 96, device=dev)
    with pytest.raises(RuntimeError, match="N %"):
        ns2lib.linear_i8_tiled(at, wt, sc, out, 64, 96, 256)
    with pytest.raises(RuntimeError, match="multiples of 64"):
        ns2lib.tile_i8_weight(wt, wt, 96, 256)


# ----------------------------------------------------------------------------- bf16 linear

@pytest.mark.parametrize("M,N,K", [(3952, 1536, 64), (3952, 1536, 1536), (3952, 64, 1536),
                                   (256, 1536, 640), (256, 640, 2048), (256, 4096, 640), (37, 200, 1024),
                                   (1, 9216, 1536), (1, 1536, 256), (3, 3072, 1536)])
def test_linear_bf16(ns2lib, M, N, K):
    g = gen(M + N + K)
    x = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    ref = O.linear_bf16(x.double(), w, bias=bias.double())
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16(x.to(dev), K, w.view(torch.int16).to(dev), out, M, N, K, bias=bias.to(dev))
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, TOL, f"linear_bf16 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(256, 640, 2048), (40, 96, 512)])
def test_linear_bf16_split_k_epilogue(ns2lib, M, N, K):
    """Short sequences take 64x64 tiles with K split over blocks and a reduce kernel that applies
    the epilogue once: alpha, bias, an added tensor and GELU(tanh), then a gated += into a column
    window of a wider output."""
    g = gen(M * 5 + N)
    x = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    add = torch.randn(M, N, generator=g) * 0.1
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16(x.to(dev), K, w.view(torch.int16).to(dev), out, M, N, K, bias=bias.to(dev),
                       add=add.to(dev), alpha=0.5, act="gelu_tanh")
    torch.cuda.synchronize()
    ref = O.linear_bf16(x.double(), w, alpha=0.5, bias=bias.double(), add=add.double(), act="gelu_tanh")
    assert_close(out.cpu(), ref, TOL, f"split-K epilogue {M}x{N}x{K}")
    ldc, cOff = N + 32, 16
    base = torch.randn(M * ldc, generator=g)
    gate = torch.randn(N + 8, generator=g)
    outd = base.to(dev)
    ns2lib.linear_bf16(x.to(dev), K, w.view(torch.int16).to(dev), outd, M, N, K, ldc=ldc, cOff=cOff,
                       resid=True, gate=gate.to(dev), gOff=8)
    torch.cuda.synchronize()
    ref = O.linear_bf16(x.double(), w, out=base.double().clone(), resid=True, gate=gate.double(), gOff=8,
                        ldc=ldc, cOff=cOff)
    assert_close(outd.cpu(), ref, TOL, f"split-K gated += {M}x{N}x{K}")


def test_linear_bf16_gemv_silu_resid(ns2lib):
    g = gen(21)
    x = torch.randn(1, 256, generator=g)
    w = (torch.randn(1536, 256, generator=g) * 0.05).to(torch.bfloat16)
    out = torch.empty(1, 1536, device=dev)
    ns2lib.linear_bf16(x.to(dev), 256, w.view(torch.int16).to(dev), out, 1, 1536, 256, act="silu")
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.linear_bf16(x.double(), w, act="silu"), TOL_F32 * 10, "gemv silu")
    base = torch.randn(1, 1536, generator=g)
    outd = base.to(dev)
    ns2lib.linear_bf16(x.to(dev), 256, w.view(torch.int16).to(dev), outd, 1, 1536, 256, resid=True)
    torch.cuda.synchronize()
    assert_close(outd.cpu(), O.linear_bf16(x.double(), w, out=base.double().clone(), resid=True), TOL_F32 * 10, "gemv resid")


@pytest.mark.parametrize("M,N,K", [
    (3952, 1536, 1536),   # the SPRINT projection (x += (g - x) W^T)
    (3952, 1536, 64),     # the patch embedder (one k-tile)
    (3952, 64, 1536),     # the final layer (one column tile: split K)
    (97, 320, 512),       # ragged rows, N not a multiple of 128
])
def test_linear_f16w_tiled(ns2lib, M, N, K):
    """bf16 weights re-tiled as fp16 (ns2_tile_bf16_weight) on tiled fp16 operands
    (ns2_to_tiled_f16): a plain store with bias and SiLU, and the residual form with the input
    formed as a difference of two fp32 streams, against the oracle's bf16 linear; the weight
    tiles against the bf16 values rounded to fp16."""
    g = gen(M + 3 * N + K)
    x = torch.randn(M, K, generator=g)
    x2 = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    wt = torch.empty(N * K, dtype=torch.int16, device=dev)
    ns2lib.tile_bf16_weight(w.view(torch.int16).to(dev), wt, N, K)
    torch.cuda.synchronize()
    assert torch.equal(f16_as_float(untile_a(wt.cpu(), N, K)), w.float().half().float())
    at = tiled_operand(M, K)
    ns2lib.to_tiled_f16(x.to(dev), K, at, M, K)
    torch.cuda.synchronize()
    assert torch.equal(f16_as_float(untile_a(at.cpu(), M, K)), x.half().float())
    out = torch.empty(M, N, device=dev)
    ns2lib.linear_f16w_tiled(at, wt, out, M, N, K, bias=bias.to(dev), act="silu")
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.linear_bf16(x.double(), w, bias=bias.double(), act="silu"), TOL,
                 f"linear_f16w_tiled {M}x{N}x{K}")
    # x += (x2 - x) W^T
    ns2lib.to_tiled_f16(x2.to(dev), K, at, M, K, sub=x.to(dev), ldsub=K)
    base = torch.randn(M, N, generator=g)
    outd = base.to(dev)
    ns2lib.linear_f16w_tiled(at, wt, outd, M, N, K, resid=True)
    torch.cuda.synchronize()
    ref = O.linear_bf16((x2 - x).double(), w, out=base.double().clone(), resid=True)
    assert_close(outd.cpu(), ref, TOL, f"linear_f16w_tiled resid {M}x{N}x{K}")


def test_to_tiled_f16_padding(ns2lib):
    """Rows past M up to the 64-row padding are written as zeros."""
    M, K = 70, 128
    x = torch.randn(M, K, generator=gen(5))
    at = torch.full(((M + 63) // 64 * 64, K), 0x3C00, dtype=torch.int16, device=dev)  # 1.0 everywhere
    ns2lib.to_tiled_f16(x.to(dev), K, at, M, K)
    torch.cuda.synchronize()
    full = f16_as_float(untile_a(at.cpu(), 128, K))
    assert torch.equal(full[:M], x.half().float()) and (full[M:] == 0).all()


@pytest.mark.parametrize("rms", [False, True])
def test_norm_mod_f16(ns2lib, rms):
    """normMod written as the tiled fp16 operand, without the rotation (the final layer)."""
    rows, cols = 300, 1536
    g = gen(44 + rms)
    x = torch.randn(rows, cols, generator=g) * 3 + 0.5
    mod = torch.randn(2 * cols, generator=g) * 0.1
    w = torch.randn(cols, generator=g) * 0.02 if rms else None
    y = tiled_operand(rows, cols)
    ns2lib.norm_mod_f16(x.to(dev), mod.to(dev), 0, cols, rows, cols, w.to(dev) if rms else None, y)
    torch.cuda.synchronize()
    ref = O.norm_mod(x.double(), mod.double(), 0, cols, w.double() if rms else None)
    assert_close(f16_as_float(untile_a(y.cpu(), rows, cols)), ref, TOL_F16_OUT, f"norm_mod_f16 rms={rms}")


@pytest.mark.parametrize("N,K", [(12288, 1536), (1000, 512), (77, 2048)])
def test_linear_bf16_gemv_one_row(ns2lib, N, K):
    """One-row bf16 linears with K a multiple of 512 (the adaLN projections, stacked): the
    multi-column GEMV, plain with bias and SiLU, and a gated += into a column window; N not a
    multiple of the 16 columns of a block."""
    g = gen(N + K)
    x = torch.randn(1, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn(N, generator=g) * 0.1
    wd = w.view(torch.int16).to(dev)
    out = torch.empty(1, N, device=dev)
    ns2lib.linear_bf16(x.to(dev), K, wd, out, 1, N, K, bias=bias.to(dev), act="silu")
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.linear_bf16(x.double(), w, bias=bias.double(), act="silu"), TOL_F32 * 10,
                 f"gemv one row {N}x{K}")
    base = torch.randn(1, N + 40, generator=g)
    gate = torch.randn(N + 8, generator=g)
    outd = base.to(dev)
    ns2lib.linear_bf16(x.to(dev), K, wd, outd, 1, N, K, ldc=N + 40, cOff=24, resid=True, gate=gate.to(dev), gOff=8)
    torch.cuda.synchronize()
    ref = O.linear_bf16(x.double(), w, out=base.double().clone(), resid=True, gate=gate.double(), gOff=8,
                        ldc=N + 40, cOff=24)
    assert_close(outd.cpu(), ref, TOL_F32 * 10, f"gemv one row gated += {N}x{K}")


# ----------------------------------------------------------------------------- attention

def _attn_inputs(seed, Lq_img, T, heads=16, hd=96):
    g = gen(seed)
    Dm = heads * hd
    Lk = Lq_img + T
    q = torch.randn(Lq_img, Dm, generator=g)
    k = torch.randn(Lk, Dm, generator=g)
    v = torch.randn(Lk, Dm, generator=g)
    w = torch.rand(T, generator=g) + 0.5
    return q, k, v, torch.log(w)


@pytest.mark.parametrize("hgrid,wgrid,T", [(48, 48, 128), (76, 52, 256), (5, 7, 3), (16, 16, 0)])
def test_joint_attention_rope_bias(ns2lib, hgrid, wgrid, T):
    """Config 0/2 op: RoPE on image q/k rows, log-weight bias on text keys."""
    L = hgrid * wgrid
    q, k, v, lb = _attn_inputs(L + T, L, T)
    cs, sin_off = O.rope2d_table(hgrid, wgrid)
    half = 48
    cos = cs[:sin_off].reshape(L, half).double()
    sin = cs[sin_off:].reshape(L, half).double()
    ref = O.joint_attention_op(q.double(), k.double(), v.double(), L, cos, sin,
                               key_bias=lb.double() if T else None, bias_start=L)
    o = torch.empty(L, 1536, device=dev)
    ns2lib.attention(q.to(dev), k.to(dev), v.to(dev), o, Lq=L, Lk=L + T, H=16, D=96, ldq=1536,
                     ldk=1536, ldv=1536, ldo=1536, key_bias=lb.to(dev) if T else None, biasStart=L,
                     rope_cs=cs.to(dev), sin_off=sin_off, rope_rows=L)
    torch.cuda.synchronize()
    assert_close(o.cpu(), ref, TOL, f"joint attention {hgrid}x{wgrid}+{T}")


def test_attention_batch2_config2(ns2lib):
    """Config 2: 832x1216 (76x52 latent), 256 text tokens, batch 2 in one call; every one of the
    2 x 16 (batch element, head) units is checked against the oracle."""
    L, T = 76 * 52, 256
    qs, ks, vs, bs = zip(*[_attn_inputs(100 + b, L, T) for b in range(2)])
    cs, sin_off = O.rope2d_table(76, 52)
    q = torch.stack(qs).to(dev)
    k = torch.stack(ks).to(dev)
    v = torch.stack(vs).to(dev)
    bias = torch.stack(bs).to(dev)
    o = torch.empty(2, L, 1536, device=dev)
    ns2lib.attention(q, k, v, o, Lq=L, Lk=L + T, H=16, D=96, ldq=1536, ldk=1536, ldv=1536, ldo=1536,
                     batch=2, qBatch=L * 1536, kBatch=(L + T) * 1536, vBatch=(L + T) * 1536,
                     oBatch=L * 1536, key_bias=bias, biasStart=L, biasBatch=T,
                     rope_cs=cs.to(dev), sin_off=sin_off, rope_rows=L)
    torch.cuda.synchronize()
    cos = cs[:sin_off].reshape(L, 48)
    sin = cs[sin_off:].reshape(L, 48)
    got = o.cpu()
    for b in range(2):
        # fp32 oracle over all 16 heads (fp32 rounding is ~1e-6, far below the 2e-3 bar)
        ref = O.joint_attention_op(qs[b], ks[b], vs[b], L, cos, sin, key_bias=bs[b], bias_start=L)
        for h in range(16):
            sl = slice(h * 96, (h + 1) * 96)
            assert_close(got[b, :, sl], ref[:, sl], TOL, f"config2 batch {b} head {h}")
        assert_close(got[b], ref, TOL, f"config2 batch {b} all heads")


def test_attention_wide_blocks(ns2lib):
    """Batch 8 x 16 heads at a ragged size (21x29 latent = 609 queries, 77 text keys, 686 keys in
    11 tiles, the last one part padding), with the fused q/k head norms, RoPE and key bias: 2 query
    blocks of 512 x 128 (batch, head) pairs fill the chip, so the call runs the 512-query-block
    kernel. Checked against the oracle per batch element, and against the same attention run one
    batch element per call (16 pairs: the 256-query-block kernel), which must agree to fp32
    rounding (the kernels differ only in the order of the row sums)."""
    hh, ww, T, B, Dm = 21, 29, 77, 8, 1536
    L = hh * ww
    Lk = L + T
    g = gen(97)
    q = torch.randn(B, L, Dm, generator=g)
    k = torch.randn(B, Lk, Dm, generator=g)
    v = torch.randn(B, Lk, Dm, generator=g)
    lb = torch.log(torch.rand(B, T, generator=g) + 0.5)
    qn = torch.randn(96, generator=g) * 0.5 + 1
    kn = torch.randn(96, generator=g) * 0.5 + 1
    cs, sin_off = O.rope2d_table(hh, ww)
    qd, kd, vd, lbd = q.to(dev), k.to(dev), v.to(dev), lb.to(dev)
    qnd, knd, csd = qn.to(dev), kn.to(dev), cs.to(dev)
    common = dict(Lq=L, Lk=Lk, H=16, D=96, ldq=Dm, ldk=Dm, ldv=Dm, ldo=Dm, biasStart=L, q_norm=qnd,
                  k_norm=knd, rope_cs=csd, sin_off=sin_off, rope_rows=L)
    wide = torch.empty(B, L, Dm, device=dev)
    ns2lib.attention(qd, kd, vd, wide, batch=B, qBatch=L * Dm, kBatch=Lk * Dm, vBatch=Lk * Dm, oBatch=L * Dm,
                     key_bias=lbd, biasBatch=T, **common)
    narrow = torch.empty(B, L, Dm, device=dev)
    for b in range(B):
        ns2lib.attention(qd[b], kd[b], vd[b], narrow[b], key_bias=lbd[b], **common)
    torch.cuda.synchronize()
    wide, narrow = wide.cpu(), narrow.cpu()
    assert_close(wide, narrow, 1e-5, "512-query blocks vs 256-query blocks")
    bias = torch.zeros(Lk, dtype=torch.float64)
    for b in range(B):
        qb = q[b].double().clone()
        kb = k[b].double().clone()
        O.head_norm_rope(qb, qn.double(), L, 16, 96, Dm, cs=cs, sinOff=sin_off)
        O.head_norm_rope(kb, kn.double(), L, 16, 96, Dm, cs=cs, sinOff=sin_off)
        O.head_norm_rope(kb, kn.double(), T, 16, 96, Dm, rowOff=L)
        bias[L:] = lb[b].double()
        ref = O.attention_heads(qb, kb, v[b].double(), 16, 96, bias)
        assert_close(wide[b], ref, TOL, f"wide blocks, batch element {b}")


@pytest.mark.parametrize("pad", [0, 1])
def test_attention_text_view(ns2lib, pad):
    """ns2_attention_text: the DiT's joint attention with the text keys and values in a second
    view (the stacked kv_y product, row stride 27648 at the block's column), against
    ns2_attention on the same rows concatenated into one packed qkv buffer: identical results,
    and the oracle. pad=1 makes the views unaligned (per-element pack path)."""
    L, T, Dm = 6 * 8, 37, 1536
    ld = 3 * Dm + pad
    ldt = 9 * 2 * Dm + 4 * pad
    slot = 4 * 2 * Dm + pad
    g = gen(71 + pad)
    img = torch.randn(L, ld, generator=g)
    txt = torch.randn(T, ldt, generator=g)
    qn = torch.randn(96, generator=g) * 0.5 + 1
    kn = torch.randn(96, generator=g) * 0.5 + 1
    lb = torch.log(torch.rand(T, generator=g) + 0.5)
    cs, sin_off = O.rope2d_table(6, 8)
    # the same keys in one buffer: text rows carry k|v at the columns of the image rows
    joint = torch.zeros(L + T, ld)
    joint[:L] = img
    joint[L:, pad + Dm:pad + 3 * Dm] = txt[:, slot:slot + 2 * Dm]
    o1 = torch.empty(L, Dm, device=dev)
    o2 = torch.empty(L, Dm, device=dev)
    kw = dict(Lq=L, Lk=L + T, H=16, D=96, ldq=ld, ldk=ld, ldv=ld, ldo=Dm, qOff=pad, kOff=Dm + pad,
              vOff=2 * Dm + pad, key_bias=lb.to(dev), biasStart=L, q_norm=qn.to(dev), k_norm=kn.to(dev),
              rope_cs=cs.to(dev), sin_off=sin_off, rope_rows=L)
    jd = joint.to(dev)
    ns2lib.attention(jd, jd, jd, o1, **kw)
    imgd, txtd = img.to(dev), txt.to(dev)
    ns2lib.attention_text(imgd, imgd, imgd, o2, k_text=txtd[:, slot:], v_text=txtd[:, slot + Dm:], ld_text=ldt,
                          text_start=L, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o1.cpu(), o2.cpu()), "text view differs from the packed buffer"
    ref_buf = joint.double()[:, pad:pad + 3 * Dm].clone()
    O.head_norm_rope(ref_buf, qn.double(), L, 16, 96, 3 * Dm, colOff=0, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref_buf, kn.double(), L, 16, 96, 3 * Dm, colOff=Dm, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref_buf, kn.double(), T, 16, 96, 3 * Dm, colOff=Dm, rowOff=L)
    bias = torch.cat([torch.zeros(L, dtype=torch.float64), lb.double()])
    ref = O.attention_heads(ref_buf[:L, :Dm], ref_buf[:, Dm:2 * Dm], ref_buf[:, 2 * Dm:], 16, 96, bias)
    assert_close(o2.cpu(), ref, TOL, f"attention with a text view (pad {pad})")


@pytest.mark.parametrize("L,T,text_view,lora", [
    (3952, 256, True, False),   # the 832x1216 joint block: text keys from the stacked kv_y view
    (4096, 256, True, False),   # 1024x1024: whole row tiles, 68 key tiles
    (496, 40, False, False),    # text rows inside the qkv buffer, a ragged last key tile
    (512, 0, False, True),      # image-only keys, a LoRA term on the qkv weight
])
def test_qkv_vpack_attention(ns2lib, L, T, text_view, lora):
    """ns2_linear_i8_tiled_vpack + ns2_attention_vpacked (the values go from the qkv GEMM's
    epilogue straight into the attention's fp16 layout) against ns2_linear_i8_tiled +
    ns2_attention / ns2_attention_text: the q|k columns and the attention output are
    bit-identical, and the v columns of the qkv buffer are neither written nor read."""
    Dm, H, HD, K = 1536, 16, 96, 1536
    N, Lk = 3 * Dm, L + T
    g = gen(L + T)
    x = torch.randn(L, K, generator=g)
    q8, s8 = int8_weight(N, K, g)
    bias = (torch.randn(N, generator=g) * 0.1).to(dev)
    sd = s8.reshape(-1).to(dev)
    wt = torch.empty(N * K, dtype=torch.int8, device=dev)
    ns2lib.tile_i8_weight(q8.to(dev), wt, N, K)
    at = tiled_operand(L, K)
    ns2lib.rotate_f16(x.to(dev), K, at, K, L, K, tiled=True)
    lo = None
    if lora:
        R = 32
        lo = ((torch.randn(R, K, generator=g) * 0.05).half().to(dev),
              (torch.randn(N, R, generator=g) * 0.05).half().to(dev), R)
    rows = L if text_view else Lk
    txt = torch.randn(T, 2 * Dm, generator=g).to(dev)
    qn = (torch.randn(HD, generator=g) * 0.5 + 1).to(dev)
    kn = (torch.randn(HD, generator=g) * 0.5 + 1).to(dev)
    lb = torch.log(torch.rand(T, generator=g) + 0.5).to(dev) if T else None
    hgrid = {3952: 52, 4096: 64}.get(L, 16)
    cs, sin_off = O.rope2d_table(hgrid, L // hgrid)
    kw = dict(Lq=L, Lk=Lk, H=H, D=HD, ldq=3 * Dm, ldk=3 * Dm, ldv=3 * Dm, ldo=Dm, qOff=0, kOff=Dm, vOff=2 * Dm,
              key_bias=lb, biasStart=L, q_norm=qn, k_norm=kn, rope_cs=cs.to(dev), sin_off=sin_off, rope_rows=L)
    tv = dict(k_text=txt[:, :Dm], v_text=txt[:, Dm:], ld_text=2 * Dm, text_start=L) if text_view else {}

    qkv1 = torch.empty(rows, 3 * Dm, device=dev)
    ns2lib.linear_i8_tiled(at, wt, sd, qkv1, L, N, K, bias=bias, ldc=3 * Dm, lora=lo)
    if T and not text_view:
        qkv1[L:, Dm:] = txt
    o1 = torch.empty(L, Dm, device=dev)
    if text_view:
        ns2lib.attention_text(qkv1, qkv1, qkv1, o1, **tv, **kw)
    else:
        ns2lib.attention(qkv1, qkv1, qkv1, o1, **kw)

    qkv2 = torch.full((rows, 3 * Dm), float("nan"), device=dev)
    vpk = torch.empty(ns2lib.attention_vpack_bytes(Lk, H, HD) // 2, dtype=torch.int16, device=dev)
    ns2lib.linear_i8_tiled_vpack(at, wt, sd, qkv2, L, N, K, vpk, vcol0=2 * Dm, H=H, D=HD, Lk=Lk, bias=bias,
                                 ldc=3 * Dm, lora=lo)
    if T and not text_view:
        qkv2[L:, Dm:] = txt
    o2 = torch.empty(L, Dm, device=dev)
    ns2lib.attention_vpacked(qkv2, qkv2, qkv2, o2, vpk, L, **tv, **kw)
    torch.cuda.synchronize()
    assert torch.equal(qkv1[:L, :2 * Dm].cpu(), qkv2[:L, :2 * Dm].cpu()), "q|k columns differ"
    assert torch.isnan(qkv2[:L, 2 * Dm:]).all().item(), "the v columns of qkv were written"
    assert torch.equal(o1.cpu(), o2.cpu()), f"packed values change the attention (L {L}, T {T})"
    assert torch.isfinite(o2).all().item()


def test_qkv_vpack_errors(ns2lib):
    vpk = torch.empty(1024, dtype=torch.int16, device=dev)
    at = tiled_operand(64, 256)
    wt = torch.empty(192 * 256, dtype=torch.int8, device=dev)
    sc = torch.ones(192, device=dev)
    out = torch.empty(64, 192, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        ns2lib.linear_i8_tiled_vpack(at, wt, sc, out, 40, 192, 256, vpk, vcol0=128, H=2, D=32, Lk=64)
    with pytest.raises(RuntimeError, match="must end the output"):
        ns2lib.linear_i8_tiled_vpack(at, wt, sc, out, 64, 192, 256, vpk, vcol0=64, H=2, D=32, Lk=64)
    q = torch.zeros(64, 3 * 96, device=dev)
    o = torch.empty(64, 96, device=dev)
    with pytest.raises(RuntimeError, match="v_rows"):
        ns2lib.attention_vpacked(q, q, q, o, vpk, 8, Lq=64, Lk=64, H=1, D=96, ldq=288, ldk=288, ldv=288, ldo=96,
                                 kOff=96, vOff=192)


@pytest.mark.parametrize("pad", [0, 1])
def test_attention_strided_qkv_views(ns2lib, pad):
    """q/k/v as column windows of one packed [Lk, 3D] buffer, like the DiT's qkv
    (app/models/nanosaur2.js:205-208), with fused per-head norms (the headNorm calls).
    pad=1 shifts every window by one float and makes the row stride odd, so the views are
    not 16-byte aligned and the per-element pack path runs instead of the vectorized one."""
    L, T, Dm = 130, 20, 1536
    ld = 3 * Dm + pad
    g = gen(31)
    qkv = torch.randn(L + T, ld, generator=g)
    qn = torch.randn(96, generator=g) * 0.5 + 1
    kn = torch.randn(96, generator=g) * 0.5 + 1
    cs, sin_off = O.rope2d_table(10, 13)
    lb = torch.log(torch.rand(T, generator=g) + 0.5)
    o = torch.empty(L, Dm, device=dev)
    qkv_d = qkv.to(dev)
    ns2lib.attention(qkv_d, qkv_d, qkv_d, o, Lq=L, Lk=L + T, H=16, D=96, ldq=ld,
                     ldk=ld, ldv=ld, ldo=Dm, qOff=pad, kOff=Dm + pad, vOff=2 * Dm + pad, key_bias=lb.to(dev),
                     biasStart=L, q_norm=qn.to(dev), k_norm=kn.to(dev), rope_cs=cs.to(dev),
                     sin_off=sin_off, rope_rows=L)
    torch.cuda.synchronize()
    ref_buf = qkv.double()[:, pad:pad + 3 * Dm].clone()
    O.head_norm_rope(ref_buf, qn.double(), L, 16, 96, 3 * Dm, colOff=0, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref_buf, kn.double(), L, 16, 96, 3 * Dm, colOff=Dm, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref_buf, kn.double(), T, 16, 96, 3 * Dm, colOff=Dm, rowOff=L)
    bias = torch.cat([torch.zeros(L, dtype=torch.float64), lb.double()])
    ref = O.attention_heads(ref_buf[:L, :Dm], ref_buf[:, Dm:2 * Dm], ref_buf[:, 2 * Dm:], 16, 96, bias)
    assert_close(o.cpu(), ref, TOL, f"strided qkv + fused head norms (pad {pad})")


@pytest.mark.parametrize("Lk", [64, 100, 150, 200, 257])
def test_attention_few_key_tiles(ns2lib, Lk):
    """1 to 5 key tiles of 64: the load pipeline's prologue and tail with fewer tiles than stages."""
    g = gen(Lk)
    Lq, H, Dh = 70, 2, 96
    q = torch.randn(Lq, H * Dh, generator=g)
    k = torch.randn(Lk, H * Dh, generator=g)
    v = torch.randn(Lk, H * Dh, generator=g)
    kb = torch.randn(Lk, generator=g)
    o = torch.empty(Lq, H * Dh, device=dev)
    # bias on keys [30, Lk): the biased tiles start inside the first tile
    ns2lib.attention(q.to(dev), k.to(dev), v.to(dev), o, Lq=Lq, Lk=Lk, H=H, D=Dh, ldq=H * Dh,
                     ldk=H * Dh, ldv=H * Dh, ldo=H * Dh, key_bias=kb[30:].to(dev), biasStart=30)
    torch.cuda.synchronize()
    bias = torch.zeros(Lk, dtype=torch.float64)
    bias[30:] = kb[30:].double()
    ref = O.attention_heads(q.double(), k.double(), v.double(), H, Dh, bias=bias)
    assert_close(o.cpu(), ref, TOL, f"Lk={Lk}")


@pytest.mark.parametrize("Dh", [32, 64, 128])
def test_attention_head_dims(ns2lib, Dh):
    g = gen(Dh)
    Lq, Lk, H = 200, 333, 3
    q = torch.randn(Lq, H * Dh, generator=g)
    k = torch.randn(Lk, H * Dh, generator=g)
    v = torch.randn(Lk, H * Dh, generator=g)
    o = torch.empty(Lq, H * Dh, device=dev)
    ns2lib.attention(q.to(dev), k.to(dev), v.to(dev), o, Lq=Lq, Lk=Lk, H=H, D=Dh, ldq=H * Dh,
                     ldk=H * Dh, ldv=H * Dh, ldo=H * Dh)
    torch.cuda.synchronize()
    assert_close(o.cpu(), O.attention_heads(q.double(), k.double(), v.double(), H, Dh), TOL, f"D={Dh}")


# ----------------------------------------------------------------------------- row kernels

@pytest.mark.parametrize("rms,cols", [(True, 1536), (False, 1536), (True, 4096), (False, 3840), (True, 512)])
def test_norm_mod(ns2lib, rms, cols):
    """normMod and the fused normMod + rotation. 1536 columns is the DiT's width; 512 and 4096
    are the smallest and widest groups per row of the modulation hoisted with the row (2) and
    loaded per group (16), 3840 one more width above the hoisting limit."""
    g = gen(41 + cols)
    rows = 517
    x = torch.randn(rows, cols, generator=g) * 3 + 0.5
    mod = torch.randn(6 * cols, generator=g) * 0.1
    w = torch.randn(cols, generator=g) * 0.02 if rms else None
    y = torch.empty(rows, cols, device=dev)
    ns2lib.norm_mod(x.to(dev), mod.to(dev), 3 * cols, 4 * cols, rows, cols, w.to(dev) if rms else None, y)
    torch.cuda.synchronize()
    ref = O.norm_mod(x.double(), mod.double(), 3 * cols, 4 * cols, w.double() if rms else None)
    assert_close(y.cpu(), ref, TOL_F32, f"norm_mod rms={rms} cols={cols}")
    yr = torch.empty(rows, cols, dtype=torch.int16, device=dev)
    ns2lib.norm_mod_rotate_f16(x.to(dev), mod.to(dev), 3 * cols, 4 * cols, rows, cols, w.to(dev) if rms else None, yr)
    torch.cuda.synchronize()
    assert_close(f16_as_float(yr.cpu()), O.rotate(ref), TOL_F16_OUT, f"norm_mod_rotate rms={rms} cols={cols}")


def test_head_norm(ns2lib):
    g = gen(51)
    L, T, Dm = 77, 9, 1536
    X = torch.randn(L + T, 3 * Dm, generator=g)
    w = torch.randn(96, generator=g)
    cs, sin_off = O.rope2d_table(7, 11)
    Xd = X.to(dev)
    ns2lib.head_norm(Xd, w.to(dev), L, 16, 96, 3 * Dm, colOff=Dm, cs=cs.to(dev), sinOff=sin_off)
    ns2lib.head_norm(Xd, w.to(dev), T, 16, 96, 3 * Dm, colOff=Dm, rowOff=L)
    torch.cuda.synchronize()
    ref = X.double().clone()
    O.head_norm_rope(ref, w.double(), L, 16, 96, 3 * Dm, colOff=Dm, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref, w.double(), T, 16, 96, 3 * Dm, colOff=Dm, rowOff=L)
    assert_close(Xd.cpu(), ref, TOL_F32, "head_norm")


def test_head_norm2(ns2lib):
    """Gemma3's q norms (4 heads of 256) and k norm (1 head) with RoPE in one launch, against
    two ns2_head_norm calls (bit-exact) and the oracle, on packed q/k/v rows (ld 1536)."""
    g = gen(52)
    L, D, ld = 37, 256, 1536
    X = torch.randn(L, ld, generator=g)
    wq = torch.randn(D, generator=g)
    wk = torch.randn(D, generator=g)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * torch.rand(D // 2, generator=g, dtype=torch.float64)[None]
    cs = torch.cat([ang.cos().flatten(), ang.sin().flatten()]).float()
    sin_off = L * D // 2
    Xd, X2 = X.to(dev), X.to(dev)
    ns2lib.head_norm2(Xd, wq.to(dev), 4, wk.to(dev), 1, L, D, ld, cs=cs.to(dev), sinOff=sin_off)
    ns2lib.head_norm(X2, wq.to(dev), L, 4, D, ld, colOff=0, cs=cs.to(dev), sinOff=sin_off)
    ns2lib.head_norm(X2, wk.to(dev), L, 1, D, ld, colOff=4 * D, cs=cs.to(dev), sinOff=sin_off)
    torch.cuda.synchronize()
    assert torch.equal(Xd, X2), "head_norm2 vs two head_norm launches"
    ref = X.double().clone()
    O.head_norm_rope(ref, wq.double(), L, 4, D, ld, colOff=0, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref, wk.double(), L, 1, D, ld, colOff=4 * D, cs=cs, sinOff=sin_off)
    assert_close(Xd.cpu(), ref, TOL_F32, "head_norm2")


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_glu(ns2lib, act):
    g = gen(61)
    rows, I = 123, 4096
    x = torch.randn(rows, 2 * I, generator=g) * 2
    y = torch.empty(rows, I, device=dev)
    ns2lib.glu(x.to(dev), y, rows, I, act)
    torch.cuda.synchronize()
    ref = O.glu(x.double(), act)
    assert_close(y.cpu(), ref, TOL_F32, f"glu {act}")
    yr = torch.empty(rows, I, dtype=torch.int16, device=dev)
    ns2lib.glu_rotate_f16(x.to(dev), yr, rows, I, act)
    torch.cuda.synchronize()
    assert_close(f16_as_float(yr.cpu()), O.rotate(ref), TOL_F16_OUT, f"glu_rotate {act}")


def test_elementwise_accumulate_rowsum_rmsnorm(ns2lib):
    g = gen(71)
    a = torch.randn(9216, generator=g)
    b = torch.randn(9216, generator=g)
    ad, bd = a.to(dev), b.to(dev)
    y = torch.empty_like(ad)
    for op, ref in [("add", a + b), ("sub", a - b), ("silu", torch.nn.functional.silu(a)), ("copy", a)]:
        ns2lib.elementwise(op, ad, bd, y, a.numel())
        torch.cuda.synchronize()
        assert_close(y.cpu(), ref, TOL_F32, f"elementwise {op}")
        # the per-element kernel: a length that is not a multiple of 4, and views 4 bytes off
        # 16-byte alignment; both kernels give the same values
        y1 = torch.zeros_like(ad)
        ns2lib.elementwise(op, ad, bd, y1, a.numel() - 3)
        ns2lib.elementwise(op, ad[1:], bd[1:], y1[1:], 8)
        torch.cuda.synchronize()
        assert torch.equal(y1.cpu()[:a.numel() - 3], y.cpu()[:a.numel() - 3]), f"elementwise {op} (scalar)"
    yd = a.to(dev)
    ns2lib.accumulate(yd, bd, a.numel())
    torch.cuda.synchronize()
    assert_close(yd.cpu(), a + b, TOL_F32, "accumulate")
    x = torch.randn(256, 1536, generator=g)
    w = torch.rand(256, generator=g) + 0.5
    out = torch.empty(1, 1536, device=dev)
    ns2lib.row_sum(x.to(dev), w.to(dev), out, 256, 1536, 1 / w.sum().item())
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.row_sum(x.double(), w.double(), 1 / w.sum().item()), TOL_F32, "row_sum")
    # rows not a multiple of the 16 row-splitting waves, columns not a multiple of 64
    x2 = torch.randn(37, 100, generator=g)
    w2 = torch.rand(37, generator=g)
    out2 = torch.empty(100, device=dev)
    ns2lib.row_sum(x2.to(dev), w2.to(dev), out2, 37, 100, 0.5)
    torch.cuda.synchronize()
    assert_close(out2.cpu(), O.row_sum(x2.double(), w2.double(), 0.5), TOL_F32, "row_sum 37x100")
    # the DiT's block modulations mod + offset_i, all blocks in one launch (exact: one add each)
    mod = torch.randn(9216, generator=g)
    offs = torch.randn(18, 9216, generator=g)
    yrows = torch.empty(18, 9216, device=dev)
    ns2lib.add_rows(mod.to(dev), offs.to(dev), yrows, 18, 9216)
    torch.cuda.synchronize()
    assert torch.equal(yrows.cpu(), mod[None, :] + offs), "add_rows"
    nw = torch.randn(1536, generator=g) * 0.02
    out = torch.empty(256, 1536, device=dev)
    ns2lib.rmsnorm(x.to(dev), nw.to(dev), out, 256, 1536)
    torch.cuda.synchronize()
    assert_close(out.cpu(), O.rms_norm(x.double(), nw.double()), TOL_F32, "rmsnorm")


@pytest.mark.parametrize("with_out", [True, False])
def test_add_rmsnorm(ns2lib, with_out):
    """The Gemma3 sandwich norm: x += rmsnorm(a) * w_add, then y = rmsnorm(x) * w_out
    (app/models/gemma3.js:76-80: ops.rmsnorm, ops.accumulate, ops.rmsnorm), at L = 37 x 640."""
    g = gen(640 + with_out)
    x = torch.randn(37, 640, generator=g) * 20
    a = torch.randn(37, 640, generator=g) * 3
    wa = torch.randn(640, generator=g) * 0.3 + 1
    wo = torch.randn(640, generator=g) * 0.3 + 1
    xd = x.to(dev)
    y = torch.empty(37, 640, device=dev) if with_out else None
    ns2lib.add_rmsnorm(xd, a.to(dev), wa.to(dev), wo.to(dev) if with_out else None, y, 37, 640)
    torch.cuda.synchronize()
    xr = x.double() + O.rms_norm(a.double(), wa.double())
    assert_close(xd.cpu(), xr, TOL_F32, "add_rmsnorm x")
    if with_out:
        assert_close(y.cpu(), O.rms_norm(xr, wo.double()), TOL_F32, "add_rmsnorm y")


@pytest.mark.parametrize("M,K,with_out,bias", [(256, 1024, True, False), (256, 2048, True, True),
                                               (37, 2048, False, False), (5, 1024, True, True)])
def test_linear_bf16_add_rmsnorm(ns2lib, M, K, with_out, bias):
    """Gemma3's output projection and the norms after it in one GEMM + row kernel
    (app/models/gemma3.js:72-80, 83-92): against the two-launch ns2_linear_bf16 + ns2_add_rmsnorm
    (bit-exact where both sum K in the same splits, M > 8) and against the oracle (fp16 products,
    TOL). N = 640; K = 1024 (o) and 2048 (down) give 4 and 8 K splits at 256 rows."""
    N = 640
    g = gen(M * K + with_out)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    x = torch.randn(M, N, generator=g) * 20
    wa = torch.randn(N, generator=g) * 0.3 + 1
    wo = torch.randn(N, generator=g) * 0.3 + 1
    ad, wd, xd = a.to(dev), w.view(torch.int16).to(dev), x.to(dev)
    bd, wad, wod = (b.to(dev) if bias else None), wa.to(dev), wo.to(dev)
    y = torch.empty(M, N, device=dev) if with_out else None
    ns2lib.linear_bf16_add_rmsnorm(ad, K, wd, bd, xd, wad, wod if with_out else None, y, M, N, K)
    # two launches: the projection into t, then the sandwich norm
    t = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16(ad, K, wd, t, M, N, K, bias=bd)
    x2 = x.to(dev)
    y2 = torch.empty(M, N, device=dev) if with_out else None
    ns2lib.add_rmsnorm(x2, t, wad, wod if with_out else None, y2, M, N)
    torch.cuda.synchronize()
    if M > 8:
        assert torch.equal(xd, x2), "fused x vs two launches"
        if with_out:
            assert torch.equal(y, y2), "fused y vs two launches"
    tr = O.linear_bf16(a.double(), w, bias=b.double() if bias else None)
    xr = x.double() + O.rms_norm(tr, wa.double())
    assert_close(xd.cpu(), xr, TOL, "linear_bf16_add_rmsnorm x")
    if with_out:
        assert_close(y.cpu(), O.rms_norm(xr, wo.double()), TOL, "linear_bf16_add_rmsnorm y")


@pytest.mark.parametrize("M,bias", [(256, False), (37, True), (5, False)])
def test_linear_bf16_glu(ns2lib, M, bias):
    """Gemma3's gate/up projection and its GELU-tanh gate in one GEMM + GLU launch
    (app/models/gemma3.js:79-82): against ns2_linear_bf16 + ns2_glu (bit-exact at 256 rows,
    where both take the same K splits) and against the oracle (TOL). N = 2 x 2048, K = 640."""
    N, K, I = 4096, 640, 2048
    g = gen(M + 7 * bias)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    ad, wd, bd = a.to(dev), w.view(torch.int16).to(dev), (b.to(dev) if bias else None)
    y = torch.empty(M, I, device=dev)
    ns2lib.linear_bf16_glu(ad, K, wd, bd, y, M, N, K, "gelu_tanh")
    t = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16(ad, K, wd, t, M, N, K, bias=bd)
    y2 = torch.empty(M, I, device=dev)
    ns2lib.glu(t, y2, M, I, "gelu_tanh")
    torch.cuda.synchronize()
    if M == 256:
        assert torch.equal(y, y2), "fused GLU vs two launches"
    tr = O.linear_bf16(a.double(), w, bias=b.double() if bias else None)
    ref = torch.nn.functional.gelu(tr[:, :I], approximate="tanh") * tr[:, I:]
    assert_close(y.cpu(), ref, TOL, "linear_bf16_glu")


@pytest.mark.parametrize("M,bias,Nd", [(256, False, 640), (37, True, 640), (1, False, 640), (100, True, 192),
                                       (300, False, 640)])  # 304 blocks: one per (16 rows, group), all columns
def test_linear_bf16_glu_down(ns2lib, M, bias, Nd):
    """ns2_linear_bf16_glu_down (Gemma3's gate/up, GELU-tanh gate and down projection,
    app/models/gemma3.js:79-83): the shares per 128-column group, summed, against
    ns2_linear_bf16_glu + ns2_linear_bf16 of its output (the same fp16 roundings of the GLU output
    and of W_d, the products summed in another association: 5e-5 of the largest output where
    that linear runs its matrix-core path; at M <= 8 it runs an fp32 GEMV: TOL), and against the
    oracle in fp64 (TOL). The GLU output itself is bit-identical to ns2_linear_bf16_glu's."""
    N, K, I = 4096, 640, 2048
    g = gen(M * 3 + 5 * bias + Nd)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    wdn = (torch.randn(Nd, I, generator=g) * 0.03).to(torch.bfloat16)
    ad, wd, bd = a.to(dev), w.view(torch.int16).to(dev), (b.to(dev) if bias else None)
    wdd = wdn.view(torch.int16).to(dev)
    wdt = torch.empty(Nd * I, dtype=torch.int16, device=dev)
    ns2lib.tile_bf16_weight(wdd, wdt, Nd, I)
    part = torch.full((I // 128, M, Nd), float("nan"), device=dev)
    ns2lib.linear_bf16_glu_down(ad, K, wd, bd, M, N, K, wdt, Nd, part, "gelu_tanh")
    y = torch.empty(M, I, device=dev)
    ns2lib.linear_bf16_glu(ad, K, wd, bd, y, M, N, K, "gelu_tanh")
    t = torch.empty(M, Nd, device=dev)
    ns2lib.linear_bf16(y, I, wdd, t, M, Nd, I)
    torch.cuda.synchronize()
    assert torch.isfinite(part.cpu()).all(), "every share written"
    got = part.cpu().double().sum(0)
    assert_close(got, t.cpu().double(), 5e-5 if M > 8 else TOL, f"GLU + down vs two launches (M={M}, Nd={Nd})")
    tr = O.linear_bf16(a.double(), w, bias=b.double() if bias else None)
    ref = (torch.nn.functional.gelu(tr[:, :I], approximate="tanh") * tr[:, I:]) @ wdn.double().t()
    assert_close(got, ref, TOL, f"GLU + down vs the oracle (M={M}, Nd={Nd})")


def to_tiled_dev(ns2lib, a):
    """fp32 [M, K] -> the tiled fp16 operand through ns2_to_tiled_f16 (padding rows zero)."""
    M, K = a.shape
    at = tiled_operand(M, K)
    ns2lib.call("ns2_to_tiled_f16", a.data_ptr(), K, None, K, at.data_ptr(), M, K)
    return at


@pytest.mark.parametrize("M,bias", [(256, False), (37, True), (1, False)])
def test_linear_f16w_tiled_head_norm_f16kv(ns2lib, M, bias):
    """The Gemma3 q/k/v projection on the tiled fp16 path (tiled operand, fp16 weight tiles, raw
    split-K products into the head-norm row kernel) against the row-major
    ns2_linear_bf16_head_norm_f16kv: the same fp16 roundings of input and weight, the K sums in
    another association (q heads within 5e-5; the fp16 k/v within one rounding step), and
    against the oracle (TOL)."""
    N, K, D = 1536, 640, 256
    g = gen(M * 11 + bias)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    wq = (torch.randn(D, generator=g) * 0.3 + 1).to(dev)
    wk = (torch.randn(D, generator=g) * 0.3 + 1).to(dev)
    ang = torch.arange(M, dtype=torch.float64)[:, None] * torch.rand(D // 2, generator=g, dtype=torch.float64)[None]
    cs = torch.cat([ang.cos().flatten(), ang.sin().flatten()]).float()
    csd, sin_off = cs.to(dev), M * D // 2
    ad, wd, bd = a.to(dev), w.view(torch.int16).to(dev), (b.to(dev) if bias else None)
    wt = torch.empty(N * K, dtype=torch.int16, device=dev)
    ns2lib.tile_bf16_weight(wd, wt, N, K)
    at = to_tiled_dev(ns2lib, ad)
    y1 = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16_head_norm_f16kv(ad, K, wd, bd, y1, M, N, K, wq, 4, wk, 1, D, y1.data_ptr() + 4 * D * 4, 2 * N,
                                       cs=csd, sin_off=sin_off, rope_rows=M)
    y2 = torch.empty(M, N, device=dev)
    ns2lib.linear_f16w_tiled_head_norm_f16kv(at, wt, bd, y2, M, N, K, wq, 4, wk, 1, D, y2.data_ptr() + 4 * D * 4,
                                             2 * N, cs=csd, sin_off=sin_off, rope_rows=M)
    torch.cuda.synchronize()
    y1, y2 = y1.cpu(), y2.cpu()
    q1, q2 = y1[:, :4 * D].double(), y2[:, :4 * D].double()
    kv1 = y1.view(torch.float16)[:, 8 * D:10 * D].double()
    kv2 = y2.view(torch.float16)[:, 8 * D:10 * D].double()
    # (the row-major path's fp32 GEMV at M <= 8 does not round its input to fp16)
    assert_close(q2, q1, 5e-5 if M > 8 else TOL, f"tiled vs row-major q heads (M={M})")
    assert_close(kv2, kv1, 2e-3, f"tiled vs row-major fp16 k/v (M={M})")
    ref = O.linear_bf16(a.double(), w, bias=b.double() if bias else None)
    O.head_norm_rope(ref, wq.double().cpu(), M, 4, D, N, colOff=0, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref, wk.double().cpu(), M, 1, D, N, colOff=4 * D, cs=cs, sinOff=sin_off)
    assert_close(q2, ref[:, :4 * D], TOL, f"tiled q heads vs the oracle (M={M})")
    assert_close(kv2, ref[:, 4 * D:], TOL, f"tiled fp16 k/v vs the oracle (M={M})")


@pytest.mark.parametrize("M,bias", [(256, False), (37, True), (1, True)])
def test_linear_f16w_tiled_glu_down(ns2lib, M, bias):
    """The Gemma3 gate/up, GLU and down shares on the tiled fp16 path against the row-major
    ns2_linear_bf16_glu_down (5e-4: the K sums in another association, then the GLU output's
    fp16 rounding) and the oracle (TOL)."""
    N, K, I, Nd = 4096, 640, 2048, 640
    g = gen(M * 17 + bias)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    wdn = (torch.randn(Nd, I, generator=g) * 0.03).to(torch.bfloat16)
    ad, wd, bd = a.to(dev), w.view(torch.int16).to(dev), (b.to(dev) if bias else None)
    wt = torch.empty(N * K, dtype=torch.int16, device=dev)
    ns2lib.tile_bf16_weight(wd, wt, N, K)
    wdd = wdn.view(torch.int16).to(dev)
    wdt = torch.empty(Nd * I, dtype=torch.int16, device=dev)
    ns2lib.tile_bf16_weight(wdd, wdt, Nd, I)
    at = to_tiled_dev(ns2lib, ad)
    p1 = torch.empty(I // 128, M, Nd, device=dev)
    ns2lib.linear_bf16_glu_down(ad, K, wd, bd, M, N, K, wdt, Nd, p1, "gelu_tanh")
    p2 = torch.full((I // 128, M, Nd), float("nan"), device=dev)
    ns2lib.linear_f16w_tiled_glu_down(at, wt, bd, M, N, K, wdt, Nd, p2, "gelu_tanh")
    torch.cuda.synchronize()
    s1, s2 = p1.cpu().double().sum(0), p2.cpu().double().sum(0)
    assert torch.isfinite(s2).all(), "every share written"
    # the GLU output is rounded to fp16 before the down product: where the two gate/up K sums
    # differ in their last bits a value can round the other way (one fp16 step, 2^-11)
    assert_close(s2, s1, 5e-4 if M > 8 else TOL, f"tiled vs row-major GLU + down (M={M})")
    tr = O.linear_bf16(a.double(), w, bias=b.double() if bias else None)
    ref = (torch.nn.functional.gelu(tr[:, :I], approximate="tanh") * tr[:, I:]) @ wdn.double().t()
    assert_close(s2, ref, TOL, f"tiled GLU + down vs the oracle (M={M})")


@pytest.mark.parametrize("M,splits", [(256, 16), (37, 4), (1, 1)])
def test_parts_add_rmsnorm_tiled(ns2lib, M, splits):
    """ns2_parts_add_rmsnorm_tiled: x as ns2_parts_add_rmsnorm updates it (bit-exact) and y as
    its fp32 y rounded once to fp16 in the tiled operand layout (bit-exact)."""
    N = 640
    g = gen(M * 19 + splits)
    part = torch.randn(splits, M, N, generator=g).to(dev)
    x = torch.randn(M, N, generator=g) * 20
    wa = (torch.randn(N, generator=g) * 0.3 + 1).to(dev)
    wo = (torch.randn(N, generator=g) * 0.3 + 1).to(dev)
    x1, x2 = x.to(dev), x.to(dev)
    y1 = torch.empty(M, N, device=dev)
    ns2lib.parts_add_rmsnorm(part, splits, None, x1, wa, wo, y1, M, N)
    yt = tiled_operand(M, N)
    ns2lib.parts_add_rmsnorm_tiled(part, splits, None, x2, wa, wo, yt, M, N)
    torch.cuda.synchronize()
    assert torch.equal(x1.cpu(), x2.cpu()), "x"
    got = untile_a(yt.cpu(), M, N).view(torch.float16)
    assert torch.equal(got.view(torch.int16), y1.cpu().half().view(torch.int16)), "tiled fp16 y"


@pytest.mark.parametrize("M,bias,rope", [(256, False, True), (37, True, True), (5, False, False)])
def test_linear_bf16_head_norm(ns2lib, M, bias, rope):
    """Gemma3's q/k/v projection with the q and k head norms (and RoPE) in its split-K sum
    (app/models/gemma3.js:62-67): against the oracle, and where ns2_linear_bf16 takes the same
    matrix-core path (M > 8; at M <= 8 it runs the fp32 GEMV) against ns2_linear_bf16 +
    ns2_head_norm2 (the same sums in a different order: fp32 rounding). N = 4 q heads + 1 k +
    1 v of 256, K = 640; the v columns pass through unnormed."""
    N, K, D = 1536, 640, 256
    g = gen(M + 3 * bias + 11 * rope)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    wq = torch.randn(D, generator=g) * 0.3 + 1
    wk = torch.randn(D, generator=g) * 0.3 + 1
    cs, sin_off = None, 0
    if rope:
        ang = torch.arange(M, dtype=torch.float64)[:, None] * torch.rand(D // 2, generator=g, dtype=torch.float64)[None]
        cs = torch.cat([ang.cos().flatten(), ang.sin().flatten()]).float()
        sin_off = M * D // 2
    ad, wd, bd = a.to(dev), w.view(torch.int16).to(dev), (b.to(dev) if bias else None)
    csd = cs.to(dev) if rope else None
    y = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16_head_norm(ad, K, wd, bd, y, M, N, K, wq.to(dev), 4, wk.to(dev), 1, D, cs=csd, sin_off=sin_off,
                                 rope_rows=M)
    t = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16(ad, K, wd, t, M, N, K, bias=bd)
    ns2lib.head_norm2(t, wq.to(dev), 4, wk.to(dev), 1, M, D, N, cs=csd, sinOff=sin_off)
    torch.cuda.synchronize()
    if M > 8:
        assert_close(y.cpu(), t.cpu().double(), TOL_F32, f"linear_bf16_head_norm vs two launches (M={M})")
    ref = O.linear_bf16(a.double(), w, bias=b.double() if bias else None)
    O.head_norm_rope(ref, wq.double(), M, 4, D, N, colOff=0, cs=cs, sinOff=sin_off)
    O.head_norm_rope(ref, wk.double(), M, 1, D, N, colOff=4 * D, cs=cs, sinOff=sin_off)
    assert_close(y.cpu(), ref, TOL, f"linear_bf16_head_norm (M={M}, bias={bias}, rope={rope})")


@pytest.mark.parametrize("M,bias,rope", [(256, False, True), (37, True, True), (5, False, False)])
def test_linear_bf16_head_norm_f16kv(ns2lib, M, bias, rope):
    """ns2_linear_bf16_head_norm_f16kv: the q heads bit-identical to ns2_linear_bf16_head_norm's,
    the k and v heads its fp32 results rounded to nearest-even fp16 (torch's .half()), written into
    the front half of their own fp32 columns (ldkv = 2N, as the Gemma3 encoder calls it) or into a
    separate buffer with a wider row stride."""
    N, K, D = 1536, 640, 256
    g = gen(M + 5 * bias + 13 * rope)
    a = torch.randn(M, K, generator=g)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    wq = (torch.randn(D, generator=g) * 0.3 + 1).to(dev)
    wk = (torch.randn(D, generator=g) * 0.3 + 1).to(dev)
    csd, sin_off = None, 0
    if rope:
        ang = torch.arange(M, dtype=torch.float64)[:, None] * torch.rand(D // 2, generator=g, dtype=torch.float64)[None]
        csd = torch.cat([ang.cos().flatten(), ang.sin().flatten()]).float().to(dev)
        sin_off = M * D // 2
    ad, wd, bd = a.to(dev), w.view(torch.int16).to(dev), (b.to(dev) if bias else None)
    y = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16_head_norm(ad, K, wd, bd, y, M, N, K, wq, 4, wk, 1, D, cs=csd, sin_off=sin_off, rope_rows=M)
    z = torch.full((M, N), float("nan"), device=dev)
    ns2lib.linear_bf16_head_norm_f16kv(ad, K, wd, bd, z, M, N, K, wq, 4, wk, 1, D, z.data_ptr() + 4 * D * 4, 2 * N,
                                       cs=csd, sin_off=sin_off, rope_rows=M)
    ld = 2 * D + 24
    sep = torch.zeros(M, ld, dtype=torch.float16, device=dev)
    zz = torch.empty(M, N, device=dev)
    ns2lib.linear_bf16_head_norm_f16kv(ad, K, wd, bd, zz, M, N, K, wq, 4, wk, 1, D, sep, ld, cs=csd,
                                       sin_off=sin_off, rope_rows=M)
    torch.cuda.synchronize()
    y, z, zz, sep = y.cpu(), z.cpu(), zz.cpu(), sep.cpu()
    assert torch.equal(z[:, :4 * D], y[:, :4 * D]) and torch.equal(zz[:, :4 * D], y[:, :4 * D])
    kv_ref = y[:, 4 * D:].half().view(torch.int16)
    kv_in = z.view(torch.int16)[:, 8 * D:10 * D]
    assert torch.equal(kv_in, kv_ref), "fp16 k/v in place"
    assert torch.equal(sep[:, :2 * D].view(torch.int16), kv_ref), "fp16 k/v in a separate buffer"
    assert (sep[:, 2 * D:] == 0).all(), "columns past the k/v heads untouched"


@pytest.mark.parametrize("rows,cols", [(64, 3952), (3952, 64), (37, 100), (1, 5)])
def test_transpose(ns2lib, rows, cols):
    """The latent <-> token layout change of forward() (exact)."""
    x = torch.randn(rows, cols, generator=gen(rows * cols))
    y = torch.empty(cols, rows, device=dev)
    ns2lib.transpose(x.to(dev), y, rows, cols)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), x.t().contiguous())


def test_fill_and_errors(ns2lib):
    import ns2

    buf = torch.full((1000,), 7, dtype=torch.int32, device=dev)
    ns2lib.call("ns2_fill_u32", buf.data_ptr(), 0, 1000)
    torch.cuda.synchronize()
    assert (buf.cpu() == 0).all()
    with pytest.raises(ns2.NS2Error, match="multiple of 256"):
        ns2lib.linear_i8(buf, 0, 100, buf, buf, buf, 4, 4, 100)
    with pytest.raises(ns2.NS2Error, match="head dim"):
        ns2lib.attention(buf, buf, buf, buf, Lq=4, Lk=4, H=1, D=80, ldq=80, ldk=80, ldv=80, ldo=80)


# ------------------------------------------------------------------ materialized-path attention

@pytest.mark.parametrize("D,H,group,causal,Lq,Lk", [
    (256, 4, 4, True, 37, 37),    # the Gemma3 text encoder: 4 query heads over 1 K/V head
    (256, 4, 4, True, 256, 256),  # its longest prompt
    (256, 2, 1, False, 5, 300),   # K rows staged in LDS: a ragged last key block, 19 blocks
    (256, 4, 2, True, 100, 37),   # more queries than keys under the causal mask
    (64, 8, 1, False, 50, 70),
    (96, 6, 2, True, 33, 33),
    (40, 3, 3, False, 9, 130),    # head dim not a multiple of 32
    (200, 2, 1, True, 1, 1),
])
def test_attention_rows(ns2lib, D, H, group, causal, Lq, Lk):
    """ns2_attention_rows (ops.attention's materialized path, app/gpu/ops.js:211-241) against the
    oracle's softmax(q k^T / sqrt(D)) v with grouped K/V heads and the causal mask. Head dims that
    are multiples of 16 run the matrix-core kernel (fp16 operands, tolerance 2e-3), the others
    the fp32 kernel (1e-4)."""
    g = gen(D * 7 + H + Lq)
    KH = H // group
    q = torch.randn(Lq, H * D, generator=g)
    k = torch.randn(Lk, KH * D, generator=g)
    v = torch.randn(Lk, KH * D, generator=g)
    o = torch.empty(Lq, H * D, device=dev)
    ns2lib.attention_rows(q.to(dev), k.to(dev), v.to(dev), o, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D,
                          ldk=KH * D, ldv=KH * D, ldo=H * D, group=group, causal=causal)
    torch.cuda.synchronize()
    ref = O.attention_rows(q.double(), k.double(), v.double(), H, D, group=group, causal=causal)
    tol = TOL if D % 16 == 0 else TOL_ROWS
    assert_close(o.cpu(), ref, tol, f"attention_rows D={D} H={H} group={group} causal={causal}")


@pytest.mark.parametrize("pad", [0, 1])
def test_attention_rows_packed_qkv_view(ns2lib, pad):
    """q, k and v as column windows of one [L, 1536] buffer (the Gemma3 layer's fused qkv).
    pad=1 shifts the windows by one float and makes the stride odd: the views are not 16-byte
    aligned and the fp32 kernel runs instead of the matrix-core one."""
    L, H, D = 29, 4, 256
    W = (H + 2) * D + pad
    g = gen(77)
    qkv = torch.randn(L, W, generator=g)
    o = torch.empty(L, H * D, device=dev)
    d = qkv.to(dev)
    ns2lib.attention_rows(d, d, d, o, Lq=L, Lk=L, H=H, D=D, ldq=W, ldk=W, ldv=W, ldo=H * D,
                          qOff=pad, kOff=H * D + pad, vOff=(H + 1) * D + pad, group=H, causal=True)
    torch.cuda.synchronize()
    x = qkv.double()[:, pad:]
    ref = O.attention_rows(x[:, :H * D], x[:, H * D:(H + 1) * D], x[:, (H + 1) * D:], H, D, group=H, causal=True)
    assert_close(o.cpu(), ref, TOL_ROWS if pad else TOL, f"attention_rows packed qkv (pad {pad})")


@pytest.mark.parametrize("D,H,group,causal,Lq,Lk", [
    (256, 4, 4, True, 256, 256),  # the Gemma3 encoder's longest prompt: one pair of key blocks per wave
    (256, 4, 4, True, 37, 37),
    (256, 2, 1, False, 5, 300),   # 19 key blocks: waves with a pair and a lone third block
    (256, 4, 2, True, 100, 37),   # more queries than keys under the causal mask
    (128, 8, 2, True, 300, 300),  # K fragments from memory, 16-byte value loads
    (64, 8, 1, False, 50, 70),    # 8-byte value loads
    (96, 6, 2, True, 33, 33),     # six 16-dim steps: per-element value loads
    (48, 3, 3, False, 9, 130),
    (16, 2, 1, True, 1, 1),
])
def test_attention_rows_f16kv(ns2lib, D, H, group, causal, Lq, Lk):
    """ns2_attention_rows_f16kv against ns2_attention_rows on the same K/V (fp16 values, given to
    the fp32 entry as fp32): both run their products on the same fp16 operands and consume each
    wave's key blocks in the same order, so the outputs are the same bit for bit; and against the
    oracle at the matrix-core tolerance."""
    g = gen(D * 5 + H + Lq + Lk)
    KH = H // group
    q = torch.randn(Lq, H * D, generator=g)
    k = torch.randn(Lk, KH * D, generator=g).half()
    v = torch.randn(Lk, KH * D, generator=g).half()
    o32 = torch.empty(Lq, H * D, device=dev)
    o16 = torch.empty(Lq, H * D, device=dev)
    qd = q.to(dev)
    ns2lib.attention_rows(qd, k.float().to(dev), v.float().to(dev), o32, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D,
                          ldk=KH * D, ldv=KH * D, ldo=H * D, group=group, causal=causal)
    ns2lib.attention_rows_f16kv(qd, k.to(dev), v.to(dev), o16, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D, ldk=KH * D,
                                ldv=KH * D, ldo=H * D, group=group, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(o16.cpu(), o32.cpu()), f"attention_rows_f16kv vs fp32 K/V D={D} Lq={Lq} Lk={Lk}"
    ref = O.attention_rows(q.double(), k.double(), v.double(), H, D, group=group, causal=causal)
    assert_close(o16.cpu(), ref, TOL, f"attention_rows_f16kv D={D} H={H} group={group} causal={causal}")


@pytest.mark.parametrize("L", [1, 37, 256])
def test_gemma_qkv_f16kv_attention(ns2lib, L):
    """The Gemma3 layer's q/k/v projection with fp16 k/v written in place, read by the fp16-K/V
    attention (the encoder's path), against the fp32 projection and ns2_attention_rows: the same
    output bit for bit."""
    N, K, D, H = 1536, 640, 256, 4
    g = gen(L + 901)
    a = torch.randn(L, K, generator=g).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).view(torch.int16).to(dev)
    wq = (torch.randn(D, generator=g) * 0.3 + 1).to(dev)
    wk = (torch.randn(D, generator=g) * 0.3 + 1).to(dev)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * torch.rand(D // 2, generator=g, dtype=torch.float64)[None]
    cs = torch.cat([ang.cos().flatten(), ang.sin().flatten()]).float().to(dev)
    y = torch.empty(L, N, device=dev)
    ns2lib.linear_bf16_head_norm(a, K, w, None, y, L, N, K, wq, H, wk, 1, D, cs=cs, sin_off=L * D // 2, rope_rows=L)
    z = torch.empty(L, N, device=dev)
    ns2lib.linear_bf16_head_norm_f16kv(a, K, w, None, z, L, N, K, wq, H, wk, 1, D, z.data_ptr() + H * D * 4, 2 * N,
                                       cs=cs, sin_off=L * D // 2, rope_rows=L)
    # the fp32 reference path sees the fp16 roundings of its k/v, as the products do
    y[:, H * D:] = y[:, H * D:].half().float()
    o32 = torch.empty(L, H * D, device=dev)
    o16 = torch.empty(L, H * D, device=dev)
    ns2lib.attention_rows(y, y, y, o32, Lq=L, Lk=L, H=H, D=D, ldq=N, ldk=N, ldv=N, ldo=H * D, qOff=0, kOff=H * D,
                          vOff=(H + 1) * D, group=H, causal=True)
    ns2lib.attention_rows_f16kv(z, z, z, o16, Lq=L, Lk=L, H=H, D=D, ldq=N, ldk=2 * N, ldv=2 * N, ldo=H * D, qOff=0,
                                kOff=2 * H * D, vOff=2 * H * D + D, group=H, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o16.cpu(), o32.cpu()), f"Gemma3 q/k/v -> attention with fp16 k/v in place (L={L})"


@pytest.mark.parametrize("L,H,group,D,N,causal", [
    (256, 4, 4, 256, 640, True),  # the Gemma3 layer at its longest prompt
    (37, 4, 4, 256, 640, True),
    (1, 4, 4, 256, 640, True),
    (500, 4, 4, 256, 640, True),   # 128 (query block, head) units: two blocks each, half the columns
    (600, 4, 4, 256, 640, True),   # 152 units: one block each, all the columns
    (100, 8, 2, 128, 256, False),  # other head dims, grouped K/V, several column rounds per wave
    (50, 2, 1, 96, 192, True),
])
def test_attention_rows_f16kv_oproj(ns2lib, L, H, group, D, N, causal):
    """ns2_attention_rows_f16kv_oproj: each head's share of the output projection, summed over the
    heads, against ns2_attention_rows_f16kv followed by ns2_linear_bf16 of the output (the same fp16
    roundings of the attention output and of W_o; the products summed over K in another order:
    5e-5 where that linear runs its matrix-core path), and against the oracle's
    attention and projection in fp64 (TOL)."""
    g = gen(L * 7 + H + D + N)
    KH = H // group
    q = torch.randn(L, H * D, generator=g)
    k = torch.randn(L, KH * D, generator=g).half()
    v = torch.randn(L, KH * D, generator=g).half()
    w = (torch.randn(N, H * D, generator=g) * 0.03).to(torch.bfloat16)
    wd = w.view(torch.int16).to(dev)
    wt = torch.empty(N * H * D, dtype=torch.int16, device=dev)
    ns2lib.tile_bf16_weight(wd, wt, N, H * D)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    part = torch.full((H, L, N), float("nan"), device=dev)
    ns2lib.attention_rows_f16kv_oproj(qd, kd, vd, wt, part, Lq=L, Lk=L, H=H, D=D, ldq=H * D, ldk=KH * D,
                                      ldv=KH * D, N=N, group=group, causal=causal)
    o = torch.empty(L, H * D, device=dev)
    ns2lib.attention_rows_f16kv(qd, kd, vd, o, Lq=L, Lk=L, H=H, D=D, ldq=H * D, ldk=KH * D, ldv=KH * D, ldo=H * D,
                                group=group, causal=causal)
    t = torch.empty(L, N, device=dev)
    ns2lib.linear_bf16(o, H * D, wd, t, L, N, H * D)
    torch.cuda.synchronize()
    got = part.cpu().double().sum(0)
    assert torch.isfinite(part.cpu()).all(), "every share written"
    # fp32 sums of up to 1024 products in another association: 5e-5 of the largest output; at
    # L <= 8 ns2_linear_bf16 runs its fp32 GEMV, which does not round its input to fp16
    assert_close(got, t.cpu().double(), 5e-5 if L > 8 else TOL, f"attention + o_proj vs two launches (L={L}, D={D})")
    ref = O.attention_rows(q.double(), k.double(), v.double(), H, D, group=group, causal=causal) @ w.double().t()
    assert_close(got, ref, TOL, f"attention + o_proj vs the oracle (L={L}, D={D})")


@pytest.mark.parametrize("M,splits,with_out,bias,N", [
    (256, 4, True, False, 640), (37, 3, False, True, 640), (1, 1, True, True, 640),
    (64, 20, True, False, 640),   # more shares than the 16 whose loads go out together
    (40, 5, True, True, 512),     # two columns per thread
    (40, 16, True, False, 1024),  # four columns per thread
])
def test_parts_add_rmsnorm(ns2lib, M, splits, with_out, bias, N):
    """ns2_parts_add_rmsnorm: the sublayer norms (app/models/gemma3.js:74-79) on a product given as
    fp32 shares, against ns2_add_rmsnorm of their sum taken in split order (bit-exact) and against
    the oracle."""
    g = gen(M * 13 + splits)
    part = torch.randn(splits, M, N, generator=g)
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    x = torch.randn(M, N, generator=g) * 20
    wa = torch.randn(N, generator=g) * 0.3 + 1
    wo = torch.randn(N, generator=g) * 0.3 + 1
    xd = x.to(dev)
    y = torch.empty(M, N, device=dev) if with_out else None
    ns2lib.parts_add_rmsnorm(part.to(dev), splits, b.to(dev) if bias else None, xd, wa.to(dev),
                             wo.to(dev) if with_out else None, y, M, N)
    t = part[0].clone()
    for z in range(1, splits):
        t += part[z]
    if bias:
        t += b
    x2 = x.to(dev)
    y2 = torch.empty(M, N, device=dev) if with_out else None
    ns2lib.add_rmsnorm(x2, t.to(dev), wa.to(dev), wo.to(dev) if with_out else None, y2, M, N)
    torch.cuda.synchronize()
    assert torch.equal(xd.cpu(), x2.cpu()), "parts_add_rmsnorm x vs ns2_add_rmsnorm of the sum"
    if with_out:
        assert torch.equal(y.cpu(), y2.cpu()), "parts_add_rmsnorm y vs ns2_add_rmsnorm of the sum"
    tr = part.double().sum(0) + (b.double() if bias else 0)
    xr = x.double() + O.rms_norm(tr, wa.double())
    assert_close(xd.cpu(), xr, TOL_F32, "parts_add_rmsnorm x")


def test_f16kv_errors(ns2lib):
    import ns2

    buf = torch.zeros(4096, device=dev)
    with pytest.raises(ns2.NS2Error, match="16-byte aligned"):
        ns2lib.attention_rows_f16kv(buf, buf, buf, buf, Lq=2, Lk=2, H=1, D=64, ldq=64, ldk=64, ldv=64, ldo=64,
                                    kOff=4)
    with pytest.raises(ns2.NS2Error, match="multiple of 16"):
        ns2lib.attention_rows_f16kv(buf, buf, buf, buf, Lq=2, Lk=2, H=1, D=40, ldq=40, ldk=40, ldv=40, ldo=40)
    out = torch.zeros(4096, device=dev)
    with pytest.raises(ns2.NS2Error, match="ldkv"):
        ns2lib.linear_bf16_head_norm_f16kv(buf, 64, buf, None, out, 2, 768, 64, buf, 1, buf, 1, 256, out, 256)


@pytest.mark.parametrize("Lq,Lk,causal", [(100, 37, True), (5, 300, False), (300, 300, True)])
def test_attention_rows_ragged_tiles(ns2lib, Lq, Lk, causal):
    """Query and key counts that are not multiples of the 16-row tiles, Lq != Lk under the causal
    mask, more keys than queries, and a full causal square of 300."""
    H, D, group = 8, 128, 2
    g = gen(Lq * 3 + Lk)
    q = torch.randn(Lq, H * D, generator=g)
    k = torch.randn(Lk, H // group * D, generator=g)
    v = torch.randn(Lk, H // group * D, generator=g)
    o = torch.empty(Lq, H * D, device=dev)
    ns2lib.attention_rows(q.to(dev), k.to(dev), v.to(dev), o, Lq=Lq, Lk=Lk, H=H, D=D, ldq=H * D,
                          ldk=H // group * D, ldv=H // group * D, ldo=H * D, group=group, causal=causal)
    torch.cuda.synchronize()
    ref = O.attention_rows(q.double(), k.double(), v.double(), H, D, group=group, causal=causal)
    assert_close(o.cpu(), ref, TOL, f"attention_rows ragged Lq={Lq} Lk={Lk} causal={causal}")
