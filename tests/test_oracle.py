"""Pins the oracle (CPU, no GPU needed): every restated function is checked against a closed
form, an invariant or a brute-force computation chosen so that a plausible slip (a wrong sign
in H4, a transposed operand, a dropped term, the wrong RoPE axis) fails. The DiT composition
is pinned by golden vectors written from the reference itself (test_golden.py)."""

import itertools
import math

import numpy as np
import pytest
import torch

import oracle.nanosaur2_oracle as O

f64 = torch.float64


# ----------------------------------------------------------------------------- Hadamard

def test_hadamard_closed_form():
    """H[i][j] = (-1)^{#base-4 digit positions with i_d + j_d = 3} / 16: the sign pattern of
    kron(H4, H4, H4, H4) with H4[a][b] = -1 exactly when a + b = 3."""
    H = O.hadamard(256, f64)
    i = np.arange(256)
    digits = lambda v: [(v >> (2 * d)) & 3 for d in range(4)]  # noqa: E731
    di, dj = digits(i[:, None]), digits(i[None, :])
    neg = sum(((a + b) == 3).astype(int) for a, b in zip(di, dj))
    want = torch.from_numpy(np.where(neg % 2 == 1, -1.0, 1.0) / 16.0)
    assert torch.equal(H, want)


def test_hadamard_invariants():
    H = O.hadamard(256, f64)
    assert torch.equal(H, H.T)
    assert torch.allclose(H @ H, torch.eye(256, dtype=f64), atol=1e-14)
    x = torch.randn(10, 256, dtype=f64)
    assert torch.allclose((x @ H).norm(dim=1), x.norm(dim=1))
    with pytest.raises(ValueError):
        O.hadamard(128)


def test_fwht_equals_dense_and_reference_stage_order():
    """The shader's 4 radix-4 stages (kernels.js:390-406) equal the dense x @ H."""
    x = torch.randn(7, 1024, dtype=f64)
    assert torch.allclose(O.fwht(x), O.rotate(x), atol=1e-13)
    # brute force on one group: y_j = sum_i x_i H[i][j]
    H = O.hadamard(256, f64)
    y = [sum(x[0, i].item() * H[i, j].item() for i in range(256)) for j in range(3)]
    assert np.allclose(O.rotate(x)[0, :3].numpy(), y)


def test_rotate_is_involution():
    x = torch.randn(3, 768, dtype=f64)
    assert torch.allclose(O.rotate(O.rotate(x)), x, atol=1e-13)  # tools/quant.py:64


# ----------------------------------------------------------------------------- int8 ConvRot

def test_quantize_bounds_and_roundtrip():
    g = torch.Generator().manual_seed(0)
    W = torch.randn(64, 512, generator=g)
    q, s = O.quantize_int8_convrot(W)
    assert q.dtype == torch.int8 and s.shape == (64, 1)
    assert (q.abs().amax(dim=1) == 127).all()          # amax maps to +-127
    rot = O.rotate(W.double())
    err = (rot - q.double() * s.double()).abs()
    assert (err <= s.double() / 2 * (1 + 1e-6)).all()   # round-to-nearest in the rotated domain
    Wd = O.dequantize(q, s, f64)
    # H orthogonal: the row error norm is preserved by the inverse rotation
    assert torch.allclose((W.double() - Wd).norm(dim=1), err.norm(dim=1), rtol=1e-6)


def test_linear_i8_identity_and_bruteforce():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 256, generator=g, dtype=f64)
    q = torch.randint(-127, 128, (3, 256), generator=g, dtype=torch.int32).to(torch.int8)
    s = torch.rand(3, 1, generator=g, dtype=f64)
    y = O.linear_i8(x, q, s)
    assert torch.allclose(y, x @ O.dequantize(q, s, f64).T, atol=1e-12)
    H = O.hadamard(256, f64)
    for m, n in itertools.product(range(5), range(3)):
        xr = [sum(x[m, i].item() * H[i, j].item() for i in range(256)) for j in range(256)]
        want = s[n, 0].item() * sum(xr[k] * q[n, k].item() for k in range(256))
        assert abs(y[m, n].item() - want) < 1e-9


def test_linear_epilogue_order():
    """gemm.js:159-164: *RS, +BIAS, +ADD, silu, then store / += / += gate."""
    acc = torch.tensor([[1.0, -2.0]], dtype=f64)
    rs, bias, add = torch.tensor([2.0, 3.0], dtype=f64), torch.tensor([0.5, 1.0], dtype=f64), torch.tensor([[0.25, -1.0]], dtype=f64)
    silu = lambda v: v / (1 + math.exp(-v))  # noqa: E731
    r = [silu(1.0 * 2 + 0.5 + 0.25), silu(-2.0 * 3 + 1.0 - 1.0)]
    got = O.linear_epilogue(acc, N=2, row_scale=rs, bias=bias, add=add, act="silu")
    assert np.allclose(got.numpy(), [r])
    out = torch.tensor([10.0, 20.0, 30.0, 40.0], dtype=f64)
    gate = torch.tensor([0, 0, 7.0, -1.0], dtype=f64)
    O.linear_epilogue(acc, N=2, out=out, resid=True, gate=gate, gOff=2, ldc=2, cOff=2)
    assert np.allclose(out.numpy(), [10, 20, 30 + 7 * 1.0, 40 - 1 * -2.0])


def test_bf16_bits():
    w = torch.tensor([1.5, -0.02, 3.0e-5], dtype=torch.bfloat16)
    assert torch.equal(O.bf16_to_float(w.view(torch.int16)), w.float())


# ----------------------------------------------------------------------------- attention

def _qkv(Lq, Lk, H, hd, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(Lq, H * hd, generator=g, dtype=f64), torch.randn(Lk, H * hd, generator=g, dtype=f64),
            torch.randn(Lk, H * hd, generator=g, dtype=f64))


def test_attention_matches_bruteforce_with_bias():
    q, k, v = _qkv(9, 13, 2, 8, 2)
    bias = torch.randn(13, dtype=f64)
    assert torch.allclose(O.attention_heads(q, k, v, 2, 8, bias), O.attention_bruteforce(q, k, v, 2, 8, bias), atol=1e-12)
    # element-level brute force for one (query, head)
    qi, h = 4, 1
    sl = slice(h * 8, (h + 1) * 8)
    s = [(q[qi, sl] @ k[j, sl]).item() / math.sqrt(8) + bias[j].item() for j in range(13)]
    m = max(s)
    p = [math.exp(x - m) for x in s]
    o = sum(p[j] * v[j, sl] for j in range(13)) / sum(p)
    assert torch.allclose(O.attention_heads(q, k, v, 2, 8, bias)[qi, sl], o, atol=1e-12)


def test_attention_invariants():
    q, k, v = _qkv(6, 10, 2, 8, 3)
    base = O.attention_heads(q, k, v, 2, 8)
    assert torch.allclose(O.attention_heads(q, k, v, 2, 8, torch.full((10,), 3.7, dtype=f64)), base, atol=1e-12)
    perm = torch.randperm(10)
    assert torch.allclose(O.attention_heads(q, k[perm], v[perm], 2, 8), base, atol=1e-12)
    mask = torch.zeros(10, dtype=f64)
    mask[7] = float("-inf")
    keep = [j for j in range(10) if j != 7]
    assert torch.allclose(O.attention_heads(q, k, v, 2, 8, mask), O.attention_heads(q, k[keep], v[keep], 2, 8), atol=1e-12)


# ----------------------------------------------------------------------------- RoPE

def test_rope_table_layout_and_axes():
    h, w = 5, 7
    cs, sin_off = O.rope2d_table(h, w)
    assert sin_off == h * w * 48 and cs.numel() == 2 * sin_off
    cos, sin = cs[:sin_off].reshape(h * w, 48).double(), cs[sin_off:].reshape(h * w, 48).double()
    assert torch.allclose(cos ** 2 + sin ** 2, torch.ones_like(cos), atol=1e-6)
    centre = (h // 2) * w + (w // 2)       # odd grid: cx = cy = 0
    assert torch.allclose(cos[centre], torch.ones(48, dtype=f64)) and torch.allclose(sin[centre], torch.zeros(48, dtype=f64))
    # pairs 0..23 follow the column (x), 24..47 the row (y); frequency 1 at pair 0
    tok = lambda y, x: y * w + x  # noqa: E731
    a = torch.atan2(sin, cos)
    assert torch.allclose(a[tok(2, 5), 0], torch.tensor(2.0, dtype=f64), atol=1e-6)       # cx = 5 - 3
    assert torch.allclose(a[tok(4, 3), 24], torch.tensor(2.0, dtype=f64), atol=1e-6)      # cy = 4 - 2
    assert torch.allclose(a[tok(4, 3), :24], torch.zeros(24, dtype=f64), atol=1e-6)       # cx = 0
    f1 = 1.0 / 10000 ** (2.0 / 48)                                                         # pair 1 frequency
    assert abs(a[tok(2, 6), 1].item() - 3 * f1) < 1e-6


def test_rope_table_matches_pytorch_form():
    h, w = 6, 9
    cs, sin_off = O.rope2d_table(h, w)
    cos, sin = O.rope_2d(h, w, dtype=f64)
    assert torch.allclose(cs[:sin_off].reshape(h * w, 48).double(), cos, atol=2e-6)
    assert torch.allclose(cs[sin_off:].reshape(h * w, 48).double(), sin, atol=2e-6)


def test_rope_preserves_pair_norms():
    cos, sin = O.rope_2d(4, 4, dtype=f64)
    x = torch.randn(16, 96, dtype=f64)
    y = O.rope_split_half(x, cos, sin)
    n = lambda t: t[:, :48] ** 2 + t[:, 48:] ** 2  # noqa: E731
    assert torch.allclose(n(y), n(x), atol=1e-12)


def test_head_norm_rope_buffer_semantics():
    """headNorm on a strided buffer touches only its window and equals the per-row formula."""
    L, H, Dh, ld = 3, 2, 8, 40
    X = torch.randn(L + 2, ld, dtype=f64)
    w = torch.randn(Dh, dtype=f64)
    cs = torch.cat([torch.cos(torch.arange(L * 4, dtype=f64)), torch.sin(torch.arange(L * 4, dtype=f64))])
    Y = O.head_norm_rope(X.clone(), w, L, H, Dh, ld, colOff=16, rowOff=1, cs=cs, sinOff=L * 4)
    mask = torch.zeros_like(X, dtype=torch.bool)
    mask[1:1 + L, 16:16 + H * Dh] = True
    assert torch.equal(Y[~mask], X[~mask])
    row, h = 2, 1
    x = X[1 + row, 16 + h * Dh: 16 + (h + 1) * Dh]
    n = x / torch.sqrt((x ** 2).mean() + 1e-6) * w
    c, s = cs[row * 4:(row + 1) * 4], cs[L * 4 + row * 4: L * 4 + (row + 1) * 4]
    want = torch.cat([n[:4] * c - n[4:] * s, n[4:] * c + n[:4] * s])
    assert torch.allclose(Y[1 + row, 16 + h * Dh: 16 + (h + 1) * Dh], want, atol=1e-12)


# ----------------------------------------------------------------------------- norms and small ops

def test_norms():
    x = torch.randn(4, 64, dtype=f64) * 5 + 2
    w = torch.randn(64, dtype=f64)
    assert torch.allclose(O.rms_norm(3.0 * x, w), O.rms_norm(x, w), atol=1e-9)
    ln = O.layer_norm(x)
    assert torch.allclose(ln.mean(-1), torch.zeros(4, dtype=f64), atol=1e-12)
    assert torch.allclose(ln.var(-1, unbiased=False), torch.ones(4, dtype=f64), atol=1e-5)
    mod = torch.randn(6 * 64, dtype=f64)
    got = O.norm_mod(x, mod, 3 * 64, 4 * 64, w)
    want = O.rms_norm(x, w) * (1 + mod[256:320]) + mod[192:256]
    assert torch.allclose(got, want)


def test_timestep_embedding_and_glu_rowsum():
    e = O.timestep_embedding(0.0, dtype=f64)
    assert torch.equal(e, torch.cat([torch.ones(128, dtype=f64), torch.zeros(128, dtype=f64)])[None])
    e = O.timestep_embedding(1000.0, dtype=f64)
    assert abs(e[0, 1].item() - math.cos(1000.0 * math.exp(-math.log(10000) / 128))) < 1e-12
    x = torch.tensor([[0.0, 2.0, 3.0, 5.0]], dtype=f64)
    assert torch.allclose(O.glu(x), torch.tensor([[0.0, 2.0 / (1 + math.exp(-2.0)) * 5.0]], dtype=f64))
    xs = torch.tensor([[1.0, 2.0], [3.0, 4.0]], dtype=f64)
    assert torch.allclose(O.row_sum(xs, torch.tensor([2.0, -1.0], dtype=f64), 0.5), torch.tensor([[-0.5, 0.0]], dtype=f64))


# ----------------------------------------------------------------------------- Gemma3 pieces

@pytest.mark.parametrize("group,causal", [(1, False), (1, True), (4, True), (2, False)])
def test_attention_rows_matches_bruteforce(group, causal):
    g = torch.Generator().manual_seed(group * 10 + causal)
    H, hd, L = 4, 16, 9
    q = torch.randn(L, H * hd, generator=g, dtype=torch.float64)
    k = torch.randn(L, H // group * hd, generator=g, dtype=torch.float64)
    v = torch.randn(L, H // group * hd, generator=g, dtype=torch.float64)
    got = O.attention_rows(q, k, v, H, hd, group=group, causal=causal)
    ref = O.attention_rows_bruteforce(q, k, v, H, hd, group=group, causal=causal)
    assert torch.allclose(got, ref, atol=1e-12)


def test_attention_rows_causal_invariants():
    g = torch.Generator().manual_seed(5)
    H, hd, L = 2, 8, 7
    q = torch.randn(L, H * hd, generator=g, dtype=torch.float64)
    k = torch.randn(L, H * hd, generator=g, dtype=torch.float64)
    v = torch.randn(L, H * hd, generator=g, dtype=torch.float64)
    o = O.attention_rows(q, k, v, H, hd, causal=True)
    # the first query sees only the first key: its output is v_0
    assert torch.allclose(o[0], v[0], atol=1e-12)
    # changing future keys leaves earlier outputs unchanged
    k2, v2 = k.clone(), v.clone()
    k2[4:] += 3.0
    v2[4:] -= 1.0
    o2 = O.attention_rows(q, k2, v2, H, hd, causal=True)
    assert torch.allclose(o[:4], o2[:4], atol=1e-12) and not torch.allclose(o[4:], o2[4:])
    # one K/V head repeated equals grouped attention with group = H
    kk = k[:, :hd].repeat(1, H)
    vv = v[:, :hd].repeat(1, H)
    assert torch.allclose(O.attention_rows(q, k[:, :hd], v[:, :hd], H, hd, group=H, causal=True),
                          O.attention_rows(q, kk, vv, H, hd, causal=True), atol=1e-12)


def test_gemma_rope_closed_form():
    cos, sin = O.gemma_rope(5, 1e4, D=8, dtype=torch.float64)
    for l in range(5):
        for i in range(4):
            a = l / 1e4 ** (2 * i / 8)
            assert abs(cos[l, i] - math.cos(a)) < 1e-12 and abs(sin[l, i] - math.sin(a)) < 1e-12
    # position 0 is the identity
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
