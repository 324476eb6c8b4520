"""CPU oracle for the Nanosaur2 DiT hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, on PyTorch CPU, of the reference's fp32 algorithm for one DiT pass: the
ConvRot int8 format and rotation (tools/quant.py), the PyTorch reference model
(tools/reference.py) and the semantics of the WGSL kernels the ops layer dispatches
(app/gpu/kernels.js, app/gpu/gemm.js, app/models/common.js). Only tests/, the smoke check
and bench.py's CPU baseline may use it, and only as the checker or the baseline; the
product path (the HIP library and its hosts) never calls it.

Every function cites the reference lines it follows. All functions take and return torch
CPU tensors; pass dtype=torch.float64 inputs where a tighter reference is wanted.

Parity status: every function here is pinned by tests/test_oracle.py (closed forms,
invariants, brute force) and, for the DiT composition, by golden vectors written from the
reference itself (tests/golden/).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

D, HEADS, HD = 1536, 16, 96          # tools/reference.py:205; app/models/nanosaur2.js:16-18
BLOCKS, SPRINT_F, SPRINT_H = 18, 2, 2  # app/models/nanosaur2.js:19-21
CH = 64                               # app/models/nanosaur2.js:22
GROUP = 256                           # tools/quant.py:18
H4 = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))  # tools/quant.py:25


# --------------------------------------------------------------------------- ConvRot format

def hadamard(size: int = GROUP, dtype=torch.float32) -> torch.Tensor:
    """Normalized regular symmetric Hadamard matrix kron(H4, ..., H4) / sqrt(size)
    (tools/quant.py:21-29)."""
    if size < 4 or round(math.log(size, 4)) != math.log(size, 4):
        raise ValueError(f"size must be a power of 4, got {size}")
    h4 = torch.tensor(H4, dtype=dtype)
    h = h4
    while h.shape[0] < size:
        h = torch.kron(h, h4)
    return h / math.sqrt(size)


def rotate(x: torch.Tensor, group: int = GROUP) -> torch.Tensor:
    """x H per contiguous group of `group` features along the last axis
    (tools/quant.py:32-36 with H symmetric; app/gpu/kernels.js:378-407 for activations)."""
    k = x.shape[-1]
    h = hadamard(group, x.dtype)
    return (x.reshape(*x.shape[:-1], k // group, group) @ h.T).reshape(x.shape)


def fwht(x: torch.Tensor) -> torch.Tensor:
    """The same rotation computed as the reference shader does it: four radix-4 stages at
    strides 1, 4, 16, 64 with the regular H4, then x 1/16 (app/gpu/kernels.js:390-406,
    app/lora.js:74-91)."""
    y = x.reshape(-1, GROUP).clone()
    stride = 1
    while stride < GROUP:
        v = y.reshape(-1, GROUP // (4 * stride), 4, stride)
        a, b, c, e = v[:, :, 0], v[:, :, 1], v[:, :, 2], v[:, :, 3]
        y = torch.stack([a + b + c - e, a + b - c + e, a - b + c + e, -a + b + c + e], dim=2).reshape(-1, GROUP)
        stride *= 4
    return (y * 0.0625).reshape(x.shape)


def quantize_int8_convrot(weight: torch.Tensor):
    """(q int8 [N,K], scale fp32 [N,1]) of the rotated weight (tools/quant.py:48-56)."""
    rot = rotate(weight.float())
    scale = (rot.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=1e-30)
    q = (rot / scale).round().clamp(-128, 127).to(torch.int8)
    return q, scale.float()


def dequantize(q: torch.Tensor, scale: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """W = rotate(q * s) (tools/quant.py:59-64): H symmetric and orthogonal."""
    return rotate(q.to(dtype) * scale.reshape(-1, 1).to(dtype))


# --------------------------------------------------------------------------- GEMM semantics

def linear_epilogue(acc, *, N, alpha=1.0, row_scale=None, bias=None, add=None, act="none",
                    out=None, resid=False, gate=None, gOff=0, ldc=None, cOff=0):
    """The matmul epilogue of app/gpu/gemm.js:159-164 on acc [M, N]:
    r = acc*alpha (*RS[n]) (+BIAS[n]) (+ADD[m,n]) (silu); store, C += r or C += G[gOff+n] r.
    `out` is the flat output buffer (needed for resid and for column windows)."""
    r = acc * alpha
    if row_scale is not None:
        r = r * row_scale.reshape(1, -1)
    if bias is not None:
        r = r + bias.reshape(1, -1)
    if add is not None:
        r = r + add.reshape(r.shape)
    if act == "silu":
        r = F.silu(r)
    elif act == "gelu_tanh":
        r = F.gelu(r, approximate="tanh")
    M = r.shape[0]
    if out is None:
        return r
    ldc = N if ldc is None else ldc
    idx = cOff + torch.arange(M).reshape(-1, 1) * ldc + torch.arange(N).reshape(1, -1)
    flat = out.reshape(-1)
    if not resid:
        flat[idx] = r.to(flat.dtype)
    elif gate is None:
        flat[idx] = flat[idx] + r.to(flat.dtype)
    else:
        flat[idx] = flat[idx] + gate.reshape(-1)[gOff:gOff + N].reshape(1, -1).to(flat.dtype) * r.to(flat.dtype)
    return out


def linear_i8(x, q, scale, **epi):
    """ops.linear on an int8 ConvRot weight (app/gpu/ops.js:50-66): the input is rotated
    (ops.rotate, :38-44) and multiplied by the integer weight; the per-row scale is applied
    in the epilogue (app/gpu/gemm.js:119-134, 160). Equal to x @ dequantize(q, s).T."""
    acc = rotate(x) @ q.to(x.dtype).T
    return linear_epilogue(acc, N=q.shape[0], row_scale=scale.reshape(-1).to(x.dtype), **epi)


def lora_delta(x, entries, N):
    """app/gpu/ops.js:70-87 (loraDelta): D [M, N] = sum_i scale_i * (x A_i^T) B_i^T in output
    columns [off_i, off_i + n_i); entries are (A [r, K], B [n, r], scale, off, n) over the
    linear's un-rotated input x (for int8 weights the app feeds the rotated input and rotated A,
    app/lora.js:61-78, which gives the same product since H is orthogonal)."""
    D = torch.zeros(x.shape[0], N, dtype=x.dtype)
    for A, B, scale, off, n in entries:
        D[:, off:off + n] += scale * ((x @ A.to(x.dtype).T) @ B.to(x.dtype).T)
    return D


def pack_lora(entries, N, K, rotate_a=False):
    """The stacked side path the *_lora entry points take: lora_a [R, K] (rotated per 256-group
    for int8 weights) and lora_b [N, R] with each entry's scale folded in and zeros outside its
    column window; R = the summed ranks rounded up to a multiple of 32. fp64 tensors; the
    callers round them to fp16."""
    rs = sum(A.shape[0] for A, *_ in entries)
    R = (rs + 31) // 32 * 32
    la = torch.zeros(R, K, dtype=torch.float64)
    lb = torch.zeros(N, R, dtype=torch.float64)
    r0 = 0
    for A, B, scale, off, n in entries:
        r = A.shape[0]
        la[r0:r0 + r] = rotate(A.double()) if rotate_a else A.double()
        lb[off:off + n, r0:r0 + r] = scale * B.double()
        r0 += r
    return la, lb, R


def bf16_to_float(w_bits: torch.Tensor) -> torch.Tensor:
    """bf16 bit patterns (int16 storage) -> fp32: the pattern is the high half of the fp32
    word (app/gpu/gemm.js:99-100)."""
    return (w_bits.to(torch.int32) & 0xFFFF).bitwise_left_shift(16).view(torch.float32)


def linear_bf16(x, w, **epi):
    """ops.linear on a bf16 weight (app/gpu/gemm.js:98-118); w is torch.bfloat16 [N, K]."""
    wf = w.float().to(x.dtype)
    return linear_epilogue(x @ wf.T, N=wf.shape[0], **epi)


# --------------------------------------------------------------------------- norms, RoPE, GLU

def rms_norm(x, w, eps=1e-6):
    """tools/reference.py:96-97; app/gpu/kernels.js:60-80."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def layer_norm(x, eps=1e-6):
    """LayerNorm without affine (tools/reference.py:328; app/gpu/kernels.js:104-113)."""
    return F.layer_norm(x, (x.shape[-1],), eps=eps)


def modulate(x, shift, scale):
    """tools/reference.py:244-245."""
    return x * (1 + scale) + shift


def norm_mod(x, mod, shiftOff, scaleOff, weight=None, eps=1e-6):
    """ops.normMod (app/gpu/ops.js:119-129; kernels.js:82-117): RMSNorm*w or LayerNorm, then
    (1 + mod[scaleOff:]) and + mod[shiftOff:]."""
    cols = x.shape[-1]
    mod = mod.reshape(-1)
    n = rms_norm(x, weight, eps) if weight is not None else layer_norm(x, eps)
    return modulate(n, mod[shiftOff:shiftOff + cols], mod[scaleOff:scaleOff + cols])


def rope_split_half(x, cos, sin):
    """tools/reference.py:100-104: pair i is (x[i], x[i + D/2])."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def rope_2d(h, w, hd=HD, dtype=torch.float32):
    """cos, sin [h*w, hd/2] of the centred 2-D RoPE (tools/reference.py:220-227): the first
    hd/4 pairs rotate by the column coordinate, the next hd/4 by the row coordinate."""
    axis = hd // 2
    inv = 1.0 / (10000.0 ** (torch.arange(0, axis, 2, dtype=dtype) / axis))
    y = torch.arange(h, dtype=dtype) - (h - 1) / 2
    x = torch.arange(w, dtype=dtype) - (w - 1) / 2
    y, x = torch.meshgrid(y, x, indexing="ij")
    a = torch.cat([torch.outer(x.flatten(), inv), torch.outer(y.flatten(), inv)], dim=-1)
    return a.cos(), a.sin()


def rope2d_table(h, w, hd=HD):
    """The flat table the ops layer uploads: cos block then sin block, each [h*w][hd/2], with
    sinOff = h*w*hd/2 (app/models/common.js:4-13, 15, 28-43; frequencies rounded to fp32
    like Math.fround, angles stored as fp32)."""
    half = hd // 2
    f = [_fround(1.0 / math.pow(10000.0, _fround(2.0 * i / half))) for i in range(half // 2)]
    f = torch.tensor(f, dtype=torch.float64)
    ys = torch.arange(h, dtype=torch.float64) - (h - 1) / 2
    xs = torch.arange(w, dtype=torch.float64) - (w - 1) / 2
    yy, xx = torch.meshgrid(ys, xs, indexing="ij")
    a = torch.cat([torch.outer(xx.flatten(), f), torch.outer(yy.flatten(), f)], dim=-1)
    a = a.to(torch.float32).to(torch.float64)  # Float32Array of angles
    cs = torch.cat([a.cos().reshape(-1), a.sin().reshape(-1)]).to(torch.float32)
    return cs, h * w * half


def _fround(v: float) -> float:
    return float(torch.tensor(v, dtype=torch.float32))


def head_norm_rope(X, w, L, H, Dh, ld, colOff=0, rowOff=0, cs=None, sinOff=0, eps=1e-6):
    """ops.headNorm in place on the flat buffer X (app/gpu/ops.js:131-138;
    app/gpu/kernels.js:307-342): per (row, head) RMSNorm * w, then split-half RoPE with
    table rows l (cos at cs[l*D/2 + i], sin at cs[sinOff + l*D/2 + i])."""
    flat = X.reshape(-1)
    rows = (rowOff + torch.arange(L)).reshape(-1, 1, 1) * ld
    idx = rows + colOff + torch.arange(H).reshape(1, -1, 1) * Dh + torch.arange(Dh).reshape(1, 1, -1)
    v = flat[idx]
    v = rms_norm(v, w.reshape(1, 1, -1), eps)
    if cs is not None:
        half = Dh // 2
        cos = cs.reshape(-1)[torch.arange(L).reshape(-1, 1) * half + torch.arange(half)].reshape(L, 1, half)
        sin = cs.reshape(-1)[sinOff + torch.arange(L).reshape(-1, 1) * half + torch.arange(half)].reshape(L, 1, half)
        v = rope_split_half(v, cos.to(v.dtype), sin.to(v.dtype))
    flat[idx] = v
    return X


def glu(x, act="silu"):
    """ops.glu (app/gpu/ops.js:140-148; kernels.js:344-360): act(x[:, :I]) * x[:, I:]."""
    I = x.shape[-1] // 2
    a = F.silu(x[..., :I]) if act == "silu" else F.gelu(x[..., :I], approximate="tanh")
    return a * x[..., I:]


def row_sum(x, w, scale=1.0):
    """ops.rowSum (app/gpu/ops.js:150-156; kernels.js:362-376)."""
    return (w.reshape(-1, 1) * x).sum(0, keepdim=True) * scale


def timestep_embedding(t, dim=256, dtype=torch.float32):
    """Sinusoidal embedding, cos half then sin half (tools/reference.py:213-217;
    app/models/nanosaur2.js:25-36)."""
    half = dim // 2
    freqs = torch.exp(-math.log(10000) * torch.arange(half, dtype=dtype) / half)
    a = torch.as_tensor(t, dtype=dtype) * freqs
    return torch.cat([a.cos(), a.sin()])[None]


# --------------------------------------------------------------------------- attention

def attention_heads(q, k, v, heads, hd, bias=None):
    """Joint attention on [L, heads*hd] operands (tools/reference.py:230-237):
    softmax(q k^T / sqrt(hd) + bias[key]) v per head, non-causal; bias [Lk] additive."""
    Lq, Lk = q.shape[0], k.shape[0]
    qh = q.reshape(Lq, heads, hd).transpose(0, 1)
    kh = k.reshape(Lk, heads, hd).transpose(0, 1)
    vh = v.reshape(Lk, heads, hd).transpose(0, 1)
    mask = None if bias is None else bias.to(q.dtype)[None, None, :].expand(1, Lq, -1)
    o = F.scaled_dot_product_attention(qh[None], kh[None], vh[None], attn_mask=mask)[0]
    return o.transpose(0, 1).reshape(Lq, heads * hd)


def attention_bruteforce(q, k, v, heads, hd, bias=None):
    """Textbook softmax attention written out with explicit max/exp/sum (no library
    attention routine); used to pin attention_heads."""
    Lq, Lk = q.shape[0], k.shape[0]
    out = torch.empty(Lq, heads * hd, dtype=q.dtype)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = (q[:, sl] @ k[:, sl].T) / math.sqrt(hd)
        if bias is not None:
            s = s + bias.reshape(1, -1).to(s.dtype)
        s = s - s.max(dim=1, keepdim=True).values
        p = torch.exp(s)
        out[:, sl] = (p @ v[:, sl]) / p.sum(dim=1, keepdim=True)
    return out


def joint_attention_op(q, k, v, L, cos, sin, key_bias=None, bias_start=None, heads=HEADS, hd=HD):
    """The benchmarked joint attention op: split-half 2-D RoPE on the first L (image) rows of
    q and k, additive key bias on keys >= bias_start, then attention_heads."""
    def rope_rows(x, n):
        y = x.clone()
        th = x[:n].reshape(n, heads, hd).transpose(0, 1)
        y[:n] = rope_split_half(th, cos[:n].to(x.dtype), sin[:n].to(x.dtype)).transpose(0, 1).reshape(n, heads * hd)
        return y
    qr = rope_rows(q, min(L, q.shape[0]))
    kr = rope_rows(k, min(L, k.shape[0]))
    bias = None
    if key_bias is not None:
        bias = torch.zeros(k.shape[0], dtype=q.dtype)
        bias[bias_start:] = key_bias.to(q.dtype)
    return attention_heads(qr, kr, v, heads, hd, bias)


def attention_rows(q, k, v, heads, hd, group=1, causal=False):
    """The materialized attention path of ops.attention (app/gpu/ops.js:211-241 with
    softmaxShader): per head h with K/V head h // group, softmax(q k^T / sqrt(hd)) v over the
    keys, masked to key <= query when causal. q [Lq, heads*hd], k/v [Lk, (heads//group)*hd]."""
    Lq, Lk = q.shape[0], k.shape[0]
    kvh = heads // group
    qh = q.reshape(Lq, heads, hd).transpose(0, 1)
    kh = k.reshape(Lk, kvh, hd).transpose(0, 1).repeat_interleave(group, 0)
    vh = v.reshape(Lk, kvh, hd).transpose(0, 1).repeat_interleave(group, 0)
    mask = None
    if causal:
        mask = torch.full((Lq, Lk), float("-inf"), dtype=q.dtype).triu(1)[None]
    o = F.scaled_dot_product_attention(qh[None], kh[None], vh[None], attn_mask=mask)[0]
    return o.transpose(0, 1).reshape(Lq, heads * hd)


def attention_rows_bruteforce(q, k, v, heads, hd, group=1, causal=False):
    """attention_rows written out query by query with explicit max/exp/sum; pins it."""
    Lq = q.shape[0]
    out = torch.empty(Lq, heads * hd, dtype=q.dtype)
    for h in range(heads):
        g = h // group
        for i in range(Lq):
            n = i + 1 if causal else k.shape[0]
            qi = q[i, h * hd:(h + 1) * hd]
            kk = k[:n, g * hd:(g + 1) * hd]
            vv = v[:n, g * hd:(g + 1) * hd]
            s = (kk @ qi) / math.sqrt(hd)
            p = torch.exp(s - s.max())
            out[i, h * hd:(h + 1) * hd] = (p @ vv) / p.sum()
    return out


# --------------------------------------------------------------------------- Gemma3 text encoder

GEMMA = {"hidden": 640, "heads": 4, "kv_heads": 1, "head_dim": 256, "layers": 17, "global_every": 6}


def gemma_rope(L, theta, D=256, dtype=torch.float32):
    """tools/reference.py:170-173: angles l / theta^(2i/D), i < D/2 (cos, sin)."""
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).to(dtype) / D))
    a = torch.arange(L).to(dtype)[:, None] * inv[None]
    return a.cos(), a.sin()


def gemma_encode(W, ids, dtype=torch.float32):
    """Hidden state after the 17th of 18 layers with the final norm applied
    (tools/reference.py:176-200; app/models/gemma3.js:49-95): scaled embeddings, pre/post norms
    around attention and MLP with RMSNorm weights stored as w - 1, q/k norms, split-half RoPE
    (theta 1e6 on every 6th layer, 1e4 otherwise), causal attention with one K/V head for the
    four query heads, GELU(tanh)-gated MLP."""
    G = GEMMA
    H, KH, HD = G["heads"], G["kv_heads"], G["head_dim"]
    x = W("model.embed_tokens.weight")[torch.tensor(ids)].to(dtype) * math.sqrt(G["hidden"])
    L = x.shape[0]
    ropes = {t: gemma_rope(L, t, HD, dtype) for t in (1e4, 1e6)}
    for i in range(G["layers"]):
        p = f"model.layers.{i}."
        n = lambda k: W(p + k + ".weight").to(dtype) + 1.0  # noqa: E731
        cos, sin = ropes[1e6 if (i + 1) % G["global_every"] == 0 else 1e4]
        h = rms_norm(x, n("input_layernorm"))
        q = (h @ W(p + "self_attn.q_proj.weight").to(dtype).T).view(L, H, HD).transpose(0, 1)
        k = (h @ W(p + "self_attn.k_proj.weight").to(dtype).T).view(L, KH, HD).transpose(0, 1)
        v = h @ W(p + "self_attn.v_proj.weight").to(dtype).T
        q = rope_split_half(rms_norm(q, n("self_attn.q_norm")), cos, sin).transpose(0, 1).reshape(L, H * HD)
        k = rope_split_half(rms_norm(k, n("self_attn.k_norm")), cos, sin).transpose(0, 1).reshape(L, KH * HD)
        a = attention_rows(q, k, v, H, HD, group=H // KH, causal=True)
        a = a @ W(p + "self_attn.o_proj.weight").to(dtype).T
        x = x + rms_norm(a, n("post_attention_layernorm"))
        h = rms_norm(x, n("pre_feedforward_layernorm"))
        g = F.gelu(h @ W(p + "mlp.gate_proj.weight").to(dtype).T, approximate="tanh")
        g = g * (h @ W(p + "mlp.up_proj.weight").to(dtype).T)
        x = x + rms_norm(g @ W(p + "mlp.down_proj.weight").to(dtype).T, n("post_feedforward_layernorm"))
    return rms_norm(x, W("model.norm.weight").to(dtype) + 1.0)


# --------------------------------------------------------------------------- DiT pass

def lin(W, name, x):
    """tools/reference.py:208-210 (weights dequantized on access like Weights.__call__, :54-64)."""
    y = x @ W(name + ".weight").T
    return y + W(name + ".bias") if W.has(name + ".bias") else y


def attention(q, k, v, bias=None):
    """tools/reference.py:230-237."""
    return attention_heads(q, k, v, HEADS, HD, bias)


def head_norm(x, w):
    """tools/reference.py:240-241."""
    return rms_norm(x.view(x.shape[0], HEADS, HD), w).view(x.shape[0], D)


class DiT:
    """Restatement of tools/reference.py:248-329 (DiT.text_refine / block / forward)."""

    def __init__(self, W):
        self.W = W

    def text_refine(self, txt, tc, keep_bias, keep):
        """tools/reference.py:252-265."""
        W = self.W
        for i in range(2):
            p = f"text_refine_blocks.{i}."
            m = lin(W, p + "adaLN_modulation.0", tc).chunk(6, -1)
            h = modulate(rms_norm(txt, W(p + "norm1.weight")), m[0], m[1])
            q, k, v = lin(W, p + "attn.qkv", h).chunk(3, -1)
            a = attention(head_norm(q, W(p + "attn.q_norm.weight")), head_norm(k, W(p + "attn.k_norm.weight")), v, keep_bias)
            txt = txt + m[2] * lin(W, p + "attn.proj", a)
            h = modulate(rms_norm(txt, W(p + "norm2.weight")), m[3], m[4])
            x1, x2 = lin(W, p + "mlp.w12", h).chunk(2, -1)
            txt = txt + m[5] * lin(W, p + "mlp.w3", F.silu(x1) * x2)
            txt = txt * keep[:, None]
        return txt

    def block(self, i, x, txt, cos, sin, mod, txt_bias):
        """tools/reference.py:267-289."""
        W = self.W
        p = f"blocks.{i}."
        m = (mod + W(f"encoder_adaLN_offsets.{i}")).chunk(6, -1)
        h = modulate(rms_norm(x, W(p + "norm1.weight")), m[0], m[1])
        q, k, v = lin(W, p + "attn.qkv_x", h).chunk(3, -1)
        L = x.shape[0]

        def rope(t, wn):
            th = rms_norm(t.view(L, HEADS, HD), W(wn)).transpose(0, 1)
            return rope_split_half(th, cos, sin).transpose(0, 1).reshape(L, D)

        q, k = rope(q, p + "attn.q_norm.weight"), rope(k, p + "attn.k_norm.weight")
        bias = None
        if W.has(p + "attn.kv_y.weight"):
            ky, vy = lin(W, p + "attn.kv_y", txt).chunk(2, -1)
            k = torch.cat([k, head_norm(ky, W(p + "attn.k_norm.weight"))])
            v = torch.cat([v, vy])
            bias = torch.cat([torch.zeros(L, dtype=x.dtype), txt_bias])
        x = x + m[2] * lin(W, p + "attn.proj", attention(q, k, v, bias))
        h = modulate(rms_norm(x, W(p + "norm2.weight")), m[3], m[4])
        x1, x2 = lin(W, p + "mlp.w12", h).chunk(2, -1)
        return x + m[5] * lin(W, p + "mlp.w3", F.silu(x1) * x2)

    @torch.no_grad()
    def forward(self, latent, sigma, context, weights, path_drop=False, dump=None):
        """tools/reference.py:291-329: latent [64, h, w] -> x0 [64, h, w]."""
        W = self.W
        dt = latent.dtype
        _, h, w = latent.shape
        keep = (weights > 0).to(dt)
        txt_bias = torch.log(weights.clamp(min=1e-4)).masked_fill(weights <= 0, float("-inf")).to(dt)
        refine_keep = weights > 0
        if not refine_keep.any():
            refine_keep[0] = True
        keep_bias = torch.zeros_like(weights, dtype=dt).masked_fill(~refine_keep, float("-inf"))

        t = lin(W, "t_embedder.mlp.2", F.silu(lin(W, "t_embedder.mlp.0", timestep_embedding(torch.tensor(sigma * 1000.0, dtype=dt), dtype=dt))))
        tc = F.silu(t)
        txt = rms_norm(lin(W, "y_embedder.proj", context), W("y_embedder.norm.weight"))
        txt = self.text_refine(txt, tc, keep_bias, keep)
        pooled = (txt * weights[:, None].to(dt)).sum(0) / weights.to(dt).sum().clamp(min=1.0)
        cond = F.silu(t + lin(W, "y_pool_proj", pooled[None]))
        mod = lin(W, "shared_encoder_adaLN.0", cond)
        if dump is not None:
            dump["txt_refined"] = txt
            dump["cond"] = cond

        cos, sin = rope_2d(h, w, dtype=dt)
        x = lin(W, "s_embedder.proj", latent.flatten(1).T)
        for i in range(SPRINT_F):
            x = self.block(i, x, txt, cos, sin, mod, txt_bias)
        if dump is not None:
            dump["block1"] = x
        if not path_drop:
            g = x
            for i in range(SPRINT_F, BLOCKS - SPRINT_H):
                g = self.block(i, g, txt, cos, sin, mod, txt_bias)
            x = x + lin(W, "sprint_out_proj", g - x)
        for i in range(BLOCKS - SPRINT_H, BLOCKS):
            x = self.block(i, x, txt, cos, sin, mod, txt_bias)
        shift, scale = lin(W, "final_layer.adaLN_modulation", cond).chunk(2, -1)
        x = modulate(layer_norm(x), shift, scale)
        return lin(W, "final_layer.linear", x).T.reshape(CH, h, w)


LORA_SUFFIXES = [(".lora_A.weight", "A"), (".lora_B.weight", "B"), (".lora_down.weight", "A"),
                 (".lora_up.weight", "B"), (".alpha", "alpha")]
LORA_PREFIXES = ["lora_unet_", "model.diffusion_model.", "diffusion_model.", "lora_te_", "text_encoder."]


def lora_deltas(loras, dtype=torch.float32):
    """tools/reference.py:70-95: module name (dots as underscores) -> [(scale, B, A)] with
    scale = strength * alpha / r (alpha absent: strength), from PEFT (lora_A/B) or kohya
    (lora_down/up) keys; `loras` holds (name -> tensor dict, strength) pairs."""
    out = {}
    for tensors, strength in loras:
        groups = {}
        for k in tensors:
            for suf, role in LORA_SUFFIXES:
                if k.endswith(suf):
                    groups.setdefault(k[: -len(suf)], {})[role] = k
        for module, ks in groups.items():
            name = module
            for p in LORA_PREFIXES:
                if name.startswith(p):
                    name = name[len(p):]
                    break
            A = tensors[ks["A"]].float().to(dtype)
            B = tensors[ks["B"]].float().to(dtype)
            scale = strength * (float(tensors[ks["alpha"]].float().item()) / A.shape[0] if "alpha" in ks else 1.0)
            out.setdefault(name.replace(".", "_"), []).append((scale, B, A))
    return out


class TensorWeights:
    """Weights from a name -> tensor dict in the reference's on-disk layout: int8 ConvRot
    linears as `<base>.weight` int8 [N,K] + `<base>.weight_scale` fp32 [N,1] (dequantized on
    access like tools/reference.py:54-64), everything else (bf16 bit patterns as int16, or
    float) converted to `dtype`. LoRAs ((tensor dict, strength) pairs) are merged into the
    weights they name on access, w + scale * B A, as tools/reference.py:62-64 does."""

    def __init__(self, tensors: dict, dtype=torch.float32, loras=()):
        self.t = tensors
        self.dtype = dtype
        self.cache = {}
        self.deltas = lora_deltas(loras, dtype)

    def has(self, name: str) -> bool:
        return name in self.t

    def __call__(self, name: str) -> torch.Tensor:
        if name in self.cache:
            return self.cache[name]
        base = name[: -len("weight")] if name.endswith("weight") else None
        if base is not None and base + "weight_scale" in self.t:
            w = dequantize(self.t[name], self.t[base + "weight_scale"], self.dtype)
        else:
            v = self.t[name]
            w = v.float().to(self.dtype)  # bf16 -> fp32 is exact
        if name.endswith(".weight"):
            for scale, B, A in self.deltas.get(name[: -len(".weight")].replace(".", "_"), []):
                w = w + scale * (B @ A)
        self.cache[name] = w
        return w
