"""Textbook float64 versions of the attention-path operators.

These are written from the mathematics (numpy matmul, complex rotation,
reshape-based windowing), not from the reference kernels, so that they
pin the oracle independently of its operation order.
"""
import math

import numpy as np


def gelu(x):
    erf = np.vectorize(math.erf)
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def layernorm(x, g, b, eps=1e-5):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def softmax(s):
    s = s.astype(np.float64)
    e = np.exp(s - s.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def rope(qkv, E, hd, npos, cs):
    """Rotate pairs (2j, 2j+1) of every head of the q and k thirds as
    complex numbers by cs[row % npos, j] = (cos, sin)."""
    qkv = qkv.astype(np.float64).copy()
    rows = qkv.shape[0]
    rot = cs[np.arange(rows) % npos].astype(np.float64)      # rows, hd/2, 2
    z = rot[..., 0] + 1j * rot[..., 1]
    for third in (0, 1):
        blk = qkv[:, third * E:(third + 1) * E].reshape(rows, E // hd, hd // 2, 2)
        c = (blk[..., 0] + 1j * blk[..., 1]) * z[:, None, :]
        blk = np.stack([c.real, c.imag], -1).reshape(rows, E)
        qkv[:, third * E:(third + 1) * E] = blk
    return qkv


def window_partition(x, H, W, ws):
    """[H*W, C] -> [nwin*ws*ws, C], zero padded, windows row-major."""
    C = x.shape[-1]
    nwy, nwx = -(-H // ws), -(-W // ws)
    g = np.zeros((nwy * ws, nwx * ws, C), x.dtype)
    g[:H, :W] = x.reshape(H, W, C)
    g = g.reshape(nwy, ws, nwx, ws, C).transpose(0, 2, 1, 3, 4)
    return g.reshape(nwy * nwx * ws * ws, C)


def window_unpartition(xw, H, W, ws):
    C = xw.shape[-1]
    nwy, nwx = -(-H // ws), -(-W // ws)
    g = xw.reshape(nwy, nwx, ws, ws, C).transpose(0, 2, 1, 3, 4)
    return g.reshape(nwy * ws, nwx * ws, C)[:H, :W].reshape(H * W, C)


def sdpa(q, k, v, scale):
    return softmax(scale * q.astype(np.float64) @ k.astype(np.float64).T) @ v.astype(np.float64)


def vit_attention(x, grid, E, heads, hd, ws, n1w, n1b, qkvw, qkvb, cs):
    """LN -> [partition] -> qkv linear -> RoPE -> per (window, head) SDPA."""
    s = ws if ws else grid
    xn = layernorm(x, n1w, n1b)
    xw = window_partition(xn, grid, grid, s) if ws else xn
    qkv = xw @ qkvw.astype(np.float64).T + qkvb
    N = s * s
    qkv = rope(qkv, E, hd, N, cs)
    rows = qkv.shape[0]
    out = np.zeros((rows, E))
    for w in range(rows // N):
        r = slice(w * N, (w + 1) * N)
        for h in range(heads):
            q = qkv[r, h * hd:(h + 1) * hd]
            k = qkv[r, E + h * hd:E + (h + 1) * hd]
            v = qkv[r, 2 * E + h * hd:2 * E + (h + 1) * hd]
            out[r, h * hd:(h + 1) * hd] = sdpa(q, k, v, 1.0 / math.sqrt(hd))
    return out, qkv


def mha(P, Nq, Nk, dint, q, sq, k, sk, v, sv, heads=8):
    """Decoder attention on projected tensors with per-prompt strides."""
    c = dint // heads
    out = np.zeros((P * Nq, dint))
    for p in range(P):
        qp = q.reshape(-1)[p * sq:p * sq + Nq * dint].reshape(Nq, dint)
        kp = k.reshape(-1)[p * sk:p * sk + Nk * dint].reshape(Nk, dint)
        vp = v.reshape(-1)[p * sv:p * sv + Nk * dint].reshape(Nk, dint)
        for h in range(heads):
            cols = slice(h * c, (h + 1) * c)
            out[p * Nq:(p + 1) * Nq, cols] = sdpa(qp[:, cols], kp[:, cols],
                                                   vp[:, cols], 1.0 / math.sqrt(c))
    return out


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def patch_im2col(img, grid, ps):
    """[3, side, side] -> [grid^2, 3 * ps^2], column c * ps^2 + ky * ps + kx
    (numpy reshape of the patch grid)."""
    p = img.reshape(3, grid, ps, grid, ps).transpose(1, 3, 0, 2, 4)
    return p.reshape(grid * grid, 3 * ps * ps)


def vit_block(x, grid, E, heads, hd, mlp, w, cs):
    """One ViT block: x + proj(attn(LN1 x)) (windowed: unpartitioned),
    then + fc2(gelu(fc1(LN2 x)))."""
    ws = w["window"]
    attn, _ = vit_attention(x, grid, E, heads, hd, ws, w["n1w"], w["n1b"],
                            w["qkvw"], w["qkvb"], cs)
    y = attn @ w["projw"].astype(np.float64).T + w["projb"]
    if ws:
        y = window_unpartition(y, grid, grid, ws)
    x = x.astype(np.float64) + y
    h = gelu(layernorm(x, w["n2w"], w["n2b"]) @ w["l1w"].astype(np.float64).T
             + w["l1b"])
    return x + h @ w["l2w"].astype(np.float64).T + w["l2b"]


def encode_trunk(img, grid, ps, E, heads, hd, mlp, pe_w, pos, lnpw, lnpb,
                 blocks, rope_win, rope_glob):
    x = patch_im2col(img.astype(np.float64), grid, ps) @ pe_w.astype(np.float64).T
    x = layernorm(x + pos, lnpw, lnpb)
    for w in blocks:
        x = vit_block(x, grid, E, heads, hd, mlp, w,
                      rope_win if w["window"] else rope_glob)
    return x


def box_bias(dy, dx):
    """SAM 3's box relative position bias by broadcasting: dy [Nq, H, nh],
    dx [Nq, W, nh] -> [Nq, H * W, nh], key j = y * W + x gets
    dy[i, y] + dx[i, x]."""
    Nq, H, nh = dy.shape
    W = dx.shape[1]
    b = dy.astype(np.float64)[:, :, None, :] + dx.astype(np.float64)[:, None, :, :]
    return b.reshape(Nq, H * W, nh)


def attend(Q, K, V, heads, hd, causal=False, bias=None):
    """softmax(Q_h K_h^T / sqrt(hd) + bias_h (or the causal mask)) V_h per
    head, heads at columns h hd."""
    Q, K, V = (a.astype(np.float64) for a in (Q, K, V))
    Nq, Nk = Q.shape[0], K.shape[0]
    out = np.zeros((Nq, heads * hd))
    for h in range(heads):
        c = slice(h * hd, (h + 1) * hd)
        s = Q[:, c] @ K[:, c].T / math.sqrt(hd)
        if causal:
            s = np.where(np.arange(Nk)[None, :] > np.arange(Nq)[:, None], -np.inf, s)
        elif bias is not None:
            s = s + bias[:, :, h]
        out[:, c] = softmax(s) @ V[:, c]
    return out
