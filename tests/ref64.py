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


# ------------------------------------------------------------ mask decoder
# Written from the PyTorch SAM 2 / SAM 3 mask decoder semantics
# (PositionEmbeddingRandom, TwoWayTransformer with skip_first_layer_pe on
# layer 0, MaskDecoder with the object-score token, LayerNorm2d, exact GELU,
# hypernetwork MLPs, sigmoid IoU head), in float64 with heads split by
# reshape.


def gelu_fast(x):
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def pe_random(gauss, xy):
    """xy [..., 2] in [0, 1] -> [..., 256] = [sin, cos](2 pi (2 xy - 1) G)."""
    c = (2.0 * np.asarray(xy, np.float64) - 1.0) @ gauss.astype(np.float64)
    c = 2.0 * math.pi * c
    return np.concatenate([np.sin(c), np.cos(c)], -1)


def _lin(x, w, b):
    return x @ w.astype(np.float64).T + b.astype(np.float64)


def dec_attention(w, prefix, q, k, v, heads=8):
    """SAM Attention: project, split heads, softmax(q k^T / sqrt(c)) v,
    merge, out-project. q [B, Nq, 256], k / v [B, Nk, 256]."""
    Q = _lin(q, w[prefix + "qw"], w[prefix + "qb"])
    K = _lin(k, w[prefix + "kw"], w[prefix + "kb"])
    V = _lin(v, w[prefix + "vw"], w[prefix + "vb"])
    B, Nq, D = Q.shape
    c = D // heads
    Qh = Q.reshape(B, Nq, heads, c).transpose(0, 2, 1, 3)
    Kh = K.reshape(B, -1, heads, c).transpose(0, 2, 1, 3)
    Vh = V.reshape(B, -1, heads, c).transpose(0, 2, 1, 3)
    s = Qh @ Kh.transpose(0, 1, 3, 2) / math.sqrt(c)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    O = (p @ Vh).transpose(0, 2, 1, 3).reshape(B, Nq, D)
    return _lin(O, w[prefix + "ow"], w[prefix + "ob"])


def conv_transpose2x2(x, wt, b):
    """ConvTranspose2d(kernel 2, stride 2) on a channel-last map x [B, H,
    W, Ci] with weight [Ci, Co, 2, 2]: out[b, 2y + i, 2x + j, o] =
    sum_c x[b, y, x, c] wt[c, o, i, j] + b[o]."""
    B, H, W, _ = x.shape
    Co = wt.shape[1]
    t = np.einsum("byxc,coij->byixjo", x, wt.astype(np.float64))
    return t.reshape(B, 2 * H, 2 * W, Co) + b.astype(np.float64)


def decode64(w, grid, img, points, emb, feat_s0, feat_s1):
    """Returns (iou [P][3], lowres [P][3][4 grid][4 grid]) in float64."""
    G, T = grid, grid * grid
    pts = np.asarray(points, np.float64).reshape(-1, 2)
    P = pts.shape[0]
    f = {k: np.asarray(v, np.float64) for k, v in w.items()}
    ys, xs = np.meshgrid(np.arange(G), np.arange(G), indexing="ij")
    pe = pe_random(f["gauss"], np.stack([(xs + 0.5) / G, (ys + 0.5) / G],
                                        -1)).reshape(T, 256)
    src = np.asarray(emb, np.float64) + f["no_mask"]
    # Tokens: obj score, IoU, 4 mask tokens, the point, the padding point.
    tok = np.zeros((P, 8, 256))
    tok[:, 0] = f["obj_token"]
    tok[:, 1] = f["iou_token"]
    tok[:, 2:6] = f["mask_tokens"]
    tok[:, 6] = pe_random(f["gauss"], (pts + 0.5) / img) + f["point_emb"][1]
    tok[:, 7] = f["not_a_point"]
    qpe = tok
    queries = tok.copy()
    keys = np.broadcast_to(src, (P, T, 256)).copy()
    kpe = np.broadcast_to(pe, (P, T, 256))

    def ln(x, pfx):
        return layernorm(x, f[pfx + "w"], f[pfx + "b"], 1e-5)

    for layer in range(2):
        p = "layers.%d." % layer
        if layer == 0:
            queries = dec_attention(f, p + "self.", queries, queries, queries)
        else:
            q = queries + qpe
            queries = queries + dec_attention(f, p + "self.", q, q, queries)
        queries = ln(queries, p + "n1")
        queries = queries + dec_attention(f, p + "t2i.", queries + qpe,
                                          keys + kpe, keys)
        queries = ln(queries, p + "n2")
        h = np.maximum(_lin(queries, f[p + "m1w"], f[p + "m1b"]), 0.0)
        queries = ln(queries + _lin(h, f[p + "m2w"], f[p + "m2b"]), p + "n3")
        keys = keys + dec_attention(f, p + "i2t.", keys + kpe, queries + qpe,
                                    queries)
        keys = ln(keys, p + "n4")
    queries = queries + dec_attention(f, "final_t2i.", queries + qpe,
                                      keys + kpe, keys)
    queries = ln(queries, "nf")
    # Upscaling.
    x = keys.reshape(P, G, G, 256)
    u = conv_transpose2x2(x, f["up0w"].reshape(256, 64, 2, 2), f["up0b"])
    u = u + np.asarray(feat_s1, np.float64).reshape(2 * G, 2 * G, 64)
    u = gelu_fast(layernorm(u, f["up1w"], f["up1b"], 1e-6))
    u = conv_transpose2x2(u, f["up3w"].reshape(64, 32, 2, 2), f["up3b"])
    u = gelu_fast(u + np.asarray(feat_s0, np.float64).reshape(4 * G, 4 * G, 32))
    # Hypernetwork MLPs (mask tokens 1..3) and the IoU head.
    hyper = np.zeros((P, 3, 32))
    for i in range(1, 4):
        h = queries[:, 2 + i]
        for j in range(3):
            h = _lin(h, f["hyper.%d.%dw" % (i, j)], f["hyper.%d.%db" % (i, j)])
            if j < 2:
                h = np.maximum(h, 0.0)
        hyper[:, i - 1] = h
    h = queries[:, 1]
    for j in range(3):
        h = _lin(h, f["iou.%dw" % j], f["iou.%db" % j])
        if j < 2:
            h = np.maximum(h, 0.0)
    iou = 1.0 / (1.0 + np.exp(-h[:, 1:4]))
    lowres = np.einsum("pkc,pyxc->pkyx", hyper, u)
    return iou, lowres
