"""ctypes view of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke()
as the checker, and by the cpu_baseline leg of bench.py. The product
library never imports or calls it.

Every wrapper takes and returns numpy float32 arrays in the reference's
token-major layout; see sam3_oracle.h for the reference file:line each
function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ACT_NONE, ACT_GELU, ACT_RELU = 0, 1, 2
GEMM_SEQ, GEMM_CPU_T = 0, 1

_lib = None

_f = ctypes.c_float
_i = ctypes.c_int
_l = ctypes.c_long
_p = ctypes.c_void_p


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        gemm_args = [_i, _i, _i, _p, _l, _i, _l, _l, _p, _l, _i, _l, _l, _i,
                     _p, _l, _i, _l, _l, _i, _i, _p, _p, _l, _f, _i]
        L.or_gemm.argtypes = [_i] + gemm_args
        L.or_gemm_dispatch.argtypes = [_i] + gemm_args
        L.or_softmax_rows.argtypes = [_p, _l, _i]
        L.or_softmax_ext.argtypes = [_p, _l, _i, _i, _i, _i, _p, _p, _i, _i]
        L.or_attend.argtypes = [_i, _i, _i, _i, _i, _p, _i, _p, _i, _p, _i, _p,
                                _i, _i, _p, _p, _i, _l]
        L.or_attend.restype = _i
        L.or_layernorm.argtypes = [_p, _p, _l, _i, _p, _p, _f, _i]
        L.or_rope_apply.argtypes = [_p, _l, _i, _i, _i, _p]
        L.or_window_partition.argtypes = [_p, _p, _i, _i, _i, _i, _i]
        L.or_window_unpartition_add.argtypes = [_p, _p, _i, _i, _i, _i, _i]
        L.or_add_bcast.argtypes = [_p, _p, _p, _l, _l]
        att = [_p, _l, _p, _l, _p, _l, _p, _i, _i, _i, _i, _i, _f]
        L.or_attn_fewkeys.argtypes = att
        L.or_attn_manykeys.argtypes = att
        L.or_mha.argtypes = [_i, _i, _i, _i, _p, _l, _p, _l, _p, _l, _p]
        L.or_mha.restype = _i
        L.or_vit_attention.argtypes = [_i, _p, _i, _i, _i, _i, _i, _p, _p, _p,
                                       _p, _p, _l, _p, _p]
        L.or_vit_attention.restype = _i
        L.or_sdpa_f64.argtypes = [_i, _i, _i, _p, _i, _p, _i, _p, _i, _p, _i,
                                  ctypes.c_double]
        L.or_threads.restype = _i
        L.or_patch_im2col.argtypes = [_p, _p, _i, _i, _i]
        L.or_vit_block.argtypes = [_i, _p, _i, _i, _i, _i, _i,
                                   ctypes.POINTER(BlockW), _p, _l]
        L.or_vit_block.restype = _i
        L.or_encode_trunk.argtypes = [_i, _p, _i, _i, _i, _i, _i, _i, _p, _p,
                                      _p, _p, ctypes.POINTER(BlockW), _i, _p,
                                      _p, _l, _p]
        L.or_encode_trunk.restype = _i
        _lib = L
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def threads():
    return lib().or_threads()


def gemm(kind, M, N, K, A, aoff, lda, sa0, sa1, B, boff, ldb, sb0, sb1,
         transb, C, coff, ldc, sc0, sc1, nb, nb1, bias=None, R=None, roff=0,
         alpha=1.0, act=ACT_NONE, dispatch_cpu=None):
    """C (updated in place) = act(alpha A op(B) + bias) + R.

    kind is GEMM_SEQ or GEMM_CPU_T; with dispatch_cpu set, the kernel is
    chosen the way sam3_model.c:230-302 chooses it instead. R may be C.
    """
    args = (M, N, K, _ptr(A), aoff, lda, sa0, sa1, _ptr(B), boff, ldb, sb0,
            sb1, transb, _ptr(C), coff, ldc, sc0, sc1, nb, nb1, _ptr(bias),
            _ptr(R), roff, alpha, act)
    if dispatch_cpu is None:
        lib().or_gemm(kind, *args)
    else:
        lib().or_gemm_dispatch(int(dispatch_cpu), *args)
    return C


def linear(X, W, b=None, act=ACT_NONE, cpu=True, Y=None, residual=False):
    """Y = act(X W^T + b) (+ Y), as linear() (sam3_model.c:305-310)."""
    X = _f32(X)
    W = _f32(W)
    rows, nin = X.shape
    nout = W.shape[0]
    if Y is None:
        Y = np.zeros((rows, nout), np.float32)
    b = None if b is None else _f32(b)
    gemm(0, rows, nout, nin, X, 0, nin, 0, 0, W, 0, nin, 0, 0, 1, Y, 0, nout,
         0, 0, 1, 1, b, Y if residual else None, 0, 1.0, act, dispatch_cpu=cpu)
    return Y


def softmax_rows(S):
    S = _f32(S).copy()
    L = S.shape[-1]
    lib().or_softmax_rows(_ptr(S), S.size // L, L)
    return S


def softmax_ext(S, Nq, h0=0, causal=False, dy=None, dx=None, W=0, nh=1):
    """softmax_ext over the rows of S [rows, L] (row = head * Nq + query,
    heads from h0); dy [Nq, L / W, nh] and dx [Nq, W, nh] the box bias."""
    S = _f32(S).copy()
    L = S.shape[-1]
    dy = None if dy is None else _f32(dy)
    dx = None if dx is None else _f32(dx)
    lib().or_softmax_ext(_ptr(S), S.size // L, L, Nq, h0, int(bool(causal)),
                         _ptr(dy), _ptr(dx), W, nh)
    return S


def attend(Q, K, V, heads, hd, causal=False, dy=None, dx=None, W=0,
           score_cap=(512 << 20) // 4, cpu=False, O=None):
    """attend() of sam3_text.c:305-343 on row-major Q [Nq, ldq], K / V
    [Nk, ld]; returns O [Nq, heads * hd] (or updates the given O)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    Nq, Nk = Q.shape[0], K.shape[0]
    if O is None:
        O = np.zeros((Nq, heads * hd), np.float32)
    dy = None if dy is None else _f32(dy)
    dx = None if dx is None else _f32(dx)
    hc = lib().or_attend(int(cpu), Nq, Nk, heads, hd, _ptr(Q), Q.shape[1],
                         _ptr(K), K.shape[1], _ptr(V), V.shape[1], _ptr(O),
                         O.shape[1], int(bool(causal)), _ptr(dy), _ptr(dx), W,
                         score_cap)
    if hc < 1:
        raise ValueError("score buffer cannot hold one head")
    return O


def layernorm(X, g, b, eps=1e-5, act=ACT_NONE):
    X = _f32(X)
    C = X.shape[-1]
    Y = np.empty_like(X)
    g = _f32(g)
    b = _f32(b)
    lib().or_layernorm(_ptr(X), _ptr(Y), X.size // C, C, _ptr(g), _ptr(b),
                       eps, act)
    return Y


def rope_apply(qkv, E, hd, npos, cs):
    """In-place RoPE on a copy of qkv [rows, 3E]; cs is [npos, hd/2, 2]."""
    qkv = _f32(qkv).copy()
    cs = _f32(cs)
    lib().or_rope_apply(_ptr(qkv), qkv.size // (3 * E), E, hd, npos, _ptr(cs))
    return qkv


def window_partition(X, H, W, C, ws):
    nwx = (H + ws - 1) // ws
    out = np.empty((nwx * nwx * ws * ws, C), np.float32)
    X = _f32(X)
    lib().or_window_partition(_ptr(X), _ptr(out), H, W, C, ws, nwx)
    return out


def window_unpartition_add(X, Wd, H, W, C, ws):
    nwx = (H + ws - 1) // ws
    X = _f32(X).copy()
    Wd = _f32(Wd)
    lib().or_window_unpartition_add(_ptr(X), _ptr(Wd), H, W, C, ws, nwx)
    return X


def add_bcast(a, b, bmod):
    a = _f32(a)
    out = np.empty_like(a)
    b = _f32(b)
    lib().or_add_bcast(_ptr(out), _ptr(a), _ptr(b), a.size, bmod)
    return out


def attn_fewkeys(Q, sq, K, sk, V, sv, P, Nq, Nk, dint, c, scale):
    O = np.zeros((P * Nq, dint), np.float32)
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    lib().or_attn_fewkeys(_ptr(Q), sq, _ptr(K), sk, _ptr(V), sv, _ptr(O), P,
                          Nq, Nk, dint, c, scale)
    return O


def attn_manykeys(Q, sq, K, sk, V, sv, P, Nq, Nk, dint, c, scale):
    O = np.zeros((P * Nq, dint), np.float32)
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    lib().or_attn_manykeys(_ptr(Q), sq, _ptr(K), sk, _ptr(V), sv, _ptr(O), P,
                           Nq, Nk, dint, c, scale)
    return O


def mha(P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv):
    O = np.zeros((P * Nq, dint), np.float32)
    qp, kp, vp = _f32(qp), _f32(kp), _f32(vp)
    rc = lib().or_mha(P, Nq, Nk, dint, _ptr(qp), sq, _ptr(kp), sk, _ptr(vp),
                      sv, _ptr(O))
    if rc != 0:
        raise ValueError("mha: unsupported shape")
    return O


def vit_attention(x, grid, E, heads, hd, ws, n1w, n1b, qkvw, qkvb, rope,
                  score_cap=(512 << 20) // 4, cpu=True, want_qkv=False):
    """Attention region of one ViT block; returns attn [rows, E] (and qkv)."""
    s = ws if ws else grid
    nwx = (grid + s - 1) // s
    rows = nwx * nwx * s * s
    attn = np.zeros((rows, E), np.float32)
    qkv = np.zeros((rows, 3 * E), np.float32) if want_qkv else None
    x, n1w, n1b = _f32(x), _f32(n1w), _f32(n1b)
    qkvw, qkvb, rope = _f32(qkvw), _f32(qkvb), _f32(rope)
    hc = lib().or_vit_attention(int(cpu), _ptr(x), grid, E, heads, hd, ws,
                                _ptr(n1w), _ptr(n1b), _ptr(qkvw), _ptr(qkvb),
                                _ptr(rope), score_cap, _ptr(attn), _ptr(qkv))
    if hc < 1:
        raise ValueError("score buffer cannot hold one head")
    return (attn, qkv) if want_qkv else attn


class BlockW(ctypes.Structure):
    """struct or_block_w."""
    _fields_ = [(n, _p) for n in ("n1w", "n1b", "qkvw", "qkvb", "projw",
                                  "projb", "n2w", "n2b", "l1w", "l1b", "l2w",
                                  "l2b")] + [("window", _i)]


BLOCK_KEYS = ("n1w", "n1b", "qkvw", "qkvb", "projw", "projb", "n2w", "n2b",
              "l1w", "l1b", "l2w", "l2b")


def _block_w(w, keep):
    """BlockW from a dict of weight arrays (float32 copies kept alive in
    `keep`)."""
    b = BlockW()
    for k in BLOCK_KEYS:
        a = _f32(w[k])
        keep.append(a)
        setattr(b, k, a.ctypes.data)
    b.window = int(w["window"])
    return b


def patch_im2col(img, side, grid, ps):
    img = _f32(img)
    out = np.zeros((grid * grid, 3 * ps * ps), np.float32)
    lib().or_patch_im2col(_ptr(img), _ptr(out), side, grid, ps)
    return out


def vit_block(x, grid, E, heads, hd, mlp, w, rope,
              score_cap=(512 << 20) // 4, cpu=True):
    """One ViT block (dict w of weights, w["window"] the window side) on
    x [grid^2, E]; returns the new x."""
    keep = []
    b = _block_w(w, keep)
    x = np.array(x, np.float32, copy=True)
    rope = _f32(rope)
    if lib().or_vit_block(int(cpu), _ptr(x), grid, E, heads, hd, mlp,
                          ctypes.byref(b), _ptr(rope), score_cap) < 1:
        raise ValueError("score buffer cannot hold one head")
    return x


def encode_trunk(img, grid, ps, E, heads, hd, mlp, pe_w, pos, lnpw, lnpb,
                 blocks, rope_win, rope_glob, score_cap=(512 << 20) // 4,
                 cpu=True):
    """Image encoder trunk: img [3, side, side] -> x [grid^2, E]."""
    keep = []
    arr = (BlockW * len(blocks))(*[_block_w(w, keep) for w in blocks])
    img, pe_w, pos = _f32(img), _f32(pe_w), _f32(pos)
    lnpw, lnpb = _f32(lnpw), _f32(lnpb)
    rw = _f32(rope_win) if rope_win is not None else None
    rg = _f32(rope_glob) if rope_glob is not None else None
    x = np.zeros((grid * grid, E), np.float32)
    if lib().or_encode_trunk(int(cpu), _ptr(img), grid, ps, E, heads, hd, mlp,
                             _ptr(pe_w), _ptr(pos), _ptr(lnpw), _ptr(lnpb),
                             arr, len(blocks), _ptr(rw), _ptr(rg), score_cap,
                             _ptr(x)) < 0:
        raise ValueError("score buffer cannot hold one head")
    return x


def sdpa_f64(Q, K, V, scale):
    Q = np.ascontiguousarray(Q, np.float64)
    K = np.ascontiguousarray(K, np.float64)
    V = np.ascontiguousarray(V, np.float64)
    Nq, d = Q.shape
    Nk = K.shape[0]
    dv = V.shape[1]
    assert dv == d
    O = np.zeros((Nq, d), np.float64)
    lib().or_sdpa_f64(Nq, Nk, d, _ptr(Q), d, _ptr(K), d, _ptr(V), d, _ptr(O),
                      d, scale)
    return O


def rope_table(side, hd=64, theta=10000.0):
    """Synthetic axial 2D RoPE table [side*side, hd/2, 2] of (cos, sin).

    Frequencies f_k = theta^(-4k/hd) for k < hd/4; pair k < hd/4 rotates
    by x * f_k and pair hd/4 + k by y * f_k at position p = y * side + x.
    The reference reads this table from its checkpoint; here it is an
    input shared by both sides.
    """
    nf = hd // 2
    q = nf // 2
    f = theta ** (-4.0 * np.arange(q, dtype=np.float64) / hd)
    pos = np.arange(side * side)
    x = (pos % side).astype(np.float64)
    y = (pos // side).astype(np.float64)
    ang = np.concatenate([np.outer(x, f), np.outer(y, f)], axis=1)
    return np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)


# ------------------------------------------------------------ mask decoder

_FP = ctypes.POINTER(ctypes.c_float)
_ATT = ("qw", "qb", "kw", "kb", "vw", "vb", "ow", "ob")
_LAYER = ("n1w", "n1b", "n2w", "n2b", "n3w", "n3b", "n4w", "n4b", "m1w",
          "m1b", "m2w", "m2b")


class OrAttnW(ctypes.Structure):
    _fields_ = [(n, _FP) for n in _ATT] + [("dint", _i)]


class OrDecLayer(ctypes.Structure):
    _fields_ = [("self_", OrAttnW), ("t2i", OrAttnW), ("i2t", OrAttnW)] + \
        [(n, _FP) for n in _LAYER]


class OrDecoder(ctypes.Structure):
    _fields_ = [("grid", _i), ("img", _i)] + \
        [(n, _FP) for n in ("gauss", "point_emb", "not_a_point", "no_mask")] + \
        [("layers", OrDecLayer * 2), ("final_t2i", OrAttnW)] + \
        [(n, _FP) for n in ("nfw", "nfb", "up0w", "up0b", "up1w", "up1b",
                            "up3w", "up3b", "obj_token", "iou_token",
                            "mask_tokens")] + \
        [("hyper_w", (_FP * 3) * 4), ("hyper_b", (_FP * 3) * 4),
         ("iou_w", _FP * 3), ("iou_b", _FP * 3)]


def _dec_lib():
    L = lib()
    if getattr(L, "_dec_ready", False):
        return L
    DP = ctypes.POINTER(OrDecoder)
    L.or_pe_encode.argtypes = [_p, _f, _f, _p]
    L.or_host_linear.argtypes = [_p, _p, _p, _i, _i, _i, _p]
    L.or_convt_scatter.argtypes = [_p, _p, _p, _p, _i, _i, _i, _i, _i]
    L.or_mask_logits.argtypes = [_p, _p, _p, _i, _i]
    L.or_mask_post.argtypes = [_p, _p, _i, _i, _i, _i, _f, _p, _p]
    L.or_fill_holes.argtypes = [_p, _i, _i]
    L.or_fill_holes.restype = _i
    L.or_postprocess.argtypes = [_p, _i, _i, _p, _i, _i, _f, _i, _i, _p, _p]
    L.or_dec_prepare.argtypes = [DP, _p, _p, _p, _p, _p, _p, _p]
    L.or_t2i_attention.argtypes = [_i, _i, _p, _p, _p, _p,
                                   ctypes.POINTER(OrAttnW), _p]
    L.or_i2t_attention.argtypes = [_i, _i, _i, _p, _p, _p, _p, _p, _p,
                                   ctypes.POINTER(OrDecLayer)]
    L.or_prompt_tokens.argtypes = [DP, _i, _p, _p]
    L.or_sam_decode.argtypes = [DP, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                _p, _p, _p]
    L._dec_ready = True
    return L


class DecoderW:
    """struct or_decoder over the numpy arrays of a weight dict (the names of
    sam3_hip.random_decoder_weights); the arrays are kept alive here."""

    def __init__(self, w, grid, img=1008):
        self.keep = {k: _f32(v) for k, v in w.items()}
        d = self.d = OrDecoder()
        d.grid, d.img = grid, img

        def fp(name):
            return self.keep[name].ctypes.data_as(_FP)

        for n in ("gauss", "point_emb", "not_a_point", "no_mask", "nfw", "nfb",
                  "up0w", "up0b", "up1w", "up1b", "up3w", "up3b", "obj_token",
                  "iou_token", "mask_tokens"):
            setattr(d, n, fp(n))

        def attn(dst, prefix, dint):
            for n in _ATT:
                setattr(dst, n, fp(prefix + n))
            dst.dint = dint

        for layer in range(2):
            p = "layers.%d." % layer
            Lw = d.layers[layer]
            attn(Lw.self_, p + "self.", 256)
            attn(Lw.t2i, p + "t2i.", 128)
            attn(Lw.i2t, p + "i2t.", 128)
            for n in _LAYER:
                setattr(Lw, n, fp(p + n))
        attn(d.final_t2i, "final_t2i.", 128)
        for i in range(4):
            for j in range(3):
                d.hyper_w[i][j] = fp("hyper.%d.%dw" % (i, j))
                d.hyper_b[i][j] = fp("hyper.%d.%db" % (i, j))
        for j in range(3):
            d.iou_w[j] = fp("iou.%dw" % j)
            d.iou_b[j] = fp("iou.%db" % j)

    @property
    def ptr(self):
        return ctypes.byref(self.d)


def pe_encode(gauss, x, y):
    out = np.zeros(256, np.float32)
    gauss = _f32(gauss)
    _dec_lib().or_pe_encode(_ptr(gauss), x, y, _ptr(out))
    return out


def host_linear(W, b, x, relu=False):
    W, b, x = _f32(W), _f32(b), _f32(x)
    y = np.zeros(W.shape[0], np.float32)
    _dec_lib().or_host_linear(_ptr(W), _ptr(b), _ptr(x), W.shape[1],
                              W.shape[0], int(relu), _ptr(y))
    return y


def convt_scatter(G, bias, add, P, H, W, Co, act=ACT_NONE):
    G, bias = _f32(G), _f32(bias)
    add = None if add is None else _f32(add)
    out = np.zeros((P, 2 * H, 2 * W, Co), np.float32)
    _dec_lib().or_convt_scatter(_ptr(G), _ptr(out), _ptr(bias), _ptr(add), P,
                                H, W, Co, act)
    return out


def mask_logits(U, hyper, P, npix):
    U, hyper = _f32(U), _f32(hyper)
    out = np.zeros((P, 3, npix), np.float32)
    _dec_lib().or_mask_logits(_ptr(U), _ptr(hyper), _ptr(out), P, npix)
    return out


def mask_post(lowres, sel, L, out_h, out_w, offset):
    """Returns (mask [n][out_h][out_w] uint8, stats [n][6])."""
    lowres = _f32(lowres)
    sel = np.ascontiguousarray(sel, np.int32)
    n = len(sel)
    mask = np.zeros((n, out_h, out_w), np.uint8)
    stats = np.tile(np.array([0, 0, 0x7fffffff, 0x7fffffff, -1, -1],
                             np.int32), (n, 1))
    _dec_lib().or_mask_post(_ptr(lowres), _ptr(sel), n, L, out_h, out_w,
                            offset, _ptr(mask), _ptr(stats))
    return mask, stats


def fill_holes(v, max_area):
    v = _f32(v).copy()
    L = v.shape[0]
    changed = _dec_lib().or_fill_holes(_ptr(v), L, max_area)
    return v, bool(changed)


def postprocess(lowres, sel, out_h, out_w, offset, fill, max_area=256):
    """sam_postprocess on a host copy: returns (lowres after filling, mask,
    stats)."""
    lowres = _f32(lowres).copy()
    L = lowres.shape[-1]
    sel = np.ascontiguousarray(sel, np.int32)
    n = len(sel)
    mask = np.zeros((n, out_h, out_w), np.uint8)
    stats = np.zeros((n, 6), np.int32)
    _dec_lib().or_postprocess(_ptr(lowres), L, n, _ptr(sel), out_h, out_w,
                              offset, int(fill), max_area, _ptr(mask),
                              _ptr(stats))
    return lowres, mask, stats


def dec_prepare(dw, emb):
    """Returns dict pe, src, srcpe, kp0, vp0, qp0 of or_dec_prepare."""
    G = dw.d.grid
    T = G * G
    emb = _f32(emb)
    out = {"pe": np.zeros((T, 256), np.float32),
           "src": np.zeros((T, 256), np.float32),
           "srcpe": np.zeros((T, 256), np.float32),
           "kp0": np.zeros((T, 128), np.float32),
           "vp0": np.zeros((T, 128), np.float32),
           "qp0": np.zeros((T, 128), np.float32)}
    _dec_lib().or_dec_prepare(dw.ptr, _ptr(emb), *(_ptr(out[k]) for k in (
        "pe", "src", "srcpe", "kp0", "vp0", "qp0")))
    return out


def prompt_tokens(dw, points):
    pts = _f32(points).reshape(-1, 2)
    P = pts.shape[0]
    tok = np.zeros((P, 8, 256), np.float32)
    _dec_lib().or_prompt_tokens(dw.ptr, P, _ptr(pts), _ptr(tok))
    return tok


def t2i_attention(P, T, qry, qpe, keys, pe, attn_w):
    """Returns (qry after the residual, kin)."""
    qry = _f32(qry).copy()
    kin = np.zeros((P, T, 256), np.float32)
    qpe, keys, pe = _f32(qpe), _f32(keys), _f32(pe)
    _dec_lib().or_t2i_attention(P, T, _ptr(qry), _ptr(qpe), _ptr(keys),
                                _ptr(pe), ctypes.byref(attn_w), _ptr(kin))
    return qry, kin


def i2t_attention(layer, P, T, qry, qpe, keys, kin, qp0, src, layer_w):
    """Returns keys after the image -> token attention and norm4."""
    keys = _f32(keys).copy()
    args = [_f32(a) if a is not None else None for a in (qry, qpe, kin, qp0,
                                                          src)]
    _dec_lib().or_i2t_attention(layer, P, T, _ptr(args[0]), _ptr(args[1]),
                                _ptr(keys), _ptr(args[2]), _ptr(args[3]),
                                _ptr(args[4]), ctypes.byref(layer_w))
    return keys


def sam_decode(dw, points, prep, feat_s0, feat_s1):
    """Returns (iou [P][3], lowres [P][3][4G][4G], tokens [P][8][256],
    hyper [P][3][32])."""
    G = dw.d.grid
    pts = _f32(points).reshape(-1, 2)
    P = pts.shape[0]
    iou = np.zeros((P, 3), np.float32)
    lowres = np.zeros((P, 3, 4 * G, 4 * G), np.float32)
    tokens = np.zeros((P, 8, 256), np.float32)
    hyper = np.zeros((P, 3, 32), np.float32)
    feat_s0, feat_s1 = _f32(feat_s0), _f32(feat_s1)
    _dec_lib().or_sam_decode(dw.ptr, P, _ptr(pts), _ptr(prep["pe"]),
                             _ptr(prep["src"]), _ptr(prep["kp0"]),
                             _ptr(prep["vp0"]), _ptr(prep["qp0"]),
                             _ptr(feat_s0), _ptr(feat_s1), _ptr(iou),
                             _ptr(lowres), _ptr(tokens), _ptr(hyper))
    return iou, lowres, tokens, hyper
