"""ctypes view of oracle/_ref/libsam3ref.so: the reference's own OpenCL
kernels (sam3_kernels.cl compiled unchanged for gfx950) launched the way
the reference host code launches them.

TEST INFRASTRUCTURE ONLY: used by tests/golden/gen_golden.py to write the
golden vectors and by GPU tests as a live cross-check. Needs an OpenCL
GPU device (the ROCm runtime on the GPU box).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")
LIB = os.path.join(REF_DIR, "libsam3ref.so")
CO = os.path.join(REF_DIR, "sam3_kernels.gfx950.co")

GEMM, GEMM_BIG, GEMM_CPU_T, GEMM_CPU_N = 0, 1, 2, 3

_lib = None


def available():
    return os.path.exists(LIB) and os.path.exists(CO)


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB)
        i, l, f, p = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_void_p
        L.ref_init.argtypes = [ctypes.c_char_p]
        L.ref_error.restype = ctypes.c_char_p
        L.ref_device.restype = ctypes.c_char_p
        L.ref_gemm.argtypes = [i, i, i, i, p, l, l, i, l, l, p, l, l, i, l, l,
                               i, p, l, l, i, l, l, i, i, p, i, l, f, i]
        L.ref_softmax_rows.argtypes = [p, l, i]
        L.ref_softmax_ext.argtypes = [p, l, i, i, i, i, p, l, p, l, i, i]
        L.ref_layernorm.argtypes = [p, p, l, i, p, p, f, i]
        L.ref_rope_apply.argtypes = [p, l, i, i, i, p]
        L.ref_window_partition.argtypes = [p, p, i, i, i, i]
        L.ref_window_unpartition_add.argtypes = [p, p, i, i, i, i]
        L.ref_mha.argtypes = [i, i, i, i, p, l, l, p, l, l, p, l, l, p]
        L.ref_convt_scatter.argtypes = [p, p, p, p, i, i, i, i, i]
        L.ref_mask_logits.argtypes = [p, p, p, i, i]
        L.ref_mask_post.argtypes = [p, i, p, i, i, i, i, f, p, p]
        if L.ref_init(CO.encode()) != 0:
            raise RuntimeError("reference OpenCL init: " + L.ref_error().decode())
        _lib = L
    return _lib


def _c(a):
    return np.ascontiguousarray(a, np.float32)


def _ok(rc):
    if rc != 0:
        raise RuntimeError(lib().ref_error().decode())


def device():
    return lib().ref_device().decode()


def gemm(kernel, M, N, K, A, aoff, lda, sa0, sa1, B, boff, ldb, sb0, sb1,
         transb, C, coff, ldc, sc0, sc1, nb, nb1, bias=None, use_r=False,
         roff=0, alpha=1.0, act=0):
    A, B, C = _c(A), _c(B), _c(C).copy()
    bias = None if bias is None else _c(bias)
    _ok(lib().ref_gemm(kernel, M, N, K, A.ctypes.data, A.size, aoff, lda, sa0,
                       sa1, B.ctypes.data, B.size, boff, ldb, sb0, sb1, transb,
                       C.ctypes.data, C.size, coff, ldc, sc0, sc1, nb, nb1,
                       None if bias is None else bias.ctypes.data, int(use_r),
                       roff, alpha, act))
    return C


def softmax_rows(S):
    S = _c(S).copy()
    _ok(lib().ref_softmax_rows(S.ctypes.data, S.size // S.shape[-1],
                               S.shape[-1]))
    return S


def softmax_ext(S, Nq, h0=0, causal=False, dy=None, dx=None, W=0, nh=1):
    S = _c(S).copy()
    L = S.shape[-1]
    dy = None if dy is None else _c(dy)
    dx = None if dx is None else _c(dx)
    _ok(lib().ref_softmax_ext(S.ctypes.data, S.size // L, L, Nq, h0,
                              int(bool(causal)),
                              None if dy is None else dy.ctypes.data,
                              0 if dy is None else dy.size,
                              None if dx is None else dx.ctypes.data,
                              0 if dx is None else dx.size, W, nh))
    return S


def layernorm(X, g, b, eps=1e-5, act=0):
    X, g, b = _c(X), _c(g), _c(b)
    Y = np.zeros_like(X)
    C = X.shape[-1]
    _ok(lib().ref_layernorm(X.ctypes.data, Y.ctypes.data, X.size // C, C,
                            g.ctypes.data, b.ctypes.data, eps, act))
    return Y


def rope_apply(qkv, E, hd, npos, cs):
    qkv, cs = _c(qkv).copy(), _c(cs)
    _ok(lib().ref_rope_apply(qkv.ctypes.data, qkv.size // (3 * E), E, hd, npos,
                             cs.ctypes.data))
    return qkv


def window_partition(X, H, C, ws):
    nwx = -(-H // ws)
    X = _c(X)
    out = np.zeros((nwx * nwx * ws * ws, C), np.float32)
    _ok(lib().ref_window_partition(X.ctypes.data, out.ctypes.data, H, C, ws,
                                   nwx))
    return out


def window_unpartition_add(X, Wd, H, C, ws):
    nwx = -(-H // ws)
    X, Wd = _c(X).copy(), _c(Wd)
    _ok(lib().ref_window_unpartition_add(X.ctypes.data, Wd.ctypes.data, H, C,
                                         ws, nwx))
    return X


def mha(P, Nq, Nk, dint, Q, sq, K, sk, V, sv):
    Q, K, V = _c(Q), _c(K), _c(V)
    O = np.zeros((P * Nq, dint), np.float32)
    _ok(lib().ref_mha(P, Nq, Nk, dint, Q.ctypes.data, Q.size, sq,
                      K.ctypes.data, K.size, sk, V.ctypes.data, V.size, sv,
                      O.ctypes.data))
    return O


def convt_scatter(G, bias, add, P, H, W, Co, act):
    G, bias = _c(G), _c(bias)
    add = None if add is None else _c(add)
    out = np.zeros((P, 2 * H, 2 * W, Co), np.float32)
    _ok(lib().ref_convt_scatter(G.ctypes.data, out.ctypes.data,
                                bias.ctypes.data,
                                None if add is None else add.ctypes.data, P, H,
                                W, Co, act))
    return out


def mask_logits(U, hyper, P, npix):
    U, hyper = _c(U), _c(hyper)
    out = np.zeros((P, 3, npix), np.float32)
    _ok(lib().ref_mask_logits(U.ctypes.data, hyper.ctypes.data,
                              out.ctypes.data, P, npix))
    return out


def mask_post(lowres, sel, L, out_h, out_w, offset):
    lowres = _c(lowres)
    sel = np.ascontiguousarray(sel, np.int32)
    n = len(sel)
    mask = np.zeros((n, out_h, out_w), np.uint8)
    stats = np.tile(np.array([0, 0, 0x7fffffff, 0x7fffffff, -1, -1], np.int32),
                    (n, 1))
    _ok(lib().ref_mask_post(lowres.ctypes.data, lowres.shape[0], sel.ctypes.data,
                            n, L, out_h, out_w, offset, mask.ctypes.data,
                            stats.ctypes.data))
    return mask, stats
