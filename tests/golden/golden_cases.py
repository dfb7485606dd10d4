"""Cases of the golden vectors: seeded inputs and the sequence of
reference kernels that produces each output.

`run_reference(name, case, impl)` runs a case through an implementation
module with the API of oracle/refk.py (the reference's own kernels) or
of OracleImpl below (the CPU oracle restating them); the golden files
hold the former's outputs, tests/test_golden.py compares the latter's,
and tests/test_gpu_golden.py the HIP path's.
"""
import math

import numpy as np

GEMM, GEMM_BIG, GEMM_CPU_T, GEMM_CPU_N = 0, 1, 2, 3


def rng(seed):
    return np.random.default_rng(seed)


def rope_table(side, hd=64, theta=10000.0):
    f = theta ** (-4.0 * np.arange(hd // 4) / hd)
    pos = np.arange(side * side)
    ang = np.concatenate([np.outer(pos % side, f), np.outer(pos // side, f)], 1)
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


# ------------------------------------------------------------------ cases

def _gemm_case(kernel, transb, seed):
    g = rng(seed)
    M, N, K, nb, nb1 = 150, 96, 68, 4, 2
    lda, ldc = K + 4, N + 4
    ldb = K + 8 if transb else N + 8
    brows = N if transb else K
    sa1, sb1, sc1 = M * lda, brows * ldb, M * ldc
    A = g.standard_normal(8 + nb * sa1).astype(np.float32)
    B = g.standard_normal(16 + nb * sb1).astype(np.float32)
    C = g.standard_normal(4 + nb * sc1).astype(np.float32)
    bias = g.standard_normal(N).astype(np.float32)
    args = dict(kernel=kernel, M=M, N=N, K=K, aoff=8, lda=lda, sa0=sa1 * nb1,
                sa1=sa1, boff=16, ldb=ldb, sb0=sb1 * nb1, sb1=sb1,
                transb=transb, coff=4, ldc=ldc, sc0=sc1 * nb1, sc1=sc1, nb=nb,
                nb1=nb1, roff=4, alpha=0.5, act=1)
    return {"kind": "gemm", "args": args, "inputs": [A, B, C, bias]}


def _softmax_case(L, seed):
    return {"kind": "softmax",
            "inputs": [(3 * rng(seed).standard_normal((16, L))).astype(np.float32)]}


def _ln_case(C, act, seed):
    g = rng(seed)
    X = (2 * g.standard_normal((8, C)) + 0.5).astype(np.float32)
    return {"kind": "layernorm", "act": act,
            "inputs": [X, g.standard_normal(C).astype(np.float32),
                       g.standard_normal(C).astype(np.float32)]}


def _rope_case(seed):
    E, side = 128, 6
    qkv = rng(seed).standard_normal((2 * side * side, 3 * E)).astype(np.float32)
    return {"kind": "rope", "E": E, "npos": side * side,
            "inputs": [qkv, rope_table(side)]}


def _window_case(seed):
    H, C, ws = 10, 8, 4
    g = rng(seed)
    X = g.standard_normal((H * H, C)).astype(np.float32)
    nwx = -(-H // ws)
    Wd = g.standard_normal((nwx * nwx * ws * ws, C)).astype(np.float32)
    return {"kind": "window", "H": H, "C": C, "ws": ws, "inputs": [X, Wd]}


def _mha_case(P, Nq, Nk, dint, shk, shq, seed):
    g = rng(seed)
    q = g.standard_normal(((1 if shq else P) * Nq, dint)).astype(np.float32)
    k = g.standard_normal(((1 if shk else P) * Nk, dint)).astype(np.float32)
    v = g.standard_normal(((1 if shk else P) * Nk, dint)).astype(np.float32)
    return {"kind": "mha", "P": P, "Nq": Nq, "Nk": Nk, "dint": dint,
            "sq": 0 if shq else Nq * dint, "sk": 0 if shk else Nk * dint,
            "inputs": [q, k, v]}


def _attn_case(N, E, heads, rope, gpu, seed):
    """Attention of one unit in the reference's row layout: optional
    rope_apply, then per head Q K^T (alpha 1/8), softmax_rows, P V, with
    the profile=cpu kernels (gemm_cpu_t / gemm_cpu_n) or the GPU ones
    (gemm_big)."""
    qkv = rng(seed).standard_normal((N, 3 * E)).astype(np.float32)
    side = math.isqrt(N)
    inputs = [qkv] + ([rope_table(side)] if rope else [])
    return {"kind": "attn", "N": N, "E": E, "heads": heads, "rope": rope,
            "gpu": gpu, "inputs": inputs,
            "sample_rows": np.arange(0, N, max(1, N // 64))[:64]}


def _vit_case(seed):
    """Attention region of a windowed block (sam3_model.c:991-1013) at a
    small size: LayerNorm, window partition, QKV linear, RoPE, attention."""
    grid, E, ws = 12, 128, 6
    g = rng(seed)
    x = g.standard_normal((grid * grid, E)).astype(np.float32)
    n1w = (1 + 0.1 * g.standard_normal(E)).astype(np.float32)
    n1b = (0.1 * g.standard_normal(E)).astype(np.float32)
    bound = math.sqrt(6.0 / (4 * E))
    w = g.uniform(-bound, bound, (3 * E, E)).astype(np.float32)
    b = g.uniform(-1 / math.sqrt(E), 1 / math.sqrt(E), 3 * E).astype(np.float32)
    return {"kind": "vit", "grid": grid, "E": E, "ws": ws,
            "inputs": [x, n1w, n1b, w, b, rope_table(ws)]}


def _softmax_ext_case(Nq, H, W, nh, h0, hc, causal, seed):
    """softmax_ext rows (row = head * Nq + query, heads from h0) of L = H W
    scores, the causal mask or the box bias dy [Nq, H, nh], dx [Nq, W, nh]."""
    g = rng(seed)
    L = H * W
    S = (3 * g.standard_normal((hc * Nq, L))).astype(np.float32)
    inputs = [S]
    if not causal:
        inputs += [g.standard_normal((Nq, H, nh)).astype(np.float32),
                   g.standard_normal((Nq, W, nh)).astype(np.float32)]
    return {"kind": "softmax_ext", "Nq": Nq, "W": W, "nh": nh, "h0": h0,
            "causal": causal, "inputs": inputs}


def _attend_case(Nq, Nk, heads, hd, mode, seed, W=0):
    """attend() (sam3_text.c:305-343) on Q [Nq, D], K / V [Nk, D],
    D = heads hd: mode "box" (bias, Nk = H W), "causal" or "plain"."""
    g = rng(seed)
    D = heads * hd
    inputs = [g.standard_normal((n, D)).astype(np.float32) for n in (Nq, Nk, Nk)]
    if mode == "box":
        inputs += [g.standard_normal((Nq, Nk // W, heads)).astype(np.float32),
                   g.standard_normal((Nq, W, heads)).astype(np.float32)]
    return {"kind": "attend", "Nq": Nq, "Nk": Nk, "heads": heads, "hd": hd,
            "mode": mode, "W": W, "inputs": inputs}


def _convt_case(P, H, W, Co, add, act, seed):
    """convt_scatter (sam3_kernels.cl:762-786) of a [P H W][Co 4] GEMM
    result, with the shared add map and the activation or without."""
    g = rng(seed)
    inputs = [g.standard_normal((P * H * W, Co * 4)).astype(np.float32),
              g.standard_normal(Co).astype(np.float32)]
    if add:
        inputs.append(g.standard_normal((2 * H, 2 * W, Co)).astype(np.float32))
    return {"kind": "convt", "P": P, "H": H, "W": W, "Co": Co, "act": act,
            "inputs": inputs}


def _logits_case(P, npix, seed):
    """mask_logits (sam3_kernels.cl:789-805): U [P npix][32], hyper [P][96]."""
    g = rng(seed)
    return {"kind": "logits", "P": P, "npix": npix,
            "inputs": [g.standard_normal((P * npix, 32)).astype(np.float32),
                       g.standard_normal((P, 96)).astype(np.float32)]}


def _mask_post_case(L, out_h, out_w, dyadic, seed):
    """mask_post (sam3_kernels.cl:807-883) of planes 3, 0, 4 of five L x L
    logit planes; dyadic: logits in multiples of 1/8 with 2x / 0.5x
    resizes, so every bilinear value is exact."""
    g = rng(seed)
    if dyadic:
        low = (g.integers(-40, 41, (5, L, L)) / 8.0).astype(np.float32)
    else:
        low = (2 * g.standard_normal((5, L, L))).astype(np.float32)
    return {"kind": "mask_post", "L": L, "out_h": out_h, "out_w": out_w,
            "offset": 0.5, "inputs": [low, np.array([3, 0, 4], np.int32)]}


CASES = {
    "gemm_t": lambda: _gemm_case(GEMM, 1, 1),
    "gemm_n": lambda: _gemm_case(GEMM, 0, 2),
    "gemm_big_t": lambda: _gemm_case(GEMM_BIG, 1, 3),
    "gemm_big_n": lambda: _gemm_case(GEMM_BIG, 0, 4),
    "gemm_cpu_t": lambda: _gemm_case(GEMM_CPU_T, 1, 5),
    "gemm_cpu_n": lambda: _gemm_case(GEMM_CPU_N, 0, 6),
    "softmax_L576": lambda: _softmax_case(576, 7),
    "softmax_L40": lambda: _softmax_case(40, 8),
    "layernorm_C1024": lambda: _ln_case(1024, 0, 9),
    "layernorm_C256_gelu": lambda: _ln_case(256, 1, 10),
    "rope": lambda: _rope_case(11),
    "window": lambda: _window_case(12),
    "mha_few_c16": lambda: _mha_case(3, 40, 7, 128, False, False, 13),
    "mha_few_c32": lambda: _mha_case(3, 8, 8, 256, False, False, 14),
    "mha_few_shared_q": lambda: _mha_case(2, 300, 8, 128, False, True, 15),
    "mha_many": lambda: _mha_case(2, 7, 300, 128, False, False, 16),
    "mha_many_shared_kv": lambda: _mha_case(2, 8, 600, 128, True, False, 17),
    "attn_window_cpu": lambda: _attn_case(576, 1024, 16, False, False, 18),
    "attn_window_gpu": lambda: _attn_case(576, 1024, 16, False, True, 18),
    "attn_global_rope_head": lambda: _attn_case(5184, 64, 1, True, False, 19),
    "vit_window_region": lambda: _vit_case(20),
    "softmax_ext_causal": lambda: _softmax_ext_case(40, 1, 40, 2, 0, 2, True, 21),
    "softmax_ext_box": lambda: _softmax_ext_case(7, 10, 12, 4, 1, 2, False, 22),
    "softmax_ext_box_L5184": lambda: _softmax_ext_case(3, 72, 72, 8, 5, 3, False, 23),
    "attend_box_hd32": lambda: _attend_case(21, 144, 8, 32, "box", 24, W=12),
    "attend_causal_hd64": lambda: _attend_case(33, 33, 4, 64, "causal", 25),
    "attend_self_hd32": lambda: _attend_case(200, 200, 8, 32, "plain", 26),
    "convt_plain": lambda: _convt_case(3, 4, 4, 64, False, 0, 27),
    "convt_add_gelu": lambda: _convt_case(2, 5, 7, 32, True, 1, 28),
    "mask_logits": lambda: _logits_case(2, 300, 29),
    "mask_post_dyadic": lambda: _mask_post_case(24, 48, 12, True, 30),
    "mask_post_random": lambda: _mask_post_case(24, 50, 37, False, 31),
}


# ------------------------------------------------------------------ running

def _attention(impl, qkv, N, E, heads, table, gpu):
    """Per-head Q K^T -> softmax_rows -> P V with impl's gemm kernels."""
    if table is not None:
        qkv = impl.rope_apply(qkv, E, 64, N, table)
    out = np.zeros((N, E), np.float32)
    kt, kn = (GEMM_BIG, GEMM_BIG) if gpu else (GEMM_CPU_T, GEMM_CPU_N)
    for h in range(heads):
        S = np.zeros((N, N), np.float32)
        S = impl.gemm(kt, N, N, 64, qkv, h * 64, 3 * E, 0, 0, qkv,
                      E + h * 64, 3 * E, 0, 0, 1, S, 0, N, 0, 0, 1, 1,
                      alpha=0.125)
        S = impl.softmax_rows(S)
        out = impl.gemm(kn, N, 64, N, S, 0, N, 0, 0, qkv, 2 * E + h * 64,
                        3 * E, 0, 0, 0, out, h * 64, E, 0, 0, 1, 1)
    return out, qkv


def run_reference(name, case, impl):
    """Outputs of `case` computed with impl (dict name -> array)."""
    k = case["kind"]
    x = case["inputs"]
    if k == "gemm":
        A, B, C, bias = x
        a = case["args"]
        out = impl.gemm(a["kernel"], a["M"], a["N"], a["K"], A, a["aoff"],
                        a["lda"], a["sa0"], a["sa1"], B, a["boff"], a["ldb"],
                        a["sb0"], a["sb1"], a["transb"], C, a["coff"], a["ldc"],
                        a["sc0"], a["sc1"], a["nb"], a["nb1"], bias=bias,
                        use_r=True, roff=a["roff"], alpha=a["alpha"],
                        act=a["act"])
        return {"C": out}
    if k == "softmax":
        return {"S": impl.softmax_rows(x[0])}
    if k == "layernorm":
        return {"Y": impl.layernorm(x[0], x[1], x[2], 1e-5, case["act"])}
    if k == "rope":
        return {"qkv": impl.rope_apply(x[0], case["E"], 64, case["npos"], x[1])}
    if k == "window":
        H, C, ws = case["H"], case["C"], case["ws"]
        return {"part": impl.window_partition(x[0], H, C, ws),
                "unpart_add": impl.window_unpartition_add(x[0], x[1], H, C, ws)}
    if k == "mha":
        return {"O": impl.mha(case["P"], case["Nq"], case["Nk"], case["dint"],
                              x[0], case["sq"], x[1], case["sk"], x[2],
                              case["sk"])}
    if k == "attn":
        out, _ = _attention(impl, x[0], case["N"], case["E"], case["heads"],
                            x[1] if case["rope"] else None, case["gpu"])
        return {"O": out}
    if k == "vit":
        xx, n1w, n1b, w, b, table = x
        grid, E, ws = case["grid"], case["E"], case["ws"]
        xn = impl.layernorm(xx, n1w, n1b, 1e-5, 0)
        xw = impl.window_partition(xn, grid, E, ws)
        rows = xw.shape[0]
        qkv = np.zeros((rows, 3 * E), np.float32)
        qkv = impl.gemm(GEMM_CPU_T, rows, 3 * E, E, xw, 0, E, 0, 0, w, 0, E, 0,
                        0, 1, qkv, 0, 3 * E, 0, 0, 1, 1, bias=b)
        qkv = impl.rope_apply(qkv, E, 64, ws * ws, table)
        N = ws * ws
        out = np.zeros((rows, E), np.float32)
        for u in range(rows // N):
            o, _ = _attention(impl, qkv[u * N:(u + 1) * N], N, E, E // 64, None,
                              False)
            out[u * N:(u + 1) * N] = o
        return {"qkv": qkv, "O": out}
    if k == "softmax_ext":
        dy, dx = (x[1], x[2]) if len(x) > 1 else (None, None)
        return {"S": impl.softmax_ext(x[0], case["Nq"], case["h0"],
                                      case["causal"], dy, dx, case["W"],
                                      case["nh"])}
    if k == "attend":
        return {"O": _attend(impl, case)}
    if k == "convt":
        add = x[2] if len(x) > 2 else None
        return {"out": impl.convt_scatter(x[0], x[1], add, case["P"], case["H"],
                                          case["W"], case["Co"], case["act"])}
    if k == "logits":
        return {"out": impl.mask_logits(x[0], x[1], case["P"], case["npix"])}
    if k == "mask_post":
        mask, stats = impl.mask_post(x[0], x[1], case["L"], case["out_h"],
                                     case["out_w"], case["offset"])
        return {"mask": mask, "stats": stats}
    raise ValueError(k)


def _gpu_kernel(M, N, K, lda, ldb):
    """The GPU dispatcher's kernel (sam3_model.c:240-255): gemm_big when
    M >= 128, N >= 64 and the rows are 16-byte aligned, else gemm."""
    big = M >= 128 and N >= 64 and K % 4 == 0 and lda % 4 == 0 and ldb % 4 == 0
    return GEMM_BIG if big else GEMM


def _attend(impl, case):
    """attend()'s sequence with impl's kernels, all heads in one chunk:
    Q K^T (alpha 1 / sqrtf(hd)), softmax_ext, P V, each GEMM on the kernel
    the GPU dispatcher picks."""
    Q, K, V = case["inputs"][:3]
    dy, dx = (case["inputs"][3], case["inputs"][4]) if case["mode"] == "box" \
        else (None, None)
    Nq, Nk, H, hd = case["Nq"], case["Nk"], case["heads"], case["hd"]
    D = H * hd
    alpha = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    S = np.zeros(H * Nq * Nk, np.float32)
    S = impl.gemm(_gpu_kernel(Nq, Nk, hd, D, D), Nq, Nk, hd, Q, 0, D, 0, hd, K,
                  0, D, 0, hd, 1, S, 0, Nk, 0, Nq * Nk, H, H, alpha=alpha)
    P = impl.softmax_ext(S.reshape(H * Nq, Nk), Nq, 0, case["mode"] == "causal",
                         dy, dx, case["W"], H)
    O = np.zeros((Nq, D), np.float32)
    return impl.gemm(_gpu_kernel(Nq, hd, Nk, Nk, D), Nq, hd, Nk, P, 0, Nk, 0,
                     Nq * Nk, V, 0, D, 0, hd, 0, O, 0, D, 0, hd, H,
                     H).reshape(Nq, D)


class OracleImpl:
    """The CPU oracle behind refk's API: gemm and gemm_big map to the
    sequential arithmetic, gemm_cpu_t to its own lane order, gemm_cpu_n to
    the sequential arithmetic (what each reference kernel computes)."""

    def __init__(self, orc):
        self.o = orc

    def gemm(self, kernel, M, N, K, A, aoff, lda, sa0, sa1, B, boff, ldb,
             sb0, sb1, transb, C, coff, ldc, sc0, sc1, nb, nb1, bias=None,
             use_r=False, roff=0, alpha=1.0, act=0):
        C = np.ascontiguousarray(C, np.float32).copy()
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        kind = self.o.GEMM_CPU_T if kernel == GEMM_CPU_T else self.o.GEMM_SEQ
        self.o.gemm(kind, M, N, K, A, aoff, lda, sa0, sa1, B, boff, ldb, sb0,
                    sb1, transb, C, coff, ldc, sc0, sc1, nb, nb1,
                    None if bias is None else np.ascontiguousarray(bias, np.float32),
                    C if use_r else None, roff, alpha, act)
        return C

    def softmax_rows(self, S):
        return self.o.softmax_rows(S)

    def softmax_ext(self, S, Nq, h0, causal, dy, dx, W, nh):
        return self.o.softmax_ext(S, Nq, h0, causal, dy, dx, W, nh)

    def layernorm(self, X, g, b, eps=1e-5, act=0):
        return self.o.layernorm(X, g, b, eps, act)

    def rope_apply(self, qkv, E, hd, npos, cs):
        return self.o.rope_apply(qkv, E, hd, npos, cs)

    def window_partition(self, X, H, C, ws):
        return self.o.window_partition(X, H, H, C, ws)

    def window_unpartition_add(self, X, Wd, H, C, ws):
        return self.o.window_unpartition_add(X, Wd, H, H, C, ws)

    def mha(self, P, Nq, Nk, dint, Q, sq, K, sk, V, sv):
        return self.o.mha(P, Nq, Nk, dint, Q, sq, K, sk, V, sv)

    def convt_scatter(self, G, bias, add, P, H, W, Co, act):
        return self.o.convt_scatter(G, bias, add, P, H, W, Co, act)

    def mask_logits(self, U, hyper, P, npix):
        return self.o.mask_logits(U, hyper, P, npix)

    def mask_post(self, lowres, sel, L, out_h, out_w, offset):
        return self.o.mask_post(lowres, sel, L, out_h, out_w, offset)
