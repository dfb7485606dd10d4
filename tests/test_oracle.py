"""Pins the CPU oracle (oracle/sam3_oracle.c) without the reference running.

Each check is chosen so that a plausible restatement mistake (transposed
operand, wrong batch stride, dropped epilogue term, wrong reduction
order, sign error in a rotation, wrong window index) fails at least one
of them: exact small-integer products, float64 textbook versions
(tests/ref64.py), closed forms and invariances. The tests marked
"teeth" plant such a mistake in the oracle's inputs and show the check
catches it.
"""
import math

import numpy as np
import pytest

import ref64


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- GEMM

def _gemm_case(orc, kind, transb, seed=0, M=37, N=45, K=40, nb=6, nb1=3,
               alpha=0.5, use_bias=True, use_r=True, act=0, ints=True):
    """Batched GEMM with offsets, padded leading dims and split batch
    strides; returns (oracle result, exact float64 result)."""
    g = rng(seed)
    lda, ldb, ldc = K + 3, (K + 5) if transb else (N + 5), N + 7
    aoff, boff, coff = 11, 7, 5
    b0n, b1n = nb // nb1, nb1
    sa0, sa1 = (M * lda) * b1n, M * lda
    sb_rows = N if transb else K
    sb0, sb1 = sb_rows * ldb * b1n, sb_rows * ldb
    sc0, sc1 = M * ldc * b1n, M * ldc
    draw = (lambda n: g.integers(-3, 4, n).astype(np.float32)) if ints else \
        (lambda n: g.standard_normal(n).astype(np.float32))
    A = draw(aoff + nb * M * lda + 16)
    B = draw(boff + nb * sb_rows * ldb + 16)
    C0 = draw(coff + nb * M * ldc + 16)
    bias = draw(N) if use_bias else None
    C = C0.copy()
    orc.gemm(kind, M, N, K, A, aoff, lda, sa0, sa1, B, boff, ldb, sb0, sb1,
             transb, C, coff, ldc, sc0, sc1, nb, nb1, bias,
             C if use_r else None, coff, alpha, act)
    want = C0.astype(np.float64).copy()
    for b in range(nb):
        q0, q1 = divmod(b, nb1)
        a = A[aoff + q0 * sa0 + q1 * sa1:][:M * lda].reshape(M, lda)[:, :K]
        bb = B[boff + q0 * sb0 + q1 * sb1:][:sb_rows * ldb].reshape(sb_rows, ldb)
        bm = bb[:, :K].T if transb else bb[:, :N]
        base = coff + q0 * sc0 + q1 * sc1
        cv = want[base:base + M * ldc].reshape(M, ldc)
        r = alpha * (a.astype(np.float64) @ bm.astype(np.float64))
        if use_bias:
            r = r + bias
        if act == 1:
            r = ref64.gelu(r)
        elif act == 2:
            r = np.maximum(r, 0)
        if use_r:
            r = r + cv[:, :N]
        cv[:, :N] = r
    return C, want


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("transb", [0, 1])
@pytest.mark.parametrize("act", [0, 2])
def test_gemm_exact_integers(orc, kind, transb, act):
    # Small integers: every product and partial sum is exact in fp32, so
    # any summation order must give the exact result bit for bit.
    C, want = _gemm_case(orc, kind, transb, act=act)
    np.testing.assert_array_equal(C, want.astype(np.float32))


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("transb", [0, 1])
@pytest.mark.parametrize("M,N,K", [(37, 45, 100), (64, 64, 64), (3, 2, 9)])
def test_gemm_float64(orc, kind, transb, M, N, K):
    C, want = _gemm_case(orc, kind, transb, seed=1, M=M, N=N, K=K, ints=False,
                         alpha=0.125)
    assert ref64.rel_l2(C, want) < 2e-6


def test_gemm_gelu_epilogue(orc):
    C, want = _gemm_case(orc, 1, 1, seed=2, ints=False, act=1, use_r=False)
    assert ref64.rel_l2(C, want) < 2e-6


def test_gemm_cpu_t_lane_order(orc):
    # gemm_cpu_t sums k in eight lanes (k mod 8), adds lanes q and q+4,
    # then the four pair sums. With B row = [2^24, 1 x7, -2^24, 0 x7] and
    # A = ones, a sequential chain absorbs the seven ones into 2^24 and
    # returns 0; the lane split returns the exact 7.
    K = 16
    A = np.ones((2, K), np.float32)
    brow = np.array([2.0 ** 24] + [1.0] * 7 + [-2.0 ** 24] + [0.0] * 7, np.float32)
    B = np.tile(brow, (4, 1))
    out = {}
    for kind in (0, 1):
        C = np.zeros((2, 4), np.float32)
        orc.gemm(kind, 2, 4, K, A, 0, K, 0, 0, B, 0, K, 0, 0, 1, C, 0, 4, 0, 0,
                 1, 1)
        out[kind] = C
    assert np.all(out[0] == 0.0)
    assert np.all(out[1] == 7.0)
    # A partial 2 x 4 block (M = 1) skips the lanes: sequential again.
    C = np.zeros((1, 4), np.float32)
    orc.gemm(1, 1, 4, K, A, 0, K, 0, 0, B, 0, K, 0, 0, 1, C, 0, 4, 0, 0, 1, 1)
    assert np.all(C == 0.0)


def test_gemm_dispatch_kernel_choice(orc):
    # profile=cpu with transb picks gemm_cpu_t (sam3_model.c:249-253).
    K = 16
    A = np.ones((2, K), np.float32)
    brow = np.array([2.0 ** 24] + [1.0] * 7 + [-2.0 ** 24] + [0.0] * 7, np.float32)
    B = np.tile(brow, (4, 1))
    for cpu, want in ((1, 7.0), (0, 0.0)):
        C = np.zeros((2, 4), np.float32)
        orc.gemm(0, 2, 4, K, A, 0, K, 0, 0, B, 0, K, 0, 0, 1, C, 0, 4, 0, 0,
                 1, 1, dispatch_cpu=cpu)
        assert np.all(C == want)


@pytest.mark.parametrize("mistake", ["transb", "stride"])
def test_gemm_teeth(orc, mistake):
    """Planted mistake: the exact-integer check rejects a transposed B or
    swapped batch strides."""
    g = rng(3)
    M = N = K = 8
    A = g.integers(-3, 4, (2, M, K)).astype(np.float32)
    B = g.integers(-3, 4, (2, N, K)).astype(np.float32)
    C = np.zeros((2, M, N), np.float32)
    transb = 0 if mistake == "transb" else 1
    sb0 = 0 if mistake == "stride" else N * K
    orc.gemm(0, M, N, K, A, 0, K, M * K, 0, B, 0, K, sb0, 0, transb, C, 0, N,
             M * N, 0, 2, 1)
    want = np.einsum("bmk,bnk->bmn", A.astype(np.float64), B.astype(np.float64))
    assert not np.array_equal(C, want.astype(np.float32))


# ---------------------------------------------------------------- softmax / LN

@pytest.mark.parametrize("L", [576, 40, 257, 64])
def test_softmax_rows(orc, L):
    g = rng(L)
    S = (3 * g.standard_normal((33, L))).astype(np.float32)
    P = orc.softmax_rows(S)
    assert ref64.rel_l2(P, ref64.softmax(S)) < 1e-6
    assert np.allclose(P.astype(np.float64).sum(-1), 1.0, atol=2e-6)
    # Shift invariance.
    P2 = orc.softmax_rows(S + np.float32(5.0))
    assert ref64.rel_l2(P2, P) < 2e-6


# ------------------------------------------------ text-path attention


@pytest.mark.parametrize("L", [40, 576])
def test_softmax_ext_without_terms_is_softmax_rows(orc, L):
    S = (3 * rng(L + 1).standard_normal((18, L))).astype(np.float32)
    assert np.array_equal(orc.softmax_ext(S, 6, h0=2), orc.softmax_rows(S))


def test_softmax_ext_causal(orc):
    Nq = L = 50
    S = (3 * rng(3).standard_normal((2 * Nq, L))).astype(np.float32)
    P = orc.softmax_ext(S, Nq, causal=True)
    mask = np.arange(L)[None, :] > np.arange(Nq)[:, None]
    want = np.concatenate([ref64.softmax(np.where(mask, -np.inf, S[h * Nq:(h + 1) * Nq]))
                           for h in range(2)])
    assert ref64.rel_l2(P, want) < 1e-6
    assert np.all(P.reshape(2, Nq, L)[:, mask] == 0.0)
    assert np.all(P[::Nq, 0] == 1.0)            # query 0 sees key 0 only


def _box_terms(seed, Nq, H, W, nh):
    g = rng(seed)
    dy = g.standard_normal((Nq, H, nh)).astype(np.float32)
    dx = g.standard_normal((Nq, W, nh)).astype(np.float32)
    return dy, dx


@pytest.mark.parametrize("Nq,H,W,nh,h0", [(7, 5, 7, 4, 1), (3, 72, 72, 8, 5)])
def test_softmax_ext_box_bias(orc, Nq, H, W, nh, h0):
    """Against softmax of the scores plus the bias built by broadcasting
    (H != W catches a swapped row / column index); heads from h0 pick
    their own bias columns."""
    L, hc = H * W, 2
    S = (2 * rng(Nq + L).standard_normal((hc * Nq, L))).astype(np.float32)
    dy, dx = _box_terms(Nq, Nq, H, W, nh)
    P = orc.softmax_ext(S, Nq, h0=h0, dy=dy, dx=dx, W=W, nh=nh)
    bias = ref64.box_bias(dy, dx)
    want = np.concatenate([ref64.softmax(S[k * Nq:(k + 1) * Nq] + bias[:, :, h0 + k])
                           for k in range(hc)])
    assert ref64.rel_l2(P, want) < 1e-6
    if H != W:
        # Teeth: the bias with the key index read x major (j = x H + y)
        # is a different function, which the check above would reject.
        bad = (dx.astype(np.float64)[:, :, None, :] +
               dy.astype(np.float64)[:, None, :, :]).reshape(Nq, L, nh)
        wrong = np.concatenate([ref64.softmax(S[k * Nq:(k + 1) * Nq] + bad[:, :, h0 + k])
                                for k in range(hc)])
        assert ref64.rel_l2(P, wrong) > 1e-2
    # A constant added to one query's dy row shifts its scores uniformly.
    dy2 = dy.copy()
    dy2[1] += np.float32(3.0)
    P2 = orc.softmax_ext(S, Nq, h0=h0, dy=dy2, dx=dx, W=W, nh=nh)
    assert ref64.rel_l2(P2, P) < 2e-6


@pytest.mark.parametrize("cpu", [False, True])
@pytest.mark.parametrize("case", ["bias_hd32", "causal_hd64", "plain_hd32"])
def test_attend_vs_float64(orc, cpu, case):
    g = rng(len(case))
    if case == "bias_hd32":
        Nq, heads, hd, H, W = 21, 8, 32, 5, 7
        Nk = H * W
    elif case == "causal_hd64":
        Nq, Nk, heads, hd = 33, 33, 4, 64
    else:
        Nq, Nk, heads, hd = 60, 60, 8, 32
    D = heads * hd
    Q = g.standard_normal((Nq, D + 8)).astype(np.float32)
    K = g.standard_normal((Nk, D)).astype(np.float32)
    V = g.standard_normal((Nk, D + 4)).astype(np.float32)
    kw = {}
    bias = None
    if case == "bias_hd32":
        dy, dx = _box_terms(5, Nq, H, W, heads)
        kw = dict(dy=dy, dx=dx, W=W)
        bias = ref64.box_bias(dy, dx)
    O = orc.attend(Q, K, V, heads, hd, causal=case == "causal_hd64", cpu=cpu, **kw)
    want = ref64.attend(Q[:, :D], K, V[:, :D], heads, hd,
                        causal=case == "causal_hd64", bias=bias)
    assert ref64.rel_l2(O, want) < 1e-5


def test_attend_head_chunks_and_causal_first_row(orc):
    """One head per score chunk gives the same bits as all heads at once
    (the chunk offset reaches the bias and the operand columns); with the
    causal mask query 0's output is V's row 0 exactly."""
    g = rng(9)
    Nq, heads, hd, H, W = 12, 4, 32, 3, 4
    Nk, D = H * W, heads * hd
    Q, K, V = (g.standard_normal((n, D)).astype(np.float32) for n in (Nq, Nk, Nk))
    dy, dx = _box_terms(10, Nq, H, W, heads)
    a = orc.attend(Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
    b = orc.attend(Q, K, V, heads, hd, dy=dy, dx=dx, W=W, score_cap=Nq * Nk)
    assert np.array_equal(a, b)
    Kc, Vc = Q.copy(), g.standard_normal((Nq, D)).astype(np.float32)
    O = orc.attend(Q, Kc, Vc, heads, hd, causal=True)
    assert np.array_equal(O[0], Vc[0])
    with pytest.raises(ValueError):
        orc.attend(Q, K, V, heads, hd, score_cap=Nq * Nk - 1)


@pytest.mark.parametrize("C", [1024, 256, 100])
def test_layernorm(orc, C):
    g = rng(C)
    X = (2 * g.standard_normal((19, C)) + 1.5).astype(np.float32)
    w = g.standard_normal(C).astype(np.float32)
    b = g.standard_normal(C).astype(np.float32)
    Y = orc.layernorm(X, w, b)
    assert ref64.rel_l2(Y, ref64.layernorm(X, w, b)) < 2e-6
    # Without affine terms every row has zero mean and unit variance.
    Y1 = orc.layernorm(X, np.ones(C), np.zeros(C)).astype(np.float64)
    assert np.allclose(Y1.mean(-1), 0, atol=1e-5)
    assert np.allclose(Y1.var(-1), 1, atol=1e-4)


# ---------------------------------------------------------------- RoPE

def _qkv(seed, rows, E):
    return rng(seed).standard_normal((rows, 3 * E)).astype(np.float32)


def test_rope_identity_table_is_noop(orc):
    E, hd, npos = 128, 64, 16
    qkv = _qkv(0, 32, E)
    cs = np.zeros((npos, hd // 2, 2), np.float32)
    cs[..., 0] = 1.0
    np.testing.assert_array_equal(orc.rope_apply(qkv, E, hd, npos, cs), qkv)


def test_rope_matches_complex_rotation(orc):
    E, hd, side = 128, 64, 6
    cs = orc.rope_table(side, hd)
    qkv = _qkv(1, 2 * side * side, E)          # rows wrap: r % npos
    out = orc.rope_apply(qkv, E, hd, side * side, cs)
    assert ref64.rel_l2(out, ref64.rope(qkv, E, hd, side * side, cs)) < 1e-6
    # v third untouched, pair norms preserved.
    np.testing.assert_array_equal(out[:, 2 * E:], qkv[:, 2 * E:])
    n0 = (qkv[:, :2 * E].reshape(-1, 2).astype(np.float64) ** 2).sum(-1)
    n1 = (out[:, :2 * E].reshape(-1, 2).astype(np.float64) ** 2).sum(-1)
    assert np.allclose(n0, n1, rtol=1e-5)


def test_rope_relative_position(orc):
    # With the axial table, q at (x1, y1) . k at (x2, y2) depends only on
    # (x1 - x2, y1 - y2): shifting both positions keeps every dot product.
    E, hd, side = 64, 64, 8
    cs = orc.rope_table(side, hd)
    g = rng(2)
    q = g.standard_normal(hd).astype(np.float32)
    k = g.standard_normal(hd).astype(np.float32)

    def at(pos):
        row = np.zeros((side * side, 3 * E), np.float32)
        row[pos, :hd] = q
        row[pos, E:E + hd] = k
        r = orc.rope_apply(row, E, hd, side * side, cs)[pos]
        return r[:hd].astype(np.float64), r[E:E + hd].astype(np.float64)

    def dot(p1, p2):
        return at(p1)[0] @ at(p2)[1]

    for (x1, y1, x2, y2, dx, dy) in [(1, 2, 4, 0, 2, 3), (0, 0, 5, 5, 1, 1)]:
        d0 = dot(y1 * side + x1, y2 * side + x2)
        d1 = dot((y1 + dy) * side + x1 + dx, (y2 + dy) * side + x2 + dx)
        assert abs(d0 - d1) < 1e-4 * (1 + abs(d0))


def test_rope_teeth(orc):
    """Planted mistake: a table with the sine negated fails the complex
    rotation check."""
    E, hd, side = 64, 64, 4
    cs = orc.rope_table(side, hd)
    bad = cs.copy()
    bad[..., 1] *= -1
    qkv = _qkv(3, side * side, E)
    out = orc.rope_apply(qkv, E, hd, side * side, bad)
    assert ref64.rel_l2(out, ref64.rope(qkv, E, hd, side * side, cs)) > 1e-2


# ---------------------------------------------------------------- windows

@pytest.mark.parametrize("H,ws", [(72 // 3, 8), (10, 4), (12, 12)])
def test_window_partition(orc, H, ws):
    C = 5
    X = rng(H).standard_normal((H * H, C)).astype(np.float32)
    Xw = orc.window_partition(X, H, H, C, ws)
    np.testing.assert_array_equal(Xw, ref64.window_partition(X, H, H, ws))
    back = orc.window_unpartition_add(np.zeros_like(X), Xw, H, H, C, ws)
    np.testing.assert_array_equal(back, X)
    # Residual add: X + unpartition(partition(Y)) == X + Y.
    Y = rng(H + 1).standard_normal((H * H, C)).astype(np.float32)
    out = orc.window_unpartition_add(X, orc.window_partition(Y, H, H, C, ws),
                                     H, H, C, ws)
    np.testing.assert_array_equal(out, X + Y)


def test_add_bcast(orc):
    a = rng(0).standard_normal(60).astype(np.float32)
    b = rng(1).standard_normal(12).astype(np.float32)
    np.testing.assert_array_equal(orc.add_bcast(a, b, 12), a + np.tile(b, 5))


# ---------------------------------------------------------------- decoder attention

def _dec_inputs(seed, P, Nq, Nk, dint, shared_k=False, shared_q=False):
    g = rng(seed)
    q = g.standard_normal(((1 if shared_q else P) * Nq, dint)).astype(np.float32)
    k = g.standard_normal(((1 if shared_k else P) * Nk, dint)).astype(np.float32)
    v = g.standard_normal(((1 if shared_k else P) * Nk, dint)).astype(np.float32)
    sq = 0 if shared_q else Nq * dint
    sk = 0 if shared_k else Nk * dint
    return q, sq, k, sk, v, sk


@pytest.mark.parametrize("P,Nq,Nk,dint,shk,shq", [
    (3, 7, 300, 128, False, False),     # token -> image, per-prompt keys
    (2, 8, 600, 128, True, False),      # token -> image, shared keys
    (2, 40, 7, 128, False, True),       # image -> token, shared queries
    (3, 8, 8, 256, False, False),       # token self-attention, c = 32
])
def test_mha_vs_float64(orc, P, Nq, Nk, dint, shk, shq):
    q, sq, k, sk, v, sv = _dec_inputs(P + Nq, P, Nq, Nk, dint, shk, shq)
    out = orc.mha(P, Nq, Nk, dint, q, sq, k, sk, v, sv)
    want = ref64.mha(P, Nq, Nk, dint, q, sq, k, sk, v, sv)
    assert ref64.rel_l2(out, want) < 2e-6


@pytest.mark.parametrize("Nk", [1, 300])
def test_attn_closed_forms(orc, Nk):
    P, Nq, dint, c = 2, 3, 128, 16
    q, sq, k, sk, v, sv = _dec_inputs(5, P, Nq, Nk, dint)
    fn = orc.attn_manykeys if Nk > 64 else orc.attn_fewkeys
    if Nk == 1:
        # One key: the output is that key's value row, exactly.
        out = fn(q, sq, k, sk, v, sv, P, Nq, Nk, dint, c, 0.25)
        np.testing.assert_array_equal(out.reshape(P, Nq, dint),
                                      np.repeat(v.reshape(P, 1, dint), Nq, 1))
        out = orc.attn_manykeys(q, sq, k, sk, v, sv, P, Nq, Nk, dint, c, 0.25)
        np.testing.assert_array_equal(out.reshape(P, Nq, dint),
                                      np.repeat(v.reshape(P, 1, dint), Nq, 1))
    else:
        # Zero queries: uniform weights, output = mean of the value rows.
        out = fn(np.zeros_like(q), sq, k, sk, v, sv, P, Nq, Nk, dint, c, 0.25)
        mean = v.reshape(P, Nk, dint).astype(np.float64).mean(1)
        assert np.allclose(out.reshape(P, Nq, dint), mean[:, None, :], atol=2e-6)
        # Permuting keys and values together changes nothing.
        perm = rng(9).permutation(Nk)
        kp = k.reshape(P, Nk, dint)[:, perm].reshape(P * Nk, dint)
        vp = v.reshape(P, Nk, dint)[:, perm].reshape(P * Nk, dint)
        o1 = fn(q, sq, k, sk, v, sv, P, Nq, Nk, dint, c, 0.25)
        o2 = fn(q, sq, kp, sk, vp, sv, P, Nq, Nk, dint, c, 0.25)
        assert ref64.rel_l2(o2, o1) < 2e-6


def test_mha_rejects_wide_heads_with_many_keys(orc):
    q, sq, k, sk, v, sv = _dec_inputs(0, 1, 4, 100, 256)
    with pytest.raises(ValueError):
        orc.mha(1, 4, 100, 256, q, sq, k, sk, v, sv)


# ---------------------------------------------------------------- ViT attention region

def _vit_inputs(seed, grid, E):
    g = rng(seed)
    x = g.standard_normal((grid * grid, E)).astype(np.float32)
    n1w = (1 + 0.1 * g.standard_normal(E)).astype(np.float32)
    n1b = (0.1 * g.standard_normal(E)).astype(np.float32)
    bound = math.sqrt(6.0 / (E + 3 * E))
    qkvw = g.uniform(-bound, bound, (3 * E, E)).astype(np.float32)
    qkvb = g.uniform(-1 / math.sqrt(E), 1 / math.sqrt(E), 3 * E).astype(np.float32)
    return x, n1w, n1b, qkvw, qkvb


@pytest.mark.parametrize("ws", [0, 4, 3])
@pytest.mark.parametrize("cpu", [1, 0])
def test_vit_attention_vs_float64(orc, ws, cpu):
    grid, E, heads, hd = 8, 128, 2, 64
    x, n1w, n1b, qkvw, qkvb = _vit_inputs(ws, grid, E)
    s = ws if ws else grid
    cs = orc.rope_table(s, hd)
    attn, qkv = orc.vit_attention(x, grid, E, heads, hd, ws, n1w, n1b, qkvw,
                                  qkvb, cs, cpu=cpu, want_qkv=True)
    want, qkv64 = ref64.vit_attention(x, grid, E, heads, hd, ws, n1w, n1b,
                                      qkvw, qkvb, cs)
    assert ref64.rel_l2(qkv, qkv64) < 2e-6
    assert ref64.rel_l2(attn, want) < 5e-6


def test_vit_attention_structure(orc):
    grid, E, heads, hd = 6, 128, 2, 64
    x, n1w, n1b, qkvw, qkvb = _vit_inputs(7, grid, E)
    cs = orc.rope_table(grid, hd)
    glob = orc.vit_attention(x, grid, E, heads, hd, 0, n1w, n1b, qkvw, qkvb, cs)
    # One window covering the grid is global attention, bit for bit.
    win = orc.vit_attention(x, grid, E, heads, hd, grid, n1w, n1b, qkvw, qkvb, cs)
    np.testing.assert_array_equal(win, glob)
    # Head chunking (one head per chunk) only changes the memory schedule.
    chunked = orc.vit_attention(x, grid, E, heads, hd, 0, n1w, n1b, qkvw, qkvb,
                                cs, score_cap=(grid * grid) ** 2)
    np.testing.assert_array_equal(chunked, glob)
    with pytest.raises(ValueError):
        orc.vit_attention(x, grid, E, heads, hd, 0, n1w, n1b, qkvw, qkvb, cs,
                          score_cap=10)


# ---------------------------------------------------------------- backbone

def test_patch_im2col(orc):
    g = rng(41)
    grid, ps = 5, 3
    img = g.standard_normal((3, grid * ps, grid * ps)).astype(np.float32)
    got = orc.patch_im2col(img, grid * ps, grid, ps)
    np.testing.assert_array_equal(got, ref64.patch_im2col(img, grid, ps))


@pytest.mark.parametrize("ws", [0, 4])
@pytest.mark.parametrize("cpu", [1, 0])
def test_vit_block_vs_float64(orc, ws, cpu):
    import backbone_case as bc
    grid, E, heads, hd, mlp = 8, 128, 2, 64, 256
    g = rng(50 + ws)
    w = bc.block_weights(g, E, mlp, ws)
    x = g.standard_normal((grid * grid, E)).astype(np.float32)
    cs = orc.rope_table(ws if ws else grid, hd)
    got = orc.vit_block(x, grid, E, heads, hd, mlp, w, cs, cpu=cpu)
    want = ref64.vit_block(x, grid, E, heads, hd, mlp, w, cs)
    assert ref64.rel_l2(got, want) < 5e-6


def test_vit_block_teeth(orc):
    """A block whose residual skips the MLP input normalisation (norm2
    weights swapped for norm1's) is caught by the float64 check."""
    import backbone_case as bc
    grid, E, heads, hd, mlp = 6, 128, 2, 64, 256
    g = rng(57)
    w = bc.block_weights(g, E, mlp, 0)
    x = g.standard_normal((grid * grid, E)).astype(np.float32)
    cs = orc.rope_table(grid, hd)
    bad = dict(w, n2w=w["n1w"], n2b=w["n1b"])
    got = orc.vit_block(x, grid, E, heads, hd, mlp, bad, cs)
    assert ref64.rel_l2(got, ref64.vit_block(x, grid, E, heads, hd, mlp, w, cs)) > 1e-3


def test_encode_trunk_vs_float64(orc):
    import backbone_case as bc
    grid, ps, E, heads, hd, mlp = 8, 4, 128, 2, 64, 256
    img, pe_w, pos, lnpw, lnpb, blocks = bc.trunk_case(60, grid, ps, E, mlp,
                                                       [4, 0, 4])
    rw, rg = orc.rope_table(4, hd), orc.rope_table(grid, hd)
    got = orc.encode_trunk(img, grid, ps, E, heads, hd, mlp, pe_w, pos, lnpw,
                           lnpb, blocks, rw, rg)
    want = ref64.encode_trunk(img, grid, ps, E, heads, hd, mlp, pe_w, pos,
                              lnpw, lnpb, blocks, rw, rg)
    assert ref64.rel_l2(got, want) < 2e-5
