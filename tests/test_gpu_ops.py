"""GPU parity of the operators (layernorm, softmax_rows, rope_apply,
window partition, add_bcast, gemm, mha) through the C ABI against the
oracle. Data movement and exact-integer products are bit-exact; float
arithmetic is held to rel-L2 <= 2e-5 (fp32 path) or 2e-2 (bf16 path)."""
import numpy as np
import pytest

from gpu_common import rel_l2, report

pytestmark = pytest.mark.gpu

FP32_TOL = 2e-5
BF16_TOL = 2e-2


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    return sam3_hip


@pytest.fixture(scope="module")
def be(hip):
    b = hip.Backend(precision="fp32")
    yield b
    b.free()


@pytest.fixture(scope="module")
def be16(hip):
    b = hip.Backend(precision="bf16")
    yield b
    b.free()


def model(hip, be, E=128):
    return hip.Model(be, embed=E, heads=E // 64)


def rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("C", [1024, 256, 100, 3000, 3072, 4096, 4608, 64, 32, 128])
def test_layernorm(hip, be, orc, C):
    m = model(hip, be)
    g = rng(C)
    X = (2 * g.standard_normal((37, C)) + 0.5).astype(np.float32)
    w = g.standard_normal(C).astype(np.float32)
    b = g.standard_normal(C).astype(np.float32)
    dX, dW, dB = be.upload(X), be.upload(w), be.upload(b)
    dY = be.alloc(X.nbytes)
    hip.layernorm(m, 37, C, dX, dY, dW, dB, 1e-5, hip.ACT_NONE)
    got = be.read(dY).reshape(37, C)
    assert report("layernorm C=%d" % C, got, orc.layernorm(X, w, b)) <= FP32_TOL
    # In place (Y aliases X), with GELU.
    hip.layernorm(m, 37, C, dX, dX, dW, dB, 1e-5, hip.ACT_GELU)
    got = be.read(dX).reshape(37, C)
    assert rel_l2(got, orc.layernorm(X, w, b, act=orc.ACT_GELU)) <= FP32_TOL


@pytest.mark.parametrize("L", [576, 5184, 40])
def test_softmax_rows(hip, be, orc, L):
    m = model(hip, be)
    S = (3 * rng(L).standard_normal((20, L))).astype(np.float32)
    dS = be.upload(S)
    hip.softmax_rows(m, dS, 20, L)
    got = be.read(dS).reshape(20, L)
    assert report("softmax_rows L=%d" % L, got, orc.softmax_rows(S)) <= FP32_TOL


def test_rope_apply_bit_exact(hip, be, orc):
    E, side = 256, 24
    m = model(hip, be, E)
    table = orc.rope_table(side)
    qkv = rng(0).standard_normal((2 * side * side, 3 * E)).astype(np.float32)
    m.m.qkv = be.upload(qkv)
    hip.rope_apply(m, be.upload(table), qkv.shape[0], side * side)
    got = be.read(m.m.qkv).reshape(qkv.shape)
    np.testing.assert_array_equal(got, orc.rope_apply(qkv, E, 64, side * side,
                                                      table))


@pytest.mark.parametrize("H,ws", [(72, 24), (10, 4)])
def test_window_partition_bit_exact(hip, be, orc, H, ws):
    C = 64
    m = model(hip, be)
    nwx = -(-H // ws)
    X = rng(H).standard_normal((H * H, C)).astype(np.float32)
    dX = be.upload(X)
    dW = be.alloc(nwx * nwx * ws * ws * C * 4)
    hip.window_partition(m, dX, dW, H, C, ws, nwx)
    Xw = be.read(dW).reshape(-1, C)
    np.testing.assert_array_equal(Xw, orc.window_partition(X, H, H, C, ws))
    Y = rng(H + 1).standard_normal((H * H, C)).astype(np.float32)
    dY = be.upload(Y)
    hip.window_unpartition_add(m, dY, dW, H, C, ws, nwx)
    np.testing.assert_array_equal(be.read(dY).reshape(-1, C),
                                  orc.window_unpartition_add(Y, Xw, H, H, C, ws))


def test_add_bcast_bit_exact(hip, be, orc):
    m = model(hip, be)
    a = rng(1).standard_normal(5184 * 3).astype(np.float32)
    b = rng(2).standard_normal(3 * 64).astype(np.float32)
    da, db = be.upload(a), be.upload(b)
    hip.add_bcast(m, da, da, db, a.size, b.size)
    np.testing.assert_array_equal(be.read(da), orc.add_bcast(a, b, b.size))


def _gemm_case(hip, be, orc, M, N, K, transb, nb=4, nb1=2, ints=False,
               act=0, residual=True, seed=0, bias=True):
    """Batched GEMM with padded leading dims and offsets on the GPU and in
    the oracle (sequential arithmetic); returns (gpu, oracle)."""
    m = model(hip, be)
    g = rng(seed)
    draw = (lambda n: g.integers(-3, 4, n).astype(np.float32)) if ints else \
        (lambda n: g.standard_normal(n).astype(np.float32))
    lda, ldc = K + 4, N + 4
    ldb = K + 8 if transb else N + 8
    brows = N if transb else K
    sa1, sb1, sc1 = M * lda, brows * ldb, M * ldc
    A = draw(8 + nb * sa1)
    B = draw(16 + nb * sb1)
    C0 = draw(4 + nb * sc1)
    bv = draw(N) if bias else None
    A_, B_, C_ = (be.upload(A), be.upload(B), be.upload(C0))
    bias_d = be.upload(bv) if bias else None
    hip.gemm(m, M, N, K, hip.bmat(A_, 8, lda, sa1 * nb1, sa1),
             hip.bmat(B_, 16, ldb, sb1 * nb1, sb1), transb,
             hip.bmat(C_, 4, ldc, sc1 * nb1, sc1), nb, nb1, bias_d,
             C_ if residual else None, 4, 0.5, act)
    got = be.read(C_)
    want = C0.copy()
    orc.gemm(orc.GEMM_SEQ, M, N, K, A, 8, lda, sa1 * nb1, sa1, B, 16, ldb,
             sb1 * nb1, sb1, transb, want, 4, ldc, sc1 * nb1, sc1, nb, nb1, bv,
             want if residual else None, 4, 0.5, act)
    return got, want


@pytest.mark.parametrize("transb", [0, 1])
@pytest.mark.parametrize("M,N,K", [(130, 70, 40), (64, 64, 64), (5, 3, 7)])
def test_gemm_exact_integers(hip, be, orc, transb, M, N, K):
    got, want = _gemm_case(hip, be, orc, M, N, K, transb, ints=True, act=2)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("transb", [0, 1])
@pytest.mark.parametrize("act", [0, 1])
def test_gemm_f32(hip, be, orc, transb, act):
    got, want = _gemm_case(hip, be, orc, 200, 150, 300, transb, act=act, seed=3)
    assert report("gemm f32 transb=%d act=%d" % (transb, act), got, want) <= FP32_TOL


@pytest.mark.parametrize("transb", [0, 1])
def test_gemm_bf16(hip, be16, orc, transb):
    got, want = _gemm_case(hip, be16, orc, 200, 150, 300, transb, seed=4)
    assert report("gemm bf16 transb=%d" % transb, got, want) <= BF16_TOL


def to_bf16(x):
    """float32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


def from_bf16(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("M,N,K,act,res,cbf", [
    (5184, 3072, 1024, 0, False, False),   # QKV projection
    (5184, 1024, 1024, 0, True, False),    # attention projection + residual
    (5184, 4096, 1024, 1, False, True),    # MLP fc1, GELU, bf16 hidden
    (5184, 1024, 4096, 0, True, False),    # MLP fc2 + residual
    (5000, 3000, 1024, 0, False, False),   # 256 x 256 tiles, ragged edges
    (5100, 3968, 1024, 1, False, True),    # 192 x 256 tiles, ragged edges
    (2100, 1000, 2048, 2, False, False),   # 192 x 128 tiles, ragged edges
    (2100, 1000, 2048, 1, False, True),    # the same, bf16 C
    (2100, 1000, 2048, 0, True, True),     # 128 x 64 tiles, bf16 C and residual
    (5184, 3072, 2048, 0, True, False),    # residual, long K: 256 x 256 tiles of k_gemm_nt
    (5184, 3072, 2048, 1, True, True),     # the same with GELU and bf16 C
    (3000, 700, 2048, 0, True, False),     # 128 x 64 tiles, residual, ragged
    (2500, 900, 1024, 1, True, False),     # GELU + residual, ragged
    (300, 200, 128, 1, True, False),       # ragged tiles on both sides
    (257, 129, 192, 2, True, True),
    (1, 1, 64, 0, False, False),
])
def test_gemm_nt_bf16(hip, be16, orc, M, N, K, act, res, cbf):
    """bf16 activations x bf16 weight rows (the NT kernel): the oracle's
    linear on the same bf16 values in float, sampled rows at full size."""
    m = model(hip, be16)
    g = rng(M + N + K)
    A = to_bf16(g.standard_normal((M, K), dtype=np.float32))
    W = to_bf16(g.uniform(-0.06, 0.06, (N, K)).astype(np.float32))
    bias = g.standard_normal(N, dtype=np.float32)
    C0 = g.standard_normal((M, N), dtype=np.float32)
    if cbf:
        C0 = from_bf16(to_bf16(C0))
    dA, dW = be16.upload_typed(A, hip.BF16), be16.upload_typed(W, hip.BF16)
    db = be16.upload(bias)
    dC = be16.upload_typed(to_bf16(C0), hip.BF16) if cbf else be16.upload(C0)
    hip.prof_reset()
    be16._b.profile = 1
    hip.linear(m, M, K, N, dA, 0, dW, db, dC, 0, act, int(res))
    be16._b.profile = 0
    assert "gemm_nt_bf16" in [r[0] for r in hip.prof_table()]
    got = be16.read(dC)
    got = (from_bf16(got) if cbf else got).reshape(M, N)
    rows = np.sort(rng(1).choice(M, min(M, 96), replace=False))
    want = orc.linear(from_bf16(A[rows]), from_bf16(W), bias, act=act,
                      cpu=False)
    if res:
        want = want + C0[rows]
    if cbf:
        want = from_bf16(to_bf16(want))
    tol = 1e-2 if cbf else 1e-5
    assert report("gemm_nt bf16 %dx%dx%d act=%d res=%d cbf=%d" %
                  (M, N, K, act, res, cbf), got[rows], want) <= tol


def test_profile_in_flow(hip, be16):
    """profile 2 brackets each launch with events without waiting: the
    results are those of an unprofiled run, and hipb_finish adds each
    launch's time to the per-kernel table (one entry per call)."""
    m = model(hip, be16)
    g = rng(5)
    M, N, K = 512, 384, 256
    A = be16.upload_typed(to_bf16(g.standard_normal((M, K), dtype=np.float32)), hip.BF16)
    W = be16.upload_typed(to_bf16(g.uniform(-0.06, 0.06, (N, K)).astype(np.float32)), hip.BF16)
    b = be16.upload(g.standard_normal(N, dtype=np.float32))
    C = be16.alloc(M * N * 4)
    hip.linear(m, M, K, N, A, 0, W, b, C, 0, 0, 0)
    plain = be16.read(C)
    hip.prof_reset()
    be16._b.profile = 2
    for _ in range(3):
        hip.linear(m, M, K, N, A, 0, W, b, C, 0, 0, 0)
    be16.finish()
    be16._b.profile = 0
    tab = {r[0]: r for r in hip.prof_table()}
    assert np.array_equal(be16.read(C), plain)
    row = tab["gemm_nt_bf16"]
    assert row[4] == 3 and row[1] > 0.0 and row[3] == 3 * 2.0 * M * N * K
    for d in (A, W, b, C):
        be16.release(d)


@pytest.mark.parametrize("M,N,K,act,res,cbf", [
    (5184, 4096, 1024, 1, False, True),    # fc1, GELU, bf16 hidden
    (5184, 1024, 4096, 0, True, False),    # fc2 + residual
])
def test_gemm_nt_every_row(hip, be16, orc, M, N, K, act, res, cbf):
    """The MLP's NT GEMMs at full size: every row against the oracle, and
    a second launch gives the same bits."""
    m = model(hip, be16)
    g = rng(M + 2 * N + K)
    A = to_bf16(g.standard_normal((M, K), dtype=np.float32))
    W = to_bf16(g.uniform(-0.06, 0.06, (N, K)).astype(np.float32))
    bias = g.standard_normal(N, dtype=np.float32)
    C0 = g.standard_normal((M, N), dtype=np.float32)
    if cbf:
        C0 = from_bf16(to_bf16(C0))
    dA, dW = be16.upload_typed(A, hip.BF16), be16.upload_typed(W, hip.BF16)
    db = be16.upload(bias)

    def run():
        dC = be16.upload_typed(to_bf16(C0), hip.BF16) if cbf else be16.upload(C0)
        hip.linear(m, M, K, N, dA, 0, dW, db, dC, 0, act, int(res))
        got = be16.read(dC)
        be16.release(dC)
        return (from_bf16(got) if cbf else got).reshape(M, N)

    print("gemm_nt every row %dx%dx%d" % (M, N, K), flush=True)
    first, second = run(), run()
    assert np.array_equal(first, second)
    want = orc.linear(from_bf16(A), from_bf16(W), bias, act=act, cpu=False)
    if res:
        want = want + C0
    if cbf:
        want = from_bf16(to_bf16(want))
    tol = 1e-2 if cbf else 1e-5
    assert report("gemm_nt every row %dx%dx%d" % (M, N, K), first, want) <= tol


def test_linear_fp16_weights(hip, orc):
    be = hip.Backend(precision="fp16")
    try:
        m = model(hip, be)
        g = rng(5)
        X = g.standard_normal((77, 96)).astype(np.float32)
        W = g.standard_normal((48, 96)).astype(np.float32)
        b = g.standard_normal(48).astype(np.float32)
        dW = be.upload_weight(W)
        assert dW.contents.dtype == hip.F16
        dX, db = be.upload(X), be.upload(b)
        dY = be.alloc(77 * 48 * 4)
        hip.linear(m, 77, 96, 48, dX, 0, dW, db, dY, 0, hip.ACT_RELU, 0)
        Wh = W.astype(np.float16).astype(np.float32)
        want = orc.linear(X, Wh, b, act=orc.ACT_RELU, cpu=False)
        assert report("linear fp16 weights", be.read(dY).reshape(77, 48),
                      want) <= FP32_TOL
    finally:
        be.free()


def test_gemm_operand_out_of_bounds_is_fatal(hip, be):
    m = model(hip, be)
    A = be.alloc(10 * 10 * 4)
    with pytest.raises(hip.Sam3HipError, match="operand A reaches element"):
        hip.gemm(m, 11, 10, 10, hip.mat(A, 0, 10), hip.mat(A, 0, 10), 1,
                 hip.mat(A, 0, 10), 1, 1)


# ---------------------------------------------------------------- decoder

def _dec(seed, P, Nq, Nk, dint, shared_k=False, shared_q=False):
    g = rng(seed)
    q = g.standard_normal(((1 if shared_q else P) * Nq, dint)).astype(np.float32)
    k = g.standard_normal(((1 if shared_k else P) * Nk, dint)).astype(np.float32)
    v = g.standard_normal(((1 if shared_k else P) * Nk, dint)).astype(np.float32)
    return (q, 0 if shared_q else Nq * dint, k, 0 if shared_k else Nk * dint,
            v, 0 if shared_k else Nk * dint)


@pytest.mark.parametrize("P,Nq,Nk,dint,shk,shq", [
    (64, 7, 4096, 128, False, False),    # token -> image, per-prompt keys
    (64, 8, 5184, 128, True, False),     # token -> image, shared keys
    (3, 9, 300, 128, False, False),      # more than 8 queries, short keys
    (64, 4096, 7, 128, False, False),    # image -> token, per-prompt queries
    (16, 5184, 8, 128, False, True),     # image -> token, shared queries
    (64, 8, 8, 256, False, False),       # token self-attention, c = 32
    (8, 2048, 65, 128, False, False),    # many keys, key range not split
    (2, 3, 261, 128, False, False),      # many keys, ragged last step
    (3, 20, 40, 128, False, False),      # 9..64 keys, generic few-keys
    (5, 17, 1, 128, False, False),       # one key: O = V
])
def test_mha(hip, be, orc, P, Nq, Nk, dint, shk, shq):
    m = model(hip, be)
    q, sq, k, sk, v, sv = _dec(P + Nq + Nk, P, Nq, Nk, dint, shk, shq)
    dq, dk, dv = be.upload(q), be.upload(k), be.upload(v)
    do = be.alloc(P * Nq * dint * 4)
    hip.mha(m, P, Nq, Nk, dint, dq, sq, dk, sk, dv, sv, do)
    got = be.read(do).reshape(P * Nq, dint)
    want = orc.mha(P, Nq, Nk, dint, q, sq, k, sk, v, sv)
    assert report("mha P=%d Nq=%d Nk=%d dint=%d" % (P, Nq, Nk, dint), got,
                  want) <= FP32_TOL
    for d in (dq, dk, dv, do):
        be.release(d)


def test_mha_unaligned_prompt_strides(hip, be, orc):
    """Per-prompt strides that are not a multiple of 4 floats take the
    generic few-keys kernel; with many keys they are a fatal error."""
    m = model(hip, be)
    P, Nq, Nk, dint = 3, 11, 7, 128
    g = rng(5)
    sq, sk = Nq * dint + 2, Nk * dint + 1
    q = g.standard_normal(P * sq).astype(np.float32)
    k = g.standard_normal(P * sk).astype(np.float32)
    v = g.standard_normal(P * sk).astype(np.float32)
    dq, dk, dv = be.upload(q), be.upload(k), be.upload(v)
    do = be.alloc(P * Nq * dint * 4)
    hip.mha(m, P, Nq, Nk, dint, dq, sq, dk, sk, dv, sk, do)
    got = be.read(do).reshape(P * Nq, dint)
    want = orc.mha(P, Nq, Nk, dint, q, sq, k, sk, v, sk)
    assert report("mha unaligned strides", got, want) <= FP32_TOL
    d = be.alloc(P * 100 * dint * 4 + 64)
    with pytest.raises(hip.Sam3HipError, match="multiples of 4"):
        hip.mha(m, P, 4, 100, dint, d, 0, d, 100 * dint + 2, d, 0, d)
    for x in (dq, dk, dv, do, d):
        be.release(x)


def test_mha_rejects_wide_heads_with_many_keys(hip, be):
    m = model(hip, be)
    d = be.alloc(100 * 256 * 4)
    with pytest.raises(hip.Sam3HipError, match="mha: unsupported shape"):
        hip.mha(m, 1, 4, 100, 256, d, 0, d, 0, d, 0, d)
