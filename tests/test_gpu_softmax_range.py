"""Online softmax at any score magnitude.

The reference's softmax_rows (sam3_kernels.cl:637-656), softmax_ext
(:885-921) and attn_manykeys merge (:604-633) subtract each row's exact
maximum, so they are exact whatever the size of the scores. The fused
kernels here keep a lazy reference point instead: k_attn_bf16 moves it
only when a score could leave a +-64 (log2 units) span, k_attn_f32 sets
it to its first key block's maximum and then moves it the same way,
k_mha_many16 and k_t2i_fused when a score passes it by 8. These tests drive scores far past
those spans so that every branch of the moves runs:

- rows whose first block already exceeds +64 (move up, nothing to
  rescale) and rows whose every score lies below -64 (move down while the
  row has no weight);
- later blocks whose maximum jumps by more than 64 (rescale of O and l),
  in the same waves as rows whose block maximum falls far below their
  reference point (which must stay put);
- key splits (merge of partials whose reference points differ), the box
  bias, the causal mask and head width 32.

Inputs. Channel `ca` of a head carries a block-periodic key component
8 + A[block % 6] and channel `cb` 8 + B[block % 6]; query rows carry 0,
+60 or -90 on `ca` or +60 on `cb` (by row % 4, in two waves of three;
the third is all plain). The other channels are integers in [-2, 2], so
every score q . k is an integer and exact in fp32.

Oracles. fp32 path: the oracle (the reference's op sequence, bar 2e-5).
bf16 path: exact float64 softmax attention of the operands the device
packed (bf16 Q in log2 units, K, V^T: read back; the box bias in float32
as the device forms it), bar 1e-2
(the kernel rounds the weights P to bf16 for the P V product). Against the
fp32 oracle the bf16 path has no fixed bar here: a score of 300 log2
units carries about 1 unit of bf16 input rounding. Each test also checks
that its construction reaches the branches it is named for.
"""
import math

import numpy as np
import pytest

from gpu_common import report

pytestmark = pytest.mark.gpu

FP32_TOL = 2e-5
PACKED_TOL = 1e-2
LOG2E = 1.4426950408889634
A = (0, 16, 24, 0, 8, 0)
B = (0, 0, 0, 24, 0, 16)


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    return sam3_hip


@pytest.fixture(scope="module", params=["fp32", "bf16"])
def be(hip, request):
    b = hip.Backend(precision=request.param)
    b.precision = request.param
    yield b
    b.free()


def pad64(n):
    return (n + 63) // 64 * 64


def ranged_heads(g, rows_q, rows_k, heads, hd, up=60.0, down=-90.0):
    """Q [rows_q, heads hd], K, V [rows_k, heads hd] as described above
    (query components `up` and `down` in place of +60 and -90)."""
    ca, cb = hd // 2 - 2, hd - 2
    Q = g.integers(-2, 3, (rows_q, heads * hd)).astype(np.float32)
    K = g.integers(-2, 3, (rows_k, heads * hd)).astype(np.float32)
    V = g.standard_normal((rows_k, heads * hd)).astype(np.float32)
    blk = np.arange(rows_k) // 64
    i = np.arange(rows_q)
    cat = np.where((i // 32) % 3 == 2, 0, i % 4)
    for h in range(heads):
        K[:, h * hd + ca] = 8 + np.take(A, blk % 6)
        K[:, h * hd + cb] = 8 + np.take(B, blk % 6)
        Q[:, h * hd + ca] = np.select([cat == 1, cat == 2], [up, down], 0.0)
        Q[:, h * hd + cb] = np.where(cat == 3, up, 0.0)
    return Q, K, V


def bf16_to_f64(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def box_bias_log2(dy, dx, W, rows):
    """The box bias [heads, Nq, Nk] the bf16 kernel adds in its exp2
    domain, rounded in float32 as the device rounds it: from bias rows
    (head width 32, W >= 64 a multiple of 8) dy[j / W] log2(e) +
    dx[j % W] log2(e), from a table (dy[j / W] + dx[j % W]) log2(e)."""
    H = dy.shape[1]
    j = np.arange(H * W)
    L = np.float32(LOG2E)
    if rows:
        b = (dy * L)[:, j // W, :] + (dx * L)[:, j % W, :]
    else:
        b = (dy[:, j // W, :] + dx[:, j % W, :]) * L
    return b.transpose(2, 0, 1)


def packed_exact(be, m, nb, N, Nk, bias=None, causal=False):
    """Exact attention [nb, N, 64] of the packed bf16 operands left on the
    device (plus `bias` [nb, N, Nk], exp2 domain, if given), and the
    scores' per-row maxima / first-block maxima."""
    Np, Npk = pad64(N), pad64(Nk)
    q = bf16_to_f64(be.read(m.m.q16, nb * Np * 64)).reshape(nb, Np, 64)[:, :N]
    k = bf16_to_f64(be.read(m.m.k16, nb * Npk * 64)).reshape(nb, Npk, 64)[:, :Nk]
    v = bf16_to_f64(be.read(m.m.vt16, nb * Npk * 64)).reshape(nb, 64, Npk)[:, :, :Nk]
    bt = bias
    out = np.empty((nb, N, 64))
    stats = {"max": [], "first": []}
    for u in range(nb):
        s = q[u] @ k[u].T
        if bt is not None:
            s += bt[u]
        if causal:
            s[np.triu_indices(N, 1, Nk)] = -np.inf
        mx = s.max(1, keepdims=True)
        stats["max"].append(mx[:, 0])
        stats["first"].append(s[:, :64].max(1))
        p = np.exp2(s - mx)
        out[u] = (p @ v[u].T) / p.sum(1, keepdims=True)
    stats = {n: np.concatenate(x) for n, x in stats.items()}
    return out, stats


def assert_ranges(stats):
    """The construction reaches both sides of the +-64 span."""
    assert (stats["max"] > 64).any() and (stats["max"] < -64).any()
    assert (stats["first"] > 64).any()
    jump = stats["max"] - stats["first"]
    assert (jump > 64).sum() > 0


def head_major(O, N, heads, nunits=1):
    """O [nunits N, heads 64] -> [nunits heads, N, 64]."""
    return O.reshape(nunits, N, heads, 64).transpose(0, 2, 1, 3).reshape(
        nunits * heads, N, 64)


@pytest.mark.parametrize("N,nunits,heads,rope", [
    (5184, 1, 16, True),    # the global block's shape, 656 workgroups
    (200, 2, 2, True),      # ragged, two key splits
    (5184, 1, 1, False),    # one unit: 18 key splits, wave-per-query merge
])
def test_vit_attention_large_scores(hip, be, orc, N, nunits, heads, rope):
    E = heads * 64
    g = np.random.default_rng(N + heads)
    qkv = np.empty((nunits * N, 3 * E), np.float32)
    for u in range(nunits):
        Q, K, V = ranged_heads(g, N, N, heads, 64)
        qkv[u * N:(u + 1) * N] = np.concatenate([Q, K, V], 1)
    m = hip.Model(be, embed=E, heads=heads)
    side = math.isqrt(N)
    table = None
    if rope and be.precision == "bf16":
        table = orc.rope_table(side if side * side == N else side + 1)[:N]
    dq = be.upload(qkv)
    dt = be.upload(table) if table is not None else None
    do = be.alloc(nunits * N * E * 4)
    st = N * 3 * E
    print("large scores N=%d units=%d heads=%d %s" % (N, nunits, heads,
                                                      be.precision), flush=True)
    try:
        hip.attn_fused(m, N, nunits * heads, heads,
                       hip.bmat(dq, 0, 3 * E, st, 64),
                       hip.bmat(dq, E, 3 * E, st, 64),
                       hip.bmat(dq, 2 * E, 3 * E, st, 64),
                       hip.bmat(do, 0, E, N * E, 64), dt, N, 0.125)
        got = be.read(do).reshape(nunits * N, E)
        assert np.isfinite(got).all()
        if be.precision == "bf16":
            want, stats = packed_exact(be, m, nunits * heads, N, N)
            assert_ranges(stats)
            err = report("large scores packed N=%d h=%d" % (N, heads),
                         head_major(got, N, heads, nunits), want)
            assert err <= PACKED_TOL
        else:
            want = np.zeros_like(got)
            for u in range(nunits):
                sl = slice(u * N, (u + 1) * N)
                for h in range(heads):
                    want[sl, h * 64:(h + 1) * 64] = orc.attend(
                        qkv[sl, h * 64:(h + 1) * 64],
                        qkv[sl, E + h * 64:E + (h + 1) * 64],
                        qkv[sl, 2 * E + h * 64:2 * E + (h + 1) * 64], 1, 64)
            assert report("large scores fp32 N=%d h=%d" % (N, heads), got,
                          want) <= FP32_TOL
    finally:
        for x in (dq, dt, do):
            if x is not None:
                be.release(x)
        m.free()


def _attend(hip, be, Q, K, V, heads, hd, causal=False, dy=None, dx=None, W=0):
    Nq, Nk, D = Q.shape[0], K.shape[0], heads * hd
    m = hip.Model(be, embed=128, heads=2)
    dq, dk, dv = be.upload(Q), be.upload(K), be.upload(V)
    do = be.alloc(Nq * D * 4)
    ddy = be.upload(dy) if dy is not None else None
    ddx = be.upload(dx) if dx is not None else None
    try:
        hip.attend(m, Nq, Nk, heads, hd, dq, D, dk, D, dv, D, do, D, causal,
                   ddy, ddx, W)
        got = be.read(do).reshape(Nq, D)
        packed = None
        if be.precision == "bf16":
            packed = packed_exact(
                be, m, heads, Nq, Nk,
                bias=box_bias_log2(dy, dx, W, hd == 32) if dy is not None else None,
                causal=causal)
        return got, packed
    finally:
        for x in (dq, dk, dv, do, ddy, ddx):
            if x is not None:
                be.release(x)
        m.free()


@pytest.mark.parametrize("Nq,Nk,heads,hd,causal,box", [
    (201, 5184, 8, 64, False, True),    # box bias, 40 key splits
    (201, 5184, 8, 32, False, True),    # the same at head width 32
    (300, 300, 4, 64, True, False),     # causal, splits past the diagonal
    (1024, 1024, 8, 32, False, False),  # head width 32 self-attention
])
def test_attend_large_scores(hip, be, orc, Nq, Nk, heads, hd, causal, box):
    g = np.random.default_rng(Nq + Nk + hd)
    Q, K, V = ranged_heads(g, Nq, Nk, heads, hd)
    dy = dx = None
    W = 0
    if box:
        W = 72
        dy = g.standard_normal((Nq, Nk // W, heads)).astype(np.float32)
        dx = g.standard_normal((Nq, W, heads)).astype(np.float32)
    print("attend large scores Nq=%d Nk=%d hd=%d %s" % (Nq, Nk, hd,
                                                        be.precision), flush=True)
    got, packed = _attend(hip, be, Q, K, V, heads, hd, causal, dy, dx, W)
    assert np.isfinite(got).all()
    if packed is not None:
        want, stats = packed
        assert (stats["max"] > 64).any() and (stats["max"] < -64).any()
        got_h = got.reshape(Nq, heads, hd).transpose(1, 0, 2)
        assert report("attend large packed Nq=%d hd=%d" % (Nq, hd), got_h,
                      want[:, :, :hd]) <= PACKED_TOL
    else:
        want = orc.attend(Q, K, V, heads, hd, causal=causal, dy=dy, dx=dx, W=W)
        assert report("attend large fp32 Nq=%d hd=%d" % (Nq, hd), got,
                      want) <= FP32_TOL


@pytest.mark.parametrize("Nq,Nk", [(7, 4096), (4096, 7), (8, 5184)])
def test_mha_large_scores(hip, be, orc, Nq, Nk):
    """Decoder cross-attention (8 heads x 16, scale 1/4) with per-prompt
    keys: token -> image through k_mha_many16, whose lazy reference point
    moves by the 2^8 rule, and image -> token through the few-keys
    kernels. Query components +4 / -6: scores span -70 .. +46 log2 units,
    far past the 8-unit rule, while the fp32 rounding of q scale (the
    kernels fold log2 e into it) stays below the bar. fp32 oracle bar on
    both paths: mha's kernels compute in fp32 on either."""
    P, dint = 4, 128
    g = np.random.default_rng(Nq * 7 + Nk)
    q = np.empty((P, Nq, dint), np.float32)
    k = np.empty((P, Nk, dint), np.float32)
    v = np.empty((P, Nk, dint), np.float32)
    for p in range(P):
        q[p], k[p], v[p] = ranged_heads(g, Nq, Nk, 8, 16, 4.0, -6.0)
    m = hip.Model(be, embed=1024, heads=16)
    dq, dk, dv = be.upload(q), be.upload(k), be.upload(v)
    do = be.alloc(P * Nq * dint * 4)
    try:
        hip.mha(m, P, Nq, Nk, dint, dq, Nq * dint, dk, Nk * dint, dv,
                Nk * dint, do)
        got = be.read(do).reshape(P * Nq, dint)
        assert np.isfinite(got).all()
        want = orc.mha(P, Nq, Nk, dint, q, Nq * dint, k, Nk * dint, v,
                       Nk * dint)
        assert report("mha large scores Nq=%d Nk=%d %s" % (Nq, Nk, be.precision),
                      got, want) <= FP32_TOL
    finally:
        for x in (dq, dk, dv, do):
            be.release(x)
        m.free()


def test_t2i_rising_scores(hip, be, orc):
    """Token -> image block of the decoder (bf16: k_t2i_fused) over image
    keys scaled per 64-key block by (1, 1, 6, 1, 4, 1)[block % 6], so that
    every key split's streams see block maxima pass their reference point
    by more than 8 log2 units after their first block (checked on the
    scores themselves), against the oracle at the precision's bar."""
    from test_gpu_decoder import Dec, TOL
    weights = hip.random_decoder_weights(7)
    G, P = 72, 2
    d = Dec(hip, be, orc, weights, G, P, 51)
    try:
        T = d.T
        g = np.random.default_rng(52)
        qry = g.standard_normal((P, 8, 256)).astype(np.float32)
        qpe = g.standard_normal((P, 8, 256)).astype(np.float32)
        f = np.take(np.float32([1, 1, 6, 1, 4, 1]), (np.arange(T) // 64) % 6)
        keys = g.standard_normal((P, T, 256)).astype(np.float32) * f[None, :, None]
        # Head 0's scores in log2 units: the scaled blocks pass the first
        # block's maximum by more than the 2^8 rule.
        pre = "layers.1.t2i."
        qh = (qry + qpe) @ weights[pre + "qw"].T + weights[pre + "qb"]
        kh = (keys + d.prep["pe"][None]) @ weights[pre + "kw"].T + weights[pre + "kb"]
        s = np.einsum("pic,pjc->pij", qh.reshape(P, 8, 8, 16)[..., 0, :],
                      kh.reshape(P, T, 8, 16)[..., 0, :]) * 0.25 * LOG2E
        assert (s.max(2) - s[:, :, :64].max(2) > 8).mean() > 0.5
        for name, x in (("qry", qry), ("qpe", qpe), ("keys", keys)):
            be.write(d.dec.buf(name), 0, x)
        hip.t2i_attention(d.model, d.dec, P, d.dec.d.layers[1].t2i)
        got = be.read_f32(d.dec.buf("qry"), P * 8 * 256).reshape(P, 8, 256)
        want, _ = orc.t2i_attention(P, T, qry, qpe, keys, d.prep["pe"],
                                    d.dw.d.layers[1].t2i)
        assert np.isfinite(got).all()
        assert report("t2i rising %s" % be.precision, got - qry,
                      want - qry) <= TOL[be.precision]
    finally:
        d.free()
