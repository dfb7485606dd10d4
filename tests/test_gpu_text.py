"""GPU parity of the text path's attention, attend() (sam3_text.c:305-343),
against the oracle's restatement (or_attend: gemm Q K^T / sqrt(hd),
softmax_ext with the causal mask or the box relative position bias, gemm
P V), at the shapes the text path runs:

- fusion encoder self-attention: 5184 image tokens, 8 heads x 32
  (sam3_text.c:797); sampled query rows;
- decoder cross-attention to the image: 201 queries over 5184 keys with
  the box bias dy / dx (sam3_text.c:860-861);
- text encoder self-attention: 32 tokens, 16 heads x 64, causal
  (sam3_text.c:489-490).

Both paths run all three in a fused kernel (bias as an additive table,
causal mask, head width 32): bf16 MFMA with the bias in the exp2 domain,
or f32 MFMA with the sums dy + dx added as softmax_ext adds them; other
head widths take the reference's chunked gemm / softmax_ext / gemm.

Bars: rel-L2 <= 2e-5 (fp32), <= 2e-2 (bf16); max-abs printed.
"""
import numpy as np
import pytest

from gpu_common import report

pytestmark = pytest.mark.gpu

TOL = {"fp32": 2e-5, "bf16": 2e-2}


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


def _run(hip, be, Q, K, V, heads, hd, causal=False, dy=None, dx=None, W=0,
         score_cap=None):
    Nq, Nk, D = Q.shape[0], K.shape[0], heads * hd
    m = hip.Model(be, embed=128, heads=2)
    if score_cap is not None:
        m.m.score_cap = score_cap
    dq, dk, dv = be.upload(Q), be.upload(K), be.upload(V)
    do = be.alloc(Nq * D * 4)
    ddy = be.upload(dy) if dy is not None else None
    ddx = be.upload(dx) if dx is not None else None
    try:
        hip.attend(m, Nq, Nk, heads, hd, dq, Q.shape[1], dk, K.shape[1], dv,
                   V.shape[1], do, D, causal, ddy, ddx, W)
        return be.read(do).reshape(Nq, D)
    finally:
        for x in (dq, dk, dv, do, ddy, ddx):
            if x is not None:
                be.release(x)
        m.free()


def test_fusion_encoder_self_attention(hip, be, orc):
    """5184 tokens (72 x 72), 8 heads x 32, no mask or bias."""
    N, heads, hd = 5184, 8, 32
    g = np.random.default_rng(31)
    Q, K, V = (g.standard_normal((N, heads * hd)).astype(np.float32)
               for _ in range(3))
    print("attend fusion self N=%d %s" % (N, be.precision), flush=True)
    got = _run(hip, be, Q, K, V, heads, hd)
    rows = np.sort(g.choice(N, 96, replace=False))
    want = orc.attend(Q[rows], K, V, heads, hd)
    assert report("fusion self %s" % be.precision, got[rows], want) <= TOL[be.precision]


def test_decoder_image_cross_attention_box_bias(hip, be, orc):
    """201 queries (presence + 200) over the 72 x 72 image tokens, 8 heads
    x 32, box relative position bias dy [201, 72, 8] + dx [201, 72, 8]."""
    Nq, W, heads, hd = 201, 72, 8, 32
    Nk = W * W
    g = np.random.default_rng(32)
    Q = g.standard_normal((Nq, heads * hd)).astype(np.float32)
    K, V = (g.standard_normal((Nk, heads * hd)).astype(np.float32) for _ in range(2))
    dy = (2 * g.standard_normal((Nq, W, heads))).astype(np.float32)
    dx = (2 * g.standard_normal((Nq, W, heads))).astype(np.float32)
    print("attend decoder box Nq=%d Nk=%d %s" % (Nq, Nk, be.precision), flush=True)
    got = _run(hip, be, Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
    want = orc.attend(Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
    assert report("decoder box %s" % be.precision, got, want) <= TOL[be.precision]


def test_text_encoder_causal(hip, be, orc):
    """32 text tokens of width 1024: 16 heads x 64, causal mask; query 0
    attends to key 0 alone."""
    n, heads, hd = 32, 16, 64
    g = np.random.default_rng(33)
    Q, K, V = (g.standard_normal((n, heads * hd)).astype(np.float32)
               for _ in range(3))
    got = _run(hip, be, Q, K, V, heads, hd, causal=True)
    want = orc.attend(Q, K, V, heads, hd, causal=True)
    assert report("text causal %s" % be.precision, got, want) <= TOL[be.precision]
    if be.precision == "fp32":
        assert np.array_equal(got[0], V[0])


def test_score_chunks_and_capacity(hip, be, orc):
    """Head widths the fused kernels do not take (16 here) run the
    reference's chunked sequence on both paths: one head per score chunk
    gives the result of all heads at once (the chunk offset reaches the
    bias and the operand columns), matching the oracle, and a buffer that
    cannot hold one head's scores is the reference's fatal error. At head
    width 32 the fused kernel needs no score buffer: the capacity leaves
    its result unchanged."""
    Nq, W, heads = 30, 6, 4
    Nk = W * 5
    g = np.random.default_rng(34)
    for hd in (16, 32):
        Q = g.standard_normal((Nq, heads * hd + 8)).astype(np.float32)
        K, V = (g.standard_normal((Nk, heads * hd)).astype(np.float32)
                for _ in range(2))
        dy = g.standard_normal((Nq, 5, heads)).astype(np.float32)
        dx = g.standard_normal((Nq, W, heads)).astype(np.float32)
        a = _run(hip, be, Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
        b = _run(hip, be, Q, K, V, heads, hd, dy=dy, dx=dx, W=W, score_cap=Nq * Nk)
        assert np.array_equal(a, b)
        want = orc.attend(Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
        assert report("chunks hd=%d %s" % (hd, be.precision), a, want) <= TOL[be.precision]
        if hd == 16:
            with pytest.raises(hip.Sam3HipError):
                _run(hip, be, Q, K, V, heads, hd, dy=dy, dx=dx, W=W,
                     score_cap=Nq * Nk - 1)
        else:
            c = _run(hip, be, Q, K, V, heads, hd, dy=dy, dx=dx, W=W,
                     score_cap=Nq * Nk - 1)
            assert np.array_equal(a, c)


def test_long_causal_split_keys(hip, be, orc):
    """600 tokens, 2 heads x 64, causal: on the bf16 path the keys split
    five ways, and splits past a query's position see no key at all
    (their partials carry l = 0 and drop out of the merge)."""
    n, heads, hd = 600, 2, 64
    g = np.random.default_rng(35)
    Q, K, V = (g.standard_normal((n, heads * hd)).astype(np.float32)
               for _ in range(3))
    got = _run(hip, be, Q, K, V, heads, hd, causal=True)
    want = orc.attend(Q, K, V, heads, hd, causal=True)
    assert report("long causal %s" % be.precision, got, want) <= TOL[be.precision]


def test_key_splits_not_a_multiple_of_four(hip, be, orc):
    """5700 causal tokens, one head of 64: 45 query tiles split the keys 17
    ways on both paths (causal attention takes the split launch on bf16
    too), merged inside the launch in groups of 8, 8 and 1 (a short last
    group), the groups then folded by the last group to finish; splits
    past a query's position see no key and drop out."""
    n, heads, hd = 5700, 1, 64
    g = np.random.default_rng(37)
    Q, K, V = (g.standard_normal((n, heads * hd)).astype(np.float32)
               for _ in range(3))
    got = _run(hip, be, Q, K, V, heads, hd, causal=True)
    want = orc.attend(Q, K, V, heads, hd, causal=True)
    assert report("17 key splits causal %s" % be.precision, got, want) <= TOL[be.precision]


def test_one_head_many_key_splits(hip, be, orc):
    """2000 tokens, one head of 64: 16 query tiles leave the GPU idle. The
    exact path splits the keys 16 ways and merges the splits inside its
    launch (two groups of eight); the bf16 path takes the grouped launch
    (four key groups per workgroup, merged in LDS). The bias case above
    takes 40 bf16 splits (five groups) and 48 exact ones (six)."""
    n, heads, hd = 2000, 1, 64
    g = np.random.default_rng(36)
    Q, K, V = (g.standard_normal((n, heads * hd)).astype(np.float32)
               for _ in range(3))
    got = _run(hip, be, Q, K, V, heads, hd)
    rows = np.sort(g.choice(n, 128, replace=False))
    want = orc.attend(Q[rows], K, V, heads, hd)
    assert report("many splits %s" % be.precision, got[rows], want) <= TOL[be.precision]


def test_sixty_four_key_splits(hip, be, orc):
    """256 queries over 8192 keys, one head of 64: two query tiles, so the
    exact path splits the keys the most it does, 64 ways (four 32-key
    blocks each), merged inside its launch in eight groups of eight, three
    records at a time (the last round of each group one record and a repeat
    that must add nothing); the bf16 path takes the grouped launch. A
    second launch gives the same bits."""
    nq, nk, heads, hd = 256, 8192, 1, 64
    g = np.random.default_rng(38)
    Q = g.standard_normal((nq, hd)).astype(np.float32)
    K, V = (g.standard_normal((nk, hd)).astype(np.float32) for _ in range(2))
    got = _run(hip, be, Q, K, V, heads, hd)
    want = orc.attend(Q, K, V, heads, hd)
    assert report("64 key splits %s" % be.precision, got, want) <= TOL[be.precision]
    assert np.array_equal(_run(hip, be, Q, K, V, heads, hd), got)


@pytest.mark.parametrize("Nq,H,W,hd", [
    (37, 8, 64, 32),    # bias rows (W >= 64 a multiple of 8, H a multiple of 4)
    (37, 8, 64, 64),    # rows on the exact path, the table on bf16 (head width 64)
    (37, 6, 64, 32),    # H not a multiple of 4: the table
    (130, 4, 72, 32),   # rows, two query tiles, a ragged last key block
    (21, 5, 80, 32),    # H = 5: the table
])
def test_box_bias_grids(hip, be, orc, Nq, H, W, hd):
    """The box bias of softmax_ext (sam3_kernels.cl:904-906) on grids that
    take the per-query dy / dx rows or the bias table, against the
    oracle's reference sequence."""
    heads = 4
    Nk = H * W
    g = np.random.default_rng(Nq * H + W + hd)
    Q = g.standard_normal((Nq, heads * hd)).astype(np.float32)
    K, V = (g.standard_normal((Nk, heads * hd)).astype(np.float32) for _ in range(2))
    dy = (2 * g.standard_normal((Nq, H, heads))).astype(np.float32)
    dx = (2 * g.standard_normal((Nq, W, heads))).astype(np.float32)
    print("attend box grid Nq=%d H=%d W=%d hd=%d %s" % (Nq, H, W, hd, be.precision),
          flush=True)
    got = _run(hip, be, Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
    want = orc.attend(Q, K, V, heads, hd, dy=dy, dx=dx, W=W)
    assert report("box grid H=%d W=%d hd=%d %s" % (H, W, hd, be.precision), got,
                  want) <= TOL[be.precision]
