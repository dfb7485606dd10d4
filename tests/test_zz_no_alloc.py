"""mha_noalloc against mha through the C ABI.

mha_noalloc runs mha's kernels with the many-keys split partials in the
library's static device scratch instead of the backend's scratch buffer.
Its outputs must equal mha's bit for bit (same kernels, same split rule,
same arithmetic), on two calls in a row where the second is smaller, on
both the split-K token -> image shape (scratch in use) and the few-keys
image -> token shape; the oracle checks both at the fp32 bar. A fresh
backend that only ever ran mha_noalloc has no backend scratch afterwards:
the call took nothing from the allocator.
"""
import numpy as np
import pytest

from gpu_common import report

pytestmark = pytest.mark.gpu

FP32_TOL = 2e-5


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    return sam3_hip


def _case(seed, P, Nq, Nk, dint=128):
    g = np.random.default_rng(seed)
    q = g.standard_normal((P, Nq, dint)).astype(np.float32)
    k = g.standard_normal((P, Nk, dint)).astype(np.float32)
    v = g.standard_normal((P, Nk, dint)).astype(np.float32)
    return q, k, v


def _run(hip, be, m, fn, q, k, v):
    P, Nq, dint = q.shape
    Nk = k.shape[1]
    dq, dk, dv = be.upload(q), be.upload(k), be.upload(v)
    do = be.alloc(P * Nq * dint * 4)
    try:
        fn(m, P, Nq, Nk, dint, dq, Nq * dint, dk, Nk * dint, dv, Nk * dint, do)
        return be.read(do).reshape(P * Nq, dint)
    finally:
        for x in (dq, dk, dv, do):
            be.release(x)


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_mha_noalloc_matches_mha(hip, orc, precision):
    # Fresh backends: one that only runs mha_noalloc, one for mha.
    b_na = hip.Backend(precision=precision)
    b_ref = hip.Backend(precision=precision)
    m_na = hip.Model(b_na, embed=1024, heads=16)
    m_ref = hip.Model(b_ref, embed=1024, heads=16)
    try:
        # Token -> image with split keys (64 prompts x 7 tokens over 4096
        # image tokens, then a smaller call), image -> token (few keys).
        for seed, (P, Nq, Nk) in enumerate([(64, 7, 4096), (3, 8, 1000),
                                            (4, 4096, 7)]):
            q, k, v = _case(100 + seed, P, Nq, Nk)
            print("mha_noalloc %s P=%d Nq=%d Nk=%d" % (precision, P, Nq, Nk),
                  flush=True)
            got = _run(hip, b_na, m_na, hip.mha_noalloc, q, k, v)
            want = _run(hip, b_ref, m_ref, hip.mha, q, k, v)
            assert np.array_equal(got, want), (P, Nq, Nk)
            ref = orc.mha(P, Nq, Nk, 128, q, Nq * 128, k, Nk * 128, v, Nk * 128)
            assert report("mha_noalloc %s P=%d Nq=%d Nk=%d" % (precision, P, Nq, Nk),
                          got, ref) <= FP32_TOL
        # The noalloc backend never grew its scratch; mha's did (split).
        assert not b_na._b.scratch and b_na._b.scratch_bytes == 0
        assert b_ref._b.scratch
    finally:
        m_na.free()
        m_ref.free()
        b_na.free()
        b_ref.free()


def test_mha_noalloc_errors_match_mha(hip):
    """Shape errors are those of mha (fatal with a message naming the
    call)."""
    be = hip.Backend(precision="fp32")
    m = hip.Model(be, embed=1024, heads=16)
    d = be.alloc(100 * 256 * 4)
    try:
        with pytest.raises(hip.Sam3HipError, match="mha_noalloc: unsupported shape"):
            hip.mha_noalloc(m, 1, 4, 100, 256, d, 0, d, 0, d, 0, d)
        with pytest.raises(hip.Sam3HipError, match="mha_noalloc: per-prompt strides"):
            hip.mha_noalloc(m, 2, 4, 100, 128, d, 0, d, 100 * 128 + 2, d, 0, d)
    finally:
        be.release(d)
        m.free()
        be.free()
