"""The HIP path against the golden vectors of the reference's own OpenCL
kernels (same seeded inputs, outputs of sam3_kernels.cl run unchanged).

Two routes per case: the reference's operator sequence replayed with this
library's operators (gemm, softmax_rows, softmax_ext, layernorm,
rope_apply, window ops, mha), and for the attention cases the fused
attn_fused / vit_attention / attend entry points. Bars: bit-exact for data movement and RoPE, rel-L2 <= 2e-5
on the fp32 path, <= 2e-2 on the bf16 path; max-abs printed."""
import os
import sys

import numpy as np
import pytest

from gpu_common import rel_l2, report
from test_golden import EXACT, load

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import golden_cases as gc  # noqa: E402

pytestmark = pytest.mark.gpu


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


class HipImpl:
    """This library's operators behind the API the golden cases use."""

    def __init__(self, hip, be):
        self.hip, self.be = hip, be
        self.m = hip.Model(be, embed=128, heads=2)

    def _up(self, a):
        return self.be.upload(np.ascontiguousarray(a, np.float32))

    def gemm(self, kernel, M, N, K, A, aoff, lda, sa0, sa1, B, boff, ldb,
             sb0, sb1, transb, C, coff, ldc, sc0, sc1, nb, nb1, bias=None,
             use_r=False, roff=0, alpha=1.0, act=0):
        h = self.hip
        dA, dB, dC = self._up(A), self._up(B), self._up(C)
        db = self._up(bias) if bias is not None else None
        h.gemm(self.m, M, N, K, h.bmat(dA, aoff, lda, sa0, sa1),
               h.bmat(dB, boff, ldb, sb0, sb1), transb,
               h.bmat(dC, coff, ldc, sc0, sc1), nb, nb1, db,
               dC if use_r else None, roff, alpha, act)
        out = self.be.read_f32(dC).reshape(np.shape(C))
        for d in (dA, dB, dC) + ((db,) if db is not None else ()):
            self.be.release(d)
        return out

    def softmax_rows(self, S):
        d = self._up(S)
        self.hip.softmax_rows(self.m, d, S.size // S.shape[-1], S.shape[-1])
        out = self.be.read(d).reshape(S.shape)
        self.be.release(d)
        return out

    def softmax_ext(self, S, Nq, h0, causal, dy, dx, W, nh):
        d = self._up(S)
        ddy = self._up(dy) if dy is not None else None
        ddx = self._up(dx) if dx is not None else None
        self.hip.softmax_ext(self.m, d, S.size // S.shape[-1], S.shape[-1], Nq,
                             h0, causal, ddy, ddx, W, nh)
        out = self.be.read(d).reshape(S.shape)
        for x in (d, ddy, ddx):
            if x is not None:
                self.be.release(x)
        return out

    def layernorm(self, X, g, b, eps=1e-5, act=0):
        dX, dg, db = self._up(X), self._up(g), self._up(b)
        dY = self.be.alloc(X.size * 4)
        C = X.shape[-1]
        self.hip.layernorm(self.m, X.size // C, C, dX, dY, dg, db, eps, act)
        return self.be.read(dY).reshape(X.shape)

    def rope_apply(self, qkv, E, hd, npos, cs):
        m = self.hip.Model(self.be, embed=E, heads=E // 64)
        m.m.qkv = self._up(qkv)
        self.hip.rope_apply(m, self._up(cs), qkv.shape[0], npos)
        return self.be.read(m.m.qkv).reshape(qkv.shape)

    def window_partition(self, X, H, C, ws):
        nwx = -(-H // ws)
        d = self.be.alloc(nwx * nwx * ws * ws * C * 4)
        self.hip.window_partition(self.m, self._up(X), d, H, C, ws, nwx)
        return self.be.read(d).reshape(-1, C)

    def window_unpartition_add(self, X, Wd, H, C, ws):
        dX = self._up(X)
        self.hip.window_unpartition_add(self.m, dX, self._up(Wd), H, C, ws,
                                        -(-H // ws))
        return self.be.read(dX).reshape(X.shape)

    def mha(self, P, Nq, Nk, dint, Q, sq, K, sk, V, sv):
        do = self.be.alloc(P * Nq * dint * 4)
        self.hip.mha(self.m, P, Nq, Nk, dint, self._up(Q), sq, self._up(K), sk,
                     self._up(V), sv, do)
        return self.be.read(do).reshape(P * Nq, dint)


    def convt_scatter(self, G, bias, add, P, H, W, Co, act):
        dG, db = self._up(G), self._up(bias)
        da = self._up(add) if add is not None else None
        do = self.be.alloc(P * 4 * H * W * Co * 4)
        self.hip.convt_scatter(self.m, dG, do, db, da, P, H, W, Co, act)
        return self.be.read_f32(do).reshape(P, 2 * H, 2 * W, Co)

    def mask_logits(self, U, hyper, P, npix):
        do = self.be.alloc(P * 3 * npix * 4)
        self.hip.mask_logits(self.m, self._up(U), self._up(hyper), do, P, npix)
        return self.be.read_f32(do).reshape(P, 3, npix)

    def mask_post(self, lowres, sel, L, out_h, out_w, offset):
        """Through sam_postprocess (no hole filling) and sam_read_mask on a
        decoder whose low-resolution planes are `lowres`."""
        hip, be = self.hip, self.be
        planes = lowres.shape[0]
        model = hip.Model(be, embed=1024, heads=16)
        model.m.grid = L // 4
        dec = hip.Decoder(model, hip.random_decoder_weights(1), -(-planes // 3),
                          img=14 * (L // 4))
        try:
            be.write(dec.buf("lowres"), 0, np.ascontiguousarray(lowres, np.float32))
            stats = dec.postprocess(sel, out_h, out_w, offset, False)
            mask = np.stack([dec.read_mask(k, out_h, out_w, 0, 0, out_w - 1,
                                           out_h - 1) for k in range(len(sel))])
        finally:
            dec.free()
            model.free()
        return mask, stats


def _check(name, got, gold, tol):
    rows = gold["sample_rows"] if "sample_rows" in gold.files else None
    for k, v in got.items():
        if rows is not None and v.ndim == 2:
            v = v[rows]
        if name in EXACT:
            np.testing.assert_array_equal(v, gold[k])
        else:
            assert report("%s %s" % (name, k), v, gold[k]) <= tol


@pytest.mark.parametrize("name", [n for n in gc.CASES
                                  if not n.startswith("mask_post")])
def test_operator_sequence(hip, be, name):
    case, gold = load(name)
    _check(name, gc.run_reference(name, case, HipImpl(hip, be)), gold, 2e-5)


@pytest.mark.parametrize("name", [n for n in gc.CASES if n.startswith("mask_post")])
def test_mask_post_against_reference(hip, be, name):
    """sam_postprocess against the reference's mask_post: masks and counts
    agree except at pixels whose exact bilinear value lies on a threshold
    (0, +-offset) within 1e-5, where the reference's 2.5-ulp OpenCL
    division may round the other way."""
    import torch
    case, gold = load(name)
    mask, stats = gc.run_reference(name, case, HipImpl(hip, be)).values()
    low, sel = case["inputs"]
    off = case["offset"]
    v = torch.nn.functional.interpolate(
        torch.from_numpy(low[sel]).double()[:, None],
        size=(case["out_h"], case["out_w"]), mode="bilinear",
        align_corners=False)[:, 0].numpy()
    diff = mask != gold["mask"]
    assert np.all(np.abs(v[diff]) < 1e-5)
    for k in range(len(sel)):
        assert abs(int(stats[k, 0]) - int(gold["stats"][k, 0])) <= \
            int((np.abs(v[k] - off) < 1e-5).sum())
        assert abs(int(stats[k, 1]) - int(gold["stats"][k, 1])) <= \
            int((np.abs(v[k] + off) < 1e-5).sum())


@pytest.mark.parametrize("name", ["attn_window_cpu", "attn_window_gpu",
                                  "attn_global_rope_head"])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_fused_attention(hip, be, be16, name, precision):
    case, gold = load(name)
    b = be if precision == "fp32" else be16
    N, E, H = case["N"], case["E"], case["heads"]
    m = hip.Model(b, embed=E, heads=H)
    dq = b.upload(case["inputs"][0])
    do = b.alloc(N * E * 4)
    table = b.upload(case["inputs"][1]) if case["rope"] else None
    hip.attn_fused(m, N, H, H, hip.bmat(dq, 0, 3 * E, 0, 64),
                   hip.bmat(dq, E, 3 * E, 0, 64),
                   hip.bmat(dq, 2 * E, 3 * E, 0, 64),
                   hip.bmat(do, 0, E, 0, 64), table, N, 0.125)
    got = b.read(do).reshape(N, E)[gold["sample_rows"]]
    tol = 2e-5 if precision == "fp32" else 2e-2
    assert report("fused %s %s" % (name, precision), got, gold["O"]) <= tol


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("unfused", [False, True])
def test_vit_region(hip, be, be16, precision, unfused):
    case, gold = load("vit_window_region")
    b = be if precision == "fp32" else be16
    x, n1w, n1b, w, bias, table = case["inputs"]
    grid, E, ws = case["grid"], case["E"], case["ws"]
    blk = hip.VitBlock()
    blk.n1w, blk.n1b = b.upload(n1w), b.upload(n1b)
    blk.qkvw, blk.qkvb = b.upload_weight(w), b.upload(bias)
    blk.window = ws
    m = hip.Model(b, grid=grid, embed=E, heads=E // 64, blocks=[blk])
    m.m.rope_win = b.upload(table)
    b.write(m.m.x, 0, x)
    hip.vit_attention(m, blk, unfused)
    rows = gold["O"].shape[0]
    got = b.read(m.m.attn, rows * E).reshape(rows, E)
    tol = 2e-5 if precision == "fp32" else 2e-2
    assert report("vit region %s unfused=%d" % (precision, unfused), got,
                  gold["O"]) <= tol
    m.free()


@pytest.mark.parametrize("name", [n for n in gc.CASES if n.startswith("attend_")])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_attend_entry_point(hip, be, be16, name, precision):
    """attend() through the C-ABI: fused for the unmasked self-attention
    (head width 32 packed to 64 on the bf16 path), the reference's
    gemm / softmax_ext / gemm sequence for the causal and box-bias cases."""
    case, gold = load(name)
    b = be if precision == "fp32" else be16
    Q, K, V = case["inputs"][:3]
    Nq, Nk, H, hd = case["Nq"], case["Nk"], case["heads"], case["hd"]
    D = H * hd
    m = hip.Model(b, embed=128, heads=2)
    dq, dk, dv = b.upload(Q), b.upload(K), b.upload(V)
    do = b.alloc(Nq * D * 4)
    dy = dx = None
    if case["mode"] == "box":
        dy, dx = b.upload(case["inputs"][3]), b.upload(case["inputs"][4])
    hip.attend(m, Nq, Nk, H, hd, dq, D, dk, D, dv, D, do, D,
               case["mode"] == "causal", dy, dx, case["W"])
    got = b.read(do).reshape(Nq, D)
    tol = 2e-5 if precision == "fp32" else 2e-2
    assert report("attend %s %s" % (name, precision), got, gold["O"]) <= tol
    m.free()
