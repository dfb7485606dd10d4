"""Pins the mask decoder part of the CPU oracle (oracle/sam3_oracle_dec.c)
without the reference running.

- The whole decoder (prompt tokens, two-way transformer, upscaling,
  hypernetwork and IoU heads, low-resolution logits) against a float64
  restatement of the PyTorch SAM mask decoder semantics (tests/ref64.py
  decode64: heads split by reshape, ConvTranspose2d by einsum, LayerNorm2d,
  exact GELU), with a planted wiring mistake that the check catches.
- convt_scatter after the upscaling GEMM against torch's
  conv_transpose2d (the column order co * 4 + dy * 2 + dx is PyTorch's
  ConvTranspose2d weight layout [in][out][2][2]).
- mask_post against torch's bilinear interpolate (align_corners=False) on
  dyadic inputs, where every interpolated value is exact in float32.
- fill_holes against scipy.ndimage.label with 8-connectivity.
- pe_encode, host_linear, mask_logits against float64 formulas.
"""
import math

import numpy as np
import pytest

import ref64


def rng(seed):
    return np.random.default_rng(seed)


@pytest.fixture(scope="module")
def weights():
    import sam3_hip
    return sam3_hip.random_decoder_weights(7)


def _image(G, seed):
    g = rng(seed)
    return (g.standard_normal((G * G, 256)).astype(np.float32),
            g.standard_normal((16 * G * G, 32)).astype(np.float32),
            g.standard_normal((4 * G * G, 64)).astype(np.float32))


@pytest.mark.parametrize("G,P", [(8, 3), (12, 2)])
def test_decode_matches_float64_sam(orc, weights, G, P):
    """Whole decoder vs the float64 PyTorch-semantics restatement."""
    emb, s0, s1 = _image(G, 10 + G)
    dw = orc.DecoderW(weights, G, img=14 * G)
    prep = orc.dec_prepare(dw, emb)
    pts = rng(G).uniform(0, 14 * G, (P, 2)).astype(np.float32)
    iou, low, _, _ = orc.sam_decode(dw, pts, prep, s0, s1)
    iou64, low64 = ref64.decode64(weights, G, 14 * G, pts, emb, s0, s1)
    assert np.abs(iou - iou64).max() < 1e-6
    assert ref64.rel_l2(low, low64) < 2e-6


def test_decode_wiring_teeth(orc, weights):
    """Teeth: the layer-1 token -> image attention with its key and value
    projections swapped (a plausible wiring slip) fails the check above."""
    G, P = 8, 2
    emb, s0, s1 = _image(G, 18)
    bad = dict(weights)
    bad["layers.1.t2i.kw"], bad["layers.1.t2i.vw"] = \
        weights["layers.1.t2i.vw"], weights["layers.1.t2i.kw"]
    dw = orc.DecoderW(bad, G, img=14 * G)
    prep = orc.dec_prepare(dw, emb)
    pts = rng(3).uniform(0, 14 * G, (P, 2)).astype(np.float32)
    _, low, _, _ = orc.sam_decode(dw, pts, prep, s0, s1)
    _, low64 = ref64.decode64(weights, G, 14 * G, pts, emb, s0, s1)
    assert ref64.rel_l2(low, low64) > 1e-3


def test_prompt_tokens(orc, weights):
    dw = orc.DecoderW(weights, 8, img=112)
    pts = np.array([[0, 0], [111, 57.5]], np.float32)
    tok = orc.prompt_tokens(dw, pts)
    assert np.array_equal(tok[:, 0], np.broadcast_to(weights["obj_token"], (2, 256)))
    assert np.array_equal(tok[:, 2:6], np.broadcast_to(weights["mask_tokens"], (2, 4, 256)))
    assert np.array_equal(tok[:, 7], np.broadcast_to(weights["not_a_point"], (2, 256)))
    want = ref64.pe_random(weights["gauss"], (pts + 0.5) / 112) + weights["point_emb"][1]
    assert np.abs(tok[:, 6] - want).max() < 2e-5


def test_pe_encode_formula(orc):
    g = rng(1).standard_normal((2, 128)).astype(np.float32)
    for x, y in ((0.0, 0.0), (0.25, 0.75), (1.0, 0.5)):
        got = orc.pe_encode(g, x, y)
        want = ref64.pe_random(g, np.array([x, y]))
        assert np.abs(got - want).max() < 2e-5
    # (0.5, 0.5) is the origin of the [-1, 1] square: sin 0 = 0, cos 0 = 1.
    got = orc.pe_encode(g, 0.5, 0.5)
    assert np.array_equal(got, np.r_[np.zeros(128), np.ones(128)].astype(np.float32))


def test_host_linear(orc):
    g = rng(2)
    W = g.standard_normal((33, 256)).astype(np.float32)
    b = g.standard_normal(33).astype(np.float32)
    x = g.standard_normal(256).astype(np.float32)
    want = W.astype(np.float64) @ x + b
    assert np.abs(orc.host_linear(W, b, x) - want).max() < 1e-5
    assert np.array_equal(orc.host_linear(W, b, x, relu=True),
                          np.maximum(orc.host_linear(W, b, x), 0))


def test_convt_scatter_is_conv_transpose(orc):
    """gemm(x, W as [Ci][Co 4]) + convt_scatter == conv_transpose2d; the
    add map and GELU on top."""
    import torch
    g = rng(3)
    P, H, W, Ci, Co = 2, 5, 7, 12, 6
    x = g.standard_normal((P, H, W, Ci)).astype(np.float32)
    wt = g.standard_normal((Ci, Co, 2, 2)).astype(np.float32)
    b = g.standard_normal(Co).astype(np.float32)
    add = g.standard_normal((2 * H, 2 * W, Co)).astype(np.float32)
    G = (x.reshape(-1, Ci).astype(np.float64) @
         wt.reshape(Ci, Co * 4).astype(np.float64)).astype(np.float32)
    got = orc.convt_scatter(G, b, None, P, H, W, Co)
    want = torch.nn.functional.conv_transpose2d(
        torch.from_numpy(x).double().permute(0, 3, 1, 2),
        torch.from_numpy(wt).double(), torch.from_numpy(b).double(),
        stride=2).permute(0, 2, 3, 1).numpy()
    assert np.abs(got - want).max() < 1e-4
    got = orc.convt_scatter(G, b, add, P, H, W, Co, act=1)
    assert np.abs(got - ref64.gelu_fast(want + add)).max() < 1e-4


def test_mask_logits_einsum(orc):
    g = rng(4)
    P, npix = 3, 50
    U = g.standard_normal((P, npix, 32)).astype(np.float32)
    hyper = g.standard_normal((P, 3, 32)).astype(np.float32)
    got = orc.mask_logits(U, hyper, P, npix)
    want = np.einsum("pkc,pnc->pkn", hyper.astype(np.float64), U.astype(np.float64))
    assert np.abs(got - want).max() < 1e-5


@pytest.mark.parametrize("L,out_h,out_w", [(16, 32, 32), (16, 8, 64), (12, 24, 6)])
def test_mask_post_matches_interpolate(orc, L, out_h, out_w):
    """Scale factors 1/2 and 2 make every source coordinate and weight a
    dyadic fraction; with logits in multiples of 1/8 every interpolated
    value is exact, so the binary mask and the counts are too."""
    import torch
    g = rng(5 + L + out_w)
    low = (g.integers(-40, 41, (4, L, L)) / 8.0).astype(np.float32)
    sel = np.array([2, 0, 3], np.int32)
    off = 0.5
    mask, stats = orc.mask_post(low, sel, L, out_h, out_w, off)
    v = torch.nn.functional.interpolate(
        torch.from_numpy(low[sel]).double()[:, None], size=(out_h, out_w),
        mode="bilinear", align_corners=False)[:, 0].numpy()
    assert np.array_equal(mask, (v > 0).astype(np.uint8))
    for k in range(len(sel)):
        assert stats[k, 0] == (v[k] > off).sum()
        assert stats[k, 1] == (v[k] > -off).sum()
        ys, xs = np.nonzero(v[k] > 0)
        if len(xs):
            assert list(stats[k, 2:]) == [xs.min(), ys.min(), xs.max(), ys.max()]
        else:
            assert list(stats[k, 2:]) == [0x7fffffff, 0x7fffffff, -1, -1]


def test_fill_holes_matches_label(orc):
    """Background components (<= 0, 8-connected) of at most max_area pixels
    become 10; larger ones and the foreground stay."""
    from scipy import ndimage
    g = rng(6)
    L, max_area = 40, 12
    v = np.where(g.random((L, L)) < 0.55, 1.0, -1.0).astype(np.float32)
    v[5:20, 5:20] = -2.0  # one large component
    got, changed = orc.fill_holes(v, max_area)
    lab, n = ndimage.label(v <= 0, structure=np.ones((3, 3)))
    want = v.copy()
    for c in range(1, n + 1):
        if (lab == c).sum() <= max_area:
            want[lab == c] = 10.0
    assert changed and np.array_equal(got, want)
    assert np.all(got[5:20, 5:20] == -2.0)
    _, changed = orc.fill_holes(np.ones((L, L), np.float32), max_area)
    assert not changed


def test_postprocess_fills_then_resizes(orc):
    g = rng(8)
    L = 16
    low = (g.integers(-40, 41, (3, L, L)) / 8.0).astype(np.float32)
    low[1, 3:5, 3:5] = -1.0
    low[1, 2, 2:6] = low[1, 5, 2:6] = low[1, 2:6, 2] = low[1, 2:6, 5] = 1.0
    filled, mask, stats = orc.postprocess(low, [1], 32, 32, 0.0, True, 256)
    assert np.all(filled[1, 3:5, 3:5] == 10.0)
    want_mask, want_stats = orc.mask_post(filled, [1], L, 32, 32, 0.0)
    assert np.array_equal(mask, want_mask) and np.array_equal(stats, want_stats)
