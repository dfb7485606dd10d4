"""GPU parity of the point-prompt mask decoder (sam3_model.c:1212-1530)
against the oracle's restatement (oracle/sam3_oracle_dec.c, itself pinned
to the float64 PyTorch-semantics decoder in test_oracle_decoder.py):

- convt_scatter, mask_logits, mask_post / sam_postprocess (with hole
  filling) and sam_read_mask at their kernel level: bit-exact where the
  arithmetic is the same fused multiply-add chain (mask logits, the
  bilinear resize and its statistics, the scatter without activation);
- the image -> token and token -> image attention blocks and the whole
  sam_decode at the 72 x 72 grid with per-prompt keys, and at a small
  grid with more prompts.

Bars: rel-L2 <= 2e-5 (fp32), <= 2e-2 (bf16); IoU max-abs alike.
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


@pytest.fixture(scope="module")
def weights(hip):
    return hip.random_decoder_weights(7)


def _image(G, seed):
    g = np.random.default_rng(seed)
    return (g.standard_normal((G * G, 256)).astype(np.float32),
            g.standard_normal((16 * G * G, 32)).astype(np.float32),
            g.standard_normal((4 * G * G, 64)).astype(np.float32))


class Dec:
    """A decoder on the device and the oracle's prepared inputs."""

    def __init__(self, hip, be, orc, w, G, batch, seed):
        self.model = hip.Model(be, embed=1024, heads=16)
        self.model.m.grid = G
        self.dec = hip.Decoder(self.model, w, batch, img=14 * G)
        self.emb, self.s0, self.s1 = _image(G, seed)
        self.dec.set_image(self.emb, self.s0, self.s1)
        self.dw = orc.DecoderW(w, G, img=14 * G)
        self.prep = orc.dec_prepare(self.dw, self.emb)
        self.G, self.T = G, G * G

    def free(self):
        self.dec.free()
        self.model.free()


def test_prepare_caches(hip, be, orc, weights):
    """sam_dec_prepare: dense PE, src, src + PE and the layer-0
    projections of the shared image keys, values and queries; on the bf16
    path also PE through the layer-1 image-query, layer-1 key and final
    key projections without their biases (the fused blocks' position
    term), against float64 products of the oracle's PE."""
    d = Dec(hip, be, orc, weights, 72, 1, 40)
    try:
        tol = TOL[be.precision]
        T = d.T
        pe = be.read_f32(d.dec.buf("pe_img"), T * 256).reshape(T, 256)
        assert np.abs(pe - d.prep["pe"]).max() < 1e-6
        for name, cols in (("src", 256), ("srcpe", 256), ("kp0", 128),
                           ("vp0", 128), ("qp0", 128)):
            got = be.read_f32(d.dec.buf(name), T * cols).reshape(T, cols)
            assert report("prepare %s %s" % (name, be.precision), got,
                          d.prep[name]) <= tol
        if be.precision == "bf16":
            pe64 = d.prep["pe"].astype(np.float64)
            for name, wname in (("pe_q1", "layers.1.i2t.qw"),
                                ("pe_k1", "layers.1.t2i.kw"),
                                ("pe_kf", "final_t2i.kw")):
                got = be.read_f32(d.dec.buf(name), T * 128).reshape(T, 128)
                want = pe64 @ np.asarray(weights[wname], np.float64).T
                assert report("prepare %s bf16" % name, got, want) <= tol
    finally:
        d.free()


@pytest.mark.parametrize("G,P", [(72, 2), (16, 6), (16, 12)])
def test_decode(hip, be, orc, weights, G, P):
    """The whole sam_decode: IoU predictions and low-resolution logits.
    P = 12 puts one or two prompts on each XCD in the fused blocks' work
    split (P >= 8 with an uneven share), P = 2 and 6 split the chunks."""
    d = Dec(hip, be, orc, weights, G, P, 41 + G)
    try:
        pts = np.random.default_rng(G).uniform(0, 14 * G, (P, 2)).astype(np.float32)
        print("sam_decode G=%d P=%d %s" % (G, P, be.precision), flush=True)
        hip.prof_reset()
        be.set_profile(True)
        try:
            iou = d.dec.decode(pts)
        finally:
            be.set_profile(False)
        ran = {r[0] for r in hip.prof_table()}
        # bf16 runs the fused attention blocks and upscaling.
        fused = {"i2t_fused", "t2i_fused", "upscale_fused"}
        assert fused <= ran if be.precision == "bf16" else not (fused & ran), ran
        low = d.dec.lowres(P)
        oiou, olow, _, _ = orc.sam_decode(d.dw, pts, d.prep, d.s0, d.s1)
        tol = TOL[be.precision]
        assert report("decode lowres G=%d %s" % (G, be.precision), low, olow) <= tol
        assert np.abs(iou - oiou).max() <= 4 * tol
        if be.precision != "fp32":
            return  # the bf16 path fuses the upscaling (no u2 map)
        # The logits kernel alone, on the device's own upscaled map and
        # hypernetwork outputs: the same fused multiply-add chain.
        T = G * G
        u2 = be.read_f32(d.dec.buf("u2"), P * 16 * T * 32)
        hyper = be.read_f32(d.dec.buf("hyper"), P * 96)
        want = orc.mask_logits(u2, hyper, P, 16 * T).reshape(low.shape)
        assert np.array_equal(low, want)
    finally:
        d.free()


def test_t2i_then_i2t_blocks(hip, be, orc, weights):
    """t2i_attention (per-prompt keys, kin left behind) and the layer-1
    image -> token block reading that kin, from seeded tokens and keys."""
    G, P = 72, 3
    d = Dec(hip, be, orc, weights, G, P, 43)
    try:
        T = d.T
        g = np.random.default_rng(44)
        qry = g.standard_normal((P, 8, 256)).astype(np.float32)
        qpe = g.standard_normal((P, 8, 256)).astype(np.float32)
        keys = g.standard_normal((P, T, 256)).astype(np.float32)
        for name, a in (("qry", qry), ("qpe", qpe), ("keys", keys)):
            be.write(d.dec.buf(name), 0, a)
        hip.t2i_attention(d.model, d.dec, P, d.dec.d.layers[1].t2i)
        got_q = be.read_f32(d.dec.buf("qry"), P * 8 * 256).reshape(P, 8, 256)
        want_q, kin = orc.t2i_attention(P, T, qry, qpe, keys, d.prep["pe"],
                                        d.dw.d.layers[1].t2i)
        tol = TOL[be.precision]
        assert report("t2i %s" % be.precision, got_q - qry, want_q - qry) <= tol
        # The image -> token block of layer 1 from the oracle's tokens.
        be.write(d.dec.buf("qry"), 0, want_q)
        hip.i2t_attention(d.model, 1, P)
        got_k = be.read_f32(d.dec.buf("keys"), P * T * 256).reshape(P, T, 256)
        want_k = orc.i2t_attention(1, P, T, want_q, qpe, keys, kin, None, None,
                                   d.dw.d.layers[1])
        assert report("i2t layer 1 %s" % be.precision, got_k, want_k) <= tol
        # Layer 0 reads the shared image queries and adds src.
        be.write(d.dec.buf("keys"), 0, keys)
        hip.i2t_attention(d.model, 0, P)
        got_k = be.read_f32(d.dec.buf("keys"), P * T * 256).reshape(P, T, 256)
        want_k = orc.i2t_attention(0, P, T, want_q, qpe, keys, None,
                                   d.prep["qp0"], d.prep["src"],
                                   d.dw.d.layers[0])
        assert report("i2t layer 0 %s" % be.precision, got_k, want_k) <= tol
    finally:
        d.free()


def test_convt_scatter_and_logits(hip, be, orc):
    """convt_scatter with and without the add map, and the logits kernel."""
    m = hip.Model(be, embed=1024, heads=16)
    g = np.random.default_rng(45)
    P, H, W, Co = 3, 9, 7, 32
    G = g.standard_normal((P * H * W, Co * 4)).astype(np.float32)
    b = g.standard_normal(Co).astype(np.float32)
    add = g.standard_normal((2 * H, 2 * W, Co)).astype(np.float32)
    dG, db, dadd = be.upload(G), be.upload(b), be.upload(add)
    dout = be.alloc(P * 4 * H * W * Co * 4)
    try:
        hip.convt_scatter(m, dG, dout, db, None, P, H, W, Co)
        got = be.read_f32(dout).reshape(P, 2 * H, 2 * W, Co)
        assert np.array_equal(got, orc.convt_scatter(G, b, None, P, H, W, Co))
        hip.convt_scatter(m, dG, dout, db, dadd, P, H, W, Co, hip.ACT_GELU)
        got = be.read_f32(dout).reshape(P, 2 * H, 2 * W, Co)
        want = orc.convt_scatter(G, b, add, P, H, W, Co, act=1)
        assert np.abs(got - want).max() < 1e-6
        with pytest.raises(hip.Sam3HipError):
            hip.convt_scatter(m, dG, dout, db, None, P + 1, H, W, Co)
    finally:
        for x in (dG, db, dadd, dout):
            be.release(x)


def test_logits_postprocess_and_read(hip, be, orc, weights):
    """sam_postprocess with and without hole filling and sam_read_mask of a
    region: the filled planes, masks and statistics bit-exact against the
    oracle on the same low-resolution logits."""
    G, P = 16, 2
    d = Dec(hip, be, orc, weights, G, P, 46)
    try:
        L = 4 * G
        g = np.random.default_rng(47)
        low = g.standard_normal((P * 3, L, L)).astype(np.float32)
        low[1, 10:13, 10:13] = -3.0
        low[1, 9, 9:14] = low[1, 13, 9:14] = 2.0
        low[1, 9:14, 9] = low[1, 9:14, 13] = 2.0
        sel = np.array([1, 4, 0], np.int32)
        for fill, (oh, ow) in ((False, (100, 77)), (True, (64, 128))):
            be.write(d.dec.buf("lowres"), 0, low)
            stats = d.dec.postprocess(sel, oh, ow, 0.3, fill)
            filled, mask, want = orc.postprocess(low, sel, oh, ow, 0.3, fill)
            assert np.array_equal(stats, want), (fill, stats, want)
            got_low = be.read_f32(d.dec.buf("lowres"), P * 3 * L * L).reshape(-1, L, L)
            assert np.array_equal(got_low, filled)
            region = d.dec.read_mask(2, oh, ow, 5, 3, ow - 2, oh - 9)
            assert np.array_equal(region, mask[2, 3:oh - 8, 5:ow - 1])
        if fill:
            assert np.all(got_low[1, 10:13, 10:13] == 10.0)
    finally:
        d.free()


def test_decode_graph_replays(hip, be, orc, weights):
    """sam_dec_graph: replays of the captured device sequence give the
    eager decode's IoU and logits bit for bit, for new points on every
    call, with eager work and host reads between the replays; another P
    runs the kernels one by one."""
    G, P = 16, 4
    d = Dec(hip, be, orc, weights, G, P, 48)
    try:
        g = np.random.default_rng(49)
        pts = [g.uniform(0, 14 * G, (P, 2)).astype(np.float32) for _ in range(3)]
        eager = [(d.dec.decode(x), d.dec.lowres(P)) for x in pts]
        d.dec.graph(P)
        for rep in range(2):
            for x, (iou, low) in zip(pts, eager):
                got_iou = d.dec.decode(x)
                assert np.array_equal(got_iou, iou)
                assert np.array_equal(d.dec.lowres(P), low)
        # A different prompt count is not the captured one: eager path
        # (its key splits differ, so the match is to the precision's bar).
        d.dec.decode(pts[0][:2])
        assert report("graph other P %s" % be.precision, d.dec.lowres(2),
                      eager[0][1][:2]) <= TOL[be.precision]
        d.dec.graph(P, False)
    finally:
        d.free()
