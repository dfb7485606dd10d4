"""GPU tests of the checkpoint upload path (pth_upload, the load_dev
helpers, sam_load / sam_free) against torch's own conversions and
against models built from the same weights by host uploads.

- pth_upload of float32 / float16 / bfloat16 storages (contiguous and
  strided views) to each device element type equals torch's .float(),
  .half() and .bfloat16() of the tensor bit for bit (round to nearest
  even, overflow to infinity, subnormals; NaN-free inputs), and complex64
  rope tables arrive as their (real, imaginary) float pairs;
- sam_load of a SAM 3-named checkpoint (on the fp32, bf16 and fp16
  backends: weight matrices float, bfloat16 or half) holds exactly the
  buffers the host-built model holds (patch embedding, tiled position embedding,
  ln_pre, every block's weights, both rope tables, the decoder's weights
  and prompt tables), and the trunk and the decoder then give identical
  results, bit for bit.
"""
import numpy as np
import pytest

import backbone_case as bc
import pth_case as pc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    return sam3_hip


@pytest.fixture(scope="module", params=["fp32", "bf16", "fp16"])
def be(hip, request):
    b = hip.Backend(precision=request.param)
    b.precision = request.param
    yield b
    b.free()


def special_values(g, n):
    """Normal values plus the edge cases of the three formats."""
    v = g.standard_normal(n).astype(np.float32) * 3
    edge = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 1e6,
                     6e-8, 3e-8, 1e-40, -1e-40, 1.0 + 2 ** -11, 1.0 + 2 ** -8,
                     3.0e38, 1.0 + 3 * 2 ** -11], np.float32)
    v[:len(edge)] = edge
    return v


def test_pth_upload_types_and_views(hip, be, tmp_path):
    import torch
    g = np.random.default_rng(5)
    base = torch.from_numpy(special_values(g, 6 * 40).reshape(6, 40))
    sd = {"f32": base, "f32_t": base.t(), "f32_cols": base[:, 5:30],
          "f16": base.half(), "f16_t": base.half().t(),
          "bf16": base.bfloat16(), "bf16_rows": base.bfloat16()[1:4],
          "c64": torch.randn(12, 32, dtype=torch.complex64),
          "c64_view": torch.randn(12, 32, dtype=torch.complex64)[::2, 1:]}
    path = str(tmp_path / "up.pt")
    torch.save(sd, path)
    ref = torch.load(path, weights_only=True)
    ck = hip.Checkpoint(path)
    conv = {hip.F32: (torch.float32, np.uint32, hip.F32),
            hip.F16: (torch.float16, np.uint16, hip.F16),
            hip.BF16: (torch.bfloat16, np.uint16, hip.BF16)}
    try:
        for name, t in ref.items():
            if t.is_complex():
                print("pth_upload %s -> f32 pairs" % name, flush=True)
                m = ck.upload(be, name, hip.F32)
                got = be.read(m).view(np.complex64).reshape(t.shape)
                be.release(m)
                assert np.array_equal(got, t.contiguous().numpy())
                continue
            for dt, (tdt, view, _) in conv.items():
                print("pth_upload %s -> %d" % (name, dt), flush=True)
                m = ck.upload(be, name, dt)
                got = be.read(m)
                be.release(m)
                want = t.to(tdt).contiguous().view(
                    torch.int32 if view == np.uint32 else torch.int16)
                assert got.view(view).tobytes() == \
                    want.numpy().view(view).tobytes(), (name, dt)
        with pytest.raises(hip.Sam3HipError, match="is complex, a real tensor "
                                                   "is expected"):
            ck.upload(be, "c64", hip.BF16)
    finally:
        ck.close()


# ------------------------------------------------------------ sam_load

GRID, PS, E, HEADS, MLP, WINDOWS = 8, 4, 128, 2, 256, (4, 0, 4)


def trunk_weights(orc):
    img, pe_w, pos, lnpw, lnpb, blocks = bc.trunk_case(31, GRID, PS, E, MLP,
                                                       WINDOWS)
    pt = 2
    # The checkpoint's pos_embed: a class token row, then the pretraining
    # grid's rows, which the tiled pos repeats.
    g = np.random.default_rng(32)
    rows = [pos[y * GRID + x] for y in range(pt) for x in range(pt)]
    pos_embed = np.concatenate([g.standard_normal((1, E)).astype(np.float32),
                                np.stack(rows)])[None]
    ropes = [orc.rope_table(w if w else GRID) for w in WINDOWS]
    return dict(img=img, pe_w=pe_w, pos=pos, pos_embed=pos_embed, lnpw=lnpw,
                lnpb=lnpb, blocks=blocks, ropes=ropes, E=E, patch=PS)


def manual_model(hip, be, tw):
    blks = []
    for w in tw["blocks"]:
        blk = hip.VitBlock()
        for k in ("n1w", "n1b", "qkvb", "projb", "n2w", "n2b", "l1b", "l2b"):
            setattr(blk, k, be.upload(w[k]))
        for k in ("qkvw", "projw", "l1w", "l2w"):
            setattr(blk, k, be.upload_weight(w[k]))
        blk.window = w["window"]
        blks.append(blk)
    m = hip.Model(be, grid=GRID, embed=E, heads=HEADS, blocks=blks, mlp=MLP)
    m.m.patch = PS
    m.m.pe_w = be.upload_weight(tw["pe_w"])
    m.m.pos, m.m.lnpw, m.m.lnpb = (be.upload(tw["pos"]), be.upload(tw["lnpw"]),
                                   be.upload(tw["lnpb"]))
    m.m.rope_win = be.upload(tw["ropes"][0])
    m.m.rope_glob = be.upload(tw["ropes"][1])
    return m


def same(be, a, b, what):
    ga, gb = be.read(a), be.read(b)
    assert a.contents.dtype == b.contents.dtype, what
    assert ga.tobytes() == gb.tobytes(), what


@pytest.mark.parametrize("storage", ["float32", "bfloat16", "float16"])
def test_sam_load_equals_host_built_model(hip, be, orc, tmp_path, storage):
    import torch
    tw = trunk_weights(orc)
    dw = hip.random_decoder_weights(7)
    if storage != "float32":
        # The host-built model gets the same values rounded to the storage.
        rnd = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)) \
            .to(getattr(torch, storage)).float().numpy()
        tw = dict(tw, pe_w=rnd(tw["pe_w"]), pos=rnd(tw["pos"]),
                  pos_embed=rnd(tw["pos_embed"]), lnpw=rnd(tw["lnpw"]),
                  lnpb=rnd(tw["lnpb"]),
                  blocks=[{k: (rnd(v) if k != "window" else v)
                           for k, v in w.items()} for w in tw["blocks"]])
        dw = {k: rnd(v) for k, v in dw.items()}
    path = str(tmp_path / "sam3.pt")
    pc.save_torch(path, pc.sam3_names(tw, dw), getattr(torch, storage))
    P = 3
    ck = hip.Checkpoint(path)
    print("sam_load storage=%s %s" % (storage, be.precision), flush=True)
    lm = hip.Model.load(be, ck, batch=P, point_head=True)
    mm = manual_model(hip, be, tw)
    dm = hip.Decoder(mm, dw, P, img=GRID * PS)
    dl = lm.decoder()
    try:
        L, M = lm.m, mm.m
        assert (L.grid, L.embed, L.heads, L.hd, L.mlp, L.depth, L.patch) == \
            (GRID, E, HEADS, 64, MLP, len(WINDOWS), PS)
        assert [b.window for b in lm.blocks] == list(WINDOWS)
        for n in ("pe_w", "pos", "lnpw", "lnpb", "rope_win", "rope_glob"):
            same(be, getattr(L, n), getattr(M, n), n)
        for i in range(len(WINDOWS)):
            for n in ("n1w", "n1b", "qkvw", "qkvb", "projw", "projb", "n2w",
                      "n2b", "l1w", "l1b", "l2w", "l2b"):
                same(be, getattr(L.blocks[i], n), getattr(M.blocks[i], n),
                     "block %d %s" % (i, n))
        for n in ("gauss", "point_emb", "not_a_point", "no_mask", "obj_token",
                  "iou_token", "mask_tokens"):
            assert bytes(getattr(dl.d, n)) == bytes(getattr(dm.d, n)), n
        assert dl.d.img == dm.d.img == GRID * PS
        for li in range(2):
            for a in ("self_", "t2i", "i2t"):
                for n in ("qw", "qb", "kw", "kb", "vw", "vb", "ow", "ob"):
                    same(be, getattr(getattr(dl.d.layers[li], a), n),
                         getattr(getattr(dm.d.layers[li], a), n),
                         "layer %d %s %s" % (li, a, n))
        for n in ("nfw", "nfb", "up0w", "up0b", "up1w", "up1b", "up3w", "up3b"):
            same(be, getattr(dl.d, n), getattr(dm.d, n), n)
        for i in range(4):
            for j in range(3):
                same(be, dl.d.hyper_w[i][j], dm.d.hyper_w[i][j], "hyper w")
                same(be, dl.d.hyper_b[i][j], dm.d.hyper_b[i][j], "hyper b")
        # The trunk on one image, then the decoder on one set of features.
        outs = []
        for m in (lm, mm):
            hip.sam_encode_trunk(m, tw["img"])
            be.finish()
            outs.append(be.read(m.m.x, GRID * GRID * E))
        assert outs[0].tobytes() == outs[1].tobytes()
        g = np.random.default_rng(33)
        feats = (g.standard_normal((GRID * GRID, 256)).astype(np.float32),
                 g.standard_normal((16 * GRID * GRID, 32)).astype(np.float32),
                 g.standard_normal((4 * GRID * GRID, 64)).astype(np.float32))
        pts = g.uniform(0, GRID * PS, (P, 2)).astype(np.float32)
        res = []
        for d in (dl, dm):
            d.set_image(*feats)
            res.append((d.decode(pts), d.lowres(P)))
        assert np.array_equal(res[0][0], res[1][0])
        assert np.array_equal(res[0][1], res[1][1])
    finally:
        dm.free()
        mm.free()
        lm.free()
        ck.close()


def test_sam_load_missing_tensor_fails_cleanly(hip, be, orc, tmp_path):
    """A checkpoint without one block weight: sam_load fails with the
    reference's message and releases what it had loaded; the backend
    stays usable."""
    import torch
    tw = trunk_weights(orc)
    sd = pc.sam3_names(tw)
    del sd[pc.TRUNK + ".blocks.2.mlp.fc2.weight"]
    path = str(tmp_path / "partial.pt")
    pc.save_torch(path, sd, torch.float32)
    ck = hip.Checkpoint(path)
    try:
        with pytest.raises(hip.Sam3HipError,
                           match="Tensor <detector.backbone.vision_backbone."
                                 "trunk.blocks.2.mlp.fc2.weight> not found"):
            hip.Model.load(be, ck)
        m = ck.upload(be, pc.TRUNK + ".ln_pre.weight")
        assert np.array_equal(be.read(m), tw["lnpw"])
        be.release(m)
    finally:
        ck.close()
