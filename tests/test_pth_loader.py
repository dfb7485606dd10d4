"""CPU tests of the checkpoint reader (include/pth_loader.h, the
reference's pth_loader.c:709-1052) through the C ABI.

The oracle is torch itself, the owner of the format: every tensor read
by pth_read_f32 / pth_read_c64 must equal torch.load(weights_only=True)
of the same file bit for bit (float16 and bfloat16 storages over all
65536 bit patterns), with the same shapes, strides and storage offsets.
The reference's own fixture form (protocol-2 GLOBAL opcodes, zero float32
tensors under "model", tests/i_sam3_opencl_test.py:21-97) and zip64
archives are written by tests/pth_case.py; the error paths carry the
reference's messages.
"""
import os
import struct
import zipfile

import numpy as np
import pytest

import pth_case as pc


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    sam3_hip.lib()
    return sam3_hip


def torch_ref(path):
    import torch
    obj = torch.load(path, weights_only=True)
    if "model" in obj and isinstance(obj["model"], dict):
        obj = obj["model"]
    return obj


def check_all(hip, path, ref_path=None):
    """Every tensor of the file against torch.load (of ref_path, the same
    objects saved at protocol 2, where torch's weights-only loader lacks
    the file's opcodes): values bit for bit, shape, stride, storage offset
    and pth_bytes."""
    import torch
    ref = {k: v.detach() for k, v in torch_ref(ref_path or path).items()
           if torch.is_tensor(v)}
    ck = hip.Checkpoint(path)
    try:
        assert ck.names() == list(ref)
        total = 0
        for name, t in ref.items():
            rec = ck.find(name)
            assert ck.shape(rec) == tuple(t.shape), name
            assert tuple(rec.stride[d] for d in range(rec.ndim)) == t.stride()
            assert rec.storage_offset == t.storage_offset()
            if t.is_complex():
                got = ck.read_c64(name)
                assert got.tobytes() == t.contiguous().numpy().tobytes(), name
            else:
                got = ck.read_f32(name)
                want = t.float().contiguous().numpy()
                if t.dtype == torch.float16:
                    # NaNs keep their payload unquieted, as the reference's
                    # half_to_float (pth_loader.c:869-894); torch's
                    # conversion quiets signalling ones.
                    h = t.contiguous().view(torch.int16).numpy().view(np.uint16)
                    nan = (h & 0x7C00) == 0x7C00
                    nan &= (h & 0x3FF) != 0
                    want = want.copy()
                    want.view(np.uint32)[nan] = ((h[nan].astype(np.uint32) &
                                                  0x8000) << 16 | 0x7F800000 |
                                                 (h[nan].astype(np.uint32) &
                                                  0x3FF) << 13)
                    assert np.isnan(want[nan]).all()
                assert got.view(np.uint32).tobytes() == \
                    want.view(np.uint32).tobytes(), name
            total += t.numel() * t.element_size()
        assert ck.bytes("") == total
    finally:
        ck.close()
    return ref


def test_dtypes_and_views(hip, tmp_path):
    import torch
    g = torch.Generator().manual_seed(1)
    base = torch.randn(6, 10, generator=g)
    sd = {
        "f32": torch.randn(3, 4, generator=g),
        "f16": torch.randn(5, 7, generator=g).half(),
        "bf16": torch.randn(2, 3, 4, generator=g).bfloat16(),
        "c64": torch.randn(9, 16, dtype=torch.complex64, generator=g),
        "scalar": torch.tensor(2.5),
        "transposed": base.t(),                 # strides (1, 10)
        "rows": base[2:5],                      # storage offset 20
        "cols": base[:, 3:7],                   # offset + row stride
        "expanded": torch.randn(1, 8, generator=g).expand(4, 8),  # stride 0
        "permuted": torch.randn(2, 3, 5, generator=g).permute(2, 0, 1),
        "c64_view": torch.randn(4, 6, dtype=torch.complex64, generator=g)[:, ::2],
        "f16_t": torch.randn(4, 6, generator=g).half().t(),
        "unit": torch.randn(3, 1, 4, generator=g),
    }
    path = str(tmp_path / "views.pt")
    torch.save(sd, path)
    ref = check_all(hip, path)
    assert ref["rows"].storage_offset() == 20 and ref["expanded"].stride()[0] == 0


def test_half_and_bfloat16_every_bit_pattern(hip, tmp_path):
    """All 65536 float16 and bfloat16 values (zeros, subnormals, normals,
    infinities, NaN payloads) convert as torch's .float() does."""
    import torch
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    path = str(tmp_path / "bits.pt")
    torch.save({"h": bits.clone().view(torch.float16),
                "b": bits.clone().view(torch.bfloat16)}, path)
    check_all(hip, path)


@pytest.mark.parametrize("protocol", [2, 4, 5])
def test_pickle_protocols_and_modules(hip, tmp_path, protocol):
    """torch.save's pickle at protocols 2 (GLOBAL, BINPUT) and 4 / 5
    (FRAME, SHORT_BINUNICODE, STACK_GLOBAL, MEMOIZE); a module state_dict
    (OrderedDict with _metadata: BUILD) and bare parameters
    (_rebuild_parameter)."""
    import torch
    torch.manual_seed(protocol)
    net = torch.nn.Sequential(torch.nn.Linear(8, 16), torch.nn.LayerNorm(16),
                              torch.nn.Linear(16, 4))
    path, p2 = str(tmp_path / "net.pt"), str(tmp_path / "net2.pt")
    params = {n: p for n, p in net.named_parameters()}
    for obj in (net.state_dict(), params):
        torch.save(obj, path, pickle_protocol=protocol)
        torch.save(obj, p2)
        check_all(hip, path, p2)


@pytest.mark.parametrize("wrap", ["model", "state_dict"])
def test_wrapped_state_dict(hip, tmp_path, wrap):
    """A training checkpoint: the weights under "model" / "state_dict",
    other entries (ints, strings, lists, nested dicts) beside them."""
    import torch
    sd = {"w": torch.randn(4, 4), "b": torch.randn(4)}
    path = str(tmp_path / "wrapped.pt")
    torch.save({"epoch": 3, "note": "x", "hist": [1.0, 2.0],
                "opt": {"lr": 0.1}, wrap: sd}, path)
    ck = hip.Checkpoint(path)
    try:
        assert ck.names() == ["w", "b"]
        assert np.array_equal(ck.read_f32("w"), sd["w"].numpy())
    finally:
        ck.close()


def test_non_tensor_values_are_skipped(hip, tmp_path):
    import torch
    path = str(tmp_path / "mixed.pt")
    torch.save({"a": torch.ones(2), "step": 5, "name": "n", "b": torch.zeros(3)},
               path)
    ck = hip.Checkpoint(path)
    try:
        assert ck.names() == ["a", "b"]
    finally:
        ck.close()


def test_reference_fixture_form(hip, tmp_path):
    """The reference test writer's format: protocol 2 with GLOBAL opcodes,
    zero float32 tensors under "model", folder "archive/"."""
    shapes = {"image_encoder.pos_embed": (1, 3, 5),
              "tracker.sam_mask_decoder.iou_token.weight": (1, 256),
              "x.bias": (7,)}
    path = str(tmp_path / "fixture.pt")
    pc.zeros_checkpoint(path, shapes)
    ck = hip.Checkpoint(path)
    try:
        assert ck.names() == list(shapes)
        for n, s in shapes.items():
            assert ck.shape(ck.find(n)) == s
            assert not ck.read_f32(n).any()
        assert ck.find("missing") is None
        assert ck.bytes("tracker.") == 4 * 256
    finally:
        ck.close()


def test_sam3_detection(hip, tmp_path):
    """sam_is_sam3 (sam3_model.c:41-46) on the reference test's kinds of
    fixture: a SAM 3 checkpoint, SAM 1 and SAM 2 checkpoints (which
    main.c:537-550 refuses by their own markers), and a SAM 3 file
    without the point-prompt neck."""
    sam3 = {pc.TRUNK + ".pos_embed": (1, 5, 8),
            pc.DEC + ".iou_token.weight": (1, 256),
            "detector.backbone.vision_backbone.sam2_convs.0.conv_1x1.weight":
                (256, 8, 1, 1)}
    cases = {"sam3": (sam3, True),
             "sam1": ({"image_encoder.pos_embed": (1, 4, 4, 8)}, False),
             "sam2": ({"image_encoder.trunk.pos_embed": (1, 8, 7, 7)}, False),
             "noneck": (dict(list(sam3.items())[:2]), False)}
    for name, (shapes, want) in cases.items():
        path = str(tmp_path / (name + ".pt"))
        pc.zeros_checkpoint(path, shapes)
        ck = hip.Checkpoint(path)
        try:
            assert ck.is_sam3() == want, name
        finally:
            ck.close()


def test_assembled_strided_tensor(hip, tmp_path):
    """A hand-assembled view (offset 3, strides (1, 4)) of one storage
    shared by two tensors, under a folder with another name."""
    data = np.arange(20, dtype=np.float32)
    pkl = pc.p_state([("v", pc.p_tensor("0", "FloatStorage", 3, (4, 3),
                                        (1, 4), 20)),
                      ("all", pc.p_tensor("0", "FloatStorage", 0, (20,),
                                          (1,), 20))])
    path = str(tmp_path / "asm.pt")
    pc.write_archive(path, pkl, {"0": data.tobytes()}, folder="weights_v2")
    ck = hip.Checkpoint(path)
    try:
        want = np.lib.stride_tricks.as_strided(data[3:], (4, 3), (4, 16))
        assert np.array_equal(ck.read_f32("v"), want)
        assert np.array_equal(ck.read_f32("all"), data)
    finally:
        ck.close()


def test_zip64_archive(hip, tmp_path):
    """A torch.save file repacked with zip64 end records and extended
    information fields (sizes and offsets only in the extra fields) reads
    the same; Python's zipfile accepts the repacked archive too."""
    import torch
    src = str(tmp_path / "plain.pt")
    torch.save({"a": torch.randn(5, 3), "h": torch.randn(7).half(),
                "z": torch.randn(3, dtype=torch.complex64)}, src)
    dst = str(tmp_path / "zip64.pt")
    pc.repack_zip64(src, dst)
    with zipfile.ZipFile(dst) as z:
        assert z.testzip() is None
    ref = torch_ref(src)
    ck = hip.Checkpoint(dst)
    try:
        assert np.array_equal(ck.read_f32("a"), ref["a"].numpy())
        assert np.array_equal(ck.read_f32("h"), ref["h"].float().numpy())
        assert np.array_equal(ck.read_c64("z"), ref["z"].numpy())
    finally:
        ck.close()


def test_read_row(hip, tmp_path):
    import torch
    emb = torch.randn(50, 12)
    path = str(tmp_path / "emb.pt")
    torch.save({"emb": emb, "t": emb.t(), "h": emb.half()}, path)
    ck = hip.Checkpoint(path)
    try:
        for r in (0, 17, 49):
            assert np.array_equal(ck.read_row_f32("emb", r), emb[r].numpy())
        with pytest.raises(hip.Sam3HipError, match=r"Row 50 out of range in "
                                                   r"tensor <emb>"):
            ck.read_row_f32("emb", 50)
        for n in ("t", "h"):
            with pytest.raises(hip.Sam3HipError,
                               match="is not a contiguous float32 matrix"):
                ck.read_row_f32(n, 0)
    finally:
        ck.close()


def test_require_and_kind_errors(hip, tmp_path):
    import torch
    path = str(tmp_path / "req.pt")
    torch.save({"w": torch.randn(6, 4), "c": torch.randn(2, dtype=torch.complex64)},
               path)
    ck = hip.Checkpoint(path)
    try:
        assert ck.shape(ck.require("w", 2, (6, 4))) == (6, 4)
        assert ck.shape(ck.require("w", 2, (-1, 4))) == (6, 4)
        assert ck.shape(ck.require("w", 2)) == (6, 4)
        with pytest.raises(hip.Sam3HipError, match="Tensor <x> not found in "
                                                   "checkpoint <.*req.pt>"):
            ck.require("x", 1)
        with pytest.raises(hip.Sam3HipError,
                           match="Tensor <w> has rank 2, expected 3"):
            ck.require("w", 3)
        with pytest.raises(hip.Sam3HipError, match="Tensor <w> has size 4 "
                                                   "along axis 1, expected 5"):
            ck.require("w", 2, (6, 5))
        with pytest.raises(hip.Sam3HipError, match="Tensor <w> is not complex"):
            ck.read_c64("w")
        with pytest.raises(hip.Sam3HipError,
                           match="Tensor <c> is complex, a real tensor is "
                                 "expected"):
            ck.read_f32("c")
    finally:
        ck.close()


def test_load_host_helpers(hip, tmp_path):
    """load_host / load_host_into (sam3_ops.h:36-39) read through
    pth_require."""
    import ctypes
    import torch
    w = torch.randn(3, 5)
    path = str(tmp_path / "host.pt")
    torch.save({"w": w}, path)
    ck = hip.Checkpoint(path)
    L = hip.lib()
    try:
        dst = np.zeros(15, np.float32)
        L.load_host_into(ck.ptr, b"w", 2, (ctypes.c_long * 2)(3, 5),
                         dst.ctypes.data)
        assert np.array_equal(dst.reshape(3, 5), w.numpy())
        p = L.load_host(ck.ptr, b"w", 2, None)
        assert np.array_equal(ck._take(p, 15).reshape(3, 5), w.numpy())
        L.load_host_into(ck.ptr, b"w", 2, (ctypes.c_long * 2)(3, 4),
                         dst.ctypes.data)
        with pytest.raises(hip.Sam3HipError, match="has size 5 along axis 1"):
            hip._check()
    finally:
        ck.close()


# ------------------------------------------------------------ failures

def expect_open_error(hip, path, pattern):
    with pytest.raises(hip.Sam3HipError, match=pattern):
        hip.Checkpoint(str(path))


def test_not_a_checkpoint(hip, tmp_path):
    expect_open_error(hip, tmp_path / "missing.pt", "Unable to open checkpoint")
    p = tmp_path / "text.pt"
    p.write_text("not a zip at all")
    expect_open_error(hip, p, r"is not a zip archive \(PyTorch >= 1.6 "
                              r"checkpoint format expected\)")
    p = tmp_path / "empty.pt"
    p.write_bytes(b"")
    expect_open_error(hip, p, "is not a zip archive")
    p = tmp_path / "other.zip"
    with zipfile.ZipFile(p, "w") as z:
        z.writestr("readme.txt", "hello")
        z.writestr("x/mydata.pkl", "nope")
    expect_open_error(hip, p, "No data.pkl in <.*other.zip>: not a PyTorch "
                              "checkpoint")


def test_compressed_entry_is_refused(hip, tmp_path):
    p = tmp_path / "deflated.pt"
    pc.write_archive(str(p), pc.p_state([("a", pc.p_tensor("0", "FloatStorage",
                                                           0, (4,), (1,), 4))]),
                     {"0": bytes(16)}, compression=zipfile.ZIP_DEFLATED)
    expect_open_error(hip, p, "Zip entry <archive/data.pkl> in <.*> is "
                              "compressed; only stored entries")


def test_unsupported_storage_type(hip, tmp_path):
    import torch
    p = tmp_path / "long.pt"
    torch.save({"w": torch.ones(2), "n": torch.tensor(5)}, str(p))
    expect_open_error(hip, p, r"Unsupported tensor storage type "
                              r"<torch.LongStorage> in checkpoint \(float32, "
                              r"float16, bfloat16 and complex64 are supported\)")


def test_structural_errors(hip, tmp_path):
    good = pc.p_tensor("0", "FloatStorage", 0, (4,), (1,), 4)
    cases = [
        ("missing", pc.p_state([("a", good)]), {},
         r"Storage <archive/data/0> of tensor <a> missing in"),
        ("exceeds", pc.p_state([("a", pc.p_tensor("0", "FloatStorage", 2,
                                                  (4,), (1,), 4))]),
         {"0": bytes(16)}, "Tensor <a> exceeds its storage in"),
        ("empty", pc.p_state([("a", pc.p_tensor("0", "FloatStorage", 0,
                                                (0, 4), (4, 1), 4))]),
         {"0": bytes(16)}, r"Empty tensor <a> in checkpoint"),
        ("notensor", b"\x80\x02}(" + pc.p_str("a") + pc.p_int(1) + b"u.", {},
         "No state_dict of tensors found in"),
        ("truncated", pc.p_state([("a", good)])[:-9], {"0": bytes(16)},
         "Truncated pickle in checkpoint"),
        ("opcode", b"\x80\x02}(" + pc.p_str("a") + b"I1\n" + b"u.", {},
         r"Unsupported pickle opcode 0x49 in checkpoint"),
        ("underflow", b"\x80\x02R.", {}, "Pickle stack underflow"),
        ("nomark", b"\x80\x02}" + pc.p_str("a") + pc.p_int(1) + b"u.", {},
         "Pickle mark not found"),
        ("memo", b"\x80\x02h\x05.", {}, "Invalid pickle memo reference 5"),
        ("memoidx", b"\x80\x02}r\xff\xff\xff\x7f.", {}, "Invalid pickle memo index"),
        ("persid", b"\x80\x02}(" + pc.p_str("a") + pc.p_str("x") + b"Qu.", {},
         "Unsupported persistent id in checkpoint"),
    ]
    for name, pkl, storages, pattern in cases:
        p = tmp_path / (name + ".pt")
        pc.write_archive(str(p), pkl, storages)
        expect_open_error(hip, p, pattern)


def test_view_extent_overflow(hip, tmp_path):
    """Views whose extent arithmetic would overflow 64 bits (huge offset,
    shape x stride, an expanded shape whose element count overflows) or
    that reach before the storage are refused, not wrapped."""
    big = 2 ** 62
    cases = [
        ("offset", 0, (4,), (1,)),
        ("offset_big", big, (4,), (1,)),
        ("negative_offset", -1, (4,), (1,)),
        ("shape_stride", 0, (2 ** 33, 2 ** 33), (2 ** 33, 1)),
        ("reach_wraps", 3, (2, 2), (big, big)),
        ("numel", 0, (2 ** 40, 2 ** 40), (0, 0)),
        ("negative_stride", 3, (4,), (-1,)),
    ]
    for name, off, shape, stride in cases:
        p = tmp_path / (name + ".pt")
        pkl = pc.p_state([("a", pc.p_tensor("0", "FloatStorage", off, shape,
                                            stride, 4))])
        pc.write_archive(str(p), pkl, {"0": bytes(16)})
        if name == "offset":
            ck = hip.Checkpoint(str(p))
            ck.close()
            continue
        expect_open_error(hip, p, "Tensor <a> exceeds its storage in")


def test_truncated_zip(hip, tmp_path):
    import torch
    src = tmp_path / "ok.pt"
    torch.save({"a": torch.randn(100)}, str(src))
    raw = src.read_bytes()
    # Central directory offset pointing past the end of the file.
    eocd = raw.rfind(struct.pack("<I", 0x06054B50))
    bad = bytearray(raw)
    bad[eocd + 16:eocd + 20] = struct.pack("<I", len(raw) + 100)
    p = tmp_path / "cdoff.pt"
    p.write_bytes(bytes(bad))
    expect_open_error(hip, p, "Truncated zip structure in")
    # torch's writer ends with a zip64 end record and its locator: a
    # zip64 sentinel with the locator's signature broken, then with the
    # end record's.
    loc = raw.rfind(struct.pack("<I", 0x07064B50))
    e64 = raw.rfind(struct.pack("<I", 0x06064B50))
    assert loc == eocd - 20 and 0 <= e64 < loc
    for name, at, what in (("noloc", loc, "Corrupt zip64 directory in"),
                           ("noe64", e64, "Corrupt zip64 end record in")):
        bad = bytearray(raw)
        bad[eocd + 10:eocd + 12] = b"\xff\xff"
        bad[at] ^= 0xFF
        p = tmp_path / (name + ".pt")
        p.write_bytes(bytes(bad))
        expect_open_error(hip, p, what)


def test_failed_open_leaves_an_empty_file(hip, tmp_path):
    """After a recorded failure the record is empty and closing it is
    harmless; the next open of a good file works."""
    import ctypes
    import torch
    p = tmp_path / "bad.pt"
    p.write_text("x")
    L = hip.lib()
    f = hip.PthFile()
    L.pth_open(ctypes.byref(f), str(p).encode())
    assert L.hipb_last_error()
    L.hipb_clear_error()
    assert f.ntensors == 0 and not f.map and not f.path
    L.pth_close(ctypes.byref(f))
    good = tmp_path / "good.pt"
    torch.save({"a": torch.ones(3)}, str(good))
    ck = hip.Checkpoint(str(good))
    assert ck.names() == ["a"]
    ck.close()
    assert os.path.exists(good)
