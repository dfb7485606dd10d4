"""Checkpoint files for the pth_loader tests, written three ways:

- by torch.save itself (the format's owner), for every storage type the
  reader supports, strided views, shared storages and wrapper dicts;
- by a small pickle assembler of this module (GLOBAL opcodes of protocol
  2, persistent storage ids, _rebuild_tensor_v2), the form of the
  reference's own test writer (tests/i_sam3_opencl_test.py:21-97) and of
  deliberately broken files;
- repacked into a zip64 archive by a writer of this module (PKWARE
  APPNOTE 4.3.14-4.3.15, 4.5.3: zip64 end record and locator, sentinel
  0xffffffff / 0xffff fields, extended information extra fields).

sam3_names() maps the random-init trunk and decoder weights of the other
test helpers to the tensor names of a SAM 3 checkpoint
(sam3_model.c:473-583, 657-758).
"""
import struct
import zipfile
import zlib

import numpy as np


# ------------------------------------------------------------ pickles

def p_str(s):
    b = s.encode()
    return b"X" + struct.pack("<I", len(b)) + b


def p_int(i):
    """BININT for 32-bit values, else LONG1 with eight bytes."""
    if -2**31 <= i < 2**31:
        return b"J" + struct.pack("<i", i)
    return b"\x8a\x08" + struct.pack("<q", i)


def p_tuple(items):
    return b"(" + b"".join(items) + b"t"


def p_global(mod, name):
    return b"c" + mod.encode() + b"\n" + name.encode() + b"\n"


def p_tensor(key, storage, offset, shape, stride, numel):
    """REDUCE(torch._utils._rebuild_tensor_v2, (persistent storage,
    offset, size, stride, False, OrderedDict()))."""
    pid = p_tuple([p_str("storage"), p_global("torch", storage), p_str(key),
                   p_str("cpu"), p_int(numel)]) + b"Q"
    args = (b"(" + pid + p_int(offset) + p_tuple([p_int(x) for x in shape]) +
            p_tuple([p_int(x) for x in stride]) + b"\x89" +
            p_global("collections", "OrderedDict") + b")R" + b"t")
    return p_global("torch._utils", "_rebuild_tensor_v2") + args + b"R"


def p_state(entries, wrap=None):
    """Protocol-2 pickle of {name: value} (values already pickled),
    optionally wrapped as {wrap: state}."""
    body = b"}(" + b"".join(p_str(n) + v for n, v in entries) + b"u"
    if wrap:
        body = b"}" + p_str(wrap) + body + b"s"
    return b"\x80\x02" + body + b"."


def write_archive(path, pkl, storages, folder="archive",
                  compression=zipfile.ZIP_STORED):
    """A torch.save-like zip: folder/data.pkl and folder/data/<key>."""
    with zipfile.ZipFile(path, "w", compression=compression) as z:
        z.writestr(folder + "/data.pkl", pkl)
        for key, data in storages.items():
            z.writestr(folder + "/data/" + key, data)


def zeros_checkpoint(path, shapes, wrap="model"):
    """Zero float32 tensors {name: shape}, one storage each, wrapped under
    "model" like the reference test's fixtures."""
    entries, storages = [], {}
    for i, (name, shape) in enumerate(shapes.items()):
        n = int(np.prod(shape))
        stride = [int(np.prod(shape[d + 1:])) for d in range(len(shape))]
        entries.append((name, p_tensor(str(i), "FloatStorage", 0, shape,
                                       stride, n)))
        storages[str(i)] = bytes(4 * n)
    write_archive(path, p_state(entries, wrap), storages)


# ------------------------------------------------------------ zip64

def write_zip64(path, members, pad=0):
    """Stored entries with every size and offset in zip64 form."""
    out = bytearray()
    central = bytearray()
    for name, data in members:
        nb = name.encode()
        crc = zlib.crc32(data)
        off = len(out)
        lx = struct.pack("<HHQQ", 1, 16, len(data), len(data))
        lx += struct.pack("<HH", 0xCAFE, pad) + bytes(pad)
        out += struct.pack("<IHHHHHIIIHH", 0x04034B50, 45, 0, 0, 0, 0, crc,
                           0xFFFFFFFF, 0xFFFFFFFF, len(nb), len(lx))
        out += nb + lx + data
        cx = struct.pack("<HHQQQ", 1, 24, len(data), len(data), off)
        central += struct.pack("<IHHHHHHIIIHHHHHII", 0x02014B50, 45, 45, 0, 0,
                               0, 0, crc, 0xFFFFFFFF, 0xFFFFFFFF, len(nb),
                               len(cx), 0, 0, 0, 0, 0xFFFFFFFF)
        central += nb + cx
    cd_off = len(out)
    out += central
    e64 = len(out)
    out += struct.pack("<IQHHIIQQQQ", 0x06064B50, 44, 45, 45, 0, 0,
                       len(members), len(members), len(central), cd_off)
    out += struct.pack("<IIQI", 0x07064B50, 0, e64, 1)
    out += struct.pack("<IHHHHIIH", 0x06054B50, 0, 0, 0xFFFF, 0xFFFF,
                       0xFFFFFFFF, 0xFFFFFFFF, 0)
    with open(path, "wb") as f:
        f.write(out)


def repack_zip64(src, dst):
    with zipfile.ZipFile(src) as z:
        members = [(i.filename, z.read(i.filename)) for i in z.infolist()]
    write_zip64(dst, members, pad=5)


# ------------------------------------------------------------ SAM 3 names

TRUNK = "detector.backbone.vision_backbone.trunk"
DEC = "tracker.sam_mask_decoder"
PROMPT = "tracker.sam_prompt_encoder"
_ATT_NAMES = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "o": "out_proj"}


def rope_c64(table, hd=64):
    """A rope table [npos][hd/2][2] as the checkpoint's complex
    freqs_cis [npos][hd/2]."""
    t = np.asarray(table, np.float32).reshape(-1, hd // 2, 2)
    return (t[..., 0] + 1j * t[..., 1]).astype(np.complex64)


def sam3_names(trunk=None, dec=None):
    """{checkpoint name: array} of a trunk (pe_w [E][3 p p], pos_embed
    [1][1 + pt^2][E], ln_pre, blocks with their rope tables) and decoder
    weights (random_decoder_weights' names)."""
    sd = {}
    if trunk is not None:
        E, p = trunk["E"], trunk["patch"]
        sd[TRUNK + ".patch_embed.proj.weight"] = \
            trunk["pe_w"].reshape(E, 3, p, p)
        sd[TRUNK + ".pos_embed"] = trunk["pos_embed"]
        sd[TRUNK + ".ln_pre.weight"] = trunk["lnpw"]
        sd[TRUNK + ".ln_pre.bias"] = trunk["lnpb"]
        for i, w in enumerate(trunk["blocks"]):
            b = "%s.blocks.%d." % (TRUNK, i)
            for ours, theirs in (("n1w", "norm1.weight"), ("n1b", "norm1.bias"),
                                 ("n2w", "norm2.weight"), ("n2b", "norm2.bias"),
                                 ("qkvw", "attn.qkv.weight"),
                                 ("qkvb", "attn.qkv.bias"),
                                 ("projw", "attn.proj.weight"),
                                 ("projb", "attn.proj.bias"),
                                 ("l1w", "mlp.fc1.weight"), ("l1b", "mlp.fc1.bias"),
                                 ("l2w", "mlp.fc2.weight"), ("l2b", "mlp.fc2.bias")):
                sd[b + theirs] = w[ours]
            sd[b + "attn.freqs_cis"] = rope_c64(trunk["ropes"][i])
    if dec is not None:
        w = dec
        sd[PROMPT + ".pe_layer.positional_encoding_gaussian_matrix"] = \
            w["gauss"].reshape(2, 128)
        for i in range(4):
            sd[PROMPT + ".point_embeddings.%d.weight" % i] = \
                w["point_emb"][i].reshape(1, 256)
        sd[PROMPT + ".not_a_point_embed.weight"] = w["not_a_point"].reshape(1, 256)
        sd[PROMPT + ".no_mask_embed.weight"] = w["no_mask"].reshape(1, 256)
        sd[DEC + ".obj_score_token.weight"] = w["obj_token"].reshape(1, 256)
        sd[DEC + ".iou_token.weight"] = w["iou_token"].reshape(1, 256)
        sd[DEC + ".mask_tokens.weight"] = w["mask_tokens"].reshape(4, 256)

        def attn(prefix, ours):
            for a, full in _ATT_NAMES.items():
                sd["%s.%s.weight" % (prefix, full)] = w[ours + a + "w"]
                sd["%s.%s.bias" % (prefix, full)] = w[ours + a + "b"]

        tl = DEC + ".transformer.layers"
        for i in range(2):
            attn("%s.%d.self_attn" % (tl, i), "layers.%d.self." % i)
            attn("%s.%d.cross_attn_token_to_image" % (tl, i), "layers.%d.t2i." % i)
            attn("%s.%d.cross_attn_image_to_token" % (tl, i), "layers.%d.i2t." % i)
            for n in range(1, 5):
                sd["%s.%d.norm%d.weight" % (tl, i, n)] = w["layers.%d.n%dw" % (i, n)]
                sd["%s.%d.norm%d.bias" % (tl, i, n)] = w["layers.%d.n%db" % (i, n)]
            for n in (1, 2):
                sd["%s.%d.mlp.lin%d.weight" % (tl, i, n)] = w["layers.%d.m%dw" % (i, n)]
                sd["%s.%d.mlp.lin%d.bias" % (tl, i, n)] = w["layers.%d.m%db" % (i, n)]
        attn(DEC + ".transformer.final_attn_token_to_image", "final_t2i.")
        sd[DEC + ".transformer.norm_final_attn.weight"] = w["nfw"]
        sd[DEC + ".transformer.norm_final_attn.bias"] = w["nfb"]
        sd[DEC + ".output_upscaling.0.weight"] = w["up0w"].reshape(256, 64, 2, 2)
        sd[DEC + ".output_upscaling.0.bias"] = w["up0b"]
        sd[DEC + ".output_upscaling.1.weight"] = w["up1w"]
        sd[DEC + ".output_upscaling.1.bias"] = w["up1b"]
        sd[DEC + ".output_upscaling.3.weight"] = w["up3w"].reshape(64, 32, 2, 2)
        sd[DEC + ".output_upscaling.3.bias"] = w["up3b"]
        for i in range(4):
            for j in range(3):
                pre = "%s.output_hypernetworks_mlps.%d.layers.%d." % (DEC, i, j)
                sd[pre + "weight"] = w["hyper.%d.%dw" % (i, j)]
                sd[pre + "bias"] = w["hyper.%d.%db" % (i, j)]
        for j in range(3):
            pre = "%s.iou_prediction_head.layers.%d." % (DEC, j)
            sd[pre + "weight"] = w["iou.%dw" % j]
            sd[pre + "bias"] = w["iou.%db" % j]
    return sd


def save_torch(path, arrays, dtype=None, wrap=None):
    """torch.save of {name: array} as torch tensors (real arrays cast to
    dtype when given), optionally under {wrap: ...}."""
    import torch
    sd = {}
    for k, a in arrays.items():
        t = torch.from_numpy(np.ascontiguousarray(a))
        if dtype is not None and not t.is_complex():
            t = t.to(dtype)
        sd[k] = t
    torch.save({wrap: sd} if wrap else sd, path)
