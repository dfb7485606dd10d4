"""CPU checks of the C ABI: the library loads, exports every function
include/sam3_hip.h declares, and its host-side error paths behave like
the reference's (fatal with a message naming the call), without a GPU.
"""
import ctypes
import os
import re

import numpy as np

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sam3_hip.h")


PTH_HEADER = os.path.join(ROOT, "include", "pth_loader.h")


def declared_functions(header=HEADER):
    src = open(header).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\([^;{]*\)\s*;", src)
    return sorted(set(n for n in names if n not in ("if", "sizeof")))


@pytest.fixture(scope="module")
def hip():
    import sam3_hip
    sam3_hip.lib()
    return sam3_hip


def test_every_declared_symbol_is_exported(hip):
    names = declared_functions()
    assert len(names) >= 35
    lib = ctypes.CDLL(hip.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(hip.EXPORTS) == names


def test_checkpoint_reader_symbols_are_exported(hip):
    names = declared_functions(PTH_HEADER)
    lib = ctypes.CDLL(hip.LIB_PATH)
    assert not [n for n in names if not hasattr(lib, n)]
    assert sorted(hip.PTH_EXPORTS) == names
    src = re.sub(r"/\*.*?\*/", "", open(PTH_HEADER).read(), flags=re.S)
    for cls, cname in ((hip.PthTensor, "pth_tensor"), (hip.PthFile, "pth_file")):
        body = re.search(r"struct %s \{(.*?)\};" % cname, src, re.S).group(1)
        fields = re.findall(r"([A-Za-z_][A-Za-z0-9_]*)\s*(?:\[[^\]]*\])*\s*;",
                            body)
        assert [f[0] for f in cls._fields_] == fields, cname


def test_struct_layouts_match_header(hip):
    # Field order of the ctypes mirrors, checked against the header text.
    src = open(HEADER).read()
    for cls, cname in ((hip.HipbBuf, "hipb_buf"), (hip.Opnd, "opnd"),
                       (hip.HipbBackend, "hipb_backend"),
                       (hip.VitBlock, "vit_block"), (hip.SamModel, "sam_model"),
                       (hip.SamAttnW, "sam_attn_w"),
                       (hip.SamDecLayer, "sam_dec_layer"),
                       (hip.SamDecoder, "sam_decoder")):
        body = re.search(r"struct %s \{(.*?)\};" % cname, src, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = re.findall(r"([A-Za-z_][A-Za-z0-9_]*)\s*(?:\[[^\]]*\])*\s*[,;]",
                            body)
        # "self" is a Python keyword-like name the mirror spells "self_".
        assert [f[0].rstrip("_") for f in cls._fields_] == fields, cname


def _has_gpu():
    return os.path.exists("/dev/kfd")


def test_invalid_precision_is_fatal(hip):
    with pytest.raises(hip.Sam3HipError, match="Invalid precision option <fp8>"):
        hip.Backend(precision="fp8")


def test_unknown_platform_is_fatal(hip):
    # Mirrors the reference's platform= check (i_sam3_opencl_test.py:369-377).
    with pytest.raises(hip.Sam3HipError,
                       match="no usable auto device found on platforms "
                             "matching no_such_platform"):
        hip.Backend(platform="no_such_platform")


def test_cpu_device_is_refused(hip):
    with pytest.raises(hip.Sam3HipError, match="no usable cpu device"):
        hip.Backend(device="cpu")


@pytest.mark.skipif(_has_gpu(), reason="a GPU is present")
def test_no_device_is_fatal(hip):
    with pytest.raises(hip.Sam3HipError, match="no usable auto device"):
        hip.Backend()


def test_error_is_cleared_after_raise(hip):
    with pytest.raises(hip.Sam3HipError):
        hip.Backend(precision="bogus")
    assert hip.lib().hipb_last_error() is None


def _round_half(hip, x, dtype):
    out = np.empty(x.size, np.uint16)
    hip.lib().hipb_round_half(x.ctypes.data, out.ctypes.data, x.size, dtype)
    return out


def _check_f16(hip, bits):
    x = bits.view(np.float32)
    got = _round_half(hip, x, hip.F16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    bad = (got != want) & ~nan
    assert not bad.any(), hex(int(bits[np.argmax(bad)]))
    g = got[nan]
    assert np.all((g & 0x7c00) == 0x7c00) and np.all(g & 0x3ff)
    assert np.array_equal(g >> 15, (bits[nan] >> 31).astype(np.uint16))


def test_round_half_f16(hip):
    """hipb_round_half to IEEE binary16 (the host rounding of
    hipb_upload_weight with precision=fp16) against numpy's float32 ->
    float16 cast: identical bits for every non-NaN input, a NaN of the
    same sign for every NaN. Every one of the 2^23 mantissas for each
    float32 exponent where a case of the conversion lives (zero and
    subnormal inputs, inputs that round to zero or to binary16 subnormals
    and up to the smallest normal, the overflow boundary at 65520,
    infinities and NaNs: biased exponents 0, 101-113, 142-143 and 255),
    and 2^16 random mantissas of each sign for every exponent."""
    mant = np.arange(1 << 23, dtype=np.uint32)
    g = np.random.default_rng(11)
    full = [0] + list(range(101, 114)) + [142, 143, 255]
    _check_f16(hip, (np.array(full, np.uint32)[:, None] << 23 | mant[None, :]).ravel())
    e = np.arange(256, dtype=np.uint32)[:, None]
    m = g.integers(0, 1 << 23, (256, 1 << 16), dtype=np.uint32)
    for sign in (0, 1):
        _check_f16(hip, (np.uint32(sign << 31) | (e << 23) | m).ravel())


def test_round_half_bf16(hip):
    """hipb_round_half to bfloat16: round to nearest even on the upper 16
    bits (restated in integer numpy arithmetic; NaN stays a NaN of the same
    sign), for all 2^16 low halves under 1024 upper halves: every upper
    half next to a class boundary (zero, the largest finite, infinity,
    NaN, both signs) and random others."""
    g = np.random.default_rng(12)
    ups = np.concatenate([
        np.array([0x0000, 0x0001, 0x007f, 0x0080, 0x3f7f, 0x3f80, 0x7f7e,
                  0x7f7f, 0x7f80, 0x7f81, 0x7fbf, 0x7fc0, 0x7fff], np.uint32),
        g.integers(0, 1 << 15, 499, dtype=np.uint32)])
    ups = np.concatenate([ups, ups | 0x8000])
    low = np.arange(1 << 16, dtype=np.uint32)
    bits = ((ups[:, None] << 16) | low[None, :]).ravel()
    got = _round_half(hip, bits.view(np.float32), hip.BF16)
    up = bits >> 16
    rem = bits & 0xffff
    want = (up + ((rem > 0x8000) | ((rem == 0x8000) & (up & 1 == 1)))).astype(np.uint16)
    nan = (bits & 0x7fffffff) > 0x7f800000
    assert np.array_equal(got[~nan], want[~nan])
    g = got[nan]
    assert np.all((g & 0x7f80) == 0x7f80) and np.all(g & 0x7f)
    assert np.array_equal(g >> 15, (bits[nan] >> 31).astype(np.uint16))
