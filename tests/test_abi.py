"""CPU checks of the C ABI: the library loads, exports every function
include/sam3_hip.h declares, and its host-side error paths behave like
the reference's (fatal with a message naming the call), without a GPU.
"""
import ctypes
import os
import re

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
