"""Python host mirror of the HIP attention path (libsam3hip.so).

Mirrors the C interface of include/sam3_hip.h, which keeps the names,
argument meaning and error behaviour of the reference's operator API
(sam3_ops.h and the attention helpers of sam3_model.c) and of its
OpenCL backend (ocl_backend.h). Buffers stay on the device; numpy arrays
are only used to move data in and out. Errors raise Sam3HipError with the
message the reference would print before exiting.

There is no CPU fallback: if libsam3hip.so is missing the import of this
module's functions fails.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsam3hip.so")

F32, F16, BF16 = 0, 1, 2
ACT_NONE, ACT_GELU, ACT_RELU = 0, 1, 2
ERR_FATAL, ERR_RECORD = 0, 1

# Every symbol include/sam3_hip.h declares.
EXPORTS = [
    "hipb_init", "hipb_arch_name", "hipb_free", "hipb_errstr", "hipb_check",
    "hipb_alloc", "hipb_alloc_typed", "hipb_upload", "hipb_upload_weight",
    "hipb_is_half", "hipb_round_half", "hipb_write", "hipb_read", "hipb_release", "hipb_finish",
    "hipb_copy", "hipb_set_error_mode", "hipb_last_error", "hipb_clear_error",
    "hipb_prof_count", "hipb_prof_entry", "hipb_prof_reset",
    "hipb_prof_print", "hipb_timer_start", "hipb_timer_stop",
    "sam_path_init", "sam_path_free", "mat", "bmat", "gemm", "linear",
    "layernorm", "add_bcast", "softmax_rows", "rope_apply",
    "window_partition", "window_unpartition_add", "mha", "mha_noalloc",
    "attn_fused",
    "attn_packed", "vit_attention", "vit_block", "sam_encode_trunk",
    "sam_trunk_graph", "softmax_ext", "attend", "sam_dec_init",
    "sam_dec_free", "sam_dec_prepare", "sam_decode", "t2i_attention",
    "i2t_attention", "convt_scatter", "sam_postprocess", "sam_read_mask",
    "sam_dec_graph", "mask_logits", "pth_upload", "load_dev", "load_dev_w",
    "load_dev_fmt", "load_dev_w_fmt", "load_host", "load_host_into",
    "sam_load", "sam_free", "sam_is_sam3",
]
# include/pth_loader.h
PTH_EXPORTS = [
    "pth_open", "pth_find", "pth_require", "pth_numel", "pth_bytes",
    "pth_read_f32", "pth_read_c64", "pth_read_row_f32", "pth_close",
]


class Sam3HipError(RuntimeError):
    pass


class HipbBuf(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("bytes", ctypes.c_size_t),
                ("dtype", ctypes.c_int), ("what", ctypes.c_char_p)]


Mem = ctypes.POINTER(HipbBuf)


class HipbBackend(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int), ("device_name", ctypes.c_char * 256),
                ("arch_name", ctypes.c_char * 64),
                ("max_alloc", ctypes.c_size_t), ("global_mem", ctypes.c_size_t),
                ("cu_count", ctypes.c_int), ("clock_khz", ctypes.c_int),
                ("arch", ctypes.c_int), ("fp16w", ctypes.c_int),
                ("bf16", ctypes.c_int), ("profile", ctypes.c_int),
                ("stream", ctypes.c_void_p), ("ev", ctypes.c_void_p * 2),
                ("scratch", ctypes.c_void_p),
                ("scratch_bytes", ctypes.c_size_t),
                ("stage", ctypes.c_void_p * 2), ("stage_ev", ctypes.c_void_p * 2),
                ("stage_next", ctypes.c_int)]


class Opnd(ctypes.Structure):
    _fields_ = [("buf", Mem), ("off", ctypes.c_long), ("ld", ctypes.c_int),
                ("s0", ctypes.c_long), ("s1", ctypes.c_long)]


class VitBlock(ctypes.Structure):
    _fields_ = [(n, Mem) for n in ("n1w", "n1b", "qkvw", "qkvb", "projw",
                                   "projb", "n2w", "n2b", "l1w", "l1b", "l2w",
                                   "l2b")] + [("window", ctypes.c_int)]


class SamModel(ctypes.Structure):
    _fields_ = [("hip", ctypes.POINTER(HipbBackend)),
                ("embed", ctypes.c_int), ("depth", ctypes.c_int),
                ("heads", ctypes.c_int), ("hd", ctypes.c_int),
                ("mlp", ctypes.c_int), ("grid", ctypes.c_int),
                ("blocks", ctypes.POINTER(VitBlock)),
                ("rope_win", Mem), ("rope_glob", Mem),
                ("score_cap", ctypes.c_long)] + \
        [(n, Mem) for n in ("x", "xn", "xw", "qkv", "scores", "attn", "xn16",
                            "q16", "k16", "vt16", "knorm")] + \
        [("patch", ctypes.c_int)] + \
        [(n, Mem) for n in ("pe_w", "pos", "lnpw", "lnpb", "img", "tmp",
                            "mlpbuf", "mlp16")] + \
        [("trunk_graph", ctypes.c_void_p), ("trunk_exec", ctypes.c_void_p),
         ("trunk_gen", ctypes.c_ulong), ("abias", Mem),
         ("apart", Mem), ("askrec", Mem), ("askcnt", Mem),
         ("dec", ctypes.c_void_p),
         ("owns_weights", ctypes.c_int)]


_FP = ctypes.POINTER(ctypes.c_float)
_ATT = ("qw", "qb", "kw", "kb", "vw", "vb", "ow", "ob")
_LAYER = ("n1w", "n1b", "n2w", "n2b", "n3w", "n3b", "n4w", "n4b", "m1w",
          "m1b", "m2w", "m2b")
_DEC_BUFS = ("emb", "feat_s0", "feat_s1", "src", "pe_img", "srcpe", "kp0",
             "vp0", "qp0", "qpe", "qry", "qin", "sq", "sk", "sv", "so", "sh",
             "keys", "kin", "bq", "bk", "bv", "bo", "u1", "g2", "u2", "hyper",
             "lowres")


class SamAttnW(ctypes.Structure):
    _fields_ = [(n, Mem) for n in _ATT] + [("dint", ctypes.c_int)]


class SamDecLayer(ctypes.Structure):
    _fields_ = [("self_", SamAttnW), ("t2i", SamAttnW), ("i2t", SamAttnW)] + \
        [(n, Mem) for n in _LAYER]


class SamDecoder(ctypes.Structure):
    _fields_ = [("img", ctypes.c_int), ("batch", ctypes.c_int),
                ("gauss", ctypes.c_float * 256),
                ("point_emb", ctypes.c_float * 1024),
                ("not_a_point", ctypes.c_float * 256),
                ("no_mask", ctypes.c_float * 256),
                ("layers", SamDecLayer * 2), ("final_t2i", SamAttnW)] + \
        [(n, Mem) for n in ("nfw", "nfb", "up0w", "up0b", "up1w", "up1b",
                            "up3w", "up3b")] + \
        [("obj_token", ctypes.c_float * 256),
         ("iou_token", ctypes.c_float * 256),
         ("mask_tokens", ctypes.c_float * 1024),
         ("hyper_w", (Mem * 3) * 4), ("hyper_b", (Mem * 3) * 4),
         ("iou_w", Mem * 3), ("iou_b", Mem * 3)] + \
        [(n, Mem) for n in _DEC_BUFS] + \
        [("h_queries", _FP), ("h_lowres", _FP)] + \
        [(n, Mem) for n in ("mask", "sel", "stats")] + \
        [("mask_cap", ctypes.c_size_t)] + \
        [(n, Mem) for n in ("fold_w", "fold_b", "fold_y", "up_w1t",
                            "up_w2t", "t2i_part", "t2i_z", "fold_c", "pe_q1",
                            "pe_k1", "pe_kf")] + \
        [("graph", ctypes.c_void_p), ("graph_exec", ctypes.c_void_p),
         ("graph_P", ctypes.c_int), ("graph_scratch", ctypes.c_void_p)]


# enum pth_dtype (pth_loader.h)
PTH_F32, PTH_F16, PTH_BF16, PTH_C64 = 0, 1, 2, 3
PTH_MAX_DIMS = 8


class PthTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_long * PTH_MAX_DIMS),
                ("stride", ctypes.c_long * PTH_MAX_DIMS),
                ("storage_offset", ctypes.c_long), ("dtype", ctypes.c_int),
                ("data_offset", ctypes.c_long),
                ("storage_bytes", ctypes.c_size_t)]


class PthFile(ctypes.Structure):
    _fields_ = [("map", ctypes.c_void_p), ("map_bytes", ctypes.c_size_t),
                ("path", ctypes.c_char_p), ("ntensors", ctypes.c_int),
                ("tensors", ctypes.POINTER(PthTensor))]


_lib = None


def lib():
    """Load libsam3hip.so (built by build.py); raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise Sam3HipError("libsam3hip.so is not built (run build.py); the "
                           "HIP path has no fallback")
    L = ctypes.CDLL(LIB_PATH)
    c_int, c_long, c_float, c_size = (ctypes.c_int, ctypes.c_long,
                                      ctypes.c_float, ctypes.c_size_t)
    vp, cp = ctypes.c_void_p, ctypes.c_char_p
    BP = ctypes.POINTER(HipbBackend)
    MP = ctypes.POINTER(SamModel)
    L.hipb_init.argtypes = [BP, cp, cp, cp, cp]
    L.hipb_arch_name.argtypes = [c_int]
    L.hipb_arch_name.restype = cp
    L.hipb_free.argtypes = [BP]
    L.hipb_errstr.argtypes = [c_int]
    L.hipb_errstr.restype = cp
    L.hipb_check.argtypes = [c_int, cp]
    L.hipb_alloc.argtypes = [BP, c_size, cp]
    L.hipb_alloc.restype = Mem
    L.hipb_alloc_typed.argtypes = [BP, c_size, c_int, cp]
    L.hipb_alloc_typed.restype = Mem
    L.hipb_upload.argtypes = [BP, vp, c_size, cp]
    L.hipb_upload.restype = Mem
    L.hipb_upload_weight.argtypes = [BP, vp, c_size, cp]
    L.hipb_upload_weight.restype = Mem
    L.hipb_is_half.argtypes = [Mem]
    L.hipb_round_half.argtypes = [vp, vp, c_size, c_int]
    L.hipb_round_half.restype = None
    L.hipb_write.argtypes = [BP, Mem, c_size, vp, c_size]
    L.hipb_read.argtypes = [BP, Mem, c_size, vp, c_size]
    L.hipb_release.argtypes = [ctypes.POINTER(Mem)]
    L.hipb_finish.argtypes = [BP]
    L.hipb_copy.argtypes = [BP, Mem, Mem, c_size, c_size, c_size]
    L.hipb_set_error_mode.argtypes = [c_int]
    L.hipb_last_error.restype = cp
    L.hipb_prof_entry.argtypes = [c_int, ctypes.POINTER(cp),
                                  ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(c_long)]
    L.hipb_timer_start.argtypes = [BP]
    L.hipb_timer_stop.argtypes = [BP]
    L.hipb_timer_stop.restype = c_float
    L.sam_path_init.argtypes = [MP, BP, c_int, c_int, c_int, c_int, c_int,
                                ctypes.POINTER(VitBlock), c_int]
    L.sam_path_free.argtypes = [MP]
    L.mat.argtypes = [Mem, c_long, c_int]
    L.mat.restype = Opnd
    L.bmat.argtypes = [Mem, c_long, c_int, c_long, c_long]
    L.bmat.restype = Opnd
    L.gemm.argtypes = [MP, c_int, c_int, c_int, Opnd, Opnd, c_int, Opnd,
                       c_int, c_int, Mem, Mem, c_long, c_float, c_int]
    L.linear.argtypes = [MP, c_int, c_int, c_int, Mem, c_long, Mem, Mem, Mem,
                         c_long, c_int, c_int]
    L.layernorm.argtypes = [MP, c_long, c_int, Mem, Mem, Mem, Mem, c_float,
                            c_int]
    L.add_bcast.argtypes = [MP, Mem, Mem, Mem, c_long, c_long]
    L.softmax_rows.argtypes = [MP, Mem, c_long, c_int]
    L.softmax_ext.argtypes = [MP, Mem, c_long, c_int, c_int, c_int, c_int, Mem,
                              Mem, c_int, c_int]
    L.attend.argtypes = [MP, c_int, c_int, c_int, c_int, Mem, c_int, Mem, c_int,
                         Mem, c_int, Mem, c_int, c_int, Mem, Mem, c_int]
    L.rope_apply.argtypes = [MP, Mem, c_long, c_int]
    L.window_partition.argtypes = [MP, Mem, Mem, c_int, c_int, c_int, c_int]
    L.window_unpartition_add.argtypes = [MP, Mem, Mem, c_int, c_int, c_int,
                                         c_int]
    L.mha.argtypes = [MP, c_int, c_int, c_int, c_int, Mem, c_long, Mem,
                      c_long, Mem, c_long, Mem]
    L.mha_noalloc.argtypes = L.mha.argtypes
    L.attn_fused.argtypes = [MP, c_int, c_int, c_int, Opnd, Opnd, Opnd, Opnd,
                             Mem, c_int, c_float]
    L.attn_packed.argtypes = [MP, c_int, c_int, c_int, Opnd]
    L.vit_attention.argtypes = [MP, ctypes.POINTER(VitBlock), c_int]
    L.vit_block.argtypes = [MP, ctypes.POINTER(VitBlock), c_int]
    L.sam_encode_trunk.argtypes = [MP, ctypes.c_void_p]
    L.sam_trunk_graph.argtypes = [MP, c_int]
    DP = ctypes.POINTER(SamDecoder)
    L.sam_dec_init.argtypes = [MP, DP, c_int]
    L.sam_dec_free.argtypes = [MP]
    L.sam_dec_prepare.argtypes = [MP]
    L.sam_decode.argtypes = [MP, c_int, vp, vp]
    L.sam_dec_graph.argtypes = [MP, c_int, c_int]
    L.mask_logits.argtypes = [MP, Mem, Mem, Mem, c_int, c_int]
    L.t2i_attention.argtypes = [MP, c_int, ctypes.POINTER(SamAttnW)]
    L.i2t_attention.argtypes = [MP, c_int, c_int]
    L.convt_scatter.argtypes = [MP, Mem, Mem, Mem, Mem, c_int, c_int, c_int,
                                c_int, c_int]
    L.sam_postprocess.argtypes = [MP, c_int, vp, c_int, c_int, c_float, c_int,
                                  vp]
    L.sam_read_mask.argtypes = [MP, c_int, c_int, c_int, c_int, c_int, c_int,
                                c_int, vp]
    FP = ctypes.POINTER(PthFile)
    TP = ctypes.POINTER(PthTensor)
    LP = ctypes.POINTER(c_long)
    L.pth_open.argtypes = [FP, cp]
    L.pth_find.argtypes = [FP, cp]
    L.pth_find.restype = TP
    L.pth_require.argtypes = [FP, cp, c_int, LP]
    L.pth_require.restype = TP
    L.pth_numel.argtypes = [TP]
    L.pth_numel.restype = c_long
    L.pth_bytes.argtypes = [FP, cp]
    L.pth_bytes.restype = ctypes.c_double
    L.pth_read_f32.argtypes = [FP, TP]
    L.pth_read_f32.restype = vp
    L.pth_read_c64.argtypes = [FP, TP]
    L.pth_read_c64.restype = vp
    L.pth_read_row_f32.argtypes = [FP, TP, c_long, vp]
    L.pth_close.argtypes = [FP]
    L.pth_upload.argtypes = [BP, FP, TP, c_int, cp]
    L.pth_upload.restype = Mem
    for n in ("load_dev", "load_dev_w"):
        getattr(L, n).argtypes = [MP, FP, cp, c_int, LP]
        getattr(L, n).restype = Mem
    L.load_host.argtypes = [FP, cp, c_int, LP]
    L.load_host.restype = vp
    L.load_host_into.argtypes = [FP, cp, c_int, LP, vp]
    L.sam_load.argtypes = [MP, BP, FP, c_int, c_int]
    L.sam_free.argtypes = [MP]
    L.sam_is_sam3.argtypes = [FP]
    L.hipb_set_error_mode(ERR_RECORD)
    _lib = L
    return L


def _check():
    msg = _lib.hipb_last_error()
    if msg:
        _lib.hipb_clear_error()
        raise Sam3HipError(msg.decode())


def _np_dtype(dt):
    return {F32: np.float32, F16: np.float16, BF16: np.uint16}[dt]


class Backend:
    """A HIP device and its stream (hipb_init, mirrors ocl_init)."""

    def __init__(self, device="auto", platform=None, profile=None,
                 precision="fp32"):
        L = lib()
        self._b = HipbBackend()
        enc = lambda s: None if s is None else s.encode()
        L.hipb_init(ctypes.byref(self._b), enc(device), enc(platform),
                    enc(profile), enc(precision))
        _check()
        self._mems = []

    @property
    def ptr(self):
        return ctypes.byref(self._b)

    @property
    def bf16(self):
        return bool(self._b.bf16)

    @property
    def fp16w(self):
        return bool(self._b.fp16w)

    @property
    def device_name(self):
        return self._b.device_name.decode()

    @property
    def arch_name(self):
        return self._b.arch_name.decode()

    @property
    def cu_count(self):
        return self._b.cu_count

    def set_profile(self, on):
        self._b.profile = int(bool(on))

    def alloc(self, nbytes, what="buffer"):
        m = _lib.hipb_alloc(self.ptr, nbytes, what.encode())
        _check()
        return m

    def alloc_typed(self, count, dtype, what="buffer"):
        m = _lib.hipb_alloc_typed(self.ptr, count, dtype, what.encode())
        _check()
        return m

    def upload(self, arr, what="buffer"):
        a = np.ascontiguousarray(arr, np.float32)
        m = _lib.hipb_upload(self.ptr, a.ctypes.data, a.nbytes, what.encode())
        _check()
        return m

    def upload_typed(self, arr, dtype, what="buffer"):
        """Upload an array already in the storage type of dtype."""
        a = np.ascontiguousarray(arr, _np_dtype(dtype))
        m = self.alloc_typed(a.size, dtype, what)
        self.write(m, 0, a)
        return m

    def upload_weight(self, arr, what="weight"):
        a = np.ascontiguousarray(arr, np.float32)
        m = _lib.hipb_upload_weight(self.ptr, a.ctypes.data, a.size,
                                    what.encode())
        _check()
        return m

    def write(self, mem, off, arr):
        a = np.ascontiguousarray(arr)
        _lib.hipb_write(self.ptr, mem, off, a.ctypes.data, a.nbytes)
        _check()

    def read(self, mem, count=None, dtype=None, off=0):
        dt = mem.contents.dtype if dtype is None else dtype
        npdt = _np_dtype(dt)
        if count is None:
            count = (mem.contents.bytes - off) // np.dtype(npdt).itemsize
        out = np.empty(count, npdt)
        _lib.hipb_read(self.ptr, mem, off, out.ctypes.data, out.nbytes)
        _check()
        return out

    def read_f32(self, mem, count=None):
        """Read as float32, converting bf16 storage."""
        a = self.read(mem, count)
        if mem.contents.dtype == BF16:
            return (a.astype(np.uint32) << 16).view(np.float32)
        return a.astype(np.float32)

    def release(self, mem):
        """Free mem and set the handle to NULL (hipb_release)."""
        _lib.hipb_release(ctypes.byref(mem))

    def finish(self):
        _lib.hipb_finish(self.ptr)
        _check()

    def copy(self, src, dst, src_off, dst_off, n):
        _lib.hipb_copy(self.ptr, src, dst, src_off, dst_off, n)
        _check()

    def timer_start(self):
        _lib.hipb_timer_start(self.ptr)
        _check()

    def timer_stop(self):
        ms = _lib.hipb_timer_stop(self.ptr)
        _check()
        return ms

    def free(self):
        if self._b.stream:
            _lib.hipb_free(self.ptr)


class Model:
    """struct sam_model for the attention path (sam_path_init)."""

    def __init__(self, backend, grid=0, embed=1024, heads=16, hd=64,
                 blocks=(), mlp=0):
        self.backend = backend
        self.m = SamModel()
        self._blocks = (VitBlock * max(1, len(blocks)))(*blocks)
        if grid:
            _lib.sam_path_init(ctypes.byref(self.m), backend.ptr, grid, embed,
                               heads, hd, mlp, self._blocks, len(blocks))
            _check()
        else:
            self.m.hip = ctypes.pointer(backend._b)
            self.m.embed, self.m.heads, self.m.hd = embed, heads, hd
            # Score buffer capacity as sam_path_init sizes it (floats).
            self.m.score_cap = min(backend._b.max_alloc, 512 << 20) // 4

    @property
    def ptr(self):
        return ctypes.byref(self.m)

    @classmethod
    def load(cls, backend, ckpt, batch=1, point_head=False):
        """sam_load: the trunk (and with point_head the decoder, for batch
        prompts) of the open Checkpoint ckpt, owned by the model."""
        self = cls.__new__(cls)
        self.backend = backend
        self.m = SamModel()
        self._blocks = None
        _lib.sam_load(ctypes.byref(self.m), backend.ptr, ckpt.ptr, batch,
                      int(bool(point_head)))
        msg = _lib.hipb_last_error()
        if msg:
            _lib.hipb_clear_error()
            _lib.sam_free(self.ptr)
            raise Sam3HipError(msg.decode())
        return self

    @property
    def blocks(self):
        return [self.m.blocks[i] for i in range(self.m.depth)]

    def decoder(self):
        """The decoder sam_load attached (a Decoder view owned by the
        model: sam_free releases it)."""
        if not self.m.dec:
            raise Sam3HipError("model has no decoder")
        return Decoder.attached(self)

    def free(self):
        _lib.sam_free(self.ptr)


_libc = ctypes.CDLL(None)
_libc.free.argtypes = [ctypes.c_void_p]


class Checkpoint:
    """An open PyTorch checkpoint (pth_open / pth_close of pth_loader.h)."""

    def __init__(self, path):
        lib()
        self.f = PthFile()
        _lib.pth_open(ctypes.byref(self.f), os.fsencode(path))
        _check()

    @property
    def ptr(self):
        return ctypes.byref(self.f)

    def names(self):
        return [self.f.tensors[i].name.decode()
                for i in range(self.f.ntensors)]

    def find(self, name):
        """pth_find: the tensor record (PthTensor) or None."""
        t = _lib.pth_find(self.ptr, name.encode())
        return t.contents if t else None

    def require(self, name, ndim, shape=None):
        arr = None if shape is None else (ctypes.c_long * ndim)(*shape)
        t = _lib.pth_require(self.ptr, name.encode(), ndim, arr)
        _check()
        return t.contents

    @staticmethod
    def shape(t):
        return tuple(t.shape[d] for d in range(t.ndim))

    def numel(self, t):
        return _lib.pth_numel(ctypes.byref(t))

    def bytes(self, prefix):
        return _lib.pth_bytes(self.ptr, prefix.encode())

    def _get(self, name):
        t = self.find(name)
        if t is None:
            raise Sam3HipError("Tensor <%s> not found in checkpoint <%s>" %
                               (name, self.f.path.decode()))
        return t

    @staticmethod
    def _take(p, count):
        """count floats of a malloc'd array, which is then freed."""
        _check()
        a = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)),
                                  (count,)).copy()
        _libc.free(p)
        return a

    def read_f32(self, name):
        """pth_read_f32: the tensor as float32, C order."""
        t = self._get(name)
        p = _lib.pth_read_f32(self.ptr, ctypes.byref(t))
        return self._take(p, self.numel(t)).reshape(self.shape(t))

    def read_c64(self, name):
        """pth_read_c64: the tensor as complex64, C order."""
        t = self._get(name)
        p = _lib.pth_read_c64(self.ptr, ctypes.byref(t))
        a = self._take(p, 2 * self.numel(t))
        return a.view(np.complex64).reshape(self.shape(t))

    def read_row_f32(self, name, r):
        t = self._get(name)
        out = np.zeros(t.shape[1] if t.ndim == 2 else 0, np.float32)
        _lib.pth_read_row_f32(self.ptr, ctypes.byref(t), r, out.ctypes.data)
        _check()
        return out

    def is_sam3(self):
        """sam_is_sam3: the SAM 3 trunk, mask decoder and point neck."""
        return bool(_lib.sam_is_sam3(self.ptr))

    def upload(self, backend, name, dtype=F32):
        """pth_upload of tensor name into a new device buffer."""
        t = self._get(name)
        m = _lib.pth_upload(backend.ptr, self.ptr, ctypes.byref(t), dtype,
                            name.encode())
        _check()
        return m

    def close(self):
        _lib.pth_close(self.ptr)


def mat(buf, off, ld):
    return Opnd(buf, off, ld, 0, 0)


def bmat(buf, off, ld, s0, s1):
    return Opnd(buf, off, ld, s0, s1)


def _call(fn, *args):
    fn(*args)
    _check()


def gemm(m, M, N, K, A, B, transb, C, nb=1, nb1=1, bias=None, R=None,
         roff=0, alpha=1.0, act=ACT_NONE):
    _call(_lib.gemm, m.ptr, M, N, K, A, B, transb, C, nb, nb1, bias, R, roff,
          alpha, act)


def linear(m, rows, nin, nout, X, xoff, W, b, Y, yoff, act=ACT_NONE,
           residual=0):
    _call(_lib.linear, m.ptr, rows, nin, nout, X, xoff, W, b, Y, yoff, act,
          residual)


def layernorm(m, rows, C, X, Y, g, b, eps=1e-5, act=ACT_NONE):
    _call(_lib.layernorm, m.ptr, rows, C, X, Y, g, b, eps, act)


def add_bcast(m, out, a, b, n, bmod):
    _call(_lib.add_bcast, m.ptr, out, a, b, n, bmod)


def softmax_rows(m, S, rows, L):
    _call(_lib.softmax_rows, m.ptr, S, rows, L)


def softmax_ext(m, S, rows, L, Nq, h0=0, causal=False, dy=None, dx=None, W=0,
                nh=1):
    _call(_lib.softmax_ext, m.ptr, S, rows, L, Nq, h0, int(bool(causal)), dy,
          dx, W, nh)


def attend(m, Nq, Nk, heads, hd, Q, ldq, K, ldk, V, ldv, O, ldo, causal=False,
           dy=None, dx=None, W=0):
    """attend() of the text path (sam3_text.c:305-343) on device buffers."""
    _call(_lib.attend, m.ptr, Nq, Nk, heads, hd, Q, ldq, K, ldk, V, ldv, O, ldo,
          int(bool(causal)), dy, dx, W)


def rope_apply(m, table, rows, npos):
    _call(_lib.rope_apply, m.ptr, table, rows, npos)


def window_partition(m, X, out, H, C, ws, nwx):
    _call(_lib.window_partition, m.ptr, X, out, H, C, ws, nwx)


def window_unpartition_add(m, X, Wd, H, C, ws, nwx):
    _call(_lib.window_unpartition_add, m.ptr, X, Wd, H, C, ws, nwx)


def mha(m, P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv, o):
    _call(_lib.mha, m.ptr, P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv, o)


def mha_noalloc(m, P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv, o):
    _call(_lib.mha_noalloc, m.ptr, P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv, o)


def attn_fused(m, N, nb, nb1, Q, K, V, O, rope=None, npos=1, scale=0.125):
    _call(_lib.attn_fused, m.ptr, N, nb, nb1, Q, K, V, O, rope, npos, scale)


def attn_packed(m, N, nb, nb1, O):
    _call(_lib.attn_packed, m.ptr, N, nb, nb1, O)


def vit_attention(m, block, unfused=False):
    _call(_lib.vit_attention, m.ptr, ctypes.byref(block), int(bool(unfused)))


def vit_block(m, block, unfused=False):
    _call(_lib.vit_block, m.ptr, ctypes.byref(block), int(bool(unfused)))


def sam_encode_trunk(m, img):
    """img: float32 [3, side, side] host array."""
    img = np.ascontiguousarray(img, np.float32)
    _call(_lib.sam_encode_trunk, m.ptr, img.ctypes.data)


def sam_trunk_graph(m, enable=True):
    """Capture the trunk's kernels into a HIP graph that later
    sam_encode_trunk calls replay (enable=False drops it)."""
    _call(_lib.sam_trunk_graph, m.ptr, int(bool(enable)))


def prof_table():
    """Per-kernel profile as a list of (name, ms, wall_ms, flops, calls)."""
    out = []
    for i in range(_lib.hipb_prof_count()):
        w = ctypes.c_char_p()
        ms, wall, fl = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        calls = ctypes.c_long()
        _lib.hipb_prof_entry(i, ctypes.byref(w), ctypes.byref(ms),
                             ctypes.byref(wall), ctypes.byref(fl),
                             ctypes.byref(calls))
        out.append((w.value.decode(), ms.value, wall.value, fl.value,
                    calls.value))
    return out


def prof_reset():
    _lib.hipb_prof_reset()


# ---------------------------------------------------------------- decoder

def random_decoder_weights(seed):
    """Synthetic random-init weights of the point-prompt head's prompt
    encoder and mask decoder, named like the fields of struct sam_decoder
    (no checkpoint is available): Linear / ConvTranspose weights and biases
    U(+-1 / sqrt(fan_in)), LayerNorm weights 1 + 0.1 N(0, 1) and biases
    0.1 N(0, 1), embeddings and the Gaussian matrix N(0, 1)."""
    g = np.random.default_rng(seed)
    f32 = np.float32

    def lin(nout, nin):
        b = 1.0 / np.sqrt(nin)
        return (g.uniform(-b, b, (nout, nin)).astype(f32),
                g.uniform(-b, b, nout).astype(f32))

    def norm(n):
        return ((1 + 0.1 * g.standard_normal(n)).astype(f32),
                (0.1 * g.standard_normal(n)).astype(f32))

    w = {"gauss": g.standard_normal((2, 128)).astype(f32),
         "point_emb": g.standard_normal((4, 256)).astype(f32),
         "not_a_point": g.standard_normal(256).astype(f32),
         "no_mask": g.standard_normal(256).astype(f32),
         "obj_token": g.standard_normal(256).astype(f32),
         "iou_token": g.standard_normal(256).astype(f32),
         "mask_tokens": g.standard_normal((4, 256)).astype(f32)}

    def attn(prefix, dint):
        for n, (o, i) in (("q", (dint, 256)), ("k", (dint, 256)),
                          ("v", (dint, 256)), ("o", (256, dint))):
            w[prefix + n + "w"], w[prefix + n + "b"] = lin(o, i)

    for layer in range(2):
        p = "layers.%d." % layer
        attn(p + "self.", 256)
        attn(p + "t2i.", 128)
        attn(p + "i2t.", 128)
        for k in range(1, 5):
            w[p + "n%dw" % k], w[p + "n%db" % k] = norm(256)
        w[p + "m1w"], w[p + "m1b"] = lin(2048, 256)
        w[p + "m2w"], w[p + "m2b"] = lin(256, 2048)
    attn("final_t2i.", 128)
    w["nfw"], w["nfb"] = norm(256)
    b0, b3 = 1 / 16.0, 1 / 8.0
    w["up0w"] = g.uniform(-b0, b0, (256, 64 * 4)).astype(f32)
    w["up0b"] = g.uniform(-b0, b0, 64).astype(f32)
    w["up1w"], w["up1b"] = norm(64)
    w["up3w"] = g.uniform(-b3, b3, (64, 32 * 4)).astype(f32)
    w["up3b"] = g.uniform(-b3, b3, 32).astype(f32)
    for i in range(4):
        for j in range(3):
            w["hyper.%d.%dw" % (i, j)], w["hyper.%d.%db" % (i, j)] = \
                lin(32 if j == 2 else 256, 256)
    for j in range(3):
        w["iou.%dw" % j], w["iou.%db" % j] = lin(4 if j == 2 else 256, 256)
    return w


class Decoder:
    """struct sam_decoder attached to a Model (sam_dec_init): uploads the
    weights of `w` (random_decoder_weights' names; matrices with
    upload_weight, so bf16 on precision=bf16) and wraps the decoder entry
    points."""

    def __init__(self, model, w, batch, img=1008):
        be = model.backend
        self.model, self.be = model, be
        d = self.d = SamDecoder()
        self._mems = []
        d.img = img

        def dev(name, weight=False):
            a = np.ascontiguousarray(w[name], np.float32)
            mem = be.upload_weight(a, name) if weight else be.upload(a, name)
            self._mems.append(mem)
            return mem

        for name in ("gauss", "point_emb", "not_a_point", "no_mask",
                     "obj_token", "iou_token", "mask_tokens"):
            a = np.ascontiguousarray(w[name], np.float32).ravel()
            ctypes.memmove(getattr(d, name), a.ctypes.data, a.nbytes)

        def attn(dst, prefix, dint):
            for n in _ATT:
                setattr(dst, n, dev(prefix + n, n.endswith("w")))
            dst.dint = dint

        for layer in range(2):
            p = "layers.%d." % layer
            L = d.layers[layer]
            attn(L.self_, p + "self.", 256)
            attn(L.t2i, p + "t2i.", 128)
            attn(L.i2t, p + "i2t.", 128)
            for n in _LAYER:
                setattr(L, n, dev(p + n, n in ("m1w", "m2w")))
        attn(d.final_t2i, "final_t2i.", 128)
        for n in ("nfw", "nfb", "up0b", "up1w", "up1b", "up3b"):
            setattr(d, n, dev(n))
        d.up0w = dev("up0w", True)
        d.up3w = dev("up3w", True)
        for i in range(4):
            for j in range(3):
                d.hyper_w[i][j] = dev("hyper.%d.%dw" % (i, j), True)
                d.hyper_b[i][j] = dev("hyper.%d.%db" % (i, j))
        for j in range(3):
            d.iou_w[j] = dev("iou.%dw" % j, True)
            d.iou_b[j] = dev("iou.%db" % j)
        _call(_lib.sam_dec_init, model.ptr, ctypes.byref(d), batch)
        self.grid = model.m.grid
        self.batch = batch

    @classmethod
    def attached(cls, model):
        """A view of the decoder sam_load attached to model."""
        self = cls.__new__(cls)
        self.model, self.be = model, model.backend
        self.d = ctypes.cast(model.m.dec, ctypes.POINTER(SamDecoder)).contents
        self._mems = []
        self._owned = False
        self.grid = model.m.grid
        self.batch = self.d.batch
        return self

    @property
    def T(self):
        return self.grid * self.grid

    def set_image(self, emb, feat_s0, feat_s1):
        """Upload the image features (emb [grid^2][256], feat_s0 [16
        grid^2][32], feat_s1 [4 grid^2][64]) and run sam_dec_prepare."""
        be, d = self.be, self.d
        for n, a in (("emb", emb), ("feat_s0", feat_s0), ("feat_s1", feat_s1)):
            old = getattr(d, n)
            if old:
                be.release(old)
            setattr(d, n, be.upload(np.ascontiguousarray(a, np.float32), n))
        _call(_lib.sam_dec_prepare, self.model.ptr)

    def decode(self, points):
        """sam_decode; returns iou [P][3]."""
        pts = np.ascontiguousarray(points, np.float32).reshape(-1, 2)
        P = pts.shape[0]
        iou = np.zeros((P, 3), np.float32)
        _call(_lib.sam_decode, self.model.ptr, P, pts.ctypes.data,
              iou.ctypes.data)
        return iou

    def graph(self, P, enable=True):
        """sam_dec_graph: capture (or drop) the device sequence for P."""
        _call(_lib.sam_dec_graph, self.model.ptr, P, int(enable))

    def lowres(self, P):
        L = 4 * self.grid
        return self.be.read_f32(self.d.lowres, P * 3 * L * L).reshape(
            P, 3, L, L)

    def buf(self, name):
        return getattr(self.d, name)

    def postprocess(self, sel, out_h, out_w, offset, fill):
        sel = np.ascontiguousarray(sel, np.int32)
        stats = np.zeros((len(sel), 6), np.int32)
        _call(_lib.sam_postprocess, self.model.ptr, len(sel), sel.ctypes.data,
              out_h, out_w, offset, int(fill), stats.ctypes.data)
        return stats

    def read_mask(self, k, out_h, out_w, x0, y0, x1, y1):
        out = np.zeros((y1 - y0 + 1, x1 - x0 + 1), np.uint8)
        _call(_lib.sam_read_mask, self.model.ptr, k, out_h, out_w, x0, y0, x1,
              y1, out.ctypes.data)
        return out

    def free(self):
        if not getattr(self, "_owned", True):
            return  # the model's sam_free releases it
        _lib.sam_dec_free(self.model.ptr)
        for mem in self._mems + [getattr(self.d, n) for n in ("emb", "feat_s0",
                                                             "feat_s1")]:
            if mem:
                self.be.release(mem)
        self._mems = []
        for n in ("emb", "feat_s0", "feat_s1"):
            setattr(self.d, n, None)


def t2i_attention(m, dec, P, a):
    _call(_lib.t2i_attention, m.ptr, P, ctypes.byref(a))


def i2t_attention(m, layer, P):
    _call(_lib.i2t_attention, m.ptr, layer, P)


def convt_scatter(m, G, out, bias, add, P, H, W, Co, act=ACT_NONE):
    _call(_lib.convt_scatter, m.ptr, G, out, bias, add, P, H, W, Co, act)


def mask_logits(m, U, hyper, out, P, npix):
    _call(_lib.mask_logits, m.ptr, U, hyper, out, P, npix)
