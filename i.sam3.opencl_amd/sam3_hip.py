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
    "hipb_is_half", "hipb_write", "hipb_read", "hipb_release", "hipb_finish",
    "hipb_copy", "hipb_set_error_mode", "hipb_last_error", "hipb_clear_error",
    "hipb_prof_count", "hipb_prof_entry", "hipb_prof_reset",
    "hipb_prof_print", "hipb_timer_start", "hipb_timer_stop",
    "sam_path_init", "sam_path_free", "mat", "bmat", "gemm", "linear",
    "layernorm", "add_bcast", "softmax_rows", "rope_apply",
    "window_partition", "window_unpartition_add", "mha", "attn_fused",
    "attn_packed", "vit_attention", "vit_block", "sam_encode_trunk",
    "sam_trunk_graph", "softmax_ext", "attend",
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
                ("scratch_bytes", ctypes.c_size_t)]


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
         ("apart", Mem)]


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
    L.attn_fused.argtypes = [MP, c_int, c_int, c_int, Opnd, Opnd, Opnd, Opnd,
                             Mem, c_int, c_float]
    L.attn_packed.argtypes = [MP, c_int, c_int, c_int, Opnd]
    L.vit_attention.argtypes = [MP, ctypes.POINTER(VitBlock), c_int]
    L.vit_block.argtypes = [MP, ctypes.POINTER(VitBlock), c_int]
    L.sam_encode_trunk.argtypes = [MP, ctypes.c_void_p]
    L.sam_trunk_graph.argtypes = [MP, c_int]
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

    def free(self):
        _lib.sam_path_free(self.ptr)


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
