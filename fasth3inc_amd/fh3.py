"""ctypes binding of libfh3hip.so -- the Python mirror of fh3's Q4_K linear
layer interface (reference include/fh3/fh3.h:82-109) and of the HIP module's
C-ABI (include/fh3/fh3_hip.h).

Functions keep the reference names and argument meaning; where the C entry
point returns an FH3_* code, the wrapper raises Fh3Error instead.  Nothing in
this module computes on the CPU: if the library or a GPU is missing, calls
raise.
"""
import ctypes
import gc
import os

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libfh3hip.so")

# GGML type ids (reference include/fh3/fh3.h:63-79)
FH3_QUANT_F32 = 0
FH3_QUANT_F16 = 1
FH3_QUANT_Q8_0 = 8
FH3_QUANT_Q2_K = 10
FH3_QUANT_Q3_K = 11
FH3_QUANT_Q4_K = 12
FH3_QUANT_Q5_K = 13
FH3_QUANT_Q6_K = 14
FH3_QUANT_BF16 = 30

FH3_OK = 0
FH3_ERR = -1
FH3_E_IO = -2
FH3_E_TRUNCATED = -3
FH3_E_BAD_MAGIC = -4
FH3_E_BAD_VERSION = -5
FH3_E_NOT_FOUND = -6
FH3_E_NOMEM = -7
FH3_E_INVALID = -8

PATH_AUTO, PATH_SKINNY, PATH_GEMM, PATH_GEMV8, PATH_MIDM, PATH_SWEEP = 0, 1, 2, 3, 4, 5

Q4K_BLOCK_BYTES = 144
Q4K_BLOCK_WEIGHTS = 256


class Fh3Error(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("%s (code %d)" % (msg, code))
        self.code = code


class Fh3W(ctypes.Structure):
    """struct Fh3W {int type; int64_t in; int64_t out; const uint8_t *data;}"""
    _fields_ = [("type", ctypes.c_int), ("in_", ctypes.c_int64),
                ("out", ctypes.c_int64), ("data", ctypes.c_void_p)]


# FH3P pack and trunk structures (include/fh3/fh3_trunk.h)
LAYER_TENSORS = ("qkv", "gate_compress", "out", "fc1", "fc2", "norm1", "norm2", "q_norm", "k_norm")
FH3_PACK_MAGIC = 0x50334846
FH3_PACK_VERSION = 1
FH3_PACK_ALIGNMENT = 4096
FH3_PACK_MAX_TENSORS_PER_LAYER = 16


class Fh3VsaCfg(ctypes.Structure):       # include/fh3/fh3.h
    _fields_ = [("tile", ctypes.c_int), ("sparsity", ctypes.c_float)]


class Fh3Seq(ctypes.Structure):          # include/fh3/fh3.h (the reference's layout)
    _fields_ = [("seq_len", ctypes.c_int), ("num_text", ctypes.c_int), ("num_audio", ctypes.c_int),
                ("num_video", ctypes.c_int), ("grid_t", ctypes.c_int), ("grid_h", ctypes.c_int),
                ("grid_w", ctypes.c_int), ("tags", ctypes.c_void_p), ("pair_index", ctypes.c_void_p),
                ("pos", ctypes.c_void_p), ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p)]


class Fh3LayerView(ctypes.Structure):
    _fields_ = [(n, Fh3W) for n in LAYER_TENSORS]


class Fh3PackTensorDesc(ctypes.Structure):
    _pack_ = 1
    _fields_ = [("name", ctypes.c_char * 64), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_int64 * 4), ("offset_in_layer", ctypes.c_uint64),
                ("size_bytes", ctypes.c_uint64), ("in_dim", ctypes.c_int64), ("out_dim", ctypes.c_int64),
                ("reserved", ctypes.c_uint8 * 32)]


class Fh3PackLayerDesc(ctypes.Structure):
    _pack_ = 1
    _fields_ = [("file_offset", ctypes.c_uint64), ("size_bytes", ctypes.c_uint64),
                ("n_tensors", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("tensors", Fh3PackTensorDesc * FH3_PACK_MAX_TENSORS_PER_LAYER)]


class Fh3PackHeader(ctypes.Structure):
    _pack_ = 1
    _fields_ = [("magic", ctypes.c_uint32), ("version", ctypes.c_uint32), ("num_layers", ctypes.c_uint32),
                ("layer_alignment", ctypes.c_uint32), ("index_offset", ctypes.c_uint64),
                ("index_bytes", ctypes.c_uint64), ("data_offset", ctypes.c_uint64),
                ("total_bytes", ctypes.c_uint64), ("reserved", ctypes.c_uint8 * 80)]


class Fh3File(ctypes.Structure):         # reference src/io/fh3_portable_io.h:220-224
    _fields_ = [("fd", ctypes.c_int), ("size", ctypes.c_uint64), ("is_direct", ctypes.c_bool)]


class Fh3Pack(ctypes.Structure):         # reference src/io/fh3_pack.h:91-101
    _fields_ = [("file", Fh3File), ("header", Fh3PackHeader),
                ("num_layers", ctypes.c_int), ("layers", ctypes.POINTER(Fh3PackLayerDesc)),
                ("mapped_base", ctypes.c_void_p), ("mapped_size", ctypes.c_size_t)]


class Fh3TrunkStats(ctypes.Structure):
    _fields_ = [("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64), ("bytes_read", ctypes.c_uint64),
                ("read_s", ctypes.c_double), ("wait_s", ctypes.c_double)]


class Fh3TrunkDevStats(ctypes.Structure):
    _fields_ = [("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64), ("uploads", ctypes.c_uint64),
                ("bytes_uploaded", ctypes.c_uint64), ("resident_bytes", ctypes.c_uint64)]


class Fh3TrunkInfo(ctypes.Structure):
    _fields_ = [("num_layers", ctypes.c_int), ("npin", ctypes.c_int), ("slot_size", ctypes.c_uint64),
                ("dpin", ctypes.c_int), ("dev_slot_size", ctypes.c_uint64)]


class Fh3Plan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("budget_bytes", "min_bytes", "pinned_bytes", "ring_bytes",
                                               "activation_bytes", "table_bytes", "total_bytes")]


_c_void_p = ctypes.c_void_p
_c_i64 = ctypes.c_int64
_c_size = ctypes.c_size_t
_c_int = ctypes.c_int
_c_u64 = ctypes.c_uint64
_c_float = ctypes.c_float

# name: (restype, argtypes).  This table is also the list of symbols the
# library must export (checked by tests/test_boundary.py against include/).
SIGNATURES = {
    # fh3.h
    "fh3_row_bytes": (_c_size, [_c_int, _c_i64]),
    "fh3_dequant": (None, [_c_int, _c_void_p, _c_void_p, _c_i64]),
    "fh3_matmul": (None, [ctypes.POINTER(Fh3W), _c_void_p, _c_void_p, _c_int, _c_void_p]),
    "fh3_matmul_scalar": (None, [ctypes.POINTER(Fh3W), _c_void_p, _c_void_p, _c_int, _c_void_p]),
    "fh3_matmul_avx2": (None, [ctypes.POINTER(Fh3W), _c_void_p, _c_void_p, _c_int, _c_void_p]),
    "fh3_attention": (None, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int]),
    "fh3_vsa_attention": (None, [ctypes.POINTER(Fh3VsaCfg), _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                 ctypes.POINTER(Fh3Seq), _c_int, _c_int]),
    # fh3_hip.h
    "fh3_hip_init": (_c_int, [_c_int]),
    "fh3_hip_shutdown": (None, []),
    "fh3_hip_last_error": (ctypes.c_char_p, []),
    "fh3_hip_stream": (_c_void_p, []),
    "fh3_hip_malloc": (_c_int, [ctypes.POINTER(_c_void_p), _c_size]),
    "fh3_hip_free": (_c_int, [_c_void_p]),
    "fh3_hip_memcpy_htod": (_c_int, [_c_void_p, _c_void_p, _c_size]),
    "fh3_hip_memcpy_dtoh": (_c_int, [_c_void_p, _c_void_p, _c_size]),
    "fh3_hip_memcpy_dtod": (_c_int, [_c_void_p, _c_void_p, _c_size]),
    "fh3_hip_memset": (_c_int, [_c_void_p, _c_int, _c_size]),
    "fh3_hip_synchronize": (_c_int, []),
    "fh3_hip_dequant_dev": (_c_int, [_c_int, _c_void_p, _c_void_p, _c_i64, _c_i64, _c_void_p]),
    "fh3_hip_matmul_dev": (_c_int, [ctypes.POINTER(Fh3W), _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p]),
    "fh3_hip_prepared_bytes": (_c_size, [_c_int, _c_i64]),
    "fh3_hip_prepare_x_dev": (_c_int, [_c_void_p, _c_int, _c_i64, _c_void_p, _c_void_p]),
    "fh3_hip_matmul_prepared_dev": (_c_int, [ctypes.POINTER(Fh3W), _c_void_p, _c_void_p, _c_int, _c_void_p,
                                             _c_void_p]),
    "fh3_hip_prepare_x_norm_dev": (_c_int, [_c_void_p, _c_int, _c_i64, _c_void_p, ctypes.c_float, _c_void_p,
                                            _c_void_p, _c_void_p, _c_void_p]),
    "fh3_hip_rownorm_dev": (_c_int, [_c_void_p, _c_int, _c_i64, _c_void_p, ctypes.c_float, _c_void_p, _c_void_p,
                                     _c_void_p, _c_void_p]),
    "fh3_hip_matmul_epi_dev": (_c_int, [ctypes.POINTER(Fh3W), _c_void_p, _c_int, _c_void_p, _c_int, _c_void_p,
                                        _c_void_p, _c_void_p]),
    "fh3_hip_matmul_prepared_epi_dev": (_c_int, [ctypes.POINTER(Fh3W), _c_void_p, _c_int, _c_void_p, _c_int,
                                                 _c_void_p, _c_void_p, _c_void_p]),
    "fh3_hip_attention_dev": (_c_int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_int,
                                       _c_void_p]),
    "fh3_hip_attention_qkv_dev": (_c_int, [_c_void_p, _c_int, _c_int, _c_int, _c_void_p, _c_void_p, ctypes.c_float,
                                           _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p]),
    "fh3_hip_vsa_attention_dev": (_c_int, [ctypes.POINTER(Fh3VsaCfg), _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                           _c_void_p, ctypes.POINTER(Fh3Seq), _c_int, _c_int, _c_void_p]),
    "fh3_hip_vsa_attention_qkv_dev": (_c_int, [ctypes.POINTER(Fh3VsaCfg), _c_void_p, _c_void_p, _c_void_p,
                                               ctypes.c_float, _c_void_p, _c_void_p, _c_int, _c_void_p, _c_void_p,
                                               ctypes.POINTER(Fh3Seq), _c_int, _c_int, _c_void_p]),
    "fh3_hip_register_weights": (_c_int, [_c_void_p, _c_size, ctypes.POINTER(_c_void_p)]),
    "fh3_hip_unregister_weights": (_c_int, [_c_void_p]),
    "fh3_hip_registered_ptr": (_c_void_p, [_c_void_p, _c_size]),
    "fh3_hip_graph_begin": (_c_int, [_c_void_p]),
    "fh3_hip_graph_end": (_c_int, [_c_void_p, ctypes.POINTER(_c_void_p)]),
    "fh3_hip_graph_launch": (_c_int, [_c_void_p, _c_void_p]),
    "fh3_hip_graph_destroy": (_c_int, [_c_void_p]),
    "fh3_hip_matmul_workspace_bytes": (_c_size, [ctypes.POINTER(Fh3W), _c_int, _c_int, _c_int]),
    "fh3_hip_matmul_noalloc_dev": (_c_int, [ctypes.POINTER(Fh3W), _c_void_p, _c_void_p, _c_int, _c_void_p,
                                            _c_void_p]),
    "fh3_hip_set_path": (_c_int, [_c_int]),
    "fh3_hip_skinny_max": (_c_int, []),
    "fh3_hip_matmul_path": (_c_int, [_c_int, _c_i64]),
    # fh3_synth.h
    "fh3_synth_rng_normal": (None, [_c_u64, _c_u64, _c_void_p, _c_size]),
    "fh3_philox4x32_10": (None, [_c_void_p, _c_void_p, _c_void_p]),
    "fh3_rng_uniform": (None, [_c_u64, _c_u64, _c_void_p, _c_size]),
    "fh3_q4k_quantize": (_c_int, [_c_void_p, _c_i64, _c_i64, _c_void_p]),
    "fh3_f32_to_f16": (ctypes.c_uint16, [_c_float]),
    "fh3_synth_q4k_weights": (_c_int, [_c_u64, _c_u64, _c_i64, _c_i64, _c_float, _c_float, _c_void_p]),
    "fh3_synth_x_normal": (None, [_c_u64, _c_u64, _c_void_p, _c_size]),
    "fh3_synth_x_outliers": (None, [_c_u64, _c_u64, _c_void_p, _c_size, _c_float]),
    "fh3_synth_x_silu_gated": (None, [_c_u64, _c_u64, _c_void_p, _c_size]),
    # fh3_trunk.h (struct pointers are passed as addresses)
    "fh3_pack_open": (_c_int, [ctypes.c_char_p, ctypes.POINTER(Fh3Pack)]),
    "fh3_pack_close": (None, [ctypes.POINTER(Fh3Pack)]),
    "fh3_pack_layer": (Fh3LayerView, [ctypes.POINTER(Fh3Pack), _c_int, _c_void_p]),
    "fh3_trunk_open": (_c_int, [ctypes.c_char_p, _c_u64, _c_void_p]),
    "fh3_trunk_close": (None, [_c_void_p]),
    "fh3_trunk_prefetch": (None, [_c_void_p, _c_int]),
    "fh3_trunk_acquire": (_c_void_p, [_c_void_p, _c_int]),
    "fh3_trunk_stats": (Fh3TrunkStats, [_c_void_p]),
    "fh3_trunk_layer": (Fh3LayerView, [_c_void_p, _c_int, _c_void_p]),
    "fh3_trunk_pack": (ctypes.POINTER(Fh3Pack), [_c_void_p]),
    "fh3_trunk_attach_device": (_c_int, [_c_void_p, _c_u64, _c_void_p]),
    "fh3_trunk_prefetch_dev": (None, [_c_void_p, _c_int]),
    "fh3_trunk_acquire_dev": (_c_void_p, [_c_void_p, _c_int]),
    "fh3_trunk_dev_stats": (Fh3TrunkDevStats, [_c_void_p]),
    "fh3_trunk_inject_upload_failure": (_c_int, [_c_void_p, _c_int]),
    "fh3_trunk_struct_bytes": (_c_size, []),
    "fh3_trunk_info": (_c_int, [_c_void_p, ctypes.POINTER(Fh3TrunkInfo)]),
    "fh3_plan_bytes": (_c_u64, [ctypes.POINTER(Fh3Plan)]),
    "fh3_plan_check": (_c_int, [ctypes.POINTER(Fh3Plan)]),
    "fh3_mem_available": (_c_u64, []),
}

_lib = None


def lib():
    """Load libfh3hip.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Fh3Error(FH3_ERR, "libfh3hip.so is not built (%s); run python -m fasth3inc_amd.build"
                           % LIB_PATH)
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _check(rc, what):
    if rc != FH3_OK:
        msg = lib().fh3_hip_last_error()
        raise Fh3Error(rc, "%s: %s" % (what, msg.decode() if msg else ""))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# Reference-named host API
# ---------------------------------------------------------------------------
def row_bytes(qtype, n):
    return lib().fh3_row_bytes(qtype, n)


def dequant(qtype, src, n):
    """fh3_dequant on one row (host bytes -> host fp32, computed on the GPU)."""
    src = np.ascontiguousarray(src, dtype=np.uint8)
    dst = np.zeros(n, dtype=np.float32)
    lib().fh3_dequant(qtype, _p(src), _p(dst), n)
    return dst


def matmul(w_bytes, K, N, x, bias=None, qtype=FH3_QUANT_Q4_K, variant="fh3_matmul"):
    """fh3_matmul on host arrays: y[M][N] = x[M][K] . W^T (+bias)."""
    w_bytes = np.ascontiguousarray(w_bytes, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.full((M, N), np.nan, dtype=np.float32)
    w = Fh3W(qtype, K, N, w_bytes.ctypes.data)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    getattr(lib(), variant)(ctypes.byref(w), _p(x), _p(y), M, None if b is None else _p(b))
    return y


def rng_normal(seed, stream, n):
    out = np.empty(n, dtype=np.float32)
    lib().fh3_synth_rng_normal(seed, stream, _p(out), n)
    return out


# ---------------------------------------------------------------------------
# Device API
# ---------------------------------------------------------------------------
def init(device=0):
    _check(lib().fh3_hip_init(device), "fh3_hip_init")


def shutdown():
    lib().fh3_hip_shutdown()


def stream():
    return lib().fh3_hip_stream()


def synchronize():
    _check(lib().fh3_hip_synchronize(), "fh3_hip_synchronize")


def set_path(path):
    _check(lib().fh3_hip_set_path(path), "fh3_hip_set_path")


def matmul_path(n_tok, k):
    return lib().fh3_hip_matmul_path(n_tok, k)


class DeviceBuffer:
    """A device allocation owned by Python (freed on close / GC)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        _check(lib().fh3_hip_malloc(ctypes.byref(ptr), self.nbytes), "fh3_hip_malloc")
        self.ptr = ptr.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib().fh3_hip_memcpy_htod(self.ptr, _p(a), a.nbytes), "fh3_hip_memcpy_htod")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        _check(lib().fh3_hip_memcpy_dtoh(_p(out), self.ptr, out.nbytes), "fh3_hip_memcpy_dtoh")
        return out

    def fill(self, value=0):
        _check(lib().fh3_hip_memset(self.ptr, value, self.nbytes), "fh3_hip_memset")

    def close(self):
        if self.ptr:
            lib().fh3_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matmul_dev(d_w, K, N, d_x, d_y, n_tok, d_bias=None, stream_ptr=None, qtype=FH3_QUANT_Q4_K):
    """fh3_hip_matmul_dev on device buffers (asynchronous on the stream)."""
    w = Fh3W(qtype, K, N, d_w.ptr if isinstance(d_w, DeviceBuffer) else d_w)
    xp = d_x.ptr if isinstance(d_x, DeviceBuffer) else d_x
    yp = d_y.ptr if isinstance(d_y, DeviceBuffer) else d_y
    bp = None if d_bias is None else (d_bias.ptr if isinstance(d_bias, DeviceBuffer) else d_bias)
    _check(lib().fh3_hip_matmul_dev(ctypes.byref(w), xp, yp, n_tok, bp, stream_ptr), "fh3_hip_matmul_dev")


def _ptr_of(b):
    return None if b is None else (b.ptr if isinstance(b, DeviceBuffer) else b)


def matmul_workspace_bytes(K, N, n_tok, epi=0, prepared=False, qtype=FH3_QUANT_Q4_K):
    """fh3_hip_matmul_workspace_bytes: library workspace a product allocates."""
    w = Fh3W(qtype, K, N, None)
    return lib().fh3_hip_matmul_workspace_bytes(ctypes.byref(w), n_tok, epi, int(prepared))


NOALLOC_SCRATCH_BYTES = 64 << 20   # FH3_HIP_NOALLOC_SCRATCH_BYTES


def matmul_noalloc_dev(d_w, K, N, d_x, d_y, n_tok, d_bias=None, stream_ptr=None, qtype=FH3_QUANT_Q4_K):
    """fh3_hip_matmul_noalloc_dev: fh3_hip_matmul_dev with its workspace in the
    library's fixed scratch array (allocates nothing)."""
    w = Fh3W(qtype, K, N, _ptr_of(d_w))
    _check(lib().fh3_hip_matmul_noalloc_dev(ctypes.byref(w), _ptr_of(d_x), _ptr_of(d_y), n_tok, _ptr_of(d_bias),
                                            stream_ptr), "fh3_hip_matmul_noalloc_dev")


def prepared_bytes(n_tok, K):
    return lib().fh3_hip_prepared_bytes(n_tok, K)


def prepare_x_dev(d_x, n_tok, K, d_prep, stream_ptr=None):
    _check(lib().fh3_hip_prepare_x_dev(_ptr_of(d_x), n_tok, K, _ptr_of(d_prep), stream_ptr),
           "fh3_hip_prepare_x_dev")


def matmul_prepared_dev(d_w, K, N, d_prep, d_y, n_tok, d_bias=None, stream_ptr=None, qtype=FH3_QUANT_Q4_K):
    w = Fh3W(qtype, K, N, _ptr_of(d_w))
    _check(lib().fh3_hip_matmul_prepared_dev(ctypes.byref(w), _ptr_of(d_prep), _ptr_of(d_y), n_tok,
                                             _ptr_of(d_bias), stream_ptr), "fh3_hip_matmul_prepared_dev")


EPI_NONE, EPI_GATE_RESIDUAL, EPI_SWIGLU = 0, 1, 2


def prepare_x_norm_dev(d_x, n_tok, K, d_norm_w, eps, d_prep, d_shift=None, d_scale=None, stream_ptr=None):
    """fh3_hip_prepare_x_norm_dev: rmsnorm (+ modulate) fused into the activation prep."""
    _check(lib().fh3_hip_prepare_x_norm_dev(_ptr_of(d_x), n_tok, K, _ptr_of(d_norm_w), eps, _ptr_of(d_shift),
                                            _ptr_of(d_scale), _ptr_of(d_prep), stream_ptr),
           "fh3_hip_prepare_x_norm_dev")


def rownorm_dev(d_x, n_tok, K, d_norm_w, eps, d_y, d_shift=None, d_scale=None, stream_ptr=None):
    _check(lib().fh3_hip_rownorm_dev(_ptr_of(d_x), n_tok, K, _ptr_of(d_norm_w), eps, _ptr_of(d_shift),
                                     _ptr_of(d_scale), _ptr_of(d_y), stream_ptr), "fh3_hip_rownorm_dev")


def matmul_epi_dev(d_w, K, N, d_x, n_tok, epi, d_out, d_aux=None, d_bias=None, stream_ptr=None,
                   qtype=FH3_QUANT_Q4_K):
    w = Fh3W(qtype, K, N, _ptr_of(d_w))
    _check(lib().fh3_hip_matmul_epi_dev(ctypes.byref(w), _ptr_of(d_x), n_tok, _ptr_of(d_bias), epi,
                                        _ptr_of(d_aux), _ptr_of(d_out), stream_ptr), "fh3_hip_matmul_epi_dev")


def matmul_prepared_epi_dev(d_w, K, N, d_prep, n_tok, epi, d_out, d_aux=None, d_bias=None, stream_ptr=None,
                            qtype=FH3_QUANT_Q4_K):
    w = Fh3W(qtype, K, N, _ptr_of(d_w))
    _check(lib().fh3_hip_matmul_prepared_epi_dev(ctypes.byref(w), _ptr_of(d_prep), n_tok, _ptr_of(d_bias), epi,
                                                 _ptr_of(d_aux), _ptr_of(d_out), stream_ptr),
           "fh3_hip_matmul_prepared_epi_dev")


def attention_dev(d_q, d_k, d_v, d_o, n, heads, hd, stream_ptr=None):
    """fh3_hip_attention_dev: dense attention over [n][heads][hd] device rows."""
    _check(lib().fh3_hip_attention_dev(_ptr_of(d_q), _ptr_of(d_k), _ptr_of(d_v), _ptr_of(d_o), n, heads, hd,
                                       stream_ptr), "fh3_hip_attention_dev")


def attention_qkv_dev(d_qkv, n, heads, hd, d_o, d_qnorm_w=None, d_knorm_w=None, eps=1e-5, d_cos=None, d_sin=None,
                      rot_dim=0, stream_ptr=None):
    """fh3_hip_attention_qkv_dev: q/k rmsnorm + rope3 + attention read in place
    from a qkv projection output [n][3*heads*hd]."""
    _check(lib().fh3_hip_attention_qkv_dev(_ptr_of(d_qkv), n, heads, hd, _ptr_of(d_qnorm_w), _ptr_of(d_knorm_w),
                                           eps, _ptr_of(d_cos), _ptr_of(d_sin), rot_dim, _ptr_of(d_o), stream_ptr),
           "fh3_hip_attention_qkv_dev")


def attention_host(q, k, v):
    """fh3_attention on host arrays [n][heads][hd] (staged through the GPU)."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    o = np.full_like(q, np.nan)
    n, heads, hd = q.shape
    lib().fh3_attention(_p(q), _p(k), _p(v), _p(o), n, heads, hd)
    return o


def seq_of(n, num_text=0, num_audio=0, num_video=None, grid=(0, 0, 0)):
    """An Fh3Seq with the fields the attention calls read."""
    return Fh3Seq(n, num_text, num_audio, n - num_text - num_audio if num_video is None else num_video, *grid,
                  None, None, None, None, None)


def vsa_attention_dev(d_q, d_k, d_v, d_gate, d_o, seq, heads, hd, sparsity=0.8, tile=64, stream_ptr=None):
    """fh3_hip_vsa_attention_dev over [n][heads][hd] device rows; seq an Fh3Seq."""
    cfg = Fh3VsaCfg(tile, sparsity)
    _check(lib().fh3_hip_vsa_attention_dev(ctypes.byref(cfg), _ptr_of(d_q), _ptr_of(d_k), _ptr_of(d_v),
                                           _ptr_of(d_gate), _ptr_of(d_o), ctypes.byref(seq), heads, hd, stream_ptr),
           "fh3_hip_vsa_attention_dev")


def vsa_attention_qkv_dev(d_qkv, d_gate, d_o, seq, heads, hd, sparsity=0.8, tile=64, d_qnorm_w=None,
                          d_knorm_w=None, eps=1e-5, d_cos=None, d_sin=None, rot_dim=0, stream_ptr=None):
    cfg = Fh3VsaCfg(tile, sparsity)
    _check(lib().fh3_hip_vsa_attention_qkv_dev(ctypes.byref(cfg), _ptr_of(d_qkv), _ptr_of(d_qnorm_w),
                                               _ptr_of(d_knorm_w), eps, _ptr_of(d_cos), _ptr_of(d_sin), rot_dim,
                                               _ptr_of(d_gate), _ptr_of(d_o), ctypes.byref(seq), heads, hd,
                                               stream_ptr), "fh3_hip_vsa_attention_qkv_dev")


def vsa_attention_host(q, k, v, gate, seq, sparsity=0.8, tile=64):
    """fh3_vsa_attention on host arrays (staged through the GPU)."""
    q, k, v = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v))
    g = None if gate is None else np.ascontiguousarray(gate, dtype=np.float32)
    o = np.full_like(q, np.nan)
    n, heads, hd = q.shape
    cfg = Fh3VsaCfg(tile, sparsity)
    lib().fh3_vsa_attention(ctypes.byref(cfg), _p(q), _p(k), _p(v), None if g is None else _p(g), _p(o),
                            ctypes.byref(seq), heads, hd)
    return o


def register_weights(host_array):
    """fh3_hip_register_weights on a numpy array (kept alive by the caller);
    returns the device address."""
    d = _c_void_p()
    _check(lib().fh3_hip_register_weights(host_array.ctypes.data, host_array.nbytes, ctypes.byref(d)),
           "fh3_hip_register_weights")
    return d.value


def unregister_weights(host_array):
    _check(lib().fh3_hip_unregister_weights(host_array.ctypes.data), "fh3_hip_unregister_weights")


class Graph:
    """A captured HIP graph of fh3_hip_* calls (see fh3_hip_graph_begin)."""

    def __init__(self, exec_ptr):
        self.ptr = exec_ptr

    def launch(self, stream_ptr=None):
        _check(lib().fh3_hip_graph_launch(self.ptr, stream_ptr), "fh3_hip_graph_launch")

    def close(self):
        if self.ptr:
            lib().fh3_hip_graph_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def capture(fn, stream_ptr=None):
    """Capture the fh3_hip_* work fn() enqueues on the stream into a Graph.

    The garbage collector is run first and paused while fn() records: a
    collection inside the capture could run a DeviceBuffer's or Graph's
    __del__ there, and destroying a graph during a capture ends it."""
    gc.collect()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        _check(lib().fh3_hip_graph_begin(stream_ptr), "fh3_hip_graph_begin")
        ex = ctypes.c_void_p()
        try:
            fn()
        except BaseException:
            # end the capture; the partial graph is of no use
            if lib().fh3_hip_graph_end(stream_ptr, ctypes.byref(ex)) == FH3_OK:
                lib().fh3_hip_graph_destroy(ex.value)
            raise
        _check(lib().fh3_hip_graph_end(stream_ptr, ctypes.byref(ex)), "fh3_hip_graph_end")
    finally:
        if was_enabled:
            gc.enable()
    return Graph(ex.value)


def dequant_dev(d_src, d_dst, rows, n, qtype=FH3_QUANT_Q4_K, stream_ptr=None):
    sp = d_src.ptr if isinstance(d_src, DeviceBuffer) else d_src
    dp = d_dst.ptr if isinstance(d_dst, DeviceBuffer) else d_dst
    _check(lib().fh3_hip_dequant_dev(qtype, sp, dp, rows, n, stream_ptr), "fh3_hip_dequant_dev")


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (host)
# ---------------------------------------------------------------------------
def philox4x32_10(ctr, key):
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().fh3_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def rng_uniform(seed, stream, n):
    out = np.empty(n, dtype=np.float32)
    lib().fh3_rng_uniform(seed, stream, _p(out), n)
    return out


def q4k_quantize(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, n = w.shape
    out = np.zeros(rows * (n // 256) * 144, dtype=np.uint8)
    _check(lib().fh3_q4k_quantize(_p(w), rows, n, _p(out)), "fh3_q4k_quantize")
    return out


def f32_to_f16_bits(f):
    return lib().fh3_f32_to_f16(float(f))


def synth_q4k_weights(seed, stream, rows, n, sigma=0.02, spread_decades=0.0):
    out = np.zeros(rows * (n // 256) * 144, dtype=np.uint8)
    _check(lib().fh3_synth_q4k_weights(seed, stream, rows, n, sigma, spread_decades, _p(out)),
           "fh3_synth_q4k_weights")
    return out


def synth_x(kind, seed, stream, rows, n, frac=0.01):
    x = np.empty((rows, n), dtype=np.float32)
    cnt = rows * n
    if kind == "normal":
        lib().fh3_synth_x_normal(seed, stream, _p(x), cnt)
    elif kind == "outliers":
        lib().fh3_synth_x_outliers(seed, stream, _p(x), cnt, frac)
    elif kind == "silu_gated":
        lib().fh3_synth_x_silu_gated(seed, stream, _p(x), cnt)
    else:
        raise ValueError(kind)
    return x


# ---------------------------------------------------------------------------
# FH3P pack and trunk streamer (include/fh3/fh3_trunk.h)
# ---------------------------------------------------------------------------
def _open_error(what, rc, path):
    return Fh3Error(rc, "%s(%s) failed" % (what, path))


class Pack:
    """An open FH3P pack (fh3_pack_open / fh3_pack_close / fh3_pack_layer)."""

    def __init__(self, path):
        self._p = Fh3Pack()
        rc = lib().fh3_pack_open(os.fsencode(path), ctypes.byref(self._p))
        if rc != FH3_OK:
            raise _open_error("fh3_pack_open", rc, path)
        self._open = True

    @property
    def num_layers(self):
        return self._p.num_layers

    @property
    def header(self):
        return self._p.header

    def layer_desc(self, L):
        if not 0 <= L < self.num_layers:
            raise IndexError(L)
        return self._p.layers[L]

    def layer(self, L, base=None):
        """Fh3LayerView of layer L at base (an address), or into the mapping."""
        return lib().fh3_pack_layer(ctypes.byref(self._p), L, base)

    def close(self):
        if self._open:
            lib().fh3_pack_close(ctypes.byref(self._p))
            self._open = False

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Trunk:
    """The layer streamer (fh3_trunk_open ... fh3_trunk_close), and its device
    extension (attach_device / prefetch_dev / acquire_dev).  acquire* return the
    layer run's address as an int (host or device), or None on a failed read."""

    def __init__(self, path, budget_bytes):
        self._buf = ctypes.create_string_buffer(lib().fh3_trunk_struct_bytes())
        self._t = ctypes.addressof(self._buf)
        rc = lib().fh3_trunk_open(os.fsencode(path), budget_bytes, self._t)
        if rc != FH3_OK:
            raise _open_error("fh3_trunk_open", rc, path)
        self._open = True

    def info(self):
        inf = Fh3TrunkInfo()
        _check(lib().fh3_trunk_info(self._t, ctypes.byref(inf)), "fh3_trunk_info")
        return inf

    def stats(self):
        return lib().fh3_trunk_stats(self._t)

    def dev_stats(self):
        return lib().fh3_trunk_dev_stats(self._t)

    def prefetch(self, L):
        lib().fh3_trunk_prefetch(self._t, L)

    def acquire(self, L):
        return lib().fh3_trunk_acquire(self._t, L)

    def layer(self, L, base=None):
        return lib().fh3_trunk_layer(self._t, L, base)

    def layer_desc(self, L):
        return lib().fh3_trunk_pack(self._t).contents.layers[L]

    def attach_device(self, dev_budget_bytes, stream_ptr=None):
        _check(lib().fh3_trunk_attach_device(self._t, dev_budget_bytes, stream_ptr), "fh3_trunk_attach_device")

    def prefetch_dev(self, L):
        lib().fh3_trunk_prefetch_dev(self._t, L)

    def acquire_dev(self, L):
        return lib().fh3_trunk_acquire_dev(self._t, L)

    def inject_upload_failure(self, what):
        """Test hook: the next slot upload fails at its copy (1) or at its
        ordering event (2); 0 clears."""
        _check(lib().fh3_trunk_inject_upload_failure(self._t, what), "fh3_trunk_inject_upload_failure")

    def close(self):
        if self._open:
            lib().fh3_trunk_close(self._t)
            self._open = False

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def host_bytes(addr, n):
    """numpy uint8 view of n host bytes at addr (no copy)."""
    return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(addr))


def plan(**fields):
    p = Fh3Plan()
    for k, v in fields.items():
        setattr(p, k, v)
    return p


def plan_bytes(p):
    return lib().fh3_plan_bytes(ctypes.byref(p))


def plan_check(p):
    return lib().fh3_plan_check(ctypes.byref(p))


def mem_available():
    return lib().fh3_mem_available()
