"""spq4k — Python host binding of libspq4k (the gfx950 Q4_K dequant-matvec).

A thin ctypes layer over the C ABI in include/spq4k.h. The method names
mirror the reference's operator interface for this path (vendored ggml in
nihilistau/shannon-prime-burnhard):

    to_float        ggml_type_traits[type].to_float   (ggml.h:2791-2804)
    from_float      ggml_type_traits_cpu[vec_dot_type].from_float (ggml-cpu.h:113-123)
    quantize_chunk  ggml_quantize_chunk(type, imatrix=NULL) (ggml.h:2764)
    vec_dot         ggml_vec_dot_t for type x vec_dot_type (ggml-cpu.h:113)
    mul_mat         GGML_OP_MUL_MAT                   (ggml.h:1414-1420)
    mul_mat_id      GGML_OP_MUL_MAT_ID                (ggml.h:1434-1438)

`type` is ggml's type id: TYPE_Q4_K (12, the default), TYPE_Q5_K (13),
TYPE_Q6_K (14) or TYPE_Q8_0 (8). The K-quants' vec_dot_type is Q8_K
(256-value blocks); Q8_0's is Q8_0 (32-value blocks).

Every call runs on the GPU through libspq4k.so; if the library is missing
or the device is absent the call raises. There is no CPU fallback.
Numpy arrays go through the *_host entry points; device work uses raw
device pointers (e.g. torch tensor .data_ptr()).
"""
from __future__ import annotations

import ctypes as C
import errno
import os

import numpy as np

QK_K = 256
Q4K_BLOCK_BYTES = 144
Q5K_BLOCK_BYTES = 176
Q6K_BLOCK_BYTES = 210
Q8K_BLOCK_BYTES = 292
QK8_0 = 32
Q8_0_BLOCK_BYTES = 34
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
BLOCK_BYTES = {TYPE_Q4_K: Q4K_BLOCK_BYTES, TYPE_Q5_K: Q5K_BLOCK_BYTES, TYPE_Q6_K: Q6K_BLOCK_BYTES,
               TYPE_Q8_0: Q8_0_BLOCK_BYTES}
BLOCK_VALUES = {TYPE_Q4_K: QK_K, TYPE_Q5_K: QK_K, TYPE_Q6_K: QK_K, TYPE_Q8_0: QK8_0}
GEMV_MAX_T = 8
DIST_NORMAL = 0
DIST_STUDENT_T4 = 1

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libspq4k.so")

_lib = None


class Spq4kError(RuntimeError):
    def __init__(self, fn, rc, msg=""):
        name = errno.errorcode.get(-rc, str(rc)) if rc < 0 else str(rc)
        super().__init__(f"{fn} failed: {name} ({rc}) {msg}".rstrip())
        self.rc = rc


def load_library(path: str | None = None):
    """Load libspq4k.so (built by `make -C shannon-prime-burnhard_amd`)."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise FileNotFoundError(f"libspq4k.so not built: {p} (run __graft_entry__.build())")
    lib = C.CDLL(p)
    V, I, I64, F, S, U64 = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t, C.c_uint64
    PV = C.POINTER(C.c_void_p)
    sig = {
        "spq4k_init": (I, [I, PV]),
        "spq4k_free": (None, [V]),
        "spq4k_set_stream": (I, [V, V]),
        "spq4k_get_stream": (V, [V]),
        "spq4k_synchronize": (I, [V]),
        "spq4k_last_error": (C.c_char_p, [V]),
        "spq4k_device_count": (I, []),
        "spq4k_weights_upload": (I, [V, V, I64, I64, I64, PV]),
        "spq4k_weights_wrap": (I, [V, V, I64, I64, I64, PV]),
        "spq4k_weights_alloc": (I, [V, I64, I64, I64, PV]),
        "spq4k_weights_free": (None, [V]),
        "spq4k_weights_data": (V, [V]),
        "spq4k_weights_nbytes": (S, [V]),
        "spq4k_dequant": (I, [V, V, V, I64]),
        "spq4k_quantize_q8K": (I, [V, V, V, I64]),
        "spq4k_quantize_q4K": (I, [V, V, V, I64, I64]),
        "spq4k_vec_dot": (I, [V, I, V, V, V]),
        "spq4k_dequant_host": (I, [V, V, V, I64]),
        "spq4k_quantize_q8K_host": (I, [V, V, V, I64]),
        "spq4k_quantize_q4K_host": (I, [V, V, V, I64, I64]),
        "spq4k_vec_dot_host": (I, [V, I, V, V, V]),
        "spq4k_gemv": (I, [V, V, V, V, I64]),
        "spq4k_gemv_multi": (I, [V, I, V, V, V, I64]),
        "spq4k_gemm": (I, [V, V, V, V, I64]),
        "spq4k_gemm_multi": (I, [V, I, V, V, V, I64]),
        "spq4k_mul_mat": (I, [V, V, V, V, I64]),
        "spq4k_moe": (I, [V, V, V, I64, I64, I64, V, V]),
        "spq4k_moe_multi": (I, [V, I, PV, V, I64, I64, I64, V, PV]),
        "spq4k_moe_ffn": (I, [V, V, V, V, V, V, I64, I64, V, V]),
        "spq4k_dequant_matvec": (I, [V, V, V, V, I64]),
        "spq4k_stream_read": (I, [V, V, S]),
        "spq4k_dequant_matvec_host": (I, [V, V, V, V, I64]),
        "spq4k_beast_moe_forward": (I, [V, V, V, V, V, I64, V, V, V, V]),
        "spq4k_beast_moe_forward_host": (I, [V, V, V, V, V, I64, V, V, V, V]),
        "spq4k_moe_ffn_host": (I, [V, V, V, V, V, V, I64, I64, V, V]),
        "spq4k_mul_mat_host": (I, [V, V, V, V, I64]),
        "spq4k_moe_host": (I, [V, V, V, I64, I64, I64, V, V]),
        "spq4k_subblock_sums": (I, [V, V, I64, I64, V, V]),
        "spq4k_weights_upload_type": (I, [V, I, V, I64, I64, I64, PV]),
        "spq4k_weights_wrap_type": (I, [V, I, V, I64, I64, I64, PV]),
        "spq4k_ptr_on_device": (I, [V, V, S]),
        "spq4k_weights_alloc_type": (I, [V, I, I64, I64, I64, PV]),
        "spq4k_weights_type": (I, [V]),
        "spq4k_to_float": (I, [V, I, V, V, I64]),
        "spq4k_quantize_chunk": (I, [V, I, V, V, I64, I64]),
        "spq4k_vec_dot_q8K": (I, [V, I, I, V, V, V]),
        "spq4k_to_float_host": (I, [V, I, V, V, I64]),
        "spq4k_quantize_chunk_host": (I, [V, I, V, V, I64, I64]),
        "spq4k_vec_dot_q8K_host": (I, [V, I, I, V, V, V]),
        "spq4k_subblock_sums_type": (I, [V, I, V, I64, I64, V, V]),
        "spq4k_get_device": (I, [V]),
        "spq4k_weights_shape": (I, [V, C.POINTER(I64), C.POINTER(I64), C.POINTER(I64)]),
        "spq4k_model_load": (I, [V, V, I, I, PV]),
        "spq4k_model_free": (None, [V]),
        "spq4k_model_weights": (V, [V, C.c_char_p]),
        "spq4k_model_expert_base": (I, [V, C.c_char_p]),
        "spq4k_model_n_tensors": (I64, [V]),
        "spq4k_model_tensor_name": (C.c_char_p, [V, I64]),
        "spq4k_model_nbytes": (S, [V]),
        "spq4k_rms_norm": (I, [V, V, V, F, V, I64, I64]),
        "spq4k_swiglu": (I, [V, V, V, V, I64]),
        "spq4k_mul_mat_rms_norm": (I, [V, I, V, V, V, F, V, I64]),
        "spq4k_mul_mat_swiglu": (I, [V, V, V, V, V, F, V, I64]),
        "spq4k_quantize_q8_0": (I, [V, V, V, I64]),
        "spq4k_vec_dot_q8_0": (I, [V, I, V, V, V]),
        "spq4k_quantize_q8_0_host": (I, [V, V, V, I64]),
        "spq4k_vec_dot_q8_0_host": (I, [V, I, V, V, V]),
        "spq4k_synth_fill": (I, [V, V, I64, U64, I, I64, F, F, F, I64]),
        "spq4k_reserve": (I, [V, S, S]),
        "spq4k_mul_mat_noalloc": (I, [V, V, V, V, I64]),
        "spq4k_chain_create": (I, [V, C.POINTER(ChainStage), I, F, PV]),
        "spq4k_chain_run": (I, [V, V]),
        "spq4k_chain_status": (I, [V, V]),
        "spq4k_chain_free": (None, [V]),
        "spq4k_chain_info": (I, [V, C.POINTER(I), C.POINTER(I), C.POINTER(I)]),
        "spq4k_chain_set_stamps": (I, [V, V, V]),
        "spq4k_set_decode_stamps": (I, [V, V, S]),
    }
    sig.update(_gguf_sig())
    _bind(lib, sig)
    _lib = lib
    return lib


def _bind(lib, sig):
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def _gguf_sig():
    """the GGUF reader's entry points (include/spq4k_gguf.h)"""
    V, I, I64, S = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
    PV = C.POINTER(C.c_void_p)
    return {
        "spq4k_gguf_open": (I, [C.c_char_p, PV]),
        "spq4k_gguf_close": (None, [V]),
        "spq4k_gguf_strerror": (C.c_char_p, []),
        "spq4k_gguf_version": (C.c_uint32, [V]),
        "spq4k_gguf_alignment": (S, [V]),
        "spq4k_gguf_data_offset": (S, [V]),
        "spq4k_gguf_data_size": (S, [V]),
        "spq4k_gguf_file_size": (S, [V]),
        "spq4k_gguf_n_kv": (I64, [V]),
        "spq4k_gguf_find_key": (I64, [V, C.c_char_p]),
        "spq4k_gguf_key": (C.c_char_p, [V, I64]),
        "spq4k_gguf_kv_type": (I, [V, I64]),
        "spq4k_gguf_arr_type": (I, [V, I64]),
        "spq4k_gguf_arr_n": (I64, [V, I64]),
        "spq4k_gguf_val_data": (V, [V, I64]),
        "spq4k_gguf_val_str": (C.c_char_p, [V, I64, I64]),
        "spq4k_gguf_n_tensors": (I64, [V]),
        "spq4k_gguf_find_tensor": (I64, [V, C.c_char_p]),
        "spq4k_gguf_tensor_name": (C.c_char_p, [V, I64]),
        "spq4k_gguf_tensor_type": (I, [V, I64]),
        "spq4k_gguf_tensor_shape": (I, [V, I64, C.POINTER(C.c_int64)]),
        "spq4k_gguf_tensor_offset": (S, [V, I64]),
        "spq4k_gguf_tensor_nbytes": (S, [V, I64]),
        "spq4k_gguf_tensor_data": (V, [V, I64]),
    }


_gguf_lib = None


def load_gguf_library():
    """The library the GGUF reader is called in: libspq4k.so, or the one the
    SPQ4K_GGUF_LIB environment variable names -- a host-only build of
    csrc/gguf.cpp that exports the same entry points, such as the
    AddressSanitizer / UndefinedBehaviorSanitizer build `make -C oracle asan`
    makes and tests with."""
    global _gguf_lib
    if _gguf_lib is None:
        p = os.environ.get("SPQ4K_GGUF_LIB")
        if p:
            lib = C.CDLL(p)
            _bind(lib, _gguf_sig())
            _gguf_lib = lib
        else:
            _gguf_lib = load_library()
    return _gguf_lib


class ChainStage(C.Structure):
    """spq4k_chain_stage (include/spq4k.h): one stage of a decode chain."""
    _fields_ = [("n", C.c_int), ("glu", C.c_int), ("W", C.c_void_p * 4), ("y", C.c_void_p * 4),
                ("in0", C.c_void_p), ("in1", C.c_void_p), ("x_out", C.c_void_p), ("norm_w", C.c_void_p)]


class Chain:
    """A prepared decode chain (spq4k_chain): dependent T = 1 stages run by one launch."""

    def __init__(self, ctx: "Context", handle, n_stages: int, refs):
        self.ctx, self.handle, self.n_stages = ctx, handle, n_stages
        self._refs = refs   # the Weights the stage table points into

    def run(self):
        """Launch the chain on the context's stream (asynchronous)."""
        self.ctx._check("spq4k_chain_run", self.ctx.lib.spq4k_chain_run(self.ctx.handle, self.handle))

    def status(self):
        """Synchronise; raises (rc -ETIMEDOUT) if a stage wait gave up."""
        self.ctx._check("spq4k_chain_status", self.ctx.lib.spq4k_chain_status(self.ctx.handle, self.handle))

    def info(self):
        """spq4k_chain_info (include/spq4k_diag.h): (form, workgroups, stages)."""
        v, g, n = C.c_int(), C.c_int(), C.c_int()
        rc = self.ctx.lib.spq4k_chain_info(self.handle, C.byref(v), C.byref(g), C.byref(n))
        if rc:
            raise Spq4kError("spq4k_chain_info", rc, "no chain")
        return v.value, g.value, n.value

    @property
    def version(self) -> int:
        return self.info()[0]

    def set_stamps(self, ptr: int | None):
        """spq4k_chain_set_stamps: a device buffer of grid * n_stages * 4 uint64, or None."""
        self.ctx._check("spq4k_chain_set_stamps",
                        self.ctx.lib.spq4k_chain_set_stamps(self.ctx.handle, self.handle, ptr or None))

    def free(self):
        if self.handle:
            self.ctx.lib.spq4k_chain_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("array must be C-contiguous")
        return a.ctypes.data
    if hasattr(a, "data_ptr"):  # torch tensor
        return a.data_ptr()
    raise TypeError(f"cannot take a pointer of {type(a)}")


GGUF_SCALAR = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
               7: np.uint8, 10: np.uint64, 11: np.int64, 12: np.float64}
GGUF_STRING, GGUF_ARRAY = 8, 9


class Gguf:
    """A GGUF model file mapped read-only (include/spq4k_gguf.h): the metadata
    and tensor tables of gguf_init_from_file, tensor bytes as views of the
    mapping. Host only."""

    def __init__(self, path: str):
        self.lib = load_gguf_library()
        h = C.c_void_p()
        rc = self.lib.spq4k_gguf_open(os.fsencode(path), C.byref(h))
        if rc != 0:
            raise Spq4kError("spq4k_gguf_open", rc, self.lib.spq4k_gguf_strerror().decode(errors="replace"))
        self.handle = h
        self.path = path

    def close(self):
        if getattr(self, "handle", None):
            self.lib.spq4k_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def version(self) -> int:
        return self.lib.spq4k_gguf_version(self.handle)

    @property
    def alignment(self) -> int:
        return self.lib.spq4k_gguf_alignment(self.handle)

    @property
    def data_offset(self) -> int:
        return self.lib.spq4k_gguf_data_offset(self.handle)

    @property
    def data_size(self) -> int:
        return self.lib.spq4k_gguf_data_size(self.handle)

    def kv(self) -> list:
        """[(key, type, arr_type, value)]: value a numpy array (non-string
        types, scalars of one element) or a list of str."""
        out = []
        for i in range(self.lib.spq4k_gguf_n_kv(self.handle)):
            key = self.lib.spq4k_gguf_key(self.handle, i).decode()
            t = self.lib.spq4k_gguf_kv_type(self.handle, i)
            at = self.lib.spq4k_gguf_arr_type(self.handle, i) if t == GGUF_ARRAY else -1
            et = at if t == GGUF_ARRAY else t
            n = self.lib.spq4k_gguf_arr_n(self.handle, i)
            if et == GGUF_STRING:
                val = [self.lib.spq4k_gguf_val_str(self.handle, i, j).decode("utf-8", "surrogateescape") for j in range(n)]
            else:
                dt = np.dtype(GGUF_SCALAR[et])
                ptr = self.lib.spq4k_gguf_val_data(self.handle, i)
                val = (np.ctypeslib.as_array((C.c_uint8 * (n * dt.itemsize)).from_address(ptr)).view(dt).copy()
                       if n else np.zeros(0, dt))
            out.append((key, t, at, val))
        return out

    def tensors(self) -> list:
        """[(name, ggml type, ne (4), n_dims, offset, nbytes)] in file order."""
        out = []
        ne = (C.c_int64 * 4)()
        for i in range(self.lib.spq4k_gguf_n_tensors(self.handle)):
            nd = self.lib.spq4k_gguf_tensor_shape(self.handle, i, ne)
            out.append((self.lib.spq4k_gguf_tensor_name(self.handle, i).decode(),
                        self.lib.spq4k_gguf_tensor_type(self.handle, i), tuple(ne), nd,
                        self.lib.spq4k_gguf_tensor_offset(self.handle, i),
                        self.lib.spq4k_gguf_tensor_nbytes(self.handle, i)))
        return out

    def find_tensor(self, name: str) -> int:
        return self.lib.spq4k_gguf_find_tensor(self.handle, name.encode())

    def tensor_bytes(self, i: int) -> np.ndarray:
        """The tensor's bytes as a read-only view of the mapping."""
        n = self.lib.spq4k_gguf_tensor_nbytes(self.handle, i)
        ptr = self.lib.spq4k_gguf_tensor_data(self.handle, i)
        if n == 0:
            return np.zeros(0, np.uint8)
        a = np.ctypeslib.as_array((C.c_uint8 * n).from_address(ptr))
        a.flags.writeable = False
        return a


class Model:
    """Weights of a GGUF file resident on the GPU (spq4k_model_load)."""

    def __init__(self, ctx: "Context", gguf: Gguf, n_gpu_layers: int = -1, experts_on_cpu: int = 0):
        self.ctx = ctx
        self.lib = ctx.lib
        h = C.c_void_p()
        rc = self.lib.spq4k_model_load(ctx.handle, gguf.handle, n_gpu_layers, experts_on_cpu, C.byref(h))
        if rc != 0:
            raise Spq4kError("spq4k_model_load", rc, self.lib.spq4k_gguf_strerror().decode(errors="replace"))
        self.handle = h

    def names(self) -> list:
        return [self.lib.spq4k_model_tensor_name(self.handle, i).decode()
                for i in range(self.lib.spq4k_model_n_tensors(self.handle))]

    @property
    def nbytes(self) -> int:
        return self.lib.spq4k_model_nbytes(self.handle)

    def weights(self, name: str):
        """Weights view of resident tensor `name` (owned by the model), or None."""
        h = self.lib.spq4k_model_weights(self.handle, name.encode())
        if not h:
            return None
        return _ModelWeights(self, h)

    def expert_base(self, name: str) -> int:
        return self.lib.spq4k_model_expert_base(self.handle, name.encode())

    def free(self):
        if getattr(self, "handle", None):
            self.lib.spq4k_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weights:
    """A quantised weight matrix (or an E-expert bank) of one type in device memory."""

    def __init__(self, ctx: "Context", handle, M, K, E, type=TYPE_Q4_K):
        self.ctx, self.handle, self.M, self.K, self.E, self.type = ctx, handle, M, K, E, type

    @property
    def data_ptr(self) -> int:
        return self.ctx.lib.spq4k_weights_data(self.handle)

    @property
    def nbytes(self) -> int:
        return self.ctx.lib.spq4k_weights_nbytes(self.handle)

    def free(self):
        if self.handle:
            self.ctx.lib.spq4k_weights_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class _ModelWeights(Weights):
    """Weights owned by a Model: freed with it, never by this object."""

    def __init__(self, model: "Model", handle):
        lib = model.lib
        M, K, E = C.c_int64(), C.c_int64(), C.c_int64()
        lib.spq4k_weights_shape(handle, C.byref(M), C.byref(K), C.byref(E))
        super().__init__(model.ctx, C.c_void_p(handle), M.value, K.value, E.value, lib.spq4k_weights_type(handle))
        self.model = model   # keeps the model alive while the view is used

    def free(self):
        self.handle = None


class Context:
    """One HIP device + stream (spq4k_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = C.c_void_p()
        rc = self.lib.spq4k_init(device, C.byref(h))
        if rc:
            raise Spq4kError("spq4k_init", rc)
        self.handle = h
        self.device = device

    # -- plumbing
    def _check(self, fn, rc):
        if rc:
            msg = self.lib.spq4k_last_error(self.handle)
            raise Spq4kError(fn, rc, msg.decode() if msg else "")

    def close(self):
        if getattr(self, "handle", None):
            self.lib.spq4k_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        """The hipStream_t work is enqueued on (for events and copies)."""
        return self.lib.spq4k_get_stream(self.handle)

    def set_stream(self, stream_handle: int | None):
        self._check("spq4k_set_stream", self.lib.spq4k_set_stream(self.handle, stream_handle))

    def synchronize(self):
        self._check("spq4k_synchronize", self.lib.spq4k_synchronize(self.handle))

    def reserve(self, scratch_bytes: int, fusion_bytes: int = 0):
        """spq4k_reserve: grow the scratch ahead of a graph capture."""
        self._check("spq4k_reserve", self.lib.spq4k_reserve(self.handle, scratch_bytes, fusion_bytes))

    # -- weights
    def upload(self, q: np.ndarray, M: int, K: int, E: int = 1, type: int = TYPE_Q4_K) -> Weights:
        h = C.c_void_p()
        self._check("spq4k_weights_upload_type",
                    self.lib.spq4k_weights_upload_type(self.handle, type, _ptr(np.ascontiguousarray(q)), M, K, E,
                                                       C.byref(h)))
        return Weights(self, h, M, K, E, type)

    def wrap(self, dev_ptr: int, M: int, K: int, E: int = 1, type: int = TYPE_Q4_K) -> Weights:
        h = C.c_void_p()
        self._check("spq4k_weights_wrap_type",
                    self.lib.spq4k_weights_wrap_type(self.handle, type, dev_ptr, M, K, E, C.byref(h)))
        return Weights(self, h, M, K, E, type)

    def alloc_weights(self, M: int, K: int, E: int = 1, type: int = TYPE_Q4_K) -> Weights:
        h = C.c_void_p()
        self._check("spq4k_weights_alloc_type",
                    self.lib.spq4k_weights_alloc_type(self.handle, type, M, K, E, C.byref(h)))
        return Weights(self, h, M, K, E, type)

    def load_model(self, gguf: Gguf, n_gpu_layers: int = -1, experts_on_cpu: int = 0) -> Model:
        return Model(self, gguf, n_gpu_layers, experts_on_cpu)

    # -- type traits on host arrays (synchronous)
    def to_float(self, q: np.ndarray, k: int, type: int = TYPE_Q4_K) -> np.ndarray:
        y = np.empty(k, np.float32)
        self._check("spq4k_to_float_host", self.lib.spq4k_to_float_host(self.handle, type, _ptr(q), _ptr(y), k))
        return y

    def from_float(self, x: np.ndarray, type: int = TYPE_Q4_K) -> np.ndarray:
        """Activations to the vec_dot_type of weight type `type` (Q8_K, or Q8_0 for TYPE_Q8_0)."""
        x = np.ascontiguousarray(x, np.float32).ravel()
        if type == TYPE_Q8_0:
            y = np.zeros(x.size // QK8_0 * Q8_0_BLOCK_BYTES, np.uint8)
            self._check("spq4k_quantize_q8_0_host",
                        self.lib.spq4k_quantize_q8_0_host(self.handle, _ptr(x), _ptr(y), x.size))
            return y
        y = np.zeros(x.size // QK_K * Q8K_BLOCK_BYTES, np.uint8)
        self._check("spq4k_quantize_q8K_host",
                    self.lib.spq4k_quantize_q8K_host(self.handle, _ptr(x), _ptr(y), x.size))
        return y

    def quantize_chunk(self, src: np.ndarray, nrow: int, n_per_row: int, type: int = TYPE_Q4_K) -> np.ndarray:
        src = np.ascontiguousarray(src, np.float32).ravel()
        y = np.zeros(nrow * (n_per_row // BLOCK_VALUES[type]) * BLOCK_BYTES[type], np.uint8)
        self._check("spq4k_quantize_chunk_host",
                    self.lib.spq4k_quantize_chunk_host(self.handle, type, _ptr(src), _ptr(y), nrow, n_per_row))
        return y

    def vec_dot(self, n: int, vx: np.ndarray, vy: np.ndarray, type: int = TYPE_Q4_K) -> float:
        s = C.c_float()
        if type == TYPE_Q8_0:
            self._check("spq4k_vec_dot_q8_0_host",
                        self.lib.spq4k_vec_dot_q8_0_host(self.handle, n, C.byref(s), _ptr(vx), _ptr(vy)))
            return s.value
        self._check("spq4k_vec_dot_q8K_host",
                    self.lib.spq4k_vec_dot_q8K_host(self.handle, type, n, C.byref(s), _ptr(vx), _ptr(vy)))
        return s.value

    def mul_mat(self, W: Weights, X: np.ndarray) -> np.ndarray:
        X = np.ascontiguousarray(X, np.float32).reshape(-1, W.K)
        Y = np.empty((X.shape[0], W.M), np.float32)
        self._check("spq4k_mul_mat_host",
                    self.lib.spq4k_mul_mat_host(self.handle, W.handle, _ptr(X), _ptr(Y), X.shape[0]))
        return Y

    def mul_mat_id(self, bank: Weights, X: np.ndarray, ids: np.ndarray) -> np.ndarray:
        """X: [T, ne11, K] with ne11 in {1, n_used}; ids: [T, n_used] int32 -> Y [T, n_used, M]."""
        ids = np.ascontiguousarray(ids, np.int32)
        T, n_used = ids.shape
        X = np.ascontiguousarray(X, np.float32).reshape(T, -1, bank.K)
        ne11 = X.shape[1]
        Y = np.empty((T, n_used, bank.M), np.float32)
        self._check("spq4k_moe_host", self.lib.spq4k_moe_host(self.handle, bank.handle, _ptr(ids), n_used, ne11, T,
                                                              _ptr(X), _ptr(Y)))
        return Y

    def subblock_sums(self, W_dev: int, M: int, K: int, x_dev: int, S_dev: int, type: int = TYPE_Q4_K):
        self._check("spq4k_subblock_sums_type",
                    self.lib.spq4k_subblock_sums_type(self.handle, type, W_dev, M, K, x_dev, S_dev))

    # -- device-pointer entry points (asynchronous on the context stream)
    def gemv_dev(self, W: Weights, x_dev: int, y_dev: int, T: int = 1):
        self._check("spq4k_gemv", self.lib.spq4k_gemv(self.handle, W.handle, x_dev, y_dev, T))

    def gemv_multi_dev(self, Ws, x_dev: int, y_devs, T: int = 1):
        n = len(Ws)
        wa = (C.c_void_p * n)(*[w.handle.value if isinstance(w.handle, C.c_void_p) else w.handle for w in Ws])
        ya = (C.c_void_p * n)(*y_devs)
        self._check("spq4k_gemv_multi", self.lib.spq4k_gemv_multi(self.handle, n, wa, x_dev, ya, T))

    def gemm_dev(self, W: Weights, X_dev: int, Y_dev: int, T: int):
        self._check("spq4k_gemm", self.lib.spq4k_gemm(self.handle, W.handle, X_dev, Y_dev, T))

    def gemm_multi_dev(self, Ws, X_dev: int, Y_devs, T: int):
        n = len(Ws)
        wa = (C.c_void_p * n)(*[w.handle.value if isinstance(w.handle, C.c_void_p) else w.handle for w in Ws])
        ya = (C.c_void_p * n)(*Y_devs)
        self._check("spq4k_gemm_multi", self.lib.spq4k_gemm_multi(self.handle, n, wa, X_dev, ya, T))

    def mul_mat_dev(self, W: Weights, X_dev: int, Y_dev: int, T: int):
        self._check("spq4k_mul_mat", self.lib.spq4k_mul_mat(self.handle, W.handle, X_dev, Y_dev, T))

    def moe_dev(self, bank: Weights, ids_dev: int, n_used: int, ne11: int, T: int, X_dev: int, Y_dev: int):
        self._check("spq4k_moe", self.lib.spq4k_moe(self.handle, bank.handle, ids_dev, n_used, ne11, T, X_dev, Y_dev))

    def moe_multi_dev(self, banks, ids_dev: int, n_used: int, ne11: int, T: int, X_dev: int, Y_devs):
        """spq4k_moe_multi: banks sharing ids and input (gate and up), Y_devs[i] per bank."""
        n = len(banks)
        hb = (C.c_void_p * n)(*[b.handle.value if isinstance(b.handle, C.c_void_p) else b.handle for b in banks])
        yb = (C.c_void_p * n)(*Y_devs)
        self._check("spq4k_moe_multi", self.lib.spq4k_moe_multi(self.handle, n, hb, ids_dev, n_used, ne11, T,
                                                               X_dev, yb))

    def set_decode_stamps(self, ptr, n: int = 0):
        """spq4k_set_decode_stamps (include/spq4k_diag.h): a device buffer of n uint64
        for the decode kernel's wave timestamps, or None to stop."""
        self._check("spq4k_set_decode_stamps", self.lib.spq4k_set_decode_stamps(self.handle, ptr or None, n))

    def stream_read_dev(self, p: int, nbytes: int):
        """spq4k_stream_read: one launch that only reads nbytes at p (the streaming floor)."""
        self._check("spq4k_stream_read", self.lib.spq4k_stream_read(self.handle, p, nbytes))

    def dequant_matvec_dev(self, W: Weights, X_dev: int, Y_dev: int, T: int = 1):
        """spq4k_dequant_matvec: beast_matvec's fp32-activation dequant-then-dot."""
        self._check("spq4k_dequant_matvec", self.lib.spq4k_dequant_matvec(self.handle, W.handle, X_dev, Y_dev, T))

    def dequant_matvec(self, W: Weights, X: np.ndarray) -> np.ndarray:
        """spq4k_dequant_matvec_host: X [T, K] -> Y [T, M]."""
        X = np.ascontiguousarray(X, np.float32).reshape(-1, W.K)
        Y = np.empty((X.shape[0], W.M), np.float32)
        self._check("spq4k_dequant_matvec_host", self.lib.spq4k_dequant_matvec_host(
            self.handle, W.handle, X.ctypes.data, Y.ctypes.data, X.shape[0]))
        return Y

    def beast_moe_forward(self, gate: Weights, up: Weights, down: Weights, logits: np.ndarray, top_k: int,
                          hidden: np.ndarray):
        """spq4k_beast_moe_forward_host: router logits [E], hidden [n_embd] ->
        (output [n_embd], expert ids [k], scores [k]), k = top_k (2 when <= 0, at most E)."""
        logits = np.ascontiguousarray(logits, np.float32).ravel()
        hidden = np.ascontiguousarray(hidden, np.float32).ravel()
        k = 2 if top_k <= 0 else min(top_k, gate.E)
        out = np.empty(gate.K, np.float32)
        ids = np.empty(k, np.int32)
        scores = np.empty(k, np.float32)
        self._check("spq4k_beast_moe_forward_host", self.lib.spq4k_beast_moe_forward_host(
            self.handle, gate.handle, up.handle, down.handle, logits.ctypes.data, top_k, hidden.ctypes.data,
            out.ctypes.data, ids.ctypes.data, scores.ctypes.data))
        return out, ids, scores

    def beast_moe_forward_dev(self, gate: Weights, up: Weights, down: Weights, logits_dev: int, top_k: int,
                              hidden_dev: int, out_dev: int, ids_dev: int = 0, scores_dev: int = 0):
        """spq4k_beast_moe_forward on device pointers (ids / scores optional)."""
        self._check("spq4k_beast_moe_forward", self.lib.spq4k_beast_moe_forward(
            self.handle, gate.handle, up.handle, down.handle, logits_dev, top_k, hidden_dev, out_dev,
            ids_dev or None, scores_dev or None))

    def moe_ffn_dev(self, gate: Weights, up: Weights, down: Weights, ids_dev: int, w_dev: int, n_used: int, T: int,
                    X_dev: int, Y_dev: int):
        """spq4k_moe_ffn: the routed-expert FFN block (gate/up, SwiGLU, down, weighted sum)."""
        self._check("spq4k_moe_ffn", self.lib.spq4k_moe_ffn(self.handle, gate.handle, up.handle, down.handle, ids_dev,
                                                           w_dev, n_used, T, X_dev, Y_dev))

    def moe_ffn(self, gate: Weights, up: Weights, down: Weights, ids: np.ndarray, weights: np.ndarray,
                X: np.ndarray) -> np.ndarray:
        """spq4k_moe_ffn_host: ids / weights [T, n_used], X [T, n_embd] -> [T, n_embd]."""
        ids = np.ascontiguousarray(ids, np.int32)
        weights = np.ascontiguousarray(weights, np.float32)
        X = np.ascontiguousarray(X, np.float32)
        T, n_used = ids.shape
        Y = np.empty((T, gate.K), np.float32)
        self._check("spq4k_moe_ffn_host", self.lib.spq4k_moe_ffn_host(
            self.handle, gate.handle, up.handle, down.handle, ids.ctypes.data, weights.ctypes.data, n_used, T,
            X.ctypes.data, Y.ctypes.data))
        return Y

    def dequant_dev(self, vx: int, y: int, k: int):
        self._check("spq4k_dequant", self.lib.spq4k_dequant(self.handle, vx, y, k))

    def quantize_q8K_dev(self, x: int, vy: int, k: int):
        self._check("spq4k_quantize_q8K", self.lib.spq4k_quantize_q8K(self.handle, x, vy, k))

    def quantize_q4K_dev(self, src: int, dst: int, nrow: int, n_per_row: int):
        self._check("spq4k_quantize_q4K", self.lib.spq4k_quantize_q4K(self.handle, src, dst, nrow, n_per_row))

    def to_float_dev(self, type: int, vx: int, y: int, k: int):
        self._check("spq4k_to_float", self.lib.spq4k_to_float(self.handle, type, vx, y, k))

    def quantize_chunk_dev(self, type: int, src: int, dst: int, nrow: int, n_per_row: int):
        self._check("spq4k_quantize_chunk", self.lib.spq4k_quantize_chunk(self.handle, type, src, dst, nrow, n_per_row))

    def vec_dot_q8K_dev(self, type: int, n: int, s_dev: int, vx: int, vy: int):
        self._check("spq4k_vec_dot_q8K", self.lib.spq4k_vec_dot_q8K(self.handle, type, n, s_dev, vx, vy))

    def rms_norm_dev(self, x: int, w: int, eps: float, y: int, K: int, T: int = 1):
        self._check("spq4k_rms_norm", self.lib.spq4k_rms_norm(self.handle, x, w, eps, y, K, T))

    def swiglu_dev(self, g: int, u: int, y: int, n: int):
        self._check("spq4k_swiglu", self.lib.spq4k_swiglu(self.handle, g, u, y, n))

    def mul_mat_rms_norm_dev(self, Ws, x_dev: int, norm_w_dev: int, eps: float, y_devs, T: int = 1):
        n = len(Ws)
        wa = (C.c_void_p * n)(*[w.handle.value if isinstance(w.handle, C.c_void_p) else w.handle for w in Ws])
        ya = (C.c_void_p * n)(*y_devs)
        self._check("spq4k_mul_mat_rms_norm",
                    self.lib.spq4k_mul_mat_rms_norm(self.handle, n, wa, x_dev, norm_w_dev, eps, ya, T))

    def mul_mat_swiglu_dev(self, Wg, Wu, x_dev: int, norm_w_dev, eps: float, y_dev: int, T: int = 1):
        self._check("spq4k_mul_mat_swiglu",
                    self.lib.spq4k_mul_mat_swiglu(self.handle, Wg.handle, Wu.handle, x_dev, norm_w_dev, eps, y_dev, T))

    def chain_create(self, stages, eps: float) -> Chain:
        """spq4k_chain_create. `stages` is a list of dicts: W (list of Weights),
        y (list of device pointers; with glu one), in0, and optionally glu,
        in1, x_out, norm_w (device pointers)."""
        n = len(stages)
        arr = (ChainStage * n)()
        refs = []
        for i, st in enumerate(stages):
            Ws = st["W"]
            arr[i].n = len(Ws)
            arr[i].glu = 1 if st.get("glu") else 0
            for j, w in enumerate(Ws):
                arr[i].W[j] = w.handle.value if isinstance(w.handle, C.c_void_p) else w.handle
                refs.append(w)
            for j, y in enumerate(st["y"]):
                arr[i].y[j] = y
            arr[i].in0 = st["in0"]
            arr[i].in1 = st.get("in1")
            arr[i].x_out = st.get("x_out")
            arr[i].norm_w = st.get("norm_w")
        h = C.c_void_p()
        self._check("spq4k_chain_create", self.lib.spq4k_chain_create(self.handle, arr, n, eps, C.byref(h)))
        return Chain(self, h, n, refs)

    def quantize_q8_0_dev(self, x: int, vy: int, k: int):
        self._check("spq4k_quantize_q8_0", self.lib.spq4k_quantize_q8_0(self.handle, x, vy, k))

    def vec_dot_q8_0_dev(self, n: int, s_dev: int, vx: int, vy: int):
        self._check("spq4k_vec_dot_q8_0", self.lib.spq4k_vec_dot_q8_0(self.handle, n, s_dev, vx, vy))

    def synth_fill_dev(self, out: int, n: int, seed: int, dist: int = DIST_NORMAL, cols: int = 0,
                       mean: float = 0.0, std: float = 1.0, outlier_mult: float = 1.0, offset: int = 0):
        self._check("spq4k_synth_fill", self.lib.spq4k_synth_fill(self.handle, out, n, seed, dist, cols, mean, std,
                                                                  outlier_mult, offset))


__all__ = ["Context", "Weights", "Spq4kError", "load_library", "load_gguf_library", "LIB_PATH", "QK_K", "Q4K_BLOCK_BYTES",
           "Q5K_BLOCK_BYTES", "Q6K_BLOCK_BYTES", "Q8K_BLOCK_BYTES", "QK8_0", "Q8_0_BLOCK_BYTES", "TYPE_Q8_0",
           "TYPE_Q4_K", "TYPE_Q5_K", "TYPE_Q6_K", "BLOCK_BYTES", "BLOCK_VALUES", "GEMV_MAX_T", "Gguf", "Model",
           "DIST_NORMAL", "DIST_STUDENT_T4"]
