"""The reference's own GGUF writer and reader (vendor/ggml/src/gguf.cpp,
compiled into oracle/_ref/*/libggml_ref.so) through ctypes: test
infrastructure that writes GGUF files the way the reference writes them and
reports what the reference's reader makes of a file."""
import ctypes as C

import numpy as np

V, I, I64, S = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
SCALAR = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
          7: np.uint8, 10: np.uint64, 11: np.int64, 12: np.float64}
STRING, ARRAY = 8, 9
SETTERS = {0: ("u8", C.c_uint8), 1: ("i8", C.c_int8), 2: ("u16", C.c_uint16), 3: ("i16", C.c_int16),
           4: ("u32", C.c_uint32), 5: ("i32", C.c_int32), 6: ("f32", C.c_float), 7: ("bool", C.c_bool),
           10: ("u64", C.c_uint64), 11: ("i64", C.c_int64), 12: ("f64", C.c_double)}


class _InitParams(C.Structure):          # struct ggml_init_params (ggml.h:658-663)
    _fields_ = [("mem_size", S), ("mem_buffer", V), ("no_alloc", C.c_bool)]


class _GgufParams(C.Structure):          # struct gguf_init_params (gguf.h:71-75)
    _fields_ = [("no_alloc", C.c_bool), ("ctx", C.POINTER(V))]


class RefGguf:
    def __init__(self, ref):
        L = C.CDLL(ref.path)
        L.ggml_init.argtypes = [_InitParams]
        L.ggml_init.restype = V
        L.ggml_free.argtypes = [V]
        L.ggml_new_tensor.argtypes = [V, I, I, C.POINTER(I64)]
        L.ggml_new_tensor.restype = V
        L.ggml_set_name.argtypes = [V, C.c_char_p]
        L.ggml_set_name.restype = V
        L.ggml_get_data.argtypes = [V]
        L.ggml_get_data.restype = V
        L.ggml_nbytes.argtypes = [V]
        L.ggml_nbytes.restype = S
        L.ggml_get_tensor.argtypes = [V, C.c_char_p]
        L.ggml_get_tensor.restype = V
        L.gguf_init_empty.restype = V
        L.gguf_free.argtypes = [V]
        L.gguf_add_tensor.argtypes = [V, V]
        L.gguf_write_to_file.argtypes = [V, C.c_char_p, C.c_bool]
        L.gguf_write_to_file.restype = C.c_bool
        L.gguf_set_val_str.argtypes = [V, C.c_char_p, C.c_char_p]
        L.gguf_set_arr_data.argtypes = [V, C.c_char_p, I, V, S]
        L.gguf_set_arr_str.argtypes = [V, C.c_char_p, C.POINTER(C.c_char_p), S]
        for t, (nm, ct) in SETTERS.items():
            f = getattr(L, f"gguf_set_val_{nm}")
            f.argtypes = [V, C.c_char_p, ct]
        L.gguf_init_from_file.argtypes = [C.c_char_p, _GgufParams]
        L.gguf_init_from_file.restype = V
        for n, r in (("gguf_get_version", C.c_uint32), ("gguf_get_alignment", S), ("gguf_get_data_offset", S),
                     ("gguf_get_n_kv", I64), ("gguf_get_n_tensors", I64)):
            getattr(L, n).argtypes = [V]
            getattr(L, n).restype = r
        for n, r in (("gguf_get_key", C.c_char_p), ("gguf_get_kv_type", I), ("gguf_get_arr_type", I),
                     ("gguf_get_arr_n", S), ("gguf_get_arr_data", V), ("gguf_get_val_data", V),
                     ("gguf_get_val_str", C.c_char_p), ("gguf_get_tensor_name", C.c_char_p),
                     ("gguf_get_tensor_type", I), ("gguf_get_tensor_offset", S), ("gguf_get_tensor_size", S)):
            getattr(L, n).argtypes = [V, I64]
            getattr(L, n).restype = r
        L.gguf_get_arr_str.argtypes = [V, I64, S]
        L.gguf_get_arr_str.restype = C.c_char_p
        self.L = L

    def write(self, path, tensors, kvs=(), alignment=None):
        """tensors: [(name, ggml type, ne tuple, uint8 bytes)]; kvs: [(key,
        gguf type, value)] with value a scalar, a str, or (element type,
        list) for an array. Returns gguf_write_to_file's result."""
        L = self.L
        mem = sum(int(np.asarray(t[3]).nbytes) + 1024 for t in tensors) + (1 << 20)
        ctx = L.ggml_init(_InitParams(mem, None, False))
        g = L.gguf_init_empty()
        keep = []
        try:
            if alignment is not None:
                L.gguf_set_val_u32(g, b"general.alignment", alignment)
            for key, t, val in kvs:
                k = key.encode()
                if t == ARRAY:
                    et, items = val
                    if et == STRING:
                        arr = (C.c_char_p * len(items))(*[s.encode() for s in items])
                        keep.append(arr)
                        L.gguf_set_arr_str(g, k, arr, len(items))
                    else:
                        a = np.ascontiguousarray(np.asarray(items, SCALAR[et]))
                        keep.append(a)
                        L.gguf_set_arr_data(g, k, et, a.ctypes.data if a.size else None, a.size)
                elif t == STRING:
                    L.gguf_set_val_str(g, k, val.encode())
                else:
                    getattr(L, f"gguf_set_val_{SETTERS[t][0]}")(g, k, val)
            for name, gt, ne, data in tensors:
                nea = (I64 * len(ne))(*ne)
                tt = L.ggml_new_tensor(ctx, gt, len(ne), nea)
                L.ggml_set_name(tt, name.encode())
                nb = L.ggml_nbytes(tt)
                buf = np.ascontiguousarray(data, np.uint8)
                assert buf.size == nb, (name, buf.size, nb)
                if nb:
                    C.memmove(L.ggml_get_data(tt), buf.ctypes.data, nb)
                L.gguf_add_tensor(g, tt)
            return bool(L.gguf_write_to_file(g, str(path).encode(), False))
        finally:
            L.gguf_free(g)
            L.ggml_free(ctx)

    def read(self, path):
        """What the reference's reader (gguf_init_from_file, no_alloc) makes
        of the file: None when it rejects it, else a dict of the header, the
        key/value pairs and the tensor table (shapes from the descriptors it
        creates)."""
        L = self.L
        meta = V()
        g = L.gguf_init_from_file(str(path).encode(), _GgufParams(True, C.pointer(meta)))
        if not g:
            return None
        try:
            out = {"version": L.gguf_get_version(g), "alignment": L.gguf_get_alignment(g),
                   "data_offset": L.gguf_get_data_offset(g), "kv": [], "tensors": []}
            for i in range(L.gguf_get_n_kv(g)):
                key = L.gguf_get_key(g, i).decode()
                t = L.gguf_get_kv_type(g, i)
                if t == ARRAY:
                    et = L.gguf_get_arr_type(g, i)
                    n = L.gguf_get_arr_n(g, i)
                    if et == STRING:
                        val = [L.gguf_get_arr_str(g, i, j).decode("utf-8", "surrogateescape") for j in range(n)]
                    else:
                        dt = np.dtype(SCALAR[et])
                        ptr = L.gguf_get_arr_data(g, i)
                        val = (np.ctypeslib.as_array((C.c_uint8 * (n * dt.itemsize)).from_address(ptr)).view(dt).copy()
                               if n else np.zeros(0, dt))
                else:
                    et = -1
                    if t == STRING:
                        val = [L.gguf_get_val_str(g, i).decode("utf-8", "surrogateescape")]
                    else:
                        dt = np.dtype(SCALAR[t])
                        ptr = L.gguf_get_val_data(g, i)
                        val = np.ctypeslib.as_array((C.c_uint8 * dt.itemsize).from_address(ptr)).view(dt).copy()
                out["kv"].append((key, t, et, val))
            for i in range(L.gguf_get_n_tensors(g)):
                name = L.gguf_get_tensor_name(g, i)
                tt = L.ggml_get_tensor(meta, name)
                ne = tuple(C.cast(tt, C.POINTER(I64))[2:6])   # struct ggml_tensor: type, buffer, ne[4] (ggml.h:666-671)
                out["tensors"].append((name.decode(), L.gguf_get_tensor_type(g, i), ne,
                                       L.gguf_get_tensor_offset(g, i), L.gguf_get_tensor_size(g, i)))
            return out
        finally:
            L.gguf_free(g)
            if meta:
                L.ggml_free(meta)
