"""ctypes access to the CPU checker (oracle/liboracle_q4k.so) and to the
reference's own ggml CPU library compiled in oracle/_ref/ (test code only)."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# SPQ4K_ORACLE_SO names another build of the oracle (the sanitizer build of
# `make -C oracle asan`)
ORACLE_SO = os.environ.get("SPQ4K_ORACLE_SO") or os.path.join(REPO, "oracle", "liboracle_q4k.so")
REF_DIR = os.path.join(REPO, "oracle", "_ref")

QK_K = 256
Q4K = 144
Q5K = 176
Q6K = 210
Q8K = 292
Q8_0 = 34
TYPE_Q8_0, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 8, 12, 13, 14            # ggml.h:392-404
BLOCK_BYTES = {TYPE_Q4_K: Q4K, TYPE_Q5_K: Q5K, TYPE_Q6_K: Q6K}
BLOCK_VALUES = {TYPE_Q8_0: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256, TYPE_Q6_K: 256}

V, I, I64, F, U64 = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_uint64


def _p(a):
    return None if a is None else a.ctypes.data


class Oracle:
    """The C restatement of the reference path (oracle/q4k_oracle.c)."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = C.CDLL(path)
        for n in ("or_quantize_row_q4K", "or_dequantize_row_q4K", "or_quantize_row_q8K"):
            getattr(L, n).argtypes = [V, V, I64]
        L.or_quantize_q4K.argtypes = [V, V, I64, I64]
        L.or_quantize_q4K.restype = C.c_size_t
        for n in ("or_vec_dot_generic", "or_vec_dot_avx2order"):
            getattr(L, n).argtypes = [I, V, V]
            getattr(L, n).restype = F
        L.or_vec_dot_exact.argtypes = [I, V, V]
        L.or_vec_dot_exact.restype = C.c_double
        L.or_subblock_sums.argtypes = [I, V, V, V]
        L.or_mul_mat.argtypes = [V, I64, I64, V, I64, V, I]
        L.or_mul_mat_id.argtypes = [V, I64, I64, I64, V, I64, V, I64, I64, V, I]
        L.or_mul_mat_id.restype = I
        L.or_mul_mat_dequant_f64.argtypes = [V, I64, I64, V, I64, V]
        L.or_mul_mat_dequant_f64_type.argtypes = [I, V, I64, I64, V, I64, V]
        L.or_mul_mat_dequant_f64_type.restype = I
        L.or_dequantize_row_q8K.argtypes = [V, V, I64]
        L.or_mul_mat_dq_f64_type.argtypes = [I, V, I64, I64, V, I64, V]
        L.or_mul_mat_dq_f64_type.restype = I
        L.or_beast_matvec_type.argtypes = [I, V, I64, I64, V, V]
        L.or_beast_matvec_type.restype = I
        L.or_beast_moe_routed.argtypes = [I, V, I, V, I, V, I64, I64, I64, V, V, I64, V, V]
        L.or_beast_moe_routed.restype = I
        L.or_synth_fill.argtypes = [V, I64, U64, I, I64, F, F, F, I64]
        L.or_rms_norm.argtypes = [V, I64, I64, V, F, V]
        L.or_swiglu.argtypes = [V, V, I64, V]
        L.or_fp16_to_fp32.argtypes = [C.c_uint16]
        L.or_fp16_to_fp32.restype = F
        L.or_fp32_to_fp16.argtypes = [F]
        L.or_fp32_to_fp16.restype = C.c_uint16
        L.or_nearest_int.argtypes = [F]
        L.or_nearest_int.restype = I
        L.or_scale_min_k4.argtypes = [I, V, V, V]
        for n in ("or_quantize_row_q6K", "or_dequantize_row_q6K"):
            getattr(L, n).argtypes = [V, V, I64]
        for n in ("or_vec_dot_q6K_generic", "or_vec_dot_q6K_avx2order"):
            getattr(L, n).argtypes = [I, V, V]
            getattr(L, n).restype = F
        L.or_vec_dot_q6K_exact.argtypes = [I, V, V]
        L.or_vec_dot_q6K_exact.restype = C.c_double
        L.or_subblock_sums_q6K.argtypes = [I, V, V, V]
        for n in ("or_quantize_row_q5K", "or_dequantize_row_q5K"):
            getattr(L, n).argtypes = [V, V, I64]
        for n in ("or_vec_dot_q5K_generic", "or_vec_dot_q5K_avx2order"):
            getattr(L, n).argtypes = [I, V, V]
            getattr(L, n).restype = F
        L.or_vec_dot_q5K_exact.argtypes = [I, V, V]
        L.or_vec_dot_q5K_exact.restype = C.c_double
        L.or_subblock_sums_q5K.argtypes = [I, V, V, V]
        for n in ("or_quantize_row_q8_0", "or_quantize_row_q8_0_ref", "or_dequantize_row_q8_0"):
            getattr(L, n).argtypes = [V, V, I64]
        for n in ("or_vec_dot_q8_0_generic", "or_vec_dot_q8_0_avx2order"):
            getattr(L, n).argtypes = [I, V, V]
            getattr(L, n).restype = F
        L.or_vec_dot_q8_0_exact.argtypes = [I, V, V]
        L.or_vec_dot_q8_0_exact.restype = C.c_double
        L.or_block_sums_q8_0.argtypes = [I, V, V, V]
        L.or_mul_mat_q8_0.argtypes = [V, I64, I64, V, I64, V, I]
        L.or_mul_mat_q8_0.restype = I
        L.or_mul_mat_id_q8_0.argtypes = [V, I64, I64, I64, V, I64, V, I64, I64, V, I]
        L.or_mul_mat_id_q8_0.restype = I
        L.or_mul_mat_type.argtypes = [I, V, I64, I64, V, I64, V, I]
        L.or_mul_mat_id_type.argtypes = [I, V, I64, I64, I64, V, I64, V, I64, I64, V, I]
        L.or_mul_mat_dequant_f64_type.argtypes = [I, V, I64, I64, V, I64, V]
        for n in ("or_mul_mat_type", "or_mul_mat_id_type", "or_mul_mat_dequant_f64_type"):
            getattr(L, n).restype = I
        self.L = L

    def quantize_q4K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // QK_K * Q4K, np.uint8)
        self.L.or_quantize_row_q4K(_p(x), _p(y), x.size)
        return y

    def dequant(self, q: np.ndarray, k: int) -> np.ndarray:
        y = np.empty(k, np.float32)
        self.L.or_dequantize_row_q4K(_p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def quantize_q8K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // QK_K * Q8K, np.uint8)
        self.L.or_quantize_row_q8K(_p(x), _p(y), x.size)
        return y

    def vec_dot(self, n, qx, qy, order="avx2"):
        f = self.L.or_vec_dot_avx2order if order == "avx2" else self.L.or_vec_dot_generic
        return f(n, _p(qx), _p(qy))

    def vec_dot_exact(self, n, qx, qy):
        return self.L.or_vec_dot_exact(n, _p(qx), _p(qy))

    def subblock_sums(self, n, qx, qy) -> np.ndarray:
        S = np.zeros(n // QK_K * 8, np.int32)
        self.L.or_subblock_sums(n, _p(qx), _p(qy), _p(S))
        return S

    def mul_mat(self, W, M, K, X, order=1):
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float32)
        self.L.or_mul_mat(_p(W), M, K, _p(X), X.shape[0], _p(Y), order)
        return Y

    def mul_mat_id(self, bank, M, K, E, X, ids, order=1):
        ids = np.ascontiguousarray(ids, np.int32)
        T, k = ids.shape
        X = np.ascontiguousarray(X, np.float32).reshape(T, -1, K)
        Y = np.empty((T, k, M), np.float32)
        rc = self.L.or_mul_mat_id(_p(bank), M, K, E, _p(X), X.shape[1], _p(ids), k, T, _p(Y), order)
        assert rc == 0
        return Y

    def mul_mat_f64(self, W, M, K, X):
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float64)
        self.L.or_mul_mat_dequant_f64(_p(W), M, K, _p(X), X.shape[0], _p(Y))
        return Y

    # ---- Q6_K (oracle/q6k_oracle.c) and type-generic drivers ----
    def quantize_q6K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // QK_K * Q6K, np.uint8)
        self.L.or_quantize_row_q6K(_p(x), _p(y), x.size)
        return y

    def dequant_q6K(self, q: np.ndarray, k: int) -> np.ndarray:
        y = np.empty(k, np.float32)
        self.L.or_dequantize_row_q6K(_p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def vec_dot_q6K(self, n, qx, qy, order="avx2"):
        f = self.L.or_vec_dot_q6K_avx2order if order == "avx2" else self.L.or_vec_dot_q6K_generic
        return f(n, _p(qx), _p(qy))

    def vec_dot_q6K_exact(self, n, qx, qy):
        return self.L.or_vec_dot_q6K_exact(n, _p(qx), _p(qy))

    def subblock_sums_q6K(self, n, qx, qy) -> np.ndarray:
        S = np.zeros(n // QK_K * 16, np.int32)
        self.L.or_subblock_sums_q6K(n, _p(qx), _p(qy), _p(S))
        return S

    # ---- Q5_K (oracle/q5k_oracle.c) ----
    def quantize_q5K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // QK_K * Q5K, np.uint8)
        self.L.or_quantize_row_q5K(_p(x), _p(y), x.size)
        return y

    def dequant_q5K(self, q: np.ndarray, k: int) -> np.ndarray:
        y = np.empty(k, np.float32)
        self.L.or_dequantize_row_q5K(_p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def vec_dot_q5K(self, n, qx, qy, order="avx2"):
        f = self.L.or_vec_dot_q5K_avx2order if order == "avx2" else self.L.or_vec_dot_q5K_generic
        return f(n, _p(qx), _p(qy))

    def vec_dot_q5K_exact(self, n, qx, qy):
        return self.L.or_vec_dot_q5K_exact(n, _p(qx), _p(qy))

    def subblock_sums_q5K(self, n, qx, qy) -> np.ndarray:
        S = np.zeros(n // QK_K * 8, np.int32)
        self.L.or_subblock_sums_q5K(n, _p(qx), _p(qy), _p(S))
        return S

    # ---- Q8_0 (oracle/q8_0_oracle.c) ----
    def quantize_q8_0(self, x: np.ndarray, ref_encoder=False) -> np.ndarray:
        """Activations (the CPU backend's quantize_row_q8_0), or with
        ref_encoder the model-file encoder quantize_row_q8_0_ref."""
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // 32 * Q8_0, np.uint8)
        f = self.L.or_quantize_row_q8_0_ref if ref_encoder else self.L.or_quantize_row_q8_0
        f(_p(x), _p(y), x.size)
        return y

    def dequant_q8_0(self, q: np.ndarray, k: int) -> np.ndarray:
        y = np.empty(k, np.float32)
        self.L.or_dequantize_row_q8_0(_p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def vec_dot_q8_0(self, n, qx, qy, order="avx2"):
        f = self.L.or_vec_dot_q8_0_avx2order if order == "avx2" else self.L.or_vec_dot_q8_0_generic
        return f(n, _p(qx), _p(qy))

    def vec_dot_q8_0_exact(self, n, qx, qy):
        return self.L.or_vec_dot_q8_0_exact(n, _p(qx), _p(qy))

    def block_sums_q8_0(self, n, qx, qy) -> np.ndarray:
        S = np.zeros(n // 32, np.int32)
        self.L.or_block_sums_q8_0(n, _p(qx), _p(qy), _p(S))
        return S

    def mul_mat_q8_0(self, W, M, K, X, order=1):
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float32)
        assert self.L.or_mul_mat_q8_0(_p(W), M, K, _p(X), X.shape[0], _p(Y), order) == 0
        return Y

    def mul_mat_id_q8_0(self, bank, M, K, E, X, ids, order=1):
        ids = np.ascontiguousarray(ids, np.int32)
        T, k = ids.shape
        X = np.ascontiguousarray(X, np.float32).reshape(T, -1, K)
        Y = np.empty((T, k, M), np.float32)
        assert self.L.or_mul_mat_id_q8_0(_p(bank), M, K, E, _p(X), X.shape[1], _p(ids), k, T, _p(Y), order) == 0
        return Y

    def quantize(self, qtype, x):
        """weights of the type (Q8_0 with the model-file encoder)"""
        if qtype == TYPE_Q8_0:
            return self.quantize_q8_0(x, ref_encoder=True)
        return {TYPE_Q4_K: self.quantize_q4K, TYPE_Q5_K: self.quantize_q5K, TYPE_Q6_K: self.quantize_q6K}[qtype](x)

    def to_float(self, qtype, q, k):
        return {TYPE_Q4_K: self.dequant, TYPE_Q5_K: self.dequant_q5K, TYPE_Q6_K: self.dequant_q6K,
                TYPE_Q8_0: self.dequant_q8_0}[qtype](q, k)

    def mul_mat_type(self, qtype, W, M, K, X, order=1):
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float32)
        assert self.L.or_mul_mat_type(qtype, _p(W), M, K, _p(X), X.shape[0], _p(Y), order) == 0
        return Y

    def mul_mat_id_type(self, qtype, bank, M, K, E, X, ids, order=1):
        ids = np.ascontiguousarray(ids, np.int32)
        T, k = ids.shape
        X = np.ascontiguousarray(X, np.float32).reshape(T, -1, K)
        Y = np.empty((T, k, M), np.float32)
        rc = self.L.or_mul_mat_id_type(qtype, _p(bank), M, K, E, _p(X), X.shape[1], _p(ids), k, T, _p(Y), order)
        assert rc == 0
        return Y

    def mul_mat_f64_type(self, qtype, W, M, K, X):
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float64)
        assert self.L.or_mul_mat_dequant_f64_type(qtype, _p(W), M, K, _p(X), X.shape[0], _p(Y)) == 0
        return Y

    # ---- fused neighbours (oracle/fusion_oracle.c) ----
    def rms_norm(self, X, w, eps) -> np.ndarray:
        """ggml_mul(ggml_rms_norm(X, eps), w), rows of X."""
        X = np.ascontiguousarray(X, np.float32)
        K = X.shape[-1]
        Y = np.empty_like(X)
        self.L.or_rms_norm(_p(X), K, X.size // K, None if w is None else _p(np.ascontiguousarray(w, np.float32)),
                           eps, _p(Y))
        return Y

    def swiglu(self, g, u) -> np.ndarray:
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        y = np.empty_like(g)
        self.L.or_swiglu(_p(g), _p(u), g.size, _p(y))
        return y

    def dequant_q8K(self, q: np.ndarray, k: int) -> np.ndarray:
        y = np.empty(k, np.float32)
        self.L.or_dequantize_row_q8K(_p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def mul_mat_dq_f64(self, qtype, W, M, K, X) -> np.ndarray:
        """sum of dequant(W) * dequant(Q(x)) in double (the second form of the parity bar)"""
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float64)
        assert self.L.or_mul_mat_dq_f64_type(qtype, _p(np.ascontiguousarray(W)), M, K, _p(X), X.shape[0], _p(Y)) == 0
        return Y

    def mul_mat_dequant_f64(self, qtype, W, M, K, X) -> np.ndarray:
        """sum of dequant(W) * x in double, x as given (fp32-activation dequant-then-dot)"""
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float64)
        assert self.L.or_mul_mat_dequant_f64_type(qtype, _p(np.ascontiguousarray(W)), M, K, _p(X), X.shape[0],
                                                  _p(Y)) == 0
        return Y

    def mul_mat_id_dq_f64(self, qtype, bank, M, K, E, X, ids) -> np.ndarray:
        """mul_mat_id of the dequant-then-dot form: Y[t][s] = mul_mat_dq_f64 of
        expert ids[t][s] on input row X[t][s % ne11]"""
        ids = np.ascontiguousarray(ids, np.int32)
        T, k = ids.shape
        X = np.ascontiguousarray(X, np.float32).reshape(T, -1, K)
        eb = bank.size // E
        Y = np.empty((T, k, M), np.float64)
        for t in range(T):
            for s_ in range(k):
                e = int(ids[t, s_])
                Y[t, s_] = self.mul_mat_dq_f64(qtype, bank[e * eb:(e + 1) * eb], M, K, X[t, s_ % X.shape[1]])[0]
        return Y

    def beast_matvec(self, qtype, W, M, K, x) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.empty(M, np.float32)
        assert self.L.or_beast_matvec_type(qtype, _p(np.ascontiguousarray(W)), M, K, _p(x), _p(y)) == 0
        return y

    def beast_moe_routed(self, types, gate, up, down, E, n_embd, n_ff, ids, scores, hidden) -> np.ndarray:
        """the MoE forward's per-expert loop over a given routing, a type per
        bank (types = (gate, up, down))"""
        ids = np.ascontiguousarray(ids, np.int32).ravel()
        scores = np.ascontiguousarray(scores, np.float32).ravel()
        hidden = np.ascontiguousarray(hidden, np.float32).ravel()
        out = np.empty(n_embd, np.float32)
        rc = self.L.or_beast_moe_routed(types[0], _p(np.ascontiguousarray(gate)), types[1],
                                        _p(np.ascontiguousarray(up)), types[2], _p(np.ascontiguousarray(down)), E,
                                        n_embd, n_ff, _p(ids), _p(scores), ids.size, _p(hidden), _p(out))
        assert rc == 0
        return out

    def synth(self, n, seed, dist=0, cols=0, mean=0.0, std=1.0, mult=1.0, offset=0) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.L.or_synth_fill(_p(out), n, seed, dist, cols, mean, std, mult, offset)
        return out


def cpu_supports_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
    except OSError:
        return False
    return all(t in flags for t in ("avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd"))


def ref_library_path():
    for v in (("v4",) if cpu_supports_avx512() else ()) + ("v3",):
        p = os.path.join(REF_DIR, v, "libggml_ref.so")
        if os.path.exists(p):
            return p
    return None


class Ref:
    """The reference's ggml CPU library built from its own sources (oracle/_ref)."""

    def __init__(self, path=None):
        path = path or ref_library_path()
        if not path:
            raise FileNotFoundError("oracle/_ref not built")
        L = C.CDLL(path)
        L.ref_quantize_q4K.argtypes = [V, V, I64, I64]
        L.ref_quantize_q4K.restype = C.c_size_t
        L.ref_dequant_q4K.argtypes = [V, V, I64]
        L.ref_quantize_q8K.argtypes = [V, V, I64]
        for n in ("ref_vec_dot", "ref_vec_dot_generic"):
            getattr(L, n).argtypes = [I, V, V]
            getattr(L, n).restype = F
        L.ref_mm_create.argtypes = [I, V, V, V, V, V, I64, I]
        L.ref_mm_create.restype = V
        L.ref_mmid_create.argtypes = [V, I64, I64, I64, V, I64, V, I64, I64, V, I]
        L.ref_mmid_create.restype = V
        L.ref_quantize_type.argtypes = [I, V, V, I64, I64]
        L.ref_quantize_type.restype = C.c_size_t
        L.ref_dequant_type.argtypes = [I, V, V, I64]
        L.ref_vec_dot_type.argtypes = [I, I, V, V, I]
        L.ref_vec_dot_type.restype = F
        L.ref_quantize_vec_dot_type.argtypes = [I, V, V, I64]
        L.ref_mm_create_type.argtypes = [I, I, V, V, V, V, V, I64, I]
        L.ref_mm_create_type.restype = V
        L.ref_mmid_create_type.argtypes = [I, V, I64, I64, I64, V, I64, V, I64, I64, V, I]
        L.ref_mmid_create_type.restype = V
        L.ref_graph_run.argtypes = [V, I, V]
        L.ref_graph_run.restype = I
        L.ref_graph_destroy.argtypes = [V]
        L.ref_rms_norm_create.argtypes = [V, I64, I64, V, F, V, I]
        L.ref_rms_norm_create.restype = V
        L.ref_swiglu_create.argtypes = [I, V, V, I64, I64, V, I64, V, F, V, I]
        L.ref_swiglu_create.restype = V
        L.ref_graph_b_run.argtypes = [V]
        L.ref_graph_b_run.restype = I
        L.ref_graph_b_destroy.argtypes = [V]
        self.L = L
        self.path = path

    def quantize_q4K(self, x, nrow, n_per_row):
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(nrow * (n_per_row // QK_K) * Q4K, np.uint8)
        self.L.ref_quantize_q4K(_p(x), _p(y), nrow, n_per_row)
        return y

    def dequant(self, q, k):
        y = np.empty(k, np.float32)
        self.L.ref_dequant_q4K(_p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def quantize_q8K(self, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // QK_K * Q8K, np.uint8)
        self.L.ref_quantize_q8K(_p(x), _p(y), x.size)
        return y

    def vec_dot(self, n, qx, qy, generic=False):
        f = self.L.ref_vec_dot_generic if generic else self.L.ref_vec_dot
        return f(n, _p(qx), _p(qy))

    def quantize_type(self, qtype, x, nrow, n_per_row):
        x = np.ascontiguousarray(x, np.float32).ravel()
        nbytes = nrow * n_per_row // 32 * Q8_0 if qtype == TYPE_Q8_0 else nrow * (n_per_row // QK_K) * BLOCK_BYTES[qtype]
        y = np.zeros(nbytes, np.uint8)
        self.L.ref_quantize_type(qtype, _p(x), _p(y), nrow, n_per_row)
        return y

    def dequant_type(self, qtype, q, k):
        y = np.empty(k, np.float32)
        self.L.ref_dequant_type(qtype, _p(np.ascontiguousarray(q)), _p(y), k)
        return y

    def quantize_q8_0_act(self, x):
        """The CPU backend's activation quantiser for Q8_0 weights."""
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.zeros(x.size // 32 * Q8_0, np.uint8)
        self.L.ref_quantize_vec_dot_type(TYPE_Q8_0, _p(x), _p(y), x.size)
        return y

    def vec_dot_type(self, qtype, n, qx, qy, generic=False):
        return self.L.ref_vec_dot_type(qtype, n, _p(qx), _p(qy), int(generic))

    def mul_mat(self, W, M, K, X, nthreads=1, qtype=TYPE_Q4_K):
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        T = X.shape[0]
        Y = np.empty((T, M), np.float32)
        arr = lambda ctype, vals: (ctype * 1)(*vals)
        h = self.L.ref_mm_create_type(qtype, 1, arr(V, [W.ctypes.data]), arr(I64, [M]), arr(I64, [K]),
                                      arr(V, [X.ctypes.data]), arr(V, [Y.ctypes.data]), T, nthreads)
        assert h
        try:
            assert self.L.ref_graph_run(h, 1, None) == 0
        finally:
            self.L.ref_graph_destroy(h)
        return Y

    def mul_mat_id(self, bank, M, K, E, X, ids, nthreads=1, qtype=TYPE_Q4_K):
        ids = np.ascontiguousarray(ids, np.int32)
        T, k = ids.shape
        X = np.ascontiguousarray(X, np.float32).reshape(T, -1, K)
        Y = np.empty((T, k, M), np.float32)
        h = self.L.ref_mmid_create_type(qtype, _p(bank), M, K, E, _p(X), X.shape[1], _p(ids), k, T, _p(Y),
                                        nthreads)
        assert h
        try:
            assert self.L.ref_graph_run(h, 1, None) == 0
        finally:
            self.L.ref_graph_destroy(h)
        return Y


def _ref_rms_norm(self, X, w, eps, nthreads=1):
    X = np.ascontiguousarray(X, np.float32)
    K = X.shape[-1]
    Y = np.empty_like(X)
    w = np.ascontiguousarray(w, np.float32)
    h = self.L.ref_rms_norm_create(_p(X), K, X.size // K, _p(w), eps, _p(Y), nthreads)
    assert h
    try:
        assert self.L.ref_graph_b_run(h) == 0
    finally:
        self.L.ref_graph_b_destroy(h)
    return Y


def _ref_swiglu_ffn(self, qtype, Wg, Wu, M, K, X, w=None, eps=1e-6, nthreads=1):
    """silu(Wg . xb) * (Wu . xb), xb = X or rms_norm(X) * w, through a ggml graph."""
    X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
    Y = np.empty((X.shape[0], M), np.float32)
    wp = None if w is None else _p(np.ascontiguousarray(w, np.float32))
    keep = None if w is None else np.ascontiguousarray(w, np.float32)
    if keep is not None:
        wp = _p(keep)
    h = self.L.ref_swiglu_create(qtype, _p(Wg), _p(Wu), M, K, _p(X), X.shape[0], wp, eps, _p(Y), nthreads)
    assert h
    try:
        assert self.L.ref_graph_b_run(h) == 0
    finally:
        self.L.ref_graph_b_destroy(h)
    return Y


def _ref_dequant_q8K(self, q, k):
    """the reference's dequantize_row_q8_K (ggml-quants.c:2731-2740)"""
    f = self.L.dequantize_row_q8_K
    f.argtypes = [V, V, I64]
    y = np.empty(k, np.float32)
    f(_p(np.ascontiguousarray(q)), _p(y), k)
    return y


Ref.rms_norm = _ref_rms_norm
Ref.swiglu_ffn = _ref_swiglu_ffn
Ref.dequant_q8K = _ref_dequant_q8K

BEAST_SO = os.path.join(REF_DIR, "beast", "libbeast_ref.so")


class BeastRef:
    """The reference's beast_matvec (desktop/beast_canyon/sp_beast_canyon.c:
    1122-1134) compiled from its source by oracle/Makefile into
    oracle/_ref/beast (oracle/beast_driver.c)."""

    def __init__(self, path=BEAST_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle ref)")
        self.L = C.CDLL(path)
        self.L.ref_beast_matvec.argtypes = [V, C.c_uint, V, V, I, I]
        self.L.ref_beast_matvec.restype = I
        self.L.ref_beast_route.argtypes = [V, I, I, V, V]
        self.L.ref_beast_route.restype = I
        self.L.ref_beast_moe.argtypes = [V, V, V, C.c_uint, I, I, I, V, I, V, V, V, V]
        self.L.ref_beast_moe.restype = I
        self.L.ref_beast_moe_types.argtypes = [V, C.c_uint, V, C.c_uint, V, C.c_uint, I, I, I, V, I, V, V, V, V]
        self.L.ref_beast_moe_types.restype = I

    def matvec(self, qtype, W, M, K, x):
        x = np.ascontiguousarray(x, np.float32).ravel()
        y = np.empty(M, np.float32)
        assert self.L.ref_beast_matvec(_p(np.ascontiguousarray(W)), qtype, _p(x), _p(y), M, K) == 0
        return y

    def route(self, logits, top_k):
        """sp_beast_route_experts (:385-443): expert ids and renormalised scores"""
        logits = np.ascontiguousarray(logits, np.float32).ravel()
        ids = np.empty(logits.size, np.int32)          # the routing selects at most every expert
        scores = np.empty(logits.size, np.float32)
        n = self.L.ref_beast_route(_p(logits), logits.size, top_k, _p(ids), _p(scores))
        assert n > 0
        return ids[:n].copy(), scores[:n].copy()

    def moe(self, qtype, gate, up, down, E, n_embd, n_ff, logits, top_k, hidden):
        """sp_beast_moe_forward (:455-562) on contiguous expert banks: output,
        ids, scores; qtype one type for all banks or a (gate, up, down) tuple"""
        types = tuple(qtype) if isinstance(qtype, (tuple, list)) else (qtype,) * 3
        logits = np.ascontiguousarray(logits, np.float32).ravel()
        hidden = np.ascontiguousarray(hidden, np.float32).ravel()
        out = np.empty(n_embd, np.float32)
        ids = np.empty(E, np.int32)
        scores = np.empty(E, np.float32)
        n = self.L.ref_beast_moe_types(_p(np.ascontiguousarray(gate)), types[0], _p(np.ascontiguousarray(up)),
                                       types[1], _p(np.ascontiguousarray(down)), types[2], E, n_embd, n_ff,
                                       _p(logits), top_k, _p(hidden), _p(out), _p(ids), _p(scores))
        assert n > 0
        return out, ids[:n].copy(), scores[:n].copy()


def close_enough(a, b, rel=1e-4, abs_=1e-5):
    """The reference's element tolerance (tests/desktop/test_sp_kernels.cpp:34-48):
    equal, or |a-b| <= 1e-5, or |a-b| / max(|a|,|b|) <= 1e-4. Returns a bool mask."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.abs(a - b)
    scale = np.maximum(np.abs(a), np.abs(b))
    with np.errstate(divide="ignore", invalid="ignore"):
        rel_ok = d <= rel * scale
    return (a == b) | (d <= abs_) | rel_ok


def parity_ok(got, exp, exact):
    """The parity bar of the matmul outputs: each output
    within close_enough of ggml_vec_dot's value (exp: the oracle in ggml's x86
    order) or of the dequant-then-dot value (exact: the sum of dequant(W) *
    dequant(Q(x)) in double, Oracle.mul_mat_dq_f64). Where a row's products
    cancel, the two fp32 summation orders can differ by more than 1e-4 of the
    small result while both stay within it of the exact sum."""
    return close_enough(got, exp) | close_enough(got, exact)
