#!/usr/bin/env python3
"""Writes tests/golden/q4k_golden.npz and q6k_golden.npz from the reference's
own ggml CPU code.

The reference (vendor/ggml of nihilistau/shannon-prime-burnhard) is compiled
from its sources by oracle/Makefile (`make -C oracle ref`) into oracle/_ref;
this script calls it through oracle/ref_driver.c and stores small input/output
vectors. Run only where /root/reference exists; the .npz travels with the
repository and pins the CPU oracle (tests/test_oracle_golden.py).

Contents (all produced by the reference):
  enc_x / enc_q    quantize_q4_K (ggml_quantize_chunk, imatrix NULL) bytes
  deq_q / deq_y    dequantize_row_q4_K
  q8_x  / q8_y     quantize_row_q8_K blocks; a block with max |x| = 0 keeps
                   the caller's zero-initialised bsums (the reference does not
                   write them in that branch)
  vd_q4 / vd_q8 / vd_K / vd_avx2 / vd_generic
                   ggml_vec_dot_q4_K_q8_K (x86 kernel) and its portable
                   ggml_vec_dot_q4_K_q8_K_generic, one row per case
  mm_*             GGML_OP_MUL_MAT through ggml_graph_compute (1 thread)
  mmid_*           GGML_OP_MUL_MAT_ID through ggml_graph_compute (1 thread)

q6k_golden.npz and q5k_golden.npz hold the same kinds of vectors for
GGML_TYPE_Q6_K and GGML_TYPE_Q5_K (quantize_q6_K / quantize_q5_K,
dequantize_row_q6_K / _q5_K, ggml_vec_dot_q6_K_q8_K / _q5_K_q8_K and their
_generic forms, MUL_MAT, MUL_MAT_ID), plus vec_dot cases on random block bytes
that reach every scale and quant value.

q8_0_golden.npz holds GGML_TYPE_Q8_0 vectors: the model-file encoder
(quantize_q8_0 -> quantize_row_q8_0_ref), dequantize_row_q8_0, the CPU
backend's activation quantiser (quantize_row_q8_0, which rounds half to even
where the encoder rounds half away from zero: tie cases included),
ggml_vec_dot_q8_0_q8_0 and its _generic form, MUL_MAT, MUL_MAT_ID.

dq_golden.npz holds dequantize_row_q8_K outputs (the activation side of the
dequant-then-dot form of the parity bar) and the reference's BurnHard scalar
matvec beast_matvec (desktop/beast_canyon/sp_beast_canyon.c:1122-1134, built
by oracle/Makefile from that file) on Q4_K and Q8_0 rows with fp32 inputs.

Usage: gen_golden.py [q4k] [q5k] [q6k] [q8_0] [dq]   (default: all)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from _oracle import TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, Q5K, Q6K, Q8_0, Ref, ref_library_path  # noqa: E402

QK = 256


def encoder_inputs(rng):
    rows = []
    rows.append((rng.standard_normal((8, 4096)) * 0.02).astype(np.float32))        # the BASELINE distribution
    t = (rng.standard_t(4, size=(4, 5120)) * 0.02).astype(np.float32)
    t[:, ::53] *= 8.0                                                                 # outlier columns
    rows.append(t)
    edge = []
    edge.append(np.zeros(QK, np.float32))                                             # all zero
    edge.append(np.full(QK, 0.25, np.float32))                                        # constant positive
    edge.append(np.full(QK, -0.25, np.float32))                                       # constant negative
    s = np.zeros(QK, np.float32); s[100] = 3.0; edge.append(s)                        # single spike
    edge.append(np.abs(rng.standard_normal(QK)).astype(np.float32))                   # all >= 0 (min clamps to 0)
    edge.append(-np.abs(rng.standard_normal(QK)).astype(np.float32))                  # all <= 0
    edge.append((rng.standard_normal(QK) * 1e-6).astype(np.float32))                  # tiny
    edge.append((rng.standard_normal(QK) * 100.0).astype(np.float32))                 # large
    z = rng.standard_normal(QK).astype(np.float32); z[32:64] = 0.0; edge.append(z)    # one zero sub-block
    a = np.linspace(-1, 1, QK, dtype=np.float32); edge.append(a)                      # ramp
    rows.append(np.stack(edge))
    return np.concatenate([r.ravel() for r in rows]).astype(np.float32)


def q8_inputs(rng):
    c = [rng.standard_normal(QK * 8).astype(np.float32)]
    c.append(np.zeros(QK, np.float32))
    t = np.zeros(QK, np.float32); t[5] = 2.0; t[77] = -2.0; c.append(t)               # tie, first is +
    t = np.zeros(QK, np.float32); t[5] = -2.0; t[77] = 2.0; c.append(t)               # tie, first is -
    c.append(((np.arange(QK) - 128) * 0.5).astype(np.float32))                        # many .5 products
    c.append((rng.standard_normal(QK) * 1e-20).astype(np.float32))
    c.append((rng.standard_normal(QK) * 1e20).astype(np.float32))
    c.append(np.full(QK, 1.0, np.float32))
    return np.concatenate(c)


def q6k_encoder_inputs(rng):
    rows = [(rng.standard_normal((8, 4096)) * 0.02).astype(np.float32).ravel()]
    t = (rng.standard_t(4, size=(4, 5120)) * 0.02).astype(np.float32)
    t[:, ::53] *= 8.0
    rows.append(t.ravel())
    edge = [np.zeros(QK, np.float32), np.full(QK, 0.25, np.float32), np.full(QK, -0.25, np.float32)]
    s = np.zeros(QK, np.float32); s[100] = 3.0; edge.append(s)                        # single spike
    s = np.zeros(QK, np.float32); s[7] = -3.0; edge.append(s)                         # negative spike
    edge.append(np.abs(rng.standard_normal(QK)).astype(np.float32))                   # all >= 0
    edge.append(-np.abs(rng.standard_normal(QK)).astype(np.float32))                  # all <= 0
    edge.append((rng.standard_normal(QK) * 1e-6).astype(np.float32))                  # tiny
    edge.append((rng.standard_normal(QK) * 1e-17).astype(np.float32))                 # below the 1e-15 cut
    edge.append((rng.standard_normal(QK) * 100.0).astype(np.float32))                 # large
    z = rng.standard_normal(QK).astype(np.float32); z[48:64] = 0.0; edge.append(z)    # one zero sub-block
    z = rng.standard_normal(QK).astype(np.float32); z[::16] *= 50; edge.append(z)     # one spike per sub-block
    edge.append(np.linspace(-1, 1, QK, dtype=np.float32))                             # ramp
    rows.append(np.stack(edge).ravel())
    return np.concatenate(rows).astype(np.float32)


def _finite_blocks(rng, n, qtype, bb, tame):
    """Random block bytes with finite fp16 scales (tame: |d| < 2^-1)."""
    b = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    mask = 0x3B if tame else 0xBF
    for hi in ((209,) if qtype == TYPE_Q6_K else (1, 3)):     # high bytes of d (and dmin)
        b[:, hi] &= mask
    return b


def gen_kquant(ref, rng, qtype, bb):
    """Golden vectors of one K-quant weight type with Q8_K activations."""
    out = {}
    x = q6k_encoder_inputs(rng)
    out["enc_x"] = x
    out["enc_q"] = ref.quantize_type(qtype, x, 1, x.size)

    q = np.concatenate([out["enc_q"].reshape(-1, bb), _finite_blocks(rng, 64, qtype, bb, False)]).ravel()
    out["deq_q"] = q
    out["deq_y"] = ref.dequant_type(qtype, q, q.size // bb * QK)

    # vec_dot: encoder output at K in {256, 768, 4096, 27648}, then random
    # block bytes (every scale and quant value) against Q8_K of N(0,1) and of
    # one-sign inputs
    vw, vq8, vK, va, vg = [], [], [], [], []
    cases = [(K, n, "enc") for K, n in ((256, 8), (768, 8), (4096, 8), (27648, 4))]
    cases += [(K, n, "rand") for K, n in ((256, 8), (4096, 8))]
    for K, n, kind in cases:
        for i in range(n):
            if kind == "enc":
                w = ref.quantize_type(qtype, (rng.standard_normal(K) * 0.02).astype(np.float32), 1, K)
            else:
                w = _finite_blocks(rng, K // QK, qtype, bb, True).ravel()
            xa = rng.standard_normal(K).astype(np.float32)
            if kind == "rand" and i % 2:
                xa = np.abs(xa)
            a = ref.quantize_q8K(xa)
            vw.append(w); vq8.append(a); vK.append(K)
            va.append(ref.vec_dot_type(qtype, K, w, a)); vg.append(ref.vec_dot_type(qtype, K, w, a, True))
    out["vd_w"] = np.concatenate(vw)
    out["vd_q8"] = np.concatenate(vq8)
    out["vd_K"] = np.array(vK, np.int64)
    out["vd_avx2"] = np.array(va, np.float32)
    out["vd_generic"] = np.array(vg, np.float32)

    M, K = 64, 512
    W = ref.quantize_type(qtype, (rng.standard_normal((M, K)) * 0.02).astype(np.float32), M, K)
    out["mm_W"] = W
    out["mm_MK"] = np.array([M, K], np.int64)
    for T in (1, 3, 8, 17):
        X = rng.standard_normal((T, K)).astype(np.float32)
        out[f"mm_X{T}"] = X
        out[f"mm_Y{T}"] = ref.mul_mat(W, M, K, X, qtype=qtype)

    E, M, K, T = 8, 32, 512, 3
    bank = ref.quantize_type(qtype, (rng.standard_normal((E * M, K)) * 0.02).astype(np.float32), E * M, K)
    out["mmid_bank"] = bank
    out["mmid_EMK"] = np.array([E, M, K], np.int64)
    for n_used, ne11 in ((2, 1), (4, 4)):
        ids = np.stack([rng.permutation(E)[:n_used] for _ in range(T)]).astype(np.int32)
        X = rng.standard_normal((T, ne11, K)).astype(np.float32)
        tag = f"{n_used}_{ne11}"
        out[f"mmid_ids_{tag}"] = ids
        out[f"mmid_X_{tag}"] = X
        out[f"mmid_Y_{tag}"] = ref.mul_mat_id(bank, M, K, E, X, ids, qtype=qtype)
    return out


def q8_0_act_inputs(rng):
    c = [rng.standard_normal(32 * 64).astype(np.float32)]
    t = np.zeros(32, np.float32); t[0] = 127.0; t[1:9] = [2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -3.5]
    c.append(t)                                                                   # exact ties after scaling
    c.append(np.zeros(32, np.float32))                                           # d = 0
    c.append((np.arange(32) - 16).astype(np.float32) * 0.25)
    c.append((rng.standard_normal(32) * 1e-30).astype(np.float32))
    c.append((rng.standard_normal(32) * 1e30).astype(np.float32))
    c.append(np.full(32, -7.0, np.float32))
    return np.concatenate(c)


def gen_q8_0(ref, rng):
    out = {}
    x = np.concatenate([q6k_encoder_inputs(rng), q8_0_act_inputs(rng)])
    out["enc_x"] = x
    out["enc_q"] = ref.quantize_type(TYPE_Q8_0, x, 1, x.size)
    rb = rng.integers(0, 256, size=(256, Q8_0), dtype=np.uint8)
    rb[:, 1] &= 0xBF                                                              # finite fp16 d
    q = np.concatenate([out["enc_q"].reshape(-1, Q8_0), rb]).ravel()
    out["deq_q"] = q
    out["deq_y"] = ref.dequant_type(TYPE_Q8_0, q, q.size // Q8_0 * 32)
    xa = q8_0_act_inputs(rng)
    out["act_x"] = xa
    out["act_q"] = ref.quantize_q8_0_act(xa)
    vw, va8, vK, va, vg = [], [], [], [], []
    for K, n, kind in ((32, 8, "enc"), (768, 8, "enc"), (4096, 8, "enc"), (27648, 4, "enc"), (4096, 8, "rand")):
        for i in range(n):
            if kind == "enc":
                w = ref.quantize_type(TYPE_Q8_0, (rng.standard_normal(K) * 0.02).astype(np.float32), 1, K)
            else:
                w = rng.integers(0, 256, size=(K // 32, Q8_0), dtype=np.uint8)
                w[:, 1] &= 0x3B
                w = w.ravel()
            a = ref.quantize_q8_0_act(rng.standard_normal(K).astype(np.float32))
            vw.append(w); va8.append(a); vK.append(K)
            va.append(ref.vec_dot_type(TYPE_Q8_0, K, w, a)); vg.append(ref.vec_dot_type(TYPE_Q8_0, K, w, a, True))
    out["vd_w"] = np.concatenate(vw)
    out["vd_a"] = np.concatenate(va8)
    out["vd_K"] = np.array(vK, np.int64)
    out["vd_avx2"] = np.array(va, np.float32)
    out["vd_generic"] = np.array(vg, np.float32)
    M, K = 64, 512
    W = ref.quantize_type(TYPE_Q8_0, (rng.standard_normal((M, K)) * 0.02).astype(np.float32), M, K)
    out["mm_W"] = W
    out["mm_MK"] = np.array([M, K], np.int64)
    for T in (1, 3, 8, 17):
        X = rng.standard_normal((T, K)).astype(np.float32)
        out[f"mm_X{T}"] = X
        out[f"mm_Y{T}"] = ref.mul_mat(W, M, K, X, qtype=TYPE_Q8_0)
    E, M, K, T = 8, 32, 512, 3
    bank = ref.quantize_type(TYPE_Q8_0, (rng.standard_normal((E * M, K)) * 0.02).astype(np.float32), E * M, K)
    out["mmid_bank"] = bank
    out["mmid_EMK"] = np.array([E, M, K], np.int64)
    for n_used, ne11 in ((2, 1), (4, 4)):
        ids = np.stack([rng.permutation(E)[:n_used] for _ in range(T)]).astype(np.int32)
        Xm = rng.standard_normal((T, ne11, K)).astype(np.float32)
        tag = f"{n_used}_{ne11}"
        out[f"mmid_ids_{tag}"] = ids
        out[f"mmid_X_{tag}"] = Xm
        out[f"mmid_Y_{tag}"] = ref.mul_mat_id(bank, M, K, E, Xm, ids, qtype=TYPE_Q8_0)
    return out


def gen_q6k(ref, rng):
    out = gen_kquant(ref, rng, TYPE_Q6_K, Q6K)
    out["vd_q6"] = out.pop("vd_w")
    return out


def gen_dq(ref, rng):
    """Dequant-then-dot vectors: the reference's dequantize_row_q8_K of Q8_K
    blocks (the activation side of the parity bar's dequant-then-dot form)
    and the reference's own beast_matvec (desktop/beast_canyon, built into
    oracle/_ref/beast) on Q4_K and Q8_0 rows with fp32 inputs."""
    from _oracle import BeastRef, TYPE_Q4_K
    beast = BeastRef()
    out = {}
    xq = np.concatenate([q8_inputs(rng), rng.standard_normal(QK * 8).astype(np.float32) * 3.0])
    q8 = ref.quantize_q8K(xq)
    out["dq8_q"] = q8
    out["dq8_y"] = ref.dequant_q8K(q8, xq.size)
    for tag, qtype in (("q4k", TYPE_Q4_K), ("q8_0", TYPE_Q8_0)):
        for K, M in ((256, 4), (4096, 16), (12288, 8)):
            w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
            W = ref.quantize_type(qtype, w, M, K)
            x = rng.standard_normal(K).astype(np.float32)
            out[f"beast_{tag}_{K}_W"] = W
            out[f"beast_{tag}_{K}_x"] = x
            out[f"beast_{tag}_{K}_y"] = beast.matvec(qtype, W, M, K, x)
    return out


def gen_beast_moe(ref, rng):
    """The reference's BurnHard routing (sp_beast_route_experts) and MoE forward
    (sp_beast_moe_forward's loop over beast_matvec and beast_silu_mul), built
    into oracle/_ref/beast: routing of logits with distinct values, ties and
    -inf, and one small forward over Q4_K banks. (A NaN logit makes the
    reference select index -1, outside its arrays: not a case to match.)"""
    from _oracle import BeastRef, TYPE_Q4_K
    beast = BeastRef()
    out = {}
    cases = [rng.standard_normal(16).astype(np.float32),
             np.array([0.5, 2.0, 2.0, -1.0, 2.0, 0.0, 1.5, 2.0], np.float32),
             np.array([1.0, -np.inf, 3.0, 2.0, 3.0, -np.inf], np.float32),
             (rng.standard_normal(128) * 3.0).astype(np.float32)]
    for i, (l, k) in enumerate(zip(cases, (4, 3, 2, 8))):
        ids, sc = beast.route(l, k)
        out[f"route{i}_logits"], out[f"route{i}_k"] = l, np.int32(k)
        out[f"route{i}_ids"], out[f"route{i}_scores"] = ids, sc
    E, k, n_embd, n_ff = 4, 2, 256, 256
    banks = {}
    for name, M, K in (("gate", n_ff, n_embd), ("up", n_ff, n_embd), ("down", n_embd, n_ff)):
        w = (rng.standard_normal((E * M, K)) * 0.05).astype(np.float32)
        banks[name] = ref.quantize_type(TYPE_Q4_K, w, E * M, K)
    logits = rng.standard_normal(E).astype(np.float32)
    hidden = rng.standard_normal(n_embd).astype(np.float32)
    y, ids, sc = beast.moe(TYPE_Q4_K, banks["gate"], banks["up"], banks["down"], E, n_embd, n_ff, logits, k, hidden)
    for name, b in banks.items():
        out[f"moe_{name}"] = b
    out["moe_shape"] = np.array([E, k, n_embd, n_ff], np.int32)
    out["moe_logits"], out["moe_hidden"] = logits, hidden
    out["moe_y"], out["moe_ids"], out["moe_scores"] = y, ids, sc
    return out


def main():
    if ref_library_path() is None:
        sys.exit("oracle/_ref is not built (make -C oracle ref)")
    which = set(sys.argv[1:]) or {"q4k", "q5k", "q6k", "q8_0", "dq", "beast_moe"}
    ref = Ref()
    if "beast_moe" in which:
        out = gen_beast_moe(ref, np.random.default_rng(0xBEA5))
        path = os.path.join(HERE, "beast_moe_golden.npz")
        np.savez_compressed(path, **out)
        print(f"wrote {path} ({os.path.getsize(path)/1024:.0f} KiB, {len(out)} arrays) using {ref.path}")
    if "dq" in which:
        out = gen_dq(ref, np.random.default_rng(0xD0D0))
        path = os.path.join(HERE, "dq_golden.npz")
        np.savez_compressed(path, **out)
        print(f"wrote {path} ({os.path.getsize(path)/1024:.0f} KiB, {len(out)} arrays) using {ref.path}")
    for tag, fn in (("q6k", lambda: gen_q6k(ref, np.random.default_rng(0x6B6B))),
                    ("q5k", lambda: gen_kquant(ref, np.random.default_rng(0x5B5B), TYPE_Q5_K, Q5K)),
                    ("q8_0", lambda: gen_q8_0(ref, np.random.default_rng(0x8080)))):
        if tag not in which:
            continue
        out = fn()
        path = os.path.join(HERE, f"{tag}_golden.npz")
        np.savez_compressed(path, **out)
        print(f"wrote {path} ({os.path.getsize(path)/1024:.0f} KiB, {len(out)} arrays) using {ref.path}")
    if "q4k" not in which:
        return
    rng = np.random.default_rng(0xDEADBEEF)
    out = {}

    x = encoder_inputs(rng)
    out["enc_x"] = x
    out["enc_q"] = ref.quantize_q4K(x, 1, x.size)

    q = out["enc_q"].reshape(-1, 144).copy()
    rb = rng.integers(0, 256, size=(64, 144), dtype=np.uint8)
    rb[:, 1] &= 0xBF            # finite fp16 d
    rb[:, 3] &= 0xBF            # finite fp16 dmin
    q = np.concatenate([q, rb]).ravel()
    out["deq_q"] = q
    out["deq_y"] = ref.dequant(q, q.size // 144 * QK)

    xq = q8_inputs(rng)
    out["q8_x"] = xq
    out["q8_y"] = ref.quantize_q8K(xq)

    # vec_dot cases: K in {256, 768, 4096, 27648}
    vq4, vq8, vK, va, vg = [], [], [], [], []
    for K, n in ((256, 8), (768, 8), (4096, 8), (27648, 4)):
        for i in range(n):
            w = ref.quantize_q4K((rng.standard_normal(K) * 0.02).astype(np.float32), 1, K)
            a = ref.quantize_q8K(rng.standard_normal(K).astype(np.float32))
            vq4.append(w); vq8.append(a); vK.append(K)
            va.append(ref.vec_dot(K, w, a)); vg.append(ref.vec_dot(K, w, a, generic=True))
    out["vd_q4"] = np.concatenate(vq4)
    out["vd_q8"] = np.concatenate(vq8)
    out["vd_K"] = np.array(vK, np.int64)
    out["vd_avx2"] = np.array(va, np.float32)
    out["vd_generic"] = np.array(vg, np.float32)

    # GGML_OP_MUL_MAT
    M, K = 64, 512
    W = ref.quantize_q4K((rng.standard_normal((M, K)) * 0.02).astype(np.float32), M, K)
    out["mm_W"] = W
    out["mm_MK"] = np.array([M, K], np.int64)
    for T in (1, 3, 8, 17):
        X = rng.standard_normal((T, K)).astype(np.float32)
        out[f"mm_X{T}"] = X
        out[f"mm_Y{T}"] = ref.mul_mat(W, M, K, X)

    # GGML_OP_MUL_MAT_ID
    E, M, K, T = 8, 32, 512, 3
    bank = ref.quantize_q4K((rng.standard_normal((E * M, K)) * 0.02).astype(np.float32), E * M, K)
    out["mmid_bank"] = bank
    out["mmid_EMK"] = np.array([E, M, K], np.int64)
    for n_used, ne11 in ((2, 1), (4, 4)):
        ids = np.stack([rng.permutation(E)[:n_used] for _ in range(T)]).astype(np.int32)
        X = rng.standard_normal((T, ne11, K)).astype(np.float32)
        tag = f"{n_used}_{ne11}"
        out[f"mmid_ids_{tag}"] = ids
        out[f"mmid_X_{tag}"] = X
        out[f"mmid_Y_{tag}"] = ref.mul_mat_id(bank, M, K, E, X, ids)

    path = os.path.join(HERE, "q4k_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)/1024:.0f} KiB, {len(out)} arrays) using {ref.path}")


if __name__ == "__main__":
    main()
