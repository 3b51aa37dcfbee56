"""GPU residency of a GGUF file's weights (spq4k_model_load,
include/spq4k_gguf.h) against the reference's loader behaviour
(LlamaWeights::load_backend_offload_, desktop/engine/src/llama_weights.cpp:
483-720).

The model file is written by the reference's own GGUF writer (oracle/_ref):
three layers of Q4_K / Q5_K / Q6_K / Q8_0 matrices and Q4_K / Q8_0 expert
banks, F32 norms, a Q4_K token embedding and a Q6_K output, weights from the
oracle's encoders (N(0, 0.02)). Checks:
  - the resident set is exactly the matrices of the runnable types that the
    offload settings place on the GPU (full, partial, none);
  - the device bytes are the file's bytes, also after the file is closed;
  - matmuls on resident weights equal the oracle on the file's bytes
    (close_enough), dense and expert-gathered;
  - the expert split keeps experts [pivot, E) on the GPU under the bank's own
    name, as the reference's loader does."""
import numpy as np
import pytest

from _gguf_ref import RefGguf
from _oracle import TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, close_enough

pytestmark = pytest.mark.gpu
spq4k = pytest.importorskip("spq4k")

D, FF, NE, MX, VOCAB, LAYERS = 512, 768, 8, 64, 1000, 3


def _quant(oracle, t, rows, k, rng):
    x = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
    if t == TYPE_Q8_0:
        return oracle.quantize_q8_0(x, ref_encoder=True)
    return oracle.quantize(t, x)


def _spec():
    """(name, ggml type, ne): the model's tensors in file order."""
    s = [("token_embd.weight", TYPE_Q4_K, (D, VOCAB))]
    for L in range(LAYERS):
        s += [(f"blk.{L}.attn_norm.weight", 0, (D,)),
              (f"blk.{L}.attn_q.weight", TYPE_Q4_K, (D, D)),
              (f"blk.{L}.attn_v.weight", TYPE_Q6_K, (D, 128)),
              (f"blk.{L}.ffn_up.weight", TYPE_Q8_0, (D, 384)),
              (f"blk.{L}.ffn_down.weight", TYPE_Q5_K, (FF, D)),
              (f"blk.{L}.ffn_gate_exps.weight", TYPE_Q4_K, (D, MX, NE)),
              (f"blk.{L}.ffn_down_exps.weight", TYPE_Q8_0, (MX, D, NE))]
    s += [("output_norm.weight", 0, (D,)), ("output.weight", TYPE_Q6_K, (D, VOCAB))]
    return s


@pytest.fixture(scope="module")
def model_file(ref, oracle, tmp_path_factory):
    rng = np.random.default_rng(41)
    tensors, data = [], {}
    for name, t, ne in _spec():
        if t == 0:
            b = rng.standard_normal(ne[0]).astype(np.float32).view(np.uint8)
        else:
            rows = int(np.prod(ne[1:]))
            b = _quant(oracle, t, rows, ne[0], rng)
        tensors.append((name, t, ne, b))
        data[name] = (t, ne, b)
    path = tmp_path_factory.mktemp("model") / "model.gguf"
    assert RefGguf(ref).write(path, tensors, [("general.architecture", 8, "llama")])
    return str(path), data


def _runnable(data):
    return {n for n, (t, ne, b) in data.items() if t != 0 and len(ne) >= 2}


def _device_bytes(w):
    from spq4k.hip import download
    return download(w.data_ptr, w.nbytes)


def test_full_offload(ctx, oracle, model_file):
    path, data = model_file
    with spq4k.Gguf(path) as g:
        m = ctx.load_model(g, -1, 0)
    assert set(m.names()) == _runnable(data)
    assert m.nbytes == sum((b.size + 255) // 256 * 256 for n, (t, ne, b) in data.items() if n in _runnable(data))
    for name in m.names():
        t, ne, b = data[name]
        w = m.weights(name)
        assert (w.type, w.K, w.M, w.E) == (t, ne[0], ne[1], ne[2] if len(ne) > 2 else 1), name
        np.testing.assert_array_equal(_device_bytes(w), b, err_msg=name)
        assert m.expert_base(name) == 0
    assert m.weights("blk.0.attn_norm.weight") is None and m.expert_base("nope") == -1
    rng = np.random.default_rng(3)
    for name in ("blk.1.attn_q.weight", "blk.2.attn_v.weight", "blk.0.ffn_up.weight", "blk.1.ffn_down.weight",
                 "output.weight"):
        t, ne, b = data[name]
        for T in (1, 5):
            X = rng.standard_normal((T, ne[0])).astype(np.float32)
            got = ctx.mul_mat(m.weights(name), X)
            exp = (oracle.mul_mat_q8_0(b, ne[1], ne[0], X) if t == TYPE_Q8_0
                   else oracle.mul_mat_type(t, b, ne[1], ne[0], X))
            assert close_enough(got, exp).all(), (name, T)
    m.free()


@pytest.mark.parametrize("n_gpu_layers", [0, 1, 2, 3, 7])
def test_partial_offload(ctx, model_file, n_gpu_layers):
    path, data = model_file
    with spq4k.Gguf(path) as g:
        m = ctx.load_model(g, n_gpu_layers, 0)
    full = n_gpu_layers >= LAYERS
    expect = {n for n in _runnable(data)
              if full or (n.startswith("blk.") and int(n.split(".")[1]) < n_gpu_layers)}
    assert set(m.names()) == expect
    for name in m.names():
        np.testing.assert_array_equal(_device_bytes(m.weights(name)), data[name][2], err_msg=name)
    if n_gpu_layers == 0:
        assert m.nbytes == 0
    m.free()


@pytest.mark.parametrize("experts_on_cpu", [3, 100])
def test_expert_split(ctx, oracle, model_file, experts_on_cpu):
    path, data = model_file
    with spq4k.Gguf(path) as g:
        m = ctx.load_model(g, -1, experts_on_cpu)
    pivot = min(experts_on_cpu, NE - 1)
    rng = np.random.default_rng(9)
    for name in ("blk.0.ffn_gate_exps.weight", "blk.2.ffn_down_exps.weight"):
        t, ne, b = data[name]
        w = m.weights(name)
        stride = b.size // NE
        assert m.expert_base(name) == pivot and w.E == NE - pivot
        np.testing.assert_array_equal(_device_bytes(w), b[pivot * stride:], err_msg=name)
        # tokens routed to experts >= pivot: the GPU bank takes ids - pivot
        T, k = 4, 2
        ids = np.stack([rng.choice(np.arange(pivot, NE), min(k, NE - pivot), replace=False) for _ in range(T)])
        ids = ids.astype(np.int32)
        X = rng.standard_normal((T, 1, ne[0])).astype(np.float32)
        got = ctx.mul_mat_id(w, X, ids - pivot)
        exp = (oracle.mul_mat_id_q8_0(b, ne[1], ne[0], NE, X, ids) if t == TYPE_Q8_0
               else oracle.mul_mat_id_type(t, b, ne[1], ne[0], NE, X, ids))
        assert close_enough(got, exp).all(), name
    # dense tensors are not split
    assert m.expert_base("blk.0.attn_q.weight") == 0
    m.free()


def test_reload_and_errors(ctx, model_file):
    path, _ = model_file
    g = spq4k.Gguf(path)
    a = ctx.load_model(g)
    b = ctx.load_model(g)
    assert a.names() == b.names() and a.nbytes == b.nbytes
    a.free()
    w = b.weights("output.weight")
    np.testing.assert_array_equal(_device_bytes(w)[:64], g.tensor_bytes(g.find_tensor("output.weight"))[:64])
    b.free()
    g.close()
