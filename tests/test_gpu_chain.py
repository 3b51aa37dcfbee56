"""GPU parity of decode chains (spq4k_chain_*, include/spq4k.h): dependent
T = 1 stages in one persistent launch -- the dense decode layer of the
reference's build_block_decode (desktop/engine/src/forward.cpp:2663-2856)
around its attention core, and the output head (:3411-3413).

Every stage is checked on the chain's own intermediate buffers (the inputs it
read are the outputs earlier stages wrote):
  - x_out == in0 + in1 bit for bit (ggml_add in fp32);
  - the stage's outputs equal the per-op entry points on the same input bit
    for bit: spq4k_mul_mat (the decode kernel, whose per-lane sums and DPP
    reduction the chain shares) for plain stages, spq4k_mul_mat_swiglu for
    the gate / up pair; normed stages are fed the oracle's rms_norm of
    in0 + in1 (the CPU's arithmetic, bit-exact), so the chain's own norm is
    checked through its outputs;
  - sampled rows are within the parity bar of the CPU oracle (each output
    within close_enough of ggml_vec_dot_q4_K_q8_K's order or of the
    dequant-then-dot sum, tests/desktop/test_sp_kernels.cpp:34-48);
  - repeated launches give identical outputs (the grid-barrier counters
    carry over between launches).
Shapes: the 8B layer (4096 / 1024 / 12288) for two layers plus an output
head, and ragged chains (rows fewer than the grid's waves, K = 256, 2048,
5120, 6144 and 12288, four matrices in a stage, a stage no wave of some
workgroups touches)."""
import numpy as np
import pytest

from _oracle import close_enough, parity_ok

pytestmark = pytest.mark.gpu
EPS = 1e-6
Q4K = 144


def _weights(ctx, M, K, seed):
    """seeded N(0, 0.02) Q4_K weights synthesised and encoded on the GPU"""
    import spq4k
    from spq4k.hip import DeviceArray, download
    tmp = DeviceArray(M * K, np.float32)
    W = ctx.alloc_weights(M, K)
    ctx.synth_fill_dev(tmp.ptr, M * K, seed, spq4k.DIST_NORMAL, K, 0.0, 0.02, 1.0, 0)
    ctx.quantize_chunk_dev(spq4k.TYPE_Q4_K, tmp.ptr, W.data_ptr, M, K)
    ctx.synchronize()
    tmp.free()
    return W, download(W.data_ptr, W.nbytes)


def _sample_rows(M, n=64):
    rows = set(range(min(M, 16))) | set(range(max(0, M - 16), M))
    rows |= set(np.linspace(0, M - 1, n).astype(int).tolist())
    return np.array(sorted(rows))


def _rows_of(wb, K, rows):
    rb = K // 256 * Q4K
    return np.ascontiguousarray(wb.reshape(-1, rb)[rows]).ravel()


def _bits_equal(a, b, what):
    a, b = np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32)
    if not np.array_equal(a.view(np.uint32), b.view(np.uint32)):
        i = int(np.argmax(a.view(np.uint32) != b.view(np.uint32)))
        raise AssertionError(f"{what}: {int((a.view(np.uint32) != b.view(np.uint32)).sum())} of {a.size} differ; "
                             f"first [{i}] {a.ravel()[i]!r} vs {b.ravel()[i]!r}")


class _Net:
    """device buffers and weights of a chain; stage dicts for Context.chain_create"""

    def __init__(self, ctx):
        self.ctx, self.bufs, self.w = ctx, {}, {}

    def buf(self, name, n, init=None):
        from spq4k.hip import DeviceArray
        d = DeviceArray.from_host(init.astype(np.float32)) if init is not None else DeviceArray(n, np.float32)
        if init is None:
            d.fill_byte(0)
        self.bufs[name] = d
        return d.ptr

    def weight(self, name, M, K, seed):
        self.w[name] = _weights(self.ctx, M, K, seed)
        return self.w[name][0]

    def host(self, name):
        return self.bufs[name].to_host()


def _check_stage(ctx, oracle, net, st, idx):
    """bit-exact against the per-op path on the same input, parity against the oracle"""
    from spq4k.hip import DeviceArray
    in0 = net.host(st["in0_name"])
    x = in0 + net.host(st["in1_name"]) if st.get("in1_name") else in0
    if st.get("x_out_name"):
        _bits_equal(net.host(st["x_out_name"]), x, f"stage {idx} x_out")
    if st.get("norm_name"):
        xb = oracle.rms_norm(x[None, :], net.host(st["norm_name"]), EPS)[0]
    else:
        xb = x
    xd = DeviceArray.from_host(xb.astype(np.float32))
    names = st["w_names"]
    K = xb.size
    if st.get("glu"):
        (Wg, gb), (Wu, ub) = net.w[names[0]], net.w[names[1]]
        ref = DeviceArray(Wg.M, np.float32)
        ctx.mul_mat_swiglu_dev(Wg, Wu, xd.ptr, None, EPS, ref.ptr, 1)
        ctx.synchronize()
        got = net.host(st["y_names"][0])
        _bits_equal(got, ref.to_host(), f"stage {idx} gate/up vs spq4k_mul_mat_swiglu")
        rows = _sample_rows(Wg.M)
        g = oracle.mul_mat(_rows_of(gb, K, rows), rows.size, K, xb[None, :])[0]
        u = oracle.mul_mat(_rows_of(ub, K, rows), rows.size, K, xb[None, :])[0]
        ok = close_enough(got[rows], oracle.swiglu(g, u))
        assert ok.all(), f"stage {idx} swiglu vs oracle: {int((~ok).sum())} of {ok.size}"
        return
    for name, yname in zip(names, st["y_names"]):
        W, wb = net.w[name]
        ref = DeviceArray(W.M, np.float32)
        ctx.mul_mat_dev(W, xd.ptr, ref.ptr, 1)
        ctx.synchronize()
        got = net.host(yname)
        if st.get("bitwise", True):
            _bits_equal(got, ref.to_host(), f"stage {idx} {name} vs spq4k_mul_mat")
        rows = _sample_rows(W.M)
        Wr = _rows_of(wb, K, rows)
        exp = oracle.mul_mat(Wr, rows.size, K, xb[None, :])[0]
        exact = oracle.mul_mat_dq_f64(12, Wr, rows.size, K, xb[None, :])[0]
        ok = parity_ok(got[rows], exp, exact)
        assert ok.all(), f"stage {idx} {name} vs oracle: {int((~ok).sum())} of {ok.size}"


def _layer_net(ctx, n_layers, n_embd, n_q, n_kv, n_ff, n_vocab, seed0=1000):
    """the stages of build_block_decode for n_layers layers and the output head,
    the attention output replaced by the q projection (same shape)"""
    net = _Net(ctx)
    rng = np.random.default_rng(seed0)
    net.buf("x0", n_embd, rng.standard_normal(n_embd).astype(np.float32))
    stages, meta = [], []
    prev = None
    for l in range(n_layers):
        for nm, M, K in (("q", n_q, n_embd), ("k", n_kv, n_embd), ("v", n_kv, n_embd), ("o", n_embd, n_q),
                         ("gate", n_ff, n_embd), ("up", n_ff, n_embd), ("down", n_embd, n_ff)):
            net.weight(f"{nm}{l}", M, K, seed0 + 17 * l + len(net.w))
        for nm, M in (("q", n_q), ("k", n_kv), ("v", n_kv), ("o", n_embd), ("g", n_ff), ("d", n_embd),
                      ("xres", n_embd), ("h", n_embd)):
            net.buf(f"{nm}{l}", M)
        net.buf(f"attn_norm{l}", n_embd, (1.0 + 0.2 * rng.standard_normal(n_embd)).astype(np.float32))
        net.buf(f"ffn_norm{l}", n_embd, (1.0 + 0.2 * rng.standard_normal(n_embd)).astype(np.float32))
        # A: x = h + down of the previous layer (the residual), rms_norm * attn_norm, q/k/v
        a = {"w_names": [f"q{l}", f"k{l}", f"v{l}"], "y_names": [f"q{l}", f"k{l}", f"v{l}"],
             "in0_name": "x0" if prev is None else f"h{prev}", "in1_name": None if prev is None else f"d{prev}",
             "x_out_name": f"xres{l}", "norm_name": f"attn_norm{l}"}
        # B: o projection of the attention output (here the q projection)
        b = {"w_names": [f"o{l}"], "y_names": [f"o{l}"], "in0_name": f"q{l}"}
        # C: x = x + o, rms_norm * ffn_norm, silu(gate) * up
        c = {"w_names": [f"gate{l}", f"up{l}"], "y_names": [f"g{l}"], "glu": 1, "in0_name": f"xres{l}",
             "in1_name": f"o{l}", "x_out_name": f"h{l}", "norm_name": f"ffn_norm{l}"}
        # D: down
        d = {"w_names": [f"down{l}"], "y_names": [f"d{l}"], "in0_name": f"g{l}"}
        meta += [a, b, c, d]
        prev = l
    net.weight("out", n_vocab, n_embd, seed0 + 999)
    net.buf("logits", n_vocab)
    net.buf("xfin", n_embd)
    net.buf("out_norm", n_embd, (1.0 + 0.2 * rng.standard_normal(n_embd)).astype(np.float32))
    meta.append({"w_names": ["out"], "y_names": ["logits"], "in0_name": f"h{prev}", "in1_name": f"d{prev}",
                 "x_out_name": "xfin", "norm_name": "out_norm"})
    for m in meta:
        stages.append(_to_stage(net, m))
    return net, stages, meta


def _to_stage(net, m):
    st = {"W": [net.w[n][0] for n in m["w_names"]], "y": [net.bufs[n].ptr for n in m["y_names"]],
          "in0": net.bufs[m["in0_name"]].ptr}
    if m.get("glu"):
        st["glu"] = 1
    for key, nk in (("in1", "in1_name"), ("x_out", "x_out_name"), ("norm_w", "norm_name")):
        if m.get(nk):
            st[key] = net.bufs[m[nk]].ptr
    return st


def _outputs(net, meta):
    names = []
    for m in meta:
        names += m["y_names"] + ([m["x_out_name"]] if m.get("x_out_name") else [])
    return {n: net.host(n) for n in names}


@pytest.fixture(params=[1, 2], ids=["form1", "form2"])
def form(request, monkeypatch):
    """the chain's form: 1 a grid barrier every stage (k_chain.hip, the
    default), 2 the one-hop exchange (k_chain2.hip, SPQ4K_CHAIN_V=2 when the
    data flow allows it)"""
    monkeypatch.setenv("SPQ4K_CHAIN_V", str(request.param))
    return request.param


def test_chain_8b_layers(ctx, oracle, form):
    """two 8B decode layers and a 4096-row output head in one launch"""
    net, stages, meta = _layer_net(ctx, 2, 4096, 4096, 1024, 12288, 4096)
    ch = ctx.chain_create(stages, EPS)
    assert ch.version == form
    ch.run()
    ch.status()
    first = _outputs(net, meta)
    for i, m in enumerate(meta):
        _check_stage(ctx, oracle, net, m, i)
    # launches after the first reuse the counters: same outputs
    for _ in range(3):
        ch.run()
    ch.status()
    again = _outputs(net, meta)
    for n in first:
        _bits_equal(again[n], first[n], f"relaunch {n}")
    ch.free()


def test_chain_ragged(ctx, oracle, form):
    """rows fewer than the grid's waves, partial 16-block passes, four matrices
    in a stage, K from 256 to 12288"""
    net = _Net(ctx)
    rng = np.random.default_rng(7)
    meta = []
    net.buf("x", 2048, rng.standard_normal(2048).astype(np.float32))
    net.buf("x2", 2048, rng.standard_normal(2048).astype(np.float32))
    net.buf("nw", 2048, (1.0 + 0.2 * rng.standard_normal(2048)).astype(np.float32))
    # 1: four matrices of K = 2048 (8 blocks: a partial pass), 37..300 rows
    for nm, M in (("a", 37), ("b", 300), ("c", 1), ("e", 129)):
        net.weight(nm, M, 2048, 50 + M)
        net.buf("y" + nm, M)
    net.buf("xo1", 2048)
    meta.append({"w_names": ["a", "b", "c", "e"], "y_names": ["ya", "yb", "yc", "ye"], "in0_name": "x",
                 "in1_name": "x2", "x_out_name": "xo1", "norm_name": "nw", "bitwise": False})
    # 2: K = 5120 from stage 1's outputs? K must match the input length: feed a
    #    5120-long vector assembled by the host, plain stage (decode kernel's NB 20)
    net.buf("x5", 5120, rng.standard_normal(5120).astype(np.float32))
    net.weight("f", 3000, 5120, 91)
    net.buf("yf", 3000)
    meta.append({"w_names": ["f"], "y_names": ["yf"], "in0_name": "x5"})
    # 3: K = 256 (one block), glu pair of 300 rows, input = 256 values of stage 2's output
    net.weight("g", 300, 256, 92)
    net.weight("u", 300, 256, 93)
    net.buf("yg", 300)
    meta.append({"w_names": ["g", "u"], "y_names": ["yg"], "glu": 1, "in0_name": "yf_head"})
    net.bufs["yf_head"] = net.bufs["yf"]    # the first 256 of stage 2's outputs
    # 4: K = 12288 over 1000 rows (three 16-block passes), input a host vector
    net.buf("x12", 12288, rng.standard_normal(12288).astype(np.float32))
    net.weight("h", 1000, 12288, 94)
    net.buf("yh", 1000)
    meta.append({"w_names": ["h"], "y_names": ["yh"], "in0_name": "x12"})
    # 5: K = 6144, normed (two vectors of 6144 fill the 12288-value staging),
    #    input = stage 4's residual-free output padded by the host: a host vector
    net.buf("x6", 6144, rng.standard_normal(6144).astype(np.float32))
    net.buf("nw6", 6144, (1.0 + 0.2 * rng.standard_normal(6144)).astype(np.float32))
    net.weight("k6", 2500, 6144, 95)
    net.buf("yk6", 2500)
    meta.append({"w_names": ["k6"], "y_names": ["yk6"], "in0_name": "x6", "norm_name": "nw6", "bitwise": False})
    stages = [_to_stage(net, m) for m in meta]
    ch = ctx.chain_create(stages, EPS)
    assert ch.version == form
    ch.run()
    ch.status()
    for i, m in enumerate(meta):
        if m["in0_name"] == "yf_head":
            # the glu stage reads the first 256 outputs of stage 2 (K = 256: the
            # per-op path runs the generic kernel here, so the oracle alone)
            xg = net.host("yf")[:256]
            g = oracle.mul_mat(net.w["g"][1], 300, 256, xg[None, :])[0]
            u = oracle.mul_mat(net.w["u"][1], 300, 256, xg[None, :])[0]
            got = net.host("yg")
            ok = close_enough(got, oracle.swiglu(g, u))
            assert ok.all(), f"glu K=256: {int((~ok).sum())} of {ok.size}"
            continue
        _check_stage(ctx, oracle, net, m, i)
    ch.free()


def test_chain_rejects_bad_stages(ctx):
    import spq4k
    from spq4k.hip import DeviceArray
    W, _ = _weights(ctx, 64, 4096, 3)
    Wbig, _ = _weights(ctx, 16, 27648, 4)
    W12, _ = _weights(ctx, 16, 12288, 5)
    x = DeviceArray(27648, np.float32)
    y = DeviceArray(4096, np.float32)
    z = DeviceArray(16384, np.float32)
    good = {"W": [W], "y": [y.ptr], "in0": x.ptr}
    bad = [
        {"W": [W, W, W], "y": [y.ptr, y.ptr, y.ptr], "glu": 1, "in0": x.ptr},          # glu needs two
        {"W": [Wbig], "y": [y.ptr], "in0": x.ptr},                                        # K > 12288
        {"W": [W], "y": [y.ptr + 4], "in0": x.ptr},                                       # misaligned output
        {"W": [W], "y": [x.ptr + 64], "in0": x.ptr},                                      # output overlaps input
        {"W": [W], "y": [z.ptr + 512], "in0": x.ptr, "norm_w": z.ptr},                    # output overlaps norm_w
        {"W": [W, W], "y": [y.ptr, y.ptr + 128], "in0": x.ptr},                           # outputs overlap
        {"W": [W], "y": [z.ptr + 256], "in0": x.ptr, "x_out": z.ptr},                     # output overlaps x_out
        {"W": [W], "y": [y.ptr], "in0": x.ptr, "x_out": z.ptr, "norm_w": z.ptr + 4096},  # x_out overlaps norm_w
        {"W": [W12], "y": [y.ptr], "in0": x.ptr, "in1": x.ptr},                          # 2 x 12288 inputs
        {"W": [W], "y": [y.ptr], "in0": 0},                                               # no input
    ]
    for i, st in enumerate(bad):
        with pytest.raises(spq4k.Spq4kError) as e:
            ctx.chain_create([good, st], EPS)
        assert e.value.rc == -22, f"case {i}: rc {e.value.rc}"
    with pytest.raises(spq4k.Spq4kError):
        ctx.chain_create([], EPS)
    ch = ctx.chain_create([good], EPS)
    ch.run()
    ch.status()
    ch.free()


def test_chain_form1_when_a_stage_overwrites_an_input(ctx, oracle, monkeypatch):
    """a stage that writes memory an earlier stage read keeps the grid barrier
    (form 1) even when form 2 is asked for: form 2 lets stages overlap, which
    only holds when no stage writes what an earlier one reads; the outputs
    still match the per-op path"""
    net = _Net(ctx)
    rng = np.random.default_rng(11)
    net.buf("x", 4096, rng.standard_normal(4096).astype(np.float32))
    net.weight("a", 4096, 4096, 61)
    net.weight("b", 4096, 4096, 62)
    net.buf("y1", 4096)
    # stage 0 reads x; stage 1 reads stage 0's output and overwrites x
    m0 = {"w_names": ["a"], "y_names": ["y1"], "in0_name": "x"}
    m1 = {"w_names": ["b"], "y_names": ["x"], "in0_name": "y1"}
    x0 = net.host("x")
    monkeypatch.setenv("SPQ4K_CHAIN_V", "2")
    ch = ctx.chain_create([_to_stage(net, m0), _to_stage(net, m1)], EPS)
    assert ch.version == 1
    ch.run()
    ch.status()
    y1 = net.host("y1")
    W, wb = net.w["a"]
    rows = _sample_rows(4096)
    ok = parity_ok(y1[rows], oracle.mul_mat(_rows_of(wb, 4096, rows), rows.size, 4096, x0[None, :])[0],
                   oracle.mul_mat_dq_f64(12, _rows_of(wb, 4096, rows), rows.size, 4096, x0[None, :])[0])
    assert ok.all()
    _check_stage(ctx, oracle, net, m1, 1)
    ch.free()


def test_chain_stamps(ctx, monkeypatch):
    """form 2's stage timestamps (include/spq4k_diag.h) are written for every
    workgroup and stage, in order: inputs gathered <= x formed <= activations
    ready <= rows done <= the next stage's inputs gathered"""
    from spq4k.hip import DeviceArray
    net, stages, meta = _layer_net(ctx, 1, 4096, 4096, 1024, 12288, 4096)
    monkeypatch.setenv("SPQ4K_CHAIN_V", "2")
    ch = ctx.chain_create(stages, EPS)
    v, grid, n = ch.info()
    assert v == 2 and n == len(stages) and grid > 0
    st = DeviceArray(grid * n * 4, np.uint64)
    st.fill_byte(0)
    ch.set_stamps(st.ptr)
    ch.run()
    ch.status()
    s = st.to_host().reshape(grid, n, 4).astype(np.int64)
    assert (s > 0).all()
    assert (s[:, :, 0] <= s[:, :, 3]).all() and (s[:, :, 3] <= s[:, :, 1]).all()
    assert (s[:, :, 1] <= s[:, :, 2]).all()
    assert (s[:, :-1, 2] <= s[:, 1:, 0]).all()
    ch.set_stamps(None)
    ch.free()
