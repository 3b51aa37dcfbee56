#!/usr/bin/env python3
"""bench.py — Q4_K dequant-matvec on one MI355X (gfx950).

Default workload: one decode step of an 8B-class
dense model at batch 1 — 36 layers of q 4096x4096, k/v 1024x4096, o 4096x4096,
gate/up 12288x4096, down 4096x12288, plus lm_head 151936x4096, all Q4_K,
weights seeded N(0, 0.02) and quantised on the GPU by the bit-exact
quantize_row_q4_K port, activations N(0, 1) fp32. A step respects the decode
dependency chain: [q,k,v] -> o -> [gate,up] -> down per layer, then lm_head
(matrices that share an input run as one grouped launch). The whole step is
captured once as a HIP graph and replayed.

Metric: effective HBM GB/s = algorithmic bytes of the step (Q4_K weights +
fp32 x and y of every matvec: 4,268,590,592 B) / step time; also tok/s-equiv
and % of the 8 TB/s peak. Every launch of the step is gemv_decode_kernel, so
the HIP events around the timed replays give that kernel's average launch
duration directly. Beside it ("chain"), the same weights run as one
dependent decode chain in one cooperative launch of chain_kernel
(spq4k_chain_run): per layer rms_norm * attn_norm -> [q,k,v] -> o -> residual
add, rms_norm * ffn_norm -> silu(gate) * up -> down -> residual add, then the
output norm and lm_head, each stage reading what the stages before it wrote
(the q projection stands in for the attention output, which is not on this
path). Each stage kind (q/k/v, o, gate/up, down, lm_head) is also
replayed on its own for a per-stage breakdown. CPU baseline: the reference's
own ggml CPU path (oracle/_ref, built from /root/reference sources) on a
bounded sample of the same workload (layers 0-9, 1.09 GB, larger than the
host's last-level cache), timed on this host with 16 and with 4 threads;
its outputs are checked against the GPU's on identical inputs.

  python bench.py [--steps K] [--warmup W] [--gpus 1]
                  [--config decode8b|gemv4096|largek|prefill|moe|q6k|q5k|q8_0|single|gguf|fusion|copy|floor]
                  [--M M --K K --T T --qtype TYPE]   (--config single)

--config q6k / q5k / q8_0 measure the Q6_K / Q5_K / Q8_0 tensors a Q4_K model
file can carry beside its Q4_K ones (attn_v, ffn_down, output; the MoE
down-projection bank) with the same cold-weight method. --config single
times one matrix shape of one weight type (ggml type id: 8 Q8_0, 12 Q4_K,
13 Q5_K, 14 Q6_K) the same way, for profiling one kernel. --config gguf writes
a synthetic GGUF file of 8B-model Q4_K / Q6_K tensors (12 layers and the
output matrix, 1.66 GB) to the temporary directory and times making it
resident (spq4k_model_load) against a per-tensor hipMemcpy from the file
mapping. --config fusion times the decode (T = 1) pre-norm projections and
SwiGLU front half of the 8B layer fused (one launch) and unfused (the norm,
the matvec, the element-wise pass), cold.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "shannon-prime-burnhard_amd"))

import spq4k  # noqa: E402
from spq4k.hip import DeviceArray, Event, Graph, mem_info  # noqa: E402

PEAK_HBM = 8.0e12
Q4K_B = 144

# 8B dense layer (Qwen3-8B-like)
HID, KV, FFN, VOCAB, LAYERS = 4096, 1024, 12288, 151936, 36


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def q4k_bytes(M, K):
    return M * (K // 256) * Q4K_B



class Synth:
    """Seeded weights synthesised and Q4_K-encoded on the device."""

    def __init__(self, ctx, max_elems):
        self.ctx = ctx
        self.tmp = DeviceArray(max_elems, np.float32)

    def weights(self, M, K, seed, dist=spq4k.DIST_NORMAL, outlier=1.0, qtype=spq4k.TYPE_Q4_K, E=1):
        w = self.ctx.alloc_weights(M, K, E, type=qtype)
        self.ctx.synth_fill_dev(self.tmp.ptr, E * M * K, seed, dist, K, 0.0, 0.02, outlier, 0)
        self.ctx.quantize_chunk_dev(qtype, self.tmp.ptr, w.data_ptr, E * M, K)
        return w

    def activations(self, n, seed):
        a = DeviceArray(n, np.float32)
        self.ctx.synth_fill_dev(a.ptr, n, seed, spq4k.DIST_NORMAL, 0, 0.0, 1.0, 1.0, 0)
        return a


# ---------------------------------------------------------------------------
def build_decode8b(ctx):
    """Weights, activations and the stage list of one 8B decode step."""
    syn = Synth(ctx, VOCAB * HID)
    stages = []   # (name, [weights], x, [y], bytes, matvecs)
    seed = 1000
    for L in range(LAYERS):
        q = syn.weights(HID, HID, seed + 0)
        k = syn.weights(KV, HID, seed + 1)
        v = syn.weights(KV, HID, seed + 2)
        o = syn.weights(HID, HID, seed + 3)
        g = syn.weights(FFN, HID, seed + 4)
        u = syn.weights(FFN, HID, seed + 5)
        d = syn.weights(HID, FFN, seed + 6)
        seed += 10
        x_att = syn.activations(HID, seed + 100000)
        x_o = syn.activations(HID, seed + 100001)
        x_ffn = syn.activations(HID, seed + 100002)
        x_dn = syn.activations(FFN, seed + 100003)
        yq, yk, yv = DeviceArray(HID), DeviceArray(KV), DeviceArray(KV)
        yo, yg, yu, yd = DeviceArray(HID), DeviceArray(FFN), DeviceArray(FFN), DeviceArray(HID)
        stages.append((f"L{L}.qkv", [q, k, v], x_att, [yq, yk, yv]))
        stages.append((f"L{L}.o", [o], x_o, [yo]))
        stages.append((f"L{L}.gate_up", [g, u], x_ffn, [yg, yu]))
        stages.append((f"L{L}.down", [d], x_dn, [yd]))
    lm = syn.weights(VOCAB, HID, seed + 7)
    x_lm = syn.activations(HID, seed + 100004)
    stages.append(("lm_head", [lm], x_lm, [DeviceArray(VOCAB)]))
    ctx.synchronize()
    syn.tmp.free()
    return stages


CHAIN_EPS = 1e-6


def build_chain8b(ctx, stages):
    """The same weights as one dependent decode step (build_block_decode,
    desktop/engine/src/forward.cpp:2663-2856, and the output head, :3411-3413):
    per layer
        A: x = h + down (the residual), xres = x, rms_norm * attn_norm, q/k/v
        B: o of the attention output (the attention core is outside this path;
           the q projection, of the same shape, stands in for its output)
        C: x = xres + o, h = x, rms_norm * ffn_norm, silu(gate) * up
        D: down
    then logits = out . (rms_norm(h + down) * out_norm). Every stage's input is
    what the stages before it wrote. Norm weights are seeded N(1, 0.2)."""
    bufs = []

    def buf(n, seed=None):
        a = DeviceArray(n, np.float32)
        if seed is None:
            a.fill_byte(0)
        else:
            ctx.synth_fill_dev(a.ptr, n, seed, spq4k.DIST_NORMAL, 0, 1.0, 0.2, 1.0, 0)
        bufs.append(a)
        return a.ptr

    x0a = DeviceArray(HID, np.float32)
    ctx.synth_fill_dev(x0a.ptr, HID, 7, spq4k.DIST_NORMAL, 0, 0.0, 1.0, 1.0, 0)
    bufs.append(x0a)
    x0 = x0a.ptr
    chain = []
    h = d = None
    for L in range(LAYERS):
        (_, (q, k, v), _, _), (_, (o,), _, _), (_, (g, u), _, _), (_, (dn,), _, _) = stages[4 * L:4 * L + 4]
        yq, yk, yv, yo = buf(HID), buf(KV), buf(KV), buf(HID)
        yg, yd, xres, hn = buf(FFN), buf(HID), buf(HID), buf(HID)
        an, fn = buf(HID, 50000 + 2 * L), buf(HID, 50001 + 2 * L)
        a = {"W": [q, k, v], "y": [yq, yk, yv], "in0": x0 if h is None else h, "x_out": xres, "norm_w": an}
        if d is not None:
            a["in1"] = d
        chain.append(a)
        chain.append({"W": [o], "y": [yo], "in0": yq})
        chain.append({"W": [g, u], "y": [yg], "glu": 1, "in0": xres, "in1": yo, "x_out": hn, "norm_w": fn})
        chain.append({"W": [dn], "y": [yd], "in0": yg})
        h, d = hn, yd
    _, (lm,), _, _ = stages[-1]
    logits = DeviceArray(VOCAB, np.float32)
    bufs.append(logits)
    chain.append({"W": [lm], "y": [logits.ptr], "in0": h, "in1": d, "x_out": buf(HID), "norm_w": buf(HID, 59999)})
    ctx.synchronize()
    return ctx.chain_create(chain, CHAIN_EPS), bufs, logits


def time_chain(ctx, ch, steps, warmup):
    """HIP events on the context stream around `steps` back-to-back launches"""
    for _ in range(warmup):
        ch.run()
    ch.status()
    e0, e1 = Event(), Event()
    e0.record(ctx.stream)
    for _ in range(steps):
        ch.run()
    e1.record(ctx.stream)
    e1.synchronize()
    ch.status()
    return e0.elapsed_ms(e1) / steps


def chain_breakdown(ctx, ch, kinds):
    """Stage timestamps of a form-2 chain (spq4k_chain_set_stamps,
    include/spq4k_diag.h): per stage kind, the medians over layers of
      exchange  the last workgroup's rows of the previous stage done -> the
                first exchange wave's inputs gathered (median over workgroups),
      staged    the same -> every exchange wave's inputs gathered and x formed,
      quant     x formed -> Q8_K activations ready (norm and quantisation),
      rows      activations ready -> the workgroup's rows done,
      spread    the last workgroup's rows done - the median workgroup's,
      stage     the last workgroup's rows done, from the previous stage's."""
    from spq4k.hip import DeviceArray
    v, grid, n = ch.info()
    if v != 2:
        return None
    buf = DeviceArray(grid * n * 4, np.uint64)
    buf.fill_byte(0)
    ch.set_stamps(buf.ptr)
    for _ in range(3):
        ch.run()
    ch.status()
    s = buf.to_host().reshape(grid, n, 4).astype(np.int64) * 10   # ns (100 MHz clock)
    ch.set_stamps(None)
    buf.free()
    last = s[:, :, 2].max(axis=0)
    rows = {}
    for t in range(1, n):
        k = kinds[t]
        d = rows.setdefault(k, {"exchange": [], "staged": [], "quant": [], "rows": [], "spread": [], "stage": []})
        d["exchange"].append(np.median(s[:, t, 0] - last[t - 1]))
        d["staged"].append(np.median(s[:, t, 3] - last[t - 1]))
        d["quant"].append(np.median(s[:, t, 1] - s[:, t, 3]))
        d["rows"].append(np.median(s[:, t, 2] - s[:, t, 1]))
        d["spread"].append(last[t] - np.median(s[:, t, 2]))
        d["stage"].append(last[t] - last[t - 1])
    out = {k: {m: round(float(np.median(v)) / 1e3, 3) for m, v in d.items()} for k, d in rows.items()}
    out["_step_us"] = round(float(last[-1] - s[:, 0, 0].min()) / 1e3, 1)
    return out


def stage_bytes(stage):
    _, ws, _, _ = stage
    # algorithmic: weights + one fp32 x and y per matvec (BASELINE accounting)
    return sum(q4k_bytes(w.M, w.K) + 4 * w.K + 4 * w.M for w in ws)


def enqueue_step(ctx, stages):
    for _, ws, x, ys in stages:
        if len(ws) == 1:
            ctx.gemv_dev(ws[0], x.ptr, ys[0].ptr, 1)
        else:
            ctx.gemv_multi_dev(ws, x.ptr, [y.ptr for y in ys], 1)


def capture_step(ctx, stages, with_events=False):
    with Graph.capture(ctx.stream) as g:
        enqueue_step(ctx, stages)
    return g, []


def time_stage_kinds(ctx, stages, reps=5):
    """Replay each stage kind (all 36 layers of it, or lm_head) on its own."""
    kinds = {}
    for st in stages:
        kind = st[0].split(".", 1)[-1] if "." in st[0] else st[0]
        kinds.setdefault(kind, []).append(st)
    out = {}
    for kind, sts in kinds.items():
        with Graph.capture(ctx.stream) as g:
            enqueue_step(ctx, sts)
        ms = time_graph(ctx, g, reps, 1)
        nb = sum(stage_bytes(x) for x in sts)
        out[kind] = {"us_per_launch": round(ms * 1e3 / len(sts), 3), "launches": len(sts),
                     "GBps": round(nb / (ms * 1e-3) / 1e9, 1)}
    return out


def time_graph(ctx, g, steps, warmup):
    for _ in range(warmup):
        g.launch()
    ctx.synchronize()
    e0, e1 = Event(), Event()
    e0.record(ctx.stream)
    for _ in range(steps):
        g.launch()
    e1.record(ctx.stream)
    e1.synchronize()
    ctx.synchronize()
    return e0.elapsed_ms(e1) / steps


# ---------------------------------------------------------------------------
def host_cpu():
    """CPU model, physical cores of the host and the CPUs this process may use"""
    model, cores = None, set()
    try:
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count()
    return {"cpu_model": model, "host_physical_cores": len(cores) or None, "cpus_allowed": allowed}


def cpu_baseline_decode(stages, budget_s=10.0):
    """Reference ggml CPU path (oracle/_ref) on layers 0-9 of the same step."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    try:
        from _oracle import Ref, ref_library_path, close_enough
    except Exception as e:  # pragma: no cover
        return None, f"oracle unavailable: {e}"
    path = ref_library_path()
    if path is None:
        return None, "oracle/_ref not built"
    import ctypes as C
    ref = Ref(path)
    sample_layers = tuple(f"L{i}." for i in range(10))
    sample = [s for s in stages if s[0].startswith(sample_layers)]
    Ws, Ms, Ks, Xs, Ys, keep = [], [], [], [], [], []
    gpu_y = []
    nbytes = 0
    for _, ws, x, ys in sample:
        xh = x.to_host()
        keep.append(xh)
        for w, y in zip(ws, ys):
            wh = np.empty(w.nbytes, np.uint8)
            from spq4k.hip import _lib, check
            check(_lib().hipMemcpy(wh.ctypes.data, w.data_ptr, w.nbytes, 2), "weights D2H")
            yh = np.empty(w.M, np.float32)
            keep += [wh, yh]
            Ws.append(wh.ctypes.data); Ms.append(w.M); Ks.append(w.K)
            Xs.append(xh.ctypes.data); Ys.append(yh.ctypes.data)
            gpu_y.append((y.to_host(), yh))
            nbytes += q4k_bytes(w.M, w.K) + 4 * w.K + 4 * w.M
    n = len(Ws)
    arr = lambda t, v: (t * n)(*v)

    def run(nthreads, budget):
        h = ref.L.ref_mm_create(n, arr(C.c_void_p, Ws), arr(C.c_int64, Ms), arr(C.c_int64, Ks),
                                arr(C.c_void_p, Xs), arr(C.c_void_p, Ys), 1, nthreads)
        if not h:
            return None, 0
        try:
            secs = (C.c_double * 1)()
            ref.L.ref_graph_run(h, 1, secs)          # warm-up
            first = secs[0]
            reps = max(5, min(20000, int(budget / max(first, 1e-4))))
            times = (C.c_double * reps)()
            ref.L.ref_graph_run(h, reps, times)
            return float(np.median(np.array(times[:reps]))), reps
        finally:
            ref.L.ref_graph_destroy(h)

    nthreads = min(16, os.cpu_count() or 1)
    med, reps = run(nthreads, budget_s)
    if med is None:
        return None, "ref graph creation failed"
    med4, reps4 = run(min(4, nthreads), budget_s / 2)
    # parity of the GPU step against the reference on the sampled stages
    worst_bad = 0
    for gy, cy in gpu_y:
        worst_bad += int((~close_enough(gy, cy)).sum())
    res = {
        "value": round(nbytes / med / 1e9, 2),
        "unit": "GB/s",
        "cores": nthreads,
        "kind": "reference",
        "sample": f"layers 0-9 of the step ({n} ggml mul_mat nodes, {nbytes/1e6:.1f} MB Q4_K+fp32), "
                  f"ggml_graph_compute with {nthreads} threads, median of {reps} runs "
                  f"({med*1e3:.2f} ms each); {os.path.basename(os.path.dirname(path))} build",
        "value_4_threads": round(nbytes / med4 / 1e9, 2) if med4 else None,
        "tok_s_equiv": round(1.0 / (med * 4268590592 / nbytes), 2),
        "parity_outside_tol": worst_bad,
    }
    res.update(host_cpu())
    return res, None


# ---------------------------------------------------------------------------
def load_traffic(name):
    p = os.path.join(REPO, "profiles", f"traffic_{name}.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f)
    return None


def run_decode8b(args):
    ctx = spq4k.Context(0)
    t0 = time.time()
    stages = build_decode8b(ctx)
    log(f"[bench] synthesised {sum(sum(w.nbytes for w in s[1]) for s in stages)/1e9:.3f} GB of Q4_K weights "
        f"on the GPU in {time.time()-t0:.1f}s")
    step_bytes = sum(stage_bytes(s) for s in stages)
    launches = len(stages)
    g, _ = capture_step(ctx, stages, with_events=False)
    ms = time_graph(ctx, g, args.steps, args.warmup)
    # Every launch in the step is the GEMV kernel; the events bracketing the
    # timed region on the context stream give its average duration per launch
    # (dispatch gaps between consecutive launches included).
    gemv_ms = ms
    value = step_bytes / (ms * 1e-3) / 1e9
    achieved = step_bytes / (gemv_ms * 1e-3) / 1e9
    log(f"[bench] step {ms*1e3:.1f} us ({launches} launches), {value:.1f} GB/s = {value*1e9/PEAK_HBM*100:.1f}% "
        f"of 8 TB/s, {1e3/ms:.0f} tok/s-equiv")
    stages_t = time_stage_kinds(ctx, stages)
    for k, v in stages_t.items():
        log(f"[bench]   {k:8s} {v['us_per_launch']:7.2f} us/launch  {v['GBps']:7.1f} GB/s")
    # The same weights as one dependent chain in one launch (chain_kernel):
    # each stage's input produced by the stages before it.
    chain = None
    if not args.no_chain:
        ch, chain_bufs, logits = build_chain8b(ctx, stages)
        form = ch.version
        ms_ch = time_chain(ctx, ch, args.steps, args.warmup)
        lg = logits.to_host()
        if not np.isfinite(lg).all() or not np.any(lg):
            raise RuntimeError("chain step produced non-finite or all-zero logits")
        ch.free()
        for b in chain_bufs:
            b.free()
        chain = {"kernel": "chain2_kernel" if form == 2 else "chain_kernel", "form": form,
                 "launches_per_step": 1, "ms_per_step": round(ms_ch, 5),
                 "GBps": round(step_bytes / (ms_ch * 1e-3) / 1e9, 2),
                 "what": "the step's 145 stages as one dependent chain (norm, q/k/v, o, residual, norm, "
                         "gate/up + SwiGLU, down, head; q stands in for the attention output)"}
        log(f"[bench] chain step {ms_ch*1e3:.1f} us (1 launch), {chain['GBps']:.1f} GB/s")
    traffic = load_traffic("decode8b")
    cpu, why = (None, "skipped")
    if not args.no_cpu:
        cpu, why = cpu_baseline_decode(stages)
        if cpu is None:
            log(f"[bench] cpu baseline unavailable: {why}")
        else:
            log(f"[bench] cpu baseline: {cpu['value']} GB/s, parity outside tolerance: {cpu['parity_outside_tol']}")
    out = {
        "metric": "Q4_K GEMV effective HBM GB/s (% of peak) + decode tok/s-equiv at 8B shapes",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: weights seeded N(0,0.02) quantised to Q4_K on the GPU by the bit-exact "
                "quantize_row_q4_K port; activations seeded N(0,1) fp32",
        "config": {
            "workload": "8B dense decode sweep, batch 1: 36 x (q 4096x4096, k/v 1024x4096, o 4096x4096, "
                        "gate/up 12288x4096, down 4096x12288) + lm_head 151936x4096, Q4_K (BASELINE configs[1])",
            "global_batch": 1,
            "seq_len": 1,
            "parallelism": "single GPU",
            "launches_per_step": launches,
            "algorithmic_bytes_per_step": step_bytes,
        },
        "pct_of_peak_hbm": round(value * 1e9 / PEAK_HBM * 100, 2),
        "tok_s_equiv": round(1e3 / ms, 1),
        "gflops": round(2 * 7568097280 / (ms * 1e-3) / 1e9, 1),
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_decode_kernel",
            "achieved": round(achieved, 2),
            "peak": 8000.0,
            "unit": "GB/s",
            "frac": round(achieved / 8000.0, 4),
            "traffic": round(traffic["step"]["bytes_per_launch"]) if traffic else None,
            "avg_launch_us": round(gemv_ms * 1e3 / launches, 3),
            "bytes_per_launch": step_bytes // launches,
        },
        "stages": stages_t,
        "chain": chain,
        "cpu_baseline": cpu,
    }
    if cpu is None:
        out["cpu_baseline_note"] = why
    print(json.dumps(out), flush=True)
    ctx.close()


def run_chain(args):
    """--config chain: the 8B decode step as one dependent chain launch, in
    each form (1: a grid barrier at every stage, k_chain.hip; 2: the one-hop
    exchange, k_chain2.hip), and form 2's per-stage breakdown from its
    timestamps (chain_breakdown)."""
    ctx = spq4k.Context(0)
    stages = build_decode8b(ctx)
    step_bytes = sum(stage_bytes(s) for s in stages)
    kinds = ["qkv", "o", "gate_up", "down"] * LAYERS + ["lm_head"]
    res = {}
    for form in (2, 1):
        os.environ["SPQ4K_CHAIN_V"] = str(form)
        ch, bufs, logits = build_chain8b(ctx, stages)
        os.environ.pop("SPQ4K_CHAIN_V", None)
        ms = time_chain(ctx, ch, args.steps, args.warmup)
        lg = logits.to_host()
        if not np.isfinite(lg).all() or not np.any(lg):
            raise RuntimeError(f"chain form {form}: non-finite or all-zero logits")
        r = {"form": ch.version, "ms_per_step": round(ms, 5), "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 2),
             "pct_of_peak_hbm": round(step_bytes / (ms * 1e-3) / PEAK_HBM * 100, 2)}
        log(f"[bench] chain form {ch.version}: {ms*1e3:.1f} us/step, {r['GBps']:.1f} GB/s")
        if ch.version == 2:
            r["breakdown_us"] = chain_breakdown(ctx, ch, kinds)
            for k, v in r["breakdown_us"].items():
                log(f"[bench]   {k:8s} {v}")
        res[f"form{ch.version}"] = r
        ch.free()
        for b in bufs:
            b.free()
    print(json.dumps({"config": "chain", "algorithmic_bytes_per_step": step_bytes, **res}), flush=True)
    ctx.close()


def run_single(args, M, K, T, dist, outlier, name, qtype=spq4k.TYPE_Q4_K):
    """A single matrix shape, timed cold (rotating >= 1 GiB of weight copies)."""
    ctx = spq4k.Context(0)
    syn = Synth(ctx, M * K)
    nb = M * (K // spq4k.BLOCK_VALUES[qtype]) * spq4k.BLOCK_BYTES[qtype]
    copies = max(2, min(128, (1 << 30) // nb + 1))
    ws = [syn.weights(M, K, 77 + i, dist, outlier, qtype) for i in range(copies)]
    x = syn.activations(T * K, 5)
    y = DeviceArray(T * M)
    ctx.synchronize()
    n = max(args.steps, copies)
    # spq4k_mul_mat (Q8_K activations, ggml's CPU arithmetic), or with
    # --op dequant_matvec spq4k_dequant_matvec (fp32 activations, beast_matvec's)
    call = ctx.dequant_matvec_dev if getattr(args, "op", "mul_mat") == "dequant_matvec" else ctx.mul_mat_dev
    with Graph.capture(ctx.stream) as g:
        for i in range(n):
            call(ws[i % copies], x.ptr, y.ptr, T)
    ms = time_graph(ctx, g, 1, max(1, args.warmup // 10)) / n
    alg = nb + 4 * K * T + 4 * M * T
    gbs = alg / (ms * 1e-3) / 1e9
    # reported beside it, never as the value: the same weights every call,
    # resident in the 256 MB Infinity Cache when they fit
    with Graph.capture(ctx.stream) as gh:
        for i in range(n):
            call(ws[0], x.ptr, y.ptr, T)
    ms_hot = time_graph(ctx, gh, 1, 1) / n
    print(json.dumps({"metric": f"{name} effective HBM GB/s", "value": round(gbs, 2), "unit": "GB/s",
                      "us_per_call": round(ms * 1e3, 3), "pct_of_peak_hbm": round(gbs * 1e9 / PEAK_HBM * 100, 2),
                      "TOPs_int8": round(2 * M * K * T / (ms * 1e-3) / 1e12, 1),
                      "hot_cache": {"us_per_call": round(ms_hot * 1e3, 3),
                                    "GBps": round(alg / (ms_hot * 1e-3) / 1e9, 1),
                                    "note": "same weights every call (Infinity Cache resident when under 256 MB)"},
                      "config": {"workload": name, "M": M, "K": K, "T": T, "weight_copies": copies,
                                 "op": getattr(args, "op", "mul_mat")}}), flush=True)
    for w in ws:
        w.free()
    syn.tmp.free()
    ctx.close()


def run_prefill(args):
    """the 8B layer shapes as a prefill matmul, T tokens.
    Weights are cold (8 distinct layers, 0.9 GB, replayed in one graph); the
    matrices that share an input run as one call, as in the decode step:
    [q,k,v] -> o -> [gate,up] -> down."""
    ctx = spq4k.Context(0)
    NL = 8
    syn = Synth(ctx, FFN * HID)
    shapes = [("q", HID, HID), ("k", KV, HID), ("v", KV, HID), ("o", HID, HID), ("gate", FFN, HID),
              ("up", FFN, HID), ("down", HID, FFN)]
    layers = [[syn.weights(M, K, 300 + 10 * L + i) for i, (_, M, K) in enumerate(shapes)] for L in range(NL)]
    ctx.synchronize()
    for T in (16, 128, 512):
        X = {K: syn.activations(T * K, 9 + K) for K in (HID, FFN)}
        Ys = [DeviceArray(T * M) for (_, M, _) in shapes]
        with Graph.capture(ctx.stream) as g:
            for ws in layers:
                ctx.gemm_multi_dev(ws[0:3], X[HID].ptr, [y.ptr for y in Ys[0:3]], T)
                ctx.gemm_dev(ws[3], X[HID].ptr, Ys[3].ptr, T)
                ctx.gemm_multi_dev(ws[4:6], X[HID].ptr, [y.ptr for y in Ys[4:6]], T)
                ctx.gemm_dev(ws[6], X[FFN].ptr, Ys[6].ptr, T)
        ms = time_graph(ctx, g, max(3, args.steps // 10), 1) / NL
        flops = 2 * T * sum(M * K for _, M, K in shapes)
        wbytes = sum(q4k_bytes(M, K) for _, M, K in shapes)
        abytes = wbytes + 4 * T * sum(M + K for _, M, K in shapes)
        tops = flops / (ms * 1e-3) / 1e12
        bound_us = max(abytes / PEAK_HBM, flops / 5.0e15) * 1e6
        print(json.dumps({"metric": f"Q4_K prefill matmul, one 8B layer, T={T}", "value": round(tops, 2),
                          "unit": "TOP/s (int8)", "us_per_layer": round(ms * 1e3, 2),
                          "pct_of_int8_mfma_peak": round(tops / 5000 * 100, 2),
                          "effective_GBps": round(abytes / (ms * 1e-3) / 1e9, 1),
                          "roofline_us": round(bound_us, 2), "frac_of_roofline": round(bound_us / (ms * 1e3), 4),
                          "tokens_per_s_36_layers": round(T / (ms * 1e-3 * LAYERS), 1),
                          "config": {"workload": f"8B layer (q,k,v,o,gate,up,down) x T={T} tokens, Q4_K, "
                                                 f"{NL} layers cold", "T": T}}), flush=True)
        for a in list(X.values()) + Ys:
            a.free()
    syn.tmp.free()
    ctx.close()


def run_beastwide(args):
    """The BurnHard MoE forward (spq4k_beast_moe_forward) at Mixtral-like
    widths: 8 experts of 4096 -> 14336 -> 4096, top-2 of seeded N(0,1)
    logits, one token; 4 layers of banks (3.2 GB, larger than the Infinity
    Cache) replayed as one graph, timed cold. The hidden rows here are longer
    than 16 blocks, so down runs the row-a-wave kernel."""
    ctx = spq4k.Context(0)
    E, k, NL, n_embd, n_ff = 8, 2, 4, 4096, 14336
    syn = Synth(ctx, E * n_ff * n_embd)
    layers = [[syn.weights(M, K, 700 + 10 * L + i, E=E) for i, (M, K) in
               enumerate(((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff)))] for L in range(NL)]
    ctx.synchronize()
    syn.tmp.free()
    xg = syn.activations(n_embd, 21)
    Yb = DeviceArray(n_embd)
    lg = [DeviceArray.from_host(np.random.default_rng(60 + L).standard_normal(E).astype(np.float32))
          for L in range(NL)]
    ctx.beast_moe_forward_dev(*layers[0], lg[0].ptr, k, xg.ptr, Yb.ptr)   # sizes the scratch
    ctx.synchronize()
    with Graph.capture(ctx.stream) as g:
        for L in range(NL):
            ctx.beast_moe_forward_dev(*layers[L], lg[L].ptr, k, xg.ptr, Yb.ptr)
    ms = time_graph(ctx, g, max(5, args.steps // 5), 2) / NL
    wbytes = k * 3 * q4k_bytes(n_ff, n_embd)
    gbs = wbytes / (ms * 1e-3) / 1e9
    print(json.dumps({"metric": "BurnHard MoE forward (routing, fp32 dequant-then-dot), T=1, wide rows",
                      "value": round(gbs, 1), "unit": "GB/s", "us_per_layer": round(ms * 1e3, 2),
                      "pct_of_peak_hbm": round(gbs * 1e9 / PEAK_HBM * 100, 2),
                      "config": {"workload": "8 experts of 4096 -> 14336 -> 4096, top-2, 4 layers of banks (cold)",
                                 "T": 1}}), flush=True)


def run_moe(args):
    """128 experts (gate/up 768x2048, down 2048x768), top-8,
    T = 1..32. Timed cold: 8 layers, each with its own three expert banks
    (2.7 GB in all, larger than the 256 MB Infinity Cache) and its own routing
    (top-8 of seeded N(0,1) logits per token), replayed as one graph; a layer
    is the gate, up and down GGML_OP_MUL_MAT_ID nodes: gate and up (same ids
    and input) as one spq4k_moe_multi call, then down."""
    ctx = spq4k.Context(0)
    E, k, NL = 128, 8, 8
    shapes = (("gate", 768, 2048), ("up", 768, 2048), ("down", 2048, 768))
    syn = Synth(ctx, E * 768 * 2048)
    layers = []
    for L in range(NL):
        banks = []
        for i, (name, M, K) in enumerate(shapes):
            w = ctx.alloc_weights(M, K, E)
            ctx.synth_fill_dev(syn.tmp.ptr, E * M * K, 500 + 10 * L + i, spq4k.DIST_NORMAL, K, 0.0, 0.02, 1.0, 0)
            ctx.quantize_q4K_dev(syn.tmp.ptr, w.data_ptr, E * M, K)
            banks.append((w, M, K))
        layers.append(banks)
    ctx.synchronize()
    syn.tmp.free()
    rng = np.random.default_rng(3)
    for T in (1, 4, 8, 32):
        ids_l = [np.argsort(-rng.standard_normal((T, E)).astype(np.float32), axis=1, kind="stable")[:, :k]
                 .astype(np.int32) for _ in range(NL)]
        idd = [DeviceArray.from_host(i) for i in ids_l]
        xg = syn.activations(T * 2048, 11)
        xd = syn.activations(T * k * 768, 12)
        Y = DeviceArray(T * k * 2048)
        Y2 = DeviceArray(T * k * 768)
        with Graph.capture(ctx.stream) as g:
            for L in range(NL):
                (wg, _, _), (wu, _, _), (wd, _, _) = layers[L]
                # gate and up share ids and input: one spq4k_moe_multi call
                ctx.moe_multi_dev([wg, wu], idd[L].ptr, k, 1, T, xg.ptr, [Y.ptr, Y2.ptr])
                ctx.moe_dev(wd, idd[L].ptr, k, k, T, xd.ptr, Y.ptr)
        ms = time_graph(ctx, g, max(5, args.steps // 5), 2) / NL
        # beside it, never as the value: layer 0's banks and routing every time
        with Graph.capture(ctx.stream) as gh:
            for L in range(NL):
                (wg, _, _), (wu, _, _), (wd, _, _) = layers[0]
                ctx.moe_multi_dev([wg, wu], idd[0].ptr, k, 1, T, xg.ptr, [Y.ptr, Y2.ptr])
                ctx.moe_dev(wd, idd[0].ptr, k, k, T, xd.ptr, Y.ptr)
        ms_hot = time_graph(ctx, gh, max(5, args.steps // 5), 2) / NL
        uniq = float(np.mean([len(np.unique(i)) for i in ids_l]))
        wbytes = uniq * sum(q4k_bytes(M, K) for (_, M, K) in shapes)
        abytes = wbytes + 4 * T * (2 * 2048 + 2 * k * 768) + 4 * T * k * (768 + 2048)
        gbs = abytes / (ms * 1e-3) / 1e9
        # the whole routed-expert FFN block per layer (spq4k_moe_ffn: gate/up,
        # SwiGLU, down on the pairs' own hidden rows, weighted sum), cold
        wts = [DeviceArray.from_host(np.full((T, k), 1.0 / k, np.float32)) for _ in range(NL)]
        Yb = DeviceArray(T * 2048)
        (wg, _, _), (wu, _, _), (wd, _, _) = layers[0]
        ctx.moe_ffn_dev(wg, wu, wd, idd[0].ptr, wts[0].ptr, k, T, xg.ptr, Yb.ptr)   # sizes the scratch
        ctx.synchronize()
        with Graph.capture(ctx.stream) as gb:
            for L in range(NL):
                (wg, _, _), (wu, _, _), (wd, _, _) = layers[L]
                ctx.moe_ffn_dev(wg, wu, wd, idd[L].ptr, wts[L].ptr, k, T, xg.ptr, Yb.ptr)
        ms_blk = time_graph(ctx, gb, max(5, args.steps // 5), 2) / NL
        # the adapter's path for one block node: host activations, ids and
        # weights copied in, the output copied out, synchronised (wall clock)
        xh = np.random.default_rng(T).standard_normal((T, 2048)).astype(np.float32)
        wh = np.full((T, k), 1.0 / k, np.float32)
        (wg, _, _), (wu, _, _), (wd, _, _) = layers[0]
        ctx.moe_ffn(wg, wu, wd, ids_l[0], wh, xh)
        host_t = []
        for _ in range(20):
            t0 = time.perf_counter()
            ctx.moe_ffn(wg, wu, wd, ids_l[0], wh, xh)
            host_t.append(time.perf_counter() - t0)
        blk_bytes = abytes + 4 * T * 2048
        beast = None
        if T == 1:
            # the reference's BurnHard MoE forward for one token (routing of
            # 128 logits to the top 8, gate / up / down in beast_matvec's fp32
            # arithmetic, score-weighted sum), per layer, cold
            lg = [DeviceArray.from_host(np.random.default_rng(50 + L).standard_normal(E).astype(np.float32))
                  for L in range(NL)]
            (wg, _, _), (wu, _, _), (wd, _, _) = layers[0]
            ctx.beast_moe_forward_dev(wg, wu, wd, lg[0].ptr, k, xg.ptr, Yb.ptr)   # sizes the scratch
            ctx.synchronize()
            with Graph.capture(ctx.stream) as gf:
                for L in range(NL):
                    (wg, _, _), (wu, _, _), (wd, _, _) = layers[L]
                    ctx.beast_moe_forward_dev(wg, wu, wd, lg[L].ptr, k, xg.ptr, Yb.ptr)
            ms_bf = time_graph(ctx, gf, max(5, args.steps // 5), 2) / NL
            bf_bytes = k * sum(q4k_bytes(M, K) for (_, M, K) in shapes) + 4 * (E + 2 * 2048)
            beast = {"us_per_layer": round(ms_bf * 1e3, 2), "GBps": round(bf_bytes / (ms_bf * 1e-3) / 1e9, 1),
                     "what": "spq4k_beast_moe_forward: routing (softmax, top-8 of 128) and the 8 experts' "
                             "gate / up / down in beast_matvec's fp32 dequant-then-dot, score-weighted sum (cold)"}
            for a in lg:
                a.free()
        print(json.dumps({"metric": f"Q4_K MoE expert matvec (gate+up+down), T={T}", "value": round(gbs, 1),
                          "unit": "GB/s", "us_per_layer": round(ms * 1e3, 2),
                          "pct_of_peak_hbm": round(gbs * 1e9 / PEAK_HBM * 100, 2), "unique_experts": uniq,
                          "hot_cache": {"us_per_layer": round(ms_hot * 1e3, 2),
                                        "note": "one layer's banks and routing every time (Infinity Cache resident)"},
                          "ffn_block": {"us_per_layer": round(ms_blk * 1e3, 2),
                                        "GBps": round(blk_bytes / (ms_blk * 1e-3) / 1e9, 1),
                                        "what": "spq4k_moe_ffn: gate/up, SwiGLU, down, router-weighted sum (cold)",
                                        "host_path_us": round(float(np.median(host_t)) * 1e6, 1),
                                        "host_path_what": "spq4k_moe_ffn_host, the ggml node's path: copies in, "
                                                          "block, copy out, synchronise (wall clock, median of 20, "
                                                          "layer 0 hot)"},
                          **({"beast_forward": beast} if beast else {}),
                          "config": {"workload": "30B-A3B-like MoE layer, 128 experts, top-8, 8 layers of banks (cold)",
                                     "T": T}}), flush=True)
        for a in idd + wts:
            a.free()
        xg.free(); xd.free(); Y.free(); Y2.free(); Yb.free()
    ctx.close()


def qtype_bytes(qtype, M, K):
    return M * (K // spq4k.BLOCK_VALUES[qtype]) * spq4k.BLOCK_BYTES[qtype]


def run_beastmix(args):
    """The fp32-activation dequant-then-dot (spq4k_dequant_matvec) and the
    BurnHard MoE forward (spq4k_beast_moe_forward) on the other weight types a
    Q4_K model file carries: the Q6_K down banks of Q4_K_M files beside Q4_K
    gate / up banks, and Q8_0 banks; configs[3] widths (128 experts of
    2048 -> 768 -> 2048, top-8 of seeded N(0,1) logits, one token), 8 layers
    of banks replayed as one graph (cold), all-Q4_K beside them. Then the
    dense matvec of Q6_K and Q8_0 rows at 8B decode shapes (4096 x 4096 and
    the down projection 4096 x 12288), 8 distinct matrices a shape (cold).
    Algorithmic bytes: the chosen experts' weights (or the matrix) + fp32 in
    and out."""
    ctx = spq4k.Context(0)
    Q4, Q6, Q8 = spq4k.TYPE_Q4_K, spq4k.TYPE_Q6_K, spq4k.TYPE_Q8_0
    E, k, NL, n_embd, n_ff = 128, 8, 8, 2048, 768
    syn = Synth(ctx, E * n_ff * n_embd)
    lg = [DeviceArray.from_host(np.random.default_rng(50 + L).standard_normal(E).astype(np.float32))
          for L in range(NL)]
    xg = syn.activations(n_embd, 11)
    Yb = DeviceArray(n_embd)
    names = {Q4: "Q4_K", Q6: "Q6_K", Q8: "Q8_0"}
    for types in ((Q4, Q4, Q6), (Q8, Q8, Q8), (Q4, Q4, Q4)):
        shapes = ((n_ff, n_embd), (n_ff, n_embd), (n_embd, n_ff))
        layers = [[syn.weights(M, K, 800 + 10 * L + i, qtype=t, E=E) for i, ((M, K), t) in
                   enumerate(zip(shapes, types))] for L in range(NL)]
        ctx.synchronize()
        ctx.beast_moe_forward_dev(*layers[0], lg[0].ptr, k, xg.ptr, Yb.ptr)   # sizes the scratch
        ctx.synchronize()
        with Graph.capture(ctx.stream) as g:
            for L in range(NL):
                ctx.beast_moe_forward_dev(*layers[L], lg[L].ptr, k, xg.ptr, Yb.ptr)
        ms = time_graph(ctx, g, max(5, args.steps // 5), 2) / NL
        nbytes = k * sum(qtype_bytes(t, M, K) for (M, K), t in zip(shapes, types)) + 4 * (E + 2 * n_embd)
        gbs = nbytes / (ms * 1e-3) / 1e9
        print(json.dumps({"metric": "BurnHard MoE forward (routing, fp32 dequant-then-dot), T=1, "
                                    f"gate/up/down {'/'.join(names[t] for t in types)}",
                          "value": round(gbs, 1), "unit": "GB/s", "us_per_layer": round(ms * 1e3, 2),
                          "pct_of_peak_hbm": round(gbs * 1e9 / PEAK_HBM * 100, 2),
                          "config": {"workload": "128 experts of 2048 -> 768 -> 2048, top-8, "
                                                 "8 layers of banks (cold)", "T": 1}}), flush=True)
        for lay in layers:
            for w in lay:
                w.free()
    for qtype in (Q6, Q8):
        for (M, K) in ((4096, 4096), (4096, 12288)):
            mats = [syn.weights(M, K, 900 + i, qtype=qtype) for i in range(8)]
            x = syn.activations(K, 13)
            y = DeviceArray(M)
            ctx.synchronize()
            with Graph.capture(ctx.stream) as g:
                for w in mats:
                    ctx.dequant_matvec_dev(w, x.ptr, y.ptr, 1)
            ms = time_graph(ctx, g, max(5, args.steps // 5), 2) / len(mats)
            nbytes = qtype_bytes(qtype, M, K) + 4 * (M + K)
            gbs = nbytes / (ms * 1e-3) / 1e9
            print(json.dumps({"metric": f"fp32-activation dequant-then-dot {names[qtype]}, T=1",
                              "value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(ms * 1e3, 2),
                              "pct_of_peak_hbm": round(gbs * 1e9 / PEAK_HBM * 100, 2),
                              "config": {"workload": f"{M} x {K}, 8 distinct matrices (cold)", "T": 1}}),
                  flush=True)
            for w in mats:
                w.free()
            x.free()
            y.free()
    for a in lg:
        a.free()
    xg.free()
    Yb.free()
    syn.tmp.free()
    ctx.close()


def run_kquant(args, qtype):
    """The other types a Q4_K model file stores some tensors in (Q6_K:
    attn_v, ffn_down, output; Q5_K in Q5_K_M files; Q8_0 for small or
    sensitive tensors). Dense decode shapes of the
    8B model at T = 1, a T = 8 batch and the down projection as a prefill
    matmul (T = 16, 128, 512; the same shape in Q4_K beside it), cold, then the
    MoE down-projection bank (128 experts of 2048x768) at T = 1..32, 8 layers
    of banks cold, as in run_moe."""
    tag = {spq4k.TYPE_Q6_K: "Q6_K", spq4k.TYPE_Q5_K: "Q5_K", spq4k.TYPE_Q8_0: "Q8_0"}[qtype]
    for name, M, K, T in ((f"{tag} attn_v 1024x4096", 1024, 4096, 1), (f"{tag} 4096x4096", 4096, 4096, 1),
                          (f"{tag} ffn_down 4096x12288", 4096, 12288, 1),
                          (f"{tag} output 151936x4096", 151936, 4096, 1), (f"{tag} 4096x4096 T=8", 4096, 4096, 8),
                          (f"{tag} ffn_down 4096x12288 T=16", 4096, 12288, 16),
                          (f"{tag} ffn_down 4096x12288 T=128", 4096, 12288, 128),
                          (f"{tag} ffn_down 4096x12288 T=512", 4096, 12288, 512),
                          ("Q4_K ffn_down 4096x12288 T=512 (same shape, Q4_K)", 4096, 12288, 512)):
        qt = spq4k.TYPE_Q4_K if name.startswith("Q4_K") else qtype
        run_single(args, M, K, T, spq4k.DIST_NORMAL, 1.0, name, qt)
    ctx = spq4k.Context(0)
    E, k, NL, M, K = 128, 8, 8, 2048, 768
    syn = Synth(ctx, E * M * K)
    banks = [syn.weights(M, K, 900 + L, qtype=qtype, E=E) for L in range(NL)]
    ctx.synchronize()
    syn.tmp.free()
    bb = spq4k.BLOCK_BYTES[qtype]
    qk = spq4k.BLOCK_VALUES[qtype]
    rng = np.random.default_rng(4)
    for T in (1, 4, 8, 32):
        ids_l = [np.argsort(-rng.standard_normal((T, E)).astype(np.float32), axis=1, kind="stable")[:, :k]
                 .astype(np.int32) for _ in range(NL)]
        idd = [DeviceArray.from_host(i) for i in ids_l]
        xd = syn.activations(T * k * K, 12)
        Y = DeviceArray(T * k * M)
        with Graph.capture(ctx.stream) as g:
            for L in range(NL):
                ctx.moe_dev(banks[L], idd[L].ptr, k, k, T, xd.ptr, Y.ptr)
        ms = time_graph(ctx, g, max(5, args.steps // 5), 2) / NL
        uniq = float(np.mean([len(np.unique(i)) for i in ids_l]))
        abytes = uniq * M * (K // qk) * bb + 4 * T * k * (K + M)
        gbs = abytes / (ms * 1e-3) / 1e9
        print(json.dumps({"metric": f"{tag} MoE down-projection matvec, T={T}", "value": round(gbs, 1),
                          "unit": "GB/s", "us_per_call": round(ms * 1e3, 2),
                          "pct_of_peak_hbm": round(gbs * 1e9 / PEAK_HBM * 100, 2), "unique_experts": uniq,
                          "config": {"workload": f"128 experts of 2048x768 {tag}, top-8, 8 banks (cold)", "T": T}}),
              flush=True)
        for a in idd:
            a.free()
        xd.free(); Y.free()
    ctx.close()


def _write_gguf(path, spec, rng):
    """A GGUF v3 file (default alignment 32) of tensors [(name, ggml type,
    ne)] with random bytes, written in chunks."""
    import struct
    bb = {spq4k.TYPE_Q4_K: (256, 144), spq4k.TYPE_Q6_K: (256, 210)}
    def gstr(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    head = bytearray(b"GGUF") + struct.pack("<Iqq", 3, len(spec), 1)
    head += gstr("general.architecture") + struct.pack("<i", 8) + gstr("llama")
    off, sizes = 0, []
    for name, t, ne in spec:
        n = int(np.prod(ne)) // bb[t][0] * bb[t][1]
        head += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<q", x) for x in ne)
        head += struct.pack("<iQ", t, off)
        sizes.append(n)
        off += (n + 31) // 32 * 32
    head += b"\0" * ((-len(head)) % 32)
    with open(path, "wb") as f:
        f.write(head)
        for n in sizes:
            left = n
            while left:
                c = min(left, 64 << 20)
                f.write(rng.bytes(c))
                left -= c
            f.write(b"\0" * ((-n) % 32))
    return sum(sizes)


def run_gguf(args):
    """GGUF residency: LlamaWeights::load_backend_offload_'s upload
    (desktop/engine/src/llama_weights.cpp:483-720) of 12 layers of the 8B
    shapes plus the output matrix, warm page cache (the file was just
    written). Roofline: the host link, PCIe 5.0 x16, 64 GB/s a direction."""
    import tempfile
    from spq4k.hip import _lib, check, H2D
    spec = []
    for L in range(12):
        spec += [(f"blk.{L}.attn_q.weight", spq4k.TYPE_Q4_K, (HID, HID)),
                 (f"blk.{L}.attn_k.weight", spq4k.TYPE_Q4_K, (HID, KV)),
                 (f"blk.{L}.attn_v.weight", spq4k.TYPE_Q6_K, (HID, KV)),
                 (f"blk.{L}.attn_output.weight", spq4k.TYPE_Q4_K, (HID, HID)),
                 (f"blk.{L}.ffn_gate.weight", spq4k.TYPE_Q4_K, (HID, FFN)),
                 (f"blk.{L}.ffn_up.weight", spq4k.TYPE_Q4_K, (HID, FFN)),
                 (f"blk.{L}.ffn_down.weight", spq4k.TYPE_Q6_K, (FFN, HID))]
    spec.append(("output.weight", spq4k.TYPE_Q6_K, (HID, VOCAB)))
    path = os.path.join(tempfile.gettempdir(), f"spq4k_bench_{os.getpid()}.gguf")
    rng = np.random.default_rng(5)
    try:
        t0 = time.perf_counter()
        total = _write_gguf(path, spec, rng)
        log(f"gguf: wrote {total / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
        ctx = spq4k.Context(0)
        g = spq4k.Gguf(path)
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            m = ctx.load_model(g)
            dt = time.perf_counter() - t0
            assert m.nbytes >= total
            m.free()
            best = dt if best is None else min(best, dt)
        # per-tensor copies from the mapping (pageable host memory)
        tens = g.tensors()
        dev = DeviceArray(sum((t[5] + 255) // 256 * 256 for t in tens), np.uint8)
        base = None
        for _ in range(2):
            ctx.synchronize()
            t0 = time.perf_counter()
            off = 0
            for i, t in enumerate(tens):
                src = g.lib.spq4k_gguf_tensor_data(g.handle, i)
                check(_lib().hipMemcpy(dev.ptr + off, src, t[5], H2D), "hipMemcpy H2D")
                off += (t[5] + 255) // 256 * 256
            dt = time.perf_counter() - t0
            base = dt if base is None else min(base, dt)
        dev.free()
        g.close()
        ctx.close()
        gbs = total / best / 1e9
        print(json.dumps({"metric": "GGUF weight residency (spq4k_model_load), host to HBM", "value": round(gbs, 2),
                          "unit": "GB/s", "seconds": round(best, 3), "bytes": total, "tensors": len(spec),
                          "roofline": {"bound": "pcie", "achieved": round(gbs, 2), "peak": 64.0, "unit": "GB/s",
                                       "frac": round(gbs / 64.0, 3)},
                          "per_tensor_hipMemcpy_GBps": round(total / base / 1e9, 2),
                          "config": {"workload": "12 layers of 8B shapes + output, Q4_K / Q6_K, warm page cache"}}),
              flush=True)
    finally:
        if os.path.exists(path):
            os.remove(path)


def run_fusion(args):
    """Decode-step neighbours of the matvec, 8B shapes, Q4_K, cold weights:
    the attention pre-norm + q/k/v (spq4k_mul_mat_rms_norm) and the FFN
    pre-norm + gate/up + SiLU * up (spq4k_mul_mat_swiglu), each fused into
    one launch and unfused (spq4k_rms_norm, the grouped matvec, spq4k_swiglu),
    captured in a graph. Algorithmic bytes: weights + x + norm weights + y."""
    ctx = spq4k.Context(0)
    K = HID
    syn = Synth(ctx, FFN * K)
    x = syn.activations(K, 3)
    nw = syn.activations(K, 4)
    xn = DeviceArray(K)
    eps = 1e-6
    cases = {
        "qkv": [(HID, K), (KV, K), (KV, K)],
        "gate_up": [(FFN, K), (FFN, K)],
    }
    for name, shapes in cases.items():
        wb = sum(q4k_bytes(M, K) for M, _ in shapes)
        copies = max(2, min(64, (1 << 30) // wb + 1))
        sets = [[syn.weights(M, K, 300 + 10 * i + j) for j, (M, _) in enumerate(shapes)] for i in range(copies)]
        ys = [DeviceArray(M) for M, _ in shapes]
        y = DeviceArray(shapes[0][0])
        ctx.synchronize()
        n = max(args.steps, copies)
        out_bytes = 4 * (shapes[0][0] if name == "gate_up" else sum(M for M, _ in shapes))
        alg = wb + 8 * K + out_bytes
        res = {}
        for fused in (True, False):
            with Graph.capture(ctx.stream) as g:
                for i in range(n):
                    W = sets[i % copies]
                    if name == "qkv":
                        if fused:
                            ctx.mul_mat_rms_norm_dev(W, x.ptr, nw.ptr, eps, [a.ptr for a in ys], 1)
                        else:
                            ctx.rms_norm_dev(x.ptr, nw.ptr, eps, xn.ptr, K, 1)
                            ctx.gemv_multi_dev(W, xn.ptr, [a.ptr for a in ys], 1)
                    else:
                        if fused:
                            ctx.mul_mat_swiglu_dev(W[0], W[1], x.ptr, nw.ptr, eps, y.ptr, 1)
                        else:
                            ctx.rms_norm_dev(x.ptr, nw.ptr, eps, xn.ptr, K, 1)
                            ctx.gemv_multi_dev(W, xn.ptr, [ys[0].ptr, ys[1].ptr], 1)
                            ctx.swiglu_dev(ys[0].ptr, ys[1].ptr, y.ptr, FFN)
            ms = time_graph(ctx, g, 1, max(1, args.warmup // 10)) / n
            res[fused] = ms
        print(json.dumps({"metric": f"decode {name} with its pre-norm" + (" and SwiGLU" if name == "gate_up" else ""),
                          "fused_us": round(res[True] * 1e3, 2), "unfused_us": round(res[False] * 1e3, 2),
                          "fused_GBps": round(alg / (res[True] * 1e-3) / 1e9, 1),
                          "unfused_GBps": round(alg / (res[False] * 1e-3) / 1e9, 1),
                          "speedup": round(res[False] / res[True], 3),
                          "config": {"workload": f"8B {name}, Q4_K, T=1, {copies} weight copies (cold)",
                                     "algorithmic_bytes": alg}}), flush=True)
        for ws in sets:
            for w in ws:
                w.free()
    ctx.close()


def run_decode_stamps(args):
    """Wave timestamps of the decode kernel inside the 8B step
    (spq4k_set_decode_stamps, include/spq4k_diag.h). The whole step is
    captured as in decode8b, with the stamps switched on for every stage of
    layers 9, 18 and 27 and for lm_head (a buffer per launch), and replayed;
    per stage kind, the medians over those layers of, in us from the launch's
    first wave start (the device's 100 MHz clock):
      start     the last wave's start,
      barrier   the median / last wave past the quantisation barrier,
      first     the median wave's first row done (its store issued, in
                the forms that store each row at once),
      end       the median / last wave's last row store issued,
      gap       from the previous stage's last store issued to this launch's
                first wave start (store completion, kernel end and dispatch)."""
    ctx = spq4k.Context(0)
    stages = build_decode8b(ctx)
    layers = (9, 18, 27)
    picked = ({f"L{L}.{k}" for L in layers for k in ("qkv", "o", "gate_up", "down")} |
              {f"L{L - 1}.down" for L in layers} | {"lm_head", f"L{LAYERS - 1}.down"})
    n = 256 * 16 * 4
    bufs = {}
    with Graph.capture(ctx.stream) as g:
        for st in stages:
            if st[0] in picked:
                bufs[st[0]] = DeviceArray(n, np.uint64)
                ctx.set_decode_stamps(bufs[st[0]].ptr, n)
            enqueue_step(ctx, [st])
            ctx.set_decode_stamps(None)
    for b in bufs.values():
        b.fill_byte(0)
    ctx.synchronize()
    # the step with and without the timestamped launches (their instances
    # carry four clock reads and one store a wave more)
    g_plain, _ = capture_step(ctx, stages)
    ms_plain = time_graph(ctx, g_plain, 20, max(args.warmup, 1))
    ms_stamped = time_graph(ctx, g, 20, max(args.warmup, 1))
    log(f"[bench] step {ms_plain * 1e3:.1f} us; with {len(bufs)} launches timestamped {ms_stamped * 1e3:.1f} us")
    stamp = {}
    for name, b in bufs.items():
        s = b.to_host().reshape(-1, 4).astype(np.int64)
        stamp[name] = s[s[:, 0] != 0]
    us = lambda v: round(float(v) / 100.0, 2)   # 100 MHz ticks -> us
    def previous(kind, L):
        if kind == "lm_head":
            return f"L{LAYERS - 1}.down"
        return {"qkv": f"L{L - 1}.down", "o": f"L{L}.qkv", "gate_up": f"L{L}.o", "down": f"L{L}.gate_up"}[kind]
    out = {}
    for kind in ("qkv", "o", "gate_up", "down", "lm_head"):
        names = [("lm_head", None)] if kind == "lm_head" else [(f"L{L}.{kind}", L) for L in layers]
        rec = {"start": [], "barrier_med": [], "barrier_last": [], "first_med": [], "end_med": [], "end_last": [],
               "gap": []}
        for nm, L in names:
            s = stamp[nm]
            t0 = s[:, 0].min()
            rec["start"].append(s[:, 0].max() - t0)
            rec["barrier_med"].append(np.median(s[:, 1]) - t0)
            rec["barrier_last"].append(s[:, 1].max() - t0)
            rows = s[s[:, 2] != 0]
            rec["first_med"].append(np.median(rows[:, 2]) - t0)
            rec["end_med"].append(np.median(rows[:, 3]) - t0)
            rec["end_last"].append(rows[:, 3].max() - t0)
            rec["gap"].append(t0 - stamp[previous(kind, L)][:, 3].max())
        out[kind] = {k: us(np.median(v)) for k, v in rec.items()}
        out[kind]["waves"] = int(len(stamp[names[0][0]]))
        log(f"[bench] {kind:8s} " + "  ".join(f"{k} {v}" for k, v in out[kind].items()))
    print(json.dumps({"metric": "decode kernel wave timestamps in the 8B step (us from the launch's first wave)",
                      "stages": out, "step_us": round(ms_plain * 1e3, 1),
                      "step_us_timestamped": round(ms_stamped * 1e3, 1),
                      "config": {"workload": "decode8b step replayed as one graph; stamps on layers 9, 18, 27 "
                                             "and lm_head"}}), flush=True)
    for b in bufs.values():
        b.free()
    ctx.close()


def run_floor(args):
    """The streaming floor of the 8B decode sweep: the same 145 dependent
    launches as decode8b, each a kernel that only reads its stage's bytes
    (spq4k_stream_read: 16-byte loads, four in flight a lane, no compute, no
    activations), over distinct buffers of the stage sizes (4.257 GB in all),
    replayed as one HIP graph; and 145 launches that read nothing (the launch
    floor). A per-op drop-in of the sweep cannot run faster than this."""
    ctx = spq4k.Context(0)
    sizes = {"qkv": q4k_bytes(HID, HID) + 2 * q4k_bytes(KV, HID), "o": q4k_bytes(HID, HID),
             "gate_up": 2 * q4k_bytes(FFN, HID), "down": q4k_bytes(HID, FFN), "lm_head": q4k_bytes(VOCAB, HID)}
    order = [k for _ in range(LAYERS) for k in ("qkv", "o", "gate_up", "down")] + ["lm_head"]
    bufs = [(k, DeviceArray(sizes[k], np.uint8)) for k in order]
    total = sum(sizes[k] for k in order)
    with Graph.capture(ctx.stream) as g:
        for _, b in bufs:
            ctx.stream_read_dev(b.ptr, sizes_of(b))
    ms = time_graph(ctx, g, args.steps, args.warmup)
    with Graph.capture(ctx.stream) as ge:
        for _, b in bufs:
            ctx.stream_read_dev(b.ptr, 0)
    ms_empty = time_graph(ctx, ge, args.steps, args.warmup)
    per = {}
    for kind in ("o", "qkv", "down", "gate_up", "lm_head"):
        sel = [b for k, b in bufs if k == kind]
        with Graph.capture(ctx.stream) as gk:
            for b in sel:
                ctx.stream_read_dev(b.ptr, sizes_of(b))
        mk = time_graph(ctx, gk, max(5, args.steps // 5), 2) / len(sel)
        per[kind] = {"MB": round(sizes[kind] / 1e6, 2), "us_per_launch": round(mk * 1e3, 3),
                     "GBps": round(sizes[kind] / (mk * 1e-3) / 1e9, 1)}
    out = {"metric": "streaming floor of the 8B decode sweep (145 dependent read-only launches)",
           "value": round(total / (ms * 1e-3) / 1e9, 1), "unit": "GB/s", "us_per_step": round(ms * 1e3, 1),
           "pct_of_peak_hbm": round(total / (ms * 1e-3) / PEAK_HBM * 100, 2),
           "empty_launch_us": round(ms_empty * 1e3 / len(bufs), 3), "per_launch": per,
           "config": {"workload": "stream reads of the decode8b stage sizes, distinct buffers", "bytes": total,
                      "launches": len(bufs)}}
    print(json.dumps(out), flush=True)
    for _, b in bufs:
        b.free()
    ctx.close()


def sizes_of(b):
    return b.nbytes


def run_copy(args):
    """A plain device-to-device copy of 1 GiB (the runtime's blit kernel): the
    known-size reference that scales rocprofv3's FETCH_SIZE / WRITE_SIZE."""
    from spq4k.hip import _lib, check, D2D
    ctx = spq4k.Context(0)
    n = 1 << 30
    a, b = DeviceArray(n // 4), DeviceArray(n // 4)
    ctx.synth_fill_dev(a.ptr, n // 4, 1, spq4k.DIST_NORMAL, 0, 0.0, 1.0, 1.0, 0)
    ctx.synchronize()
    reps = 3
    e0, e1 = Event(), Event()
    e0.record(ctx.stream)
    for _ in range(reps):
        check(_lib().hipMemcpyAsync(b.ptr, a.ptr, n, D2D, ctx.stream), "hipMemcpyAsync D2D")
    e1.record(ctx.stream)
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / reps
    print(json.dumps({"metric": "device-to-device copy", "bytes_per_copy": n, "copies": reps,
                      "us_per_copy": round(ms * 1e3, 2), "GBps_read_plus_write": round(2 * n / (ms * 1e-3) / 1e9, 1)}),
          flush=True)
    ctx.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="decode8b", choices=["decode8b", "gemv4096", "largek", "prefill", "moe", "q6k", "q5k", "q8_0",
                                                          "single", "gguf", "fusion", "copy", "floor", "beastwide", "beastmix", "chain",
                                                          "decode_stamps"])
    ap.add_argument("--M", type=int, default=4096, help="rows (--config single)")
    ap.add_argument("--K", type=int, default=4096, help="inputs (--config single)")
    ap.add_argument("--T", type=int, default=1, help="tokens (--config single)")
    ap.add_argument("--qtype", type=int, default=spq4k.TYPE_Q4_K, help="ggml weight type (--config single)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-chain", action="store_true", help="decode8b: skip the one-launch chain leg")
    ap.add_argument("--op", default="mul_mat", choices=["mul_mat", "dequant_matvec"],
                    help="--config single: the entry point timed (dequant_matvec: fp32 activations, any --qtype)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested). The Q4_K path "
              "shards by output rows / experts; see DESIGN.md. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.config == "decode8b":
        run_decode8b(args)
    elif args.config == "gemv4096":
        run_single(args, 4096, 4096, 1, spq4k.DIST_NORMAL, 1.0, "Q4_K GEMV 4096x4096 T=1")
    elif args.config == "prefill":
        run_prefill(args)
    elif args.config == "moe":
        run_moe(args)
    elif args.config == "beastwide":
        run_beastwide(args)
    elif args.config == "beastmix":
        run_beastmix(args)
    elif args.config == "q6k":
        run_kquant(args, spq4k.TYPE_Q6_K)
    elif args.config == "q5k":
        run_kquant(args, spq4k.TYPE_Q5_K)
    elif args.config == "q8_0":
        run_kquant(args, spq4k.TYPE_Q8_0)
    elif args.config == "gguf":
        run_gguf(args)
    elif args.config == "fusion":
        run_fusion(args)
    elif args.config == "single":
        tag = {spq4k.TYPE_Q4_K: "Q4_K", spq4k.TYPE_Q5_K: "Q5_K", spq4k.TYPE_Q6_K: "Q6_K", spq4k.TYPE_Q8_0: "Q8_0"}
        run_single(args, args.M, args.K, args.T, spq4k.DIST_NORMAL, 1.0,
                   f"{tag[args.qtype]} {args.M}x{args.K} T={args.T}", args.qtype)
    elif args.config == "floor":
        run_floor(args)
    elif args.config == "decode_stamps":
        run_decode_stamps(args)
    elif args.config == "chain":
        run_chain(args)
    elif args.config == "copy":
        run_copy(args)
    elif args.config == "largek":
        for (M, K) in ((5120, 27648), (27648, 5120)):
            for T in (1, 4, 8):
                run_single(args, M, K, T, spq4k.DIST_STUDENT_T4, 8.0, f"Q4_K GEMV {M}x{K} T={T} t4+outliers")


if __name__ == "__main__":
    main()
