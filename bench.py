"""Benchmark of the quantized-matmul hot path on one MI355X.

Default workload: the Q4_K decode GEMV set at
Llama-3-8B layer shapes, batch M = 1 -- q_proj 4096x4096, k_proj / v_proj
1024x4096, gate / up 14336x4096, down 4096x14336. One step is one pass over
the set as a decoder layer runs it: quantize the 4096-wide activation to Q8_K
on the device, q/k/v/gate/up GEMVs, quantize the 14336-wide activation, down
GEMV. Weights are N(0, 0.02^2) seed 2, activations N(0, 1) seed 3
(SplitMix64 + Box-Muller), quantized on the GPU (bit-identical to the CPU
quantizer). Several weight copies (> 2x the 256 MB Infinity Cache) are
rotated so every step streams its weights from HBM.

Steps are captured into HIP graphs (torch.cuda.graph) and replayed; the timed
region is bracketed by torch.cuda.synchronize(). `value` is algorithmic bytes
(weights + f32 activations + f32 outputs) per second over the timed steps.
The roofline object times the dominant kernel (the gate/up GEMV) alone with
HIP events on the stream it runs on; its `traffic` (HBM bytes per launch) comes
from the committed rocprofv3 counter summary profiles/gemv_q4k_gate_pmc.json
(FETCH_SIZE / WRITE_SIZE of that kernel, each scaled by the counter's reading
for a copy of known size), measured with `--kernel-only gate|copy`. Every
timing reports mean / median / p10 / p90 over 120 HIP-event samples. The CPU
baseline is the oracle's C restatement of Candle's CPU quantized matmul
(k_quants::matmul), with candle's generic vec_dot bodies (the reference's
default build) and with its AVX2 + FMA bodies, on the host's CPU share for
one GPU (16 threads) over bounded samples of configs 1, 2, 4 and one config-3
token; `value` is config 2 with the faster build.

Further legs: config 1 (the Q8_0 4096x4096 matvec, GB/s, checked against
the oracle), config 3 (greedy decode tok/s of the Llama-3-8B-shape Q4_K_M
model), config 4 (prefill GEMM, MFMA utilisation against the dense int8
peak) and config 5 (MoE expert FFN, weight GB/s of the active experts).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K GEMV GB/s (% of HBM peak) + decode tok/s, Llama-3-8B-shape Q4_K_M"

# (name, out, in) of the config-2 set
GEMV_SET = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096),
            ("gate_proj", 14336, 4096), ("up_proj", 14336, 4096), ("down_proj", 4096, 14336)]


def gemv_bytes(dt, n, k):
    from inference_amd import GgmlDType
    dt = GgmlDType(dt)
    w = n * (k // dt.block_size()) * dt.type_size()
    return w + 4 * k + 4 * n  # weights + f32 activation + f32 output


def log(msg):
    print(msg, file=sys.stderr, flush=True)


SPREAD_SAMPLES = 120  # HIP-event samples behind every median / p10 / p90
LAUNCH_GRAPH_MIN = 48  # launches per graph when one launch kind is timed alone


def replay_samples(torch, g, n, stream):
    """Replay graph g n times with a HIP event between consecutive replays on `stream` (where the graph
    runs); returns the milliseconds of each replay."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    evs[0].record(stream)
    for i in range(n):
        g.replay()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    return np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(n)])


def spread(us):
    """mean / median / p10 / p90 of per-unit microseconds."""
    us = np.asarray(us, dtype=np.float64)
    return {"mean": round(float(us.mean()), 3), "median": round(float(np.median(us)), 3),
            "p10": round(float(np.percentile(us, 10)), 3), "p90": round(float(np.percentile(us, 90)), 3),
            "samples": int(us.size)}


def build_set(torch, dev, dt, copies):
    """`copies` independent weight sets of GEMV_SET, quantized on the GPU: weight i of copy c is
    N(0, 0.02^2) from SplitMix64 seed 2 + 1000 c + 17 i (synth.normal_torch, on the device)."""
    from inference_amd import QTensor
    from inference_amd.synth import normal_torch
    sets = []
    for c in range(copies):
        layer = {}
        for i, (name, n, k) in enumerate(GEMV_SET):
            wt = normal_torch(2 + 1000 * c + 17 * i, (n, k), 0.02, dev)
            layer[name] = QTensor.quantize(wt, dt)
            del wt
        sets.append(layer)
    return sets


QKVGU = ("q_proj", "k_proj", "v_proj", "gate_proj", "up_proj")  # the K = 4096 projections


def run_gemv_set(torch, dev, args):
    from inference_amd import GgmlDType, QTensor, qmm
    from inference_amd.synth import normal, normal_torch

    dt = GgmlDType.Q4K
    vt = dt.vec_dot_type()
    set_weight_bytes = sum(n * (k // 256) * 144 for _, n, k in GEMV_SET)
    copies = max(2, -(-args.rotate_mb * 2 ** 20 // set_weight_bytes))
    log(f"[bench] building {copies} weight copies of the Q4_K GEMV set ({copies * set_weight_bytes / 2**20:.0f} MiB)")
    sets = build_set(torch, dev, dt, copies)

    shapes = {name: (n, k) for name, n, k in GEMV_SET}
    x4096 = torch.from_numpy(normal(3, (1, 4096))).to(dev)
    x14336 = torch.from_numpy(normal(3, (1, 14336))).to(dev)
    xq4096 = torch.empty((1, 16 * 292), dtype=torch.uint8, device=dev)
    xq14336 = torch.empty((1, 56 * 292), dtype=torch.uint8, device=dev)
    outs = {name: torch.empty((1, n), dtype=torch.float32, device=dev) for name, n, _ in GEMV_SET}
    L = qmm.lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64

    def q8k(x, xq, k):
        qmm._check(L.qmm_quantize_rows(int(vt), x.data_ptr(), 1, k, k, xq.data_ptr(), qmm._stream(dev)))

    def gemv(layer, name):
        n, k = shapes[name]
        xq = xq4096 if k == 4096 else xq14336
        qmm._check(L.qmm_matmul_q(layer[name].handle, xq.data_ptr(), 1, outs[name].data_ptr(), n, None, 0,
                                  qmm._stream(dev)))

    # job tables of the one-launch schedules (handles per weight copy)
    hs5 = [(vp * 5)(*[layer[nm].handle.value for nm in QKVGU]) for layer in sets]
    y5 = (vp * 5)(*[outs[nm].data_ptr() for nm in QKVGU])
    ld5 = (i64 * 5)(*[shapes[nm][0] for nm in QKVGU])
    hsd = [(vp * 1)(layer["down_proj"].handle.value) for layer in sets]
    yd = (vp * 1)(outs["down_proj"].data_ptr())
    ldd = (i64 * 1)(4096)
    cidx = {id(layer): c for c, layer in enumerate(sets)}

    def qkvgu(layer, fused):
        c = cidx[id(layer)]
        if fused:
            qmm._check(L.qmm_matmul_ex(hs5[c], 5, x4096.data_ptr(), 1, 4096, None, ctypes.c_float(0), 0, y5, ld5,
                                       None, 0, qmm._stream(dev)))
        else:
            qmm._check(L.qmm_matmul_multi_q(hs5[c], 5, xq4096.data_ptr(), 1, y5, ld5, None, 0, qmm._stream(dev)))

    def down_fused(layer):
        c = cidx[id(layer)]
        qmm._check(L.qmm_matmul_ex(hsd[c], 1, x14336.data_ptr(), 1, 14336, None, ctypes.c_float(0), 0, yd, ldd,
                                   None, 0, qmm._stream(dev)))

    def step_serial(layer):
        q8k(x4096, xq4096, 4096)
        for name in QKVGU:
            gemv(layer, name)
        q8k(x14336, xq14336, 14336)
        gemv(layer, "down_proj")

    def step_staged(layer):
        q8k(x4096, xq4096, 4096)
        qkvgu(layer, False)
        q8k(x14336, xq14336, 14336)
        gemv(layer, "down_proj")

    def step_fused(layer):
        qkvgu(layer, True)
        down_fused(layer)

    # grouped: the six GEMVs as one launch (qmm_matmul_grouped): q/k/v/gate/up on the 4096-wide row,
    # down on the 14336-wide row, each row quantized to Q8_K in the prologue of its workgroups
    grp_w = [(vp * 6)(*([layer[nm].handle.value for nm in QKVGU] + [layer["down_proj"].handle.value]))
             for layer in sets]
    grp_g = (ctypes.c_int * 6)(0, 0, 0, 0, 0, 1)
    grp_x = (vp * 2)(x4096.data_ptr(), x14336.data_ptr())
    grp_y = (vp * 6)(*([outs[nm].data_ptr() for nm in QKVGU] + [outs["down_proj"].data_ptr()]))

    def step_grouped(layer):
        qmm._check(L.qmm_matmul_grouped(grp_w[cidx[id(layer)]], grp_g, 6, grp_x, grp_y, qmm._stream(dev)))

    step = {"serial": step_serial, "staged": step_staged, "fused": step_fused,
            "grouped": step_grouped}[args.schedule]

    # warm up eagerly (module load, kernel lookup), then capture graphs
    for c in range(copies):
        step_serial(sets[c])
        step(sets[c])
    torch.cuda.synchronize()

    def capture(fn, reps):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for r in range(reps):
                fn(sets[r % copies])
        return g

    # the timed region runs exactly args.steps steps: whole graphs of per_graph steps, then a graph of
    # the remaining steps (each graph walks the copies from the first, so a copy's weights are never
    # re-read from the MALL by the step after it). A graph holds all the steps (up to 1200): each
    # replay's start-up then falls once into the timed region, not once per few steps
    per_graph = min(max(1, args.steps), 1200)
    g_step = capture(step, per_graph)
    reps, rem = divmod(args.steps, per_graph)
    g_rem = capture(step, rem) if rem else None
    g_spread = capture(step, copies * max(1, 24 // copies))  # the spread's samples: 24-step replays
    for _ in range(max(1, -(-args.warmup // per_graph))):
        g_step.replay()
    if g_rem is not None:
        g_rem.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g_step.replay()
    if g_rem is not None:
        g_rem.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    steps = args.steps

    step_bytes = sum(gemv_bytes(dt, n, k) for _, n, k in GEMV_SET)
    value = step_bytes * steps / elapsed / 1e9

    stream = torch.cuda.current_stream(dev)

    # spread of the step time: SPREAD_SAMPLES replays of the step graph, a HIP event between consecutive
    # replays
    replay_samples(torch, g_spread, 4, stream)
    step_spread = spread(replay_samples(torch, g_spread, SPREAD_SAMPLES, stream) * 1e3 / (copies * max(1, 24 // copies)))

    # single-launch graphs hold at least LAUNCH_GRAPH_MIN launches, so a replay's own start-up is a small
    # share of the per-launch figure
    per_launch_graph = copies * max(1, -(-LAUNCH_GRAPH_MIN // copies))

    def time_launch(fn):
        """us per launch of fn(layer) alone: SPREAD_SAMPLES replays of a graph of per_launch_graph launches over
        the rotated copies, HIP events between replays on the stream the graph runs on, after untimed replays
        (the first pass over the copies runs a few % slower). Returns the spread of the per-launch time;
        its mean is the average launch."""
        g = capture(fn, per_launch_graph)
        replay_samples(torch, g, 4, stream)
        return spread(replay_samples(torch, g, SPREAD_SAMPLES, stream) * 1e3 / per_launch_graph)

    # per-shape single launches (pre-quantized activation); each shape rotates
    # its own copies over >= rotate_mb MiB, so no launch reads from the MALL
    per_shape = {}
    for name, n, k in GEMV_SET:
        wb = n * (k // 256) * 144
        nc = max(2, -(-args.rotate_mb * 2 ** 20 // wb))
        own = [{name: QTensor.quantize(normal_torch(7000 + n + k + 101 * c, (n, k), 0.02, dev), dt)}
               for c in range(nc)]
        gph = torch.cuda.CUDAGraph()
        gemv(own[0], name)
        torch.cuda.synchronize()
        passes = max(1, -(-LAUNCH_GRAPH_MIN // nc))
        with torch.cuda.graph(gph):
            for r in range(nc * passes):
                gemv(own[r % nc], name)
        replay_samples(torch, gph, 4, stream)  # untimed passes over the copies
        sp = spread(replay_samples(torch, gph, SPREAD_SAMPLES, stream) * 1e3 / (nc * passes))
        us = sp["mean"]
        b = gemv_bytes(dt, n, k)
        per_shape[name] = {"shape": [n, k], "us": round(us, 3), "GB/s": round(b / us / 1e3, 1),
                           "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "copies": nc, "us_spread": sp}
        del own, gph
        torch.cuda.empty_cache()

    # the FFN pair as the decoder runs it (LlamaMlp's gate and up on one row): one launch over both
    # weights with the RMSNorm + Q8_K of the f32 row in the prologue, rotated over the set copies
    ffn_norm = torch.from_numpy(normal(4, (4096,))).to(dev)
    hs_gu = [(vp * 2)(layer["gate_proj"].handle.value, layer["up_proj"].handle.value) for layer in sets]
    y_gu = (vp * 2)(outs["gate_proj"].data_ptr(), outs["up_proj"].data_ptr())
    ld_gu = (i64 * 2)(14336, 14336)

    def gate_up_pair(layer):
        qmm._check(L.qmm_matmul_ex(hs_gu[cidx[id(layer)]], 2, x4096.data_ptr(), 1, 4096, ffn_norm.data_ptr(),
                                   ctypes.c_float(1e-5), 0, y_gu, ld_gu, None, 0, qmm._stream(dev)))
    gate_up_pair(sets[0])
    torch.cuda.synchronize()
    sp = time_launch(gate_up_pair)
    b = 2 * gemv_bytes(dt, 14336, 4096) - 4 * 4096 + 4 * 4096  # the row once, plus the norm weight
    per_shape["gate_up_pair_rmsnorm"] = {"shape": [[14336, 4096], [14336, 4096]], "us": round(sp["mean"], 3),
                                         "GB/s": round(b / sp["mean"] / 1e3, 1),
                                         "frac": round(b / sp["mean"] / 1e3 / HBM_PEAK_GBS, 4),
                                         "copies": copies, "us_spread": sp}

    # small batches (the GEMV path serves m <= 8): gate_proj at m = 2, 4, 8 through qmm_matmul (Q8_K of the
    # rows, then the multi-row GEMV), weights rotated over the set copies
    small_m = {}
    for m in (2, 4, 8):
        xm = torch.from_numpy(normal(30 + m, (m, 4096))).to(dev)
        ym = torch.empty((m, 14336), dtype=torch.float32, device=dev)
        wsm = int(L.qmm_matmul_workspace_size(sets[0]["gate_proj"].handle, m))
        wsbuf = torch.empty(max(wsm, 1), dtype=torch.uint8, device=dev)

        def gate_m(layer, m=m, xm=xm, ym=ym, wsbuf=wsbuf, wsm=wsm):
            qmm._check(L.qmm_matmul(layer["gate_proj"].handle, xm.data_ptr(), m, 4096, ym.data_ptr(), 14336,
                                    wsbuf.data_ptr(), wsm, qmm._stream(dev)))
        gate_m(sets[0])
        torch.cuda.synchronize()
        sp = time_launch(gate_m)
        b = 14336 * 16 * 144 + m * 4 * (4096 + 14336)
        small_m[f"m{m}"] = {"shape": [m, 14336, 4096], "us": round(sp["mean"], 3),
                            "GB/s": round(b / sp["mean"] / 1e3, 1),
                            "frac": round(b / sp["mean"] / 1e3 / HBM_PEAK_GBS, 4), "us_spread": sp}

    # dominant launch of the step
    if args.schedule == "grouped":
        # the step is this one launch: algorithmic bytes of the six GEMVs, each activation row read once
        rsp = time_launch(step_grouped)
        rb = step_bytes - 4 * 4096 * (len(QKVGU) - 1)
        kernel = "qmm_gemv1g_q4k_w16 (q, k, v, gate, up on one row and down on another: one launch, Q8_K in the " \
                 "prologue)"
    elif args.schedule == "serial":
        kernel, rb = "qmm_gemv1_q4k_w4 (gate_proj 14336x4096, one launch)", gemv_bytes(dt, 14336, 4096)
        rsp = time_launch(lambda layer: gemv(layer, "gate_proj"))
    else:
        fused = args.schedule == "fused"
        rsp = time_launch(lambda layer: qkvgu(layer, fused))
        rb = sum(gemv_bytes(dt, *shapes[nm]) for nm in QKVGU) - 4 * 4096 * (len(QKVGU) - 1)  # x read once
        kernel = ("qmm_gemv1f_q4k_w16_j8" if fused else "qmm_gemv1_q4k_w4_j8") + \
            " (q, k, v, gate, up: 5 weights, one launch" + (", Q8_K in the prologue)" if fused else ")")
    rus = rsp["mean"]
    achieved = rb / (rus * 1e-6) / 1e9
    result = {
        "value": value,
        "ms_per_step": elapsed / steps * 1e3,
        "steps": steps,
        "step_us": step_spread,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(args.schedule),
                     "kernel": kernel, "avg_us": round(rus, 3), "us": rsp, "algorithmic_bytes": rb},
        "per_shape": per_shape,
        "small_batch_gemv": small_m,
        "weight_copies": copies,
    }
    return result, sets


def run_q8_0(torch, dev, args, cpu):
    """Config 1: the Q8_0 4096x4096 matvec (QMatMul::forward on a Q8 projection, quant.rs:26-43): weight
    N(0, 0.02^2) seed 0 (SplitMix64 + Box-Muller, quantized on the GPU, bit-identical to the CPU
    quantizer), activation 1x4096 N(0, 1) seed 1. One qmm_matmul call = one launch: the f32 row is
    quantized to Q8_0 in the GEMV's prologue. Copies beyond the first (same distribution, device
    generator: SplitMix64 seeds 101, 102, ...) are rotated over > 2x the MALL. The first copy's output is
    checked against the oracle."""
    from inference_amd import GgmlDType, QTensor, qmm
    from inference_amd.synth import normal, normal_torch
    L = qmm.lib()
    n = k = 4096
    wb = n * (k // 32) * 34
    copies = max(2, -(-args.rotate_mb * 2 ** 20 // wb))
    qts = [QTensor.quantize(torch.from_numpy(normal(0, (n, k), 0.02)).to(dev), GgmlDType.Q8_0)]
    qts += [QTensor.quantize(normal_torch(100 + c, (n, k), 0.02, dev), GgmlDType.Q8_0) for c in range(1, copies)]
    xh = normal(1, (1, k))
    x = torch.from_numpy(xh).to(dev)
    y = torch.empty((1, n), dtype=torch.float32, device=dev)
    wsb = int(L.qmm_matmul_workspace_size(qts[0].handle, 1))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    it = iter(range(10 ** 9))

    def fn():
        qmm._check(L.qmm_matmul(qts[next(it) % copies].handle, x.data_ptr(), 1, k, y.data_ptr(), n, ws.data_ptr(),
                                wsb, qmm._stream(dev)))
    sp = timed_graph(torch, fn, copies)
    from oracle import oracle as orc
    w0 = qts[0].to_ggml()
    qmm._check(L.qmm_matmul(qts[0].handle, x.data_ptr(), 1, k, y.data_ptr(), n, ws.data_ptr(), wsb,
                            qmm._stream(dev)))
    want = orc.matmul(orc.Q8_0, xh, w0, k)
    rel = float(np.abs(y.cpu().numpy() - want).max() / np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    b = wb + 4 * k + 4 * n
    us = sp["mean"]
    out = {"shape": [n, k], "us": round(us, 3), "GB/s": round(b / us / 1e3, 1),
           "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "algorithmic_bytes": b, "copies": copies,
           "kernel": "qmm_gemv1f_q8_0_w16 (Q8_0 quantization of the row in the prologue, one launch)", "us_spread": sp,
           "parity_max_rel_vs_oracle": round(rel, 8)}
    if cpu is not None:
        cpu["config1_q8_0_matvec"] = cpu_leg(lambda impl: orc.matmul(orc.Q8_0, xh, w0, k, CPU_THREADS, impl),
                                             b, "GB/s", cpu["budget_s"])
    del qts
    return out


def run_decode(torch, dev, args, cpu=None):
    """Config 3: greedy decode of a random-init Llama-3-8B-shaped Q4_K_M model at batch 1.

    The prompt's first 127 positions run as one batched prefill (matmuls
    with m = 127 on the MFMA GEMM path, batched RoPE + KV append, causal
    attention), timed on its own; then the captured step processes the last
    prompt token and `decode_tokens` - 1 more, one per graph replay. decode
    tok/s is timed over the generated tokens only.
    """
    from inference_amd.llama_decode import DecodeSession, LlamaConfig, LlamaWeights
    cfg = LlamaConfig.llama3_8b()
    log(f"[bench] decode: building the 8B-shape Q4_K_M model (seed 4)")
    t0 = time.perf_counter()
    w = LlamaWeights.random(cfg, 4, dev)
    torch.cuda.synchronize()
    log(f"[bench] decode: weights ready in {time.perf_counter() - t0:.1f} s")
    prompt_len, gen = 128, args.decode_tokens
    rng = np.random.default_rng(4)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab, prompt_len)]
    sess = DecodeSession(w, prompt_len + gen)
    sess.reset(prompt)
    sess.capture()
    # one untimed pass, then the timed pass from a fresh reset (same graph)
    for timed in (False, True):
        sess.reset(prompt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        rows = sess.prefill()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        sess.run(gen)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
    toks = sess.generated(prompt_len + gen)
    assert toks[:prompt_len] == prompt
    tok_s = gen / (t2 - t1)
    if cpu is not None:
        # one config-3 token on the CPU: the oracle's decode step over the same weights (32 layers + head),
        # at position 0 of a fresh cache for every repetition
        from oracle import llama as ol
        from oracle import oracle as orc
        ex = w.export()

        def tok(impl):
            ol.LlamaOracle(cfg, ex, 1, impl).step(prompt[0], 0)
        cpu["config3_decode_token"] = cpu_leg(tok, 1, "tok/s", cpu["budget_s"])
        del ex
    wb = cfg.weight_bytes_per_token()
    return {"tok_s": round(tok_s, 2), "ms_per_token": round((t2 - t1) / gen * 1e3, 4),
            "prompt_tokens": prompt_len, "generated_tokens": gen,
            "prefill": {"rows": rows, "ms": round((t1 - t0) * 1e3, 3), "tok_s": round(rows / (t1 - t0), 1),
                        "schedule": "batched: m = rows GEMMs, causal attention; the last prompt token in the step"},
            "weight_bytes_per_token": wb, "weight_GB_s": round(wb * tok_s / 1e9, 1),
            "weight_hbm_frac": round(wb * tok_s / 1e9 / HBM_PEAK_GBS, 4),
            "model": "llama3-8b-shape Q4_K_M (q/k/o/gate/up Q4_K, v/down/head Q6_K), random init seed 4",
            "schedule": "one HIP graph per token step after a batched prefill of the prompt",
            "first_generated": toks[prompt_len:prompt_len + 8]}


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def timed_graph(torch, fn, per_graph, samples=SPREAD_SAMPLES):
    """Spread of microseconds per fn() call (fn launches on the current stream): a graph of per_graph calls,
    replayed `samples` times with a HIP event between replays, after untimed replays."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    stream = torch.cuda.current_stream()
    replay_samples(torch, g, 2, stream)
    return spread(replay_samples(torch, g, samples, stream) * 1e3 / per_graph)


def run_prefill(torch, dev, cpu=None):
    """Config 4: M = 512 tokens x 4096 (N(0,1), seed 5) through Q4_K 14336x4096 and 4096x14336
    (N(0, 0.02^2), SplitMix64 seeds 6 and 16 on the device; the Q6_K and Q8_0 legs 26 .. 56).
    qmm_matmul: activation quantization to Q8_K planes + the int8-MFMA GEMM. MFMA utilisation =
    2*M*N*K / time / dense int8 peak."""
    from inference_amd import GgmlDType, QTensor, qmm
    from inference_amd.synth import normal, normal_torch
    L = qmm.lib()
    m = 512
    out = {}
    # config 4 proper (Q4_K), then the same shapes in Q6_K (the Q4_K_M down / v projections) and Q8_0 (the
    # engine's Q8 projections)
    legs = [(GgmlDType.Q4K, "gate_up_shape", 14336, 4096), (GgmlDType.Q4K, "down_shape", 4096, 14336),
            (GgmlDType.Q6K, "q6k_gate_up_shape", 14336, 4096), (GgmlDType.Q6K, "q6k_down_shape", 4096, 14336),
            (GgmlDType.Q8_0, "q8_0_gate_up_shape", 14336, 4096), (GgmlDType.Q8_0, "q8_0_down_shape", 4096, 14336)]
    for li, (dt, name, n, k) in enumerate(legs):
        qt = QTensor.quantize(normal_torch(6 + 10 * li, (n, k), 0.02, dev), dt)
        x = torch.from_numpy(normal(5, (m, k))).to(dev)
        y = torch.empty((m, n), dtype=torch.float32, device=dev)
        wsb = int(L.qmm_matmul_workspace_size(qt.handle, m))
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)

        def fn(qt=qt, x=x, y=y, ws=ws, wsb=wsb, n=n, k=k):
            qmm._check(L.qmm_matmul(qt.handle, x.data_ptr(), m, k, y.data_ptr(), n, ws.data_ptr(), wsb,
                                    qmm._stream(dev)))
        sp = timed_graph(torch, fn, 4)
        us = sp["mean"]
        tops = 2.0 * m * n * k / us / 1e6
        out[name] = {"dtype": dt.name, "m_n_k": [m, n, k], "us": round(us, 2), "TOPS": round(tops, 1),
                     "mfma_util": round(tops / INT8_PEAK_TOPS, 4), "us_spread": sp}
        if cpu is not None and dt == GgmlDType.Q4K:
            from oracle import oracle as orc
            wq, xs = qt.to_ggml(), x[:CPU_PREFILL_ROWS].cpu().numpy()
            cpu[f"config4_{name}"] = cpu_leg(lambda impl: orc.matmul(orc.Q4K, xs, wq, k, CPU_THREADS, impl),
                                             2.0 * CPU_PREFILL_ROWS * n * k / 1e12, "TOPS", cpu["budget_s"])
            cpu[f"config4_{name}"]["rows"] = CPU_PREFILL_ROWS
        del qt
    return out


def run_moe(torch, dev):
    """Config 5: 8 experts (Q4_K gate/up 14336x4096, Q6_K down 4096x14336, N(0, 0.02^2) from SplitMix64
    seeds 71 / 72 / 73 on the device), 8 tokens N(0,1) seed 7, router logits N(0,1) seed 8, top-2. One qmm_moe_ffn call:
    routing, gathered Q8_K activations, expert GEMVs streaming each active expert once, SiLU*mul, combine.
    Then MoE prefill on the same experts (512 tokens through the grouped MFMA GEMMs)."""
    from inference_amd import GgmlDType, QTensor, qmm
    from inference_amd.synth import normal, normal_torch
    L = qmm.lib()
    E, H, F, T, k = 8, 4096, 14336, 8, 2
    gate = QTensor.quantize(normal_torch(71, (E * F, H), 0.02, dev), GgmlDType.Q4K)
    up = QTensor.quantize(normal_torch(72, (E * F, H), 0.02, dev), GgmlDType.Q4K)
    down = QTensor.quantize(normal_torch(73, (E * H, F), 0.02, dev), GgmlDType.Q6K)
    x = torch.from_numpy(normal(7, (T, H))).to(dev)
    logits_np = normal(8, (T, E))
    logits = torch.from_numpy(logits_np).to(dev)
    y = torch.empty((T, H), dtype=torch.float32, device=dev)
    wsb = int(L.qmm_moe_ffn_workspace_size(gate.handle, down.handle, T, E, k))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)

    def fn():
        qmm._check(L.qmm_moe_ffn(x.data_ptr(), T, H, logits.data_ptr(), E, k, gate.handle, up.handle, down.handle,
                                 y.data_ptr(), H, ws.data_ptr(), wsb, qmm._stream(dev)))
    sp = timed_graph(torch, fn, 4)
    us = sp["mean"]
    # active experts: those in some token's top-k
    active = set()
    for row in logits_np:
        active.update(np.argsort(-row, kind="stable")[:k].tolist())
    per_expert = F * (H // 256) * 144 * 2 + H * (F // 256) * 210
    wbytes = per_expert * len(active)
    out = {"us": round(us, 2), "active_experts": len(active), "weight_bytes": wbytes,
           "GB/s": round(wbytes / us / 1e3, 1), "hbm_frac": round(wbytes / us / 1e3 / HBM_PEAK_GBS, 4),
           "tokens": T, "topk": k, "us_spread": sp}

    # MoE prefill on the same experts: 512 tokens N(0,1) seed 9, router logits seed 10, top-2; the
    # routed pairs average 128 rows per expert, so qmm_moe_ffn takes the grouped MFMA GEMMs.
    Tp = 512
    xp = torch.from_numpy(normal(9, (Tp, H))).to(dev)
    lp = torch.from_numpy(normal(10, (Tp, E))).to(dev)
    yp = torch.empty((Tp, H), dtype=torch.float32, device=dev)
    wsp = int(L.qmm_moe_ffn_workspace_size(gate.handle, down.handle, Tp, E, k))
    wsv = torch.empty(wsp, dtype=torch.uint8, device=dev)

    def fnp():
        qmm._check(L.qmm_moe_ffn(xp.data_ptr(), Tp, H, lp.data_ptr(), E, k, gate.handle, up.handle, down.handle,
                                 yp.data_ptr(), H, wsv.data_ptr(), wsp, qmm._stream(dev)))
    spp = timed_graph(torch, fnp, 1, 60)
    usp = spp["mean"]
    ops = 2 * Tp * k * 3 * F * H  # int8 ops of the three projections over every routed pair
    out["prefill"] = {"tokens": Tp, "us": round(usp, 2), "TOPS": round(ops / usp / 1e6, 1),
                      "mfma_util": round(ops / usp / 1e6 / INT8_PEAK_TOPS, 4),
                      "schedule": "route, gathered rows quantized to GEMM planes, grouped split-scale MFMA GEMM gate/up, "
                                  "SiLU*mul quantized to planes, grouped GEMM down, combine",
                      "us_spread": spp}
    return out


CPU_THREADS = min(16, len(os.sched_getaffinity(0)))  # the GPU box's CPU share for one GPU is 16
CPU_PREFILL_ROWS = 64  # rows of the config-4 activation timed on the CPU (the CPU matmul is linear in rows)


def cpu_host():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "cpus_in_affinity": len(os.sched_getaffinity(0)),
            "threads_used": CPU_THREADS}


def cpu_leg(fn, units, unit, budget_s):
    """Time fn(impl) for both vec_dot builds of the oracle (candle's generic bodies = the reference's
    default build; its AVX2 + FMA bodies): one warm-up, then >= 5 repetitions within the budget; the median
    gives units / second."""
    from oracle import oracle as orc
    out = {"unit": unit}
    for name, impl in (("avx2", orc.AVX2), ("generic", orc.GENERIC)):
        if impl == orc.AVX2 and not orc.simd_supported():
            continue
        fn(impl)
        times, t_end = [], time.perf_counter() + budget_s
        while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 1000):
            t0 = time.perf_counter()
            fn(impl)
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        out[name] = {"value": round(units / med / (1e9 if unit == "GB/s" else 1), 4), "median_s": round(med, 6),
                     "reps": len(times)}
    return out


def cpu_gemv_set(sets, cpu):
    """Config 2 on the CPU: the oracle's k_quants::matmul over the same Q4_K GEMV set (M = 1), each pass on
    the next of the GPU's rotated weight copies (> 2x the 256 MB MALL, so beyond the host's caches too)."""
    from oracle import oracle as orc
    from inference_amd.synth import normal
    ws = [{name: layer[name].to_ggml() for name, _, _ in GEMV_SET} for layer in sets]
    x4096, x14336 = normal(3, (1, 4096)), normal(3, (1, 14336))
    total_bytes = sum(gemv_bytes(12, n, k) for _, n, k in GEMV_SET)
    turn = iter(range(10 ** 9))

    def one_pass(impl):
        w = ws[next(turn) % len(ws)]
        for name, n, k in GEMV_SET:
            orc.matmul(orc.Q4K, x4096 if k == 4096 else x14336, w[name], k, CPU_THREADS, impl)
    cpu["config2_q4k_gemv_set"] = cpu_leg(one_pass, total_bytes, "GB/s", cpu["budget_s"])


def cpu_summary(cpu):
    """The bench line's cpu_baseline: config 2 with the faster (AVX2) build as `value`, every timed
    config under `configs`."""
    legs = {k: v for k, v in cpu.items() if k not in ("budget_s",)}
    c2 = legs["config2_q4k_gemv_set"]
    best = "avx2" if "avx2" in c2 else "generic"
    return {"value": c2[best]["value"], "unit": "GB/s", "cores": CPU_THREADS, "kind": "port",
            "build": best, "host": cpu_host(),
            "sample": (f"config 2 (the Q4_K GEMV set, M = 1, 6 projections, rotated over the GPU's weight copies) "
                       f"through the oracle's C restatement "
                       f"of candle's k_quants::matmul, {best} vec_dot, {CPU_THREADS} OpenMP threads; median of "
                       f">= 5 repetitions. Also timed, both builds: config 1 (Q8_0 4096x4096 matvec), config 4 "
                       f"({CPU_PREFILL_ROWS} of the 512 rows of each prefill GEMM) and one config-3 decode token "
                       f"(32 layers + head at position 0)"),
            "configs": legs}


def kernel_only(torch, dev, which, launches):
    """Launch one kernel `launches` times, eagerly (every dispatch visible to a counter run):
    `gate` = the Q4_K gate GEMV (14336x4096, M = 1, rotated weight copies); `qkvgu` / `qkvgu_staged`
    = the q/k/v/gate/up set in one launch (Q8_K in the prologue / pre-quantized activation);
    `copy` = a 256 MiB device copy (the calibration for FETCH_SIZE / WRITE_SIZE); `gemm_gate` / `gemm_down` =
    the config-4 GEMMs (M = 512; `gemm_q6k_*` / `gemm_q8_0_*`: its Q6_K / Q8_0 legs); `moe` = the config-5 expert
    FFN (`moe32`: at 32 tokens; `moe_prefill`: at 512 tokens); `gate_m8` = the gate GEMV on eight pre-quantized rows; `gate_up` = gate and up
    in one launch with the RMSNorm + Q8_K prologue (the FFN pair as the decoder runs it); `decode` / `prefill` =
    config-3 token steps / batched 127-row prefills, eagerly."""
    from inference_amd import GgmlDType, QTensor, qmm
    from inference_amd.synth import normal, normal_torch
    if which == "copy":
        a = torch.ones(64 * 2 ** 20, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        for _ in range(launches):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": "copy", "bytes_read": a.numel() * 4, "bytes_written": b.numel() * 4,
                          "launches": launches}), flush=True)
        return
    if which in ("gemm_gate", "gemm_down", "gemm_q6k_gate", "gemm_q6k_down", "gemm_q8_0_gate", "gemm_q8_0_down"):
        # config-4 GEMM: 512 rows N(0,1) seed 5 against a Q4_K weight N(0, 0.02^2) seed 6 / 16, or the Q6_K /
        # Q8_0 legs' weights (seeds 26 / 36, 46 / 56)
        n, k = (14336, 4096) if which.endswith("gate") else (4096, 14336)
        dt = GgmlDType.Q6K if "q6k" in which else GgmlDType.Q8_0 if "q8_0" in which else GgmlDType.Q4K
        base = {GgmlDType.Q4K: 6, GgmlDType.Q6K: 26, GgmlDType.Q8_0: 46}[dt]
        seed = base if which.endswith("gate") else base + 10
        w = QTensor.quantize(normal_torch(seed, (n, k), 0.02, dev), dt)
        x = torch.from_numpy(normal(5, (512, k))).to(dev)
        y = torch.empty((512, n), dtype=torch.float32, device=dev)
        L = qmm.lib()
        wsb = int(L.qmm_matmul_workspace_size(w.handle, 512))
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        for _ in range(launches):
            qmm._check(L.qmm_matmul(w.handle, x.data_ptr(), 512, k, y.data_ptr(), n, ws.data_ptr(), wsb,
                                    qmm._stream(dev)))
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": which, "int8_ops": 2 * 512 * n * k, "launches": launches}), flush=True)
        return
    if which in ("moe", "moe32", "moe_prefill"):
        # config 5: one qmm_moe_ffn call per launch (route, gather, expert GEMVs, SiLU*mul, combine);
        # moe32: the same experts at 32 tokens (the matrix-core expert GEMV for gate / up); moe_prefill: 512
        # tokens (seeds 9 / 10, the bench's MoE prefill: grouped GEMMs and their tails)
        E, H, F, k = 8, 4096, 14336, 2
        T = {"moe": 8, "moe32": 32, "moe_prefill": 512}[which]
        gate = QTensor.quantize(normal_torch(71, (E * F, H), 0.02, dev), GgmlDType.Q4K)
        up = QTensor.quantize(normal_torch(72, (E * F, H), 0.02, dev), GgmlDType.Q4K)
        down = QTensor.quantize(normal_torch(73, (E * H, F), 0.02, dev), GgmlDType.Q6K)
        pre = which == "moe_prefill"
        x = torch.from_numpy(normal(9 if pre else 7, (T, H))).to(dev)
        lg = torch.from_numpy(normal(10 if pre else 8, (T, E))).to(dev)
        y = torch.empty((T, H), dtype=torch.float32, device=dev)
        L = qmm.lib()
        wsb = int(L.qmm_moe_ffn_workspace_size(gate.handle, down.handle, T, E, k))
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        for _ in range(launches):
            qmm._check(L.qmm_moe_ffn(x.data_ptr(), T, H, lg.data_ptr(), E, k, gate.handle, up.handle, down.handle,
                                     y.data_ptr(), H, ws.data_ptr(), wsb, qmm._stream(dev)))
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": which, "tokens": T, "launches": launches}), flush=True)
        return
    if which.startswith("read_") and which != "read_graph":
        # plain streaming reads of a buffer of the GEMV launches' sizes (q 9.5 MB, gate 33 MB, the five-weight
        # launch 80 MB, 1 GB), rotating copies over > 512 MB: every read variant (grid-stride 4 / 8 in flight,
        # chunked nontemporal) at 8 and 16 workgroups per CU, `launches` each; the fastest is the ceiling a
        # launch of that size can reach
        from inference_amd import qmm
        L = qmm.lib()
        nbytes = {"read_9mb": 9469952, "read_33mb": 33103872, "read_80mb": 80371712, "read_1gb": 1 << 30}[which]
        nbytes = (nbytes + 15) // 16 * 16
        nc = max(1, -(-(640 << 20) // nbytes))
        bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device=dev) for _ in range(nc)]
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        runs = [(v, w) for v in (0, 1, 2) for w in (8, 16)]
        for v, w in runs:
            for i in range(launches):
                qmm._check(L.qmm_stream_read(bufs[i % nc].data_ptr(), nbytes, sink.data_ptr(), v, w,
                                             qmm._stream(dev)))
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": which, "bytes": nbytes, "copies": nc, "launches_per_variant": launches,
                          "variants_wgs_per_cu": runs}), flush=True)
        return
    if which == "read_graph":
        # the read variants of the read_* modes timed in HIP-graph replays (back-to-back launches over the
        # rotated copies, median of `launches`-sample spreads) at every size: the graph-replay ceiling
        from inference_amd import qmm
        L = qmm.lib()
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        for nbytes in (9469952, 33103872, 80371712, 1 << 30):
            nc = max(1, -(-(640 << 20) // nbytes))
            bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device=dev) for _ in range(nc)]
            for v, name in enumerate(("gs4", "gs8", "ch8nt")):
                for w in (8, 16):
                    j = [0]

                    def rd():
                        qmm._check(L.qmm_stream_read(bufs[j[0] % nc].data_ptr(), nbytes, sink.data_ptr(), v, w,
                                                     qmm._stream(dev)))
                        j[0] += 1
                    sp = timed_graph(torch, rd, max(2 * nc, 4), min(launches, 20 if nbytes > (1 << 29) else 40))
                    print(json.dumps({"kernel_only": "read_graph", "bytes": nbytes, "variant": name,
                                      "wgs_per_cu": w, "us": sp}), flush=True)
            del bufs
        return
    if which == "decode":
        # config 3: the 8B-shape Q4_K_M model, a 128-token prompt through the batched prefill, then
        # `launches` token steps run eagerly (every kernel of a step is its own dispatch in a trace)
        from inference_amd.llama_decode import DecodeSession, LlamaConfig, LlamaWeights
        cfg = LlamaConfig.llama3_8b()
        w = LlamaWeights.random(cfg, 4, dev)
        prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.vocab, 128)]
        sess = DecodeSession(w, 128 + launches)
        sess.reset(prompt)
        sess.prefill()
        sess.run(launches, use_graph=False)
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": "decode", "steps": launches, "positions": [127, 127 + launches - 1]}),
              flush=True)
        return
    if which == "prefill":
        # config 3: the 8B-shape Q4_K_M model, `launches` eager batched prefills of a 128-token prompt (127
        # rows through the GEMM path; every kernel its own dispatch in a trace)
        from inference_amd.llama_decode import DecodeSession, LlamaConfig, LlamaWeights
        cfg = LlamaConfig.llama3_8b()
        w = LlamaWeights.random(cfg, 4, dev)
        prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.vocab, 128)]
        sess = DecodeSession(w, 128 + 8)
        ms = []
        for _ in range(launches):
            sess.reset(prompt)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            rows = sess.prefill()
            torch.cuda.synchronize()
            ms.append(round((time.perf_counter() - t0) * 1e3, 3))
        print(json.dumps({"kernel_only": "prefill", "prefills": launches, "rows": rows, "ms": ms}), flush=True)
        return
    if which in ("q8_0", "down_q6k"):
        # config 1: the Q8_0 4096x4096 matvec, one qmm_matmul (fused Q8_0 prologue) per launch; or the
        # decode step's Q6_K down projection 4096x14336 with a pre-quantized Q8_K row. Rotated copies.
        L = qmm.lib()
        dt, n, k = (GgmlDType.Q8_0, 4096, 4096) if which == "q8_0" else (GgmlDType.Q6K, 4096, 14336)
        nc = 38 if which == "q8_0" else 14
        ws = [QTensor.quantize(normal_torch(200 + c, (n, k), 0.02, dev), dt) for c in range(nc)]
        x = torch.randn(k, device=dev)
        y = torch.empty(n, dtype=torch.float32, device=dev)
        if which == "q8_0":
            wsb = int(L.qmm_matmul_workspace_size(ws[0].handle, 1))
            buf = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
            for i in range(launches):
                qmm._check(L.qmm_matmul(ws[i % nc].handle, x.data_ptr(), 1, k, y.data_ptr(), n, buf.data_ptr(), wsb,
                                        qmm._stream(dev)))
            alg = n * (k // 32) * 34 + 4 * k + 4 * n
        else:
            xq = torch.zeros(k // 256 * 292, dtype=torch.uint8, device=dev)
            qmm._check(L.qmm_quantize_rows(15, x.data_ptr(), 1, k, k, xq.data_ptr(), qmm._stream(dev)))
            for i in range(launches):
                qmm._check(L.qmm_matmul_q(ws[i % nc].handle, xq.data_ptr(), 1, y.data_ptr(), n, None, 0,
                                          qmm._stream(dev)))
            alg = n * (k // 256) * 210 + 4 * k + 4 * n
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": which, "algorithmic_bytes": alg, "launches": launches}), flush=True)
        return
    L = qmm.lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    x = torch.randn(4096, device=dev)
    xq = torch.zeros(16 * 292, dtype=torch.uint8, device=dev)
    qmm._check(L.qmm_quantize_rows(15, x.data_ptr(), 1, 4096, 4096, xq.data_ptr(), qmm._stream(dev)))
    if which == "grouped":
        # the config-2 set as one qmm_matmul_grouped launch, over rotated copies
        nc = 6
        sets = [[QTensor.quantize(normal_torch(2 + 1000 * c + 17 * i, (n, k), 0.02, dev), GgmlDType.Q4K)
                 for i, (_, n, k) in enumerate(GEMV_SET)] for c in range(nc)]
        x14 = torch.randn(14336, device=dev)
        ys = [torch.empty(n, dtype=torch.float32, device=dev) for _, n, _ in GEMV_SET]
        hs = [(vp * 6)(*[t.handle.value for t in c]) for c in sets]
        gp = (ctypes.c_int * 6)(0, 0, 0, 0, 0, 1)
        xp = (vp * 2)(x.data_ptr(), x14.data_ptr())
        yp = (vp * 6)(*[y.data_ptr() for y in ys])
        for i in range(launches):
            qmm._check(L.qmm_matmul_grouped(hs[i % nc], gp, 6, xp, yp, qmm._stream(dev)))
        alg = sum(gemv_bytes(12, n, k) for _, n, k in GEMV_SET) - 4 * 4096 * 4
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": which, "algorithmic_bytes": alg, "launches": launches}), flush=True)
        return
    if which == "gate_up":
        # the FFN pair as the decoder runs it: gate and up in one launch, RMSNorm + Q8_K of the f32 row in
        # the prologue; 8 rotated copies of the pair (530 MB, more than the MALL)
        pairs = [[QTensor.quantize(normal_torch(2 + 1000 * c + 17 * j, (14336, 4096), 0.02, dev), GgmlDType.Q4K)
                  for j in (3, 4)] for c in range(8)]
        hs = [(vp * 2)(*[q.handle.value for q in pr]) for pr in pairs]
        nw = torch.from_numpy(normal(4, (4096,))).to(dev)
        ys = [torch.empty(14336, dtype=torch.float32, device=dev) for _ in range(2)]
        yp = (vp * 2)(*[y.data_ptr() for y in ys])
        ld = (i64 * 2)(14336, 14336)
        for i in range(launches):
            qmm._check(L.qmm_matmul_ex(hs[i % 8], 2, x.data_ptr(), 1, 4096, nw.data_ptr(), ctypes.c_float(1e-5), 0,
                                       yp, ld, None, 0, qmm._stream(dev)))
        alg = 2 * gemv_bytes(12, 14336, 4096)  # the row once plus the norm weight: 2 x 4 x 4096
        torch.cuda.synchronize()
        print(json.dumps({"kernel_only": which, "algorithmic_bytes": alg, "launches": launches}), flush=True)
        return
    if which in ("gate", "gate_m8"):
        # gate_m8: eight pre-quantized Q8_K rows (the matrix-core multi-token GEMV)
        m = 8 if which == "gate_m8" else 1
        ws = [QTensor.quantize(normal_torch(2 + 1000 * c + 17 * 3, (14336, 4096), 0.02, dev), GgmlDType.Q4K)
              for c in range(8)]
        if m > 1:
            xm = torch.from_numpy(normal(11, (m, 4096))).to(dev)
            xq = torch.zeros(m * 16 * 292, dtype=torch.uint8, device=dev)
            qmm._check(L.qmm_quantize_rows(15, xm.data_ptr(), m, 4096, 4096, xq.data_ptr(), qmm._stream(dev)))
        y = torch.empty(m * 14336, dtype=torch.float32, device=dev)
        for i in range(launches):
            qmm._check(L.qmm_matmul_q(ws[i % 8].handle, xq.data_ptr(), m, y.data_ptr(), 14336, None, 0,
                                      qmm._stream(dev)))
        alg = gemv_bytes(12, 14336, 4096) + (m - 1) * 4 * (4096 + 14336)
    else:
        names = [nm for nm, _, _ in GEMV_SET if nm != "down_proj"]
        shp = {nm: (n, k) for nm, n, k in GEMV_SET}
        copies = [[QTensor.quantize(normal_torch(2 + 1000 * c + 17 * i, shp[nm], 0.02, dev), GgmlDType.Q4K)
                   for i, nm in enumerate(names)] for c in range(6)]
        hs = [(vp * 5)(*[t.handle.value for t in c]) for c in copies]
        ys = [torch.empty(shp[nm][0], dtype=torch.float32, device=dev) for nm in names]
        yp = (vp * 5)(*[y.data_ptr() for y in ys])
        ld = (i64 * 5)(*[shp[nm][0] for nm in names])
        for i in range(launches):
            if which == "qkvgu":
                qmm._check(L.qmm_matmul_ex(hs[i % 6], 5, x.data_ptr(), 1, 4096, None, ctypes.c_float(0), 0, yp, ld,
                                           None, 0, qmm._stream(dev)))
            else:
                qmm._check(L.qmm_matmul_multi_q(hs[i % 6], 5, xq.data_ptr(), 1, yp, ld, None, 0, qmm._stream(dev)))
        alg = sum(gemv_bytes(12, *shp[nm]) for nm in names) - 4 * 4096 * (len(names) - 1)
    torch.cuda.synchronize()
    print(json.dumps({"kernel_only": which, "algorithmic_bytes": alg, "launches": launches}), flush=True)


PMC_PROFILES = {"serial": "gemv_q4k_gate_pmc.json", "staged": "gemv_q4k_qkvgu_staged_pmc.json",
                "fused": "gemv_q4k_qkvgu_fused_pmc.json", "grouped": "gemv_q4k_grouped_set_pmc.json"}


def traffic_from_profile(schedule):
    """HBM bytes per launch of the schedule's roofline kernel from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", PMC_PROFILES[schedule])
    try:
        with open(path) as f:
            d = json.load(f)
        return int(d["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--rotate-mb", type=int, default=640, help="distinct weight bytes rotated (MiB)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--schedule", choices=("grouped", "fused", "staged", "serial"), default="grouped",
                    help="grouped: the six GEMVs in one launch (q/k/v/gate/up on one row, down on the other, "
                         "Q8_K quantization in the prologue); staged: quantize x (Q8_K), q/k/v/gate/up in one "
                         "launch, quantize, down; fused: the same two GEMV launches with Q8_K quantization in "
                         "their prologues; serial: one launch per projection")
    ap.add_argument("--decode-tokens", type=int, default=256, help="config-3 generated tokens (0 = skip)")
    ap.add_argument("--kernel-only", choices=("gate", "gate_m8", "gate_up", "qkvgu", "qkvgu_staged", "grouped", "copy",
                                              "gemm_gate", "gemm_down", "gemm_q6k_gate", "gemm_q6k_down",
                                              "gemm_q8_0_gate", "gemm_q8_0_down", "moe", "moe32", "moe_prefill",
                                              "q8_0", "down_q6k", "decode", "prefill", "read_9mb", "read_33mb",
                                              "read_80mb", "read_1gb", "read_graph"),
                    default=None,
                    help="launch only one GEMV launch kind or a calibration copy --steps times (counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              f"(the path runs on one GPU; it is measured at one GPU's share of the work)", file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.kernel_only:
        kernel_only(torch, dev, args.kernel_only, args.steps)
        return
    cpu = {"budget_s": args.cpu_seconds / 10.0} if args.cpu_seconds > 0 else None
    res, sets = run_gemv_set(torch, dev, args)
    if cpu is not None:
        log("[bench] CPU baseline: config 2")
        cpu_gemv_set(sets, cpu)
    del sets
    torch.cuda.empty_cache()
    log("[bench] Q8_0 matvec (config 1)")
    q80 = run_q8_0(torch, dev, args, cpu)
    torch.cuda.empty_cache()
    dec = run_decode(torch, dev, args, cpu) if args.decode_tokens > 0 else None
    torch.cuda.empty_cache()
    log("[bench] prefill GEMM (config 4)")
    pre = run_prefill(torch, dev, cpu)
    torch.cuda.empty_cache()
    log("[bench] MoE expert FFN (config 5)")
    moe = run_moe(torch, dev)
    line = {
        "metric": METRIC,
        "value": round(res["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "q4k_decode_gemv_set_llama3_8b_m1", "shapes_out_in": [[n, k] for _, n, k in GEMV_SET],
                   "batch_m": 1, "weights": "Q4_K, N(0,0.02^2) SplitMix64 + Box-Muller, seed 2 + 1000 copy + 17 index", "activations": "Q8_K on device, seed 3",
                   "weight_copies_rotated": res["weight_copies"], "schedule": args.schedule},
        "hbm_frac": round(res["value"] / HBM_PEAK_GBS, 4),
        "step_us": res["step_us"],
        "roofline": res["roofline"],
        "per_shape": res["per_shape"],
        "small_batch_gemv": res["small_batch_gemv"],
        "q8_0_matvec": q80,
        "decode_tok_s": dec["tok_s"] if dec else None,
        "decode": dec,
        "prefill_gemm": pre,
        "moe_ffn": moe,
        "cpu_baseline": cpu_summary(cpu) if cpu is not None else None,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
