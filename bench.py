"""Benchmark of the quantized-linear hot path on one MI355X.

Workload: one 27B-class dense decoder layer's linears -- hidden 5120, q
[6144, 5120], k and v [1024, 5120], o [5120, 6144], gate and up
[17408, 5120], down [5120, 17408]; 340,787,200 weights per layer.  Weights
are N(0, 0.02), quantized on the GPU by the library's own quantizers;
activations are bf16 N(0, 1).

A step is one decode pass (M = 1) over the layer's seven linears in W8A16
(int8 per row + bf16 scale), as DIAL's split projections call them: q / k / v
on one activation and gate / up on another run as grouped forwards
(dialq_linear_forward_group, the replacement of QkvProjection::Split and
MlpGateUpProjection::Split: one launch each), o and down alone -- four
launches, captured once per layer copy in a HIP graph and replayed (the
serving loop's launch path; no host work per linear).  The same seven
linears as seven separate forwards are reported as decode_gbs_ungrouped.
Layer copies rotate so the weight working set (COPIES x 341 MB) exceeds the
256 MB Infinity Cache and the figure measures HBM.  `value` = algorithmic
weight bytes streamed / wall time of the timed steps, in GB/s.  Extra keys
report the same decode for Q4_K / Q8_0 / FP8-128 / MXFP4, the prefill GEMM
TFLOP/s (W8A16, Q4_K and Q8_0 at M = 2048 -- Q4_K also with f16 activations, the dtype
of DIAL's GGUF worker, and Q6_K on the gate shape from synthetic blocks --, FP8-128 and MXFP4 native at M = 1024; q / k / v
and gate / up as grouped forwards like the decode step, and as seven
forwards in prefill_tflops_ungrouped; also over
the fused qkv / o / gate_up / down projections DIAL's layers call, with and
without gate_up's SwiGLU epilogue), the quantized lm_head decode GEMV (vocab
248320 x 5120) and the device token selection after it, the roofline of the
dominant kernel and the CPU baseline.

`--profile` runs only the dominant kernel (the grouped W8A16 gate / up
decode launch, eager, over rotating copies; `--profile-format` another
weight format) plus a 256 MiB device-to-device copy used to scale the HBM
byte counters; `--profile-layer` replays only the headline decode step;
`--profile-lm-head` the same for the lm_head GEMV;
`--profile-prefill` runs only the prefill GEMMs of one
layer per format, `--profile-prefill-gate` only the gate-shape prefill GEMM
per format (the counter runs), `--profile-swiglu` the fused gate_up with and without its
SwiGLU epilogue, `--profile-select` the token selection.  They are the
programs the committed rocprofv3 summaries run.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "dial-27b_amd"))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "fp8": 5000.0, "fp4": 10100.0}
LAYER_27B = [("q", 6144, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 6144),
             ("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]
# The same weights as the fused projections DIAL's Qwen3-VL layers run
# (cat(q, k, v) rows and cat(gate, up) rows, qwen3_vl/text.rs): four linears.
LAYER_27B_FUSED = [("qkv", 8192, 5120), ("o", 5120, 6144), ("gate_up", 34816, 5120), ("down", 5120, 17408)]
LM_HEAD_27B = (248320, 5120)  # vocab x hidden
METRIC = "quant GEMV weight GB/s (% HBM peak) + prefill GEMM TFLOP/s, 27B shapes, 1 GPU"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--copies", type=int, default=3, help="layer copies rotated per step")
    ap.add_argument("--settle-seconds", type=float, default=2.0,
                    help="untimed replays of the decode step before the timed region, so that the GPU "
                         "clocks have left their idle state (reported as settle_s)")
    ap.add_argument("--prefill-iters", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the lm_head decode line")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--sweep", default="w8a16,q4_k,q8_0,fp8_block,mxfp4",
                    help="formats for the extra decode / prefill numbers ('' = none)")
    ap.add_argument("--profile", action="store_true",
                    help="only the dominant kernel's launches and the calibration copy (for rocprofv3)")
    ap.add_argument("--profile-launches", type=int, default=50)
    ap.add_argument("--profile-format", default="w8a16", choices=["w8a16", "q4_k", "fp8_block", "mxfp4"],
                    help="weight format of the --profile launches")
    ap.add_argument("--profile-layer", action="store_true",
                    help="only decode-step replays of the W8A16 layer (for a per-launch kernel trace)")
    ap.add_argument("--profile-lm-head", action="store_true",
                    help="run only the W8A16 lm_head GEMV (vocab 248320 x 5120) for rocprofv3")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="only the prefill GEMMs of one layer per format (for rocprofv3)")
    ap.add_argument("--profile-swiglu", action="store_true",
                    help="only the fused gate_up GEMV / GEMM, plain and with the SwiGLU epilogue (for rocprofv3)")
    ap.add_argument("--profile-select", action="store_true",
                    help="only the token selection over the 27B vocabulary (for rocprofv3)")
    ap.add_argument("--profile-prefill-gate", action="store_true",
                    help="only the prefill GEMM of the gate shape 17408x5120 per format, eager (for "
                         "rocprofv3 counter runs)")
    return ap.parse_args()


DOM = ("gate", 17408, 5120)   # the layer's largest linear (gate/up/down tie on bytes)
DOM_COPIES = 6                # 6 x 89 MB rotated: beyond the 256 MB Infinity Cache
# The decode pass as DIAL's split projections call it: q / k / v on one x
# and gate / up on another, each pair or triple one grouped forward
# (dialq_linear_forward_group, the replacement of QkvProjection::Split and
# MlpGateUpProjection::Split), o and down alone -- four launches.
LAYER_27B_GROUPS = [("qkv", (0, 1, 2)), ("o", (3,)), ("gate_up", (4, 5)), ("down", (6,))]
DOM_GROUP = ("gate_up", [17408, 17408], 5120)  # the dominant launch of the grouped pass
DOM_GROUP_COPIES = 3                            # 3 x 178 MB rotated


def capture(torch, fn):
    """Capture fn(stream) into a HIP graph (torch.cuda.CUDAGraph)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn(torch.cuda.current_stream())
    return g


def read_traffic():
    """HBM bytes per launch of the dominant kernel from the committed PMC
    summary (profiles/gemv_w8a16_gate_up_group_2x17408x5120_traffic.txt), if
    present."""
    path = os.path.join(ROOT, "profiles", "gemv_w8a16_gate_up_group_2x17408x5120_traffic.txt")
    try:
        vals = {}
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch") or line.startswith("fetch_bytes") or \
               line.startswith("write_bytes"):
                k, v = line.split("=", 1)
                vals[k.strip()] = float(v.split()[0])
        return vals
    except (OSError, ValueError):
        return None


def build_layers(dq, torch, fmt, copies, dev, seed=0, shapes=LAYER_27B):
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = []
    for _ in range(copies):
        lins = []
        for name, n, k in shapes:
            w = torch.randn(n, k, device=dev, generator=g, dtype=torch.float32) * 0.02
            lins.append(dq.Linear.quantize(fmt, w, scale_dtype=dq.BF16))
            del w
        layers.append(lins)
    torch.cuda.synchronize()
    return layers


def layer_bytes(dq, fmt, shapes=LAYER_27B):
    return sum(dq.raw_weight_bytes(fmt, n, k) for _, n, k in shapes)


def out_cols(name, n, swiglu):
    """Output width of a linear: half the rows when the fused gate_up runs
    with the SwiGLU epilogue (silu(gate) * up)."""
    return n // 2 if name in swiglu else n


def run_linear(lin, name, x, y, swiglu, **kw):
    if name in swiglu:
        lin.forward_swiglu(x, y, **kw)
    else:
        lin.forward(x, y, **kw)


def decode_pass(dq, lins, xs, ys, stream, shapes=LAYER_27B, swiglu=(), groups=None, rows=1):
    if groups is not None:
        for (gname, idx), x, y in zip(groups, xs, ys):
            if len(idx) == 1:
                lins[idx[0]].forward(x, y, rows=rows, path=dq.PATH_GEMV, stream=stream)
            else:
                dq.forward_group([lins[i] for i in idx], x, y, rows=rows, path=dq.PATH_GEMV, stream=stream)
        return
    for lin, x, y, (name, _, _) in zip(lins, xs, ys, shapes):
        run_linear(lin, name, x, y, swiglu, rows=rows, path=dq.PATH_GEMV, stream=stream)


def time_decode(dq, torch, layers, steps, warmup, dev, shapes=LAYER_27B, swiglu=(), xdtype=None, settle=0.0,
                groups=None, rows=1):
    """Wall time of `steps` decode passes, one HIP-graph replay per pass,
    rotating layer copies.  Linears named in `swiglu` (a fused gate_up) run
    with the SwiGLU epilogue; activations and outputs are bf16 unless
    `xdtype` says otherwise.  After `warmup` replays, replays continue
    untimed for `settle` seconds of wall time (clock ramp-up), then exactly
    `steps` replays are timed.  With `groups` ([(name, indices of shapes)]),
    the linears of a group share one x and run as one grouped forward into
    their concatenated output.  `rows`: tokens per pass (decode GEMV)."""
    xdtype = xdtype or torch.bfloat16
    if groups is not None:
        xs = [torch.randn(rows, shapes[idx[0]][2], device=dev).to(xdtype) for _, idx in groups]
        ys = [torch.empty(rows, sum(shapes[i][1] for i in idx), device=dev, dtype=xdtype) for _, idx in groups]
    else:
        xs = [torch.randn(rows, k, device=dev).to(xdtype) for _, n, k in shapes]
        ys = [torch.empty(rows, out_cols(name, n, swiglu), device=dev, dtype=xdtype) for name, n, k in shapes]
    stream = torch.cuda.current_stream()
    for lins in layers:  # eager first: sizes the GEMV workspaces outside capture
        decode_pass(dq, lins, xs, ys, stream, shapes, swiglu, groups, rows)
    torch.cuda.synchronize()
    graphs = [capture(torch, lambda st, l=lins: decode_pass(dq, l, xs, ys, st, shapes, swiglu, groups, rows))
              for lins in layers]
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    t_settle = time.perf_counter()
    i = 0
    while time.perf_counter() - t_settle < settle:
        for _ in range(20):
            graphs[i % len(graphs)].replay()
            i += 1
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def time_launches(dq, torch, lins, k, n, dev, reps=60):
    """Average device time of one GEMV launch: `reps` launches over the
    rotating `lins` captured in a graph, bracketed by HIP events on the
    stream the graph (and so every kernel) runs on."""
    x = torch.randn(1, k, device=dev).to(torch.bfloat16)
    y = torch.empty(1, n, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream()
    for lin in lins:
        lin.forward(x, y, rows=1, path=dq.PATH_GEMV, stream=stream)
    torch.cuda.synchronize()

    def body(st):
        for i in range(reps):
            lins[i % len(lins)].forward(x, y, rows=1, path=dq.PATH_GEMV, stream=st)
    g = capture(torch, body)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3  # seconds per launch


def time_group_launches(dq, torch, groups_of_lins, k, n_total, dev, reps=60):
    """Average device time of one grouped decode launch: `reps` grouped
    forwards over the rotating member lists, in a graph between HIP events
    on the replay stream."""
    x = torch.randn(1, k, device=dev).to(torch.bfloat16)
    y = torch.empty(1, n_total, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream()
    for lins in groups_of_lins:
        dq.forward_group(lins, x, y, rows=1, path=dq.PATH_GEMV, stream=stream)
    torch.cuda.synchronize()

    def body(st):
        for i in range(reps):
            dq.forward_group(groups_of_lins[i % len(groups_of_lins)], x, y, rows=1, path=dq.PATH_GEMV, stream=st)
    g = capture(torch, body)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3


def time_per_group(dq, torch, layers, dev):
    out = {}
    for gname, idx in LAYER_27B_GROUPS:
        members = [[l[i] for i in idx] for l in layers]
        out[gname] = time_group_launches(dq, torch, members, LAYER_27B[idx[0]][2],
                                         sum(LAYER_27B[i][1] for i in idx), dev)
    return out


def time_per_linear(dq, torch, layers, dev):
    out = {}
    for li, (name, n, k) in enumerate(LAYER_27B):
        out[name] = time_launches(dq, torch, [l[li] for l in layers], k, n, dev)
    return out


def profile_run(dq, torch, dev, launches, fmt_name="w8a16"):
    """Dominant kernel only -- the grouped gate / up decode launch (two
    17408x5120 members, 178 MB in W8A16) over rotating copies, eager -- plus
    the calibration copy.  `fmt_name` picks the weight format (copies enough
    to exceed the 256 MB last-level cache)."""
    name, ns, k = DOM_GROUP
    fmt = {"w8a16": dq.W8A16, "q4_k": dq.Q4_K, "fp8_block": dq.FP8_BLOCK, "mxfp4": dq.MXFP4}[fmt_name]
    copies = DOM_GROUP_COPIES if fmt == dq.W8A16 else 6
    g = torch.Generator(device=dev).manual_seed(7)
    groups = []
    for _ in range(copies):
        groups.append([dq.Linear.quantize(fmt, torch.randn(n, k, device=dev, generator=g) * 0.02,
                                          scale_dtype=dq.BF16) for n in ns])
    x = torch.randn(1, k, device=dev).to(torch.bfloat16)
    y = torch.empty(1, sum(ns), device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream()
    for i in range(launches):
        dq.forward_group(groups[i % copies], x, y, rows=1, path=dq.PATH_GEMV, stream=stream)
    torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"# profile: {launches} grouped launches of {fmt_name} {name} 2 x [{ns[0]}x{k}] M=1; 3 copies of 256 MiB "
          "(calibration: 268435456 bytes read and written per copy)", flush=True)


def profile_layer_run(dq, torch, dev, replays=200):
    """The headline decode step as timed: the 27B layer's four grouped /
    single launches (q/k/v, o, gate/up, down) captured per layer copy and
    replayed `replays` times, so a kernel trace shows every launch of the
    step and the gaps between them."""
    layers = build_layers(dq, torch, dq.W8A16, 3, dev)
    time_decode(dq, torch, layers, replays, 20, dev, groups=LAYER_27B_GROUPS)
    print(f"# profile: {replays} decode-step replays of the W8A16 27B layer (4 launches each), 3 copies",
          flush=True)


def profile_swiglu_run(dq, torch, dev, launches=20):
    """The 27B fused gate_up (34816 x 5120, W8A16), eager: decode (M = 1)
    and prefill (M = 2048), plain then with the SwiGLU epilogue."""
    n, k = 34816, 5120
    g = torch.Generator(device=dev).manual_seed(13)
    lins = [dq.Linear.quantize(dq.W8A16, torch.randn(n, k, device=dev, generator=g) * 0.02, scale_dtype=dq.BF16)
            for _ in range(3)]
    stream = torch.cuda.current_stream()
    for m, path in ((1, dq.PATH_GEMV), (2048, dq.PATH_GEMM)):
        x = torch.randn(m, k, device=dev).to(torch.bfloat16)
        y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        h = torch.empty(m, n // 2, device=dev, dtype=torch.bfloat16)
        for i in range(launches):
            lins[i % 3].forward(x, y, path=path, stream=stream)
        for i in range(launches):
            lins[i % 3].forward_swiglu(x, h, path=path, stream=stream)
        torch.cuda.synchronize()
    print(f"# profile: W8A16 gate_up [{n}x{k}], {launches} launches each of M=1 GEMV and M=2048 GEMM, "
          "plain then SwiGLU", flush=True)


def profile_select_run(dq, torch, dev, calls=20):
    """dialq_logits_select over 248320 bf16 logits: argmax, top-8, top-50 and
    top-256 with temperature 0.8."""
    vocab = LM_HEAD_27B[0]
    x = (torch.randn(vocab, device=dev, generator=torch.Generator(device=dev).manual_seed(17)) * 3).to(torch.bfloat16)
    ws = torch.empty(dq.logits_select_workspace_bytes(vocab), dtype=torch.uint8, device=dev)
    for k, rule, t in ((1, dq.SELECT_FIRST_MAX, 0.0), (8, dq.SELECT_TOTAL_LAST_MAX, 0.8),
                       (50, dq.SELECT_TOTAL_LAST_MAX, 0.8), (256, dq.SELECT_TOTAL_LAST_MAX, 0.8)):
        for _ in range(calls):
            dq.logits_select(x, k, rule=rule, temperature=t, workspace=ws)
    torch.cuda.synchronize()
    print(f"# profile: token selection over {vocab} bf16 logits, {calls} calls each of k = 1, 8, 50, 256", flush=True)


def profile_lm_head_run(dq, torch, dev, launches=20):
    """The quantized lm_head GEMV (vocab 248320 x 5120, W8A16, one 1.27 GB
    copy, eager launches) plus the calibration copy."""
    vn, vk = LM_HEAD_27B
    g = torch.Generator(device=dev).manual_seed(21)
    lin = dq.Linear.quantize(dq.W8A16, torch.randn(vn, vk, device=dev, generator=g) * 0.02, scale_dtype=dq.BF16)
    torch.cuda.empty_cache()
    x = torch.randn(1, vk, device=dev).to(torch.bfloat16)
    y = torch.empty(1, vn, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream()
    for _ in range(launches):
        lin.forward(x, y, rows=1, path=dq.PATH_GEMV, stream=stream)
    torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"# profile: {launches} launches of W8A16 lm_head [{vn}x{vk}] M=1 "
          f"({dq.raw_weight_bytes(dq.W8A16, vn, vk)} weight bytes per launch); 3 copies of 256 MiB "
          "(calibration: 268435456 bytes read and written per copy)", flush=True)


def profile_prefill_run(dq, torch, dev, iters=5):
    """Prefill GEMMs of one 27B layer: FP8-128 and MXFP4 native at M = 1024,
    W8A16 and Q4_K weight-only at M = 2048; each layer runs once eagerly,
    once from its captured graph and `iters` more graph replays timed."""
    for fmt, m, path in ((dq.FP8_BLOCK, 1024, dq.PATH_GEMM_NATIVE), (dq.MXFP4, 1024, dq.PATH_GEMM_NATIVE),
                         (dq.W8A16, 2048, dq.PATH_GEMM), (dq.Q4_K, 2048, dq.PATH_GEMM)):
        lins = build_layers(dq, torch, fmt, 1, dev)[0]
        tf, secs = time_prefill(dq, torch, lins, m, iters, dev, path)
        print(f"# profile prefill {dq.FORMAT_NAMES[fmt]} M={m}: {tf:.1f} TFLOP/s ({secs * 1e3:.3f} ms/layer)",
              flush=True)
        del lins
        torch.cuda.empty_cache()


def time_prefill(dq, torch, lins, m, iters, dev, path, shapes=LAYER_27B, swiglu=(), act="bfloat16", groups=None):
    """Device time of one prefill pass over the layer's seven linears
    (activation quantization included for the native paths), captured in a
    HIP graph like the decode step and replayed `iters` times between HIP
    events on the replay stream.  With `groups` ([(name, indices of
    shapes)]), the linears of a group share one x and run as one grouped
    forward into their concatenated output, as in the decode step."""
    stream = torch.cuda.current_stream()
    dt = getattr(torch, act)
    if groups is not None:
        xs = [torch.randn(m, shapes[idx[0]][2], device=dev).to(dt) for _, idx in groups]
        ys = [torch.empty(m, sum(shapes[i][1] for i in idx), device=dev, dtype=dt) for _, idx in groups]
    else:
        xs = [torch.randn(m, k, device=dev).to(dt) for _, n, k in shapes]
        ys = [torch.empty(m, out_cols(name, n, swiglu), device=dev, dtype=dt) for name, n, k in shapes]

    def body(st):
        if groups is not None:
            for (_, idx), x, y in zip(groups, xs, ys):
                if len(idx) == 1:
                    lins[idx[0]].forward(x, y, path=path, stream=st)
                else:
                    dq.forward_group([lins[i] for i in idx], x, y, path=path, stream=st)
            return
        for lin, x, y, (name, _, _) in zip(lins, xs, ys, shapes):
            run_linear(lin, name, x, y, swiglu, path=path, stream=st)
    body(stream)  # eager first: sizes the handles' scratch outside capture
    torch.cuda.synchronize()
    g = capture(torch, body)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        g.replay()
    e1.record(stream)
    e1.synchronize()
    secs = e0.elapsed_time(e1) * 1e-3 / iters
    flops = 2.0 * m * sum(n * k for _, n, k in shapes)
    return flops / secs / 1e12, secs


def time_select(dq, torch, vocab, dev, reps=50):
    """Device time of dialq_logits_select over one row of bf16 logits: the
    greedy argmax and the top-50 candidates with softmax statistics (what
    sampling with top_k = 50 reads back), captured in a graph and replayed."""
    x = (torch.randn(vocab, device=dev) * 3).to(torch.bfloat16)
    ws = torch.empty(dq.logits_select_workspace_bytes(vocab), dtype=torch.uint8, device=dev)
    out = {}
    for name, k, rule, t in (("argmax", 1, dq.SELECT_FIRST_MAX, 0.0), ("top50_t0.8", 50, dq.SELECT_TOTAL_LAST_MAX, 0.8)):
        stream = torch.cuda.current_stream()
        dq.logits_select(x, k, rule=rule, temperature=t, workspace=ws, stream=stream)
        torch.cuda.synchronize()

        def body(st):
            for _ in range(reps):
                dq.logits_select(x, k, rule=rule, temperature=t, workspace=ws, stream=st)
        g = capture(torch, body)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        e1.synchronize()
        out[name] = round(e0.elapsed_time(e1) * 1e3 / reps, 2)
    return out


def _cpu_host():
    """What the CPU baseline ran on: model string, core counts, thread setting."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    threads = affinity
    if env and env.isdigit() and int(env) > 0:
        threads = min(threads, int(env))
    return {"cpu_model": model, "nproc_affinity": affinity, "os_cpu_count": os.cpu_count(),
            "omp_num_threads_env": env, "threads": threads}


def cpu_baseline(seconds):
    """The CPU baseline (oracle/cpu_baseline.c) on this host's cores, over a
    bounded sample of the same workload: the W8A16 decode GEMV of the gate
    linear [17408, 5120] at M = 1 (the headline unit, GB/s of weight bytes),
    `seconds` split between the portable build and one compiled here with
    -march=native (the faster is reported), then the Q4_K GEMV of the same
    shape and the W8A16 prefill GEMM at M = 256 (blocked f32, on-the-fly
    dequant), native build, for about a third of that each."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # the checker library; timed here as the CPU baseline
    host = _cpu_host()
    threads = host["threads"]
    n, k = 17408, 5120
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (n, k), dtype=np.int8)
    s = np.full(n, 0x3c00, np.uint16)
    x = (rng.normal(size=(1, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)

    def timed(fn, budget):
        fn()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget or reps == 0:
            fn()
            reps += 1
        return (time.perf_counter() - t0) / reps, reps

    # both builds of the GEMV, the portable one (x86-64-v3, liboracle.so) and
    # the -march=native one; the faster is the baseline
    builds = {}
    for native in (False, True):
        dt_, reps_ = timed(lambda: O.cpu_w8a16_gemv(x, q, s, threads, native=native), seconds / 2)
        builds["native" if native else "portable"] = ((n * k + 2 * n) / dt_ / 1e9, reps_)
    best = max(builds, key=lambda b: builds[b][0])
    gbs, reps = builds[best]
    # random Q4_K super-blocks (the GEMV's cost does not depend on the
    # values): random codes and 6-bit scales, f16 d = dmin = 2^-10
    blocks = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    blocks[:, :, 0:4] = np.array([0x00, 0x14, 0x00, 0x14], np.uint8)
    blocks = blocks.reshape(n, k // 256 * 144)
    dq4, reps4 = timed(lambda: O.cpu_q4_k_gemv(x, blocks, n, threads, native=True), seconds / 3)
    xm = (rng.normal(size=(256, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    dgm, repsm = timed(lambda: O.cpu_w8a16_gemm(xm, q, s, threads, native=True), seconds / 3)
    why = (f"{threads} threads: this host's CPU affinity ({host['nproc_affinity']} CPUs)"
           + (f" capped by OMP_NUM_THREADS={host['omp_num_threads_env']}" if host["omp_num_threads_env"] else ""))
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"W8A16 decode GEMV [17408x5120] M=1 (the layer's gate linear), {reps} reps, "
                      f"{threads} OpenMP threads, dequantize-on-the-fly f32 dot per row (rows in chunks of 64)",
            "build": {"portable": "gcc -O3 -march=x86-64-v3 -fopenmp (oracle/lib/liboracle.so)",
                      "native": "gcc -O3 -march=native -fopenmp, compiled on this host (oracle/Makefile: native)",
                      "reported": best},
            "threads_reason": why, **{k_: v for k_, v in host.items() if k_ != "threads"},
            "legs": {
                "w8a16_gemv_gate_m1_gbs": round(gbs, 2),
                "w8a16_gemv_gate_m1_gbs_by_build": {b: round(v[0], 2) for b, v in builds.items()},
                "q4_k_gemv_gate_m1_gbs": round(n * (k // 256) * 144 / dq4 / 1e9, 2),
                "q4_k_gemv_reps": reps4,
                "w8a16_gemm_gate_m256_tflops": round(2.0 * 256 * n * k / dgm / 1e12, 3),
                "w8a16_gemm_reps": repsm,
            }}


# (key, rows, path, peak, activation dtype).  q4_k_f16act: Q4_K with the f16
# activations of DIAL's GGUF worker, whose prefill multiplies f16-dequantized
# weights (qwen3_vl/worker_gguf.rs:426-455).  q6_k: the second block type of a
# Q4_K_M file (worker_gguf.rs:536-540).
PREFILL_GATE = [("w8a16", 2048, "PATH_GEMM", "bf16", "bfloat16"), ("q4_k", 2048, "PATH_GEMM", "bf16", "bfloat16"),
                ("q4_k_f16act", 2048, "PATH_GEMM", "f16", "float16"), ("q8_0", 2048, "PATH_GEMM", "f16", "bfloat16"),
                ("q6_k", 2048, "PATH_GEMM", "f16", "bfloat16"),
                ("fp8_block", 1024, "PATH_GEMM_NATIVE", "fp8", "bfloat16"),
                ("mxfp4", 1024, "PATH_GEMM_NATIVE", "fp4", "bfloat16")]


def q6_k_synthetic_blocks(n, k, seed=23):
    """Synthetic Q6_K weight bytes (Q6_K arrives only from GGUF files and has
    no quantizer here): uniform 6-bit codes and i8 sub-block scales, the f16
    super-block scale d in [1e-4, 3e-4)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    nb = n * (k // 256)
    b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    b[:, 208:210] = (1e-4 * rng.uniform(1.0, 3.0, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(n, (k // 256) * 210)


def prefill_gate_linears(dq, torch, dev, name):
    _, n, k = DOM
    if name == "q6_k":
        return dq.Linear.create(dq.Q6_K, n, k, q6_k_synthetic_blocks(n, k))
    fmt = {"w8a16": dq.W8A16, "q4_k": dq.Q4_K, "q4_k_f16act": dq.Q4_K, "q8_0": dq.Q8_0, "fp8_block": dq.FP8_BLOCK,
           "mxfp4": dq.MXFP4}[name]
    g = torch.Generator(device=dev).manual_seed(23)
    return dq.Linear.quantize(fmt, torch.randn(n, k, device=dev, generator=g) * 0.02, scale_dtype=dq.BF16)


def profile_prefill_gate_run(dq, torch, dev, launches=5):
    """Eager launches of the gate-shape prefill per format (the programs of
    the committed MFMA counter summaries)."""
    _, n, k = DOM
    for name, m, path, _, act in PREFILL_GATE:
        lin = prefill_gate_linears(dq, torch, dev, name)
        x = torch.randn(m, k, device=dev).to(getattr(torch, act))
        y = torch.empty(m, n, device=dev, dtype=getattr(torch, act))
        for _ in range(launches):
            lin.forward(x, y, path=getattr(dq, path))
        torch.cuda.synchronize()
        print(f"# profile: {launches} launches of {name} prefill [{n}x{k}] M={m}", flush=True)
        del lin
        torch.cuda.empty_cache()


def read_mfma_counters():
    """Per-format MFMA busy fraction and LDS bank-conflict cycles of the gate
    prefill GEMM from the committed counter summary
    (profiles/prefill_gate_17408x5120_mfma_counters.md), if present."""
    path = os.path.join(ROOT, "profiles", "prefill_gate_17408x5120_mfma_counters.md")
    out = {}
    try:
        for line in open(path):
            if line.startswith("counters:"):
                _, name, rest = line.split(None, 2)
                out[name] = {kv.split("=")[0]: float(kv.split("=")[1]) for kv in rest.split()}
    except (OSError, ValueError, IndexError):
        return {}
    return out


def time_prefill_gate(dq, torch, dev, reps=10):
    """The prefill roofline per format: the gate linear 17408x5120 (the
    layer's largest; gate / up / down tie on flops), `reps` forwards in a
    captured graph between HIP events on the replay stream.  For the native
    paths a forward is the activation quantizer plus the GEMM, so the rate
    is a lower bound for the GEMM kernel."""
    _, n, k = DOM
    counters = read_mfma_counters()
    out = {}
    for name, m, path, peak_key, act in PREFILL_GATE:
        lin = prefill_gate_linears(dq, torch, dev, name)
        x = torch.randn(m, k, device=dev).to(getattr(torch, act))
        y = torch.empty(m, n, device=dev, dtype=getattr(torch, act))
        stream = torch.cuda.current_stream()
        lin.forward(x, y, path=getattr(dq, path), stream=stream)
        torch.cuda.synchronize()

        def body(st):
            for _ in range(reps):
                lin.forward(x, y, path=getattr(dq, path), stream=st)
        g = capture(torch, body)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        e1.synchronize()
        secs = e0.elapsed_time(e1) * 1e-3 / reps
        tf = 2.0 * m * n * k / secs / 1e12
        peak = MFMA_PEAK_TFLOPS[peak_key]
        out[name] = {"bound": "mfma", "m": m, "achieved": round(tf, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tf / peak, 4), "us_per_forward": round(secs * 1e6, 2),
                     "flops_per_launch": 2 * m * n * k, **counters.get(name, {})}
        del lin, g
        torch.cuda.empty_cache()
    return out


def time_dense_library(torch, dev, reps=20):
    """The vendor library's dense GEMMs on the gate shape, on this GPU in
    this run (torch.matmul / torch._scaled_mm -> hipBLASLt): bf16 and f16
    at M = 2048 and per-tensor-scaled fp8 e4m3 at M = 1024 -- the dense
    products the quantized kernels' MFMA fractions can be read against."""
    _, n, k = DOM
    out = {}

    def rate(m, fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.synchronize()
        secs = e0.elapsed_time(e1) * 1e-3 / reps
        return round(2.0 * m * n * k / secs / 1e12, 1)

    for dt in ("bfloat16", "float16"):
        a_ = torch.randn(2048, k, device=dev).to(getattr(torch, dt))
        b_ = torch.randn(n, k, device=dev).to(getattr(torch, dt))
        out[("bf16" if dt == "bfloat16" else "f16") + "_m2048"] = rate(2048, lambda: torch.matmul(a_, b_.t()))
        del a_, b_
    try:
        a_ = torch.randn(1024, k, device=dev).to(torch.float8_e4m3fn)
        b_ = torch.randn(n, k, device=dev).to(torch.float8_e4m3fn)
        one = torch.tensor(1.0, device=dev)
        out["fp8_e4m3_m1024"] = rate(1024, lambda: torch._scaled_mm(a_, b_.t(), scale_a=one, scale_b=one,
                                                                    out_dtype=torch.bfloat16))
        del a_, b_
    except Exception as ex:  # a torch build without the fp8 GEMM
        out["fp8_e4m3_m1024"] = None
        out["fp8_error"] = str(ex)[:120]
    torch.cuda.empty_cache()
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {a.gpus} is not supported (the library "
              "has no multi-GPU path)", file=sys.stderr)
        sys.exit(2)
    import torch
    import dialq as dq

    dev = torch.device("cuda:0")
    if a.profile:
        profile_run(dq, torch, dev, a.profile_launches, a.profile_format)
        return
    if a.profile_layer:
        profile_layer_run(dq, torch, dev)
        return
    if a.profile_lm_head:
        profile_lm_head_run(dq, torch, dev)
        return
    if a.profile_prefill:
        profile_prefill_run(dq, torch, dev)
        return
    if a.profile_swiglu:
        profile_swiglu_run(dq, torch, dev)
        return
    if a.profile_select:
        profile_select_run(dq, torch, dev)
        return
    if a.profile_prefill_gate:
        profile_prefill_gate_run(dq, torch, dev)
        return
    fmt_of = {"w8a16": dq.W8A16, "q4_k": dq.Q4_K, "q8_0": dq.Q8_0, "fp8_block": dq.FP8_BLOCK, "mxfp4": dq.MXFP4}

    # ---- headline: W8A16 decode over the 27B layer -----------------------
    layers = build_layers(dq, torch, dq.W8A16, a.copies, dev)
    secs = time_decode(dq, torch, layers, a.steps, a.warmup, dev, settle=a.settle_seconds, groups=LAYER_27B_GROUPS)
    lbytes = layer_bytes(dq, dq.W8A16)
    value = lbytes * a.steps / secs / 1e9
    per_group = time_per_group(dq, torch, layers, dev)
    # the same seven linears as seven separate forwards (no grouping)
    usteps = max(a.steps // 3, 10)
    su = time_decode(dq, torch, layers, usteps, 10, dev, settle=a.settle_seconds / 4)
    value_ungrouped = lbytes * usteps / su / 1e9
    per = time_per_linear(dq, torch, layers, dev)
    # the same decode with f16 activations (the GGUF worker's runtime dtype)
    fsteps16 = max(a.steps // 3, 10)
    s16 = time_decode(dq, torch, layers, fsteps16, 10, dev, xdtype=torch.float16, groups=LAYER_27B_GROUPS)
    value_f16 = layer_bytes(dq, dq.W8A16) * fsteps16 / s16 / 1e9
    # the 27B sweep's other decode row count (8 tokens per pass)
    s8 = time_decode(dq, torch, layers, fsteps16, 10, dev, groups=LAYER_27B_GROUPS, rows=8)
    value_m8 = layer_bytes(dq, dq.W8A16) * fsteps16 / s8 / 1e9
    del layers
    torch.cuda.empty_cache()
    # dominant kernel: the grouped gate / up launch (the largest of the four),
    # timed over DOM_GROUP_COPIES rotating copies so no launch finds its
    # weights in the cache
    dom, dns, dk = DOM_GROUP
    gd = torch.Generator(device=dev).manual_seed(11)
    dgroups = [[dq.Linear.quantize(dq.W8A16, torch.randn(n, dk, device=dev, generator=gd) * 0.02,
                                   scale_dtype=dq.BF16) for n in dns] for _ in range(DOM_GROUP_COPIES)]
    dom_secs = time_group_launches(dq, torch, dgroups, dk, sum(dns), dev)
    del dgroups
    torch.cuda.empty_cache()
    # algorithmic bytes per launch: int8 codes + bf16 row scales of both
    # members + x + y
    dbytes = sum(dq.raw_weight_bytes(dq.W8A16, n, dk) for n in dns) + 2 * dk + 2 * sum(dns)
    achieved = dbytes / dom_secs / 1e9
    traffic = read_traffic()
    print(f"# w8a16 decode: {value:.1f} GB/s over the layer (4 launches: q/k/v and gate/up grouped); per-launch us: "
          + ", ".join(f"{k}={v * 1e6:.1f}" for k, v in per_group.items()), file=sys.stderr, flush=True)
    print(f"# w8a16 decode, seven separate forwards: {value_ungrouped:.1f} GB/s; per-launch us: "
          + ", ".join(f"{k}={v * 1e6:.1f}" for k, v in per.items()), file=sys.stderr, flush=True)
    print(f"# w8a16 decode with f16 activations: {value_f16:.1f} GB/s", file=sys.stderr, flush=True)
    layers = build_layers(dq, torch, dq.W8A16, 1, dev)
    extra = {"decode_gbs": {"w8a16": round(value, 1)}, "decode_gbs_f16_activations": {"w8a16": round(value_f16, 1)},
             "decode_gbs_ungrouped": {"w8a16": round(value_ungrouped, 1)},
             "decode_us_per_launch_w8a16_grouped": {k: round(v * 1e6, 2) for k, v in per_group.items()},
             "decode_us_per_launch_w8a16":
             {k: round(v * 1e6, 2) for k, v in per.items()}, "prefill_tflops": {}, "prefill_pct_mfma_peak": {},
             "sweep_27b": {"w8a16": {"decode_gbs_m1": round(value, 1), "decode_gbs_m8": round(value_m8, 1)}}}
    sweep = [s for s in a.sweep.split(",") if s]
    extra["prefill_tflops_ungrouped"] = {}
    if "w8a16" in sweep:
        tf, s2 = time_prefill(dq, torch, layers[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM,
                              groups=LAYER_27B_GROUPS)
        extra["prefill_tflops"]["w8a16_m2048"] = round(tf, 1)
        extra["prefill_pct_mfma_peak"]["w8a16_m2048"] = round(100.0 * tf / MFMA_PEAK_TFLOPS["bf16"], 1)
        tfu, _ = time_prefill(dq, torch, layers[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM)
        extra["prefill_tflops_ungrouped"]["w8a16_m2048"] = round(tfu, 1)
        t256, _ = time_prefill(dq, torch, layers[0], 256, a.prefill_iters, dev, dq.PATH_GEMM, groups=LAYER_27B_GROUPS)
        extra["sweep_27b"]["w8a16"].update({"prefill_tflops_m256": round(t256, 1), "prefill_tflops_m2048": round(tf, 1)})
        print(f"# w8a16 prefill M=2048: {tf:.1f} TFLOP/s ({s2 * 1e3:.2f} ms/layer; {tfu:.1f} as seven forwards)",
              file=sys.stderr, flush=True)
    del layers
    torch.cuda.empty_cache()
    # the same layer with fused qkv / gate_up projections (four linears)
    fl = build_layers(dq, torch, dq.W8A16, a.copies, dev, seed=3, shapes=LAYER_27B_FUSED)
    fsteps = max(a.steps // 3, 10)
    fs = time_decode(dq, torch, fl, fsteps, 10, dev, shapes=LAYER_27B_FUSED)
    extra["decode_gbs_fused_qkv_gate_up"] = {"w8a16": round(layer_bytes(dq, dq.W8A16, LAYER_27B_FUSED) * fsteps / fs / 1e9, 1)}
    # ... and with gate_up's SwiGLU epilogue, which writes silu(gate) * up
    # (the down projection's input) instead of the [M, 34816] gate_up output
    fs2 = time_decode(dq, torch, fl, fsteps, 10, dev, shapes=LAYER_27B_FUSED, swiglu=("gate_up",))
    extra["decode_gbs_fused_swiglu"] = {"w8a16": round(layer_bytes(dq, dq.W8A16, LAYER_27B_FUSED) * fsteps / fs2 / 1e9, 1)}
    print(f"# w8a16 decode, fused qkv / gate_up: {extra['decode_gbs_fused_qkv_gate_up']['w8a16']} GB/s; "
          f"with the SwiGLU epilogue: {extra['decode_gbs_fused_swiglu']['w8a16']} GB/s", file=sys.stderr, flush=True)
    if "w8a16" in sweep:
        tf, s2 = time_prefill(dq, torch, fl[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM, shapes=LAYER_27B_FUSED)
        extra.setdefault("prefill_tflops_fused_qkv_gate_up", {})["w8a16_m2048"] = round(tf, 1)
        tf2, _ = time_prefill(dq, torch, fl[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM, shapes=LAYER_27B_FUSED,
                              swiglu=("gate_up",))
        extra.setdefault("prefill_tflops_fused_swiglu", {})["w8a16_m2048"] = round(tf2, 1)
    del fl
    torch.cuda.empty_cache()
    # quantized lm_head GEMV (vocab 248320 x hidden 5120): one copy is 1.27 GB
    # (W8A16) / 0.68 GB (MXFP4), far past the 256 MB last-level cache
    if not a.no_lm_head:
        vn, vk = LM_HEAD_27B
        extra["decode_lm_head"] = {}
        for name, fmt in (("w8a16", dq.W8A16), ("mxfp4", dq.MXFP4)):
            gl = torch.Generator(device=dev).manual_seed(21)
            lin = dq.Linear.quantize(fmt, torch.randn(vn, vk, device=dev, generator=gl) * 0.02, scale_dtype=dq.BF16)
            torch.cuda.empty_cache()
            ls_ = time_launches(dq, torch, [lin], vk, vn, dev, reps=20)
            gbs = dq.raw_weight_bytes(fmt, vn, vk) / ls_ / 1e9
            extra["decode_lm_head"][name] = {"us": round(ls_ * 1e6, 1), "gbs": round(gbs, 1),
                                             "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 1)}
            print(f"# lm_head {vn}x{vk} {name} decode: {ls_ * 1e6:.1f} us, {gbs:.1f} GB/s", file=sys.stderr, flush=True)
            del lin
            torch.cuda.empty_cache()
        extra["select_after_lm_head_us"] = time_select(dq, torch, vn, dev)
        print(f"# token selection over {vn} bf16 logits (us): {extra['select_after_lm_head_us']}",
              file=sys.stderr, flush=True)
    for name in sweep:
        if name == "w8a16":
            continue
        fmt = fmt_of[name]
        ls = build_layers(dq, torch, fmt, a.copies if fmt != dq.MXFP4 and fmt != dq.Q4_K else a.copies + 2, dev)
        sd = time_decode(dq, torch, ls, max(a.steps // 3, 10), 10, dev, groups=LAYER_27B_GROUPS)
        gbs = layer_bytes(dq, fmt) * max(a.steps // 3, 10) / sd / 1e9
        extra["decode_gbs"][name] = round(gbs, 1)
        if fmt in (dq.FP8_BLOCK, dq.MXFP4):
            tf, s2 = time_prefill(dq, torch, ls[0], 1024, a.prefill_iters, dev, dq.PATH_GEMM_NATIVE,
                                  groups=LAYER_27B_GROUPS)
            extra["prefill_tflops"][name + "_native_m1024"] = round(tf, 1)
            peak = MFMA_PEAK_TFLOPS["fp8" if fmt == dq.FP8_BLOCK else "fp4"]
            extra["prefill_pct_mfma_peak"][name + "_native_m1024"] = round(100.0 * tf / peak, 1)
            tfu, _ = time_prefill(dq, torch, ls[0], 1024, a.prefill_iters, dev, dq.PATH_GEMM_NATIVE)
            extra["prefill_tflops_ungrouped"][name + "_native_m1024"] = round(tfu, 1)
            # the fused projections DIAL's layers call (qkv, o, gate_up, down)
            del ls
            torch.cuda.empty_cache()
            ls = build_layers(dq, torch, fmt, 1, dev, seed=5, shapes=LAYER_27B_FUSED)
            tff, _ = time_prefill(dq, torch, ls[0], 1024, a.prefill_iters, dev, dq.PATH_GEMM_NATIVE,
                                  shapes=LAYER_27B_FUSED)
            extra.setdefault("prefill_tflops_fused_qkv_gate_up", {})[name + "_native_m1024"] = round(tff, 1)
            tff2, _ = time_prefill(dq, torch, ls[0], 1024, a.prefill_iters, dev, dq.PATH_GEMM_NATIVE,
                                   shapes=LAYER_27B_FUSED, swiglu=("gate_up",))
            extra.setdefault("prefill_tflops_fused_swiglu", {})[name + "_native_m1024"] = round(tff2, 1)
        else:
            tf, s2 = time_prefill(dq, torch, ls[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM, groups=LAYER_27B_GROUPS)
            extra["prefill_tflops"][name + "_m2048"] = round(tf, 1)
            extra["prefill_pct_mfma_peak"][name + "_m2048"] = round(100.0 * tf / MFMA_PEAK_TFLOPS["bf16"], 1)
            tfu, _ = time_prefill(dq, torch, ls[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM)
            extra["prefill_tflops_ungrouped"][name + "_m2048"] = round(tfu, 1)
            if fmt == dq.Q4_K:  # the 27B sweep's other row counts: decode 8, prefill 256
                s8q = time_decode(dq, torch, ls, max(a.steps // 3, 10), 10, dev, groups=LAYER_27B_GROUPS, rows=8)
                t256q, _ = time_prefill(dq, torch, ls[0], 256, a.prefill_iters, dev, dq.PATH_GEMM,
                                        groups=LAYER_27B_GROUPS)
                extra["sweep_27b"]["q4_k"] = {"decode_gbs_m1": round(gbs, 1),
                                              "decode_gbs_m8": round(layer_bytes(dq, fmt) * max(a.steps // 3, 10)
                                                                     / s8q / 1e9, 1),
                                              "prefill_tflops_m256": round(t256q, 1),
                                              "prefill_tflops_m2048": round(tf, 1)}
            if fmt == dq.Q4_K:  # the GGUF worker's f16 activations
                tfh, _ = time_prefill(dq, torch, ls[0], 2048, a.prefill_iters, dev, dq.PATH_GEMM, act="float16",
                                      groups=LAYER_27B_GROUPS)
                extra["prefill_tflops"][name + "_f16act_m2048"] = round(tfh, 1)
                extra["prefill_pct_mfma_peak"][name + "_f16act_m2048"] = round(100.0 * tfh / MFMA_PEAK_TFLOPS["f16"], 1)
        print(f"# {name}: decode {gbs:.1f} GB/s, prefill {tf:.1f} TFLOP/s", file=sys.stderr, flush=True)
        del ls
        torch.cuda.empty_cache()

    roof_prefill = time_prefill_gate(dq, torch, dev) if sweep else None
    dense_lib = time_dense_library(torch, dev) if sweep else None
    if dense_lib:
        print("# dense library GEMMs (gate 17408x5120): " + ", ".join(f"{k_} {v}" for k_, v in dense_lib.items()),
              file=sys.stderr, flush=True)
    if roof_prefill:
        print("# prefill roofline (gate 17408x5120): " + ", ".join(
            f"{k_} {v['achieved']} TFLOP/s ({100 * v['frac']:.1f} %)" for k_, v in roof_prefill.items()),
            file=sys.stderr, flush=True)
    cpu = None if a.no_cpu else cpu_baseline(a.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(secs / a.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "27B-class dense layer linears (hidden 5120; q 6144x5120, k/v 1024x5120, "
                        "o 5120x6144, gate/up 17408x5120, down 5120x17408), W8A16 decode GEMV, M=1; "
                        "q/k/v and gate/up as grouped forwards (4 launches)",
            "weights_per_layer": sum(n * k for _, n, k in LAYER_27B),
            "weight_bytes_per_step": lbytes,
            "layer_copies_rotated": a.copies,
            "settle_s": a.settle_seconds,
            "rows": 1,
            "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 1),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"k_gemv W8A16 bf16, grouped {dom} (2 x {dns[0]}x{dk}, M=1)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (round(traffic["traffic_bytes_per_launch"]) if traffic else None),
            "algorithmic_bytes": dbytes,
            "us_per_launch": round(dom_secs * 1e6, 2),
        },
        "roofline_prefill": roof_prefill,
        "dense_library_tflops_gate": dense_lib,
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
