#!/usr/bin/env python3
"""Benchmark of the compressed-KV hot path on one MI355X.

Metric: "KV quant GB/s (4-bit, 262K ctx) + CSA sparse-decode tokens/s, 1 GPU".

`value` is the TurboQuant 4-bit encode throughput on benchmark configuration cfg2 — one full decode KV layer,
262144 tokens x 1536 (12 heads x 128) bf16, N(0,1) with 2% outlier channels x8, seed 1 — in GB/s of
algorithmic bytes (805,306,368 read + 201,326,592 codes + 12,582,912 scales = 1,019,215,872 B per
step), inputs resident in HBM.  One step = one encode of the whole layer (one kernel launch).
The same line carries, under "secondary", cfg2 decode GB/s, CSA sparse decode tokens/s (cfg5 and
cfg3), HCA decode tokens/s (cfg4), chunked-prefill targets/s through the quantised reader (a chunk of
256 targets per sequence over cfg3's and cfg4's caches) and the reference microbenchmark shape of
sparse_sink_attention.

Timing: a settle period (60 ms of continuous launches of the timed call: the box runs a slower
phase during the first ~20 ms of sustained load), W untimed warmup steps, then K steps bracketed
by torch.cuda.synchronize() and HIP events recorded on the stream the kernels run on (torch's
current stream).  The encode is also timed without the settle period (secondary
tq_encode_cfg2_from_idle).  Decode steps (indexer +
attention) are captured 8 at a time in a HIP graph and replayed, as a serving loop would run them;
the eager (per-call Python) step time is reported beside it.

cpu_baseline: the reference's own encode op sequence in torch eager ops (oracle/torch_ref.py) on
this host's cores over a quarter of the cfg2 layer, with the C oracle's encode of the whole layer
beside it (c_port).  The CSA lines carry their own cpu_baseline: the oracle's decode step
(dequantise every step or memoised, scores, exact top-256, attention) and the reference's torch op
sequence of the step, on the first 8 rows of the config.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "deepseek-v4-codebase_amd"))

import torch  # noqa: E402

METRIC = "KV quant GB/s (4-bit, 262K ctx) + CSA sparse-decode tokens/s, 1 GPU"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

# cfg2 algorithmic bytes per encode (and per decode)
T2, H2, D2 = 262144, 12, 128
N_VEC2 = T2 * H2
ENC_BYTES = N_VEC2 * (D2 * 2 + D2 // 2 + 4)   # 1,019,215,872


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


SETTLE_S = 0.06  # seconds of continuous launches before each timed section


def settle(fn, seconds: float = SETTLE_S) -> None:
    """Keeps the GPU busy with fn for `seconds` of wall time.  Under sustained load the box goes
    through a slower phase that starts a few ms in and ends about 20 ms in: measured on the cfg2
    encode, launches 1-100 after an idle period average 195 us and every later one 171 us (the
    early ones ~164 us, then ~215 us, then steady).  A timed section that starts from idle would
    measure that transition rather than the kernel, so each one is preceded by this."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()  # bounded queue; the GPU idles only for the host's turnaround


def timed(fn, steps: int, warmup: int, settle_first: bool = True):
    """Average ms per call with HIP events on the current stream (bracketed by synchronize), after
    settle() unless settle_first is False."""
    if settle_first:
        settle(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


GRAPH_STEPS = 8  # decode steps captured per HIP graph


def timed_graph(fn, steps: int, warmup: int, inner: int = GRAPH_STEPS):
    """Average ms per fn call when `inner` consecutive calls are captured in one HIP graph and the
    graph is replayed, the way a serving loop replays its decode step (every replay runs every
    kernel of every call); same events and synchronisation as timed()."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(inner):
            fn()
    ms = timed(g.replay, steps, warmup) / inner
    del g
    return ms


# Infinity Cache (MALL) of MI355X: a step's caches that fit in it stay there across replays of the
# same inputs.  The cold timing rotates enough distinct layer caches that more than twice this much
# is touched between two visits of one layer.
MALL_BYTES = 256 << 20


def timed_graph_layers(fns, steps: int, warmup: int):
    """Average ms per call when the calls fns[0], fns[1], ... (one per layer, each on its own
    caches) are captured in that order in one HIP graph and the graph is replayed: the engine's
    token step visits every layer once (aether_2b/serving.py:709-721), so a layer's caches are cold
    again by its next visit whenever the layers' working sets together exceed the caches."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for fn in fns[:3]:
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fns:
            fn()
    ms = timed(g.replay, max(1, steps // 4), max(1, warmup // 4)) / len(fns)
    del g
    return ms


def cpu_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def bench_encode(args, dev, out):
    from aetherkv import PolarQuant
    from aetherkv.synthetic import normal_with_outliers

    log("cfg2: generating 262144x12x128 bf16 (seed 1, 2% outliers x8)")
    x = normal_with_outliers((T2, H2, D2), 1, device=dev)
    pq = PolarQuant(4)
    codes = torch.empty((T2, H2, D2 // 2), dtype=torch.uint8, device=dev)
    scale = torch.empty((T2, H2, 1), dtype=torch.float32, device=dev)
    import aetherkv._lib as L

    lib = L.lib()
    diag = pq._diag(D2, dev)
    stream = L.stream_of(x)
    xp, dp, cp, sp = L.ptr(x), L.ptr(diag), L.ptr(codes), L.ptr(scale)

    def enc():
        L.check(lib.aekv_tq_encode(xp, L.BF16, N_VEC2, D2, 4, dp, cp, sp, stream), "encode")

    ms_idle = timed(enc, args.steps, args.warmup, settle_first=False)
    log(f"cfg2 encode from idle (W warmup steps only): {ms_idle * 1e3:.1f} us/step, "
        f"{ENC_BYTES / ms_idle / 1e6:.1f} GB/s")
    ms = timed(enc, args.steps, args.warmup)
    log(f"cfg2 encode: {ms * 1e3:.1f} us/step, {ENC_BYTES / ms / 1e6:.1f} GB/s")
    out["encode_ms"] = ms
    out["encode_ms_from_idle"] = ms_idle
    rec = torch.empty((T2, H2, D2), dtype=torch.bfloat16, device=dev)
    rp = L.ptr(rec)

    def dec():
        L.check(lib.aekv_tq_decode(cp, sp, N_VEC2, D2, 4, dp, rp, L.BF16, stream), "decode")

    ms_d = timed(dec, args.steps, args.warmup)
    log(f"cfg2 decode: {ms_d * 1e3:.1f} us/step, {ENC_BYTES / ms_d / 1e6:.1f} GB/s")
    out["decode_ms"] = ms_d
    # the practical ceiling of the encode's own traffic: the same bytes, access pattern and
    # non-temporal stores, no transform (aekv_stream_probe)
    c2, s2 = torch.empty_like(codes), torch.empty_like(scale)
    c2p, s2p = L.ptr(c2), L.ptr(s2)

    plib = ctypes.CDLL(str(Path(L.__file__).with_name("libaetherkv_probe.so")))
    plib.aekv_stream_probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p]
    plib.aekv_stream_probe.restype = ctypes.c_int

    def probe():
        if plib.aekv_stream_probe(xp, N_VEC2, c2p, s2p, stream) != 0:
            raise RuntimeError("aekv_stream_probe rejected its arguments or failed to launch")

    ms_p = timed(probe, args.steps, args.warmup)
    out["stream_ceiling_gbs"] = ENC_BYTES / ms_p / 1e6
    log(f"streaming ceiling of the encode's traffic: {ms_p * 1e3:.1f} us, {out['stream_ceiling_gbs']:.1f} GB/s "
        f"(encode at {ms_p / ms:.3f} of it)")
    del c2, s2
    # copy-bandwidth reference (torch copy of the same layer)
    y = torch.empty_like(x)
    ms_c = timed(lambda: y.copy_(x), args.steps, args.warmup)
    out["copy_gbs"] = 2 * x.numel() * 2 / ms_c / 1e6
    log(f"torch copy of the layer: {out['copy_gbs']:.1f} GB/s")
    if not args.no_cpu_baseline:
        out["x_host"] = x.view(torch.int16).cpu()
    del y, rec


def bench_codec_shapes(args, dev):
    """The engine's other TurboQuant shapes over the same 805 MB of bf16 input as cfg2 (seed 1, 2%
    outliers): 8-bit D=128 (cfg1/cfg3's KV blocks, turbo_quant.py:150-154), and 4- and 8-bit D=64
    (the CSA index keys, aether_2b/serving.py:567-577), encode and decode, GB/s of algorithmic bytes
    (D*2 in + codes + 4 B scale per vector)."""
    from aetherkv import PolarQuant
    from aetherkv.synthetic import normal_with_outliers
    import aetherkv._lib as L

    lib = L.lib()
    x = normal_with_outliers((T2, H2, D2), 1, device=dev)
    res = {}
    for bits, D in ((8, 128), (4, 64), (8, 64)):
        n_vec = x.numel() // D
        cb = D if bits == 8 else D // 2
        pq = PolarQuant(bits)
        codes = torch.empty((n_vec, cb), dtype=torch.int8 if bits == 8 else torch.uint8, device=dev)
        scale = torch.empty((n_vec,), dtype=torch.float32, device=dev)
        rec = torch.empty((n_vec, D), dtype=torch.bfloat16, device=dev)
        diag = pq._diag(D, dev)
        stream = L.stream_of(x)
        xp, dp, cp, sp, rp = L.ptr(x), L.ptr(diag), L.ptr(codes), L.ptr(scale), L.ptr(rec)
        nbytes = n_vec * (2 * D + cb + 4)
        enc = lambda: L.check(lib.aekv_tq_encode(xp, L.BF16, n_vec, D, bits, dp, cp, sp, stream), "encode")  # noqa
        dec = lambda: L.check(lib.aekv_tq_decode(cp, sp, n_vec, D, bits, dp, rp, L.BF16, stream), "decode")  # noqa
        ms_e = timed(enc, args.steps, args.warmup)
        ms_d = timed(dec, args.steps, args.warmup)
        key = f"{bits}bit_d{D}"
        res[key] = {"vectors": n_vec, "bytes": nbytes,
                    "encode": {"ms": round(ms_e, 5), "GB/s": round(nbytes / ms_e / 1e6, 1),
                               "frac": round(nbytes / ms_e / 1e6 / HBM_PEAK_GBS, 4)},
                    "decode": {"ms": round(ms_d, 5), "GB/s": round(nbytes / ms_d / 1e6, 1),
                               "frac": round(nbytes / ms_d / 1e6 / HBM_PEAK_GBS, 4)}}
        log(f"codec {key}: encode {ms_e * 1e3:.1f} us ({res[key]['encode']['GB/s']:.0f} GB/s), decode "
            f"{ms_d * 1e3:.1f} us ({res[key]['decode']['GB/s']:.0f} GB/s)")
        del codes, scale, rec
    del x
    torch.cuda.empty_cache()
    return res


CPU_RUNS = 5  # CPU baseline: median of this many timed runs after one warm-up


def median_seconds(fn, runs: int = CPU_RUNS) -> float:
    """Median wall time of `runs` calls of fn (the caller has run it once as a warm-up)."""
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return sorted(times)[len(times) // 2]


def bench_cpu_encode(out):
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    xb = out.pop("x_host").numpy().view(np.uint16)
    dg = O.diag(42, D2)
    cores = cpu_cores()
    O.encode(xb, "bf16", 4, dg, threads=cores)
    med = median_seconds(lambda: O.encode(xb, "bf16", 4, dg, threads=cores))
    log(f"cpu oracle encode (cfg2, {cores} threads): {med:.3f} s, {ENC_BYTES / med / 1e9:.2f} GB/s")
    c_port = {"value": round(ENC_BYTES / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
              "sample": f"full cfg2 layer (3,145,728 vectors), median of {CPU_RUNS} passes after one warm-up of the C oracle encode "
                        "(oracle/aekv_oracle.c, OpenMP over vectors)"}
    # the reference's own op sequence (turbo_quant.py:127-166 in torch eager ops), all host cores, on a
    # quarter of the layer: 65536 tokens x 12 heads
    import torch_ref as T

    torch.set_num_threads(cores)
    n_tok = T2 // 4
    xs = torch.from_numpy(xb.reshape(T2, H2, D2)[:n_tok].copy()).view(torch.bfloat16)
    dgt = torch.from_numpy(dg)
    T.encode(xs, 4, dgt)
    med_t = median_seconds(lambda: T.encode(xs, 4, dgt))
    bytes_t = ENC_BYTES // 4
    log(f"cpu torch op sequence encode ({n_tok} tokens, {cores} threads): {med_t:.3f} s, "
        f"{bytes_t / med_t / 1e9:.2f} GB/s")
    return {"value": round(bytes_t / med_t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"the reference's encode op sequence (turbo_quant.py:127-166: torch.cat butterflies, amax, "
                      f"divide, multiply, round, clamp, nibble pack; oracle/torch_ref.py) on torch CPU with "
                      f"{cores} threads, over {n_tok} tokens x 12 heads (a quarter of the cfg2 layer), median of "
                      f"{CPU_RUNS} after one warm-up",
            "c_port": c_port}


def bench_cpu_csa(inp, rows, name, bits):
    """The CPU oracle's restatement of the reference decode step (aether_2b/serving.py:597-625) on the
    first `rows` rows of a CSA config, timed on this host: dequantise the index and KV caches (every
    step, as _read_compressed does, or memoised as its cache does), score all blocks (softplus
    rule), exact top-256, gather + window + sink attention.  Median of CPU_RUNS after one warm-up."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    cores = cpu_cores()
    h = {k: v[:rows].cpu() for k, v in inp.items() if isinstance(v, torch.Tensor) and k != "sink"}
    sink = inp["sink"].cpu().numpy()
    f32 = lambda t: t.float().numpy()
    ixc, ixs = h["ix_codes"].numpy(), h["ix_scale"].numpy()
    kvc, kvs = h["kv_codes"].numpy(), h["kv_scale"].numpy()
    q, iq, iw, win = f32(h["q"])[:, 0], f32(h["index_q"]), f32(h["index_w"]), f32(h["win"])
    d64, d128 = O.diag(42, 64), O.diag(42, 128)

    def step(dequant: bool):
        if dequant:
            O.decode(ixc.reshape(-1, ixc.shape[-1]), ixs.reshape(-1), bits, d64, "f32", threads=cores)
            O.decode(kvc.reshape(-1, kvc.shape[-1]), kvs.reshape(-1), bits, d128, "bf16", threads=cores)
        keys = keys_memo
        sc = O.index_scores(iq, iw, keys, threads=cores)
        idx, _ = O.topk(sc, 256)
        O.quant_attention(q, kvc, kvs, idx, win, sink, d128, bits, 128 ** -0.5, threads=cores)

    keys_memo = O.decode(ixc.reshape(-1, ixc.shape[-1]), ixs.reshape(-1), bits, d64, "f32",
                         threads=cores).reshape(rows, ixc.shape[1], 64)
    res = {"rows": rows, "cores": cores, "kind": "port"}
    for label, dq in (("dequant_every_step", True), ("memoised_dequant", False)):
        step(dq)
        med = median_seconds(lambda: step(dq))
        res[label] = {"s_per_step": round(med, 5), "tokens_per_s": round(rows / med, 2)}
    log(f"cpu oracle {name} ({rows} rows, {cores} threads): {res['dequant_every_step']['tokens_per_s']:.1f} tok/s "
        f"dequantising every step, {res['memoised_dequant']['tokens_per_s']:.1f} tok/s memoised")
    res["sample"] = (f"first {rows} rows of {name}: dequant (index f32 + KV bf16), scores, exact top-256, gather + "
                     f"window + sink attention, C oracle with OpenMP; median of {CPU_RUNS} after one warm-up")
    res["torch_op_sequence"] = bench_torch_csa(inp, rows, name, bits)
    return res


def bench_torch_csa(inp, rows, name, bits):
    """The reference decode step's own torch op sequence (oracle/torch_ref.py: serving.py:597-625 with
    the PyTorch attention backend, bf16 attention as the engine runs it) on the first `rows` rows,
    torch on all host cores; dequantising every step and memoised.  Median of CPU_RUNS after one warm-up."""
    import torch_ref as T

    cores = cpu_cores()
    torch.set_num_threads(cores)
    h = {k: v[:rows].cpu() for k, v in inp.items() if isinstance(v, torch.Tensor) and k != "sink"}
    h["sink"] = inp["sink"].cpu()
    d64 = torch.from_numpy(__import__("oracle").diag(42, 64))
    d128 = torch.from_numpy(__import__("oracle").diag(42, 128))
    res = {"rows": rows, "cores": cores, "kind": "port", "cpu": cpu_model()}
    for label, memo in (("dequant_every_step", None), ("memoised_dequant", {})):
        def step():
            T.csa_decode_step(h["q"], h["index_q"], h["index_w"], h["ix_codes"], h["ix_scale"], h["kv_codes"],
                              h["kv_scale"], h["win"], h["sink"], bits, d64, d128, 256, memo=memo)
        step()
        med = median_seconds(step)
        res[label] = {"s_per_step": round(med, 5), "tokens_per_s": round(rows / med, 2)}
    log(f"cpu torch op sequence {name} ({rows} rows, {cores} threads): "
        f"{res['dequant_every_step']['tokens_per_s']:.1f} tok/s dequantising every step, "
        f"{res['memoised_dequant']['tokens_per_s']:.1f} tok/s memoised")
    res["sample"] = (f"first {rows} rows of {name}: the reference's torch ops (decode, einsum, relu, softplus weights, "
                     f"topk, gather, cat, PyTorch sink attention in bf16); median of {CPU_RUNS} after one warm-up")
    return res


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def make_csa_inputs(dev, B, S, bits, seed, outliers):
    from aetherkv import PolarQuant
    from aetherkv.synthetic import normal, normal_with_outliers

    H, D, W, IH, IC = 12, 128, 128, 4, 64
    pq = PolarQuant(bits)
    gen = (lambda shape, s: normal_with_outliers(shape, s, device=dev, trailing_dims=1)) if outliers else \
        (lambda shape, s: normal(shape, s, device=dev))
    kv_codes, kv_scale = pq.encode(gen((B, S, D), seed))
    ix_codes, ix_scale = pq.encode(gen((B, S, IC), seed + 1000))
    torch.cuda.empty_cache()
    return dict(
        pq=pq, kv_codes=kv_codes, kv_scale=kv_scale, ix_codes=ix_codes, ix_scale=ix_scale,
        q=normal((B, 1, H, D), seed + 1, device=dev),
        index_q=normal((B, IH, IC), seed + 2, dtype=torch.float32, device=dev),
        index_w=normal((B, IH), seed + 3, dtype=torch.float32, device=dev),
        win=normal((B, W, D), seed + 4, device=dev),
        sink=normal((H,), seed + 5, dtype=torch.float32, device=dev),
    )


def csa_step_bytes(B, S, bits, k=256, H=12, D=128, W=128, IH=4, IC=64):
    """Algorithmic bytes of one CSA decode step: the index scan (codes + scale of every block), the
    k selected KV rows (codes + scale), the bf16 window, q in and out, the index query and weights,
    and the selected indices out."""
    row_bytes = (D if bits == 8 else D // 2) + 4
    ix_bytes = (IC if bits == 8 else IC // 2) + 4
    return B * (S * ix_bytes + k * row_bytes + W * D * 2 + H * D * 2 * 2 + IH * IC * 4 + IH * 4 + k * 8)


def scan_ceiling(args, layers, B, S, bits, dev):
    """The score pass's streaming ceiling, cold like the step (one probe launch per layer's index
    cache in one graph): aekv_scan_probe reads every key's codes and scale in the score kernel's
    groups, and writes 4 bytes per key and per 16-key slot as its order keys and slot maxima, or
    only reads."""
    import aetherkv._lib as L

    plib = ctypes.CDLL(str(Path(L.__file__).with_name("libaetherkv_probe.so")))
    plib.aekv_scan_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    plib.aekv_scan_probe.restype = ctypes.c_int
    keys = torch.empty(B * S, dtype=torch.int32, device=dev)
    smax = torch.empty(B * S // 16, dtype=torch.int32, device=dev)
    row_bytes = 64 if bits == 8 else 32

    def probe(x, kp):
        cp, sp, mp = L.ptr(x["ix_codes"]), L.ptr(x["ix_scale"]), L.ptr(smax)

        def run():
            if plib.aekv_scan_probe(cp, sp, B * S, row_bytes, kp, mp, L.stream_of(smax)) != 0:
                raise RuntimeError("aekv_scan_probe rejected its arguments or failed to launch")
        return run

    ms_rw = timed_graph_layers([probe(x, L.ptr(keys)) for x in layers], args.steps, args.warmup)
    ms_r = timed_graph_layers([probe(x, None) for x in layers], args.steps, args.warmup)
    ix = B * S * (row_bytes + 4)
    out = {"read_write_ms": round(ms_rw, 5), "read_only_ms": round(ms_r, 5), "bytes_read": ix,
           "bytes_written": B * S * 4 + B * S // 16 * 4,
           "what": "aekv_scan_probe over the same layers' index caches, cold: the score pass's reads (codes + "
                   "scales, 128 keys per wave) and writes (4 B per key, 4 B per 16-key slot), no arithmetic; "
                   "read_only: the reads alone"}
    log(f"score pass ceiling: {ms_rw * 1e3:.1f} us with its writes, {ms_r * 1e3:.1f} us reads only "
        f"({ix / ms_r / 1e6:.0f} GB/s)")
    del keys, smax
    return out


def bench_csa(args, dev, B, S, bits, seed, outliers, name, cpu_rows=0):
    from aetherkv.decode import (attention_workspace, csa_decode_step, csa_indexer_topk_quant, decode_workspace,
                                 indexer_workspace, quant_sink_attention)

    log(f"{name}: CSA decode B={B} S={S} {bits}-bit")
    inp = make_csa_inputs(dev, B, S, bits, seed, outliers)
    k = 256
    H, D, W = 12, 128, 128
    ws_i = indexer_workspace(B, S, k, dev)
    ws_a = attention_workspace(B, H, D, k, W, dev)
    ws_s = decode_workspace(B, S, k, H, D, W, dev)
    idx = torch.empty((B, k), dtype=torch.int64, device=dev)
    out = torch.empty((B, H, D), dtype=torch.bfloat16, device=dev)
    pq = inp["pq"]
    step_bytes = csa_step_bytes(B, S, bits)

    def index_only():
        csa_indexer_topk_quant(inp["index_q"], inp["index_w"], inp["ix_codes"], inp["ix_scale"], k, quant=pq,
                               workspace=ws_i, out=idx)

    def attn_only():
        quant_sink_attention(inp["q"], inp["kv_codes"], inp["kv_scale"], idx, inp["win"], inp["sink"], D ** -0.5,
                             quant=pq, workspace=ws_a, out=out)

    def step_separate():
        index_only()
        attn_only()

    def step():
        # the decode step as one call: score kernel, then selection + attention fused per row
        csa_decode_step(inp["q"], inp["index_q"], inp["index_w"], inp["ix_codes"], inp["ix_scale"], inp["kv_codes"],
                        inp["kv_scale"], inp["win"], inp["sink"], D ** -0.5, k, kv_quant=pq, index_quant=pq,
                        workspace=ws_s, out_idx=idx, out=out)

    if args.cold_only:  # (profiling the cold step alone)
        ms_eager = ms_warm = ms_sep = ms_i = ms_a = float("nan")
    else:
        ms_eager = timed(step, args.steps, args.warmup)
        ms_warm = timed_graph(step, args.steps, args.warmup)
        ms_sep = timed_graph(step_separate, args.steps, args.warmup)
        ms_i = timed_graph(index_only, args.steps, args.warmup)
        ms_a = timed_graph(attn_only, args.steps, args.warmup)
    cpu = bench_cpu_csa(inp, cpu_rows, name, bits) if cpu_rows else None

    # cold: L layers' caches (layer 0 = the inputs above, layer l > 0 seeded seed + 10007 l), one step
    # per layer in one graph, sharing one workspace and output as the engine's layer loop would
    n_layers = max(8, -(-2 * MALL_BYTES // step_bytes) + 1)
    layers = [inp] + [make_csa_inputs(dev, B, S, bits, seed + 10007 * l, outliers) for l in range(1, n_layers)]

    def layer_step(li):
        x = layers[li]
        return lambda: csa_decode_step(x["q"], x["index_q"], x["index_w"], x["ix_codes"], x["ix_scale"],
                                       x["kv_codes"], x["kv_scale"], x["win"], x["sink"], D ** -0.5, k,
                                       kv_quant=pq, index_quant=pq, workspace=ws_s, out_idx=idx, out=out)

    ms = timed_graph_layers([layer_step(li) for li in range(n_layers)], args.steps, args.warmup)
    scan = scan_ceiling(args, layers, B, S, bits, dev)
    res = {"B": B, "S": S, "bits": bits, "ms_per_step": round(ms, 5), "tokens_per_s": round(B / ms * 1e3, 1),
           "hbm_frac": round(step_bytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes_per_step": step_bytes,
           "timing": f"cold: {n_layers} layers' distinct caches ({n_layers * step_bytes / 2 ** 20:.0f} MiB touched "
                     f"per pass, > 2x the 256 MiB Infinity Cache), one step per layer captured in one HIP graph "
                     f"and replayed",
           "warm": {"ms_per_step": round(ms_warm, 5), "tokens_per_s": round(B / ms_warm * 1e3, 1),
                    "hbm_frac": round(step_bytes / ms_warm / 1e6 / HBM_PEAK_GBS, 4),
                    "timing": f"one layer's inputs, HIP graph of {GRAPH_STEPS} steps replayed (caches stay warm)"},
           "ms_per_step_eager_warm": round(ms_eager, 5),
           "step": "aekv_csa_decode_quant: score kernel + fused select/attention kernel",
           "ms_per_step_separate_kernels_warm": round(ms_sep, 5),
           "separate_indexer_ms_warm": round(ms_i, 5), "separate_attention_ms_warm": round(ms_a, 5)}
    log(f"{name}: cold {ms * 1e3:.1f} us/step ({n_layers} layers) -> {res['tokens_per_s']:.0f} tok/s, "
        f"{res['hbm_frac'] * 100:.1f}% of HBM peak; warm {ms_warm * 1e3:.1f} (eager {ms_eager * 1e3:.1f}); separate "
        f"kernels warm {ms_sep * 1e3:.1f} ({ms_i * 1e3:.1f} indexer + {ms_a * 1e3:.1f} attention)")
    res["score_pass_ceiling"] = scan
    if cpu:
        res["cpu_baseline"] = cpu
    del inp, layers
    torch.cuda.empty_cache()
    return res


def bench_hca(args, dev):
    from aetherkv import PolarQuant
    from aetherkv.decode import attention_workspace, quant_sink_attention
    from aetherkv.synthetic import normal, rope_interleaved

    B, H, D, S, W = 32, 12, 128, 2048, 128
    log(f"cfg4: HCA decode B={B} S={S} 4-bit")
    pq = PolarQuant(4)
    ws = attention_workspace(B, H, D, S, W, dev)
    out = torch.empty((B, H, D), dtype=torch.bfloat16, device=dev)
    flops = 2 * 2 * B * H * (S + W) * D
    step_bytes = B * (S * (D // 2 + 4) + W * D * 2 + H * D * 4)

    def make_layer(seed):
        # layer 0: seed 3 (blocks), 4 (q), 5 (window), 6 (sink); layer l > 0 the same seeds + 10007 l
        blocks = rope_interleaved(normal((B, S, D), seed, device=dev), torch.arange(S, device=dev) * 128 + 127)
        codes, scale = pq.encode(blocks)
        return dict(codes=codes, scale=scale, q=normal((B, 1, H, D), seed + 1, device=dev),
                    win=normal((B, W, D), seed + 2, device=dev),
                    sink=normal((H,), seed + 3, dtype=torch.float32, device=dev))

    def layer_step(x):
        return lambda: quant_sink_attention(x["q"], x["codes"], x["scale"], None, x["win"], x["sink"], D ** -0.5,
                                            quant=pq, workspace=ws, out=out)

    n_layers = max(8, -(-2 * MALL_BYTES // step_bytes) + 1)
    layers = [make_layer(3 + 10007 * l) for l in range(n_layers)]
    step = layer_step(layers[0])
    if args.cold_only:  # (profiling the cold step alone)
        ms_eager = ms_warm = float("nan")
    else:
        ms_eager = timed(step, args.steps, args.warmup)
        ms_warm = timed_graph(step, args.steps, args.warmup)
    ms = timed_graph_layers([layer_step(x) for x in layers], args.steps, args.warmup)
    res = {"B": B, "S": S, "bits": 4, "ms_per_step": round(ms, 5), "tokens_per_s": round(B / ms * 1e3, 1),
           "timing": f"cold: {n_layers} layers' distinct caches ({n_layers * step_bytes / 2 ** 20:.0f} MiB per pass), "
                     f"one step per layer captured in one HIP graph and replayed",
           "tflops": round(flops / ms / 1e9, 3), "mfma_frac": round(flops / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 5),
           "hbm_frac": round(step_bytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes_per_step": step_bytes,
           "warm": {"ms_per_step": round(ms_warm, 5), "tokens_per_s": round(B / ms_warm * 1e3, 1),
                    "timing": f"one layer's inputs, HIP graph of {GRAPH_STEPS} steps replayed (caches stay warm)"},
           "ms_per_step_eager_warm": round(ms_eager, 5)}
    log(f"cfg4: cold {ms * 1e3:.1f} us/step ({n_layers} layers) -> {res['tokens_per_s']:.0f} tok/s; warm "
        f"{ms_warm * 1e3:.1f} (eager {ms_eager * 1e3:.1f})")
    del layers
    torch.cuda.empty_cache()
    return res


def bench_prefill(args, dev, kind):
    """One chunk of T = 256 prefill targets per sequence at the end of a long prompt, through the
    quantised reader (modeling.py:293-337 HCA, :496-550 CSA): CSA over cfg3's cache (B=8, 65536-token
    prompt -> 16384 8-bit blocks, top-256), HCA over cfg4's (262144-token prompt -> 2048 4-bit
    blocks, B=8).  Window W=128: the buffer holds the W-1 entries before the chunk and its T."""
    from aetherkv import PolarQuant
    from aetherkv.decode import indexer_workspace
    from aetherkv.prefill import (csa_prefill_indexer_topk_quant, prefill_sources, prefill_workspace,
                                  quant_prefill_attention)
    from aetherkv.synthetic import normal

    B, T, H, D, W, IH, IC = 8, 256, 12, 128, 128, 4, 64
    M, bits, seed = (4, 8, 2) if kind == "csa" else (128, 4, 3)
    S = 16384 if kind == "csa" else 2048
    start = S * M - T  # the prompt's last chunk
    Wt = W - 1 + T
    log(f"prefill {kind}: B={B} T={T} targets at positions {start}..{start + T - 1}, {S} {bits}-bit blocks")
    pq = PolarQuant(bits)
    codes, scale = pq.encode(normal((B, S, D), seed, device=dev))
    q = normal((B, T, H, D), seed + 1, device=dev)
    win = normal((B, Wt, D), seed + 4, device=dev)
    sink = normal((H,), seed + 5, dtype=torch.float32, device=dev)
    vis, ws, wl = prefill_sources(T, start, S, compression=M, sliding_window=W, window_base=start - (W - 1),
                                  window_len=Wt)
    vis, ws, wl = (x.to(dev).expand(B, T).contiguous() for x in (vis, ws, wl))
    out = torch.empty((B, T, H, D), dtype=torch.bfloat16, device=dev)
    res = {"B": B, "T": T, "positions": [start, start + T - 1], "blocks": S, "bits": bits, "window": W}
    if kind == "csa":
        k = 256
        ix_codes, ix_scale = pq.encode(normal((B, S, IC), seed + 1000, device=dev))
        index_q = normal((B, T, IH, IC), seed + 2, dtype=torch.float32, device=dev)
        index_w = normal((B, T, IH), seed + 3, dtype=torch.float32, device=dev)
        idx = torch.empty((B, T, k), dtype=torch.int64, device=dev)
        ws_i = indexer_workspace(B * T, S, k, dev)
        n_sel = torch.clamp(vis, max=k)
        ws_a = prefill_workspace(B, T, H, k, Wt, dev)

        def index_only():
            csa_prefill_indexer_topk_quant(index_q, index_w, ix_codes, ix_scale, k, quant=pq, valid=vis,
                                           workspace=ws_i, out=idx)

        def attn_only():
            quant_prefill_attention(q, codes, scale, idx, win, sink, D ** -0.5, quant=pq, visible=n_sel,
                                    win_start=ws, win_len=wl, workspace=ws_a, out=out)

        def step():
            index_only()
            attn_only()

        res["indexer_ms"] = round(timed(index_only, args.steps, args.warmup), 5)
        res["attention_ms"] = round(timed(attn_only, args.steps, args.warmup), 5)
        n_src = k + W
    else:
        ws_a = prefill_workspace(B, T, H, S, Wt, dev)

        def step():
            quant_prefill_attention(q, codes, scale, None, win, sink, D ** -0.5, quant=pq, visible=vis,
                                    win_start=ws, win_len=wl, workspace=ws_a, out=out)

        n_src = S + W
    ms = timed(step, args.steps, args.warmup)
    flops = 2 * 2 * B * T * H * n_src * D  # QK^T and PV over every target's sources
    res.update({"ms_per_chunk": round(ms, 5), "targets_per_s": round(B * T / ms * 1e3, 1),
                "attention_tflops": round(flops / (res.get("attention_ms", ms)) / 1e9, 3)})
    res["mfma_frac"] = round(res["attention_tflops"] / MFMA_BF16_PEAK_TFLOPS, 5)
    log(f"prefill {kind}: {ms * 1e3:.1f} us/chunk -> {res['targets_per_s']:.0f} targets/s "
        + (f"({res['indexer_ms'] * 1e3:.1f} indexer + {res['attention_ms'] * 1e3:.1f} attention) " if kind == "csa"
           else "") + f"attention {res['attention_tflops']:.1f} TFLOP/s")
    del codes, scale, q, win, out
    torch.cuda.empty_cache()
    return res


def bench_paging(args, dev):
    """Code pages vs the reference's bf16 pages for one CSA layer (KV D=128 + index IC=64, 32 blocks per
    128-token page) and one HCA layer (1 block per page), 4-bit: bytes per page, the per-page flush
    (pack codes + scales; the bf16 format needs a decode of the page's blocks), and materialising a
    65536-token prefix (512 pages) back into rings."""
    from aetherkv import PolarQuant
    from aetherkv.cache import CodeRing, compressed_to_bf16_for_paging
    from aetherkv.storage import code_page_shape, materialize_pages, pack_rows
    from aetherkv.synthetic import normal

    pq = PolarQuant(4)
    n_pages, per_page = 512, 32
    shape = {"layer0.hca": (1, 128), "layer1.csa": (per_page, 128), "layer1.csa_index": (per_page, 64)}
    bf16_bytes = sum(b * d * 2 for b, d in shape.values())
    code_bytes = sum(b * w for b, w in code_page_shape(shape, 4).values())
    kv_c, kv_s = pq.encode(normal((1, n_pages * per_page, 128), 11, device=dev))
    ix_c, ix_s = pq.encode(normal((1, n_pages * per_page, 64), 12, device=dev))
    hc_c, hc_s = pq.encode(normal((1, n_pages, 128), 13, device=dev))

    def flush_codes():
        return {"layer0.hca": pack_rows(hc_c[0, :1], hc_s[0, :1]),
                "layer1.csa": pack_rows(kv_c[0, :per_page], kv_s[0, :per_page]),
                "layer1.csa_index": pack_rows(ix_c[0, :per_page], ix_s[0, :per_page])}

    def flush_bf16():
        return {"layer0.hca": compressed_to_bf16_for_paging(pq, hc_c, hc_s, 0, 1, torch.bfloat16)[0],
                "layer1.csa": compressed_to_bf16_for_paging(pq, kv_c, kv_s, 0, per_page, torch.bfloat16)[0],
                "layer1.csa_index": compressed_to_bf16_for_paging(pq, ix_c, ix_s, 0, per_page, torch.bfloat16)[0]}

    pages = [{"layer1.csa": pack_rows(kv_c[0, i * per_page:(i + 1) * per_page], kv_s[0, i * per_page:(i + 1) * per_page]),
              "layer1.csa_index": pack_rows(ix_c[0, i * per_page:(i + 1) * per_page],
                                            ix_s[0, i * per_page:(i + 1) * per_page])} for i in range(n_pages)]

    def materialize():
        materialize_pages(pages, "layer1.csa", pq, 128, device=dev)
        materialize_pages(pages, "layer1.csa_index", pq, 64, device=dev)

    ms_fc = timed(flush_codes, args.steps, args.warmup)
    ms_fb = timed(flush_bf16, args.steps, args.warmup)
    ms_mat = timed(materialize, max(3, args.steps // 4), 1)
    res = {"page_bytes_codes": code_bytes, "page_bytes_bf16": bf16_bytes,
           "flush_ms_codes": round(ms_fc, 5), "flush_ms_bf16_decode": round(ms_fb, 5),
           "materialize_512_pages_ms": round(ms_mat, 4),
           "materialize_GB/s": round(n_pages * per_page * (68 + 36) / ms_mat / 1e6, 2),
           "layout": "uint8 rows [codes | fp32 scale] per block; 1 HCA + 32 CSA (+32 index) blocks per 128-token page"}
    log(f"paging: {code_bytes} B per code page vs {bf16_bytes} B bf16; flush {ms_fc * 1e3:.1f} us (codes) vs "
        f"{ms_fb * 1e3:.1f} us (decode to bf16); materialise 512 pages {ms_mat * 1e3:.0f} us")
    return res


def bench_attention_io(args, dev):
    """Query prep (q_norm(rope(q))), window entry (kv_norm(rope(kv))) and the output's inverse RoPE for a
    cfg5 decode step (B=64, H=12, D=128, rope_dim 64): one aekv_rope_rmsnorm launch each vs the
    reference's bf16 torch op sequence (apply_rope + F.rms_norm) on the same GPU, both replayed from
    HIP graphs."""
    import torch.nn.functional as F

    from aetherkv.attention_io import rope_rmsnorm
    from aetherkv.cache import rope_inv_freq
    from aetherkv.synthetic import normal

    B, H, D, rope = 64, 12, 128, 64
    q = normal((B, H, D), 21, device=dev)
    kv = normal((B, 1, D), 22, device=dev)
    o = normal((B, H, D), 23, device=dev)
    w = torch.ones(D, dtype=torch.bfloat16, device=dev)
    inv = rope_inv_freq(rope, 10000.0).to(dev)
    pos = torch.full((B,), 65535, dtype=torch.int64, device=dev)
    outs = [torch.empty_like(q), torch.empty_like(kv), torch.empty_like(o)]

    def fused():
        rope_rmsnorm(q, pos, rope_dim=rope, inv_freq=inv, norm_weight=w, out=outs[0])
        rope_rmsnorm(kv, pos, rope_dim=rope, inv_freq=inv, norm_weight=w, out=outs[1])
        rope_rmsnorm(o, pos, rope_dim=rope, inv_freq=inv, inverse=True, out=outs[2])

    pf = pos.float()

    def torch_rope(x, sign):
        pp, rp = x[..., :-rope], x[..., -rope:]
        ang = (sign * pf).unsqueeze(-1) * inv
        cos = torch.repeat_interleave(ang.cos(), 2, dim=-1).to(x.dtype).view(B, 1, rope)
        sin = torch.repeat_interleave(ang.sin(), 2, dim=-1).to(x.dtype).view(B, 1, rope)
        x1, x2 = rp[..., ::2], rp[..., 1::2]
        return torch.cat([pp, rp * cos + torch.stack((-x2, x1), dim=-1).flatten(-2) * sin], dim=-1)

    def reference_ops():
        outs[0].copy_(F.rms_norm(torch_rope(q, 1), (D,), w, 1e-6))
        outs[1].copy_(F.rms_norm(torch_rope(kv, 1), (D,), w, 1e-6))
        outs[2].copy_(torch_rope(o, -1))

    ms_f = timed_graph(fused, args.steps, args.warmup)
    ms_r = timed_graph(reference_ops, args.steps, args.warmup)
    log(f"attention io (cfg5 step): fused {ms_f * 1e3:.1f} us vs torch op sequence {ms_r * 1e3:.1f} us")
    return {"shape": "B=64 H=12 D=128 rope_dim=64: query prep + window entry + inverse rope",
            "fused_ms": round(ms_f, 5), "torch_ops_ms": round(ms_r, 5), "timing": "HIP graph replay"}


def bench_sparse_report_shape(args, dev):
    """The reference's kernel microbenchmark shape (scripts/benchmark_cuda_kernels.py:12-57, published
    in TECHNICAL_REPORT.md:228-235): eager calls through the drop-in entry point, as the reference
    times it, and the same call replayed from a HIP graph (the kernel without the host's per-call
    cost)."""
    from aetherkv import sparse_sink_attention

    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, 128, 16, 128, device=dev, generator=g).half()
    kv = torch.randn(1, 8192, 2, 128, device=dev, generator=g).half()
    topk = torch.randint(0, 8192, (1, 128, 64), device=dev, generator=g, dtype=torch.int32)
    sink = torch.zeros(16, device=dev).half()
    fn = lambda: sparse_sink_attention(q, kv, topk, sink, 128 ** -0.5)  # noqa: E731
    ms = timed(fn, args.steps, args.warmup)
    ms_g = timed_graph(fn, args.steps, args.warmup)
    log(f"sparse_sink_attention report shape: {ms * 1e3:.1f} us eager, {ms_g * 1e3:.1f} us graphed "
        "(reference published 75.9 us)")
    return {"shape": "fp16 B=1 T=128 H=16 D=128 S=8192 top_k=64", "ms": round(ms, 5), "ms_graphed": round(ms_g, 5),
            "reference_published_ms": 0.0759}


def bench_tiled_prefill(args, dev):
    """tiled_prefill_attention (aether_kernels/sparse_attention.py:19-42) at two shapes: T = 256
    targets over S = 8192 sources (16 heads, bf16, separate K and V), and the per-target call the
    model makes in its tiled prefill (modeling.py:322,534: q [1, 1, 16, 128] over top-512 blocks +
    a 128-entry window stacked as K = V)."""
    from aetherkv import tiled_prefill_attention

    res = {}
    g = torch.Generator(device=dev).manual_seed(1)
    B, T, H, S, D = 1, 256, 16, 8192, 128
    q = torch.randn(B, T, H, D, device=dev, generator=g).to(torch.bfloat16)
    kv = torch.randn(B, S, 2, D, device=dev, generator=g).to(torch.bfloat16)
    sink = torch.randn(H, device=dev, generator=g).to(torch.bfloat16)
    ms = timed(lambda: tiled_prefill_attention(q, kv, sink, D ** -0.5), args.steps, args.warmup)
    tflops = 4 * B * T * H * S * D / ms / 1e9
    res["prefill"] = {"shape": "bf16 B=1 T=256 H=16 D=128 S=8192", "ms": round(ms, 5), "tflops": round(tflops, 2),
                      "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 5)}
    log(f"tiled_prefill_attention T={T} S={S}: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s")
    S1 = 640
    q1 = torch.randn(1, 1, H, D, device=dev, generator=g).to(torch.bfloat16)
    src = torch.randn(1, S1, D, device=dev, generator=g).to(torch.bfloat16)
    kv1 = torch.stack([src, src], dim=2)
    fn = lambda: tiled_prefill_attention(q1, kv1, sink, D ** -0.5)  # noqa: E731
    ms1 = timed(fn, args.steps, args.warmup)
    ms1_g = timed_graph(fn, args.steps, args.warmup)
    res["model_call"] = {"shape": "bf16 B=1 T=1 H=16 D=128 S=640 (K = V)", "ms": round(ms1, 5),
                         "ms_graphed": round(ms1_g, 5)}
    log(f"tiled_prefill_attention per-target call S={S1}: {ms1 * 1e3:.1f} us eager, {ms1_g * 1e3:.1f} us graphed")
    del q, kv, q1, kv1, src
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["all", "encode", "codec", "csa", "hca", "prefill", "paging", "io", "sparse"],
                    default="all")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cold-only", action="store_true",
                    help="decode lines: time only the cold layer rotation (for profiling it alone)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (sharding is a "
              "design note, not code). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    import aetherkv._lib as L

    if not L.available():
        print("libaetherkv.so is not built; run `python __graft_entry__.py` first", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    res = {}
    secondary = {}
    cpu = None
    if args.only in ("all", "encode"):
        bench_encode(args, dev, res)
        if not args.no_cpu_baseline:
            cpu = bench_cpu_encode(res)
        torch.cuda.empty_cache()
    if args.only in ("all", "codec"):
        secondary["codec_shapes"] = bench_codec_shapes(args, dev)
    if args.only in ("all", "csa"):
        cpu_rows = (0, 0) if args.no_cpu_baseline else (8, 8)
        secondary["csa_decode_cfg5"] = bench_csa(args, dev, 64, 65536, 4, 4, True, "cfg5", cpu_rows[0])
        secondary["csa_decode_cfg3"] = bench_csa(args, dev, 8, 16384, 8, 2, False, "cfg3", cpu_rows[1])
    if args.only in ("all", "hca"):
        secondary["hca_decode_cfg4"] = bench_hca(args, dev)
    if args.only in ("all", "prefill"):
        secondary["csa_prefill_chunk"] = bench_prefill(args, dev, "csa")
        secondary["hca_prefill_chunk"] = bench_prefill(args, dev, "hca")
    if args.only in ("all", "io"):
        secondary["attention_io"] = bench_attention_io(args, dev)
    if args.only in ("all", "paging"):
        secondary["code_pages"] = bench_paging(args, dev)
    if args.only in ("all", "sparse"):
        secondary["sparse_sink_attention_report_shape"] = bench_sparse_report_shape(args, dev)
        secondary["tiled_prefill_attention"] = bench_tiled_prefill(args, dev)

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic"}
    if "encode_ms" in res:
        ms = res["encode_ms"]
        gbs = ENC_BYTES / ms / 1e6
        traffic = None
        pmc = ROOT / "profiles" / "tq_encode_cfg2_traffic.json"
        if pmc.exists():
            traffic = json.loads(pmc.read_text()).get("hbm_bytes_per_launch")
        line.update({
            "value": round(gbs, 2), "unit": "GB/s", "ms_per_step": round(ms, 5),
            "config": {"workload": "cfg2: TurboQuant 4-bit encode (WHT + absmax quantise + nibble pack) of one "
                                   "262144-token x 1536 (12x128) bf16 KV layer, N(0,1) with 2% outlier channels x8, "
                                   "seed 1", "tokens": T2, "heads": H2, "head_dim": D2, "bits": 4,
                       "bytes_per_step": ENC_BYTES},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                         "traffic_from": "profiles/tq_encode_cfg2_traffic.json: rocprofv3 --pmc FETCH_SIZE and "
                                         "WRITE_SIZE passes over this kernel at this workload, scaled by the factors "
                                         "that make a copy kernel's counters read its size (not measured in this run)",
                         "kernel": "tq_encode4_d128_bf16_kernel"},
        })
        secondary["tq_decode_cfg2"] = {"ms": round(res["decode_ms"], 5),
                                       "GB/s": round(ENC_BYTES / res["decode_ms"] / 1e6, 2),
                                       "frac": round(ENC_BYTES / res["decode_ms"] / 1e6 / HBM_PEAK_GBS, 4)}
        secondary["copy_GB/s"] = round(res["copy_gbs"], 1)
        secondary["stream_ceiling"] = {
            "GB/s": round(res["stream_ceiling_gbs"], 1),
            "encode_of_ceiling": round(ENC_BYTES / res["encode_ms"] / 1e6 / res["stream_ceiling_gbs"], 4),
            "what": "aekv_stream_probe: the encode's bytes and access pattern (64 B per lane in, 16 B codes per "
                    "lane and 4 B scale per vector out, non-temporal stores) with no transform"}
        ms_i = res["encode_ms_from_idle"]
        secondary["tq_encode_cfg2_from_idle"] = {
            "ms": round(ms_i, 5), "GB/s": round(ENC_BYTES / ms_i / 1e6, 2),
            "note": "the same K steps after only the W warmup steps, i.e. inside the slower phase of the "
                    "first ~20 ms of load after idle; `value` is timed after a settle period of continuous launches"}
    else:
        first = next(iter(secondary.values()), {})
        line.update({"value": first.get("tokens_per_s"), "unit": "tokens/s", "ms_per_step": first.get("ms_per_step"),
                     "config": {"workload": args.only}})
    line["cpu_baseline"] = cpu
    line["secondary"] = secondary
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
