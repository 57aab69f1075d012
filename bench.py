"""Benchmark of the MI355X quantized-weight path (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
                    [--workload NAME[,NAME...]|all|headline|hbm_copy_64mb] [--no-cpu]
                    [--graph]

A step is one pass of the hot path over one batch of synthetic input with the
weights already resident in HBM. The headline workload (value / metric) is
the Q4_K dequant-fused matvec y = W x, W 4096 x 2048 (4,718,592 packed bytes),
batch 1; `value` is algorithmic HBM bytes per step / time per step in GB/s.
The same JSON line carries every other workload (Q8_0 / Q6_K matvecs,
64M-weight dequant, 512-expert top-10 MoE decode in tokens/s, the Q6_K
151936 x 2048 LM head with argmax at batch 1 and 4, MoE prefill T=512),
the roofline of the headline kernel and the CPU baseline (the C oracle,
timed on this host on a bounded sample).

Timing: W untimed warmup steps and a device synchronisation; then the
stream gets a 512 MiB device copy (which evicts the ~256 MB Infinity Cache)
and a hold kernel of 100 us + 25 us per step, the first HIP event, the K
steps' launches and the second event, all enqueued by the host while the
copy and the hold run, so the events bracket the K launches running back to
back. Device synchronisation on both sides. Weight replicas (bit-identical
device copies at distinct addresses) rotate so that the bytes touched
between two uses of a replica within the timed steps exceed 512 MB, twice
the Infinity Cache: every weight read in the timed region is an HBM read,
for any K. --graph captures the K steps in a HIP graph instead (replayed
once untimed, then timed the same way); its replay adds about 12 us per
timed region on this part (per step: 0.6 us at K = 20, 0.06 us at 200).

Floors measured the same way (libkq_floor.so): an empty launch, and plain
streaming reads of the headline's, the 131072 x 2048 matvec's and the LM
head's weight bytes.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kestrel-q_amd"))

import kq_hip  # noqa: E402
import kq_synth as S  # noqa: E402

HBM_PEAK_GBS = 8000.0
MALL_DEFEAT_BYTES = 512 << 20
FLUSH_BYTES = 256 << 20  # copied between the untimed and the timed replay

# ---------------------------------------------------------------- HIP runtime
_hip = None


def hip():
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [C.c_void_p]
        _hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        _hip.hipEventSynchronize.argtypes = [C.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        _hip.hipEventDestroy.argtypes = [C.c_void_p]
        _hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        _hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.c_void_p]
        _hip.hipGraphInstantiate.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                             C.c_size_t]
        _hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        _hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
        _hip.hipGraphDestroy.argtypes = [C.c_void_p]
        _hip.hipStreamSynchronize.argtypes = [C.c_void_p]
        _hip.hipDeviceSynchronize.argtypes = []
        _hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    return _hip


def hcheck(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed with hipError {rc}")


class Events:
    def __init__(self):
        self.a, self.b = C.c_void_p(), C.c_void_p()
        hcheck(hip().hipEventCreate(C.byref(self.a)), "hipEventCreate")
        hcheck(hip().hipEventCreate(C.byref(self.b)), "hipEventCreate")

    def ms(self) -> float:
        hcheck(hip().hipEventSynchronize(self.b), "hipEventSynchronize")
        v = C.c_float()
        hcheck(hip().hipEventElapsedTime(C.byref(v), self.a, self.b), "hipEventElapsedTime")
        return v.value

    def close(self):
        hip().hipEventDestroy(self.a)
        hip().hipEventDestroy(self.b)


def d2d(ctx, dst, src, nbytes):
    hcheck(hip().hipMemcpyAsync(C.c_void_p(dst), C.c_void_p(src), nbytes, 3,
                                C.c_void_p(ctx.stream)), "hipMemcpyAsync")


_flush = {}


def flush_mall(ctx):
    """Device copy of FLUSH_BYTES (2 x FLUSH_BYTES touched) on ctx's stream:
    evicts the Infinity Cache before a timed replay."""
    if "bufs" not in _flush:
        _flush["bufs"] = (ctx.alloc(FLUSH_BYTES), ctx.alloc(FLUSH_BYTES))
    a, b = _flush["bufs"]
    d2d(ctx, b.ptr, a.ptr, FLUSH_BYTES)


def lead_in(ctx, flush: bool, steps: int) -> None:
    """Work the device runs right before the timed region's first event, so
    the host has enqueued the whole region before it starts: the 512 MiB
    copy (flush) and a hold of 100 us plus 25 us per step (at most 10 ms)."""
    if flush:
        flush_mall(ctx)
    hcheck(floor_lib().kq_floor_hold(min(10000, 100 + 25 * steps), C.c_void_p(ctx.stream)),
           "kq_floor_hold")


def time_steps(ctx, step, warmup: int, steps: int, graph: bool, flush: bool = True) -> float:
    """ms per step over `steps` steps; `step(i)` enqueues step i on ctx's stream.
    flush: evict the Infinity Cache before the timed steps."""
    stream = C.c_void_p(ctx.stream)
    ctx.set_async(True)
    for i in range(warmup):
        step(i)
    ctx.synchronize()
    hcheck(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
    ev = Events()
    if graph:
        g, ge = C.c_void_p(), C.c_void_p()
        hcheck(hip().hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
        for i in range(steps):
            step(warmup + i)
        hcheck(hip().hipStreamEndCapture(stream, C.byref(g)), "hipStreamEndCapture")
        hcheck(hip().hipGraphInstantiate(C.byref(ge), g, None, None, 0), "hipGraphInstantiate")
        hcheck(hip().hipGraphLaunch(ge, stream), "hipGraphLaunch")  # untimed replay
        hcheck(hip().hipStreamSynchronize(stream), "hipStreamSynchronize")
        lead_in(ctx, flush, steps)
        hcheck(hip().hipEventRecord(ev.a, stream), "hipEventRecord")
        hcheck(hip().hipGraphLaunch(ge, stream), "hipGraphLaunch")
        hcheck(hip().hipEventRecord(ev.b, stream), "hipEventRecord")
        ms = ev.ms()
        hip().hipGraphExecDestroy(ge)
        hip().hipGraphDestroy(g)
    else:
        lead_in(ctx, flush, steps)
        hcheck(hip().hipEventRecord(ev.a, stream), "hipEventRecord")
        for i in range(steps):
            step(warmup + i)
        hcheck(hip().hipEventRecord(ev.b, stream), "hipEventRecord")
        ms = ev.ms()
    hcheck(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
    ev.close()
    ctx.synchronize()  # reports any device-detected failure
    ctx.set_async(False)
    return ms / steps


def time_each(ctx, step, warmup: int, steps: int) -> float:
    """Mean duration of one launch on its own, in ms: a pair of HIP events
    brackets every launch of `steps` consecutive ones (the same sequence as
    time_steps, behind the same flush and hold). Each pair times the
    dispatch with its start and completion, as a kernel trace does; the
    spacing of back-to-back launches (time_steps) is shorter for short
    kernels, whose start and end overheads overlap their neighbours'."""
    stream = C.c_void_p(ctx.stream)
    ctx.set_async(True)
    for i in range(warmup):
        step(i)
    ctx.synchronize()
    hcheck(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
    evs = [Events() for _ in range(steps)]
    lead_in(ctx, True, steps)
    for i in range(steps):
        hcheck(hip().hipEventRecord(evs[i].a, stream), "hipEventRecord")
        step(warmup + i)
        hcheck(hip().hipEventRecord(evs[i].b, stream), "hipEventRecord")
    ms = [e.ms() for e in evs]
    hcheck(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
    for e in evs:
        e.close()
    ctx.synchronize()
    ctx.set_async(False)
    return float(np.mean(ms))


def replicas(ctx, host: np.ndarray, want_bytes: int, cap: int = 256):
    """Bit-identical device copies of `host` at distinct addresses."""
    n = max(1, min(cap, -(-want_bytes // max(1, host.nbytes))))
    first = ctx.upload(host)
    out = [first]
    for _ in range(n - 1):
        b = ctx.alloc(host.nbytes)
        d2d(ctx, b.ptr, first.ptr, host.nbytes)
        out.append(b)
    ctx.synchronize()
    return out


def reuse_bytes(nrep: int, nbytes: int, steps: int, warm: bool = False):
    """Weight bytes read between two uses of one replica in the timed
    replay (None: no replica is read twice). The copy before the replay
    separates it from the untimed one."""
    if warm:
        return 0
    return nrep * nbytes if steps > nrep else None


# ---------------------------------------------------------------- workloads
def wl_matvec(ctx, fmt, rows, cols, batch, warmup, steps, graph, warm=False, each=False):
    """warm: one weight copy, re-read every step from the caches (a
    single-call latency with a warm cache, not an HBM rate). each: also the
    mean duration of one launch on its own (time_each)."""
    t = kq_hip.TYPE_IDS[fmt]
    w = S.quant_matrix(fmt, S.stream_key(S.W_MATVEC_Q4K, S.R_WEIGHT), rows, cols)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q4K, S.R_X), batch * cols)
    reps = replicas(ctx, w, 0 if warm else MALL_DEFEAT_BYTES, cap=1 if warm else 256)
    dx, dy = ctx.upload(x), ctx.alloc(rows * batch * 4)
    step = lambda i: ctx.matvec(t, reps[i % len(reps)], rows, cols, dx, batch, dy)  # noqa: E731
    ms = time_steps(ctx, step, warmup, steps, graph, flush=not warm)
    nbytes = w.nbytes + x.nbytes + rows * batch * 4
    out = {"ms_per_step": ms, "bytes_per_step": nbytes, "GBps": nbytes / ms / 1e6,
           "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS, "replicas": len(reps),
           "bytes_between_reuse": reuse_bytes(len(reps), w.nbytes, steps, warm),
           "flops_per_step": 2 * rows * cols * batch}
    if each:
        one = time_each(ctx, step, warmup, steps)
        out.update({"dispatch_ms": one, "dispatch_GBps": nbytes / one / 1e6})
    for b in reps + [dx, dy]:
        b.close()
    return out


def wl_dequant(ctx, fmt, warmup, steps, graph):
    t = kq_hip.TYPE_IDS[fmt]
    gen, qk, bb = S.BLOCK_GEN[fmt]
    blocks = (1 << 26) // qk
    w = gen(S.stream_key(S.W_DEQUANT, S.R_WEIGHT, t), blocks).reshape(-1)
    reps = replicas(ctx, w, 2 * w.nbytes, cap=2)
    n = blocks * qk
    out = ctx.alloc(n * 4)
    ms = time_steps(ctx, lambda i: ctx.dequantize(t, reps[i % len(reps)], w.nbytes, out, n),
                    warmup, steps, graph)
    nbytes = w.nbytes + n * 4
    for b in reps + [out]:
        b.close()
    return {"ms_per_step": ms, "bytes_per_step": nbytes, "GBps": nbytes / ms / 1e6,
            "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS, "weights": n}


# MoE layers measured: the configuration the headline MoE figures are quoted
# on, and the reference model's own layers (hidden 2560, intermediate 640,
# Q4_K gate/up, Q5_1 routed down, Q8_0 shared expert; its layer 2 with Q5_K
# gate/up and a Q8_0 routed down).
MOE_LAYERS = {
    "2048x512": dict(H=2048, E=512, K=10, I=512, gate="Q4_K", down="Q6_K", sgate="Q4_K",
                     sdown="Q6_K", seed=S.W_MOE),
    "2560x640": dict(H=2560, E=512, K=10, I=640, gate="Q4_K", down="Q5_1", sgate="Q8_0",
                     sdown="Q8_0", seed=S.W_MOE + 2560),
    "2560x640_l2": dict(H=2560, E=512, K=10, I=640, gate="Q5_K", down="Q8_0", sgate="Q8_0",
                        sdown="Q8_0", seed=S.W_MOE + 2562),
}


def near_tie(router, x, K, c):
    """x moved (least-norm, binary64) so that the K-th and (K+1)-th logits
    by binary64 value are c times the sum of their certification bounds
    apart (1.001 * 2^-24 * sum of |prefix sums| each)."""
    r64, x64 = router.astype(np.float64), x.astype(np.float64)
    a = r64 @ x64
    order = np.argsort(-a, kind="stable")
    hi, lo = order[K - 1], order[K]

    def bound(e):
        return 1.001 * 2.0 ** -24 * np.abs(np.cumsum((router[e] * x).astype(np.float64))).sum()
    d = r64[hi] - r64[lo]
    g = c * (bound(hi) + bound(lo))
    return (x64 - ((a[hi] - a[lo] - g) / (d @ d)) * d).astype(np.float32)


def wl_moe(ctx, tokens, warmup, steps, graph, layer_cache, layer="2048x512", block=False,
           inputs="random"):
    """block: the MoE block (4 residual branches, hyper-connection read with
    rank-320 Q8_0 projections, MoE, write) instead of the bare MoE.
    inputs (one token): "random" ~N(0,1) activations; "near_tie" the same
    moved so that the selection's boundary pair is 1/4 of its certification
    bounds apart (the refined route: exact chains of the contenders);
    "all_tie" zero activations, every logit equal (the exact route: every
    row's chain, then the route finish)."""
    L = MOE_LAYERS[layer]
    H, E, K, I = L["H"], L["E"], L["K"], L["I"]
    if layer_cache.get("layer") != layer:
        layer_cache.clear()
        layer_cache["layer"] = layer
        layer_cache["w"] = S.moe_weights(L["seed"], H, E, I, I, gate_fmt=L["gate"],
                                         down_fmt=L["down"], shared_gate_fmt=L["sgate"],
                                         shared_down_fmt=L["sdown"])
        layer_cache["cfg"] = kq_hip.MoeConfig(H, E, K, I, I)
    w, cfg = layer_cache["w"], layer_cache["cfg"]
    layer_bytes = sum(v.nbytes for v in w.values())
    # bytes one decode step reads: the router, K routed experts' gate, up and
    # down, the shared expert and its gate vector (26.6 MB for 2048x512);
    # whole-layer replicas rotate so that reuse does not hit the MALL
    expert = (w["gate"].nbytes + w["up"].nbytes + w["down"].nbytes) // E
    shared = w["shared_gate"].nbytes + w["shared_up"].nbytes + w["shared_down"].nbytes
    touched = w["router"].nbytes + K * expert + shared + w["shared_gate_weight"].nbytes
    if tokens > 1:
        touched = layer_bytes
    allw = dict(w)
    width = H
    if block:
        nb, rank = 4, 320
        width = nb * H
        key = lambda i: S.stream_key(L["seed"], 90, i)
        allw.update({"gr_norm": S.normal_f32(key(1), width, 0.1),
                     "gr_down": S.quant_matrix("Q8_0", key(2), rank, width),
                     "gr_up": S.quant_matrix("Q8_0", key(3), width, rank),
                     "gr_inject": S.normal_f32(key(4), nb * width, 0.01)})
        touched += sum(v.nbytes for k, v in allw.items() if k.startswith("gr_"))
        gdims = kq_hip.gr_dims(nb, H, rank)
    nrep = max(2, min(24, -(-MALL_DEFEAT_BYTES // touched)))
    if tokens > 1:
        nrep = 1
    layers = []
    for r in range(nrep):
        if r == 0:
            bufs = {k: ctx.upload(v) for k, v in allw.items()}
        else:
            bufs = {}
            for k, v in allw.items():
                b = ctx.alloc(v.nbytes)
                d2d(ctx, b.ptr, layers[0][k].ptr, v.nbytes)
                bufs[k] = b
        layers.append(bufs)
    ctx.synchronize()
    t = kq_hip.TYPE_IDS
    mw = [kq_hip.moe_weights(b, t[L["gate"]], t[L["down"]], t[L["sgate"]], t[L["sdown"]])
          for b in layers]
    ntok_inputs = 16
    x = S.normal_f32(S.stream_key(L["seed"], S.R_HIDDEN, 1000 + tokens),
                     ntok_inputs * tokens * width).reshape(ntok_inputs, tokens * width)
    if inputs == "near_tie":
        router = w["router"].reshape(E, H)
        x = np.stack([near_tie(router, x[j], K, 0.25) for j in range(ntok_inputs)])
    elif inputs == "all_tie":
        x = np.zeros_like(x)
    dxs = [ctx.upload(x[j]) for j in range(ntok_inputs)]
    n = kq_hip.moe_block_scratch_bytes(gdims, cfg, tokens) if block else cfg.scratch_bytes(tokens)
    scratch = ctx.alloc(n)
    out = ctx.alloc(tokens * width * 4)
    if block:
        q8 = kq_hip.TYPE_Q8_0
        gws = [kq_hip.gr_weights({k: b["gr_" + k] for k in ("norm", "down", "up", "inject")},
                                 q8, q8) for b in layers]

    def step(i):
        if block:
            ctx.moe_block(gdims, gws[i % nrep], cfg, mw[i % nrep], dxs[i % ntok_inputs], tokens,
                          out, None, scratch, n)
        else:
            ctx.moe_execute(cfg, mw[i % nrep], dxs[i % ntok_inputs], tokens, out, None, scratch,
                            n)

    paths = None
    if tokens == 1 and not block:
        # the certification word (the workspace's last 256-byte slot): 1
        # certified, 2 refined, 0 exact route
        paths = {"certified": 0, "refined": 0, "exact": 0}
        for j in range(ntok_inputs):
            step(j)
            ctx.synchronize()
            f = int(ctx.download(scratch.ptr + n - 256, np.uint32, 1)[0])
            paths[{1: "certified", 2: "refined"}.get(f, "exact")] += 1
    ms = time_steps(ctx, step, warmup, steps, graph)
    for bufs in layers:
        for b in bufs.values():
            b.close()
    for b in dxs + [scratch, out]:
        b.close()
    nbytes = touched + 2 * tokens * width * 4
    return {"ms_per_step": ms, "tokens_per_s": tokens / ms * 1e3, "bytes_per_step": nbytes,
            "GBps": nbytes / ms / 1e6, "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS,
            "layer_replicas": nrep, "tokens": tokens, "layer": layer + ("+gr" if block else ""),
            **({"inputs": inputs, "route_paths": paths} if paths else {})}


def wl_lm_head(ctx, batch, warmup, steps, graph, fmt="Q6_K", V=151936, H=2048):
    t = kq_hip.TYPE_IDS[fmt]
    w = S.quant_matrix(fmt, S.stream_key(S.W_LM_HEAD, S.R_WEIGHT), V, H)
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, batch), batch * H)
    reps = replicas(ctx, w, MALL_DEFEAT_BYTES + w.nbytes, cap=3)
    dh, dl, di = ctx.upload(h), ctx.alloc(V * batch * 4), ctx.alloc(batch * 4)
    ms = time_steps(ctx, lambda i: ctx.lm_head(t, reps[i % len(reps)], V, H, dh,
                                               batch, dl, di), warmup, steps, graph)
    nbytes = w.nbytes + h.nbytes + V * batch * 4
    for b in reps + [dh, dl, di]:
        b.close()
    return {"ms_per_step": ms, "bytes_per_step": nbytes, "GBps": nbytes / ms / 1e6,
            "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS, "tokens_per_s": batch / ms * 1e3,
            "replicas": len(reps)}


def wl_sample(ctx, pol, warmup, steps, lm=None):
    """One synchronous kq_hip_sampling_select_f32 per step on the reference
    model's 248,320 logits (device resident), or with lm = (fmt, H) the
    fused LM head + sampler on W[248320][H]. Host wall clock per call: the
    launches, the device sort and walks, and the result's copy back."""
    V = kq_hip.QWEN38_VOCAB
    cfg = kq_hip.SamplingConfig(kq_hip.sampling_policy(**pol))
    scratch = ctx.alloc(cfg.scratch_bytes)
    lg = (np.random.default_rng(7).standard_normal(V) * 3).astype(np.float32)
    dl = ctx.upload(lg)
    st = kq_hip.rng_seed(1, kq_hip.SAMPLING_DEFAULT_STREAM)
    bufs = [scratch, dl]
    if lm is None:
        step = lambda: ctx.sample(cfg, st, dl, scratch)
        nbytes = V * 4
    else:
        fmt, H = lm
        t = kq_hip.TYPE_IDS[fmt]
        w = S.quant_matrix(fmt, S.stream_key(S.W_LM_HEAD, S.R_WEIGHT, 1), V, H)
        dw, dh = ctx.upload(w), ctx.upload(S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN), H))
        bufs += [dw, dh]
        step = lambda: ctx.lm_head_sample(cfg, st, t, dw, V, H, dh, dl, scratch)
        nbytes = w.nbytes + H * 4 + V * 4
    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    for b in bufs:
        b.close()
    cfg.close()
    return {"ms_per_step": ms, "tokens_per_s": 1e3 / ms, "bytes_per_step": nbytes,
            "policy": pol, "time_source": "host wall clock per synchronous call"}


def wl_copy(ctx, nbytes, warmup, steps, graph):
    """Device-to-device copy of a known size: the reference point that scales
    the FETCH_SIZE / WRITE_SIZE counters to bytes. Not part of `all`."""
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    ms = time_steps(ctx, lambda i: d2d(ctx, b.ptr, a.ptr, nbytes), warmup, steps, graph)
    for buf in (a, b):
        buf.close()
    return {"ms_per_step": ms, "bytes_per_step": 2 * nbytes, "GBps": 2 * nbytes / ms / 1e6,
            "hbm_frac": 2 * nbytes / ms / 1e6 / HBM_PEAK_GBS, "copy_bytes": nbytes}


_floor = None


def floor_lib():
    global _floor
    if _floor is None:
        path = ROOT / "kestrel-q_amd" / "_build" / "libkq_floor.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: build with __graft_entry__.build()")
        _floor = C.CDLL(str(path))
        _floor.kq_floor_empty.argtypes = [C.c_void_p]
        _floor.kq_floor_hold.argtypes = [C.c_uint32, C.c_void_p]
        _floor.kq_floor_read.argtypes = [C.c_void_p, C.c_uint64, C.c_int, C.c_void_p, C.c_void_p]
    return _floor


def wl_floor_empty(ctx, warmup, steps, graph):
    """An empty kernel per step: the launch cost every workload pays."""
    ms = time_steps(ctx, lambda i: hcheck(floor_lib().kq_floor_empty(C.c_void_p(ctx.stream)),
                                          "kq_floor_empty"), warmup, steps, graph)
    return {"ms_per_step": ms}


def wl_floor_read(ctx, nbytes, loads, warmup, steps, graph):
    """A plain streaming read of nbytes per step (replicas rotate as for the
    matvecs): the fastest this size can be read in one launch, over the
    given numbers of 16-byte loads per thread (the best one is reported)."""
    host = np.zeros(nbytes, np.uint8)
    reps = replicas(ctx, host, MALL_DEFEAT_BYTES, cap=256)
    sink = ctx.alloc(4)
    per = {}
    for ld in loads:
        per[ld] = time_steps(ctx, lambda i: hcheck(floor_lib().kq_floor_read(
            C.c_void_p(reps[i % len(reps)].ptr), nbytes, ld, C.c_void_p(sink.ptr),
            C.c_void_p(ctx.stream)), "kq_floor_read"), warmup, steps, graph)
    for b in reps + [sink]:
        b.close()
    best = min(per, key=per.get)
    ms = per[best]
    return {"ms_per_step": ms, "bytes_per_step": nbytes, "GBps": nbytes / ms / 1e6,
            "hbm_frac": nbytes / ms / 1e6 / HBM_PEAK_GBS, "replicas": len(reps),
            "loads_per_thread": best, "us_by_loads_per_thread":
                {str(k): round(v * 1e3, 3) for k, v in per.items()},
            "bytes_between_reuse": reuse_bytes(len(reps), nbytes, steps)}


# ---------------------------------------------------------------- CPU baseline
def cpu_baseline(threads: int, budget_s: float = 3.0) -> dict:
    """The C oracle (restatement of the reference's scalar path, reference fp
    flags) on this host: the headline matvec at 1 thread and `threads`
    threads with identical per-row arithmetic, plus one MoE decode step and
    one LM-head step."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import kq_oracle as O

    def timeit(fn, budget):
        fn()
        ts = []
        t_end = time.perf_counter() + budget
        while len(ts) < 3 or (time.perf_counter() < t_end and len(ts) < 50):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)), len(ts)

    res = {}
    w = S.quant_matrix("Q4_K", S.stream_key(S.W_MATVEC_Q4K, S.R_WEIGHT), 4096, 2048)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q4K, S.R_X), 2048)[None, :]
    nbytes = w.nbytes + x.nbytes + 4096 * 4
    for th in sorted({1, threads}):
        s, n = timeit(lambda: O.matvec(O.Q4_K, w, 4096, 2048, x, threads=th), budget_s)
        res[f"q4k_matvec_{th}t"] = {"s_per_step": s, "GBps": nbytes / s / 1e9, "runs": n}
    L = MOE_LAYERS["2048x512"]
    wts = S.moe_weights(L["seed"], 2048, 512, 512, 512)
    roles = {"router": O.F32, "gate": O.Q4_K, "up": O.Q4_K, "down": O.Q6_K,
             "shared_gate": O.Q4_K, "shared_up": O.Q4_K, "shared_down": O.Q6_K,
             "shared_gate_weight": O.F32}
    dims = dict(hidden=2048, experts=512, top_k=10, inter=512, shared_inter=512)
    xm = S.normal_f32(S.stream_key(S.W_MOE, S.R_HIDDEN, 1001), 2048)[None, :]
    wr = {k: (t, wts[k]) for k, t in roles.items()}
    for th in sorted({1, threads}):
        s, n = timeit(lambda: O.moe_execute(dims, wr, xm, threads=th), budget_s)
        res[f"moe_decode_{th}t"] = {"s_per_step": s, "tokens_per_s": 1.0 / s, "runs": n}
    wl = S.quant_matrix("Q6_K", S.stream_key(S.W_LM_HEAD, S.R_WEIGHT), 151936, 2048)
    hl = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, 1), 2048)[None, :]
    for th in sorted({1, threads}):
        s, n = timeit(lambda: O.argmax(O.matvec(O.Q6_K, wl, 151936, 2048, hl, threads=th)[0]),
                      budget_s if th > 1 else 0.0)
        res[f"lm_head_b1_{th}t"] = {"s_per_step": s, "tokens_per_s": 1.0 / s, "runs": n}
    return res


def host_cpus() -> dict:
    """The host's CPUs as this process sees them: nproc, the affinity mask,
    the cgroup CPU quota and the lscpu model. `usable` = the smaller of the
    affinity count and the quota: threads beyond it only wait for a share."""
    info = {"nproc": os.cpu_count() or 1}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["affinity"] = info["nproc"]
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    info["cgroup_cpu_quota"] = quota
    usable = info["affinity"]
    if quota is not None:
        usable = max(1, min(usable, int(quota)))
    info["usable"] = usable
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info["lscpu_" + k.strip().lower().replace("(s)", "s").replace(" ", "_")] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


# ---------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="all")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--graph", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="stream launches (the default)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    graph = args.graph
    K, W = args.steps, args.warmup
    wanted = args.workload
    work = {}
    with kq_hip.Context(0) as ctx:
        names = set(wanted.split(","))

        def run(name, fn):
            if names & {"all", name} or ("headline" in names and name == HEADLINE):
                print(f"[bench] {name} ...", file=sys.stderr, flush=True)
                t0 = time.time()
                work[name] = fn()
                work[name]["wall_s"] = round(time.time() - t0, 2)
                print(f"[bench] {name}: {json.dumps(work[name])}", file=sys.stderr, flush=True)

        HEADLINE = "q4k_matvec_4096x2048_b1"
        run(HEADLINE, lambda: wl_matvec(ctx, "Q4_K", 4096, 2048, 1, W, K, graph, each=True))
        # what any launch costs, and a plain read of the headline's weight
        # bytes in one launch
        run("floor_empty_launch", lambda: wl_floor_empty(ctx, W, K, graph))
        run("floor_read_4718592b", lambda: wl_floor_read(ctx, 4718592, (1, 2, 4), W, K, graph))
        run("q8_0_matvec_4096x2048_b1", lambda: wl_matvec(ctx, "Q8_0", 4096, 2048, 1, W, K, graph))
        run("q6k_matvec_4096x2048_b1", lambda: wl_matvec(ctx, "Q6_K", 4096, 2048, 1, W, K, graph))
        run("q5k_matvec_4096x2048_b1", lambda: wl_matvec(ctx, "Q5_K", 4096, 2048, 1, W, K, graph))
        run("q5_1_matvec_4096x2048_b1", lambda: wl_matvec(ctx, "Q5_1", 4096, 2048, 1, W, K, graph))
        run("iq4_nl_matvec_4096x2048_b1",
            lambda: wl_matvec(ctx, "IQ4_NL", 4096, 2048, 1, W, K, graph))
        run("q4k_matvec_4096x2048_b1_warm_cache",
            lambda: wl_matvec(ctx, "Q4_K", 4096, 2048, 1, W, K, graph, warm=True))
        # the same kernel family on a matrix large enough to amortise the
        # launch and the first-load latency (151 MB per step): the rate the
        # Q4_K row engine sustains
        run("q4k_matvec_131072x2048_b1",
            lambda: wl_matvec(ctx, "Q4_K", 131072, 2048, 1, 10, max(10, K // 2), graph,
                              each=True))
        run("floor_read_150994944b",
            lambda: wl_floor_read(ctx, 150994944, (2, 4, 8), 10, max(10, K // 2), graph))
        run("floor_read_255252480b",
            lambda: wl_floor_read(ctx, 255252480, (2, 4, 8), 10, max(10, K // 2), graph))
        # the reference model's GDN projections (Q8_0), on their canonical
        # copies (kq_hip_gdn_canonicalize): attn_qkv, attn_gate, ssm_out
        for nm, r, c in (("qkv", 10240, 2560), ("gate", 6144, 2560), ("out", 2560, 6144)):
            run(f"gdn_{nm}_q8_0_{r}x{c}_b1",
                lambda r=r, c=c: wl_matvec(ctx, "Q8_0", r, c, 1, W, K, graph))
        for f in ("Q4_K", "Q8_0", "Q6_K", "Q5_K", "Q5_1", "IQ4_NL"):
            run(f"dequant_64m_{f.lower()}",
                lambda f=f: wl_dequant(ctx, f, 5, max(10, K // 4), graph))
        cache = {}
        run("moe_decode_1tok", lambda: wl_moe(ctx, 1, W, K, graph, cache))
        # the same layer on tokens the bounds cannot certify: the refined
        # route and the exact route
        run("moe_decode_1tok_near_tie",
            lambda: wl_moe(ctx, 1, W, K, graph, cache, inputs="near_tie"))
        run("moe_decode_1tok_all_tie",
            lambda: wl_moe(ctx, 1, W, K, graph, cache, inputs="all_tie"))
        # the large workloads run 100 / 10 timed steps (several ms): shorter
        # timed regions read up to 10% slower per step
        run("lm_head_q6k_151936x2048_b1",
            lambda: wl_lm_head(ctx, 1, 10, max(10, K // 2), graph))
        run("lm_head_q6k_151936x2048_b4",
            lambda: wl_lm_head(ctx, 4, 10, max(10, K // 2), graph))
        run("lm_head_q8_0_248320x2560_b1",
            lambda: wl_lm_head(ctx, 1, 10, max(10, K // 2), graph, "Q8_0", 248320, 2560))
        # the token sampler on the reference model's vocabulary: the default
        # policy (top-k 20, top-p 0.95), the whole vocabulary (top-k off,
        # top-p 1: every sum walks 248,320 ids), and the fused LM head +
        # sampler on its Q8_0 248320 x 2560 head
        run("sample_default_248320",
            lambda: wl_sample(ctx, {"temperature": 1.0, "top_k": 20, "top_p": 0.95}, 5,
                              max(10, K // 4)))
        run("sample_full_vocab_248320",
            lambda: wl_sample(ctx, {"temperature": 1.0, "top_k": 0, "top_p": 1.0}, 2, 10))
        run("lm_head_sample_q8_0_248320x2560",
            lambda: wl_sample(ctx, {"temperature": 1.0, "top_k": 20, "top_p": 0.95}, 5,
                              max(10, K // 4), lm=("Q8_0", 2560)))
        run("moe_prefill_512", lambda: wl_moe(ctx, 512, 2, max(3, K // 20), graph, cache))
        run("moe_prefill_512_2560x640",
            lambda: wl_moe(ctx, 512, 1, max(3, K // 40), graph, cache, "2560x640"))
        run("moe_decode_1tok_2560x640",
            lambda: wl_moe(ctx, 1, W, K, graph, cache, "2560x640"))
        run("moe_block_decode_1tok_4x2560",
            lambda: wl_moe(ctx, 1, W, K, graph, cache, "2560x640", block=True))
        run("moe_block_prefill_512_4x2560",
            lambda: wl_moe(ctx, 512, 1, max(3, K // 40), graph, cache, "2560x640", block=True))
        # the reference model's layer 2 (Q5_K gate/up, Q8_0 routed down)
        run("moe_prefill_512_2560x640_l2",
            lambda: wl_moe(ctx, 512, 1, max(3, K // 40), graph, cache, "2560x640_l2"))
        run("moe_decode_1tok_2560x640_l2",
            lambda: wl_moe(ctx, 1, W, K, graph, cache, "2560x640_l2"))
        if "hbm_copy_64mb" in names:
            run("hbm_copy_64mb", lambda: wl_copy(ctx, 64 << 20, W, K, graph))
    head = work.get(HEADLINE)
    cpus = host_cpus()
    threads = int(os.environ.get("KQ_CPU_THREADS", cpus["usable"]))
    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline ...", file=sys.stderr, flush=True)
        t0 = time.time()
        cpu = cpu_baseline(threads)
        print(f"[bench] cpu baseline done in {time.time() - t0:.1f}s: {json.dumps(cpu)}",
              file=sys.stderr, flush=True)
    line = {
        "metric": "quant matvec HBM GB/s (% of ~8 TB/s peak); MoE-layer decode tokens/s",
        "value": round(head["GBps"], 2) if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(head["ms_per_step"], 6) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, fp32 activations/accumulation",
        "data": "synthetic (seeded SplitMix64 GGUF blocks, N(0,1) activations)",
        "config": {"workload": HEADLINE, "rows": 4096, "cols": 2048, "batch": 1,
                   "format": "Q4_K", "timing": "hip graph of K launches, hip events" if graph
                   else "K stream launches behind a hold kernel, hip events"},
        "hbm_frac": round(head["hbm_frac"], 4) if head else None,
        "moe_decode_tokens_per_s": round(work["moe_decode_1tok"]["tokens_per_s"], 1)
        if "moe_decode_1tok" in work else None,
        "roofline": None,
        "cpu_baseline": None,
        "workloads": work,
    }
    if head:
        # achieved: algorithmic bytes per launch / the kernel's traced mean
        # duration in the committed profile of this command (rocprofv3
        # --kernel-trace); traffic: FETCH_SIZE + WRITE_SIZE per dispatch from
        # the counter runs of the same profile. The HIP-event figures of this
        # run sit beside it: the spacing of back-to-back launches (the
        # throughput `value` reports) and the duration of one launch between
        # its own pair of events.
        prof = profile_figures(HEADLINE)
        traced_us = prof.get("traced_avg_ns", 0) / 1e3 if prof else 0.0
        kern_us = traced_us if traced_us > 0 else head["ms_per_step"] * 1e3
        achieved = head["bytes_per_step"] / (kern_us * 1e3)
        line["roofline"] = {"bound": "hbm", "achieved": round(achieved, 2),
                            "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(achieved / HBM_PEAK_GBS, 4),
                            "traffic": prof.get("hbm_bytes_per_launch") if prof else None,
                            "kernel_us": round(kern_us, 3),
                            "time_source": ("rocprofv3 kernel trace, mean duration of the kernel "
                                            "(profiles/q4k_matvec_4096x2048_b1.md)"
                                            if traced_us > 0 else
                                            "hip events (no committed trace)"),
                            "traffic_source": "the same profile's rocprofv3 --pmc FETCH_SIZE and "
                                              "WRITE_SIZE runs, scaled by a 64 MiB copy",
                            "hip_events": {
                                "back_to_back_us": round(head["ms_per_step"] * 1e3, 3),
                                "frac_back_to_back": round(head["hbm_frac"], 4),
                                "one_launch_us": round(head.get("dispatch_ms", 0.0) * 1e3, 3)}}
        floors = {k: work[k]["ms_per_step"] * 1e3 for k in ("floor_empty_launch",
                                                             "floor_read_4718592b") if k in work}
        if floors:
            line["roofline"]["floors_us"] = {k: round(v, 3) for k, v in floors.items()}
    if cpu:
        key = f"q4k_matvec_{threads}t"
        line["cpu_baseline"] = {"value": round(cpu[key]["GBps"], 4), "unit": "GB/s",
                                "cores": threads, "kind": "port",
                                "sample": "the same 4096x2048 Q4_K matvec, median of repeated "
                                          "full runs (C oracle, reference fp flags, row-parallel "
                                          f"OpenMP over {threads} threads = the CPUs this process "
                                          "may use); also one MoE decode step and one LM-head "
                                          "step at 1 and that many threads",
                                "host": cpus, "runs": cpu}
        # GPU speed-up over the CPU baseline at `threads` threads, per case
        sp = {}
        for gk, ck in (("moe_decode_1tok", f"moe_decode_{threads}t"),
                       ("lm_head_q6k_151936x2048_b1", f"lm_head_b1_{threads}t"),
                       (HEADLINE, f"q4k_matvec_{threads}t")):
            if gk in work and ck in cpu:
                sp[gk] = round(cpu[ck]["s_per_step"] * 1e3 / work[gk]["ms_per_step"], 1)
        line["cpu_baseline"]["gpu_speedup_at_cores"] = sp
    print(json.dumps(line))
    return 0


def profile_figures(workload: str) -> dict:
    """The committed profile figures of a workload (profiles/traffic.json):
    traced mean kernel duration and HBM bytes per launch."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return {}
    try:
        return json.loads(p.read_text()).get(workload, {})
    except (ValueError, OSError):
        return {}


if __name__ == "__main__":
    sys.exit(main())
