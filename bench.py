"""Benchmark of the one-Qwen-layer hot path on one MI355X.

Default workload (the BASELINE metric's configuration, configs[1]): a full
Qwen2.5-0.5B-shaped layer decoding one token at context 1024.  One step =
one layer decode of one token.  Inputs are synthetic (seeded N(0,0.02)
weights -> Q4_0, N(0,1) activations and fp16 KV) and resident in HBM before
the timed region.  The step cycles through enough distinct copies of the
layer (weights + KV cache) to exceed the 256 MB Infinity Cache, so the
reported GB/s is HBM traffic, not cache hits: with fewer steps than copies,
the timed HIP graphs start at staggered copies and are replayed in turn, so
every copy is visited before any is reused.  Each figure is the median over
at least five timed replays, with their min and max.

The JSON line's "roofline" is the time-dominant kernel of that step (and
"roofline_second" the kernel moving the most bytes), each timed by HIP
events attached to its own dispatches; "configs" carries every BASELINE
configuration (1 QKV mat-vec, 2 the decode layer, 3 and 4 the 0.5B and 7B
prefills, 5 the 7B batched decode) with its dominant kernel's roofline and
a CPU baseline: the oracle's C restatement of the reference's portable path
on one pinned host core, each a bounded sample stated in the line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
    python bench.py --profile N     # configuration N's GPU legs only (rocprofv3)
"""
import argparse
import ctypes
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "simple-inference_amd"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA, TOP/s
MALL_BYTES = 256 << 20      # Infinity Cache
METRIC = "decode layer µs + HBM GB/s; prefill tokens/s + int8 MFMA % (one GPU)"
# HBM bytes per launch of a configuration's kernels, from two rocprofv3
# --pmc runs of `bench.py --profile N` (FETCH_SIZE, then WRITE_SIZE, KiB per
# dispatch, medians over the run's dispatches of that kernel), scaled by what
# the counters read for a 256 MiB copy (FETCH_SIZE x2.000, WRITE_SIZE
# x1.000): {(config, kernel): (FETCH_SIZE KiB, WRITE_SIZE KiB, csrc digest)}.
# The digest (csrc_digest()) names the kernel sources the counters were read
# from; a roofline block whose kernel sources have changed since reports its
# traffic with "traffic_current": false.  Kernels not listed report traffic
# null.  Summaries: profiles/cfgN_*.md.
PMC_KIB = {
    ("1", "k_matvec<8, 128, false>"): (330.9, 4.5, "4041115cd2c8"),
    ("2", "k_dec_attn<64, 8, false, false, 1, true>"): (2709.0, 35.5, "4041115cd2c8"),
    ("2", "k_dec_gateup<64, 512, false>"): (2534.9, 9.8, "4041115cd2c8"),
    ("2", "k_dec_wo<8, 512, false>"): (571.6, 3.5, "4041115cd2c8"),
    ("2", "k_matvec<8, 512, false>"): (1256.0, 3.5, "4041115cd2c8"),
    ("3", "k_gemm_f6<2, 2, 1, 2, true>"): (28135.5, 5320.0, "4041115cd2c8"),
    ("4", "k_gemm_f6<2, 2, 2, 2, true>"): (513303.4, 44773.9, "4041115cd2c8"),
    ("5", "k_dec_attn_rows<128, 4, false, false>"): (266837.5, 8192.0, "4041115cd2c8"),
}
FETCH_SCALE, WRITE_SCALE = 2.000, 1.000
_DIGEST = None


def csrc_digest():
    """sha256 (first 12 hex digits) of the HIP sources (csrc/*.hip, *.hpp)."""
    global _DIGEST
    if _DIGEST is None:
        h = hashlib.sha256()
        d = os.path.join(ROOT, "simple-inference_amd", "csrc")
        for f in sorted(os.listdir(d)):
            if f.endswith((".hip", ".hpp")):
                h.update(f.encode())
                with open(os.path.join(d, f), "rb") as fh:
                    h.update(fh.read())
        _DIGEST = h.hexdigest()[:12]
    return _DIGEST


def pmc_traffic(cfg, kernel):
    """(bytes per launch or None, digest the counters were read at or None)."""
    f, w, src = PMC_KIB.get((cfg, kernel), (None, None, None))
    return (None, None) if f is None else (round((f * FETCH_SCALE + w * WRITE_SCALE) * 1024), src)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# synthetic inputs
# ---------------------------------------------------------------------------
def make_layer_tensors(si_amd, shape, seed):
    rng = np.random.default_rng(seed)
    H, QD = shape.hidden, shape.qheads * shape.hdim
    KVD, F = shape.kvheads * shape.hdim, shape.ffn
    q4 = lambda n, k: si_amd.quantize_q4_0(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    return dict(wq=q4(QD, H), wk=q4(KVD, H), wv=q4(KVD, H), wo=q4(H, QD),
                norm=rng.normal(1, 0.1, H).astype(np.float32),
                bq=rng.normal(0, 0.02, QD).astype(np.float32),
                bk=rng.normal(0, 0.02, KVD).astype(np.float32),
                bv=rng.normal(0, 0.02, KVD).astype(np.float32),
                post_norm=rng.normal(1, 0.1, H).astype(np.float32),
                wgate=q4(F, H), wup=q4(F, H), wdown=q4(H, F))


def weight_bytes(shape):
    H, QD, KVD, F = shape.hidden, shape.qheads * shape.hdim, shape.kvheads * shape.hdim, shape.ffn
    q4 = lambda n, k: n * k // 32 * 18
    return q4(QD + 2 * KVD, H) + q4(H, QD) + q4(2 * F, H) + q4(H, F)


def small_bytes(shape):
    """norm gains and QKV bias read once per token."""
    QD, KVD = shape.qheads * shape.hdim, shape.kvheads * shape.hdim
    return 4 * (2 * shape.hidden + QD + 2 * KVD)


def gemm_int_ops(shape, m):
    H, QD, KVD, F = shape.hidden, shape.qheads * shape.hdim, shape.kvheads * shape.hdim, shape.ffn
    return 2 * m * ((QD + 2 * KVD) * H + H * QD + 2 * F * H + H * F)


def graph_time(torch, stream, fn, count, replays=5, offsets=(0,)):
    """Capture fn(o), fn(o + 1), ..., fn(o + count - 1) into one HIP graph per
    offset o on `stream`; replay each graph once to warm up, then `replays`
    times in turn (graph r % len(offsets)), each replay timed alone with HIP
    events recorded on that stream.  Returns ms per fn call: the median over
    the replays ("ms"), their min and max.  The launches are enqueued by C
    code through ctypes; replaying a graph removes the host-side issue cost,
    so the events time the GPU work."""
    graphs = []
    for o in offsets:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(count):
                fn(o + i)
        graphs.append(g)
    per = []
    with torch.cuda.stream(stream):
        for g in graphs:
            g.replay()
        stream.synchronize()
        t = Timer(torch, stream)
        for r in range(replays):
            t.start()
            graphs[r % len(graphs)].replay()
            per.append(t.stop_ms() / count)
    torch.cuda.synchronize()
    del graphs
    return dict(ms=float(np.median(per)), min=float(np.min(per)), max=float(np.max(per)),
                replays=replays, graphs=len(offsets), steps_per_replay=count)


def spread_us(gt):
    """The replay statistics of graph_time in microseconds per step."""
    return {"median": round(gt["ms"] * 1e3, 3), "min": round(gt["min"] * 1e3, 3),
            "max": round(gt["max"] * 1e3, 3), "replays": gt["replays"]}


def kernel_sequence(si_amd, fn, kernel_filter, capacity=16384):
    """[(kernel, us)] in launch order: per-dispatch durations of the kernels
    fn() launches whose names match kernel_filter (HIP events attached to
    each dispatch by si_kernel_timing_*, on the stream it is launched on)."""
    return [(n, ms * 1e3) for n, ms in si_amd.kernel_times_ms(kernel_filter, fn, capacity)]


def kernel_durations(si_amd, fn, kernel_filter, capacity=16384):
    """{kernel: [us, ...]} of kernel_sequence."""
    out = {}
    for name, us in kernel_sequence(si_amd, fn, kernel_filter, capacity):
        out.setdefault(name, []).append(us)
    return out


def roofline_entry(kernel, us, work, bound, cfg, launches):
    """One roofline block: work per launch (bytes for "hbm", int ops for
    "mfma") over the kernel's mean per-dispatch duration."""
    if bound == "hbm":
        achieved, peak, unit = work / (us * 1e-6) / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = work / (us * 1e-6) / 1e12, INT8_PEAK_TOPS, "TOP/s"
    traffic, src = pmc_traffic(cfg, kernel)
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic,
            "traffic_src": src, "traffic_current": None if src is None else src == csrc_digest(),
            "kernel": kernel, "kernel_us": round(us, 3), "launches": launches,
            ("alg_bytes_per_launch" if bound == "hbm" else "int_ops_per_launch"): int(work),
            "timing": "mean of per-dispatch HIP events (si_kernel_timing_*)"}


DECODE_PHASES = ["qkv", "attention", "out_proj", "gate_up", "down"]
# a small layer projects Q|K|V inside its attention kernel (k_dec_attn<..., true>)
DECODE_PHASES_FUSED = ["qkv_attention", "out_proj", "gate_up", "down"]


def decode_kernel_work(s, ctx, nseq=1):
    """Algorithmic bytes per launch of the decode layer's kernels by phase
    (k_dec_qkv; k_dec_attn / k_dec_attn_rows; W_O: k_dec_wo or k_matvec;
    k_dec_gateup; k_matvec for down): weights, the cache rows attention must
    read, the new K/V rows, activation rows in and out, norm gains and
    biases.  Partial states of a split context are implementation traffic,
    not counted."""
    H, QD, KVD, F = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim, s.ffn
    NQKV = QD + 2 * KVD
    q4 = lambda n, k: n * k // 32 * 18  # noqa: E731
    q8 = lambda k: k + (k // 32) * 4  # noqa: E731  values, fp16 scale, int16 sum
    work = {
        "qkv": q4(NQKV, H) + nseq * (H * 4) + H * 4 + NQKV * 4 + nseq * NQKV * 4,
        "attention": nseq * ((ctx - 1) * KVD * 2 * 2 + KVD * 2 * 2 + NQKV * 4 + QD * 4)
                     + s.hdim * 4,
        "out_proj": q4(H, QD) + nseq * (QD * 4 + H * 4 + H * 4),
        "gate_up": q4(2 * F, H) + nseq * (H * 4 + q8(F)) + H * 4,
        "down": q4(H, F) + nseq * (q8(F) + H * 4 + H * 4),
    }
    # the fused kernel: both, without the q|k|v row written and read back
    work["qkv_attention"] = work["qkv"] + work["attention"] - 2 * nseq * NQKV * 4
    return work


class _DevArray:
    def __init__(self, addr, count, typestr):
        self.__cuda_array_interface__ = {"shape": (count,), "typestr": typestr,
                                         "data": (int(addr), False), "version": 2}


def si_amd_view(torch, addr, count, dtype):
    """torch tensor aliasing a device buffer owned by the library."""
    typestr = {torch.uint8: "|u1", torch.int16: "<i2", torch.float32: "<f4"}[dtype]
    return torch.as_tensor(_DevArray(addr, count, typestr), device="cuda")


class Timer:
    """HIP events on a given torch stream."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream
        self.a = torch.cuda.Event(enable_timing=True)
        self.b = torch.cuda.Event(enable_timing=True)

    def start(self):
        self.a.record(self.stream)

    def stop_ms(self):
        self.b.record(self.stream)
        self.b.synchronize()
        return self.a.elapsed_time(self.b)


# ---------------------------------------------------------------------------
# configurations
# ---------------------------------------------------------------------------
def bench_decode_layer(torch, si_amd, stream, steps, warmup, ctx=1024, shape_name="0.5b"):
    """BASELINE config 2 (default workload); with shape_name="7b" the same
    single-token decode step of a Qwen2.5-7B-shaped layer."""
    s = si_amd.make_shape(**si_amd.SHAPES[shape_name])
    tens = make_layer_tensors(si_amd, s, 1)
    kvd = s.kvheads * s.hdim
    per_copy = weight_bytes(s) + 2 * ctx * kvd * 2 + small_bytes(s)
    copies = int(np.ceil(1.25 * MALL_BYTES / per_copy))
    gen = torch.Generator(device="cuda").manual_seed(3)
    layers, caches = [], []
    ws = si_amd.Workspace(s, 1, ctx)  # one workspace for all layers, as in a model
    for _ in range(copies):
        layers.append(si_amd.Layer(s, tens, workspace=ws))
        kc = torch.randn(ctx * kvd, generator=gen, device="cuda").half()
        vc = torch.randn(ctx * kvd, generator=gen, device="cuda").half()
        caches.append((kc, vc))
    x = torch.randn(s.hidden, generator=gen, device="cuda")
    out = torch.empty(s.hidden, device="cuda")
    sh = si_amd.stream_handle(stream)
    L = si_amd.lib()

    def step(i):
        lay = layers[i % copies]
        kc, vc = caches[i % copies]
        rc = L.si_layer_decode(lay.h, si_amd.ptr(x), si_amd.ptr(kc), si_amd.ptr(vc), ctx,
                               si_amd.ptr(out), si_amd.SI_LAYER_FULL,
                               si_amd.stream_handle(torch.cuda.current_stream()))
        if rc:
            raise si_amd.SiError(rc, L.si_last_error().decode())

    with torch.cuda.stream(stream):
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        # eager: one C call per step from Python (host launch cost included)
        t = Timer(torch, stream)
        t.start()
        for i in range(steps):
            step(i)
        eager_ms = t.stop_ms() / steps
        torch.cuda.synchronize()
        # per-phase breakdown (events between stages, eager), averaged
        layers[0].set_timing(True)
        acc = {}
        for i in range(20):
            step(i * copies)  # copy 0 (timing enabled)
            for k, v in layers[0].phase_ms().items():
                acc[k] = acc.get(k, 0.0) + v / 20
        layers[0].set_timing(False)
        torch.cuda.synchronize()
        # per-dispatch durations of the step's kernels over whole rotations
        # of the copies (every copy visited, about 200 steps), by position in
        # the step
        nk = copies * max(1, 200 // copies)
        seq = kernel_sequence(si_amd, lambda: [step(i) for i in range(nk)],
                              "k_dec_|k_matvec<")
        torch.cuda.synchronize()
    phases = DECODE_PHASES_FUSED if len(seq) == len(DECODE_PHASES_FUSED) * nk else DECODE_PHASES
    per = len(phases)
    assert len(seq) == per * nk, f"{len(seq)} timed launches for {nk} steps"
    kern = {ph: (seq[j][0], [us for _, us in seq[j::per]]) for j, ph in enumerate(phases)}
    # timed region: exactly `steps` decode steps per replay, one HIP graph per
    # starting copy; with fewer steps than copies the graphs start `steps`
    # copies apart and are replayed in turn, so consecutive replays walk the
    # whole rotation and a copy is reused only after every other copy
    # (copies x per_copy bytes, 1.25 x the Infinity Cache) has been touched
    ngraphs = 1 if steps >= copies else -(-copies // steps)
    offsets = [(j * steps) % copies for j in range(ngraphs)]
    gt = graph_time(torch, stream, step, steps, replays=max(5, 2 * ngraphs), offsets=offsets)
    ms = gt["ms"]
    alg = per_copy
    kus = {ph: float(np.mean(v)) for ph, (n, v) in kern.items()}
    res = dict(us=ms * 1e3, gbs=alg / (ms * 1e-3) / 1e9, alg_bytes=alg, copies=copies,
               spread_us=spread_us(gt),
               rotation={"copies": copies, "bytes_per_copy": per_copy,
                         "graphs": ngraphs, "steps_per_replay": steps,
                         "copies_per_replay": min(steps, copies),
                         "bytes_between_reuse_of_a_copy": copies * per_copy,
                         "infinity_cache_bytes": MALL_BYTES},
               eager_us=eager_ms * 1e3,
               phases_us_eager={k: round(v * 1e3, 2) for k, v in acc.items()},
               kernels={ph: {"kernel": n, "us": round(kus[ph], 3), "launches": len(v)}
                        for ph, (n, v) in kern.items()},
               kernels_sum_us=round(sum(kus.values()), 3),
               step_minus_kernels_us=round(ms * 1e3 - sum(kus.values()), 3))
    return res, (layers, caches, s, x, ws)


def decode_rooflines(res, s, ctx, cfg, nseq=1):
    """Roofline blocks of a decode run's kernels by phase, the time-dominant
    one first."""
    work = decode_kernel_work(s, ctx, nseq)
    out = []
    for ph, k in sorted(res["kernels"].items(), key=lambda kv: -kv[1]["us"]):
        e = roofline_entry(k["kernel"], k["us"], work[ph], "hbm", cfg, k["launches"])
        e["phase"] = ph
        out.append(e)
    return out


def bench_qkv_gemv(torch, si_amd, stream, launches=1000):
    """fused QKV mat-vec, K=896 N=1152, one token."""
    from_seed = np.random.default_rng(11)
    n, k = 1152, 896
    w = si_amd.quantize_q4_0(from_seed.normal(0, 0.02, (n, k)).astype(np.float32))
    L = si_amd.lib()
    sh = si_amd.stream_handle(stream)
    per = n * k // 32 * 18
    copies = int(np.ceil(1.25 * MALL_BYTES / per))
    wdev = torch.from_numpy(w).cuda()
    mats = []
    tile = L.si_q4_tile(n, k)
    for _ in range(copies):
        qs = torch.empty(n * k // 2, dtype=torch.uint8, device="cuda")
        d = torch.zeros(L.si_q4_scale_count(n, k, tile), dtype=torch.int16, device="cuda")
        si_amd.call("si_q4_repack", si_amd.ptr(wdev), n, k, tile, si_amd.ptr(qs), si_amd.ptr(d),
                    sh)
        mats.append((qs, d))
    x = torch.randn(k, device="cuda")
    xq = torch.empty(k, dtype=torch.int8, device="cuda")
    xd = torch.empty(k // 32, dtype=torch.int16, device="cuda")
    xs = torch.empty(k // 32, dtype=torch.int16, device="cuda")
    si_amd.call("si_quantize_q8_rows", si_amd.ptr(x), 1, k, si_amd.ptr(xq), si_amd.ptr(xd),
                si_amd.ptr(xs), sh)
    bias = torch.randn(n, device="cuda") * 0.02
    out = torch.empty(n, device="cuda")

    def launch(i):
        qs, d = mats[i % copies]
        rc = L.si_matvec_q4q8(si_amd.ptr(qs), si_amd.ptr(d), tile, n, k, si_amd.ptr(xq),
                              si_amd.ptr(xd), si_amd.ptr(xs), si_amd.ptr(bias), None,
                              si_amd.ptr(out), 0,
                              si_amd.stream_handle(torch.cuda.current_stream()))
        if rc:
            raise si_amd.SiError(rc, L.si_last_error().decode())

    with torch.cuda.stream(stream):
        for i in range(50):
            launch(i)
        torch.cuda.synchronize()
        kern = kernel_durations(si_amd, lambda: [launch(i) for i in range(launches)],
                                "k_matvec<")
        torch.cuda.synchronize()
    gt = graph_time(torch, stream, launch, launches, replays=5)
    ms = gt["ms"]
    alg = 586168  # W 580,608 + x 952 + y 4,608 bytes (config 1)
    name, durs = next(iter(kern.items()))
    return dict(us=ms * 1e3, gbs=alg / (ms * 1e-3) / 1e9, copies=copies,
                spread_us=spread_us(gt),
                timing="HIP graph of the launches (us includes the launch-to-launch gap)",
                roofline=roofline_entry(name, float(np.mean(durs)), alg, "hbm", "1", len(durs)))


def bench_gemv_7b(torch, si_amd, stream, launches=200):
    """Qwen2.5-7B decode projections as stand-alone mat-vecs (si_matvec_q4q8,
    k_matvec) on cold weights: the north-star target is >= 70 % of HBM peak.
    Weights are random Q4_0 bytes (values do not affect the timing), copies
    rotated to exceed the Infinity Cache."""
    L = si_amd.lib()
    gen = torch.Generator(device="cuda").manual_seed(12)
    res = {}
    for name, n, k in (("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584),
                       ("down", 3584, 18944)):
        per = n * k // 32 * 18
        copies = int(np.ceil(1.25 * MALL_BYTES / per))
        tile = L.si_q4_tile(n, k)
        mats = []
        for _ in range(copies):
            qs = torch.randint(0, 256, (n * k // 2,), generator=gen, device="cuda",
                               dtype=torch.uint8)
            d = torch.full((L.si_q4_scale_count(n, k, tile),), 0x2000, dtype=torch.int16,
                           device="cuda")
            mats.append((qs, d))
        xq = torch.randint(-127, 128, (k,), generator=gen, device="cuda", dtype=torch.int8)
        xd = torch.full((k // 32,), 0x2c00, dtype=torch.int16, device="cuda")
        xs = xq.view(-1, 32).sum(1, dtype=torch.int32).to(torch.int16)
        out = torch.empty(n, device="cuda")

        def launch(i):
            qs, d = mats[i % copies]
            rc = L.si_matvec_q4q8(si_amd.ptr(qs), si_amd.ptr(d), tile, n, k, si_amd.ptr(xq),
                                  si_amd.ptr(xd), si_amd.ptr(xs), None, None, si_amd.ptr(out), 0,
                                  si_amd.stream_handle(torch.cuda.current_stream()))
            if rc:
                raise si_amd.SiError(rc, L.si_last_error().decode())

        with torch.cuda.stream(stream):
            for i in range(copies + 5):
                launch(i)
        torch.cuda.synchronize()
        ms = graph_time(torch, stream, launch, launches, replays=5)["ms"]
        alg = per + k + (k // 32) * 4 + n * 4
        gbs = alg / (ms * 1e-3) / 1e9
        res[name] = dict(n=n, k=k, tile=tile, us=round(ms * 1e3, 3), gbs=round(gbs, 1),
                         hbm_frac=round(gbs / HBM_PEAK_GBS, 4))
        del mats
        torch.cuda.empty_cache()
    return res


def bench_stream_read(torch, si_amd, stream, sizes_mb=(9, 76, 537), launches=40):
    """The plain streaming-read ceiling (si_stream_read: one pass, 16-byte
    loads, nothing else) at the traffic sizes of the path's kernels: ~9 MB
    (the 0.5B decode layer, a 7B QKV mat-vec), 76 MB (the 7B gate|up
    matrix), 537 MB (config 5's K/V cache).  Buffers are rotated over enough
    copies to exceed the Infinity Cache; each size is swept over grids of
    256 to 8192 workgroups and 4, 8 or 16 loads in flight per thread and
    the best is reported, per launch in a HIP graph (back-to-back) and per
    dispatch (HIP events on the dispatch)."""
    L = si_amd.lib()
    res = {}
    for mb in sizes_mb:
        nbytes = (mb * 1000 * 1000) // 4096 * 4096
        copies = max(1, int(np.ceil(1.25 * MALL_BYTES / nbytes)))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        for b in bufs:
            b.fill_(1)
        sink = torch.empty(8192, dtype=torch.int32, device="cuda")
        best = None
        for wgs, depth in [(w, dp) for w in (256, 512, 1024, 2048, 4096, 8192)
                           for dp in (4, 8, 16)]:
            def launch(i, wgs=wgs, depth=depth):
                si_amd.call("si_stream_read", si_amd.ptr(bufs[i % copies]), nbytes,
                            si_amd.ptr(sink), wgs, depth,
                            si_amd.stream_handle(torch.cuda.current_stream()))
            n = max(launches // 2, copies)
            with torch.cuda.stream(stream):
                for i in range(copies):
                    launch(i)
            torch.cuda.synchronize()
            ms = graph_time(torch, stream, launch, n, replays=5)["ms"]
            with torch.cuda.stream(stream):
                d = kernel_durations(si_amd, lambda: [launch(i) for i in range(n)],
                                     "k_stream_read")
            torch.cuda.synchronize()
            us_d = float(np.mean(next(iter(d.values()))))
            if best is None or ms < best[1]:
                best = (wgs, depth, ms, us_d)
        wgs, depth, ms, us_d = best
        res[f"{mb}MB"] = dict(bytes=nbytes, copies=copies, workgroups=wgs, depth=depth,
                              us_graph=round(ms * 1e3, 3),
                              gbs_graph=round(nbytes / (ms * 1e-3) / 1e9, 1),
                              us_dispatch=round(us_d, 3),
                              gbs_dispatch=round(nbytes / (us_d * 1e-6) / 1e9, 1),
                              hbm_frac_dispatch=round(nbytes / (us_d * 1e-6) / 1e9 /
                                                      HBM_PEAK_GBS, 4))
        del bufs
        torch.cuda.empty_cache()
    return res


def bench_attention_modes(torch, si_amd, shape_name="7b", ctx=4096, count=100):
    """The two attention methods of one decode step (attention_kernels.h:33-78
    and :80-164) on the same query and cache, each call's K/V rotated over
    enough copies to defeat the Infinity Cache: si_attention_standard (scores
    materialized in a [qheads][ctx] buffer, softmax in place, weighted V sum)
    and si_attention (the streaming flash-decoding kernels, Q8 of the output
    included).  Algorithmic bytes: K and V read once per KV group, plus the
    standard method's score buffer (written, read and written by the
    softmax, read by the V sum)."""
    s = si_amd.make_shape(**si_amd.SHAPES[shape_name])
    kvd, QD = s.kvheads * s.hdim, s.qheads * s.hdim
    kv_bytes = 2 * ctx * kvd * 2
    copies = int(np.ceil(1.25 * MALL_BYTES / kv_bytes))
    gen = torch.Generator(device="cuda").manual_seed(11)
    caches = [(torch.randn(ctx * kvd, generator=gen, device="cuda").half(),
               torch.randn(ctx * kvd, generator=gen, device="cuda").half())
              for _ in range(copies)]
    q = torch.randn(QD, generator=gen, device="cuda")
    out = torch.empty(QD, device="cuda")
    scores = torch.empty(s.qheads * ctx, device="cuda")
    wsb = si_amd.lib().si_attention_workspace(ctypes.byref(s), 1, ctx)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    qs = torch.empty(QD, dtype=torch.int8, device="cuda")
    qd = torch.empty(QD // 32, dtype=torch.int16, device="cuda")
    cur = lambda: si_amd.stream_handle(torch.cuda.current_stream())  # noqa: E731

    def standard(i):
        kc, vc = caches[i % copies]
        si_amd.call("si_attention_standard", ctypes.byref(s), si_amd.ptr(q), si_amd.ptr(kc),
                    si_amd.ptr(vc), ctx, si_amd.ptr(out), si_amd.ptr(scores), cur())

    def flash(i):
        kc, vc = caches[i % copies]
        si_amd.call("si_attention", ctypes.byref(s), si_amd.ptr(q), 1, si_amd.ptr(kc),
                    si_amd.ptr(vc), 0, None, ctx, 0, ctx, si_amd.ptr(out), si_amd.ptr(qs),
                    si_amd.ptr(qd), None, si_amd.ptr(ws), wsb, cur())

    stream = torch.cuda.Stream()
    res = {"shape": shape_name, "context": ctx, "kv_copies_rotated": copies}
    score_bytes = 4 * s.qheads * ctx * 4
    for name, fn, alg in (("standard", standard, kv_bytes + score_bytes),
                          ("flash", flash, kv_bytes)):
        with torch.cuda.stream(stream):
            for i in range(4):
                fn(i)
        torch.cuda.synchronize()
        ms = graph_time(torch, stream, fn, count, replays=5)["ms"]
        res[name + "_us"] = round(ms * 1e3, 3)
        res[name + "_gbs"] = round(alg / (ms * 1e-3) / 1e9, 1)
    res["speedup_flash"] = round(res["standard_us"] / res["flash_us"], 3)
    del caches
    torch.cuda.empty_cache()
    return res


def bench_gguf_ingest(torch, si_amd, shape_name="7b", reps=3):
    """GGUF ingest of one layer (si_amd.gguf): a Q4_0 GGUF written to a
    temporary file, then, timed, index + memory map + si_amd.Layer (host to
    device copy and the GPU repack), synchronized.  The file is in the page
    cache (just written): this is the parse + copy + repack rate."""
    import shutil
    import tempfile
    from si_amd import gguf
    sd = dict(si_amd.SHAPES[shape_name])
    s = si_amd.make_shape(**sd)
    tens = make_layer_tensors(si_amd, s, 31)
    tmp = tempfile.mkdtemp()
    try:
        path = os.path.join(tmp, "layer.gguf")
        gguf.write_gguf(path, gguf.layer_meta(sd), gguf.layer_tensors_gguf(sd, tens, layer=0))
        size = os.path.getsize(path)
        best = None
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with gguf.GGUFFile(path) as gf:
                gsd, gt = gguf.load_layer(gf, 0)
                lay = si_amd.Layer(si_amd.make_shape(**gsd), gt, 1, 16)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                lay.close()
                del gt
            best = dt if best is None else min(best, dt)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return dict(shape=shape_name, file_bytes=size, ms=round(best * 1e3, 2),
                gbs=round(size / best / 1e9, 2))


def bench_prefill(torch, si_amd, stream, shape_name, ntok, steps):
    """BASELINE configs 3 (0.5B, 512 tokens) and 4 (7B, 2048 tokens)."""
    s = si_amd.make_shape(**si_amd.SHAPES[shape_name])
    tens = make_layer_tensors(si_amd, s, 5)
    lay = si_amd.Layer(s, tens, ntok, ntok)
    kvd = s.kvheads * s.hdim
    gen = torch.Generator(device="cuda").manual_seed(6)
    x = torch.randn(ntok * s.hidden, generator=gen, device="cuda")
    kc = torch.zeros(ntok * kvd, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    out = torch.empty(ntok * s.hidden, device="cuda")
    def call(i):
        lay.prefill(x, ntok, 0, kc, vc, out, stream=torch.cuda.current_stream(), capture=False)

    with torch.cuda.stream(stream):
        for i in range(2):
            call(i)
        lay.set_timing(True)
        call(0)
        ph = lay.phase_ms()
        lay.set_timing(False)
        torch.cuda.synchronize()
        # every kernel of `reps` prefill calls, per dispatch
        reps = max(2, min(steps, 5))
        kern = kernel_durations(si_amd, lambda: [call(i) for i in range(reps)], "k_")
        torch.cuda.synchronize()
    gt = graph_time(torch, stream, call, steps, replays=5)
    ms = gt["ms"]
    # past 64 rows the layer runs its gate|up GEMM in the fp6 formulation,
    # past 512 all four
    f6 = ntok > 64
    gemm_ms, gu, gu16 = gemm_graph_ms(torch, si_amd, stream, lay, s, ntok, steps, f6)
    ops = gemm_int_ops(s, ntok)
    lay.close()
    cfg = "3" if shape_name == "0.5b" else "4"
    per_call = {k: round(float(np.sum(v)) / reps, 3) for k, v in kern.items()}
    if f6:
        # the layer's own GEMM dispatches and the conversions of their inputs
        # (the ABI's fp6 call would also convert the weights, which the layer
        # does once when built)
        # the graph-timed step times the GEMM dispatches' share of the
        # per-dispatch kernel times (eager per-dispatch times add up to more
        # than a graph replay of the step)
        gsum = sum(v for k, v in per_call.items() if k.startswith(("k_gemm", "k_q8_to_x6")))
        gemm_ms = ms * gsum / sum(per_call.values())
        gemm_timing = ("the step (graph replays) x the share of the layer's GEMM and "
                       "k_q8_to_x6 dispatches in its per-dispatch kernel times")
    else:
        gemm_timing = "the four projections alone, one HIP graph (gemm_graph_ms)"
    # the dominant kernel: the fused gate|up instance the layer dispatched,
    # timed per dispatch inside the layer calls (the roofline), and the same
    # instance launched alone on the layer's buffers (roofline_alone)
    gname = next((k for k in kern if k in gu), None)
    if gname is None:  # not dispatched by the layer: the stand-alone instance
        gname = max(gu, key=lambda k: len(gu[k]))
    gdur = gu[gname]
    gu_ops = 2 * ntok * 2 * s.ffn * s.hidden
    in_layer = kern.get(gname, gdur)
    return dict(ms=ms, tokens_per_s=ntok / (ms * 1e-3), spread_us=spread_us(gt),
                gemm_ms=gemm_ms, gemm_tops=ops / (gemm_ms * 1e-3) / 1e12,
                mfma_pct_gemm=100.0 * ops / (gemm_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                mfma_pct_layer=100.0 * ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS,
                gemm_timing=gemm_timing,
                phases_ms={k: round(v, 4) for k, v in ph.items()},
                kernels_us_per_call=dict(sorted(per_call.items(), key=lambda kv: -kv[1])),
                kernels_sum_us=round(sum(per_call.values()), 3),
                step_minus_kernels_us=round(ms * 1e3 - sum(per_call.values()), 3),
                roofline=dict(roofline_entry(gname, float(np.mean(in_layer)), gu_ops, "mfma",
                                             cfg, len(in_layer)),
                              where="inside the layer calls"),
                roofline_alone=dict(roofline_entry(gname, float(np.mean(gdur)), gu_ops, "mfma",
                                                   cfg, len(gdur)),
                                    where="launched alone on the layer's buffers"),
                gateup_f16_formulation={
                    k16: {"us": round(float(np.mean(v16)), 3),
                          "mfma_frac": round(gu_ops / (float(np.mean(v16)) * 1e-6) / 1e12 /
                                             INT8_PEAK_TOPS, 4),
                          "launches": len(v16),
                          "note": "SI_GEMM_F16, bit-identical results; launched alone"}
                    for k16, v16 in gu16.items()})


def gemm_graph_ms(torch, si_amd, stream, lay, s, m, steps, f6=False):
    """The layer's four projections alone (the same kernels, weights and
    activation buffers a prefill call uses, left valid by it), captured as one
    HIP graph: the GEMM time without per-phase event gaps; and the gate|up
    instance alone, per dispatch (f6: in the fp6 formulation, as the layer
    runs it past 64 rows)."""
    L = si_amd.lib()
    H, F = s.hidden, s.ffn
    W = [lay.weights(i) for i in range(4)]  # QKV, O, gate|up, down
    b = lambda n: ctypes.c_void_p(lay.buffer(n))
    ws_bytes = max(L.si_gemm_workspace(m, w[3], w[4]) for w in W)
    if f6:
        ws_bytes = max(ws_bytes, L.si_gemm_f6_workspace(m, 2 * F, W[2][4]))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
    out = torch.empty(m * H, device="cuda")
    wsp = si_amd.ptr(ws)

    def gemm(w, xq, xd, dst, ldo, res=None):
        qs, d, tile, n, k = w
        si_amd.call("si_gemm_q4q8", ctypes.c_void_p(qs), ctypes.c_void_p(d), tile, n, k,
                    b(xq), b(xd), m, None, res, dst, ldo, 0, wsp, ws_bytes,
                    si_amd.stream_handle(torch.cuda.current_stream()))

    def gateup(flags=0):
        qs, d, tile, n, k = W[2]
        # no gu / act outputs: the layer writes neither without SI_LAYER_CAPTURE
        si_amd.call("si_gemm_gateup_q8", ctypes.c_void_p(qs), ctypes.c_void_p(d), tile, F, k,
                    b("XQ2_QS"), b("XQ2_D"), m, None, None, b("ACTQ_QS"), b("ACTQ_D"),
                    b("ACTQ_S"), flags, wsp, ws_bytes,
                    si_amd.stream_handle(torch.cuda.current_stream()))

    def step(i):
        gemm(W[0], "XQ_QS", "XQ_D", b("QKV"), W[0][3])
        gemm(W[1], "ATTQ_QS", "ATTQ_D", b("ATTN_OUT"), H)
        gateup()
        gemm(W[3], "ACTQ_QS", "ACTQ_D", si_amd.ptr(out), H, b("H"))

    # the gate|up GEMM (the prefill's time-dominant kernel) alone, per
    # dispatch; and its f16 formulation (SI_GEMM_F16, bit-identical results)
    with torch.cuda.stream(stream):
        gu_flags = si_amd.SI_GEMM_F6 if f6 else 0
        gu = kernel_durations(si_amd, lambda: [gateup(gu_flags) for _ in range(max(3, steps))],
                              "k_gemm")
        gu16 = kernel_durations(si_amd, lambda: [gateup(si_amd.SI_GEMM_F16)
                                                 for _ in range(max(3, steps))], "k_gemm")
        torch.cuda.synchronize()
    return graph_time(torch, stream, step, steps, replays=5)["ms"], gu, gu16


def bench_batched_decode(torch, si_amd, stream, steps, nseq=64, ctx=4096):
    """7B layer, 64 sequences x 1 token, 4096-position caches."""
    s = si_amd.make_shape(**si_amd.SHAPES["7b"])
    tens = make_layer_tensors(si_amd, s, 7)
    lay = si_amd.Layer(s, tens, nseq, ctx)
    kvd = s.kvheads * s.hdim
    stride = ctx * kvd
    gen = torch.Generator(device="cuda").manual_seed(8)
    kc = torch.randn(nseq * stride, generator=gen, device="cuda").half()
    vc = torch.randn(nseq * stride, generator=gen, device="cuda").half()
    x = torch.randn(nseq * s.hidden, generator=gen, device="cuda")
    out = torch.empty(nseq * s.hidden, device="cuda")
    def call(i):
        lay.decode_batch(x, nseq, kc, vc, stride, ctx, ctx, out,
                         stream=torch.cuda.current_stream(), capture=False)

    with torch.cuda.stream(stream):
        for i in range(2):
            call(i)
        lay.set_timing(True)
        call(0)
        ph = lay.phase_ms()
        lay.set_timing(False)
        torch.cuda.synchronize()
        reps = max(2, min(steps, 5))
        kern = kernel_durations(si_amd, lambda: [call(i) for i in range(reps)], "k_")
        torch.cuda.synchronize()
    gt = graph_time(torch, stream, call, steps, replays=5)
    ms = gt["ms"]
    alg = weight_bytes(s) + nseq * 2 * ctx * kvd * 2 + small_bytes(s)
    lay.close()
    per_call = {k: round(float(np.sum(v)) / reps, 3) for k, v in kern.items()}
    res = dict(us=ms * 1e3, gbs=alg / (ms * 1e-3) / 1e9, alg_bytes=alg,
               spread_us=spread_us(gt),
               phases_us={k: round(v * 1e3, 2) for k, v in ph.items()},
               kernels_us_per_call=dict(sorted(per_call.items(), key=lambda kv: -kv[1])),
               kernels_sum_us=round(sum(per_call.values()), 3),
               step_minus_kernels_us=round(ms * 1e3 - sum(per_call.values()), 3))
    att = [k for k in kern if k.startswith("k_dec_attn")]
    if att:
        a = att[0]
        res["roofline"] = roofline_entry(a, float(np.mean(kern[a])),
                                         decode_kernel_work(s, ctx, nseq)["attention"],
                                         "hbm", "5", len(kern[a]))
    return res


def bench_paged_decode(torch, si_amd, stream, steps, nseq=64, ctx=4096, page_size=64,
                       nlayers=2):
    """Batched decode of BASELINE config 5's shape (7B layer, 64 sequences,
    4096 positions) with the K/V rows in a paged pool (pages shuffled, so no
    sequence is contiguous), per layer, next to the same call on contiguous
    caches; then a decode step of an nlayers-deep stack (libsi_host.so
    si_stack_*: one page table for every layer, residual stream between
    layers)."""
    s = si_amd.make_shape(**si_amd.SHAPES["7b"])
    tens = make_layer_tensors(si_amd, s, 7)
    lay = si_amd.Layer(s, tens, nseq, ctx)
    kvd = s.kvheads * s.hdim
    max_pages = ctx // page_size
    npages = nseq * max_pages
    gen = torch.Generator(device="cuda").manual_seed(9)
    kp = torch.randn(npages * page_size * kvd, generator=gen, device="cuda").half()
    vp = torch.randn(npages * page_size * kvd, generator=gen, device="cuda").half()
    perm = np.random.default_rng(5).permutation(npages).astype(np.int32)
    table = torch.from_numpy(perm.reshape(nseq, max_pages)).cuda()
    ctx_dev = torch.full((nseq,), ctx, dtype=torch.int32, device="cuda")
    x = torch.randn(nseq * s.hidden, generator=gen, device="cuda")
    out = torch.empty(nseq * s.hidden, device="cuda")

    def call(i):
        lay.decode_paged(x, nseq, kp, vp, npages, page_size, table, max_pages, ctx_dev, ctx, out,
                         stream=torch.cuda.current_stream(), capture=False)

    with torch.cuda.stream(stream):
        for i in range(2):
            call(i)
        lay.set_timing(True)
        call(0)
        ph = lay.phase_ms()
        lay.set_timing(False)
    torch.cuda.synchronize()
    ms = graph_time(torch, stream, call, steps, replays=5)["ms"]
    alg = weight_bytes(s) + nseq * 2 * ctx * kvd * 2 + small_bytes(s)
    lay.close()
    del kp, vp
    torch.cuda.empty_cache()
    res = dict(page_size=page_size, us=round(ms * 1e3, 2),
               gbs=round(alg / (ms * 1e-3) / 1e9, 1), alg_bytes=alg,
               phases_us={k: round(v * 1e3, 2) for k, v in ph.items()})
    # the stack: nlayers layers, sequences filled to ctx - 1 positions, one step
    H = si_amd.host_lib()
    keep = [dict((k, np.ascontiguousarray(v)) for k, v in tens.items() if v is not None)
            for _ in range(nlayers)]
    hosts = (si_amd.LayerHost * nlayers)(
        *[si_amd.LayerHost(**{k: v.ctypes.data for k, v in kk.items()}) for kk in keep])
    st = H.si_stack_create(ctypes.byref(s), ctypes.cast(hosts, ctypes.c_void_p), nlayers, nseq,
                           ctx, npages, page_size)
    pg = H.si_stack_pages(st)
    ids = [H.si_kv_seq_add(pg) for _ in range(nseq)]
    for i in ids:
        assert H.si_kv_seq_grow(pg, i, ctx - 1) == 0
    arr = (ctypes.c_int * nseq)(*ids)
    assert H.si_stack_prepare(st, arr, nseq) == 0
    sh = lambda: si_amd.stream_handle(torch.cuda.current_stream())  # noqa: E731

    def step(i):
        H.si_stack_decode(st, si_amd.ptr(x), si_amd.ptr(out), si_amd.SI_LAYER_FULL, sh())

    with torch.cuda.stream(stream):
        step(0)
    torch.cuda.synchronize()
    ms_s = graph_time(torch, stream, step, max(1, steps // 2), replays=5)["ms"]
    H.si_stack_destroy(st)
    res.update(stack_layers=nlayers, stack_step_us=round(ms_s * 1e3, 2),
               stack_us_per_layer=round(ms_s * 1e3 / nlayers, 2))
    return res


# ---------------------------------------------------------------------------
# CPU baselines: the oracle (C restatement of the reference's portable path,
# oracle/libsi_oracle.so built -O2 -ffp-contract=off as the reference's
# Makefile:7), one pinned host core, medians after a warm-up call
# (audit_fusion_timing.c:65-74, :272-317)
# ---------------------------------------------------------------------------
def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


class _Pinned:
    """Runs the block on the first core this process may use."""

    def __enter__(self):
        self.old = os.sched_getaffinity(0)
        self.core = sorted(self.old)[0]
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *a):
        os.sched_setaffinity(0, self.old)


def _median_time(fn, budget_s, max_n=2000, min_n=1, warm=True):
    if warm:
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_n or (time.perf_counter() < t_end and len(times) < max_n):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def _oracle_inputs(si_amd, name, ctx, seed):
    from oracle.oracle_py import Oracle, make_shape as or_shape
    o = Oracle()
    sd = si_amd.SHAPES[name]
    s = or_shape(**sd)
    tens = make_layer_tensors(si_amd, si_amd.make_shape(**sd), seed)
    rng = np.random.default_rng(3)
    kvd = s.kvheads * s.hdim
    kc = o.f32_to_f16(rng.standard_normal(ctx * kvd).astype(np.float32))
    vc = o.f32_to_f16(rng.standard_normal(ctx * kvd).astype(np.float32))
    return o, s, tens, kc, vc, rng


def cpu_baselines(si_amd, budget_s=10.0):
    """Per-configuration CPU legs, each a bounded sample (stated in "sample")
    in the unit of that configuration's GPU figure."""
    cpu = _cpu_name()
    common = f"oracle/libsi_oracle.so (-O2 -ffp-contract=off), 1 pinned core of '{cpu}'"
    out = {}
    with _Pinned() as pin:
        where = f"core {pin.core}; {common}"
        # config 2: full 0.5B layer decode at context 1024
        o, s, tens, kc, vc, rng = _oracle_inputs(si_amd, "0.5b", 1024, 1)
        x = rng.standard_normal(s.hidden).astype(np.float32)
        med, n = _median_time(lambda: o.layer_decode(s, tens, x, kc, vc, 1024), budget_s)
        sh = si_amd.make_shape(**si_amd.SHAPES["0.5b"])
        alg = weight_bytes(sh) + 2 * 1024 * s.kvheads * s.hdim * 2 + small_bytes(sh)
        out["2"] = dict(value=alg / med / 1e9, unit="GB/s", cores=1, kind="port",
                        us_per_token=med * 1e6,
                        sample=f"{n} layer decodes at context 1024, median {med * 1e3:.2f} "
                               f"ms/token; {where}")
        # config 1: the QKV mat-vec (K 896, N 1152) alone
        wqkv = np.concatenate([tens["wq"].reshape(-1), tens["wk"].reshape(-1),
                               tens["wv"].reshape(-1)])
        bias = np.concatenate([tens["bq"], tens["bk"], tens["bv"]])
        xq = o.quantize_q8(x)
        med, n = _median_time(lambda: o.matvec(wqkv, xq, 896, 1152, bias), budget_s / 4)
        out["1"] = dict(value=586168 / med / 1e9, unit="GB/s", cores=1, kind="port",
                        us=med * 1e6,
                        sample=f"{n} matvec_q4q8 calls (K 896, N 1152), median "
                               f"{med * 1e6:.1f} us; {where}")
        # config 3: 0.5B prefill of 512 tokens, in full
        x3 = rng.standard_normal(512 * s.hidden).astype(np.float32)
        kc3 = np.zeros(512 * s.kvheads * s.hdim, np.uint16)
        vc3 = np.zeros_like(kc3)
        med, n = _median_time(lambda: o.layer_prefill(s, tens, x3, 512, 0, kc3, vc3), 0.0,
                              warm=False)
        out["3"] = dict(value=512 / med, unit="tokens/s", cores=1, kind="port",
                        s_per_prefill=med,
                        sample=f"{n} full 512-token prefill{'s' if n > 1 else ''}, "
                               f"{'median ' if n > 1 else ''}{med:.2f} s; {where}")
        del o, tens, kc, vc, kc3, vc3
        # configs 4 and 5: the 7B layer
        o, s, tens, kc, vc, rng = _oracle_inputs(si_amd, "7b", 4096, 5)
        H, KVD = s.hidden, s.kvheads * s.hdim
        # config 4 (2048-token prefill): K/V of 256 tokens, one token's full
        # row, attention at context 2048, extrapolated linearly
        x4 = rng.standard_normal(256 * H).astype(np.float32)
        empty = np.zeros(0, np.int32)
        t_kv, _ = _median_time(lambda: o.layer_prefill(s, tens, x4, 256, 0, kc, vc, rows=empty),
                               0.0, warm=False)
        t_row, _ = _median_time(lambda: o.layer_prefill(s, tens, x4[:H], 1, 0, kc, vc,
                                                        rows=np.zeros(1, np.int32)), 0.0,
                                min_n=3)
        q = rng.standard_normal(s.qheads * s.hdim).astype(np.float32)
        t_att, _ = _median_time(lambda: o.attention_flash(s, q, kc, vc, 2048), 0.0, min_n=5)
        t_row_proj = t_row - t_kv / 256  # the single token's own K/V is in t_kv
        total = 8 * t_kv + 2048 * t_row_proj + t_att * 2049 / 2
        out["4"] = dict(value=2048 / total, unit="tokens/s", cores=1, kind="port",
                        s_per_prefill_extrapolated=total,
                        sample=f"measured: K/V of 256 tokens {t_kv:.2f} s, one token's full "
                               f"row {t_row * 1e3:.0f} ms, attention at context 2048 "
                               f"{t_att * 1e3:.1f} ms; extrapolated to 2048 tokens as 8 x "
                               f"K/V(256) + 2048 x row + attention(2048) x 2049/2 (projections "
                               f"exactly linear in tokens, attention linear in context); "
                               f"{where}")
        # config 5 (64 sequences x context 4096): 16 of the 64 single-token
        # decodes (independent sequences: x4)
        x5 = rng.standard_normal(H).astype(np.float32)
        o.layer_decode(s, tens, x5, kc, vc, 4096)  # warm-up
        t0 = time.perf_counter()
        for _ in range(16):
            o.layer_decode(s, tens, x5, kc, vc, 4096)
        t16 = time.perf_counter() - t0
        sh7 = si_amd.make_shape(**si_amd.SHAPES["7b"])
        alg5 = weight_bytes(sh7) + 64 * 2 * 4096 * KVD * 2 + small_bytes(sh7)
        out["5"] = dict(value=alg5 / (4 * t16) / 1e9, unit="GB/s", cores=1, kind="port",
                        us_per_step_extrapolated=4 * t16 * 1e6,
                        sample=f"16 of the 64 sequences' decodes at context 4096 in "
                               f"{t16:.2f} s, x4 for the 64-sequence step (sequences are "
                               f"independent); {where}")
    return out


# ---------------------------------------------------------------------------
WORKLOADS = {
    "1": "fused QKV Q4_0 x Q8_0 mat-vec, 1 token, 0.5B shape (K 896, N 1152)",
    "2": "full Qwen2.5-0.5B-shaped layer, decode of 1 token at context 1024",
    "3": "Qwen2.5-0.5B-shaped layer, prefill of 512 tokens",
    "4": "Qwen2.5-7B-shaped layer, prefill of 2048 tokens",
    "5": "Qwen2.5-7B-shaped layer, batched decode of 64 sequences x 1 token at context 4096",
}


def run_config(cfg, torch, si_amd, stream, steps, warmup):
    """One BASELINE configuration's GPU figures and roofline block."""
    if cfg == "1":
        r = bench_qkv_gemv(torch, si_amd, stream)
        r["hbm_frac"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
        return r
    if cfg == "2":
        r, held = bench_decode_layer(torch, si_amd, stream, steps, warmup)
        s = si_amd.make_shape(**si_amd.SHAPES["0.5b"])
        roofs = decode_rooflines(r, s, 1024, "2")
        r["roofline"] = roofs[0]
        r["kernel_rooflines"] = roofs
        r["hbm_frac"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
        for lay in held[0]:
            lay.close()
        held[4].close()
        return r
    if cfg in ("3", "4"):
        name, ntok = ("0.5b", 512) if cfg == "3" else ("7b", 2048)
        return bench_prefill(torch, si_amd, stream, name, ntok, 10 if cfg == "3" else 3)
    r = bench_batched_decode(torch, si_amd, stream, 5)
    r["hbm_frac"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--quick", action="store_true", help="configuration 2 and the 7B decode only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--profile", choices=sorted(WORKLOADS),
                    help="run one configuration's GPU legs only (for rocprofv3)")
    ap.add_argument("--only", choices=["gguf-7b", "attention-7b", "paged-7b", "decode-7b",
                                       "stream-read"],
                    help="run one of the other measurements only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py --gpus {args.gpus}: this build runs on one GPU only; "
              "the path is measured on one GPU's share and no multi-GPU run exists.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import si_amd
    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    if args.only:
        if args.only == "gguf-7b":
            r = bench_gguf_ingest(torch, si_amd)
        elif args.only == "attention-7b":
            r = bench_attention_modes(torch, si_amd)
        elif args.only == "paged-7b":
            r = bench_paged_decode(torch, si_amd, stream, 5)
        elif args.only == "stream-read":
            r = bench_stream_read(torch, si_amd, stream)
        else:
            r, _ = bench_decode_layer(torch, si_amd, stream, 100, 10, ctx=4096, shape_name="7b")
        print(json.dumps({"only": args.only, **r}), flush=True)
        return
    if args.profile:
        steps = min(args.steps, 100)
        r = run_config(args.profile, torch, si_amd, stream, steps, min(args.warmup, 10))
        print(json.dumps({"profile": args.profile, **r}), flush=True)
        return
    t0 = time.time()
    configs = {}
    log("config 2: 0.5B decode layer, ctx 1024 ...")
    dec = run_config("2", torch, si_amd, stream, args.steps, args.warmup)
    configs["2"] = dec
    log(f"  {dec['us']:.2f} us/token, {dec['gbs']:.1f} GB/s; kernels {dec['kernels']} "
        f"({time.time() - t0:.0f} s)")
    extra = {}
    log("streaming-read ceiling (si_stream_read) at 9, 76 and 537 MB ...")
    extra["stream_read_ceiling"] = bench_stream_read(torch, si_amd, stream)
    log(f"  {extra['stream_read_ceiling']}")
    log("7B decode projections (k_matvec) ...")
    extra["gemv_7b_cold"] = bench_gemv_7b(torch, si_amd, stream)
    log(f"  {extra['gemv_7b_cold']}")
    log("7B decode layer, ctx 4096 ...")
    d7, held = bench_decode_layer(torch, si_amd, stream, 100, 10, ctx=4096, shape_name="7b")
    for lay in held[0]:
        lay.close()
    held[4].close()
    del held
    s7 = si_amd.make_shape(**si_amd.SHAPES["7b"])
    d7["kernel_rooflines"] = decode_rooflines(d7, s7, 4096, "7b-decode")
    d7["hbm_frac"] = round(d7["gbs"] / HBM_PEAK_GBS, 4)
    extra["decode_7b_ctx4096"] = d7
    log(f"  {d7['us']:.2f} us/token; kernels {d7['kernels']}")
    torch.cuda.empty_cache()
    if not args.quick:
        for cfg in ("1", "3", "4", "5"):
            log(f"config {cfg}: {WORKLOADS[cfg]} ...")
            configs[cfg] = run_config(cfg, torch, si_amd, stream, args.steps, args.warmup)
            log(f"  {configs[cfg]}")
            torch.cuda.empty_cache()
        log("attention methods, 7B-shaped, ctx 4096 ...")
        extra["attention_standard_vs_flash_7b_ctx4096"] = bench_attention_modes(torch, si_amd)
        log(f"  {extra['attention_standard_vs_flash_7b_ctx4096']}")
        log("GGUF ingest, 7B-shaped layer ...")
        extra["gguf_ingest_7b_layer"] = bench_gguf_ingest(torch, si_amd)
        log(f"  {extra['gguf_ingest_7b_layer']}")
        log("config 5 shape over a paged KV pool, and a 2-layer stack ...")
        extra["paged_batched_decode_7b_64x4096"] = bench_paged_decode(torch, si_amd, stream, 5)
        log(f"  {extra['paged_batched_decode_7b_64x4096']}")
    cpu = {}
    if not args.no_cpu:
        log("CPU baselines (oracle, 1 pinned core) ...")
        t1 = time.time()
        cpu = cpu_baselines(si_amd)
        log(f"  {cpu} ({time.time() - t1:.0f} s)")
    gpu_value = {"1": ("gbs", "GB/s"), "2": ("gbs", "GB/s"), "3": ("tokens_per_s", "tokens/s"),
                 "4": ("tokens_per_s", "tokens/s"), "5": ("gbs", "GB/s")}
    for cfg, r in configs.items():
        r["workload"] = WORKLOADS[cfg]
        if cfg in cpu:
            r["cpu_baseline"] = cpu[cfg]
            key, unit = gpu_value[cfg]
            assert cpu[cfg]["unit"] == unit
            r["gpu_over_cpu"] = round(r[key] / cpu[cfg]["value"], 1)
    second = [e for e in dec["kernel_rooflines"] if e["phase"] == "gate_up"]
    line = {
        "metric": METRIC,
        "value": round(dec["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["us"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint4 (fp32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) weights -> Q4_0, N(0,1) activations and fp16 KV)",
        "config": {"workload": WORKLOADS["2"] + " (BASELINE configs[1])",
                   "hidden": 896, "qheads": 14, "kvheads": 2, "head_dim": 64, "ffn": 4864,
                   "context": 1024, "layer_copies_rotated": dec["copies"],
                   "rotation": dec["rotation"], "alg_bytes_per_step": dec["alg_bytes"]},
        "decode_layer_us": round(dec["us"], 3),
        "decode_layer_spread_us": dec["spread_us"],
        "decode_kernels_sum_us": dec["kernels_sum_us"],
        "decode_step_minus_kernels_us": dec["step_minus_kernels_us"],
        "decode_layer_us_eager": round(dec["eager_us"], 3),
        "timing": "median over >= 5 replays of a HIP graph of the K steps (graphs starting at "
                  "staggered layer copies, replayed in turn), HIP events on the bench stream",
        "roofline": dec["roofline"],
        "roofline_second": second[0] if second else None,
        "cpu_baseline": cpu.get("2"),
        "configs": configs,
        "other": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
