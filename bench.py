#!/usr/bin/env python3
"""Benchmark of the fused layer-kernel hot path on one MI355X.

Headline workload (one "step"): the epilogue chain of one T2S decode step for B = 64 sequences,
d_model 512, FFN 2048, 24 layers, fp16 storage / fp32 arithmetic — the decode-input gather +
alpha*PE, then per layer residual+LayerNorm (norm1), bias+ReLU on the FFN activations, residual+
LayerNorm (norm2). The step runs as ONE kernel launch (gsvk_t2s_step_fused: one wave per
sequence walks the row-local LayerNorm chain, the other waves run the ReLU tiles), replayed as a
one-node HIP graph per step; the 73 per-op launches of the same step (one graph) are timed beside
it. `value` is the algorithmic bytes of a step (every input read once, every output written once,
parameters once) divided by the measured step time, with all inputs resident in HBM.

Also reported (same JSON line):
  roofline      the step's kernel (t2s_step_fused) — bytes per launch over its device time per
                launch from HIP events, against 8 TB/s; traffic from two rocprofv3 --pmc runs;
  cpu_baseline  the oracle's C restatement of the same step on the host cores;
  whole_decode_step  the whole decode step (GEMVs, attention, epilogues) summary next to it;
  kernels       every fused kernel of the configurations at its stated shape (device time per launch
                in a graph of back-to-back launches, inputs cache-resident) and as a replicated
                batch of independent instances (> 0.4 GB moved, the 256 MB MALL cleared between
                repetitions by reading a 512 MiB buffer), in GB/s, rows/s and fraction of 8 TB/s;
  copy_GBps     a plain device-to-device copy of 1 GiB measured the same way (achievable-bandwidth
                reference for the replicated figures);
  write_only_GBps  a 1 GiB write-only stream measured the same way (the ceiling of write-dominated
                kernels such as the gather);
  sovits_decoder  the SoVITS ResBlock epilogues at every decoder stage shape (reference 768-channel
                geometry and the 512-start geometry), with the per-stage launch counts summed into
                epilogue microseconds per 10 s of audio;
  t2s_whole_decode_step  the whole decode step (GEMVs, attention with KV append, epilogues, logits)
                for 64 sequences at KV lengths 1024 and 2048, as one graph: microseconds per step,
                tokens/s and algorithmic GB/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-kernels] [--no-cpu]
       python bench.py --only KERNEL   (one kernel of the suite, for rocprofv3 runs)
       python bench.py --pmc           (the step kernel + a 256 MiB copy, for rocprofv3 --pmc runs)
       python bench.py --whole-step 1024   (the whole decode step alone, for rocprofv3 runs)
       python bench.py --conv          (SoVITS convolutions per stage, stages and whole decoder)
       python bench.py --decoder       (Generator stages and the whole decoder graph alone)
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "gpt-sovits-native_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of MI355X peak) per fused kernel; T2S decode-step µs"
SEED = 20250823

B, D, FF, LAYERS, VOCAB, MAX_POS = 64, 512, 2048, 24, 1025, 2048


LOG = []          # every measurement line of the run; written to the detail file
VERBOSE = False   # --verbose: also print them to stderr as they come


def log(*a):
    msg = " ".join(str(x) for x in a)
    LOG.append(msg)
    if VERBOSE:
        print(msg, file=sys.stderr, flush=True)


def progress(msg):
    """One short line per finished section, always on stderr (the run's progress)."""
    LOG.append(msg)
    print(f"bench: {msg}", file=sys.stderr, flush=True)


# ---- the headline line and the detail file ---------------------------------------------------------

HEADLINE_MAX_CHARS = 3000
HEADLINE_KEYS = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                 "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                 "roofline", "cpu_baseline")
# dropped in this order when the line would exceed HEADLINE_MAX_CHARS
HEADLINE_OPTIONAL = ("detail_file", "sovits", "whole_decode_step", "configs")


def config_summary(kernels):
    """Per configuration (1-5): how many kernel lines it has, the range of their fractions of 8 TB/s
    at the stated shape and replicated, and the range of the oracle's best CPU GB/s."""
    out = {}
    for k in kernels or ():
        c = out.setdefault(str(k["config"]), {"lines": 0, "stated_frac": [], "replicated_frac": [],
                                              "cpu_best_GBps": []})
        c["lines"] += 1
        c["stated_frac"].append(k["stated_shape"]["frac_of_peak"])
        c["replicated_frac"].append(k["replicated"]["frac_of_peak"])
        if k.get("cpu"):
            c["cpu_best_GBps"].append(k["cpu"]["best_GBps"])
    for c in out.values():
        for key in ("stated_frac", "replicated_frac", "cpu_best_GBps"):
            v = c[key]
            c[key] = [min(v), max(v)] if v else None
    return out


def headline_line(rec):
    """The one JSON line the bench prints last: the headline keys, roofline and cpu_baseline, and
    compact summaries of the rest (the full record is in the detail file). At most
    HEADLINE_MAX_CHARS characters: optional summaries are dropped, last first, until it fits."""
    line = {k: rec.get(k) for k in HEADLINE_KEYS}
    full = rec.get("t2s_whole_decode_step")
    if full:
        line["whole_decode_step"] = {f"kv{r['kv_len']}": {"us": r["us_per_step"],
                                                          "tokens_per_s": r["tokens_per_s"],
                                                          "frac": r["frac_of_peak"]} for r in full}
    if rec.get("kernels"):
        line["configs"] = config_summary(rec["kernels"])
    conv = rec.get("sovits_conv")
    if conv:
        gen = conv.get("generator") or {}
        dec_us = (gen.get("decoder") or {}).get("us")
        line["sovits"] = {"conv_frac_mfma": conv["roofline"]["frac"],
                          "conv_frac_of_bound": conv.get("frac_of_bound_by_stage"),
                          "decoder_graph_us": dec_us,
                          "decoder_eager_us": (gen.get("decoder") or {}).get("eager_us")}
        # the same algorithmic flops over the decoder graph's time (its ResBlocks run side by
        # side, so the graph takes less than the convolutions' one-at-a-time sum)
        if dec_us and conv["roofline"].get("flops"):
            line["sovits"]["decoder_frac_mfma"] = round(
                conv["roofline"]["flops"] / dec_us / 1e6 / conv["roofline"]["peak"], 4)
    if rec.get("detail_file"):
        line["detail_file"] = rec["detail_file"]
    s = json.dumps(line, separators=(",", ":"))
    for key in HEADLINE_OPTIONAL:
        if len(s) <= HEADLINE_MAX_CHARS:
            break
        line.pop(key, None)
        s = json.dumps(line, separators=(",", ":"))
    return s


def write_detail(rec, path):
    """The full record (every kernel line, per-op breakdown, decoder and convolution sweeps, CPU
    baselines) and the run's measurement log as JSON at `path`; returns the path, or None when it
    cannot be written."""
    if not path:
        return None
    try:
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "w") as f:
            json.dump(dict(rec, log=LOG), f, indent=1)
        return os.path.relpath(path, ROOT)
    except OSError:
        return None


# ---- algorithmic bytes ---------------------------------------------------------------------------

def ln_bytes(rows, n, esz, bias=True, res=True):
    """x (+ residual) read, y written, gamma/beta (+ bias) fp32 read once."""
    return rows * n * esz * (2 + (1 if res else 0)) + n * 4 * (2 + (1 if bias else 0))


def bias_act_bytes(rows, n, esz, bias=True):
    return 2 * rows * n * esz + (n * 4 if bias else 0)


def embed_bytes(rows, d, out_esz, tab_esz, id_esz=8, per_row_pos=True):
    return rows * (id_esz + (8 if per_row_pos else 0) + d * tab_esz + d * 4 + d * out_esz)


def embed_unique_bytes(rows, d, out_esz, tab_esz, vocab=VOCAB, max_pos=MAX_POS):
    """HBM floor of a gather over one shared table: ids, positions and output rows once per row,
    the table and the PE table once (their rows repeat and are served from L2 / MALL)."""
    return rows * (8 + 8 + d * out_esz) + vocab * d * tab_esz + max_pos * d * 4


def gn_bytes(C, T, esz):
    return 2 * C * T * esz + 2 * C * 4


def step_bytes():
    return (embed_bytes(B, D, 2, 2) + 2 * LAYERS * ln_bytes(B, D, 2)
            + LAYERS * bias_act_bytes(B, FF, 2))


# ---- T2S decode-step buffers ---------------------------------------------------------------------

def make_step_buffers(torch, gsvk, dev):
    g = torch.Generator(device="cpu").manual_seed(SEED + 2000)

    def rn(*shape, std=1.0, mean=0.0, dtype=torch.float16):
        return (torch.randn(*shape, generator=g) * std + mean).to(dtype).to(dev)

    bufs = {
        "table": rn(VOCAB, D, std=0.02),
        "ids": torch.randint(0, VOCAB, (B,), generator=g).to(dev),
        "pos": torch.randint(512, MAX_POS, (B,), generator=g).to(dev),
        "pe": torch.from_numpy(gsvk.pe_table(MAX_POS, D)).to(dev),
        "alpha": float(torch.empty(1).uniform_(0.5, 1.5, generator=g)),
        "x": torch.empty(B, D, dtype=torch.float16, device=dev),
        "h": torch.empty(B, D, dtype=torch.float16, device=dev),
        "err": torch.zeros(1, dtype=torch.int32, device=dev),
    }
    for name, shape in (("attn_out", (B, D)), ("ff", (B, FF)), ("ffn_out", (B, D))):
        bufs[name] = [rn(*shape) for _ in range(LAYERS)]
    for name, n in (("bout", D), ("b1", FF), ("b2", D)):
        bufs[name] = [rn(n, std=0.02, dtype=torch.float32) for _ in range(LAYERS)]
    for name in ("n1g", "n2g"):
        bufs[name] = [rn(D, std=0.1, mean=1.0, dtype=torch.float32) for _ in range(LAYERS)]
    for name in ("n1b", "n2b"):
        bufs[name] = [rn(D, std=0.1, dtype=torch.float32) for _ in range(LAYERS)]
    return bufs


def time_loop(torch, fn, iters, warmup=3):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / iters  # ms


def graph_of(torch, fn, n):
    """Capture n calls of fn into a CUDA/HIP graph on a side stream."""
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        fn()  # warm
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=st):
        for _ in range(n):
            fn()
    torch.cuda.synchronize()
    return gr


# ---- per-kernel suite ------------------------------------------------------------------------------

class Flusher:
    """Reads a 512 MiB buffer between timed repetitions so the 256 MB MALL holds none of the
    kernel's inputs. A read, not a write: a written flush buffer leaves dirty MALL lines whose
    write-back then runs inside the timed kernel (measured on MI355X: it halves a 64 MB read)."""

    def __init__(self, torch, dev):
        self.torch = torch
        self.buf = torch.ones(128 << 20, dtype=torch.float32, device=dev)
        self.out = torch.empty((), dtype=torch.float32, device=dev)

    def __call__(self):
        self.torch.sum(self.buf, 0, out=self.out)


def measure_reps(torch, fn, flush, reps=9):
    """Median of single-launch durations (HIP events), MALL flushed before each."""
    times = []
    fn()
    torch.cuda.synchronize()
    for _ in range(reps):
        flush()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        e.synchronize()
        times.append(s.elapsed_time(e))
    return statistics.median(times)


def graph_us_per_launch(torch, fn, launches=32, replays=10):
    """Device time per launch: a graph of `launches` back-to-back calls, replayed `replays` times
    between HIP events on the launch stream."""
    gr = graph_of(torch, fn, launches)
    us = time_loop(torch, gr.replay, replays) * 1e3 / launches
    del gr
    return us


def kernel_suite(torch, gsvk, dev, only=None, capture=None):
    """Each fused kernel at its stated shape and as a replicated batch. only: run that line alone.
    capture (a dict, with only): build the line's replicated launch and put it into capture
    ("fn", "instances", "bytes") without timing anything. only="__names__": return the line names
    and build nothing."""
    f16, f32 = torch.float16, torch.float32
    g = torch.Generator(device=dev).manual_seed(SEED)
    names = only == "__names__"
    flush = None if names or capture is not None else Flusher(torch, dev)
    out = []

    def rn(*shape, dtype=f16, std=1.0, mean=0.0):
        t = torch.empty(*shape, dtype=f32, device=dev).normal_(mean, std, generator=g)
        return t.to(dtype)

    def run(name, cfg, stated, replicated, bytes_fn, count, rep_bytes_fn=None, rows=None):
        """stated / replicated: (setup -> launch fn) builders taking a replication factor.
        rep_bytes_fn: HBM-unique bytes of the replicated launch when they differ from
        bytes_fn (the gather re-reads shared tables from cache). rows: k -> rows one launch of k
        instances produces (sequences, tokens or channel rows), for rows/s."""
        if names:
            out.append(name)
            return
        if only and only != name:
            return
        if capture is not None:
            rep, fnr = replicated()
            capture.update(fn=fnr, instances=rep, bytes=(rep_bytes_fn or bytes_fn)(rep))
            return
        rec = {"kernel": name, "config": cfg}
        fn1 = stated()
        us1 = graph_us_per_launch(torch, fn1)
        rec["stated_shape"] = {"us_per_launch": round(us1, 3), "bytes": bytes_fn(1),
                               "GBps": round(bytes_fn(1) / us1 / 1e3, 1),
                               "frac_of_peak": round(bytes_fn(1) / us1 / 1e3 / PEAK_GBS, 4),
                               "calls_per_config": count}
        if rows:
            rec["stated_shape"]["rows"] = rows(1)
            rec["stated_shape"]["rows_per_s"] = round(rows(1) / us1 * 1e6, 0)
        del fn1
        rep, fnr = replicated()
        msr = measure_reps(torch, fnr, flush)
        rb = (rep_bytes_fn or bytes_fn)(rep)
        gbs = rb / msr / 1e6
        rec["replicated"] = {"instances": rep, "bytes": rb, "us": round(msr * 1e3, 2),
                             "GBps": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4)}
        if rows:
            rec["replicated"]["rows"] = rows(rep)
            rec["replicated"]["rows_per_s"] = round(rows(rep) / msr * 1e3, 0)
        del fnr
        torch.cuda.empty_cache()
        out.append(rec)
        log(f"  {name}: stated {rec['stated_shape']['us_per_launch']} us, replicated "
            f"{rec['replicated']['GBps']} GB/s ({100 * gbs / PEAK_GBS:.1f}%)")

    def ln_case(rows, n, dt, eps, bias, res, rep):
        def make(k):
            x = rn(rows * k, n, dtype=dt)
            r = rn(rows * k, n, dtype=dt) if res else None
            gm, bt = rn(n, dtype=f32, std=0.1, mean=1.0), rn(n, dtype=f32, std=0.1)
            bi = rn(n, dtype=f32, std=0.02) if bias else None
            y = torch.empty_like(x)
            return lambda: gsvk.add_layernorm(x, gm, bt, y, eps, bias=bi, residual=r)
        esz = 4 if dt == f32 else 2
        return (lambda: make(1), lambda: (rep, make(rep)),
                lambda k: ln_bytes(rows * k, n, esz, bias, res))

    def ba_case(rows, n, act, rep):
        def make(k):
            x = rn(rows * k, n)
            bi = rn(n, dtype=f32, std=0.02)
            return lambda: gsvk.bias_act(act, x, x, bias=bi)
        return (lambda: make(1), lambda: (rep, make(rep)), lambda k: bias_act_bytes(rows * k, n, 2))

    # config 1: residual + LayerNorm fp32 [256, 512]
    run("residual_layernorm_f32_256x512", 1, *ln_case(256, 512, f32, 1e-5, False, True, 1024), 1,
        rows=lambda k: 256 * k)
    # config 2: gather + PE prefill/decode, LN [64,512], bias+ReLU [64,2048]
    pe = torch.from_numpy(gsvk.pe_table(MAX_POS, D)).to(dev)

    def emb_case(rows, rep):
        def make(k):
            tab = rn(VOCAB, D, std=0.02)
            ids = torch.randint(0, VOCAB, (rows * k,), device=dev, generator=g)
            pos = torch.randint(0, MAX_POS, (rows * k,), device=dev, generator=g)
            o = torch.empty(rows * k, D, dtype=f16, device=dev)
            return lambda: gsvk.embed_pe(tab, ids, pe, 0.93, o, pos=pos)
        return (lambda: make(1), lambda: (rep, make(rep)), lambda k: embed_bytes(rows * k, D, 2, 2),
                lambda k: embed_unique_bytes(rows * k, D, 2, 2))

    def run_emb(name, rows, rep):
        st_, rp_, b_, ub_ = emb_case(rows, rep)
        run(name, 2, st_, rp_, b_, 1, rep_bytes_fn=ub_, rows=lambda k: rows * k)

    run_emb("embed_pe_prefill_1024x512", 1024, 512)

    def hot_case(rows, rep):
        """The gather at the same granularity with every id 0 and every position 0: its table and
        PE reads hit one 3 KiB working set in L1, so what remains is the id / position reads and
        the 1 KiB row writes per wave. The ceiling of the gather's write path on this GPU."""
        def make(k):
            tab = rn(1, D, std=0.02)
            ids = torch.zeros(rows * k, dtype=torch.int64, device=dev)
            pos = torch.zeros(rows * k, dtype=torch.int64, device=dev)
            o = torch.empty(rows * k, D, dtype=f16, device=dev)
            return lambda: gsvk.embed_pe(tab, ids, pe, 0.93, o, pos=pos)
        return (lambda: make(1), lambda: (rep, make(rep)), lambda k: embed_bytes(rows * k, D, 2, 2),
                lambda k: rows * k * (8 + 8 + 2 * D) + D * 2 + D * 4)

    st_, rp_, b_, ub_ = hot_case(1024, 512)
    run("embed_pe_hot_row_ceiling_1024x512", 2, st_, rp_, b_, 1, rep_bytes_fn=ub_,
        rows=lambda k: 1024 * k)

    def prefill_case(rep):
        """The stated prefill pattern: 512 phone ids from the [732, 512] table and 512 semantic ids
        from the [1025, 512] table, both at positions 0..511 (pe_row(t) in row order,
        t2s_engine.cpp:1778, 1784): one launch per table, positions implicit (pos0 = 0). The
        replicated batch is `rep` such prompts, explicit positions t mod 512 per row; its HBM
        floor counts ids, positions and output rows per row and the tables and the 512 PE rows
        once."""
        def make(k):
            tp, ts = rn(732, D, std=0.02), rn(VOCAB, D, std=0.02)
            ip = torch.randint(0, 732, (512 * k,), device=dev, generator=g)
            isem = torch.randint(0, VOCAB, (512 * k,), device=dev, generator=g)
            op = torch.empty(512 * k, D, dtype=f16, device=dev)
            osem = torch.empty(512 * k, D, dtype=f16, device=dev)
            if k == 1:
                return lambda: (gsvk.embed_pe(tp, ip, pe, 0.93, op, pos0=0),
                                gsvk.embed_pe(ts, isem, pe, 1.07, osem, pos0=0))
            pos = torch.arange(512 * k, device=dev, dtype=torch.int64) % 512
            return lambda: (gsvk.embed_pe(tp, ip, pe, 0.93, op, pos=pos),
                            gsvk.embed_pe(ts, isem, pe, 1.07, osem, pos=pos))
        per = lambda k: 1024 * k * (8 + 2 * D + 4 * D + 2 * D)
        floor = lambda k: 1024 * k * (16 + 2 * D) + (732 + VOCAB) * D * 2 + 512 * D * 4
        return (lambda: make(1), lambda: (rep, make(rep)), per, floor)

    st_, rp_, b_, ub_ = prefill_case(512)
    run("embed_pe_prefill_pos0_511_2x512x512", 2, st_, rp_, b_, 1, rep_bytes_fn=ub_,
        rows=lambda k: 1024 * k)

    def prefill_input_case(rep):
        """The same prefill input as one launch (gsvk_t2s_prefill_input): xy [1024, 512] f16 = 512
        text rows and 512 prompt rows at positions 0..511, each PE row read once for both. The
        replicated case is one call over 512 * rep positions with a PE table of as many rows, so
        every PE row is read from HBM exactly once; its floor counts the ids, both output rows and
        the PE row per position, and the tables once."""
        def make(k):
            n = 512 * k
            tp, ts = rn(732, D, std=0.02), rn(VOCAB, D, std=0.02)
            ip = torch.randint(0, 732, (n,), device=dev, generator=g)
            isem = torch.randint(0, VOCAB, (n,), device=dev, generator=g)
            pe_k = pe if k == 1 else rn(n, D, dtype=f32)
            xy = torch.empty(2 * n, D, dtype=f16, device=dev)
            return lambda: gsvk.t2s_prefill_input(tp, ip, 0.93, ts, isem, 1.07, pe_k, xy)
        per = lambda k: 1024 * k * (8 + 2 * D + 2 * D) + 512 * k * 4 * D
        floor = lambda k: (512 * k * (16 + 2 * 2 * D + 4 * D) + (732 + VOCAB) * D * 2 if k > 1
                           else per(1))
        return (lambda: make(1), lambda: (rep, make(rep)), per, floor)

    st_, rp_, b_, ub_ = prefill_input_case(512)
    run("t2s_prefill_input_pos0_511_2x512x512", 2, st_, rp_, b_, 1, rep_bytes_fn=ub_,
        rows=lambda k: 1024 * k)

    def prefill_distinct_case(rep):
        """The two-gather form of the same prefill input over the one-launch line's workload: at
        the stated shape the two gathers at positions 0..511; replicated, 512 * rep positions with
        a PE table of as many rows, so each PE row comes from HBM as in the one-launch line, and
        the same floor (ids, both output rows and the PE row per position, the tables once)."""
        def make(k):
            n = 512 * k
            tp, ts = rn(732, D, std=0.02), rn(VOCAB, D, std=0.02)
            ip = torch.randint(0, 732, (n,), device=dev, generator=g)
            isem = torch.randint(0, VOCAB, (n,), device=dev, generator=g)
            pe_k = pe if k == 1 else rn(n, D, dtype=f32)
            op = torch.empty(n, D, dtype=f16, device=dev)
            osem = torch.empty(n, D, dtype=f16, device=dev)
            return lambda: (gsvk.embed_pe(tp, ip, pe_k, 0.93, op, pos0=0),
                            gsvk.embed_pe(ts, isem, pe_k, 1.07, osem, pos0=0))
        per = lambda k: 1024 * k * (8 + 2 * D + 4 * D + 2 * D)
        floor = lambda k: (512 * k * (16 + 2 * 2 * D + 4 * D) + (732 + VOCAB) * D * 2 if k > 1
                           else per(1))
        return (lambda: make(1), lambda: (rep, make(rep)), per, floor)

    st_, rp_, b_, ub_ = prefill_distinct_case(512)
    run("embed_pe_prefill_distinct_pos_2x512x512", 2, st_, rp_, b_, 1, rep_bytes_fn=ub_,
        rows=lambda k: 1024 * k)
    run_emb("embed_pe_decode_64x512", 64, 8192)

    def text_case(rows, rep):
        """Text rows: out = mm + (e + bert_b) + alpha*PE(t) (t2s_engine.cpp:1774-1780)."""
        def make(k):
            tab = rn(732, D, std=0.02)
            ids = torch.randint(0, 732, (rows * k,), device=dev, generator=g)
            mm = rn(rows * k, D)
            bb = rn(D, dtype=f32, std=0.02)
            o = torch.empty(rows * k, D, dtype=f16, device=dev)
            if k == 1:  # one sequence: positions 0..rows-1 implicit, as the reference passes them
                return lambda: gsvk.embed_pe(tab, ids, pe, 0.93, o, pos0=0, mm=mm, bias=bb)
            # k sequences of `rows` each: explicit positions restart at 0 for every sequence
            pos = torch.arange(rows * k, device=dev, dtype=torch.int64) % rows
            return lambda: gsvk.embed_pe(tab, ids, pe, 0.93, o, pos=pos, mm=mm, bias=bb)
        # per row: id, table row, PE row, mm row, out row; bias once. The replicated batch also
        # reads an explicit position per row, and its floor counts the 732-row table and the
        # `rows` PE rows once (they stay in cache across sequences).
        per_row = lambda k: rows * k * (8 + 2 * D + 4 * D + 2 * D + 2 * D) + 4 * D
        floor = lambda k: rows * k * (16 + 4 * D) + 732 * D * 2 + rows * D * 4 + 4 * D
        return (lambda: make(1), lambda: (rep, make(rep)), per_row, floor)

    st_, rp_, b_, ub_ = text_case(512, 1024)
    run("embed_pe_text_rows_512x512", 2, st_, rp_, b_, 1, rep_bytes_fn=ub_, rows=lambda k: 512 * k)
    run("residual_layernorm_f16_64x512", 2, *ln_case(64, 512, f16, 1e-5, True, True, 8192), 48,
        rows=lambda k: 64 * k)
    run("bias_relu_f16_64x2048", 2, *ba_case(64, 2048, gsvk.ACT_RELU, 4096), 24,
        rows=lambda k: 64 * k)
    # config 3: bias + GELU [512, 4096], residual + LN(1024, eps 1e-12)
    run("bias_gelu_f16_512x4096", 3, *ba_case(512, 4096, gsvk.ACT_GELU_ERF, 128), 1,
        rows=lambda k: 512 * k)
    run("residual_layernorm_f16_512x1024_eps1e-12", 3,
        *ln_case(512, 1024, f16, 1e-12, False, True, 512), 24, rows=lambda k: 512 * k)
    # config 4: GroupNorm + GELU [512, 31999] fp32, LN(768), bias + GELU [499, 3072]

    def gn_case(rep):
        def make(k):
            x = rn(512 * k, 31999, dtype=f32, std=0.5)
            gm, bt = rn(512 * k, dtype=f32, std=0.1, mean=1.0), rn(512 * k, dtype=f32, std=0.1)
            y = torch.empty_like(x)
            return lambda: gsvk.groupnorm_gelu(x, gm, bt, y, 1e-5)
        return (lambda: make(1), lambda: (rep, make(rep)), lambda k: gn_bytes(512 * k, 31999, 4))

    run("groupnorm_gelu_f32_512x31999", 4, *gn_case(8), 1, rows=lambda k: 512 * k)
    run("residual_layernorm_f16_499x768", 4, *ln_case(499, 768, f16, 1e-5, True, True, 512), 24,
        rows=lambda k: 499 * k)
    run("bias_gelu_f16_499x3072", 4, *ba_case(499, 3072, gsvk.ACT_GELU_ERF, 192), 12,
        rows=lambda k: 499 * k)

    # config 5: SoVITS ResBlock epilogues at the largest stage [24, 320000]
    def sv_case(kind, dt, rep):
        E = 24 * 320000
        esz = 4 if dt == f32 else 2

        def make(k):
            n = E * k
            if kind == "K1":
                t = rn(n, dtype=dt)
                return lambda: gsvk.leaky_relu(t, t, 0.1)
            if kind == "K2":
                cur, tb, tin = rn(n, dtype=dt), rn(n, dtype=dt), torch.empty(n, dtype=dt, device=dev)
                return lambda: gsvk.resblock_add_lrelu(cur, tb, tin, 0.1)
            curs = [rn(n, dtype=dt) for _ in range(3)]
            tbs = [rn(n, dtype=dt) for _ in range(3)]
            o = torch.empty(n, dtype=dt, device=dev)
            return lambda: gsvk.resblock_branch_mean(curs, tbs, o, True, 0.1)
        per = {"K1": 2, "K2": 4, "K3": 7}[kind]
        return (lambda: make(1), lambda: (rep, make(rep)), lambda k: per * E * k * esz)

    for kind, count in (("K3", 1), ("K2", 6), ("K1", 9)):
        for dt, nm, rep in ((f32, "f32", 8), (f16, "f16", 16)):
            run(f"sovits_{kind}_{nm}_24x320000", 5, *sv_case(kind, dt, rep), count,
                rows=lambda k: 24 * k)

    # T2S decode GEMVs with their fused epilogues, B = 64 rows (t2s_engine.cpp:1044-1116): the
    # stated shape cycles through 24 distinct weight matrices (one per layer, as a decode step
    # does); the replicated case is one weight stream of `rep` such matrices stacked along N.
    def gemv_case(N, K, act, use_bias, use_res, ydt, rep, layers=24, M=B):
        yesz = 4 if ydt == f32 else 2

        def make(k):
            n = N * k
            nw = layers if k == 1 else 1
            Ws = [rn(n, K, std=0.05) for _ in range(nw)]
            x = rn(M, K)
            bi = rn(n, dtype=f32, std=0.02) if use_bias else None
            y = torch.empty(M, n, dtype=ydt, device=dev)
            res = rn(M, n, dtype=ydt) if use_res else None
            it = [0]

            def call():
                w = Ws[it[0] % nw]
                it[0] += 1
                gsvk.gemv_f16w(x, w, y, bias=bi, act=act, residual=res)
            return call

        def nbytes(k):
            n = N * k
            return (n * K * 2 + M * K * 2 + M * n * yesz + (n * 4 if use_bias else 0) +
                    (M * n * yesz if use_res else 0))
        return (lambda: make(1), lambda: (rep, make(rep)), nbytes)

    for name, N, K, act, ub, ur, ydt, rep, count in (
            ("qkv_bias_f32out", 1536, 512, gsvk.ACT_NONE, True, False, f32, 128, 24),
            ("outproj_bias_residual", 512, 512, gsvk.ACT_NONE, True, True, f16, 256, 24),
            ("w1_bias_relu", 2048, 512, gsvk.ACT_RELU, True, False, f16, 64, 24),
            ("w2_bias_residual", 512, 2048, gsvk.ACT_NONE, True, True, f16, 128, 24),
            ("logits_f32out", 1025, 512, gsvk.ACT_NONE, False, False, f32, 128, 1)):
        run(f"gemv_{name}_64x{N}x{K}", 2, *gemv_case(N, K, act, ub, ur, ydt, rep), count,
            rows=lambda k: B)
    # The same long-stream kernel with little to write: 16 rows over 2048 x 128 columns, 268 MB of
    # weights read for 8 MB of output, against 4-5 bytes read per byte written on the 64-row lines
    # above. The difference is what the output stores cost the weight stream.
    run("gemv_read_dominated_16x2048x512", 2,
        *gemv_case(2048, 512, gsvk.ACT_NONE, False, False, f16, 128, M=16), 0, rows=lambda k: 16)

    # T2S decode attention with the KV append (t2s_engine.cpp:1051-1087): B = 64 sequences, 16 heads
    # of 32, fp16 caches, every sequence at position L - 1. One call already streams 2 B L D cache
    # elements, so the replicated case is the same call at twice the length.
    def attn_case(Ln, rep):
        def make(k):
            n = Ln * k
            kc, vc = rn(B, n, D), rn(B, n, D)
            q = rn(B, 3 * D, dtype=f32)
            pos = torch.full((B,), n - 1, dtype=torch.int64, device=dev)
            o = torch.empty(B, D, dtype=f16, device=dev)
            return lambda: gsvk.decode_attention(q, kc, vc, pos, o, 16, len_bound=n)
        nbytes = lambda k: 2 * B * Ln * k * D * 2 + B * 3 * D * 4 + B * D * 2
        return (lambda: make(1), lambda: (rep, make(rep)), nbytes)

    run("decode_attention_f16kv_64x1024x512", 2, *attn_case(1024, 2), 24, rows=lambda k: B)
    return out


# ---- SoVITS decoder stage sweep ----------------------------------------------------------------------

DECODER_GEOMETRIES = {
    # Generator with 768 initial channels, upsample rates 10,8,2,2,2, 500 input frames
    # (dec.hpp:55-76): the geometry the reference runs
    "reference_768": [(384, 5000), (192, 40000), (96, 80000), (48, 160000), (24, 320000)],
    # the configuration text's 512-start geometry, final stage 32 x 320000 as written
    "literal_512": [(256, 5000), (128, 40000), (64, 80000), (32, 160000), (32, 320000)],
}


def sovits_decoder(torch, gsvk, dev):
    """Per stage (C, T): graph-timed launches of K1 (LeakyReLU in place), K2 (residual add +
    LeakyReLU write) and K3 (3-branch mean + next LeakyReLU) at that stage's shape, fp32 and fp16,
    and the stage's epilogue time with the reference's per-stage counts (9 x K1, 6 x K2, 1 x K3;
    dec.hpp:283-336). Totals are per 10 s of 32 kHz audio."""
    out = {}
    for geo, stages in DECODER_GEOMETRIES.items():
        for dt, nm in ((torch.float32, "f32"), (torch.float16, "f16")):
            esz = 4 if dt == torch.float32 else 2
            rows, total = [], 0.0
            for C, T in stages:
                n = C * T
                t = torch.randn(n, device=dev).to(dt)
                cur = torch.randn(n, device=dev).to(dt)
                tb = torch.randn(n, device=dev).to(dt)
                tin = torch.empty_like(t)
                curs = [torch.randn(n, device=dev).to(dt) for _ in range(3)]
                tbs = [torch.randn(n, device=dev).to(dt) for _ in range(3)]
                o = torch.empty_like(t)
                k1 = graph_us_per_launch(torch, lambda: gsvk.leaky_relu(t, t, 0.1), 16, 5)
                k2 = graph_us_per_launch(torch, lambda: gsvk.resblock_add_lrelu(cur, tb, tin, 0.1),
                                         16, 5)
                k3 = graph_us_per_launch(torch, lambda: gsvk.resblock_branch_mean(curs, tbs, o, True,
                                                                                  0.1), 16, 5)
                stage_us = 9 * k1 + 6 * k2 + k3
                stage_bytes = (9 * 2 + 6 * 4 + 7) * n * esz
                total += stage_us
                rows.append({"C": C, "T": T, "K1_us": round(k1, 2), "K2_us": round(k2, 2),
                             "K3_us": round(k3, 2), "stage_us": round(stage_us, 1),
                             "stage_GBps": round(stage_bytes / stage_us / 1e3, 1)})
                del t, cur, tb, tin, curs, tbs, o
            torch.cuda.empty_cache()
            out[f"{geo}_{nm}"] = {"stages": rows, "epilogue_us_per_10s_audio": round(total, 1)}
            log(f"  sovits decoder {geo} {nm}: {total:.1f} us of epilogues per 10 s of audio")
    return out


# ---- SoVITS ResBlock convolutions --------------------------------------------------------------------

RES_KERNELS = (3, 7, 11)      # ResBlock1 kernel sizes (dec.hpp:55-76)
UPS = {"reference_768": [(768, 10, 20), (384, 8, 16), (192, 2, 8), (96, 2, 2), (48, 2, 2)],
       "literal_512": [(512, 10, 20), (256, 8, 16), (128, 2, 8), (64, 2, 2), (32, 2, 2)]}
# (input channels, stride u, kernel k) of Generator.ups per stage (dec.hpp:55-76)
RES_DILATIONS = (1, 3, 5)     # conv1 dilations; every conv2 has dilation 1
PEAK_F16_TFLOPS = 2500.0      # MI355X dense fp16 matrix-core peak


def conv_us(torch, fn, iters=10):
    """Device time of one launch: HIP events around `iters` back-to-back launches."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e3 / iters


def conv_bound(flops, nbytes, us):
    """A convolution launch against the resource that bounds it: MFMA when its time at the dense
    fp16 peak (the fp32 path's hi/lo split doubles the matrix-core work) exceeds its HBM bytes' time
    at 8 TB/s, else HBM."""
    t_mfma = 2 * flops / (PEAK_F16_TFLOPS * 1e12)
    t_hbm = nbytes / (PEAK_GBS * 1e9)
    bound = "mfma" if t_mfma >= t_hbm else "hbm"
    frac = max(t_mfma, t_hbm) / (us * 1e-6)
    return {"bytes": nbytes, "GBps": round(nbytes / us / 1e3, 1), "bound": bound,
            "frac_of_bound": round(frac, 4)}


def conv_one(torch, gsvk, dev, spec, launches=20):
    """One SoVITS ResBlock convolution, C -> C channels over T frames with kernel k, dilation dil and
    epilogue epi (spec "C,T,k,dil,epi"; fp32 activations, exact): 2 warm-up launches, then
    `launches` timed ones. For rocprofv3 --pmc runs on one convolution shape."""
    C, T, k, dil, epi = (int(v) for v in spec.split(","))
    x = torch.randn(C, T, device=dev)
    y = torch.empty(C, T, device=dev)
    cur = torch.randn(C, T, device=dev)
    conv = gsvk.Conv1d((torch.randn(C, C, k, device=dev) / (C * k) ** 0.5).half(),
                       torch.randn(C, device=dev) * 0.05, dil)
    fn = lambda: conv.forward(x, y, epi=epi, cur=cur)
    us = time_loop(torch, fn, launches, warmup=2) * 1e3
    fl = 2.0 * C * C * k * T
    res = (epi in (gsvk.CONV_EPI_RES_LRELU, gsvk.CONV_EPI_RES))
    nb = C * T * 4 * (2 + (2 if res else 0)) + C * C * k * 2 + C * 4
    return {"conv": spec, "launches": launches, "us_per_launch": round(us, 2),
            "TFLOPs": round(fl / us / 1e6, 1), **conv_bound(fl, nb, us)}


def sovits_conv(torch, gsvk, dev, geometry="reference_768"):
    """Per decoder stage (C, T): the upsampler (ConvT1d into the stage) and every distinct ResBlock
    convolution timed once (conv1: k x dilation 1 / 3 / 5 with the LeakyReLU epilogue; conv2: k,
    dilation 1, with the residual + LeakyReLU epilogue); the stage total is the upsampler plus its
    18 convolutions (3 ResBlocks x 3 pairs). fp32
    activations multiplied exactly (the reference's sgemm path) and, as a second figure, rounded to
    fp16 (its AMX path). Algorithmic flops 2 C^2 k T per convolution."""
    stages, tot, tot_rx, flops_tot = [], 0.0, 0.0, 0.0
    for (C, T), (cin_up, u, k_up) in zip(DECODER_GEOMETRIES[geometry], UPS[geometry]):
        # the stage's upsampler: ConvT1d cin_up -> C, T / u -> T frames
        xu = torch.randn(cin_up, T // u, device=dev)
        yu = torch.empty(C, T, device=dev)
        up = gsvk.ConvT1d((torch.randn(cin_up, C, k_up, device=dev) / (cin_up * k_up / u) ** 0.5)
                          .half(), torch.randn(C, device=dev) * 0.05, u)
        up_us = conv_us(torch, lambda: up.forward(xu, yu))
        up_us_rx = conv_us(torch, lambda: up.forward(xu, yu, round_x=True))
        up_fl = 2.0 * cin_up * C * k_up * (T // u)
        del xu, yu, up
        x = torch.randn(C, T, device=dev)
        y = torch.empty(C, T, device=dev)
        cur = torch.randn(C, T, device=dev)
        row = {"C": C, "T": T, "convs": []}
        st, st_rx, st_fl = 0.0, 0.0, 0.0
        for k in RES_KERNELS:
            conv = gsvk.Conv1d((torch.randn(C, C, k, device=dev) / (C * k) ** 0.5).half(),
                               torch.randn(C, device=dev) * 0.05, 1)
            fl = 2.0 * C * C * k * T
            for dil, epi, n in [(d, gsvk.CONV_EPI_LRELU, 1) for d in RES_DILATIONS] + \
                               [(1, gsvk.CONV_EPI_RES_LRELU, 3)]:
                conv.dilation = dil
                us = conv_us(torch, lambda: conv.forward(x, y, epi=epi, cur=cur))
                us_rx = conv_us(torch, lambda: conv.forward(x, y, epi=epi, cur=cur, round_x=True))
                # HBM bytes: x read, y written, the residual epilogue's cur read and written, the
                # fp16 weights and the bias once
                nb = C * T * 4 * (2 + (2 if epi == gsvk.CONV_EPI_RES_LRELU else 0)) + C * C * k * 2 + C * 4
                row["convs"].append({"k": k, "dil": dil, "epi": epi, "count": n,
                                     "us": round(us, 2), "us_round_x": round(us_rx, 2),
                                     "TFLOPs": round(fl / us / 1e6, 1),
                                     **conv_bound(fl, nb, us)})
                st += n * us
                st_rx += n * us_rx
                st_fl += n * fl
        row["upsample"] = {"c_in": cin_up, "stride": u, "k": k_up, "us": round(up_us, 2),
                           "us_round_x": round(up_us_rx, 2),
                           "TFLOPs": round(up_fl / up_us / 1e6, 1),
                           "out_GBps": round(C * T * 4 / up_us / 1e3, 1),
                           **conv_bound(up_fl, cin_up * (T // u) * 4 + C * T * 4 * 2 +
                                        cin_up * C * k_up * 2 + C * 4, up_us)}
        st, st_rx, st_fl = st + up_us, st_rx + up_us_rx, st_fl + up_fl
        # the stage's binding resource: the time-weighted mean of its launches' fractions of
        # their own bound
        bound_us = sum(c["count"] * c["us"] * c["frac_of_bound"] for c in row["convs"]) + \
            up_us * row["upsample"]["frac_of_bound"]
        row.update({"stage_us": round(st, 1), "stage_us_round_x": round(st_rx, 1),
                    "stage_TFLOPs": round(st_fl / st / 1e6, 1),
                    "stage_frac_of_bound": round(bound_us / st, 4)})
        stages.append(row)
        tot, tot_rx, flops_tot = tot + st, tot_rx + st_rx, flops_tot + st_fl
        log(f"  conv stage {C}x{T}: {st:.1f} us incl. upsampler {up_us:.1f} us (round_x "
            f"{st_rx:.1f} us), {st_fl / st / 1e6:.0f} TFLOP/s")
        del x, y, cur, conv
    torch.cuda.empty_cache()
    ach = flops_tot / tot / 1e6
    log("  conv stages against their binding resource: " + ", ".join(
        f"{r['C']}x{r['T']} {100 * r['stage_frac_of_bound']:.1f}%" for r in stages))
    return {"geometry": geometry, "stages": stages, "conv_us_per_10s_audio": round(tot, 1),
            "conv_us_per_10s_audio_round_x": round(tot_rx, 1),
            "frac_of_bound_by_stage": {f"{r['C']}x{r['T']}": r["stage_frac_of_bound"]
                                       for r in stages},
            "roofline": {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_F16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / PEAK_F16_TFLOPS, 4),
                         "flops": flops_tot,
                         "note": "algorithmic flops; fp32 activations (hi/lo fp16 split, ~22 bits) run two fp16 products per term"}}


def sovits_generator(torch, gsvk, dev, geometry="reference_768", reps=5, frames=500):
    """The decoder's five Generator stages (gsvk.GeneratorStage: upsampler with the LeakyReLU copy
    fused, 3 ResBlocks x 3 fused conv pairs, branch mean + next LeakyReLU; 20 launches per stage)
    timed one by one as eager launches, then the whole decoder (gsvk.SovitsDecoder: cond folded into
    conv_pre's bias, conv_pre + LeakyReLU, the 5 stages, conv_post + tanh; 104 launches) replayed as
    one HIP graph on z [192, frames]. fp32 activations (hi/lo fp16 split, ~22 bits), random-init
    weights of the reference's shapes.
    Each figure is the median of `reps` timed runs after one warm run; 500 frames = 10 s of 32 kHz
    audio."""
    g = lambda *shape: torch.randn(*shape, device=dev)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            e.synchronize()
            ts.append(s.elapsed_time(e) * 1e3)
        return sorted(ts)[len(ts) // 2]

    out, tot, stages = [], 0.0, []
    for (C, T), (cin_up, u, k_up) in zip(DECODER_GEOMETRIES[geometry], UPS[geometry]):
        ups = gsvk.ConvT1d((g(cin_up, C, k_up) / (cin_up * k_up / u) ** 0.5).half(), g(C) * 0.05, u)
        blocks = []
        for k in RES_KERNELS:
            w = lambda: (g(C, C, k) / (C * k) ** 0.5).half()
            blocks.append(gsvk.ResBlock1([w() for _ in range(3)], [g(C) * 0.05 for _ in range(3)],
                                         [w() for _ in range(3)], [g(C) * 0.05 for _ in range(3)]))
        stage = gsvk.GeneratorStage(ups, blocks)
        stages.append(stage)
        x = g(cin_up, T // u)
        y = torch.empty(C, T, device=dev)
        us = timed(lambda: stage.forward(x, y))
        tot += us
        out.append({"C": C, "T": T, "stage_us": round(us, 1), "launches": 20})
        log(f"  generator stage {C}x{T}: {us:.1f} us end to end")
        del x, y
        stage._buf = None  # the decoder below brings its own activations
        torch.cuda.empty_cache()
    c0, c_last, c_z, g_in = UPS[geometry][0][0], DECODER_GEOMETRIES[geometry][-1][0], 192, 1024
    pre = gsvk.Conv1d((g(c0, c_z, 7) / (c_z * 7) ** 0.5).half(), g(c0) * 0.05)
    cond = ((g(c0, g_in) / g_in ** 0.5).half(), g(c0) * 0.05)  # k = 1: the [c0, g_in] matrix
    post = gsvk.Conv1d((g(1, c_last, 7) / (c_last * 7) ** 0.5).half(), None)
    z, ge = g(c_z, frames), g(g_in)
    n_out = frames
    for _, u, _ in UPS[geometry]:
        n_out *= u
    audio_s = n_out / 32000.0
    res = {"geometry": geometry, "stages": out, "stages_us_per_10s_audio": round(tot, 1)}
    # fp32 as a hi/lo fp16 pair (the reference's default sgemm numerics to ~22 bits), fp32 with
    # fp16-rounded convolution inputs
    # (its AMX numerics), fp16 storage
    for name, zz, rx in (("decoder", z, False), ("decoder_round_x", z, True),
                         ("decoder_f16", z.half(), False)):
        wav = torch.empty(n_out, dtype=zz.dtype, device=dev)
        dec = gsvk.SovitsDecoder(pre, cond, stages, post, zz, ge, wav, round_x=rx, graph=True)
        dus = timed(dec.run)
        log(f"  whole {name} (graph, {dec.launches} launches): {dus:.1f} us for {audio_s:g} s of audio")
        res[name] = {"frames": frames, "samples": n_out, "launches": dec.launches, "graph": True,
                     "us": round(dus, 1), "realtime_factor": round(audio_s / (dus * 1e-6), 1),
                     "workspace_bytes": dec.ws.numel(),
                     "activations": "f16" if zz.dtype == torch.float16 else "f32",
                     "round_x": rx}
        if name == "decoder":  # the same launches issued directly (gsvk_sovits_decoder_eager)
            eager = gsvk.SovitsDecoder(pre, cond, stages, post, zz, ge, wav, round_x=rx,
                                       graph=False)
            eus = timed(eager.run)
            log(f"  whole {name} (eager, {eager.launches} launches): {eus:.1f} us")
            res[name]["eager_us"] = round(eus, 1)
            del eager
        del dec, wav
        torch.cuda.empty_cache()
    del stages, pre, cond, post, z, ge
    torch.cuda.empty_cache()
    return res


# ---- whole T2S decode step ---------------------------------------------------------------------------

def full_decode_step(torch, gsvk, dev, kv_len=1024, steps=50, warmup=5):
    """One whole decode step (gsvk_t2s_decode: embedding, 24 x [QKV GEMV, attention with KV append,
    out-proj GEMV + bias + residual, LN1, W1 GEMV + bias + ReLU, W2 GEMV + bias + residual, LN2],
    logits GEMV) for B = 64 sequences whose caches hold kv_len tokens, replayed as one graph.
    Random-init weights of the T2S shapes (fp16), fp16 caches and activations."""
    g = torch.Generator(device=dev).manual_seed(SEED + 7)
    f16, f32 = torch.float16, torch.float32
    H, V, max_len = 16, VOCAB, kv_len + 64

    def rn(*shape, std=1.0, mean=0.0, dtype=f16):
        return torch.empty(*shape, dtype=f32, device=dev).normal_(mean, std, generator=g).to(dtype)

    layers = []
    for _ in range(LAYERS):
        layers.append(dict(
            wqkv=rn(3 * D, D, std=0.05), bqkv=rn(3 * D, std=0.02, dtype=f32),
            wout=rn(D, D, std=0.05), bout=rn(D, std=0.02, dtype=f32),
            n1g=rn(D, std=0.1, mean=1.0, dtype=f32), n1b=rn(D, std=0.1, dtype=f32),
            w1=rn(FF, D, std=0.05), b1=rn(FF, std=0.02, dtype=f32),
            w2=rn(D, FF, std=0.05), b2=rn(D, std=0.02, dtype=f32),
            n2g=rn(D, std=0.1, mean=1.0, dtype=f32), n2b=rn(D, std=0.1, dtype=f32),
            k_cache=rn(B, max_len, D), v_cache=rn(B, max_len, D)))
    m = dict(table=rn(V, D, std=0.02), pe=torch.from_numpy(gsvk.pe_table(MAX_POS, D)).to(dev),
             alpha=0.93, heads=H, layers=layers, w_logits=rn(V, D, std=0.05))
    io = dict(ids=torch.randint(0, V, (B,), device=dev, generator=g),
              pos=torch.full((B,), 512, dtype=torch.int64, device=dev),
              kv_pos=torch.full((B,), kv_len - 1, dtype=torch.int64, device=dev),
              err=torch.zeros(1, dtype=torch.int32, device=dev),
              x=torch.empty(B, D, dtype=f16, device=dev), h=torch.empty(B, D, dtype=f16, device=dev),
              z=torch.empty(B, D, dtype=f16, device=dev),
              attn=torch.empty(B, D, dtype=f16, device=dev),
              ff=torch.empty(B, FF, dtype=f16, device=dev),
              qkv=torch.empty(B, 3 * D, dtype=f32, device=dev),
              logits=torch.empty(B, V, dtype=f32, device=dev))
    # The step as built (B = 64 runs as two halves on two graph branches) and as one chain of
    # launches, timed alternately.
    step = gsvk.T2SDecode(m, io, len_bound=max_len, graph=True)
    one = gsvk.T2SDecode(m, io, len_bound=max_len, graph=True, split=False)
    for _ in range(warmup):
        step.run()
        one.run()
    torch.cuda.synchronize()
    t_split, t_one = [], []
    for _ in range(3):
        t_split.append(time_loop(torch, step.run, steps))
        t_one.append(time_loop(torch, one.run, steps))
    ms, ms_one = statistics.median(t_split), statistics.median(t_one)
    one_launches = one.launches
    one.close()
    # One half of the batch alone (the first 32 sequences as one chain): how much of the step is
    # the chain's launch latency rather than its rows.
    sl = slice(0, B // 2)
    half = gsvk.T2SDecode(
        dict(m, layers=[dict(ly, k_cache=ly["k_cache"][sl], v_cache=ly["v_cache"][sl])
                        for ly in layers]),
        {n: (t[sl] if n != "err" else t) for n, t in io.items()}, len_bound=max_len, graph=True)
    for _ in range(warmup):
        half.run()
    ms_half = statistics.median(time_loop(torch, half.run, steps) for _ in range(3))
    half.close()
    assert int(io["err"].item()) == 0
    # algorithmic bytes: every weight and parameter once, the kv_len cached rows of K and V per
    # layer once, the appended rows, and each activation read / written once
    w_bytes = LAYERS * ((3 * D * D + D * D + 2 * FF * D) * 2 + (3 * D + 6 * D + FF) * 4) + V * D * 2
    kv_bytes = LAYERS * (2 * B * kv_len * D * 2)
    act_bytes = LAYERS * B * (D * 2 + 3 * D * 4 * 2 + D * 2 * 2 + D * 2 * 3 + D * 2 * 2 +
                              FF * 2 * 2 + D * 2 * 3 + D * 2 * 2) + B * V * 4 + B * D * 2
    nbytes = w_bytes + kv_bytes + act_bytes
    out = {"batch": B, "layers": LAYERS, "d_model": D, "ffn": FF, "heads": H, "vocab": V,
           "kv_len": kv_len, "storage": "f16", "kv_storage": "f16", "launches": step.launches,
           "us_per_step": round(ms * 1e3, 1), "tokens_per_s": round(B / ms * 1e3, 0),
           "one_chain_us_per_step": round(ms_one * 1e3, 1), "one_chain_launches": one_launches,
           "half_batch_chain_us_per_step": round(ms_half * 1e3, 1),
           "bytes_per_step": nbytes, "GBps": round(nbytes / ms / 1e6, 1),
           "frac_of_peak": round(nbytes / ms / 1e6 / PEAK_GBS, 4)}
    log(f"  whole decode step (B={B}, kv_len={kv_len}, graph of {step.launches} launches): "
        f"{out['us_per_step']} us, {out['tokens_per_s']:.0f} tokens/s, {out['GBps']} GB/s; "
        f"as one chain of {one_launches} launches {out['one_chain_us_per_step']} us; "
        f"half the batch alone {out['half_batch_chain_us_per_step']} us")
    step.close()
    del m, io, layers
    torch.cuda.empty_cache()
    return out


# ---- CPU baseline ----------------------------------------------------------------------------------

def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_topology():
    """Logical CPUs this process may run on, and the physical cores behind them (from
    /proc/cpuinfo: distinct (physical id, core id) pairs), so `cores` can be read either way."""
    logical = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    pairs, phys, core = set(), None, None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("physical id"):
                phys = line.split(":", 1)[1].strip()
            elif line.startswith("core id"):
                core = line.split(":", 1)[1].strip()
            elif not line.strip() and core is not None:
                pairs.add((phys, core))
                phys = core = None
    except OSError:
        pass
    return {"logical_cpus_allowed": logical, "hardware_threads": os.cpu_count(),
            "physical_cores_on_host": len(pairs) or None}


def cpu_baseline(torch, bufs, rep_s=0.3, reps=9):
    """The oracle's restatement of the same decode step on host copies of the same buffers, with
    the reference's bench convention (src/kern/bench_harness.hpp:8-13): 2 warm-up steps, then the
    median of `reps` repetitions (each a batch of steps lasting ~rep_s) and their coefficient of
    variation. Run on 1 thread and on every thread this process may use (rows split into bands, as
    rt::parallel_for does)."""
    import numpy as np

    import oracle as O

    def hostcopy(t):
        a = t.detach().cpu().contiguous()
        if a.dtype == torch.float16:
            return a.view(torch.int16).numpy().view(np.uint16).copy()
        return a.numpy().copy()

    hb = {k: ([hostcopy(t) for t in v] if isinstance(v, list) else
              (hostcopy(v) if hasattr(v, "device") else v)) for k, v in bufs.items()}
    hb["table_dtype"] = O.F16
    threads_all = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads_all = max(1, min(threads_all, 16, B))
    res = {}
    for threads in sorted({1, threads_all}):
        for _ in range(2):
            O.t2s_step(O.F16, hb, threads=threads)
        t0 = time.perf_counter()
        O.t2s_step(O.F16, hb, threads=threads)
        per_rep = max(1, int(rep_s / max(time.perf_counter() - t0, 1e-6)))
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            for _ in range(per_rep):
                O.t2s_step(O.F16, hb, threads=threads)
            times.append((time.perf_counter() - t0) / per_rep)
        med = statistics.median(times)
        cv = statistics.pstdev(times) / statistics.mean(times)
        res[threads] = {"s_per_step": med, "cv": cv, "steps": reps * per_rep, "per_rep": per_rep}
    return res, threads_all


def cpu_threads_all():
    """Every thread this process may run on, at most 16 (one GPU's share of the host)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return max(1, min(n or 1, 16))


def _bands(n, parts):
    """[lo, hi) bands of n items over at most `parts` workers (rt::parallel_for's even split)."""
    parts = max(1, min(parts, n))
    step = -(-n // parts)
    return [(lo, min(n, lo + step)) for lo in range(0, n, step)]


def cpu_kernel_lines():
    """The oracle's C restatement of every fused kernel line of the suite at its stated shape, as
    (make(threads) -> list of band calls, algorithmic bytes, rows). Each band call covers a band of
    rows (channels, output columns, sequences or elements) with preallocated outputs, so `threads`
    bands run at once from a thread pool (ctypes releases the interpreter lock for the call)."""
    import ctypes

    import numpy as np

    import oracle as O
    L = O.lib()
    r = np.random.default_rng(SEED + 21)
    ptr = lambda a, off=0: None if a is None else a.ctypes.data + off
    lines = {}

    def st(dt, *shape, std=1.0):
        return O.to_storage(dt, (std * r.standard_normal(shape)).astype(np.float32))

    def vec(n, mean=0.0, std=0.02):
        return (mean + std * r.standard_normal(n)).astype(np.float32)

    def ln(name, rows, n, dt, eps, bias, res, mode):
        esz = 4 if dt == O.F32 else 2
        x, rr = st(dt, rows, n), (st(dt, rows, n) if res else None)
        g, b, bi = vec(n, 1.0, 0.1), vec(n, 0.0, 0.1), (vec(n) if bias else None)
        y = np.empty_like(x)
        make = lambda T: [
            (lambda lo=lo, hi=hi: L.oracle_add_layernorm(
                dt, ptr(x, lo * n * esz), ptr(bi), ptr(rr, lo * n * esz), ptr(g), ptr(b),
                ptr(y, lo * n * esz), hi - lo, n, n, eps, mode)) for lo, hi in _bands(rows, T)]
        lines[name] = (make, ln_bytes(rows, n, esz, bias, res), rows)

    def bact(name, rows, n, act):
        x, bi = st(O.F16, rows, n), vec(n)
        make = lambda T: [
            (lambda lo=lo, hi=hi: L.oracle_bias_act(O.F16, act, ptr(x, lo * n * 2), ptr(bi),
                                                    ptr(x, lo * n * 2), hi - lo, n, n, 0.0))
            for lo, hi in _bands(rows, T)]
        lines[name] = (make, bias_act_bytes(rows, n, 2), rows)

    pe = O.pe_table(MAX_POS, D)

    def gathers(specs):
        """specs: (table, ids, pos or None, pos0, alpha, mm, bias, out) per gather of one call."""
        def make(T):
            calls = []
            for tab, ids, pos, pos0, alpha, mm, bias, out in specs:
                rows = ids.size
                for lo, hi in _bands(rows, T):
                    calls.append(lambda tab=tab, ids=ids, pos=pos, pos0=pos0, alpha=alpha, mm=mm,
                                 bias=bias, out=out, lo=lo, hi=hi: L.oracle_embed_pe(
                                     O.F16, O.F16, 0, ptr(tab), tab.shape[0], ptr(ids, 8 * lo),
                                     ptr(pos, 8 * lo), pos0 + lo, ptr(pe), MAX_POS, alpha,
                                     ptr(mm, lo * D * 2), ptr(bias), ptr(out, lo * D * 2), hi - lo, D))
            return calls
        return make

    def gather_line(name, rows, vocab, positions, nbytes, mm=False):
        tab = st(O.F16, vocab, D, std=0.02)
        ids = r.integers(0, vocab, rows).astype(np.int64)
        pos = positions(rows)
        out = np.empty((rows, D), np.uint16)
        m = st(O.F16, rows, D) if mm else None
        bias = vec(D) if mm else None
        lines[name] = (gathers([(tab, ids, pos, 0, 0.93, m, bias, out)]), nbytes, rows)

    rand_pos = lambda n: r.integers(0, MAX_POS, n).astype(np.int64)
    gather_line("embed_pe_prefill_1024x512", 1024, VOCAB, rand_pos, embed_bytes(1024, D, 2, 2))
    tab1 = st(O.F16, 1, D, std=0.02)
    z = np.zeros(1024, np.int64)
    lines["embed_pe_hot_row_ceiling_1024x512"] = (
        gathers([(tab1, z, z, 0, 0.93, None, None, np.empty((1024, D), np.uint16))]),
        embed_bytes(1024, D, 2, 2), 1024)
    tp, ts = st(O.F16, 732, D, std=0.02), st(O.F16, VOCAB, D, std=0.02)
    ip, isem = r.integers(0, 732, 512).astype(np.int64), r.integers(0, VOCAB, 512).astype(np.int64)
    two = gathers([(tp, ip, None, 0, 0.93, None, None, np.empty((512, D), np.uint16)),
                   (ts, isem, None, 0, 1.07, None, None, np.empty((512, D), np.uint16))])
    lines["embed_pe_prefill_pos0_511_2x512x512"] = (two, 1024 * (8 + 2 * D + 4 * D + 2 * D), 1024)
    lines["t2s_prefill_input_pos0_511_2x512x512"] = (
        two, 1024 * (8 + 2 * D + 2 * D) + 512 * 4 * D, 1024)
    lines["embed_pe_prefill_distinct_pos_2x512x512"] = (two, 1024 * (8 + 2 * D + 4 * D + 2 * D), 1024)
    gather_line("embed_pe_decode_64x512", 64, VOCAB, rand_pos, embed_bytes(64, D, 2, 2))
    tt = st(O.F16, 732, D, std=0.02)
    it = r.integers(0, 732, 512).astype(np.int64)
    mm, bb = st(O.F16, 512, D), vec(D)
    lines["embed_pe_text_rows_512x512"] = (
        gathers([(tt, it, None, 0, 0.93, mm, bb, np.empty((512, D), np.uint16))]),
        512 * (8 + 2 * D + 4 * D + 2 * D + 2 * D) + 4 * D, 512)

    ln("residual_layernorm_f32_256x512", 256, 512, O.F32, 1e-5, False, True, 0)
    ln("residual_layernorm_f16_64x512", 64, 512, O.F16, 1e-5, True, True, 0)
    bact("bias_relu_f16_64x2048", 64, 2048, 1)
    bact("bias_gelu_f16_512x4096", 512, 4096, 2)
    ln("residual_layernorm_f16_512x1024_eps1e-12", 512, 1024, O.F16, 1e-12, False, True, 1)
    ln("residual_layernorm_f16_499x768", 499, 768, O.F16, 1e-5, True, True, 0)
    bact("bias_gelu_f16_499x3072", 499, 3072, 2)

    C, T = 512, 31999
    gx = O.to_storage(O.F32, (0.5 * r.standard_normal((C, T))).astype(np.float32))
    gg, gb, gy = vec(C, 1.0, 0.1), vec(C, 0.0, 0.1), np.empty((C, T), np.float32)
    lines["groupnorm_gelu_f32_512x31999"] = (
        lambda Tn: [(lambda lo=lo, hi=hi: L.oracle_groupnorm_gelu(
            O.F32, ptr(gx, lo * T * 4), ptr(gg, 4 * lo), ptr(gb, 4 * lo), ptr(gy, lo * T * 4),
            hi - lo, T, T, 1e-5, 1)) for lo, hi in _bands(C, Tn)],
        gn_bytes(C, T, 4), C)

    E = 24 * 320000
    for dt, nm in ((O.F32, "f32"), (O.F16, "f16")):
        esz = 4 if dt == O.F32 else 2
        t, cur, tb, tin = st(dt, E), st(dt, E), st(dt, E), np.empty(E, O.storage_dtype(dt))
        curs, tbs, o = [st(dt, E) for _ in range(3)], [st(dt, E) for _ in range(3)], np.empty_like(t)

        def k3(lo, hi, dt=dt, esz=esz, curs=curs, tbs=tbs, o=o):
            ca = (ctypes.c_void_p * 3)(*[ptr(c, lo * esz) for c in curs])
            ta = (ctypes.c_void_p * 3)(*[ptr(c, lo * esz) for c in tbs])
            return lambda: L.oracle_resblock_branch_mean(dt, ca, ta, 3, ptr(o, lo * esz), hi - lo, 1,
                                                         0.1)
        lines[f"sovits_K1_{nm}_24x320000"] = (
            lambda T, dt=dt, esz=esz, t=t: [
                (lambda lo=lo, hi=hi: L.oracle_leaky_relu(dt, ptr(t, lo * esz), ptr(t, lo * esz),
                                                          hi - lo, 0.1)) for lo, hi in _bands(E, T)],
            2 * E * esz, 24)
        lines[f"sovits_K2_{nm}_24x320000"] = (
            lambda T, dt=dt, esz=esz, cur=cur, tb=tb, tin=tin: [
                (lambda lo=lo, hi=hi: L.oracle_resblock_add_lrelu(
                    dt, ptr(cur, lo * esz), ptr(tb, lo * esz), ptr(tin, lo * esz), hi - lo, 0.1))
                for lo, hi in _bands(E, T)],
            4 * E * esz, 24)
        lines[f"sovits_K3_{nm}_24x320000"] = (
            lambda T, k3=k3: [k3(lo, hi) for lo, hi in _bands(E, T)], 7 * E * esz, 24)

    def gemv(name, N, K, act, use_bias, use_res, ydt, M=B):
        yesz = 4 if ydt == O.F32 else 2
        x, w = st(O.F16, M, K), st(O.F16, N, K, std=0.05)
        bi = vec(N) if use_bias else None
        y = np.empty((M, N), O.storage_dtype(ydt))
        res = st(ydt, M, N) if use_res else None
        # bands of output columns: every band reads all M activation rows and its own weight rows
        make = lambda T: [
            (lambda lo=lo, hi=hi: L.oracle_gemv_f16w(
                O.F16, 1, ptr(x), K, ptr(w, lo * K * 2), ptr(bi, 4 * lo) if bi is not None else None,
                act, 0.0, ptr(res, lo * yesz), ydt, ptr(y, lo * yesz), N, M, hi - lo, K))
            for lo, hi in _bands(N, T)]
        nbytes = (N * K * 2 + M * K * 2 + M * N * yesz + (N * 4 if use_bias else 0) +
                  (M * N * yesz if use_res else 0))
        lines[name] = (make, nbytes, M)

    gemv("gemv_qkv_bias_f32out_64x1536x512", 1536, 512, 0, True, False, O.F32)
    gemv("gemv_outproj_bias_residual_64x512x512", 512, 512, 0, True, True, O.F16)
    gemv("gemv_w1_bias_relu_64x2048x512", 2048, 512, 1, True, False, O.F16)
    gemv("gemv_w2_bias_residual_64x512x2048", 512, 2048, 0, True, True, O.F16)
    gemv("gemv_logits_f32out_64x1025x512", 1025, 512, 0, False, False, O.F32)
    gemv("gemv_read_dominated_16x2048x512", 2048, 512, 0, False, False, O.F16, M=16)

    Ln, H = 1024, 16
    kc, vc = st(O.F16, B, Ln, D), st(O.F16, B, Ln, D)
    q = r.standard_normal((B, 3 * D)).astype(np.float32)
    apos = np.full(B, Ln - 1, np.int64)
    ao = np.empty((B, D), np.float32)
    lines["decode_attention_f16kv_64x1024x512"] = (
        lambda T: [(lambda lo=lo, hi=hi: L.oracle_decode_attention(
            O.F16, ptr(q, lo * 3 * D * 4), 3 * D, ptr(kc, lo * Ln * D * 2), ptr(vc, lo * Ln * D * 2),
            Ln, ptr(apos, 8 * lo), ptr(ao, lo * D * 4), D, hi - lo, H, D // H))
            for lo, hi in _bands(B, T)],
        2 * B * Ln * D * 2 + B * 3 * D * 4 + B * D * 2, B)
    return lines


def time_cpu_line(pool, calls, rep_s=0.03, reps=9):
    """The reference's bench convention (src/kern/bench_harness.hpp:8-13): 2 warm-up calls, then the
    median of `reps` repetitions (each a batch of calls lasting ~rep_s) and their coefficient of
    variation. The band calls of one call run at once on the pool (or inline for one band)."""
    if len(calls) == 1:
        run = calls[0]
    else:
        run = lambda: [f.result() for f in [pool.submit(c) for c in calls]]
    for _ in range(2):
        run()
    t0 = time.perf_counter()
    run()
    per_rep = max(1, int(rep_s / max(time.perf_counter() - t0, 1e-7)))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for _ in range(per_rep):
            run()
        times.append((time.perf_counter() - t0) / per_rep)
    med = statistics.median(times)
    return med, statistics.pstdev(times) / statistics.mean(times), per_rep


def cpu_kernel_baselines(names=None):
    """Per kernel line: the oracle at the stated shape on 1 thread and on every allowed thread
    (cpu_threads_all), GB/s over the line's algorithmic bytes and rows/s. Returns name -> record."""
    from concurrent.futures import ThreadPoolExecutor
    lines = cpu_kernel_lines()
    tall = cpu_threads_all()
    out = {}
    with ThreadPoolExecutor(max_workers=tall) as pool:
        for name, (make, nbytes, rows) in lines.items():
            if names is not None and name not in names:
                continue
            rec = {"bytes": nbytes, "rows": rows}
            for threads in sorted({1, tall}):
                s, cv, per_rep = time_cpu_line(pool, make(threads))
                rec[f"t{threads}"] = {"us": round(s * 1e6, 2), "GBps": round(nbytes / s / 1e9, 3),
                                      "rows_per_s": round(rows / s, 0), "cv": round(cv, 4),
                                      "calls_per_rep": per_rep}
            best = min((rec[k] for k in rec if k.startswith("t")), key=lambda v: v["us"])
            rec["best_GBps"] = best["GBps"]
            out[name] = rec
            log(f"  CPU {name}: 1 thread {rec['t1']['GBps']} GB/s, best {best['GBps']} GB/s")
    return out, tall


def next_tier_cpu(reps=3, which=("step", "conv")):
    """The next-tier rows whole, on the oracle's C restatement (the reference's own NEON /
    Accelerate code does not build on x86), on every allowed host thread (cpu_threads_all; ctypes
    releases the interpreter lock for each oracle call):
    - the whole T2S decode step at B = 64, kv_len 1024: 24 decoder layers, each with its own
      weights and fp16 K / V caches (3.2 GB in all), and the logits GEMV; the sequences split into
      one band per thread, each band running every layer on its sequences;
    - the 192 x 40000, k 11, dilation 5 ResBlock convolution with the LeakyReLU epilogue, its
      columns split into one band per thread, each band with its halo of (k - 1) dil columns.
    Median of `reps` runs each (after one untimed run); `which` picks the rows."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle as O
    r = np.random.default_rng(SEED + 11)
    threads = cpu_threads_all()

    def filled(shape):
        # fp16 storage tiled from a block of random values: every element finite, quick to build
        return np.resize(O.to_storage(O.F16, r.standard_normal(1 << 20).astype(np.float32)), shape)

    w = lambda n, k: (0.05 * r.standard_normal((n, k))).astype(np.float16).view(np.uint16)
    vec = lambda n, m=0.0: (m + 0.02 * r.standard_normal(n)).astype(np.float32)
    H, KV = 16, 1024
    layers = [] if "step" not in which else [dict(wqkv=w(3 * D, D), bqkv=vec(3 * D), wout=w(D, D), bout=vec(D),
                   n1g=vec(D, 1.0), n1b=vec(D), w1=w(FF, D), b1=vec(FF), w2=w(D, FF), b2=vec(D),
                   n2g=vec(D, 1.0), n2b=vec(D),
                   kc=filled((B, KV + 1, D)), vc=filled((B, KV + 1, D)))
              for _ in range(LAYERS)]
    x0 = O.to_storage(O.F16, r.standard_normal((B, D)).astype(np.float32))
    kv_pos = np.full(B, KV, np.int64)
    w_logits = w(VOCAB, D)

    def step_band(lo, hi):
        x = x0[lo:hi]
        for ly in layers:
            qkv = O.gemv_f16w(O.F16, x, ly["wqkv"], O.F32, bias=ly["bqkv"])
            attn = O.to_storage(O.F16, O.decode_attention(O.F16, qkv, ly["kc"][lo:hi],
                                                          ly["vc"][lo:hi], kv_pos[lo:hi], H,
                                                          D // H))
            z = O.gemv_f16w(O.F16, attn, ly["wout"], O.F16, bias=ly["bout"], residual=x)
            h = O.add_layernorm(O.F16, z, ly["n1g"], ly["n1b"], 1e-5)
            ff = O.gemv_f16w(O.F16, h, ly["w1"], O.F16, bias=ly["b1"], act=1)
            z = O.gemv_f16w(O.F16, ff, ly["w2"], O.F16, bias=ly["b2"], residual=h)
            x = O.add_layernorm(O.F16, z, ly["n2g"], ly["n2b"], 1e-5)
        return O.gemv_f16w(O.F16, x, w_logits, O.F32)

    C, T, k, dil = 192, 40000, 11, 5
    halo = (k - 1) * dil
    xs = r.standard_normal((C, T + halo)).astype(np.float32)
    wc = (r.standard_normal((C, C, k)) / np.sqrt(C * k)).astype(np.float16).view(np.uint16)
    bc = vec(C)
    conv_bands = _bands(T, threads)

    def conv_band(lo, hi):
        return O.conv1d(O.F32, np.ascontiguousarray(xs[:, lo:hi + halo]), wc, bc, dil, epi=1)

    def med(pool, calls):
        run = lambda: [f.result() for f in [pool.submit(c) for c in calls]]
        run()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            run()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    out = {}
    model = cpu_model()
    with ThreadPoolExecutor(max_workers=threads) as pool:
        if "step" in which:
            step_s = med(pool, [lambda lo=lo, hi=hi: step_band(lo, hi)
                                for lo, hi in _bands(B, threads)])
        if "conv" in which:
            t_conv = med(pool, [lambda lo=lo, hi=hi: conv_band(lo, hi) for lo, hi in conv_bands])
    del layers
    if "step" in which:
        out["t2s_whole_decode_step"] = {
            "value": round(B / step_s, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "us_per_step": round(step_s * 1e6, 0),
            "sample": f"the whole step: {LAYERS} decoder layers (QKV GEMV, attention over {KV} "
                      f"cached fp16 rows, out-proj, LN1, W1 + ReLU, W2, LN2), each with its own "
                      f"weights and caches, and the logits GEMV, at B={B}; sequences in {threads} "
                      f"bands; median of {reps}", "cpu_model": model}
    if "conv" in which:
        out["sovits_conv_192x40000_k11_d5"] = {
            "value": round(2.0 * C * C * k * T / t_conv / 1e12, 4), "unit": "TFLOP/s",
            "cores": threads, "kind": "port", "us": round(t_conv * 1e6, 0),
            "sample": f"all {T} columns in {len(conv_bands)} bands, each with its {halo}-column "
                      f"halo ({len(conv_bands) * halo} halo columns computed in all), fp32 (the "
                      f"oracle multiplies exactly) with the LeakyReLU epilogue; median of {reps}",
            "cpu_model": model}
    return out


# ---- decode-step ops, copy reference, counter workload ---------------------------------------------

def step_ops(gsvk, bufs):
    """Layer-0 launches of the step's three ops (residual+LN, bias+ReLU, gather+PE)."""
    x, h = bufs["x"], bufs["h"]
    L0 = lambda: gsvk.add_layernorm(bufs["attn_out"][0], bufs["n1g"][0], bufs["n1b"][0], h, 1e-5,
                                    bias=bufs["bout"][0], residual=x)
    R0 = lambda: gsvk.bias_act(gsvk.ACT_RELU, bufs["ff"][0], bufs["ff"][0], bias=bufs["b1"][0])
    E0 = lambda: gsvk.embed_pe(bufs["table"], bufs["ids"], bufs["pe"], bufs["alpha"], x,
                               pos=bufs["pos"], err=bufs["err"])
    return L0, R0, E0


def step_layer_sweep(torch, gsvk, bufs, layers=(1, 2, 4, 8, 16, 24)):
    """The fused step over the first L layers of the same buffers, device time per launch (a graph
    of 32 back-to-back launches; eager launches from Python would measure the host's launch rate
    at few layers): the per-layer slope of the chain and the fixed cost of one launch."""
    out = {}
    for L in layers:
        b = dict(bufs)
        for k in ("attn_out", "ff", "ffn_out", "bout", "b1", "b2", "n1g", "n2g", "n1b", "n2b"):
            b[k] = bufs[k][:L]
        st = gsvk.T2SStep(b, eps=1e-5, graph=False, fused=True)
        us = graph_us_per_launch(torch, st.run, launches=32, replays=20)
        st.close()
        out[L] = round(us, 3)
        log(f"  fused step, {L} layers: {us:.3f} us")
    return out


def copy_bandwidth(torch, dev, nbytes=1 << 30):
    """A plain device-to-device copy of 1 GiB (read + write counted), timed like the replicated
    kernels: the achievable-bandwidth reference of this GPU under the same method."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    ms = measure_reps(torch, lambda: dst.copy_(src), Flusher(torch, dev))
    del src, dst
    torch.cuda.empty_cache()
    gbs = 2 * nbytes / ms / 1e6
    log(f"  copy 1 GiB: {gbs:.1f} GB/s ({100 * gbs / PEAK_GBS:.1f}%)")
    return round(gbs, 1)


DIAG_COPY = ("row_resident_nt_stores", "row_resident_cached_stores", "block_nt_stores",
             "block_cached_stores")
DIAG_READ = ("gemv_fragment_loads", "contiguous_rows", "direct_to_lds_depth2",
             "direct_to_lds_depth4", "block_read")


def diag_forms(torch, dev):
    """Ceilings of the access patterns the streaming kernels use, from the measurement kernels of
    gpt-sovits-native_amd/diag/gsvk_diag.hip (libgsvk_diag.so):

    - copy forms over a [4096, 32000] fp32-sized tensor (524 MB read + 524 MB written), as a whole
      row per workgroup (all of a row's loads before any store: GroupNorm's order) and as one-shot
      32 KiB blocks (the element-wise streams' order), each with non-temporal or cached stores;
    - read forms of a 128 MiB weight stream in 32-row batches, one 4-wave workgroup per CU (the
      long-stream GEMV's partition): its fragment loads, contiguous rows, direct-to-LDS loads at
      two and four batches in flight, and a plain one-shot read.

    Each form: the median of 9 launches with the MALL cleared before each (how every suite line is
    timed), and 10 launches back to back (per launch; no clearing: a launch then also pays for the
    write-back of the dirty lines the one before it left in the MALL)."""
    import ctypes
    path = os.path.join(ROOT, "gpt-sovits-native_amd", "libgsvk_diag.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run make -C gpt-sovits-native_amd libgsvk_diag.so")
    lib = ctypes.CDLL(path)
    lib.gsvk_diag_copy.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_size_t, ctypes.c_void_p]
    lib.gsvk_diag_stream_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_void_p, ctypes.c_void_p]
    flush = Flusher(torch, dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    out = {"copy": {}, "read": {}}

    def timed(call, nbytes):
        rc = call()
        if rc != 0:
            raise RuntimeError(f"diag call returned {rc}")
        one = measure_reps(torch, call, flush)
        flush()
        ten = time_loop(torch, call, 10, warmup=0)
        return {"one_us": round(one * 1e3, 1), "one_frac": round(nbytes / one / 1e6 / PEAK_GBS, 4),
                "x10_us": round(ten * 1e3, 1), "x10_frac": round(nbytes / ten / 1e6 / PEAK_GBS, 4)}

    rows, row_bytes = 4096, 128000
    x = torch.ones(rows * row_bytes, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    for f, name in enumerate(DIAG_COPY):
        out["copy"][name] = timed(
            lambda f=f: lib.gsvk_diag_copy(f, x.data_ptr(), y.data_ptr(), rows, row_bytes, stream),
            2 * rows * row_bytes)
        progress(f"diag copy {name}: {out['copy'][name]}")
    del x, y
    torch.cuda.empty_cache()
    wrows = 131072
    w = torch.ones(wrows * 1024, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    for f, name in enumerate(DIAG_READ):
        out["read"][name] = timed(
            lambda f=f: lib.gsvk_diag_stream_read(f, w.data_ptr(), wrows, sink.data_ptr(), stream),
            wrows * 1024)
        progress(f"diag read {name}: {out['read'][name]}")
    del w
    torch.cuda.empty_cache()
    return out


def write_bandwidth(torch, dev, nbytes=1 << 30):
    """A write-only stream of 1 GiB (torch's fill kernel: 16-byte stores, nothing read), timed like
    the replicated kernels: the achievable HBM write bandwidth, the ceiling of write-dominated
    kernels such as the gather (1 KiB row written per 16 B of ids read; its table and PE reads are
    served from the caches)."""
    dst = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    ms = measure_reps(torch, lambda: dst.fill_(1.0), Flusher(torch, dev))
    del dst
    torch.cuda.empty_cache()
    gbs = nbytes / ms / 1e6
    log(f"  write-only 1 GiB: {gbs:.1f} GB/s ({100 * gbs / PEAK_GBS:.1f}%)")
    return round(gbs, 1)


PMC_COPY_BYTES = 256 << 20
PMC_LAUNCHES = 30
PMC_KERNEL = "t2s_step_fused"


def pmc_workload(torch, gsvk, bufs):
    """For `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`: PMC_LAUNCHES launches of the step's
    kernel (t2s_step_fused, the whole decode-step epilogue chain), each after a 512 MiB read that
    clears the MALL (so the step's inputs come from HBM, as in a decode loop where the GEMVs
    stream 150 MB of weights between steps), and 10 plain copies of PMC_COPY_BYTES (the
    calibration: its counters per dispatch against its known bytes)."""
    step = gsvk.T2SStep(bufs, eps=1e-5, graph=False, fused=True)
    flush = Flusher(torch, bufs["x"].device)
    for _ in range(PMC_LAUNCHES):
        flush()
        step.run()
    src = torch.ones(PMC_COPY_BYTES // 4, dtype=torch.float32, device=bufs["x"].device)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"pmc workload: {PMC_LAUNCHES} x {PMC_KERNEL} (MALL cleared before each), "
        f"10 x copy {PMC_COPY_BYTES} B")


def ln_param_traffic_workload(torch, gsvk, bufs):
    """For `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE`: 100 launches of residual+LN [64, 512] f16
    with its bias / gamma / beta (6 KiB of fp32 parameters), then 100 launches of the same call
    without them, each after a 512 MiB read that clears the MALL, and 10 copies of PMC_COPY_BYTES
    (the counter calibration). The per-dispatch difference of the two sets is the parameter
    vectors' share of the launch's fetched bytes."""
    L0, _, _ = step_ops(gsvk, bufs)
    x, h = bufs["x"], bufs["h"]
    bare = lambda: gsvk.add_layernorm(bufs["attn_out"][0], None, None, h, 1e-5, residual=x)
    flush = Flusher(torch, x.device)
    for fn in (L0, bare):
        for _ in range(100):
            flush()
            fn()
    src = torch.ones(PMC_COPY_BYTES // 4, dtype=torch.float32, device=x.device)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("ln param traffic workload: 100 x LN [64,512] f16 with parameters, 100 without, "
        f"10 x copy {PMC_COPY_BYTES} B")


def measure_traffic(timeout_s=150):
    """HBM-side traffic of one launch of the step's kernel: two `rocprofv3 --pmc` child runs of
    this script's --pmc workload (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what
    the same counter reads for the PMC_COPY_BYTES copy in that workload. Returns (dict, None) or
    (None, reason)."""
    import csv
    import glob
    import subprocess
    import tempfile

    vals = {}
    with tempfile.TemporaryDirectory(prefix="gsvk_pmc_") as td:
        for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
            cmd = ["rocprofv3", "--pmc", ctr, "-f", "csv", "-d", td, "-o", ctr.lower(), "--",
                   sys.executable, os.path.abspath(__file__), "--pmc"]
            try:
                subprocess.run(cmd, cwd=td, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                               timeout=timeout_s, env=dict(os.environ, TMPDIR=td))
            except (OSError, subprocess.TimeoutExpired) as exc:
                return None, f"{ctr}: {type(exc).__name__}"
            # rocprofv3 can exit non-zero after writing complete results; the CSV decides
            files = glob.glob(os.path.join(td, "**", f"{ctr.lower()}_counter_collection.csv"),
                              recursive=True)
            if not files:
                return None, f"{ctr}: no counter file"
            ln, cp = [], []
            for r in csv.DictReader(open(files[0])):
                if r["Counter_Name"] != ctr:
                    continue
                v = float(r["Counter_Value"])
                if PMC_KERNEL in r["Kernel_Name"]:
                    ln.append(v)
                elif "copyBuffer" in r["Kernel_Name"] or "copy" in r["Kernel_Name"].lower():
                    cp.append(v)
            if len(ln) < PMC_LAUNCHES or not cp:
                return None, f"{ctr}: {len(ln)} kernel / {len(cp)} copy dispatches found"
            vals[ctr] = (statistics.median(ln), max(cp))
    kib = PMC_COPY_BYTES / 1024
    f_fetch, f_write = kib / vals["FETCH_SIZE"][1], kib / vals["WRITE_SIZE"][1]
    traffic = 1024 * (vals["FETCH_SIZE"][0] * f_fetch + vals["WRITE_SIZE"][0] * f_write)
    return {"bytes": round(traffic), "fetch_kib": vals["FETCH_SIZE"][0],
            "write_kib": vals["WRITE_SIZE"][0], "fetch_scale": round(f_fetch, 4),
            "write_scale": round(f_write, 4)}, None


PMC_LINE_LAUNCHES = 5


def pmc_line_workload(torch, gsvk, dev, name):
    """For `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE`: the replicated launch of one suite line
    once to warm, then PMC_LINE_LAUNCHES times each after a 512 MiB read that clears the MALL, then
    10 plain copies of PMC_COPY_BYTES (the calibration). Prints the line's algorithmic bytes."""
    cap = {}
    kernel_suite(torch, gsvk, dev, only=name, capture=cap)
    if not cap:
        raise SystemExit(f"no suite line named {name}")
    flush = Flusher(torch, dev)
    cap["fn"]()
    torch.cuda.synchronize()
    for _ in range(PMC_LINE_LAUNCHES):
        flush()
        cap["fn"]()
    torch.cuda.synchronize()
    src = torch.ones(PMC_COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"line": name, "instances": cap["instances"], "bytes": cap["bytes"]}), flush=True)


def _counter_rows(path, ctr):
    """(kernel name, value) per dispatch of counter `ctr` in a rocprofv3 counter CSV, in dispatch
    order."""
    import csv
    rows = []
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == ctr:
            rows.append((int(r.get("Dispatch_Id") or r.get("Correlation_Id") or len(rows)),
                         r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(k, v) for _, k, v in rows]


def line_traffic(names, timeout_s=180):
    """HBM traffic per replicated launch of each named suite line: two `rocprofv3 --pmc` child runs
    of this script's --pmc-line workload (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch). The
    library's dispatches (kernel names in namespace gsvk) of one call are summed, the median over
    the PMC_LINE_LAUNCHES timed calls taken, and each counter scaled by what it reads for the
    PMC_COPY_BYTES copy of the same run. Returns name -> record."""
    import glob
    import subprocess
    import tempfile

    out = {}
    for name in names:
        rec = {}
        with tempfile.TemporaryDirectory(prefix="gsvk_pmc_") as td:
            for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
                cmd = ["rocprofv3", "--pmc", ctr, "-f", "csv", "-d", td, "-o", ctr.lower(), "--",
                       sys.executable, os.path.abspath(__file__), "--pmc-line", name]
                try:
                    p = subprocess.run(cmd, cwd=td, capture_output=True, text=True,
                                       timeout=timeout_s, env=dict(os.environ, TMPDIR=td))
                except (OSError, subprocess.TimeoutExpired) as exc:
                    rec["error"] = f"{ctr}: {type(exc).__name__}"
                    break
                for ln in p.stdout.splitlines():
                    if ln.startswith("{") and '"line"' in ln:
                        rec.update({k: v for k, v in json.loads(ln).items() if k != "line"})
                files = glob.glob(os.path.join(td, "**", f"{ctr.lower()}_counter_collection.csv"),
                                  recursive=True)
                if not files:
                    rec["error"] = f"{ctr}: no counter file (rc {p.returncode})"
                    break
                rows = _counter_rows(files[0], ctr)
                lib_rows = [v for k, v in rows if "gsvk::" in k]
                copies = [v for k, v in rows if "copy" in k.lower()][-10:]
                n = PMC_LINE_LAUNCHES + 1
                if not copies or not lib_rows or len(lib_rows) % n:
                    rec["error"] = f"{ctr}: {len(lib_rows)} library / {len(copies)} copy dispatches"
                    break
                kpc = len(lib_rows) // n
                calls = [sum(lib_rows[i * kpc:(i + 1) * kpc]) for i in range(1, n)]
                scale = PMC_COPY_BYTES / 1024 / statistics.median(copies)
                rec[ctr.lower() + "_bytes"] = round(statistics.median(calls) * scale * 1024)
                rec[ctr.lower() + "_scale"] = round(scale, 4)
                rec["dispatches_per_call"] = kpc
        if "error" not in rec:
            rec["traffic"] = rec["fetch_size_bytes"] + rec["write_size_bytes"]
            rec["traffic_over_algorithmic"] = round(rec["traffic"] / rec["bytes"], 3)
        out[name] = rec
        progress(f"traffic {name}: " + (rec.get("error") or
                                        f"{rec['traffic']} B for {rec['bytes']} algorithmic "
                                        f"({rec['traffic_over_algorithmic']}x)"))
    return out


def traffic_table(res):
    """Markdown table of line_traffic's records."""
    rows = ["| line | instances | algorithmic B | FETCH B | WRITE B | traffic / algorithmic |",
            "|---|---|---|---|---|---|"]
    for name, r in res.items():
        if "error" in r:
            rows.append(f"| {name} | | | | | {r['error']} |")
        else:
            rows.append(f"| {name} | {r['instances']} | {r['bytes']:,} | {r['fetch_size_bytes']:,} "
                        f"| {r['write_size_bytes']:,} | {r['traffic_over_algorithmic']:.3f} |")
    return "\n".join(rows)


# ---- main --------------------------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-kernels", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, help="run one kernel of the suite and exit")
    ap.add_argument("--pmc", action="store_true",
                    help="run the step kernel and a plain copy only (for rocprofv3 --pmc)")
    ap.add_argument("--step-layers", action="store_true",
                    help="the fused step over 1..24 layers of the same buffers (per-layer slope)")
    ap.add_argument("--ln-traffic", action="store_true",
                    help="LN [64,512] with and without parameters + a copy (rocprofv3 --pmc runs)")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc child runs that measure roofline.traffic")
    ap.add_argument("--conv", action="store_true",
                    help="time the SoVITS ResBlock convolutions per decoder stage and exit")
    ap.add_argument("--decoder", action="store_true",
                    help="the SoVITS Generator stages and the whole decoder graph only (rocprofv3 runs)")
    ap.add_argument("--whole-step", type=int, default=0, metavar="KV_LEN",
                    help="run only the whole T2S decode step at this KV length (rocprofv3 runs)")
    ap.add_argument("--pmc-line", default=None, metavar="LINE",
                    help="one suite line's replicated launch + a copy (for rocprofv3 --pmc runs)")
    ap.add_argument("--line-traffic", default=None, metavar="LINES",
                    help="FETCH_SIZE / WRITE_SIZE per replicated launch of the named suite lines "
                         "(comma-separated, or 'all'), each from two rocprofv3 --pmc child runs")
    ap.add_argument("--conv-one", default=None, metavar="C,T,K,DIL,EPI",
                    help="one SoVITS ResBlock convolution shape, 22 launches (rocprofv3 --pmc runs)")
    ap.add_argument("--diag", action="store_true",
                    help="the copy and weight-stream read forms of libgsvk_diag.so (access-pattern "
                         "ceilings) and exit")
    ap.add_argument("--cpu-lines", action="store_true",
                    help="the oracle's CPU baseline of every suite line only")
    ap.add_argument("--detail", default=os.path.join(ROOT, "gpurun_out", "bench_detail.json"),
                    help="where the full record goes (the last stdout line is the headline only)")
    ap.add_argument("--verbose", action="store_true",
                    help="print every measurement line to stderr as it comes")
    a = ap.parse_args()
    global VERBOSE
    VERBOSE = a.verbose
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every kernel here is row- or element-local, so more "
              "GPUs would each run an independent share (no figure at several GPUs is produced).",
              file=sys.stderr)
        sys.exit(2)

    if a.cpu_lines:
        res, tall = cpu_kernel_baselines()
        print(json.dumps({"threads_all": tall, "cpu_model": cpu_model(), **cpu_topology(),
                          "lines": res}), flush=True)
        return
    if a.line_traffic:
        import gsvk
        import torch
        names = (kernel_suite(torch, gsvk, None, only="__names__") if a.line_traffic == "all"
                 else a.line_traffic.split(","))
        res = line_traffic(names)
        write_detail({"line_traffic": res}, a.detail)
        print(traffic_table(res), flush=True)
        return

    import torch

    import gsvk
    gsvk.lib()  # fails loudly when libgsvk.so is missing
    dev = torch.device("cuda:0")

    if a.pmc_line:
        pmc_line_workload(torch, gsvk, dev, a.pmc_line)
        return
    if a.only == "write_bandwidth":
        write_bandwidth(torch, dev)
        return
    if a.diag:
        print(json.dumps(diag_forms(torch, dev)), flush=True)
        return
    if a.conv_one:
        print(json.dumps(conv_one(torch, gsvk, dev, a.conv_one)), flush=True)
        return
    if a.only:
        kernel_suite(torch, gsvk, dev, only=a.only)
        return
    if a.whole_step:
        print(json.dumps(full_decode_step(torch, gsvk, dev, kv_len=a.whole_step)), flush=True)
        return
    if a.decoder:
        print(json.dumps(sovits_generator(torch, gsvk, dev)), flush=True)
        return
    if a.conv:
        res = sovits_conv(torch, gsvk, dev)
        res["generator"] = sovits_generator(torch, gsvk, dev)
        if not a.no_cpu:
            res["cpu_baseline"] = next_tier_cpu(which=("conv",))["sovits_conv_192x40000_k11_d5"]
        print(json.dumps(res), flush=True)
        return

    bufs = make_step_buffers(torch, gsvk, dev)
    if a.pmc:
        pmc_workload(torch, gsvk, bufs)
        return
    if a.ln_traffic:
        ln_param_traffic_workload(torch, gsvk, bufs)
        return
    if a.step_layers:
        print(json.dumps({"fused_step_us_by_layers": step_layer_sweep(torch, gsvk, bufs)}))
        return
    nbytes = step_bytes()

    def time_step(st):
        for _ in range(a.warmup):
            st.run()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(a.steps):
            st.run()
        e.record()
        e.synchronize()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / a.steps

    # The step as one launch (gsvk_t2s_step_fused), launched directly per step: the headline.
    # The same launch recorded as a one-node graph is timed beside it.
    step = gsvk.T2SStep(bufs, eps=1e-5, graph=False, fused=True)
    ms = time_step(step)
    assert int(bufs["err"].item()) == 0
    log(f"decode step (one fused launch): {ms * 1e3:.2f} us")
    step_g = gsvk.T2SStep(bufs, eps=1e-5, graph=True, fused=True)
    ms_g = time_step(step_g)
    step_g.close()
    log(f"decode step (one fused launch as a one-node graph): {ms_g * 1e3:.2f} us")
    # The same step as the 73 per-op launches (one graph), for comparison.
    step73 = gsvk.T2SStep(bufs, eps=1e-5, graph=True)
    ms73 = time_step(step73)
    log(f"decode step (graph, {step73.launches} launches): {ms73 * 1e3:.2f} us")
    step73.close()
    progress(f"decode step: {ms * 1e3:.2f} us eager (one launch), {ms_g * 1e3:.2f} us as a "
             f"one-node graph, {ms73 * 1e3:.2f} us as {1 + 3 * LAYERS} launches")

    # per-op breakdown at the step's shapes: graphs of 48 back-to-back launches of each op
    L0, R0, E0 = step_ops(gsvk, bufs)
    per_op = {}
    for name, fn, cnt, byt in (("residual_layernorm", L0, 48, ln_bytes(B, D, 2)),
                               ("bias_relu", R0, 24, bias_act_bytes(B, FF, 2)),
                               ("embed_pe", E0, 1, embed_bytes(B, D, 2, 2))):
        gr = graph_of(torch, fn, 48)
        us = time_loop(torch, gr.replay, 20) * 1e3 / 48
        per_op[name] = {"us_per_launch": round(us, 3), "launches_per_step": cnt, "bytes": byt,
                        "GBps": round(byt / us / 1e3, 1),
                        "rows_per_s": round(B / us * 1e6, 0)}
        del gr

    # Roofline of the step's one kernel (t2s_step_fused): the step's algorithmic bytes over its
    # device time per launch, HIP events around a graph of 32 back-to-back launches on the launch
    # stream.
    us_fused = graph_us_per_launch(torch, step.run, launches=32, replays=20)
    ach = nbytes / us_fused / 1e3
    roofline = {"kernel": f"t2s_step_fused [B={B}, D={D}, FF={FF}, {LAYERS} layers] f16",
                "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_GBS, 5), "traffic": None,
                "bytes_per_launch": nbytes, "us_per_launch": round(us_fused, 3),
                "rows_per_s": round(B * (1 + 3 * LAYERS) / us_fused * 1e6, 0)}

    if not a.no_traffic:
        tr, why = measure_traffic()
        if tr:
            roofline["traffic"] = tr["bytes"]
            roofline["traffic_detail"] = tr
            log(f"  traffic: {tr['bytes']} B per launch ({tr})")
        else:
            roofline["traffic_error"] = why
            log(f"  traffic not measured: {why}")

    progress(f"roofline: t2s_step_fused {us_fused:.2f} us per launch = {ach:.0f} GB/s "
             f"({100 * ach / PEAK_GBS:.1f}% of 8 TB/s), traffic {roofline['traffic']}")
    cpu = None
    if not a.no_cpu:
        res, tall = cpu_baseline(torch, bufs)
        best = res[tall]
        cpu = {"value": round(nbytes / best["s_per_step"] / 1e9, 3), "unit": "GB/s", "cores": tall,
               "kind": "port",
               "sample": f"median of 9 repetitions x {best['per_rep']} decode steps (B={B}, "
                         f"{LAYERS} layers, fp16 storage) of the oracle's C restatement, rows split "
                         f"over {tall} threads; 2 warm-up steps",
               "us_per_step": round(best["s_per_step"] * 1e6, 1), "cv": round(best["cv"], 4),
               "rows_per_s": round(B * (1 + 3 * LAYERS) / best["s_per_step"], 0),
               "single_thread_us_per_step": round(res[1]["s_per_step"] * 1e6, 1),
               "single_thread_cv": round(res[1]["cv"], 4),
               "cpu_model": cpu_model(), **cpu_topology(), "threads_used": tall}

    kernels = copy_gbs = write_gbs = decoder = full = conv = cpu_lines = None
    if not a.no_kernels:
        copy_gbs = copy_bandwidth(torch, dev)
        write_gbs = write_bandwidth(torch, dev)
        kernels = kernel_suite(torch, gsvk, dev)
        progress(f"kernel suite: {len(kernels)} lines")
        decoder = sovits_decoder(torch, gsvk, dev)
        full = [full_decode_step(torch, gsvk, dev, kv_len=n) for n in (1024, 2048)]
        progress("whole decode step: " + ", ".join(f"kv {r['kv_len']} {r['us_per_step']} us"
                                                  for r in full))
        conv = sovits_conv(torch, gsvk, dev)
        conv["generator"] = sovits_generator(torch, gsvk, dev)
        progress(f"SoVITS decoder graph: {conv['generator']['decoder']['us']} us per 10 s of audio "
                 f"(eager on three streams: {conv['generator']['decoder'].get('eager_us')} us)")
        if not a.no_cpu:
            cpu_lines, tall = cpu_kernel_baselines()
            for rec in kernels:
                c = cpu_lines.get(rec["kernel"])
                if c:
                    rec["cpu"] = c
                    rec["vs_cpu_best"] = round(rec["stated_shape"]["GBps"] / c["best_GBps"], 1)
            progress(f"CPU baselines: {len(cpu_lines)} kernel lines on 1 and {tall} threads")
            nt = next_tier_cpu()
            full[0]["cpu_baseline"] = nt["t2s_whole_decode_step"]
            full[0]["vs_cpu"] = round(full[0]["tokens_per_s"] / nt["t2s_whole_decode_step"]["value"], 1)
            conv["cpu_baseline"] = nt["sovits_conv_192x40000_k11_d5"]
            big = [c for c in conv["stages"][1]["convs"] if c["k"] == 11 and c["dil"] == 5][0]
            conv["vs_cpu"] = round(conv["cpu_baseline"]["us"] / big["us"], 1)

    rec = {
        "metric": METRIC, "value": round(nbytes / ms / 1e6, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded normal activations / parameters, uniform ids and positions)",
        "config": {"workload": "t2s_decode_step_epilogues", "batch": B, "d_model": D, "ffn": FF,
                   "layers": LAYERS, "storage": "f16", "launches_per_step": step.launches,
                   "fused": True, "bytes_per_step": nbytes, "us_per_step": round(ms * 1e3, 3),
                   "frac_of_peak": round(nbytes / ms / 1e6 / PEAK_GBS, 5),
                   "rows_per_s": round(B * (1 + 3 * LAYERS) / ms * 1e3, 0),
                   "tokens_per_s": round(B / ms * 1e3, 0), "graph": False,
                   "one_node_graph_us_per_step": round(ms_g * 1e3, 3),
                   "per_op_graph_us_per_step": round(ms73 * 1e3, 3),
                   "per_op_graph_launches": 1 + 3 * LAYERS},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "per_op": per_op,
        "copy_GBps": copy_gbs,
        "write_only_GBps": write_gbs,
        "kernels": kernels,
        "sovits_decoder": decoder,
        "t2s_whole_decode_step": full,
        "sovits_conv": conv,
    }
    rec["detail_file"] = write_detail(rec, a.detail)
    step.close()
    print(headline_line(rec), flush=True)


if __name__ == "__main__":
    main()
