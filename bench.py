"""Benchmark of the per-layer op chain on one MI355X.

Default run (the driver's contract): BASELINE.json configs[2] -- the
Llama-3-8B-shape prefill chain at T = 4096 tokens, fp32:
    gather (F32 embedding, Zipf(1.1) ids) -> residual add + RMSNorm
    -> RoPE on Q [T, 32, 128] and K [T, 8, 128] (positions 0..T-1)
    -> SwiGLU over gate/up [T, 14336]
One step is one pass of the four kernels over one of three rotating buffer
sets (~1 GB each, so no step finds its inputs in the 256 MB MALL).  Inputs
are synthetic, generated on the device, resident in HBM before timing.
`value` is whole-chain GB/s over K timed steps (events only at the two
ends); the gather counts each distinct table row once (Zipf ids repeat hot
rows, which come from cache).  Per-kernel durations come from a second
timed pass that launches each kernel K times back to back between two HIP
events recorded on the stream the kernels run on.

The same run measures the other configs of BASELINE.json into "configs":
configs[0] (the tiny chain), configs[1] (decode steps at T = 1..64, eager
and graph-replayed), configs[3] (Q8_0/Q4_0/Q4_1 gathers) and configs[4]
(the 70B chain), each beside the reference's CPU code timed on this host;
and "decode_layer_8b": one Llama-3-8B layer through mlk_forward_layer_batch
as a decode step (one token at position 8191, and 16 tokens at positions in
0..8191; Q8_0 / Q4_0 on their planar copies), Q8_0 / Q4_0 / F32, weights
rotated over 4 layers; and "prefill_layer_8b": the same layer (Q8_0) over
a 4096-token prompt chunk at positions 0..4095.
Before each measured section a ZeroKernel launch of 4096 * (100 + i) bytes
marks section i in a rocprofv3 trace (bench.py --rocprof-report uses it).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

W (default 500) untimed steps precede the K timed ones: the GPU raises its
clock over tens of ms of sustained work, so a short warmup times the ramp.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402

mlk_pkg = entry.load_package()
import cpp_minilamma_amd.workloads as workloads  # noqa: E402

METRIC = ("HBM GB/s (% of peak) per fused op; µs per layer op-chain, 8B shape T=1/4096")
PMC_FILE = os.path.join(ROOT, "profiles", "swiglu_c3_prefill_8b_traffic.json")
N_SETS = 3


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    # 500 steps (about 0.1 s of the C3 chain): the GPU's clock reaches its
    # steady state only after tens of ms of sustained work, and 10 steps
    # (2 ms) timed the chain about 2.5% slower
    p.add_argument("--warmup", type=int, default=500)
    p.add_argument("--linear", default=None,
                   help="only measure the seven linear projections of one Llama-3-8B layer "
                        "(F32, Q8_0, Q4_0, Q4_1 weights; T = 1, 4, 16 token rows) into this "
                        "JSON file")
    p.add_argument("--linear-eager", action="store_true",
                   help="with --linear: issue each projection's calls as eager launches "
                        "instead of one replayed HIP graph (for a rocprofv3 kernel trace: "
                        "rocprofv3 7.2 faults tracing replays of the three-kernel planar calls); "
                        "the same marker kernels bracket the timed calls")
    p.add_argument("--gemm", default=None,
                   help="only measure the seven Llama-3-8B layer projections at prefill row counts "
                        "(32 to 4096; the matrix-core GEMM) into this JSON file")
    p.add_argument("--layer", default=None,
                   help="only measure one Llama-3-8B layer over a 4096-token prompt chunk "
                        "(mlk_forward_layer_batch), with a token-by-token comparison, into "
                        "this JSON file")
    p.add_argument("--decode-layer", default=None,
                   help="only measure one Llama-3-8B layer as a decode step (one token at "
                        "position 8191; 16 tokens at positions in 0..8191; Q8_0 / Q4_0 on "
                        "planar copies, F32), the default run's decode_layer_8b section, into "
                        "this JSON file")
    p.add_argument("--attention", default=None,
                   help="only measure decode attention (Llama-3-8B and 70B head shapes, one "
                        "token at several context lengths and configs[1]'s 64 tokens) into "
                        "this JSON file")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--rocprof-report", nargs=5, default=None,
                   metavar=("KERNEL_TRACE_DIR", "FETCH_DIR", "WRITE_DIR", "CALIB_FETCH_DIR",
                            "CALIB_WRITE_DIR"),
                   help="summarize rocprofv3 CSV output of the default command (kernel trace) "
                        "and of the --pmc FETCH_SIZE / WRITE_SIZE runs into profiles/")
    p.add_argument("--kernel-summary", nargs="+", default=None,
                   metavar="ARG",
                   help="OUT_MD TITLE BENCH_JSON KERNEL_TRACE_DIR [FETCH_DIR WRITE_DIR]: write a "
                        "rocprofv3 summary (per kernel and grid: calls, avg/min us, and HBM bytes "
                        "from FETCH_SIZE / WRITE_SIZE scaled by the committed calibration) of a "
                        "--linear or --attention run, with that run's JSON results, into OUT_MD; "
                        "the commands that produced the inputs are read from the environment "
                        "variable PROFILE_COMMANDS (one per line)")
    p.add_argument("--pmc-summary", nargs=3, default=None,
                   metavar=("OUT_MD", "TITLE", "COUNTER_DIR"),
                   help="write the mean of every counter of a rocprofv3 --pmc run per kernel and "
                        "grid into OUT_MD (the commands from PROFILE_COMMANDS, one per line)")
    p.add_argument("--calibrate", action="store_true",
                   help="only run the counter-calibration kernel (SiLU over 256 MiB: "
                        "reads 256 MiB, writes 256 MiB per launch)")
    return p.parse_args()


# buffers each op touches; run_ops rotates an op over extra sets of only these
OP_FIELDS = {"gather_f32": ("x",), "add_rmsnorm": ("x", "delta", "y"), "rope": ("q", "k"),
             "swiglu": ("gate", "up", "out")}
OP_WORKING_SET = 768 << 20  # bytes one pass of an op's rotation touches: 3x the 256 MB MALL
OP_MAX_SETS = 16  # decode-size buffers stay cache-resident, as in a real decode step


class ChainSet:
    """Device buffers of one op-chain input/output set (or of `fields` only).
    x is the gather's output in a chain step; it is filled when the set has
    no gather (`fill_x`) or holds only some fields."""

    def __init__(self, mlk, cfg, T, seed, fields=None, fill_x=False):
        D, H, KV, hd, F = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"]
        shapes = {"x": (T, D), "delta": (T, D), "y": (T, D), "q": (T, H * hd),
                  "k": (T, KV * hd), "gate": (T, F), "up": (T, F), "out": (T, F)}
        filled = {"x": 0, "delta": 1, "q": 2, "k": 3, "gate": 4, "up": 5}
        std = cfg.get("act_std", 0.02)  # activations: N(0, 1) for configs[0], else N(0, 0.02)
        self.nbytes = 0
        for name in fields or shapes:
            buf = mlk.DeviceBuffer.empty(shapes[name])
            setattr(self, name, buf)
            self.nbytes += buf.nbytes
            if name in filled and (fields is not None or fill_x or name != "x"):
                mlk.fill_normal(buf, buf.nbytes // 4, 0.0, std, seed + filled[name])


class Chain:
    """gather -> add+RMSNorm -> RoPE -> SwiGLU on rotating sets (without the
    gather when `gather` is False: the 70B config has none)."""

    def __init__(self, mlk, cfg, T, seed, n_sets=N_SETS, ids=None, positions=None, table=None,
                 gather=True):
        self.mlk, self.cfg, self.T = mlk, cfg, T
        self.OPS = (("gather_f32",) if gather else ()) + ("add_rmsnorm", "rope", "swiglu")
        D = cfg["dim"]
        self.table = None
        if gather and table is not None:
            self.table = table
        elif gather:
            self.table = mlk.DeviceBuffer.empty((cfg["vocab"], D))
            mlk.fill_normal(self.table, cfg["vocab"] * D, 0.0, 0.02, seed)
        self.norm_w = mlk.DeviceBuffer.empty((D,))
        mlk.fill_normal(self.norm_w, D, 1.0, 0.1, seed + 100)
        self.ids_host = None
        if gather:
            self.ids_host = ids if ids is not None else workloads.zipf_ids(T, cfg["vocab"], 1.1,
                                                                           seed)
            self.ids = mlk.DeviceBuffer.from_array(self.ids_host)
        self.positions_host = positions
        self.positions = mlk.DeviceBuffer.from_array(positions) if positions is not None else None
        self.sets = [ChainSet(mlk, cfg, T, seed + 10 * (i + 1), fill_x=not gather)
                     for i in range(n_sets)]
        self.stream = mlk.Stream()
        mlk.synchronize()

    def launch(self, s, op):
        mlk, c, T = self.mlk, self.cfg, self.T
        st = self.stream
        if op == "gather_f32":
            mlk.gather_f32(self.table, c["vocab"], c["dim"], self.ids, T, s.x, stream=st)
        elif op == "add_rmsnorm":
            mlk.add_rmsnorm(s.x, s.delta, self.norm_w, s.y, T, c["dim"], c["eps"], stream=st)
        elif op == "rope":
            mlk.rope(s.q, s.k, T, c["n_heads"], c["n_kv_heads"], c["head_dim"],
                     positions=self.positions, pos0=0, theta=c["theta"], stream=st)
        else:
            mlk.swiglu(s.gate, s.up, s.out, T * c["ffn"], stream=st)

    def run(self, steps, warmup):
        """Times `steps` chain steps between two events on the chain's stream
        (no events inside, so nothing but the kernels is timed); returns
        total_ms."""
        mlk = self.mlk
        for i in range(warmup):
            for op in self.OPS:
                self.launch(self.sets[i % len(self.sets)], op)
        self.stream.synchronize()
        start, stop = mlk.Event(), mlk.Event()
        start.record(self.stream)
        for i in range(steps):
            s = self.sets[i % len(self.sets)]
            for op in self.OPS:
                self.launch(s, op)
        stop.record(self.stream)
        stop.synchronize()
        return start.elapsed_ms(stop)

    def run_graph(self, steps, warmup=3):
        """One chain step captured into a HIP graph on the chain's stream and
        replayed `steps` times between two events; returns ms per step."""
        mlk = self.mlk
        with mlk.Graph.capture(self.stream) as graph:
            for op in self.OPS:
                self.launch(self.sets[0], op)
        for _ in range(warmup):
            graph.launch()
        self.stream.synchronize()
        start, stop = mlk.Event(), mlk.Event()
        start.record(self.stream)
        for _ in range(steps):
            graph.launch()
        stop.record(self.stream)
        stop.synchronize()
        graph.close()
        return start.elapsed_ms(stop) / steps

    def op_sets(self, op):
        """The chain's sets, plus sets of only `op`'s buffers until one pass
        over them touches OP_WORKING_SET bytes (or OP_MAX_SETS sets), so no
        prefill-size launch finds its buffers in the MALL from the previous
        pass."""
        sets = list(self.sets)
        fields = OP_FIELDS[op]
        one = sum(getattr(self.sets[0], f).nbytes for f in fields)
        seed = self.cfg["seed"] + 1000
        while one * len(sets) < OP_WORKING_SET and len(sets) < OP_MAX_SETS:
            sets.append(ChainSet(self.mlk, self.cfg, self.T, seed + 10 * len(sets), fields))
        return sets

    def run_ops(self, steps, warmup=3):
        """Per-kernel launch duration: each op launched `steps` times back to
        back over its cold rotation (op_sets) between two events; returns
        {op: ms per launch}."""
        mlk = self.mlk
        out = {}
        for op in self.OPS:
            sets = self.op_sets(op)
            self.mlk.synchronize()
            for i in range(warmup):
                self.launch(sets[i % len(sets)], op)
            self.stream.synchronize()
            start, stop = mlk.Event(), mlk.Event()
            start.record(self.stream)
            for i in range(steps):
                self.launch(sets[i % len(sets)], op)
            stop.record(self.stream)
            stop.synchronize()
            out[op] = start.elapsed_ms(stop) / steps
        return out


def op_bytes(workloads, cfg, T):
    return {
        "gather_f32": workloads.bytes_gather_f32(T, cfg["dim"]),
        "add_rmsnorm": workloads.bytes_add_rmsnorm(T, cfg["dim"]),
        "rope": workloads.bytes_rope(T, cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]),
        "swiglu": workloads.bytes_swiglu(T, cfg["ffn"]),
    }


def summarize(per_op, nbytes, peak):
    """per_op: {op: ms per launch}"""
    out = {}
    for op, ms in per_op.items():
        gbs = nbytes[op] / (ms * 1e-3) / 1e9
        out[op] = {"us": round(ms * 1e3, 2), "bytes": nbytes[op], "GBps": round(gbs, 1),
                   "frac_of_peak": round(gbs / peak, 4)}
    return out


def add_unique(entry, unique_bytes, peak):
    """Zipf ids repeat hot rows: beside the algorithmic figure, the bytes and
    GB/s when each distinct table row is counted once."""
    gbs = unique_bytes / (entry["us"] * 1e-6) / 1e9
    entry.update(unique_row_bytes=unique_bytes, unique_row_GBps=round(gbs, 1),
                 unique_row_frac_of_peak=round(gbs / peak, 4))


# ------------------------------------------------------------ CPU baselines

def _cpu_impl():
    """The reference's own CPU code (AVX2/FMA build of its sources), or the C
    port (oracle/liboracle.so) where that build is absent."""
    import oracle as O

    if O.reference_available(avx2=True):
        return O.reference(avx2=True), "reference", "oracle/_ref/libref_avx2.so"
    return O.oracle(), "port", "oracle/liboracle.so"


def _cpu_threads():
    """Threads for the multi-threaded baselines: the CPUs this process may
    run on, capped at 16, the GPU box's CPU share for one GPU (nproc there
    reports the whole host)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def _host_facts():
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"nproc": os.cpu_count(), "affinity_cpus": affinity, "cpu_model": _cpu_model()}


def _median_s(fn, reps):
    """Median wall time of `reps` calls of fn after one warmup call."""
    times = []
    for _ in range(reps + 1):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times[1:])


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def chain_host_bufs(chain, cfg, rows, table_host=None):
    """Host copies of the first `rows` token rows of a chain's set 0 (the
    CPU baseline's inputs) and its output arrays; table_host: a host copy of
    the chain's token table already downloaded (else it is downloaded)."""
    D, H, KV, hd, F = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"]
    s = chain.sets[0]
    pos = (chain.positions_host[:rows] if chain.positions_host is not None
           else np.arange(rows, dtype=np.int32))
    bufs = dict(table=None, vocab=cfg.get("vocab", 1), dim=D, ids=None,
                x=np.empty((rows, D), np.float32), delta=s.delta.download((rows, D)),
                norm_w=chain.norm_w.download(), y=np.empty((rows, D), np.float32),
                eps=cfg["eps"], q=s.q.download((rows, H * hd)), k=s.k.download((rows, KV * hd)),
                n_heads=H, n_kv_heads=KV, head_dim=hd, positions=np.ascontiguousarray(pos, np.int32),
                theta=cfg["theta"], gate=s.gate.download((rows, F)), up=s.up.download((rows, F)),
                ffn_out=np.empty((rows, F), np.float32), ffn_dim=F)
    if chain.table is not None:
        bufs["table"] = table_host if table_host is not None else chain.table.download()
        bufs["ids"] = np.ascontiguousarray(chain.ids_host[:rows], np.int32)
    else:
        bufs["x_in"] = s.x.download((rows, D))
    return bufs


def cpu_chain_baseline(bufs, rows, nbytes, sample, reps=5):
    """The chain on the CPU, one token at a time as ForwardBatch runs it:
    spread over tokens with the reference's ParallelFor, and on one thread.
    `nbytes`: the bytes the GPU figure of the same workload counts."""
    impl, kind, build = _cpu_impl()
    threads = _cpu_threads()
    model = None
    if kind == "reference" and bufs.get("table") is not None:
        model = bufs["model"] = impl.embedding_model(bufs["table"])
    elif kind == "port" and bufs.get("table") is None:
        # the C port always gathers: the residual rows become a table read in order
        bufs.update(table=bufs["x_in"], ids=np.arange(rows, dtype=np.int32), vocab=rows)

    def run(n_threads):
        rc = impl.chain(bufs, rows, n_threads)
        if rc != 0:
            raise RuntimeError(f"CPU baseline failed (status {rc})")

    try:
        t_mt = _median_s(lambda: run(threads), reps)
        t_st = _median_s(lambda: run(1), max(1, reps - 2))
    finally:
        if model is not None:
            impl.free_model(model)
            bufs.pop("model", None)
    return {"value": round(nbytes / t_mt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": kind, "sample": f"{sample}; {build}, ParallelFor over tokens; median of "
                                    f"{reps} reps after 1 warmup",
            "ms_per_chain": round(t_mt * 1e3, 3),
            "single_thread_value": round(nbytes / t_st / 1e9, 3),
            "single_thread_ms_per_chain": round(t_st * 1e3, 3), **_host_facts()}


def traffic_from_profiles():
    """HBM bytes per SwiGLU launch from the committed rocprofv3 --pmc runs."""
    try:
        with open(PMC_FILE) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def counter_traffic():
    """{section: {op: HBM bytes per launch}} from the committed rocprofv3
    --pmc runs of this command (bench.py --rocprof-report), or {}."""
    try:
        with open(PMC_FILE) as f:
            return json.load(f).get("per_section_hbm_bytes", {})
    except (OSError, ValueError):
        return {}


def add_counter(entry, hbm_bytes, peak):
    """Beside the algorithmic figure: the HBM bytes the counters measured for
    this launch, and the rate they give."""
    if not hbm_bytes:
        return
    gbs = hbm_bytes / (entry["us"] * 1e-6) / 1e9
    entry.update(counter_bytes=int(hbm_bytes), counter_GBps=round(gbs, 1),
                 counter_frac_of_peak=round(gbs / peak, 4))


def gather_fractions(entry):
    """A Zipf gather's frac_of_peak counts each distinct table row once (hot
    rows come from cache); the algorithmic fraction is kept beside it."""
    entry["algorithmic_frac_of_peak"] = entry["frac_of_peak"]
    entry["frac_of_peak"] = entry["unique_row_frac_of_peak"]
    entry["frac_basis"] = "unique table rows"


# ------------------------------------------------------------ sections
# Before each measured section a ZeroKernel launch of 4096 * (PHASE_BASE + i)
# bytes (a grid of PHASE_BASE + i workgroups of 256) marks section i in a
# rocprofv3 trace, so the summary can tell which config each launch belongs
# to (the chain kernels run at several shapes in one command).

PHASE_BASE = 100
PHASES = ("c3_chain", "c3_ops", "c2_decode", "c1_tiny", "c4_gather", "c5_chain", "c5_ops",
          "c2_decode_graph", "c1_tiny_graph", "decode_layer_8b", "prefill_layer_8b")


class Marks:
    def __init__(self, mlk):
        self.mlk = mlk
        self.buf = mlk.DeviceBuffer(4096 * (PHASE_BASE + len(PHASES) + 1), np.uint8)

    def __call__(self, phase, stream=None):
        n = 4096 * (PHASE_BASE + PHASES.index(phase) + 1)
        self.mlk.check(self.mlk.lib.mlk_zero_async(self.buf.ptr, n,
                                                   None if stream is None else stream.handle),
                       "mark")


def phase_of_grid(grid):
    """The section a ZeroKernel launch of `grid` work-items marks, or None."""
    i = grid // 256 - PHASE_BASE - 1
    return PHASES[i] if grid % 256 == 0 and 0 <= i < len(PHASES) else None


# ------------------------------------------------------------ other configs

def c1_tiny(mlk, steps, warmup, marks):
    """the tiny chain (6 tokens at positions 0..5) on the GPU,
    eager and graph-replayed, and on the CPU."""
    c1 = workloads.CONFIGS["c1_tiny"]
    ids = np.array(c1["ids"], np.int32)
    T = ids.size
    ch = Chain(mlk, c1, T, seed=c1["seed"], n_sets=1, ids=ids)
    n = max(steps, 200)
    marks("c1_tiny", ch.stream)
    eager = ch.run(n, warmup) / n
    marks("c1_tiny_graph", ch.stream)
    graph = ch.run_graph(n)
    out = {"tokens": T, "us_per_chain_eager": round(eager * 1e3, 2),
           "us_per_chain_graph": round(graph * 1e3, 2), "warmup_steps": warmup,
           "chain_bytes": workloads.bytes_chain(c1, T)}
    bufs = chain_host_bufs(ch, c1, T)
    impl, kind, build = _cpu_impl()
    model = impl.embedding_model(bufs["table"]) if kind == "reference" else None
    if model is not None:
        bufs["model"] = model
    reps = 2000
    t0 = time.perf_counter()
    for _ in range(reps):
        impl.chain(bufs, T, 1)
    t = (time.perf_counter() - t0) / reps
    if model is not None:
        impl.free_model(model)
    out["cpu_baseline"] = {"us_per_chain": round(t * 1e6, 2), "unit": "us", "cores": 1,
                           "kind": kind,
                           "sample": f"the whole chain (6 tokens), mean of {reps} calls, the "
                                     f"Python call overhead included; {build}",
                           **_host_facts()}
    return out


C2_CPU_TOKENS = {1: 200, 64: 20}  # decode sizes timed on the CPU: calls per median


def cpu_decode_baseline(impl, kind, build, bufs, rows, reps):
    """The configs[1] chain on the CPU for one decode step of `rows` tokens,
    one token at a time as ForwardBatch runs it (src/forward.cc:482-486):
    µs per step, spread over tokens with the reference's ParallelFor and on
    one thread; bufs["model"] holds the reference's token table."""
    threads = _cpu_threads()

    def run(n_threads):
        rc = impl.chain(bufs, rows, n_threads)
        if rc != 0:
            raise RuntimeError(f"CPU baseline failed (status {rc})")

    t_mt = _median_s(lambda: run(threads), reps)
    t_st = _median_s(lambda: run(1), reps)
    return {"value": round(t_mt * 1e6, 2), "unit": "us per chain", "cores": threads,
            "kind": kind,
            "sample": f"the whole configs[1] chain at T={rows} (gather, add+RMSNorm, RoPE at "
                      f"the step's positions, SwiGLU; Llama-3-8B shapes); {build}, ParallelFor "
                      f"over tokens; median of {reps} calls after 1 warmup, each call's Python "
                      "overhead (a few us) included",
            "single_thread_value": round(t_st * 1e6, 2), **_host_facts()}


def c2_decode(mlk, steps, warmup, marks, table, table_host=None):
    """the 8B chain as a decode step at T = 1..64 tokens at
    positions uniform in [0, 8191]: latency-bound, µs per chain, eager
    launches and one HIP graph replay per step; with table_host (a host copy
    of `table`), the reference's CPU chain at T = 1 and T = 64 beside it."""
    c2 = workloads.CONFIGS["c2_decode_8b"]
    out = {}
    impl = model = None
    if table_host is not None:
        impl, kind, build = _cpu_impl()
        if kind == "reference":
            model = impl.embedding_model(table_host)
    for t in c2["tokens"]:
        pos = workloads.decode_positions(t, c2["max_pos"], c2["seed"])
        dch = Chain(mlk, c2, t, seed=c2["seed"], n_sets=2, positions=pos, table=table)
        marks("c2_decode", dch.stream)
        n = max(steps, 100)
        eager = dch.run(n, warmup) / n
        marks("c2_decode_graph", dch.stream)
        graph = dch.run_graph(n)
        out[str(t)] = {"us_per_chain_eager": round(eager * 1e3, 2),
                       "us_per_chain_graph": round(graph * 1e3, 2), "warmup_steps": warmup,
                       "chain_bytes": workloads.bytes_chain(c2, t)}
        if impl is not None and t in C2_CPU_TOKENS:
            bufs = chain_host_bufs(dch, c2, t, table_host)
            if model is not None:
                bufs["model"] = model
            out[str(t)]["cpu_baseline"] = cpu_decode_baseline(impl, kind, build, bufs, t,
                                                              C2_CPU_TOKENS[t])
        del dch
    if model is not None:
        impl.free_model(model)
    return out


def c4_gathers(mlk, steps, peak, marks, with_cpu):
    """Q8_0 / Q4_0 / Q4_1 token gathers, T = 4096 Zipf(1.1) ids
    from a [128256, 4096] table quantized on the device, cold output rotation;
    beside them the reference's dequantizer over the same rows on the CPU."""
    c4 = workloads.CONFIGS["c4_quant_gather"]
    T, V, D = c4["tokens"], c4["vocab"], c4["dim"]
    table = mlk.DeviceBuffer.empty((V, D))
    mlk.fill_normal(table, V * D, 0.0, 0.02, c4["seed"])
    ids_host = workloads.zipf_ids(T, V, 1.1, c4["seed"])
    ids = mlk.DeviceBuffer.from_array(ids_host)
    outs = [mlk.DeviceBuffer.empty((T, D)) for _ in range(N_SETS)]
    st = mlk.Stream()
    counters = counter_traffic().get("c4_gather", {})
    res, cpu = {}, {}
    marks("c4_gather", st)
    for qt in ("q8_0", "q4_0", "q4_1"):
        blocks = mlk.DeviceBuffer(mlk.quant_bytes(qt, V, D), np.uint8)
        mlk.quantize(qt, table, V, D, blocks, stream=st)
        for i in range(10):
            mlk.gather_quant(qt, blocks, V, D, ids, T, outs[i % N_SETS], stream=st)
        st.synchronize()
        e0, e1 = mlk.Event(), mlk.Event()
        e0.record(st)
        for i in range(steps):
            mlk.gather_quant(qt, blocks, V, D, ids, T, outs[i % N_SETS], stream=st)
        e1.record(st)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / steps
        e = summarize({qt: ms}, {qt: workloads.bytes_gather_quant(qt, T, D)}, peak)[qt]
        add_unique(e, workloads.bytes_gather_unique(ids_host, D, qt), peak)
        gather_fractions(e)
        add_counter(e, counters.get(qt), peak)
        res[qt] = e
        if with_cpu:
            impl, kind, build = _cpu_impl()
            hb = blocks.download(dtype=np.uint8)
            threads = _cpu_threads() if kind == "reference" else 1

            def run(n):
                if kind == "reference":
                    impl.gather_quant(qt, hb, V, D, ids_host, n)
                else:
                    impl.gather_quant(qt, hb, V, D, ids_host)

            t_mt = _median_s(lambda: run(threads), 5)
            t_st = _median_s(lambda: run(1), 3)
            nb = workloads.bytes_gather_unique(ids_host, D, qt)
            cpu[qt] = {"value": round(nb / t_mt / 1e9, 3), "unit": "GB/s (unique rows)",
                       "cores": threads, "kind": kind,
                       "sample": f"the whole gather ({T} rows), each row's blocks through the "
                                 f"reference's Q*ToTensor; {build}, ParallelFor over tokens; "
                                 "median of 5 reps after 1 warmup",
                       "ms": round(t_mt * 1e3, 3), "single_thread_ms": round(t_st * 1e3, 3),
                       "single_thread_value": round(nb / t_st / 1e9, 3), **_host_facts()}
            del hb
        del blocks
    if with_cpu:
        res["cpu_baseline"] = cpu
    return res


def c5_chain(mlk, steps, warmup, peak, marks, with_cpu):
    """the Llama-3-70B-shape chain add+RMSNorm -> RoPE -> SwiGLU
    at T = 8192 (no gather), cold rotating sets; beside it the reference's CPU
    chain over a 1024-token sample of the same rows."""
    c5 = workloads.CONFIGS["c5_70b"]
    T = c5["tokens"]
    ch = Chain(mlk, c5, T, seed=c5["seed"], n_sets=2, gather=False)
    marks("c5_chain", ch.stream)
    total = ch.run(steps, warmup)
    nbytes = {"add_rmsnorm": workloads.bytes_add_rmsnorm(T, c5["dim"]),
              "rope": workloads.bytes_rope(T, c5["n_heads"], c5["n_kv_heads"], c5["head_dim"]),
              "swiglu": workloads.bytes_swiglu(T, c5["ffn"])}
    marks("c5_ops", ch.stream)
    ops = summarize(ch.run_ops(steps), nbytes, peak)
    for op, hbm in counter_traffic().get("c5_ops", {}).items():
        if op in ops:
            add_counter(ops[op], hbm, peak)
    chain_bytes = workloads.bytes_chain(c5, T, with_gather=False)
    gbs = chain_bytes * steps / (total * 1e-3) / 1e9
    out = {"tokens": T, "us_per_chain": round(total * 1e3 / steps, 2), "chain_bytes": chain_bytes,
           "GBps": round(gbs, 1), "frac_of_peak": round(gbs / peak, 4), "ops": ops}
    if with_cpu:
        rows = 1024
        bufs = chain_host_bufs(ch, c5, rows)
        out["cpu_baseline"] = cpu_chain_baseline(
            bufs, rows, workloads.bytes_chain(c5, rows, with_gather=False),
            f"{rows} of the {T} token rows (the per-token work is the same for every row)")
    del ch
    return out


# ------------------------------------------------------------ linear layers

LINEAR_TYPES = ("q8_0", "q4_0", "q4_1", "f32")
# the decode GEMV bench also runs the planar copies (mlk_linear_planar)
LINEAR_DECODE_TYPES = LINEAR_TYPES + ("q8_0_planar", "q4_0_planar")


def base_type(qtype):
    """The block format of a weight type name ("q8_0_planar" -> "q8_0"):
    a planar copy holds the same bytes in another order."""
    return qtype[:-len("_planar")] if qtype.endswith("_planar") else qtype
LINEAR_TOKENS = (1, 4, 16)
LINEAR_WORKING_SET = 768 << 20  # rotate layer copies until the weights exceed 3x the MALL


class LinearLayers:
    """Device copies of the seven projection weights of one Llama-3-8B layer
    in one weight format: every matrix has enough copies that one pass over
    its copies exceeds 768 MB, three times the 256 MB MALL, so a launch never
    finds its weights in cache (the per-projection loop rotates over a
    matrix's copies, the whole-layer loop over all of them)."""

    def __init__(self, mlk, cfg, qtype, seed, working_set=LINEAR_WORKING_SET):
        self.mlk, self.qtype = mlk, qtype
        self.base = base_type(qtype)
        self.planar = qtype != self.base
        self.shapes = workloads.layer_linears(cfg)
        biggest = max(k * o for _, k, o in self.shapes)
        tmp = mlk.DeviceBuffer.empty((biggest,)) if qtype != "f32" else None
        blk = (mlk.DeviceBuffer(max(mlk.quant_bytes(self.base, o, k) for _, k, o in self.shapes),
                                np.uint8) if self.planar else None)
        self.copies = {}
        for j, (name, k, o) in enumerate(self.shapes):
            n = max(1 if working_set == 0 else 2,
                    -(-working_set // workloads.weight_bytes(self.base, k, o)))
            mats = []
            for c in range(n):
                sd = seed + 97 * c + j
                if qtype == "f32":
                    w = mlk.DeviceBuffer.empty((o, k))
                    mlk.fill_normal(w, o * k, 0.0, 0.02, sd)
                elif self.planar:  # the same blocks, repacked
                    mlk.fill_normal(tmp, o * k, 0.0, 0.02, sd)
                    mlk.quantize(self.base, tmp, o, k, blk)
                    w = mlk.DeviceBuffer(mlk.quant_planar_bytes(self.base, o, k), np.uint8)
                    mlk.quant_to_planar(self.base, blk, o, k, w)
                else:
                    mlk.fill_normal(tmp, o * k, 0.0, 0.02, sd)
                    w = mlk.DeviceBuffer(mlk.quant_bytes(qtype, o, k), np.uint8)
                    mlk.quantize(qtype, tmp, o, k, w)
                mats.append(w)
            self.copies[name] = mats
        mlk.synchronize()
        for b in (tmp, blk):
            if b is not None:
                b.close()

    def n_copies(self, name):
        return len(self.copies[name])

    def launch(self, i, name, k, o, x, y, T, stream):
        mats = self.copies[name]
        w = mats[i % len(mats)]
        if self.qtype == "f32":
            self.mlk.linear_f32(x, w, y, T, k, o, stream=stream)
        elif self.planar:
            self.mlk.linear_planar(self.base, x, w, y, T, k, o, stream=stream)
        else:
            self.mlk.linear_quant(self.qtype, x, w, y, T, k, o, stream=stream)


# marker grids 256 * (LINEAR_MARK_BASE + i): timed calls i of --linear; 256 *
# LINEAR_MARK_END: their end.  Below 1024 workgroups, the most a zero fill
# launches on a 256-CU GPU (4 a CU), so the grid is the marker's own.
LINEAR_MARK_BASE = 600
LINEAR_MARK_END = 599


def _linear_mark(mlk, buf, k, st):
    """A ZeroKernel of grid 256 * k work-items on `st`: a rocprofv3 trace of
    --linear tells the timed replays' kernels apart by these."""
    mlk.check(mlk.lib.mlk_zero_async(buf.ptr, 4096 * k, st.handle), "mark")


def _eager_ms(mlk, st, launches, n, mark=None):
    """_graph_ms with the n calls issued as eager launches (Python dispatch
    included in the event time; a kernel trace of this run gives the
    kernels' own durations)."""
    for i in range(min(n, 3)):
        launches(i)
    st.synchronize()
    if mark is not None:
        _linear_mark(mlk, mark[0], LINEAR_MARK_BASE + mark[1], st)
    e0, e1 = mlk.Event(), mlk.Event()
    e0.record(st)
    for i in range(n):
        launches(i)
    e1.record(st)
    if mark is not None:
        _linear_mark(mlk, mark[0], LINEAR_MARK_END, st)
    e1.synchronize()
    return e0.elapsed_ms(e1) / n


def _graph_ms(mlk, st, launches, n, mark=None):
    """ms per item of `launches(i)` for i < n, issued as one captured HIP
    graph and timed over one replay between two events on `st` (after one
    untimed replay): the host dispatches one graph instead of n ctypes calls
    and their HIP launches, so the time is the kernels' and the gaps the GPU
    leaves between graph nodes.  mark: (buffer, index) -- marker kernels
    bracket the timed replay (outside the events)."""
    with mlk.Graph.capture(st) as graph:
        for i in range(n):
            launches(i)
    try:
        graph.launch()
        st.synchronize()
        if mark is not None:
            _linear_mark(mlk, mark[0], LINEAR_MARK_BASE + mark[1], st)
        e0, e1 = mlk.Event(), mlk.Event()
        e0.record(st)
        graph.launch()
        e1.record(st)
        if mark is not None:
            _linear_mark(mlk, mark[0], LINEAR_MARK_END, st)
        e1.synchronize()
        return e0.elapsed_ms(e1) / n
    finally:
        graph.close()


def linear_bench(mlk, steps, peak, path, eager=False):
    """Per-projection launch time and the time of one whole layer's seven
    projections.  Each projection's `steps` calls (over its rotating weight
    copies) are captured into one HIP graph and timed over a replay, so the
    figure is the kernels' time on the GPU, not Python's dispatch of the
    calls (a planar call of 2..32 rows is three kernels: x split, the
    matrix-core GEMV and the split-K sum).  Workspaces are sized by one eager
    call of each shape before its capture."""
    cfg = workloads.CONFIGS["c2_decode_8b"]
    big = max(max(k, o) for _, k, o in workloads.layer_linears(cfg))
    T_max = max(LINEAR_TOKENS)
    x = mlk.DeviceBuffer.empty((T_max, big))
    y = mlk.DeviceBuffer.empty((T_max, big))
    mlk.fill_normal(x, T_max * big, 0.0, 1.0, 5)
    st = mlk.Stream()
    out = {"workload": "Llama-3-8B layer projections (configs[1] shapes), weights N(0,0.02) "
                       "quantized on the device; x N(0,1)",
           "timing": (f"each projection's {steps} calls as eager launches between two events"
                      if eager else
                      f"each projection's {steps} calls captured into one HIP graph over the "
                      "rotating weight copies, one replay timed between two events"),
           "peak_GBps": peak, "calls_per_replay": steps, "markers": {}}
    mark_buf = mlk.DeviceBuffer(4096 * 1024, np.uint8)
    timed = _eager_ms if eager else _graph_ms
    marks = out["markers"]

    def mark(label):
        marks[len(marks)] = label
        return (mark_buf, len(marks) - 1)
    for qt in LINEAR_DECODE_TYPES:
        layers = LinearLayers(mlk, cfg, qt, seed=300)
        res = {"weight_copies": {n: layers.n_copies(n) for n, _, _ in layers.shapes}}
        for T in LINEAR_TOKENS:
            per = {}
            for name, k, o in layers.shapes:
                for i in range(3):  # eager: sizes the auto workspace before the capture
                    layers.launch(i, name, k, o, x, y, T, st)
                st.synchronize()
                ms = timed(mlk, st, lambda i: layers.launch(3 + i, name, k, o, x, y, T, st),
                           steps, mark(f"{qt} / {T} / {name}"))
                nb = workloads.bytes_linear(base_type(qt), T, k, o)
                gbs = nb / (ms * 1e-3) / 1e9
                per[name] = {"in": k, "out": o, "us": round(ms * 1e3, 2), "bytes": nb,
                             "GBps": round(gbs, 1), "frac_of_peak": round(gbs / peak, 4)}

            def layer_call(i):
                for name, k, o in layers.shapes:
                    layers.launch(3 + steps + i, name, k, o, x, y, T, st)
            ms = timed(mlk, st, layer_call, steps, mark(f"{qt} / {T} / layer"))
            nb = sum(workloads.bytes_linear(base_type(qt), T, k, o) for _, k, o in layers.shapes)
            gbs = nb / (ms * 1e-3) / 1e9
            res[str(T)] = {"layer_us": round(ms * 1e3, 2), "layer_bytes": nb,
                           "layer_GBps": round(gbs, 1), "layer_frac_of_peak": round(gbs / peak, 4),
                           "ops": per}
            print(f"linear {qt} T={T}: layer {ms * 1e3:.1f} us, {gbs:.0f} GB/s; "
                  + " ".join(f"{n}={v['us']}" for n, v in per.items()), flush=True)
        out[qt] = res
        del layers
    with open(path, "w") as f:
        json.dump(out, f, indent=1)


# ------------------------------------------------------------ prefill GEMM

GEMM_TOKENS = (8, 16, 32, 64, 128, 512, 4096)
MFMA_FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix-core peak
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix-core peak
# Q8_0 / Q4_0 tiles of more than 64 token rows (and the attention at head_dim
# 128) form each product from three exact bf16 pieces: three bf16 MACs per
# useful MAC, so their ceiling in useful TFLOP/s is a third of the bf16 peak.
PIECES_PEAK_TFLOPS = MFMA_BF16_PEAK_TFLOPS / 3


def attention_peak(hd):
    """(peak TFLOP/s of useful MACs, basis) of the tile attention: at
    head_dim 128 the scores and the values each take 6 bf16 piece products
    per useful MAC, at 64 the fp32 instruction."""
    if hd == 128:
        return MFMA_BF16_PEAK_TFLOPS / 6, "bf16 MFMA / 6 (piece products)"
    return MFMA_FP32_PEAK_TFLOPS, "fp32 MFMA"


def gemm_peak(wt, T):
    """(peak TFLOP/s of useful MACs, basis) of the kernel the tiled GEMM
    runs for weight type `wt` at T token rows (K a multiple of 256)."""
    if wt in ("q8_0", "q4_0") and T > 64:
        return PIECES_PEAK_TFLOPS, "bf16 MFMA / 3 (three-piece products)"
    return MFMA_FP32_PEAK_TFLOPS, "fp32 MFMA"


def gemm_bench(mlk, steps, path):
    """The seven projections of one Llama-3-8B layer at prefill row counts
    (the matrix-core GEMM path): per-projection launch time, each launched
    `steps` times back to back between two events on its stream, and one
    whole layer's seven projections; TFLOP/s = 2 T K O / time against the
    peak of the instruction the kernel uses (gemm_peak).  One weight copy per projection: from 128 rows on these
    shapes are compute-bound, and below that the split-K launches read each
    weight byte once per call either way."""
    cfg = workloads.CONFIGS["c3_prefill_8b"]
    shapes = workloads.layer_linears(cfg)
    big = max(max(k, o) for _, k, o in shapes)
    T_max = max(GEMM_TOKENS)
    x = mlk.DeviceBuffer.empty((T_max, big))
    y = mlk.DeviceBuffer.empty((T_max, big))
    mlk.fill_normal(x, T_max * big, 0.0, 1.0, 5)
    st = mlk.Stream()
    out = {"workload": "Llama-3-8B layer projections at prefill row counts, weights N(0,0.02) "
                       "quantized on the device; x N(0,1)",
           "peak_TFLOPs": MFMA_FP32_PEAK_TFLOPS}
    for qt in LINEAR_TYPES:
        layers = LinearLayers(mlk, cfg, qt, seed=300, working_set=0)
        res = {}
        for T in GEMM_TOKENS:
            per = {}
            for name, k, o in shapes:
                if T >= 64:  # matrix-core bound: the clock's steady state
                    _warm_clock(mlk, st, lambda i: layers.launch(i, name, k, o, x, y, T, st))
                for i in range(2):
                    layers.launch(i, name, k, o, x, y, T, st)
                st.synchronize()
                e0, e1 = mlk.Event(), mlk.Event()
                e0.record(st)
                for i in range(steps):
                    layers.launch(i, name, k, o, x, y, T, st)
                e1.record(st)
                e1.synchronize()
                ms = e0.elapsed_ms(e1) / steps
                tf = workloads.flops_linear(T, k, o) / (ms * 1e-3) / 1e12
                peak, _ = gemm_peak(qt, T)
                per[name] = {"in": k, "out": o, "us": round(ms * 1e3, 2),
                             "TFLOPs": round(tf, 2), "frac_of_peak": round(tf / peak, 4)}
            e0, e1 = mlk.Event(), mlk.Event()
            e0.record(st)
            for i in range(steps):
                for name, k, o in shapes:
                    layers.launch(i, name, k, o, x, y, T, st)
            e1.record(st)
            e1.synchronize()
            ms = e0.elapsed_ms(e1) / steps
            fl = sum(workloads.flops_linear(T, k, o) for _, k, o in shapes)
            tf = fl / (ms * 1e-3) / 1e12
            peak, basis = gemm_peak(qt, T)
            res[str(T)] = {"layer_us": round(ms * 1e3, 2), "layer_flops": fl,
                           "layer_TFLOPs": round(tf, 2), "peak_TFLOPs": round(peak, 1),
                           "peak_basis": basis,
                           "layer_frac_of_peak": round(tf / peak, 4), "ops": per}
            print(f"gemm {qt} T={T}: layer {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s "
                  f"({100 * tf / peak:.1f}% of {basis}) "
                  + " ".join(f"{n}={v['TFLOPs']}" for n, v in per.items()), flush=True)
        out[qt] = res
        del layers
    with open(path, "w") as f:
        json.dump(out, f, indent=1)


# ------------------------------------------------------------ batched layer

LAYER_TOKENS = 4096
LAYER_LOOP_SAMPLE = 64  # tokens of the token-by-token comparison


def _device_layer(mlk, fwd, cfg, wt, seed):
    """One Llama-3-8B-shaped layer's weights on the device (N(0, 0.02),
    quantized on the device; norm weights N(1, 0.1)) as LayerWeights, plus
    the buffers that hold them.  Q8_0 / Q4_0 weights also get a planar copy
    (mlk_quant_to_planar), which calls of 1..32 tokens run on."""
    D, F = cfg["dim"], cfg["hidden_dim"]
    QD, KD = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = {"wq": (QD, D), "wk": (KD, D), "wv": (KD, D), "wo": (D, QD), "w_gate": (F, D),
              "w_up": (F, D), "w_down": (D, F)}
    keep = []
    tmp = mlk.DeviceBuffer.empty((max(o * i for o, i in shapes.values()),))
    w = fwd.LayerWeights()
    for j, (name, (o, i)) in enumerate(shapes.items()):
        lw = fwd.LinearWeight()
        if wt == "f32":
            buf = mlk.DeviceBuffer.empty((o, i))
            mlk.fill_normal(buf, o * i, 0.0, 0.02, seed + j)
            lw.type = fwd.WEIGHT_F32
        else:
            mlk.fill_normal(tmp, o * i, 0.0, 0.02, seed + j)
            buf = mlk.DeviceBuffer(mlk.quant_bytes(wt, o, i), np.uint8)
            mlk.quantize(wt, tmp, o, i, buf)
            lw.type = mlk.QUANT[wt]
            n_planar = mlk.quant_planar_bytes(wt, o, i)
            if n_planar > 0:  # the planar copy the 1..32-token calls run on
                pl = mlk.DeviceBuffer(n_planar, np.uint8)
                mlk.quant_to_planar(wt, buf, o, i, pl)
                lw.planar = pl.ptr
                keep.append(pl)
        lw.data, lw.bias = buf.ptr, None
        setattr(w, name, lw)
        keep.append(buf)
    for name in ("attention_norm", "ffn_norm"):
        buf = mlk.DeviceBuffer.empty((D,))
        mlk.fill_normal(buf, D, 1.0, 0.1, seed + 50 + len(keep))
        setattr(w, name, buf.ptr)
        keep.append(buf)
    mlk.synchronize()
    tmp.close()
    return w, keep


CLOCK_WARM_MS = 150.0  # untimed matrix-core work before a timed matrix-core case
LAUNCH_BOUND_WARMUP = 10  # warmup steps of the launch-bound C1 / C2 chains


def _warm_clock(mlk, st, launch, ms=CLOCK_WARM_MS):
    """Runs launch(i) on `st`, untimed, until about `ms` of GPU time have
    passed.  The GPU raises its clock over tens of ms of sustained matrix
    work that follows memory-bound phases (the prefill gate GEMM's
    GRBM_GUI_ACTIVE cycle count stays the same while its duration falls from
    about 1.8 to 1.36 ms over its first ~25 back-to-back calls), so the
    matrix-core benches time the clock's steady state, which a long prefill
    runs at."""
    e0, e1 = mlk.Event(), mlk.Event()
    e0.record(st)
    launch(0)
    e1.record(st)
    e1.synchronize()
    n = int(min(max(ms / max(e0.elapsed_ms(e1), 1e-3), 1), 2000))
    for i in range(n):
        launch(i)
    st.synchronize()


def prefill_layer_bench(mlk, fwd, steps, types=("q8_0", "q4_0", "f32"), token_loop=True,
                        log=sys.stdout, marks=None):
    """One Llama-3-8B layer (attention + SwiGLU FFN) over a T = 4096 prompt
    chunk at positions 0..4095 through mlk_forward_layer_batch, per weight
    type: `steps` calls timed between two events after the clock warm-up;
    with token_loop, the same layer run the reference's way beside it, one
    token at a time (T = 1 calls at positions 0..63)."""
    cfg = dict(workloads.CONFIGS["c3_prefill_8b"])
    cfg.update(hidden_dim=cfg["ffn"], max_seq=LAYER_TOKENS)
    T = LAYER_TOKENS
    D, KV, hd = cfg["dim"], cfg["n_kv_heads"], cfg["head_dim"]
    fl_lin = sum(workloads.flops_linear(T, k, o) for _, k, o in workloads.layer_linears(cfg))
    fl_att = workloads.flops_prefill_attention(T, cfg["n_heads"], hd)
    out = {"workload": "one Llama-3-8B layer, T = 4096 prompt chunk at positions 0..4095, "
                       "weights N(0, 0.02) quantized on the device, x N(0, 1)",
           "layer_flops": fl_lin + fl_att, "linear_flops": fl_lin, "attention_flops": fl_att}
    st = mlk.Stream()
    if marks is not None:
        marks("prefill_layer_8b", st)
    kc = mlk.DeviceBuffer.empty((1, T, KV, hd))
    vc = mlk.DeviceBuffer.empty((1, T, KV, hd))
    kc.zero()
    vc.zero()
    x = mlk.DeviceBuffer.empty((T, D))
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, T, T, True), np.uint8)
    ws1 = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, 1, T, True), np.uint8)
    for wt in types:
        w, keep = _device_layer(mlk, fwd, cfg, wt, 400)
        mlk.fill_normal(x, T * D, 0.0, 1.0, 21)
        _warm_clock(mlk, st, lambda i: fwd.forward_layer_batch(cfg, w, x, T, kc, vc, 1, T, 0, T, ws,
                                                               stream=st))
        e0, e1 = mlk.Event(), mlk.Event()
        e0.record(st)
        for _ in range(steps):
            fwd.forward_layer_batch(cfg, w, x, T, kc, vc, 1, T, 0, T, ws, stream=st)
        e1.record(st)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / steps
        tf = (fl_lin + fl_att) / (ms * 1e-3) / 1e12
        peak, basis = gemm_peak(wt, T)
        out[wt] = {"us": round(ms * 1e3, 1), "layer_ms": round(ms, 3),
                   "tokens_per_s": round(T / (ms * 1e-3), 1),
                   "TFLOPs": round(tf, 2), "peak_TFLOPs": round(peak, 1), "peak_basis": basis,
                   "frac_of_peak": round(tf / peak, 4)}
        msg = f"layer {wt} T={T}: {ms:.2f} ms ({T / (ms * 1e-3):.0f} tokens/s, {tf:.1f} TFLOP/s)"
        if token_loop:
            # token t alone at position t (its cache prefix as the batched
            # call left it); one untimed token first: the first one-token
            # call of a weight type loads its kernels, which would dominate
            # the sample's average
            n = LAYER_LOOP_SAMPLE
            x1 = mlk.DeviceBuffer.empty((n, D))
            mlk.fill_normal(x1, n * D, 0.0, 1.0, 22)
            fwd.forward_layer_batch(cfg, w, x1.ptr, 1, kc, vc, 1, T, 0, T, ws1, pos0=0, stream=st)
            st.synchronize()
            e2, e3 = mlk.Event(), mlk.Event()
            e2.record(st)
            for t in range(n):
                fwd.forward_layer_batch(cfg, w, x1.ptr + t * D * 4, 1, kc, vc, 1, T, 0, T, ws1,
                                        pos0=t, stream=st)
            e3.record(st)
            e3.synchronize()
            loop_us = e2.elapsed_ms(e3) / n * 1e3
            out[wt].update({"token_loop_us_per_token": round(loop_us, 1),
                            "token_loop_tokens_per_s": round(1e6 / loop_us, 1),
                            "batch_speedup_over_token_loop": round(loop_us * T / (ms * 1e3), 1)})
            msg += f"; token loop {loop_us:.0f} us/token"
            x1.close()
        print(msg, file=log, flush=True)
        del keep
    return out


def layer_bench(mlk, steps, path):
    """bench.py --layer: the prefill layer (prefill_layer_bench, Q8_0 /
    Q4_0 / F32 with the token loop), the decode layer, and the reference's
    own CPU forward pass (oracle/_ref, one layer, a few tokens)."""
    import importlib
    fwd = importlib.import_module(mlk.__name__ + ".forward")
    cfg = dict(workloads.CONFIGS["c3_prefill_8b"])
    cfg.update(hidden_dim=cfg["ffn"], max_seq=LAYER_TOKENS)
    out = prefill_layer_bench(mlk, fwd, steps)
    out["peak_TFLOPs"] = MFMA_FP32_PEAK_TFLOPS
    out["decode"] = decode_layer_bench(mlk, fwd, steps)
    out["cpu_reference"] = layer_cpu_reference(cfg)
    with open(path, "w") as f:
        json.dump(out, f, indent=1)


DECODE_COPIES = 4   # layers rotated per call: 4 x 232 MB of Q8_0 weights exceed the MALL
DECODE_POS = 8191   # the token's position: it attends to 8192 cache rows
DECODE_BATCH = 16   # tokens of the batched decode case (configs[1] positions)


def decode_layer_bench(mlk, fwd, steps, log=sys.stdout, marks=None):
    """One decode step of one Llama-3-8B layer through mlk_forward_layer_batch:
    a single token at position 8191 (the top of configs[1]'s position
    range), and a batch of DECODE_BATCH tokens at positions uniform in
    0..8191; rotating over DECODE_COPIES layers' weights and caches so that
    every call reads its weights and K/V from HBM, timed between two events.
    Bytes = the layer's weights + the K/V rows attended + activations (each
    read once)."""
    cfg = dict(workloads.CONFIGS["c2_decode_8b"])
    S = DECODE_POS + 1
    cfg.update(hidden_dim=cfg["ffn"], max_seq=S)
    D, KV, hd = cfg["dim"], cfg["n_kv_heads"], cfg["head_dim"]
    st = mlk.Stream()
    if marks is not None:
        marks("decode_layer_8b", st)
    L = DECODE_COPIES
    kc = mlk.DeviceBuffer.empty((L, S, KV, hd))
    vc = mlk.DeviceBuffer.empty((L, S, KV, hd))
    mlk.fill_normal(kc, L * S * KV * hd, 0.0, 0.02, 31)
    mlk.fill_normal(vc, L * S * KV * hd, 0.0, 0.02, 32)
    x = mlk.DeviceBuffer.empty((1, D))
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, 1, S, True), np.uint8)
    res = {"workload": f"one Llama-3-8B layer, one token at position {DECODE_POS} (8192 cache "
                       f"rows), weights and caches of {L} layers rotated, weights N(0, 0.02)"}
    # a batch of DECODE_BATCH tokens at positions uniform in [0, 8191]
    rng = np.random.default_rng(42)
    bpos = np.sort(rng.choice(S, DECODE_BATCH, replace=False)).astype(np.int32)
    bpos[-1] = DECODE_POS
    d_bpos = mlk.DeviceBuffer.from_array(bpos)
    xb = mlk.DeviceBuffer.empty((DECODE_BATCH, D))
    wsb = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, DECODE_BATCH, S, False), np.uint8)
    for wt in ("q8_0", "q4_0", "f32"):
        layers = [_device_layer(mlk, fwd, cfg, wt, 500 + 10 * i) for i in range(L)]
        for T, xx, w_s, kw in ((1, x, ws, dict(pos0=DECODE_POS)),
                               (DECODE_BATCH, xb, wsb, dict(positions=d_bpos))):
            mlk.fill_normal(xx, T * D, 0.0, 1.0, 23)

            def run(i):
                fwd.forward_layer_batch(cfg, layers[i][0], xx, T, kc, vc, L, S, i, S, w_s,
                                        stream=st, **kw)
            _warm_clock(mlk, st, lambda i: run(i % L))
            for i in range(L):
                run(i)
            st.synchronize()
            e0, e1 = mlk.Event(), mlk.Event()
            e0.record(st)
            for _ in range(steps):
                for i in range(L):
                    run(i)
            e1.record(st)
            e1.synchronize()
            us = e0.elapsed_ms(e1) / (steps * L) * 1e3
            nb = sum(workloads.bytes_linear(wt, T, k, o) for _, k, o in workloads.layer_linears(cfg))
            # K/V rows 0..max position once: the batch's tokens share each cache tile
            top = DECODE_POS if T == 1 else int(np.max(bpos))
            nb += workloads.bytes_attention([top], cfg["n_heads"], KV, hd)
            nb += 8 * (T - 1) * cfg["n_heads"] * hd  # the other tokens' q and out
            gbs = nb / (us * 1e-6) / 1e9
            key = wt if T == 1 else f"{wt}_T{T}"
            res[key] = {"tokens": T, "us": round(us, 1), "bytes": nb, "GBps": round(gbs, 1),
                        "frac_of_peak": round(gbs / workloads.HBM_PEAK_GBS, 4),
                        "tokens_per_s_32_layers": round(T * 1e6 / (32 * us), 1)}
            where = f"at position {DECODE_POS}" if T == 1 else "at positions uniform in 0..8191"
            print(f"decode layer {wt}, {T} token(s) {where}: {us:.1f} us ({gbs:.0f} GB/s, "
                  f"{T * 1e6 / (32 * us):.0f} tokens/s over 32 layers)", file=log, flush=True)
        del layers
    return res


def layer_cpu_reference(cfg, n_tokens=2):
    """The reference's own CPU forward pass (oracle/_ref AVX2 build,
    ForwardToken) on a one-layer 8B-shaped Q8_0 model with a 256-token
    vocabulary (so lm_head does not dominate): seconds per token."""
    try:
        import oracle as O
        if not O.reference_available(avx2=True):
            return None
        c = dict(vocab=256, dim=cfg["dim"], hidden_dim=cfg["hidden_dim"], layers=1,
                 n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv_heads"], head_dim=cfg["head_dim"],
                 max_seq=64, rope_type=0, theta=cfg["theta"], eps=cfg["eps"])
        model = O.forward_model(c, seed=1, weight_type="q8_0")
        ref = O.reference(avx2=True)
        tokens = np.arange(n_tokens, dtype=np.int32)
        ref.forward_tokens(model, tokens[:1], tokens[:1])  # warm
        t0 = time.perf_counter()
        ref.forward_tokens(model, tokens, tokens)
        s = (time.perf_counter() - t0) / n_tokens
        return {"seconds_per_token_layer": round(s, 4), "tokens_per_s": round(1 / s, 2),
                "threads": os.cpu_count(), "sample": f"{n_tokens} tokens, 1 layer, Q8_0"}
    except Exception as e:  # the baseline is informative only
        return {"error": str(e)}


# ------------------------------------------------------------ attention

ATT_LAYERS = 16  # cache layers rotated per launch: 16 x 64 MB K+V at 8B, S = 8192
PREFILL_TOKENS = (512, 4096)  # causal prompt chunks from position 0
PREFILL_IMAGE_MIN_TOKENS = 1024  # the library's pre-split tile images from here (head_dim 128)


def attention_bench(mlk, steps, peak, path):
    """Decode attention launches over a cache of ATT_LAYERS layers (each
    launch reads another layer, so a pass over the rotation exceeds the
    MALL), timed between two events on the stream they run on."""
    out = {"workload": "decode attention over a device KV cache (and causal prefill of a "
                       "prompt chunk), N(0, 0.02) cache and queries",
           "peak_GBps": peak, "peak_TFLOPs": MFMA_FP32_PEAK_TFLOPS}
    st = mlk.Stream()
    S = 8192
    for name, H, KV, hd in (("llama3_8b", 32, 8, 128), ("llama3_70b", 64, 8, 128)):
        n = ATT_LAYERS * S * KV * hd
        kc, vc = mlk.DeviceBuffer.empty((n,)), mlk.DeviceBuffer.empty((n,))
        mlk.fill_normal(kc, n, 0.0, 0.02, 11)
        mlk.fill_normal(vc, n, 0.0, 0.02, 12)
        rows = {}
        cases = [("T1_pos%d" % p, np.array([p], np.int32)) for p in (511, 2047, 4095, 8191)]
        if name == "llama3_8b":
            for t in (16, 64):
                cases.append((f"T{t}_uniform0_8191", workloads.decode_positions(t, S - 1, 42)))
        for case, pos in cases:
            T = pos.size
            q = mlk.DeviceBuffer.empty((T, H * hd))
            mlk.fill_normal(q, T * H * hd, 0.0, 0.02, 13)
            o = mlk.DeviceBuffer.empty((T, H * hd))
            d_pos = mlk.DeviceBuffer.from_array(pos)
            max_ctx = int(pos.max()) + 1
            wsb = mlk.attention_workspace_bytes(T, H, KV, hd, max_ctx)
            ws = mlk.DeviceBuffer(max(wsb, 4), np.uint8)

            def launch(i):
                mlk.attention_decode(q, kc, vc, ATT_LAYERS, S, H, KV, hd, i % ATT_LAYERS, T, o,
                                     max_ctx, positions=d_pos, workspace=ws, workspace_bytes=wsb,
                                     stream=st)
            if T >= 5:  # the shared tiles: matrix-core work at the clock's steady state
                _warm_clock(mlk, st, launch)
            for i in range(3):
                launch(i)
            st.synchronize()
            e0, e1 = mlk.Event(), mlk.Event()
            e0.record(st)
            for i in range(3, 3 + steps):
                launch(i)
            e1.record(st)
            e1.synchronize()
            ms = e0.elapsed_ms(e1) / steps
            nb = workloads.bytes_attention(pos, H, KV, hd)
            gbs = nb / (ms * 1e-3) / 1e9
            if T < 4:  # one token per launch row: each token streams its own prefix (HBM)
                rows[case] = {"us": round(ms * 1e3, 2), "bytes": nb, "GBps": round(gbs, 1),
                              "frac_of_peak": round(gbs / peak, 4), "workspace_bytes": wsb}
                print(f"attention {name} {case}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s", flush=True)
            else:  # tokens share each K/V tile on the matrix cores: against the MFMA peak
                fl = workloads.flops_decode_attention(pos, H, hd)
                tf = fl / (ms * 1e-3) / 1e12
                apk, abasis = attention_peak(hd)
                rows[case] = {"us": round(ms * 1e3, 2), "flops": fl, "TFLOPs": round(tf, 2),
                              "peak_TFLOPs": round(apk, 1), "peak_basis": abasis,
                              "frac_of_peak": round(tf / apk, 4),
                              "token_prefix_bytes": nb, "token_prefix_GBps": round(gbs, 1),
                              "workspace_bytes": wsb}
                print(f"attention {name} {case}: {ms * 1e3:.2f} us, {tf:.1f} TFLOP/s "
                      f"({100 * tf / apk:.1f}% of {abasis}; per-token prefixes "
                      f"{gbs:.0f} GB/s)", flush=True)
        # causal prefill of a prompt chunk at positions 0..T-1 (matrix cores):
        # its own entry (each workgroup splits its K/V tiles into bf16
        # pieces), and the decode entry with a workspace for the pre-split
        # tile images (one split launch, then the tiles: the batched layer's
        # path), both launches timed
        for T, images in [(T, im) for T in PREFILL_TOKENS for im in (False, True)]:
            q = mlk.DeviceBuffer.empty((T, H * hd))
            mlk.fill_normal(q, T * H * hd, 0.0, 0.02, 14)
            o = mlk.DeviceBuffer.empty((T, H * hd))
            img_bytes = KV * ((T + 31) // 32) * 2 * 3 * 32 * 128 * 2 if hd == 128 else 0
            if images and (img_bytes == 0 or T < PREFILL_IMAGE_MIN_TOKENS):
                continue
            img = mlk.DeviceBuffer(img_bytes, np.uint8) if images else None

            def launch(i):
                if images:
                    mlk.attention_decode(q, kc, vc, ATT_LAYERS, S, H, KV, hd, i % ATT_LAYERS, T,
                                         o, T, pos0=0, workspace=img, workspace_bytes=img_bytes,
                                         stream=st)
                else:
                    mlk.attention_prefill(q, kc, vc, ATT_LAYERS, S, H, KV, hd, i % ATT_LAYERS,
                                          0, T, o, stream=st)
            _warm_clock(mlk, st, launch)
            for i in range(2):
                launch(i)
            st.synchronize()
            n_pf = max(2, steps // 10)
            e0, e1 = mlk.Event(), mlk.Event()
            e0.record(st)
            for i in range(2, 2 + n_pf):
                launch(i)
            e1.record(st)
            e1.synchronize()
            ms = e0.elapsed_ms(e1) / n_pf
            fl = workloads.flops_prefill_attention(T, H, hd)
            tf = fl / (ms * 1e-3) / 1e12
            apk, abasis = attention_peak(hd)
            key = "prefill_T%d%s" % (T, "_images" if images else "")
            rows[key] = {"us": round(ms * 1e3, 2), "flops": fl,
                         "TFLOPs": round(tf, 2), "peak_TFLOPs": round(apk, 1),
                         "peak_basis": abasis, "frac_of_peak": round(tf / apk, 4)}
            print(f"attention {name} prefill T={T}{' (tile images)' if images else ''}: "
                  f"{ms * 1e3:.1f} us, {tf:.1f} TFLOP/s ({100 * tf / apk:.1f}% of {abasis})",
                  flush=True)
            if img is not None:
                img.close()
        out[name] = {"n_heads": H, "n_kv_heads": KV, "head_dim": hd, "cases": rows}
        del kc, vc
    with open(path, "w") as f:
        json.dump(out, f, indent=1)


CALIB_FLOATS = 64 << 20  # 256 MiB per buffer


def calibrate(mlk, steps):
    """A plain streaming kernel of known traffic for scaling rocprofv3's
    FETCH_SIZE / WRITE_SIZE: SiLU reads one 256 MiB buffer and writes
    another, on three rotating buffer pairs."""
    pairs = [(mlk.DeviceBuffer.empty((CALIB_FLOATS,)), mlk.DeviceBuffer.empty((CALIB_FLOATS,)))
             for _ in range(N_SETS)]
    for i, (x, _) in enumerate(pairs):
        mlk.fill_normal(x, CALIB_FLOATS, 0.0, 1.0, 1000 + i)
    mlk.synchronize()
    e0, e1 = mlk.Event(), mlk.Event()
    e0.record()
    for i in range(steps):
        x, y = pairs[i % N_SETS]
        mlk.silu(x, y, CALIB_FLOATS)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_ms(e1) / steps
    print(json.dumps({"calibration": "silu", "bytes_read": 4 * CALIB_FLOATS,
                      "bytes_written": 4 * CALIB_FLOATS, "launches": steps,
                      "us_per_launch": round(ms * 1e3, 2),
                      "GBps": round(8 * CALIB_FLOATS / (ms * 1e-3) / 1e9, 1)}))


# ------------------------------------------------------- rocprof summaries

CHAIN_KERNELS = {"GatherF32Vec": "gather_f32", "AddRmsNormVec": "add_rmsnorm",
                 "RopePipe": "rope", "StreamKernel": "swiglu"}
GATHER_QUANT_ORDER = ("q8_0", "q4_0", "q4_1")  # the order c4_gathers runs them in

PROFILE_COMMANDS = [
    "rocprofv3 --kernel-trace --stats --output-format csv -d gpurun_out/prof_kt -o bench "
    "-- python3 bench.py",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/prof_fetch -o bench "
    "-- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/prof_write -o bench "
    "-- python3 bench.py --no-cpu-baseline --steps 5 --warmup 1",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/prof_cfetch -o calib "
    "-- python3 bench.py --calibrate --steps 5",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/prof_cwrite -o calib "
    "-- python3 bench.py --calibrate --steps 5",
    "python3 bench.py --rocprof-report gpurun_out/prof_kt gpurun_out/prof_fetch "
    "gpurun_out/prof_write gpurun_out/prof_cfetch gpurun_out/prof_cwrite",
]


def _one_csv(d, suffix):
    import glob
    files = glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return files[0]


def _counter_means(d, counter):
    """{(kernel, grid): mean counter value in KiB} of a --pmc run."""
    import csv
    sums = {}
    for r in csv.DictReader(open(_one_csv(d, "counter_collection.csv"))):
        if r["Counter_Name"] != counter:
            continue
        key = (r["Kernel_Name"], int(r["Grid_Size"]))
        acc = sums.setdefault(key, [0.0, 0])
        acc[0] += float(r["Counter_Value"])
        acc[1] += 1
    return {k: v[0] / v[1] for k, v in sums.items()}


def _short(name):
    """"void mlk::(anonymous namespace)::K<...>(args)" -> "K<...>"."""
    import re
    name = name.replace("(anonymous namespace)::", "").replace("mlk::", "")
    m = re.search(r"(\w+(?:<[^()]*>)?)\(", name)
    return m.group(1) if m else name


def _base(name):
    return _short(name).split("<")[0]


def _sections(rows):
    """rows: (dispatch_id, kernel name, grid, value) in any order.  Walks them
    in dispatch order, assigning each launch to the section the last marker
    (a ZeroKernel of a marking grid) opened; returns
    {section: [(short name, grid, value)]}.  Input generation, quantization
    and copy kernels are left out, except that QuantizeKernel launches are
    kept as separators."""
    out = {}
    phase = None
    for _, name, grid, value in sorted(rows, key=lambda r: r[0]):
        base = _base(name)
        if base == "ZeroKernel":
            phase = phase_of_grid(grid) or phase
            continue
        if phase is None or base in ("FillNormalKernel",) or base.startswith("__amd"):
            continue
        out.setdefault(phase, []).append((_short(name), base, grid, value))
    return out


def _op_of(section_rows):
    """Labels each launch of a section with its op: the chain kernels by name,
    the quantized gathers by their place after each QuantizeKernel."""
    labelled = []
    q = -1
    for short, base, grid, value in section_rows:
        if base == "QuantizeKernel":
            q += 1
            continue
        if base == "GatherQuantKernel":
            op = GATHER_QUANT_ORDER[q] if 0 <= q < len(GATHER_QUANT_ORDER) else base
        else:
            op = CHAIN_KERNELS.get(base, short)
        labelled.append((op, short, grid, value))
    return labelled


def rocprof_report(kt_dir, fetch_dir, write_dir, cfetch_dir, cwrite_dir):
    import csv
    peak = workloads.HBM_PEAK_GBS
    trace = [(int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Grid_Size_X"]) *
              int(r.get("Grid_Size_Y", 1) or 1) * int(r.get("Grid_Size_Z", 1) or 1),
              (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
             for r in csv.DictReader(open(_one_csv(kt_dir, "kernel_trace.csv")))]

    def counters(d, counter):
        return [(int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["Grid_Size"]),
                 float(r["Counter_Value"]))
                for r in csv.DictReader(open(_one_csv(d, "counter_collection.csv")))
                if r["Counter_Name"] == counter]

    # calibration: SiLU over 256 MiB reads and writes 256 MiB per launch
    calib_kib = 4 * CALIB_FLOATS / 1024
    cf = [v for _, n, _, v in counters(cfetch_dir, "FETCH_SIZE") if _base(n) == "StreamKernel"]
    cw = [v for _, n, _, v in counters(cwrite_dir, "WRITE_SIZE") if _base(n) == "StreamKernel"]
    f_factor, w_factor = (sum(cf) / len(cf)) / calib_kib, (sum(cw) / len(cw)) / calib_kib
    durations = {k: _op_of(v) for k, v in _sections(trace).items()}
    fetch = {k: _op_of(v) for k, v in _sections(counters(fetch_dir, "FETCH_SIZE")).items()}
    write = {k: _op_of(v) for k, v in _sections(counters(write_dir, "WRITE_SIZE")).items()}

    def mean(xs):
        return sum(xs) / len(xs) if xs else None

    def table(section, nbytes):
        """(op, kernel, calls, avg us, min us, algorithmic GB/s, FETCH KiB,
        WRITE KiB, HBM bytes, algorithmic bytes) per op of a section (its
        largest grid per op: the per-op timing pass)."""
        rows = []
        for op in dict.fromkeys(o for o, *_ in durations.get(section, [])):
            grids = [g for o, _, g, _ in durations[section] if o == op]
            g = max(grids)
            d = [v for o, _, gg, v in durations[section] if o == op and gg == g]
            kname = [k for o, k, gg, _ in durations[section] if o == op and gg == g][0]
            fk = mean([v for o, _, gg, v in fetch.get(section, []) if o == op and gg == g])
            wk = mean([v for o, _, gg, v in write.get(section, []) if o == op and gg == g])
            hbm = (fk / f_factor + wk / w_factor) * 1024 if fk is not None and wk is not None else None
            avg = mean(d)
            nb = nbytes.get(op)
            rows.append((op, kname, len(d), avg, min(d),
                         nb / (avg * 1e-6) / 1e9 if nb else float("nan"), fk, wk, hbm, nb))
        return rows

    def fmt(r):
        op, k, n, avg, mn, gbs, fk, wk, hbm, nb = r
        f = lambda x, spec: (spec % x) if x is not None else "n/a"  # noqa: E731
        return "| %s | %s | %d | %.2f | %.2f | %.1f | %s | %s | %s | %s |" % (
            op, k, n, avg, mn, gbs, f(fk, "%.0f"), f(wk, "%.0f"), f(hbm, "%.0f"), f(nb, "%d"))

    head = ["| op | kernel | calls | avg us | min us | algorithmic GB/s (avg) | FETCH_SIZE KiB | "
            "WRITE_SIZE KiB | HBM bytes / launch | algorithmic bytes / launch |",
            "|---|---|---|---|---|---|---|---|---|---|"]
    preamble = ["Commands (run from the repo root on one MI355X; the last line writes this "
                "file and the other summaries of the same command):", ""]
    preamble += ["    " + c for c in PROFILE_COMMANDS]
    preamble += ["", "Counter calibration (SiLU over 256 MiB: 256 MiB read + 256 MiB written per "
                 "launch): FETCH_SIZE reads %.4f x the true bytes, WRITE_SIZE %.4f x; HBM bytes "
                 "below are the counters divided by these factors.  Launches are attributed to "
                 "configs by the section markers bench.py launches (a ZeroKernel whose grid "
                 "names the section); the rows are each op's per-launch timing pass (its "
                 "largest grid in the section)." % (f_factor, w_factor), ""]
    out_dir = os.path.join(ROOT, "profiles")
    os.makedirs(out_dir, exist_ok=True)
    traffic = {}

    def write_md(fname, title, parts, unique=None):
        """unique: {op: unique-row bytes} of Zipf gathers, quoted beside."""
        md = [f"# {title}: rocprofv3 summary", ""] + preamble
        for sub, rows, note in parts:
            md += [f"## {sub}", ""] + ([note, ""] if note else []) + head + [fmt(r) for r in rows] + [""]
            ur = [r for r in rows if unique and r[0] in unique]
            if ur:
                md += ["Zipf gathers, each distinct table row counted once (the fraction bench.py "
                       "quotes):", "", "| op | unique-row bytes / launch | GB/s (avg us) | "
                       "fraction of 8 TB/s |", "|---|---|---|---|"]
                for r in ur:
                    gbs = unique[r[0]] / (r[3] * 1e-6) / 1e9
                    md.append("| %s | %d | %.1f | %.4f |" % (r[0], unique[r[0]], gbs, gbs / peak))
                md.append("")
        with open(os.path.join(out_dir, fname), "w") as f:
            f.write("\n".join(md))
        return md

    c3 = workloads.CONFIGS["c3_prefill_8b"]
    c3_rows = table("c3_ops", op_bytes(workloads, c3, c3["tokens"]))
    c4 = workloads.CONFIGS["c4_quant_gather"]
    c4_rows = table("c4_gather", {q: workloads.bytes_gather_quant(q, c4["tokens"], c4["dim"])
                                  for q in GATHER_QUANT_ORDER})
    c5 = workloads.CONFIGS["c5_70b"]
    T5 = c5["tokens"]
    c5_rows = table("c5_ops", {"add_rmsnorm": workloads.bytes_add_rmsnorm(T5, c5["dim"]),
                               "rope": workloads.bytes_rope(T5, c5["n_heads"], c5["n_kv_heads"],
                                                            c5["head_dim"]),
                               "swiglu": workloads.bytes_swiglu(T5, c5["ffn"])})
    for sec, rows in (("c3_ops", c3_rows), ("c4_gather", c4_rows), ("c5_ops", c5_rows)):
        traffic[sec] = {r[0]: round(r[8]) for r in rows if r[8] is not None}
    ids3 = workloads.zipf_ids(c3["tokens"], c3["vocab"], 1.1, c3["seed"])
    md = write_md("chain_c3_prefill_8b_rocprof.md",
                  "Op chain, configs[2] (Llama-3-8B shape, T = 4096)",
                  [("Per-launch timing pass (bench.py ops)", c3_rows,
                    "The gather's table rows repeat (Zipf ids): its counter bytes are below its "
                    "algorithmic bytes, and its fraction of peak is quoted on distinct rows.")],
                  {"gather_f32": workloads.bytes_gather_unique(ids3, c3["dim"])})
    ids4 = workloads.zipf_ids(c4["tokens"], c4["vocab"], 1.1, c4["seed"])
    write_md("gather_quant_c4_rocprof.md",
             "Quantized token gathers, configs[3] (table 128256 x 4096, T = 4096 Zipf(1.1) ids)",
             [("Q8_0 / Q4_0 / Q4_1 gathers", c4_rows,
               "Hot rows repeat: counter bytes fall below the algorithmic bytes.")],
             {q: workloads.bytes_gather_unique(ids4, c4["dim"], q) for q in GATHER_QUANT_ORDER})
    write_md("chain_c5_70b_rocprof.md", "Op chain, configs[4] (Llama-3-70B shape, T = 8192)",
             [("Per-launch timing pass (bench.py configs.c5_70b.ops)", c5_rows, None)])
    # decode and tiny: latency-bound; every launch of the sections by kernel and grid
    lines = ["# Decode steps, configs[1], and the tiny chain, configs[0]: rocprofv3 summary",
             ""] + preamble
    for sec, title in (("c2_decode", "configs[1]: 8B chain at T = 1..64, eager launches"),
                       ("c2_decode_graph", "configs[1]: 8B chain at T = 1..64, graph-replayed launches"),
                       ("c1_tiny", "configs[0]: tiny chain, 6 tokens, eager launches"),
                       ("c1_tiny_graph", "configs[0]: tiny chain, 6 tokens, graph-replayed launches")):
        lines += [f"## {title}", "", "| op | kernel | grid (work-items) | launches | avg us | min us |",
                  "|---|---|---|---|---|---|"]
        groups = {}
        for op, k, g, v in durations.get(sec, []):
            groups.setdefault((op, k, g), []).append(v)
        for (op, k, g), d in sorted(groups.items(), key=lambda kv: (kv[0][0], kv[0][2])):
            lines.append("| %s | %s | %d | %d | %.2f | %.2f |" % (op, k, g, len(d), mean(d), min(d)))
        lines.append("")
    with open(os.path.join(out_dir, "chain_decode_tiny_rocprof.md"), "w") as f:
        f.write("\n".join(lines))
    # the 8B decode layer (decode_layer_8b): every kernel of the section by
    # name and grid, with the counters' HBM bytes
    fsec, wsec = fetch.get("decode_layer_8b", []), write.get("decode_layer_8b", [])
    lines = ["# One Llama-3-8B layer as a decode step (bench.py decode_layer_8b): rocprofv3 "
             "summary", ""] + preamble
    lines += ["The section runs, in this order, Q8_0, Q4_0 and F32 weights (Q8_0 / Q4_0 on "
              "their planar copies), each for one token at position 8191 and for 16 tokens at "
              "positions in 0..8191, over 4 rotated layers.  Weight preparation (quantization, "
              "planar repacking) is left out.", "",
              "| kernel | grid (work-items) | launches | avg us | min us | HBM bytes / launch |",
              "|---|---|---|---|---|---|"]
    groups = {}
    for op, k, g, v in durations.get("decode_layer_8b", []):
        if _base(k) in ("QuantizeKernel", "ToPlanar"):
            continue
        groups.setdefault((k, g), []).append(v)
    for (k, g), d in groups.items():
        fk = mean([v for _, kk, gg, v in fsec if kk == k and gg == g])
        wk = mean([v for _, kk, gg, v in wsec if kk == k and gg == g])
        hbm = "%.0f" % ((fk / f_factor + wk / w_factor) * 1024) if fk is not None and wk is not None else "n/a"
        lines.append("| %s | %d | %d | %.2f | %.2f | %s |" % (k, g, len(d), mean(d), min(d), hbm))
    lines.append("")
    with open(os.path.join(out_dir, "decode_layer_8b_rocprof.md"), "w") as f:
        f.write("\n".join(lines))
    sw = [r for r in c3_rows if r[0] == "swiglu"][0]
    with open(PMC_FILE, "w") as f:
        json.dump({"kernel": "StreamKernel<SwiGluOp> (swiglu)", "workload": "c3_prefill_8b",
                   "hbm_bytes_per_launch": round(sw[8]),
                   "algorithmic_bytes_per_launch": sw[9],
                   "fetch_size_kib": round(sw[6], 1), "write_size_kib": round(sw[7], 1),
                   "fetch_factor": round(f_factor, 5), "write_factor": round(w_factor, 5),
                   "rocprof_avg_us": round(sw[3], 2),
                   "per_section_hbm_bytes": traffic,
                   "commands": PROFILE_COMMANDS}, f, indent=1)
    print("\n".join(md))


def kernel_summary(out_md, title, bench_json, kt_dir, fetch_dir=None, write_dir=None):
    """Markdown summary of a rocprofv3 kernel trace (and optional counter runs)
    next to the bench JSON of the same command."""
    import csv
    launches = {}
    for r in csv.DictReader(open(_one_csv(kt_dir, "kernel_trace.csv"))):
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y", 1) or 1) *
               int(r.get("Grid_Size_Z", 1) or 1))
        launches.setdefault(key, []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    fetch = _counter_means(fetch_dir, "FETCH_SIZE") if fetch_dir else {}
    write = _counter_means(write_dir, "WRITE_SIZE") if write_dir else {}
    with open(PMC_FILE) as f:
        calib = json.load(f)
    ff, wf = calib["fetch_factor"], calib["write_factor"]
    cmds = [c for c in os.environ.get("PROFILE_COMMANDS", "").split("\n") if c.strip()]
    md = [f"# {title}: rocprofv3 summary", "", "Commands (repo root, one MI355X):", ""]
    md += ["    " + c for c in cmds]
    md += ["", "Kernel durations from the kernel trace (grid = total work-items)"
           + (", HBM bytes per launch = FETCH_SIZE / %.4f + WRITE_SIZE / %.4f (KiB -> bytes), "
              "the factors of the committed copy-kernel calibration" % (ff, wf)
              if fetch else "") + ":", "",
           "| kernel | grid | calls | avg us | min us |" + (" HBM bytes / launch |" if fetch else ""),
           "|---|---|---|---|---|" + ("---|" if fetch else "")]
    def short(name):
        # "void mlk::(anonymous namespace)::K<...>(args)" -> "K<...>"
        import re
        name = name.replace("(anonymous namespace)::", "").replace("mlk::", "")
        m = re.search(r"(\w+(?:<[^()]*>)?)\(", name)
        return m.group(1) if m else name

    for (name, grid), d in sorted(launches.items(), key=lambda kv: (short(kv[0][0]), kv[0][1])):
        if name.startswith("__amd") or "Fill" in name or "Quantize" in name or "ZeroKernel" in name:
            continue
        row = "| %s | %d | %d | %.2f | %.2f |" % (short(name), grid, len(d), sum(d) / len(d),
                                                  min(d))
        if fetch:
            fk = [v for (k, g), v in fetch.items() if k == name and g == grid]
            wk = [v for (k, g), v in write.items() if k == name and g == grid]
            row += " %s |" % (("%.0f" % ((fk[0] / ff + wk[0] / wf) * 1024)) if fk and wk else "n/a")
        md.append(row)
    md += ["", "Results of the same command (bench.py JSON, events around back-to-back "
           "launches -- for --linear, around one replay of a HIP graph holding each "
           "projection's calls, so the figure is kernel time, not Python dispatch; HBM-bound "
           "cases on rotating cold copies, against 8 TB/s; "
           "matrix-core cases against the peak of the instruction they run: 157.3 TFLOP/s fp32 MFMA, or for bf16 piece products the 2.5 PFLOP/s bf16 peak over the bf16 MACs per useful MAC, 3 in the GEMM and 6 in the attention):", "",
           "| case | us | throughput | fraction of peak |", "|---|---|---|---|"]

    def rate(node, prefix=""):
        if prefix + "GBps" in node:
            return "%.1f GB/s" % node[prefix + "GBps"]
        return "%.2f TFLOP/s" % node[prefix + "TFLOPs"]

    def walk(node, path):
        if isinstance(node, dict):
            # GEMM results: per projection only at the largest row count
            per_op_skipped = ("TFLOPs" in node and len(path) >= 2 and path[-2].isdigit()
                              and path[-2] != str(max(GEMM_TOKENS)))
            if "us" in node and ("GBps" in node or "TFLOPs" in node) and not per_op_skipped:
                md.append("| %s | %.2f | %s | %.3f |" % (" / ".join(path), node["us"], rate(node),
                                                         node["frac_of_peak"]))
            if "layer_us" in node:
                md.append("| %s | %.2f | %s | %.3f |" % (" / ".join(path + ["layer"]),
                                                         node["layer_us"], rate(node, "layer_"),
                                                         node["layer_frac_of_peak"]))
            for k, v in node.items():
                if k not in ("ops",) or isinstance(v, dict):
                    walk(v, path + ([k] if k not in ("ops", "cases") else []))

    res = json.load(open(bench_json))
    walk(res, [])
    if res.get("markers"):
        # --linear: each timed graph replay sits between a start marker
        # (grid 256 * (LINEAR_MARK_BASE + i)) and an end marker; the
        # kernels in between are that replay's, calls_per_replay calls
        rows = sorted(csv.DictReader(open(_one_csv(kt_dir, "kernel_trace.csv"))),
                      key=lambda r: int(r["Dispatch_Id"]))
        sums, spans, cur = {}, {}, None
        for r in rows:
            g = int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y", 1) or 1) * int(r.get("Grid_Size_Z", 1) or 1)
            t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
            if _base(r["Kernel_Name"]) == "ZeroKernel" and g % 256 == 0:
                k = g // 256
                if k == LINEAR_MARK_END:
                    cur = None
                    continue
                if k >= LINEAR_MARK_BASE:
                    cur = k - LINEAR_MARK_BASE
                    continue
            if cur is None:
                continue
            sums[cur] = sums.get(cur, 0.0) + (t1 - t0) / 1e3
            lo, hi = spans.get(cur, (t0, t1))
            spans[cur] = (min(lo, t0), max(hi, t1))
        n = res["calls_per_replay"]

        def event_us(label):
            qt, t, name = label.split(" / ")
            node = res[qt][t]
            return node["layer_us"] if name == "layer" else node["ops"][name]["us"]
        md += ["", "Event time per call (the bench JSON's run: one replayed HIP graph per "
               "projection) against the kernels of the same calls in the kernel trace (kernel "
               "sum: the durations of their kernels; span: first start to last end, the gaps "
               "between launches included; both per call):", "",
               "| case | event us / call | trace kernel sum us / call | trace span us / call | "
               "event / kernel sum |", "|---|---|---|---|---|"]
        for i, label in sorted(((int(k), v) for k, v in res["markers"].items())):
            if i not in sums:
                continue
            ev = event_us(label)
            ks = sums[i] / n
            sp = (spans[i][1] - spans[i][0]) / 1e3 / n
            md.append("| %s | %.2f | %.2f | %.2f | %.3f |" % (label, ev, ks, sp, ev / ks))
    with open(out_md, "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n".join(md[:40]))


def progress(msg):
    """A progress line on stderr (the JSON result is the only stdout line)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


def pmc_summary(out_md, title, d):
    """Mean counter values per dispatch, by kernel and grid, of a --pmc run
    (input generation, quantization, repacking and markers left out)."""
    import csv
    acc = {}
    for r in csv.DictReader(open(_one_csv(d, "counter_collection.csv"))):
        if _base(r["Kernel_Name"]) in ("FillNormalKernel", "QuantizeKernel", "ToPlanar",
                                       "ZeroKernel") or r["Kernel_Name"].startswith("__amd"):
            continue
        key = (_short(r["Kernel_Name"]), int(r["Grid_Size"]))
        acc.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    names = sorted({c for v in acc.values() for c in v})
    cmds = [c for c in os.environ.get("PROFILE_COMMANDS", "").split("\n") if c.strip()]
    md = [f"# {title}: rocprofv3 counters", "", "Commands (repo root, one MI355X):", ""]
    md += ["    " + c for c in cmds]
    md += ["", "Mean value per dispatch (the SQ counters summed over the GPU), by kernel and grid "
           "(total work-items):", "",
           "| kernel | grid | " + " | ".join(names) + " |", "|---|---|" + "---|" * len(names)]
    for (k, g), v in acc.items():
        md.append("| %s | %d | " % (k, g) + " | ".join(
            "%.0f" % (sum(v[n]) / len(v[n])) if n in v else "n/a" for n in names) + " |")
    with open(out_md, "w") as f:
        f.write("\n".join(md) + "\n")
    print("\n".join(md))


def main():
    args = parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.kernel_summary:
        kernel_summary(*args.kernel_summary)
        return
    if args.rocprof_report:
        rocprof_report(*args.rocprof_report)
        return
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(the per-layer ops are row-independent: a data-parallel shard per GPU needs no "
              "exchange, see the sharding notes)", file=sys.stderr)
        sys.exit(2)
    mlk = mlk_pkg
    mlk.set_device(0)
    if args.calibrate:
        calibrate(mlk, args.steps)
        return
    if args.linear:
        linear_bench(mlk, args.steps, workloads.HBM_PEAK_GBS, args.linear, eager=args.linear_eager)
        return
    if args.attention:
        attention_bench(mlk, args.steps, workloads.HBM_PEAK_GBS, args.attention)
        return
    if args.gemm:
        gemm_bench(mlk, args.steps, args.gemm)
        return
    if args.layer:
        layer_bench(mlk, args.steps, args.layer)
        return
    if args.decode_layer:
        import importlib
        fwd = importlib.import_module(mlk.__name__ + ".forward")
        res = decode_layer_bench(mlk, fwd, args.steps, log=sys.stderr)
        with open(args.decode_layer, "w") as f:
            json.dump(res, f, indent=1)
        return
    peak = workloads.HBM_PEAK_GBS
    cfg = workloads.CONFIGS["c3_prefill_8b"]
    T = cfg["tokens"]
    marks = Marks(mlk)
    chain = Chain(mlk, cfg, T, seed=cfg["seed"])
    marks("c3_chain", chain.stream)
    total_ms = chain.run(args.steps, args.warmup)
    nbytes = op_bytes(workloads, cfg, T)
    unique_gather = workloads.bytes_gather_unique(chain.ids_host, cfg["dim"])
    # the gather's hot Zipf rows come from cache: each distinct row counts once
    chain_bytes = sum(nbytes.values()) - nbytes["gather_f32"] + unique_gather
    marks("c3_ops", chain.stream)
    ops = summarize(chain.run_ops(args.steps), nbytes, peak)
    add_unique(ops["gather_f32"], unique_gather, peak)
    gather_fractions(ops["gather_f32"])
    for op, hbm in counter_traffic().get("c3_ops", {}).items():
        if op in ops:
            add_counter(ops[op], hbm, peak)
    value = chain_bytes * args.steps / (total_ms * 1e-3) / 1e9
    sw = ops["swiglu"]
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (device-generated N(0,0.02) activations/table, N(1,0.1) norm weight, "
                "Zipf(1.1) ids seed 42)",
        "config": {"workload": "c3_prefill_8b op chain: gather -> add+rmsnorm -> rope -> swiglu",
                   "tokens": T, "dim": cfg["dim"], "n_heads": cfg["n_heads"],
                   "n_kv_heads": cfg["n_kv_heads"], "head_dim": cfg["head_dim"],
                   "ffn_dim": cfg["ffn"], "vocab": cfg["vocab"], "rope_theta": cfg["theta"],
                   "positions": "0..T-1", "chain_bytes": chain_bytes,
                   "chain_bytes_algorithmic": sum(nbytes.values()),
                   "rotating_sets": N_SETS},
        "frac_of_peak": round(value / peak, 4),
        "us_per_chain": round(total_ms * 1e3 / args.steps, 2),
        "ops": ops,
        "roofline": {"bound": "hbm", "kernel": "swiglu (StreamKernel<SwiGluOp>)",
                     "achieved": sw["GBps"], "peak": peak, "unit": "GB/s",
                     "frac": round(sw["GBps"] / peak, 4),
                     "bytes_per_launch": sw["bytes"], "us_per_launch": sw["us"],
                     "traffic": traffic_from_profiles()},
        "device": mlk.device_info(0),
    }
    with_cpu = not args.no_cpu_baseline
    table_host = chain.table.download() if with_cpu else None  # shared by C3 and C2
    if with_cpu:
        result["cpu_baseline"] = cpu_chain_baseline(
            chain_host_bufs(chain, cfg, T, table_host), T, chain_bytes,
            f"the whole configs[2] chain (T={T}, Llama-3-8B shapes)")
    progress("configs[2] chain and its CPU baseline done")
    # the launch-bound decode chains keep a 10-step warmup: hundreds of their
    # steps alone leave the GPU idle between launches most of the time and
    # its clock falls (500 steps: C1 20.8 and C2 23.5 us per chain against
    # 16.9 and 17.2-18.0 after 10), where a decode step interleaves them with
    # weight GEMVs that keep it busy
    w_chain = min(args.warmup, LAUNCH_BOUND_WARMUP)
    configs = {"c1_tiny": None, "c2_decode_8b": c2_decode(mlk, args.steps, w_chain, marks,
                                                          chain.table, table_host)}
    del chain, table_host
    progress("configs[1] decode steps done")
    configs["c1_tiny"] = c1_tiny(mlk, args.steps, w_chain, marks)
    progress("configs[0] tiny chain done")
    configs["c4_quant_gather"] = c4_gathers(mlk, args.steps, peak, marks, with_cpu)
    progress("configs[3] quantized gathers done")
    configs["c5_70b"] = c5_chain(mlk, args.steps, args.warmup, peak, marks, with_cpu)
    progress("configs[4] 70B chain done")
    result["configs"] = configs
    # beside the op chain: one 8B layer through mlk_forward_layer_batch as a
    # decode step (one token at position 8191; 16 tokens at positions in
    # 0..8191 on the planar weights), weights rotated over 4 layers
    import importlib
    fwd = importlib.import_module(mlk.__name__ + ".forward")
    result["decode_layer_8b"] = decode_layer_bench(mlk, fwd, min(args.steps, 10), log=sys.stderr,
                                                   marks=marks)
    # and the same layer over a 4096-token prompt chunk (Q8_0)
    result["prefill_layer_8b"] = prefill_layer_bench(mlk, fwd, min(args.steps, 10), ("q8_0",),
                                                     token_loop=False, log=sys.stderr,
                                                     marks=marks)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
