"""Benchmark of the per-layer op chain on one MI355X.

Default run (the driver's contract): BASELINE.json configs[2] -- the
Llama-3-8B-shape prefill chain at T = 4096 tokens, fp32:
    gather (F32 embedding, Zipf(1.1) ids) -> residual add + RMSNorm
    -> RoPE on Q [T, 32, 128] and K [T, 8, 128] (positions 0..T-1)
    -> SwiGLU over gate/up [T, 14336]
One step is one pass of the four kernels over one of three rotating buffer
sets (~1 GB each, so no step finds its inputs in the 256 MB MALL).  Inputs
are synthetic, generated on the device, resident in HBM before timing.
`value` is whole-chain algorithmic GB/s over K timed steps (events only at
the two ends).  Per-kernel durations come from a second timed pass that
launches each kernel K times back to back between two HIP events recorded
on the stream the kernels run on.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--extra FILE]

--extra FILE also measures configs 1, 3 and 4 (decode latency at T = 1..64,
the quantized gathers, the 70B chain) and writes them to FILE as JSON; it is
off by default so a rocprofv3 summary of the default command holds only the
chain's launches.
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
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--extra", default=None, help="also measure configs 1, 3, 4 into this JSON file")
    p.add_argument("--no-cpu-baseline", action="store_true")
    return p.parse_args()


class ChainSet:
    """Device buffers of one op-chain input/output set."""

    def __init__(self, mlk, cfg, T, seed):
        D, H, KV, hd, F = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"]
        E = mlk.DeviceBuffer.empty
        self.x = E((T, D))
        self.delta = E((T, D))
        self.y = E((T, D))
        self.q = E((T, H * hd))
        self.k = E((T, KV * hd))
        self.gate = E((T, F))
        self.up = E((T, F))
        self.out = E((T, F))
        mlk.fill_normal(self.delta, T * D, 0.0, 0.02, seed + 1)
        mlk.fill_normal(self.q, T * H * hd, 0.0, 0.02, seed + 2)
        mlk.fill_normal(self.k, T * KV * hd, 0.0, 0.02, seed + 3)
        mlk.fill_normal(self.gate, T * F, 0.0, 0.02, seed + 4)
        mlk.fill_normal(self.up, T * F, 0.0, 0.02, seed + 5)


class Chain:
    """gather -> add+RMSNorm -> RoPE -> SwiGLU on rotating sets."""

    OPS = ("gather_f32", "add_rmsnorm", "rope", "swiglu")

    def __init__(self, mlk, cfg, T, seed, n_sets=N_SETS, ids=None, positions=None):
        self.mlk, self.cfg, self.T = mlk, cfg, T
        D = cfg["dim"]
        self.table = mlk.DeviceBuffer.empty((cfg["vocab"], D))
        mlk.fill_normal(self.table, cfg["vocab"] * D, 0.0, 0.02, seed)
        self.norm_w = mlk.DeviceBuffer.empty((D,))
        mlk.fill_normal(self.norm_w, D, 1.0, 0.1, seed + 100)
        self.ids_host = ids if ids is not None else workloads.zipf_ids(T, cfg["vocab"], 1.1, seed)
        self.ids = mlk.DeviceBuffer.from_array(self.ids_host)
        self.positions_host = positions
        self.positions = mlk.DeviceBuffer.from_array(positions) if positions is not None else None
        self.sets = [ChainSet(mlk, cfg, T, seed + 10 * (i + 1)) for i in range(n_sets)]
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

    def run_ops(self, steps, warmup=3):
        """Per-kernel launch duration: each op launched `steps` times back to
        back over the rotating sets between two events; returns
        {op: ms per launch}."""
        mlk = self.mlk
        out = {}
        for op in self.OPS:
            for i in range(warmup):
                self.launch(self.sets[i % len(self.sets)], op)
            self.stream.synchronize()
            start, stop = mlk.Event(), mlk.Event()
            start.record(self.stream)
            for i in range(steps):
                self.launch(self.sets[i % len(self.sets)], op)
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


# ------------------------------------------------------------ CPU baseline

def cpu_baseline(mlk, chain, cfg, T, workloads):
    """The reference's own CPU ops (oracle/_ref, AVX2/FMA build) over the same
    chain, one token at a time as ForwardBatch runs them; ThreadPool variant
    (ParallelFor over tokens) and single thread.  Falls back to the C port
    (oracle/liboracle.so) when the reference build is absent."""
    import oracle as O

    D, H, KV, hd, F = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"]
    s = chain.sets[0]
    bufs = dict(table=chain.table.download(), vocab=cfg["vocab"], dim=D, ids=chain.ids_host,
                x=np.empty((T, D), np.float32), delta=s.delta.download(),
                norm_w=chain.norm_w.download(), y=np.empty((T, D), np.float32), eps=cfg["eps"],
                q=s.q.download(), k=s.k.download(), n_heads=H, n_kv_heads=KV, head_dim=hd,
                positions=np.arange(T, dtype=np.int32), theta=cfg["theta"],
                gate=s.gate.download(), up=s.up.download(), ffn_out=np.empty((T, F), np.float32),
                ffn_dim=F)
    if O.reference_available(avx2=True):
        impl, kind, build = O.reference(avx2=True), "reference", "oracle/_ref/libref_avx2.so"
    else:
        impl, kind, build = O.oracle(), "port", "oracle/liboracle.so"
    # the box's CPU share for one GPU is 16 cores, whatever nproc reports
    threads = max(1, min(16, os.cpu_count() or 1))
    nbytes = workloads.bytes_chain(cfg, T)

    def timed(n_threads, reps):
        times = []
        for _ in range(reps + 1):  # first rep is warmup
            t0 = time.perf_counter()
            rc = impl.chain(bufs, T, n_threads)
            times.append(time.perf_counter() - t0)
            if rc != 0:
                raise RuntimeError(f"CPU baseline failed (status {rc})")
        return statistics.median(times[1:])

    t_mt = timed(threads, 5)
    t_st = timed(1, 3)
    return {"value": round(nbytes / t_mt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": kind,
            "sample": (f"full config-2 chain (T={T}, 8B shapes), median of 5 reps after 1 warmup; "
                       f"{build}, ParallelFor over tokens"),
            "ms_per_chain": round(t_mt * 1e3, 2),
            "single_thread_value": round(nbytes / t_st / 1e9, 3),
            "single_thread_ms_per_chain": round(t_st * 1e3, 2),
            "cpu_model": _cpu_model()}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def traffic_from_profiles():
    """HBM bytes per SwiGLU launch from the committed rocprofv3 --pmc runs."""
    try:
        with open(PMC_FILE) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------ extra configs

def extra_configs(mlk, workloads, steps, peak):
    res = {}
    c8 = workloads.CONFIGS["c2_decode_8b"]
    dec = {}
    for T in c8["tokens"]:
        pos = workloads.decode_positions(T, c8["max_pos"], c8["seed"])
        ch = Chain(mlk, c8, T, seed=c8["seed"], n_sets=2, positions=pos)
        n = max(steps, 100)
        total = ch.run(n, 10)
        dec[str(T)] = {"us_per_chain": round(total * 1e3 / n, 2),
                       "ops": summarize(ch.run_ops(n), op_bytes(workloads, c8, T), peak)}
        del ch
    res["c2_decode_8b"] = dec
    c4 = workloads.CONFIGS["c4_quant_gather"]
    T, V, D = c4["tokens"], c4["vocab"], c4["dim"]
    table = mlk.DeviceBuffer.empty((V, D))
    mlk.fill_normal(table, V * D, 0.0, 0.02, c4["seed"])
    ids = mlk.DeviceBuffer.from_array(workloads.zipf_ids(T, V, 1.1, c4["seed"]))
    outs = [mlk.DeviceBuffer.empty((T, D)) for _ in range(N_SETS)]
    st = mlk.Stream()
    q = {}
    for qt in ("q8_0", "q4_0", "q4_1"):
        blocks = mlk.DeviceBuffer(mlk.quant_bytes(qt, V, D), np.uint8)
        mlk.quantize(qt, table, V, D, blocks, stream=st)
        for i in range(10):
            mlk.gather_quant(qt, blocks, V, D, ids, T, outs[i % N_SETS], stream=st)
        e0, e1 = mlk.Event(), mlk.Event()
        st.synchronize()
        e0.record(st)
        for i in range(steps):
            mlk.gather_quant(qt, blocks, V, D, ids, T, outs[i % N_SETS], stream=st)
        e1.record(st)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / steps
        q[qt] = summarize({qt: ms}, {qt: workloads.bytes_gather_quant(qt, T, D)}, peak)[qt]
        del blocks
    res["c4_quant_gather"] = q
    del table
    c5 = dict(workloads.CONFIGS["c5_70b"], vocab=1)
    T = c5["tokens"]
    ch = Chain(mlk, c5, T, seed=c5["seed"], n_sets=2, ids=np.zeros(T, np.int32))
    total = ch.run(steps, 5)
    ops = summarize(ch.run_ops(steps), op_bytes(workloads, c5, T), peak)
    ops.pop("gather_f32")  # the 70B config has no gather
    res["c5_70b"] = {"ops": ops}
    return res


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build targets one GPU; --gpus {args.gpus} is not supported "
              "(the per-layer ops are row-independent: a data-parallel shard per GPU needs no "
              "exchange, see the sharding notes)", file=sys.stderr)
        sys.exit(2)
    mlk = mlk_pkg
    mlk.set_device(0)
    peak = workloads.HBM_PEAK_GBS
    cfg = workloads.CONFIGS["c3_prefill_8b"]
    T = cfg["tokens"]
    chain = Chain(mlk, cfg, T, seed=cfg["seed"])
    total_ms = chain.run(args.steps, args.warmup)
    nbytes = op_bytes(workloads, cfg, T)
    chain_bytes = sum(nbytes.values())
    ops = summarize(chain.run_ops(args.steps), nbytes, peak)
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
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(mlk, chain, cfg, T, workloads)
    del chain
    if args.extra:
        extra = extra_configs(mlk, workloads, max(10, args.steps // 2), peak)
        with open(args.extra, "w") as f:
            json.dump(extra, f, indent=1)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
