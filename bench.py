"""Benchmark of the random-walk hot path on one MI355X.

Default workload: uniform random walk on an R-MAT
graph with 2^20 nodes and 2^24 edge samples (a,b,c,d = .57,.19,.19,.05,
deduplicated, int64 CSR), 10 walks per node (10,485,760 walks), walk_length
80, rand = Philox float32 uniforms [N, 80] (seed 2).  One step = one
random_walk() call over the whole batch, inputs resident in HBM.

Prints ONE JSON line with walk-steps/s, the roofline of the walk kernel (HBM
random gather: one 64-B line per dependent read, streams at their byte
count) and a CPU baseline (the oracle's single-threaded restatement of the
reference's eval_cpu loop, timed on a bounded sample of the same walks).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2|c3|c4|c5|csr2|csr4|...]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "walk steps/sec at 1 MI355X + achieved GB/s vs random-gather roofline"
PEAK_HBM_GBS = 8000.0
LINE = 64  # bytes charged per dependent random read

CONFIGS = {
    # name: (description, kind, graph builder args, walks per node, L, extra)
    "c1": ("Cora-like graph (2,708 nodes, 10,556 entries), 2,000 uniform walks, L=5: the "
           "reference tests' workload, bound by launch latency", "uniform", dict(cora=True), 1, 5,
           dict(num_walks=2000)),
    "c1n": ("Cora-like graph, 2,000 node2vec walks, L=5, p=1 q=3 (reference chain): the "
            "reference's rejection-sampling test workload, bound by launch latency", "node2vec",
            dict(cora=True), 1, 5, dict(num_walks=2000, p=1.0, q=3.0, seed=1, rule="ref_chain")),
    "c2": ("R-MAT 2^20 uniform walk, 10 walks/node, L=80", "uniform",
           dict(scale=20, samples=1 << 24, symmetrize=False), 10, 80, {}),
    "c2s": ("R-MAT 2^20 uniform walk, 10 walks/node, L=80, uniforms generated in the kernel "
            "(seed=2, the stream of c2's rand tensor)", "uniform_seeded",
            dict(scale=20, samples=1 << 24, symmetrize=False), 10, 80, {}),
    "c2i": ("R-MAT 2^20 uniform walk, 10 walks/node, L=80, compact int32 output "
            "(out_dtype=torch.int32; same walks as c2)", "uniform",
            dict(scale=20, samples=1 << 24, symmetrize=False), 10, 80, dict(out_dtype="int32")),
    "c3": ("node2vec p=0.5 q=2 on symmetrized R-MAT 2^20, 4 walks/node, L=40", "node2vec",
           dict(scale=20, samples=1 << 24, symmetrize=True), 4, 40,
           dict(p=0.5, q=2.0, seed=3, rule="ref_chain")),
    "c3y": ("node2vec p=0.5 q=2 on symmetrized R-MAT 2^20, 4 walks/node, L=40, with the "
            "symmetric-graph hint (the neighbour test searches the shorter row; same walks as c3)",
            "node2vec", dict(scale=20, samples=1 << 24, symmetrize=True), 4, 40,
            dict(p=0.5, q=2.0, seed=3, rule="ref_chain", symmetric=True)),
    "c3b": ("node2vec p=0.5 q=2 on symmetrized R-MAT 2^20 (the graph of c3), 2,000 walks, "
            "L=40: a call of few walks on a large graph, bound by the walks' chains of dependent "
            "reads", "node2vec", dict(scale=20, samples=1 << 24, symmetrize=True), 1, 40,
            dict(num_walks=2000, p=0.5, q=2.0, seed=3, rule="ref_chain")),
    "c4": ("R-MAT 2^24 uniform walk, 1 walk/node, L=20", "uniform",
           dict(scale=24, samples=1 << 28, symmetrize=False), 1, 20, {}),
    "c5": ("node2vec p=4 q=0.25 (reference chain) on BA 4M nodes m=20 + 64 hubs of 500K, "
           "2 walks/node, L=30", "node2vec", dict(ba=(4_000_000, 20, 64, 500_000)), 2, 30,
           dict(p=4.0, q=0.25, seed=5, rule="ref_chain")),
    "c5x": ("node2vec p=4 q=0.25 (analytic rule) on BA 4M nodes m=20 + 64 hubs of 500K, "
            "2 walks/node, L=30", "node2vec", dict(ba=(4_000_000, 20, 64, 500_000)), 2, 30,
            dict(p=4.0, q=0.25, seed=5, rule="node2vec")),
    "c5xy": ("node2vec p=4 q=0.25 (analytic rule) on BA 4M nodes m=20 + 64 hubs of 500K, "
             "2 walks/node, L=30, with the symmetric-graph hint (same walks as c5x)", "node2vec",
             dict(ba=(4_000_000, 20, 64, 500_000)), 2, 30,
             dict(p=4.0, q=0.25, seed=5, rule="node2vec", symmetric=True)),
}
RULE_ID = {"ref_chain": 0, "node2vec": 1}

# CSR construction from an edge list (the step before the walk): name ->
# (description, R-MAT scale, samples, symmetrize).  Both deduplicate, as the
# walk configurations' graphs do.
CSR_CONFIGS = {
    "csr2": ("CSR build (sort + dedup) of R-MAT 2^20, 2^24 edge samples (the graph of c2)",
             20, 1 << 24, False),
    "csr3": ("CSR build (symmetrize + sort + dedup) of R-MAT 2^20, 2^24 edge samples "
             "(the graph of c3)", 20, 1 << 24, True),
    "csr4": ("CSR build (sort + dedup) of R-MAT 2^24, 2^28 edge samples (the graph of c4)",
             24, 1 << 28, False),
}
CSR_METRIC = "CSR build: input edges/sec at 1 MI355X + achieved GB/s vs HBM roofline"

# Skip-gram context windows after the walk (torch_geometric Node2Vec.sample's
# defaults: walk_length 20, context_size 10, walks_per_node 10, one negative
# walk per positive): name -> (description, R-MAT scale, samples, walks per
# node, L, C).
WIN_CONFIGS = {
    "win2": ("positive + negative context windows (C=10) of 10 uniform walks/node, L=20, "
             "on R-MAT 2^20 (the graph of c2)", 20, 1 << 24, 10, 20, 10),
}
WIN_METRIC = "context windows/sec at 1 MI355X + achieved GB/s vs HBM roofline"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def kernel_source_hash(kind: str) -> str:
    """sha256[:16] over the code (not the comments) of the source files of
    libmlxc.so that one kernel family is built from."""
    from mlx_cluster_amd.build_lib import source_hash
    return source_hash(kind)


# What roofline.traffic counts: rocprofv3 FETCH_SIZE + WRITE_SIZE, the bytes
# between the L2 and the data fabric.  Reads served by the Infinity Cache
# (MALL) are included, so this is an upper bound on DRAM traffic.
TRAFFIC_KIND = ("L2-to-fabric bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated); "
                "Infinity Cache hits included")


def traffic_from_profile(name: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary of the
    same kernel source (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-
    kernel calibration), or None when no summary for this source exists."""
    from mlx_cluster_amd.build_lib import KERNEL_SOURCES
    family = next((k for k in KERNEL_SOURCES if name.startswith(k + "_")), None)
    path = os.path.join(REPO, "profiles", f"{name}_traffic.json")
    if family is None or not os.path.exists(path):
        return None
    d = json.load(open(path))
    if (d.get("kernel_family") != family or
            d.get("kernel_source_sha256_16") != kernel_source_hash(family)):
        return None
    return d.get("hbm_bytes_per_launch")


def uniform_counts(torch, rowptr, walks):
    """Moving steps M (from a node with deg > 0) and sink walks Z (walks that
    meet a deg-0 node before their last step) of a finished uniform walk."""
    L = walks.shape[1] - 1
    M = 0
    sunk = torch.zeros(walks.shape[0], dtype=torch.bool, device=walks.device)
    for l in range(L):
        u = walks[:, l].long()
        deg = rowptr[u + 1] - rowptr[u]
        M += int((deg > 0).sum())
        sunk |= deg == 0
    return M, int(sunk.sum())


class one_core:
    """Pins this process to one core of its affinity set for the block (the
    single-threaded CPU baseline), restoring the set afterwards."""

    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        self.core = min(self.saved)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)


def cpu_baseline_uniform(np, oracle, rowptr_h, col_h, start, rand, L, target_s=12.0):
    """Single-threaded oracle walk on an evenly strided sample of walks, with
    the edge-id store of RandomWalk.cpp:58 (the reference's loop writes both
    outputs, whichever the op returns)."""
    N = start.shape[0]
    probe = min(N, 20_000)
    idx = np.linspace(0, N - 1, probe).astype(np.int64)
    t0 = time.perf_counter()
    oracle.uniform_walk(rowptr_h, col_h, start[idx], rand[idx], L, with_edges=True)
    rate = probe * L / (time.perf_counter() - t0)
    walks = int(min(N, max(probe, target_s * rate / L)))
    idx = np.linspace(0, N - 1, walks).astype(np.int64)
    s, r = start[idx], rand[idx]
    reps, dt = timed_reps(lambda: oracle.uniform_walk(rowptr_h, col_h, s, r, L, with_edges=True),
                          lambda res: res[2] == 0)
    return reps * walks * L / dt, walks, dt, reps


def runs_text(reps, dt):
    return f"{dt:.1f} s" if reps == 1 else f"{reps} runs of it in {dt:.2f} s"


def timed_reps(call, ok, min_s=0.5, max_reps=100_000):
    """Runs call() once, or, when one run of the whole sample takes under
    min_s (the reference tests' small workloads), repeats it until min_s
    have passed; returns (runs, seconds).  ok(result) must hold."""
    reps, t0 = 0, time.perf_counter()
    while True:
        res = call()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or reps >= max_reps:
            break
    assert ok(res)
    return reps, dt


def host_info():
    """CPU model and the cores this process may use (its affinity set)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model, len(os.sched_getaffinity(0))


def cpu_all_cores_context(np, torch, mc, kind, rowptr_h, col_h, start, rand, L, extra, walks,
                          threads):
    """The library's own host evaluation (stream='cpu', all threads) on the
    same walk sample as the baseline: context for the one-thread baseline."""
    idx = torch.from_numpy(np.linspace(0, start.shape[0] - 1, walks).astype(np.int64))
    rp, cl = torch.from_numpy(rowptr_h), torch.from_numpy(col_h)
    s = torch.from_numpy(start)[idx]
    t0 = time.perf_counter()
    if kind == "uniform":
        mc.random_walk(rp, cl, s, torch.from_numpy(rand)[idx], L, stream="cpu", threads=threads,
                       return_edges=True)
    else:
        mc.rejection_sampling(rp, cl, s, L, extra["p"], extra["q"], seed=extra["seed"],
                              rule=extra["rule"], rows_sorted=True, stream="cpu", threads=threads)
    dt = time.perf_counter() - t0
    return {"value": walks * L / dt, "unit": "walk-steps/s", "threads": threads,
            "seconds": dt,
            "what": "mlx_cluster_amd host twin (stream='cpu'), same sample, on up to `threads` "
                    "threads (small calls use fewer: one per 2^16 uniform or 2^12 node2vec steps)"}


# Table sizes of the random-read ceiling: from tables the L2s and the
# Infinity Cache hold to ones only HBM holds (the walk configurations' random
# footprints lie between 100 MB and 6 GB).
CEILING_MIB = (32, 128, 256, 512, 1024, 2048, 4096, 8192)


def gather_ceiling(torch, dev, variant=None, target_loads=150_000_000):
    """Random-read ceiling of the device (mlxc_gather_probe): for each table
    size, reads at addresses uniform over the table, swept over independent
    and dependent chains (each address depending on the value the chain read
    before, as in a walk), 1 to 8 chains per lane, 2 to 8 blocks of 256 threads
    per compute unit and 16- or 4-byte reads; HIP events over 3 launches after
    a warm-up, median.  Every read of a table beyond the L2s costs one 128-byte
    line between the L2 and the fabric, so reads/s is the line rate a walk
    kernel can reach at most.  variant = (dependent, chains, blocks_per_cu,
    bytes) runs that one variant per size (for counter passes)."""
    import statistics
    from mlx_cluster_amd import _lib
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    table = torch.randint(-2**31, 2**31 - 1, (max(CEILING_MIB) << 18,), dtype=torch.int32,
                          device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    issued = _lib.ctypes.c_int64(0)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    variants = ([variant] if variant else
                [(d, k, b, 16) for d in (0, 1) for k in (1, 2, 4, 8) for b in (2, 4, 8)])

    def run(mib, d, k, b, nbytes):
        iters = max(1, -(-target_loads // (cus * b * 256 * k)))
        args = (table.data_ptr(), mib << 20, nbytes, k, d, b, iters, 12345, sink.data_ptr(),
                _lib.ctypes.addressof(issued), stream.cuda_stream)
        if lib.mlxc_gather_probe(*args) != 0:
            raise RuntimeError(_lib.last_error())
        ms = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            lib.mlxc_gather_probe(*args)
            e1.record(stream)
            e1.synchronize()
            ms.append(e0.elapsed_time(e1))
        t = statistics.median(ms)
        return {"dependent": d, "chains_per_lane": k, "blocks_per_cu": b, "load_bytes": nbytes,
                "reads": issued.value, "ms": t, "reads_per_s": issued.value / (t / 1e3)}

    sizes = []
    for mib in CEILING_MIB:
        runs = [run(mib, *v) for v in variants]
        if variant is None:  # the best independent variant again with 4-byte reads
            best = max((r for r in runs if not r["dependent"]), key=lambda r: r["reads_per_s"])
            runs.append(run(mib, 0, best["chains_per_lane"], best["blocks_per_cu"], 4))
        top = max(runs, key=lambda r: r["reads_per_s"])
        dep = [r for r in runs if r["dependent"]]
        sizes.append({"table_MiB": mib, "lines_per_s": top["reads_per_s"], "best": top,
                      "dependent_lines_per_s": max(r["reads_per_s"] for r in dep) if dep else None,
                      "runs": runs})
        log(f"ceiling {mib} MiB: {top['reads_per_s']:.3e} reads/s "
            f"(dependent={top['dependent']} k={top['chains_per_lane']} "
            f"blocks/CU={top['blocks_per_cu']} {top['load_bytes']} B)")
    from mlx_cluster_amd.build_lib import source_hash
    return {"gather_ceiling": sizes, "kernel_family": "gather_probe",
            "kernel_source_sha256_16": source_hash("gather_probe"),
            "device": torch.cuda.get_device_name(dev), "compute_units": cus}


def line_ceiling(table_bytes):
    """Random-read ceiling (lines/s) at a random footprint of table_bytes,
    interpolated log-linearly in size between the committed measurements
    (profiles/gather_ceiling.json, for the current probe source), clamped to
    the measured range; None without a matching measurement."""
    import math
    from mlx_cluster_amd.build_lib import source_hash
    path = os.path.join(REPO, "profiles", "gather_ceiling.json")
    if not table_bytes or not os.path.exists(path):
        return None
    d = json.load(open(path))
    if d.get("kernel_source_sha256_16") != source_hash("gather_probe"):
        return None
    pts = sorted((s["table_MiB"] * 2**20, s["lines_per_s"]) for s in d["gather_ceiling"])
    if table_bytes <= pts[0][0]:
        return pts[0][1]
    for (b0, r0), (b1, r1) in zip(pts, pts[1:]):
        if table_bytes <= b1:
            f = math.log(table_bytes / b0) / math.log(b1 / b0)
            return r0 + f * (r1 - r0)
    return pts[-1][1]


def random_footprint(mc, kind, V, E, N, L, extra):
    """Bytes of the tables a walk call reads at random addresses, by the layout
    its workspace query selects: the uniform record walk its edge records (8
    or 16 bytes each), the uniform CSR walk col and rowptr; the node2vec walk
    its workspace less the start records (edge records or the CSR mode's row
    starts, the search index, the hub bitmaps).  None for the LDS walks, which
    read no global table at random."""
    lib = mc._lib.load()
    if kind == "uniform":
        ws = lib.mlxc_random_walk_workspace_bytes(V, E, N, L)
        if ws <= 256:
            return None
        rec = 8 if (V - 1).bit_length() + E.bit_length() <= 48 else 16
        return rec * E if ws >= 256 + rec * (E + N) else 8 * E + 8 * (V + 1)
    ws = lib.mlxc_rejection_sampling_workspace_bytes(V, E, N, L, extra["p"], extra["q"],
                                                     RULE_ID[extra["rule"]])
    return None if ws <= 256 else ws - 256 - 16 * N


def walk_kernel_event_ms(torch, mc, stream, step, calls):
    """The walk kernel's own duration in each of `calls` calls, from HIP events
    the library records around it on `stream` (mlxc_set_walk_events)."""
    lib = mc._lib.load()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(calls)]
    for a, b in pairs:  # torch creates an event's HIP handle at its first record
        a.record(stream)
        b.record(stream)
    torch.cuda.synchronize()
    try:
        for a, b in pairs:
            mc._lib.check(lib.mlxc_set_walk_events(a.cuda_event, b.cuda_event),
                          "mlxc_set_walk_events")
            step()
    finally:
        lib.mlxc_set_walk_events(None, None)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in pairs]


def line_roofline(mc, kind, config, V, E, N, L, extra):
    """lines/s of the walk kernel and its fraction of the ceiling at the call's
    random footprint (nulls where a profile or the ceiling is missing)."""
    foot = random_footprint(mc, kind, V, E, N, L, extra)
    ceiling = line_ceiling(foot)
    prof = walk_profile(f"{kind}_walk_{config}")
    rate = prof["walk_kernel_ea_rdreq"] / (prof["walk_kernel_avg_ms"] / 1e3) if prof else None
    return {"random_table_bytes": foot, "line_ceiling_per_s": ceiling,
            "walk_kernel": prof["walk_kernel"] if prof else None,
            "walk_kernel_ms_rocprof": prof["walk_kernel_avg_ms"] if prof else None,
            "walk_kernel_lines_per_launch": prof["walk_kernel_ea_rdreq"] if prof else None,
            "lines_per_s": rate,
            "line_frac": rate / ceiling if rate and ceiling else None,
            "line_frac_source": "TCC_EA0_RDREQ of the walk kernel per dispatch / its rocprofv3 "
                                "average duration, over the random-read ceiling "
                                "(profiles/gather_ceiling.json) at random_table_bytes"}


def walk_profile(name: str):
    """The committed rocprofv3 figures of a walk configuration's main kernel
    (its average duration and TCC_EA0_RDREQ per dispatch), when the summary
    matches the current kernel source; else None."""
    from mlx_cluster_amd.build_lib import KERNEL_SOURCES
    family = next((k for k in KERNEL_SOURCES if name.startswith(k + "_")), None)
    path = os.path.join(REPO, "profiles", f"{name}_traffic.json")
    if family is None or not os.path.exists(path):
        return None
    d = json.load(open(path))
    if (d.get("kernel_family") != family or
            d.get("kernel_source_sha256_16") != kernel_source_hash(family) or
            "walk_kernel_ea_rdreq" not in d):
        return None
    return d


def node2vec_bytes(np, oracle, rowptr_h, col_h, start_h, L, extra, walks=200_000):
    """Roofline bytes of a node2vec call under the measurement contract's
    formula, 64*S_move + 64*T + 64*P + 8*N*(L+1) (a 64-byte line per moving
    step's row read, per trial's candidate read and per col line a lower_bound
    search touches; the output stream at its bytes), with the counts from the
    oracle over an evenly strided sample of walks scaled to N.  Also returns
    the bytes of a wider formula that adds a row line per membership test and
    per sink walk and the start stream, 64*(S+Z) + 64*T + 64*(Q+P) +
    8*N*(L+1) + 8*N."""
    N = start_h.shape[0]
    idx = np.linspace(0, N - 1, min(N, walks)).astype(np.int64)
    _, _, st, c = oracle.node2vec_walk(rowptr_h, col_h, start_h[idx], L, extra["p"], extra["q"],
                                       extra["seed"], rule=RULE_ID[extra["rule"]],
                                       rows_sorted=True)
    f = N / idx.size
    S, Z, T = c["moving_steps"] * f, c["sink_walks"] * f, c["trials"] * f
    Q, P = c["member_tests"] * f, c["member_lines"] * f
    b = LINE * S + LINE * T + LINE * P + 8 * N * (L + 1)
    wide = LINE * (S + Z) + LINE * T + LINE * (Q + P) + 8 * N * (L + 1) + 8 * N
    useful = 16 * (S + Z) + 8 * T + 8 * P + 8 * N * (L + 1) + 8 * N
    return int(b), int(useful), dict(moving_steps=int(S), sink_walks=int(Z), trials=int(T),
                        member_tests=int(Q), member_lines=int(P), counts_sample_walks=int(idx.size),
                        bytes_formula="64*S + 64*T + 64*P + 8*N*(L+1)",
                        wide_bytes_per_launch=int(wide),
                        wide_bytes_formula="64*(S+Z) + 64*T + 64*(Q+P) + 8*N*(L+1) + 8*N")


def cpu_baseline_node2vec(np, oracle, rowptr_h, col_h, start, L, extra, target_s=12.0):
    N = start.shape[0]
    probe = min(N, 2_000)
    idx = np.linspace(0, N - 1, probe).astype(np.int64)
    rule = RULE_ID[extra["rule"]]
    t0 = time.perf_counter()
    oracle.node2vec_walk_libc(rowptr_h, col_h, start[idx], L, extra["p"], extra["q"], 1, rule=rule)
    rate = probe * L / (time.perf_counter() - t0)
    walks = int(min(N, max(probe, target_s * rate / L)))
    idx = np.linspace(0, N - 1, walks).astype(np.int64)
    s = start[idx]
    reps, dt = timed_reps(lambda: oracle.node2vec_walk_libc(rowptr_h, col_h, s, L, extra["p"],
                                                            extra["q"], 1, rule=rule),
                          lambda res: res[1] == 0)
    return reps * walks * L / dt, walks, dt, reps


def bench_csr(args, np, torch, mc, synth, dev):
    """One line for a CSR_CONFIGS entry: mlxc_csr_build on an edge list
    resident in HBM, preallocated outputs and workspace."""
    import oracle
    from mlx_cluster_amd import _lib
    desc, scale, samples, sym = CSR_CONFIGS[args.config]
    log(f"config {args.config}: {desc} on {torch.cuda.get_device_name(dev)}")
    V = 1 << scale
    row, col = synth.rmat_edges(scale, samples, seed=0, device=dev)
    ei = torch.stack([row, col])
    del row, col
    E = ei.shape[1]
    flags = _lib.MLXC_CSR_DEDUP | (_lib.MLXC_CSR_SYMMETRIZE if sym else 0)
    total = 2 * E if sym else E
    lib = _lib.load()
    nbytes = lib.mlxc_csr_build_workspace_bytes(V, E, flags)
    work = torch.empty((nbytes + 7) // 8, dtype=torch.int64, device=dev)
    rowptr = torch.empty(V + 1, dtype=torch.int64, device=dev)
    col_out = torch.empty(total, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    args_c = (ei[0].data_ptr(), ei[1].data_ptr(), E, V, flags, rowptr.data_ptr(),
              col_out.data_ptr(), work.data_ptr(), nbytes, stream.cuda_stream)

    def step():
        rc = lib.mlxc_csr_build(*args_c)
        if rc != 0:
            raise RuntimeError(_lib.last_error())

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    t0 = time.perf_counter()
    for ev0, ev1 in events:
        ev0.record(stream)
        step()
        ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    event_ms = [a.elapsed_time(b) for a, b in events]
    kernel_ms = float(np.mean(event_ms))
    ms_per_step = wall / args.steps * 1e3
    value = E / (ms_per_step / 1e3)
    status, kept = (int(x) for x in work[:2].tolist())
    assert status == 0
    log(f"{ms_per_step:.3f} ms/step wall, {kernel_ms:.3f} ms/launch (events); "
        f"E={E} -> {kept} entries")

    # End to end through to_csr with fresh allocations (it synchronises once).
    del work
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    t0 = time.perf_counter()
    rp2, c2 = mc.to_csr(ei, V, symmetrize=sym, dedup=True)
    torch.cuda.synchronize()
    e2e_ms = (time.perf_counter() - t0) * 1e3
    same = bool(torch.equal(rp2, rowptr) and torch.equal(c2, col_out[:kept]))
    del rp2, c2

    # The sort-based torch path this replaces (torch.unique of row*V+col,
    # bincount, cumsum), timed as context; its result must be ours.
    def torch_path():
        r, c = ei[0], ei[1]
        if sym:
            r, c = torch.cat([r, c]), torch.cat([c, r])
        key = torch.unique(r * V + c, sorted=True)
        rr = key // V
        rp = torch.zeros(V + 1, dtype=torch.int64, device=dev)
        torch.cumsum(torch.bincount(rr, minlength=V), 0, out=rp[1:])
        return rp, key - rr * V
    torch_path()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    trp, tcol = torch_path()
    torch.cuda.synchronize()
    torch_ms = (time.perf_counter() - t0) * 1e3
    full_equal = bool(torch.equal(trp, rowptr) and torch.equal(tcol, col_out[:kept]))
    del trp, tcol

    # Bit-exact parity of a prefix of the list against the oracle.
    S = min(E, 1 << 22)
    r_h, c_h = ei[0, :S].cpu().numpy(), ei[1, :S].cpu().numpy()
    prp, pc = mc.to_csr(ei[:, :S], V, symmetrize=sym, dedup=True)
    orp, oc = oracle.csr_build(r_h, c_h, V, symmetrize=sym, dedup=True)
    parity = bool(np.array_equal(prp.cpu().numpy(), orp) and np.array_equal(pc.cpu().numpy(), oc))
    del prp, pc

    # Bytes: any CSR build reads the two id arrays and writes col and rowptr
    # once.  The radix passes move more; their stream volume is reported too:
    # keys of k bytes (4, 5 or 6 as 32 + 8 or 16 bits, or 8), the first histogram reads
    # the col ids (both ids below 8 col bits), each scatter but the last
    # writes a digit byte per key that the next histogram reads, the finish
    # reads the keys twice (dedup count, emit), and every pass writes, scans
    # and reads 256 digit counts per 8192-key tile.
    algo_bytes = 16 * E + 8 * kept + 8 * (V + 1)
    cbits = (V - 1).bit_length()
    k = 4 if 2 * cbits <= 32 else 5 if 2 * cbits <= 40 else 6 if 2 * cbits <= 48 else 8
    passes = max(1, -(-2 * cbits // 8))
    tiles = -(-total // 8192)
    first_hist = 8 if cbits >= 8 else 16
    pass_bytes = (total * (first_hist + 16 + k + (1 if passes > 1 else 0))
                  + (passes - 1) * total * (1 + 2 * k) + max(passes - 2, 0) * total
                  + total * 2 * k + 8 * kept + 4 * 8 * (V + 1)
                  + passes * 4 * 8 * 256 * tiles)
    achieved = algo_bytes / (kernel_ms / 1e3) / 1e9
    traffic = traffic_from_profile(f"csr_build_{args.config}")
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                "algorithmic_bytes_per_launch": algo_bytes,
                "bytes_formula": "16*E (row, col) + 8*E_out (col) + 8*(V+1) (rowptr)",
                "kernel_ms": kernel_ms, "kernel_ms_median": float(np.median(event_ms)),
                "e2e_ms_with_allocation": e2e_ms,
                "kernel_ms_source": "HIP events around each call on its stream (mean; median beside it)",
                "radix_passes": passes, "key_bytes": k,
                "radix_stream_bytes_per_launch": pass_bytes,
                "radix_stream_gbs": pass_bytes / (kernel_ms / 1e3) / 1e9,
                "fabric_gbs_measured": (traffic / (kernel_ms / 1e3) / 1e9) if traffic else None,
                "traffic_kind": TRAFFIC_KIND}

    cpu = None
    if not args.no_cpu_baseline:
        model, cores = host_info()
        with one_core() as pin:
            n = min(E, 1 << 20)
            t0 = time.perf_counter()
            oracle.csr_build(ei[0, :n].cpu().numpy(), ei[1, :n].cpu().numpy(), V,
                             symmetrize=sym, dedup=True)
            rate = n / (time.perf_counter() - t0)
            n = int(min(E, max(n, args.cpu_seconds * rate)))
            r_h, c_h = ei[0, :n].cpu().numpy(), ei[1, :n].cpu().numpy()
            t0 = time.perf_counter()
            oracle.csr_build(r_h, c_h, V, symmetrize=sym, dedup=True)
            dt = time.perf_counter() - t0
        cpu = {"value": n / dt, "unit": "edges/s", "cores": 1, "kind": "port",
               "sample": f"first {n} of {E} edges, {dt:.1f} s, oracle.csr_build (numpy lexsort, "
                         f"bincount, cumsum: the reference tests' pipeline), 1 thread pinned "
                         f"to one core",
               "host_cpu": model, "host_cores_available": cores, "pinned_core": pin.core}
        log(f"cpu baseline {n / dt:.3e} edges/s over {n} edges")
    line = {
        "metric": CSR_METRIC, "value": value, "unit": "edges/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int64", "data": "synthetic",
        "config": {"workload": f"{args.config}: {desc}", "num_nodes": V, "num_edges_in": E,
                   "entries_sorted": total, "entries_out": kept,
                   "parity_prefix_bit_exact": parity, "prefix_edges": S,
                   "full_size_equals_torch_sort_path": full_equal,
                   "to_csr_equals_abi_call": same},
        "roofline": roofline, "cpu_baseline": cpu,
        "torch_sort_path_ms": torch_ms,
    }
    if cpu:
        line["speedup_vs_cpu_baseline"] = value / cpu["value"]
    print(json.dumps(line), flush=True)


def bench_windows(args, np, torch, mc, synth, dev):
    """One line for a WIN_CONFIGS entry: a step is the positive windows of the
    walks plus as many negative windows (mlxc_context_windows +
    mlxc_negative_windows), walks and starts resident in HBM."""
    import oracle
    desc, scale, samples, per_node, L, C = WIN_CONFIGS[args.config]
    log(f"config {args.config}: {desc} on {torch.cuda.get_device_name(dev)}")
    rowptr, col = synth.rmat_csr(scale, samples, seed=0, device=dev)
    V = rowptr.numel() - 1
    start = torch.arange(per_node * V, device=dev, dtype=torch.int64) % V
    walks = mc.random_walk(rowptr, col, start, None, L, seed=2)
    N = walks.shape[0]
    W = L + 2 - C
    stream = torch.cuda.current_stream(dev)

    def step():
        return mc.context_windows(walks, C), mc.negative_windows(start, L, C, V, seed=7)

    for _ in range(args.warmup):
        out = step()
    del out
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    t0 = time.perf_counter()
    for ev0, ev1 in events:
        ev0.record(stream)
        pos, neg = step()
        ev1.record(stream)
        del pos, neg
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    event_ms = [a.elapsed_time(b) for a, b in events]
    kernel_ms = float(np.mean(event_ms))
    ms_per_step = wall / args.steps * 1e3
    windows = 2 * W * N
    value = windows / (ms_per_step / 1e3)
    log(f"{ms_per_step:.3f} ms/step wall, {kernel_ms:.3f} ms/launch (events)")

    pos, neg = step()
    ref = walks.unfold(1, C, 1).transpose(0, 1).reshape(W * N, C)
    full_equal = bool(torch.equal(pos, ref))
    del ref
    s = torch.arange(0, N, 997, device=dev)
    rw = oracle.negative_walks(start[s].cpu().numpy(), L, V, 7, walk_ids=s.cpu().numpy())
    parity = all(np.array_equal(neg[j * N + s].cpu().numpy(), rw[:, j:j + C]) for j in range(W))
    del pos, neg

    # bytes: the walks read once, the starts once, both window sets written once
    algo_bytes = 8 * N * (L + 1) + 8 * N + 2 * 8 * W * N * C
    achieved = algo_bytes / (kernel_ms / 1e3) / 1e9
    traffic = traffic_from_profile(f"context_windows_{args.config}")
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                "algorithmic_bytes_per_launch": algo_bytes,
                "bytes_formula": "8*N*(L+1) (walks) + 8*N (starts) + 2 * 8*W*N*C (windows)",
                "kernel_ms": kernel_ms, "kernel_ms_median": float(np.median(event_ms)),
                "kernel_ms_source": "HIP events around each step on its stream (mean; median beside it)",
                "fabric_gbs_measured": (traffic / (kernel_ms / 1e3) / 1e9) if traffic else None,
                "traffic_kind": TRAFFIC_KIND}
    cpu = None
    if not args.no_cpu_baseline:
        model, cores = host_info()
        w_h, s_h = walks.cpu().numpy(), start.cpu().numpy()
        with one_core() as pin:
            n = min(N, 20_000)
            t0 = time.perf_counter()
            oracle.context_windows(w_h[:n], C)
            oracle.negative_windows(s_h[:n], L, C, V, 7)
            rate = 2 * W * n / (time.perf_counter() - t0)
            n = int(min(N, max(n, args.cpu_seconds * rate / (2 * W))))
            t0 = time.perf_counter()
            oracle.context_windows(w_h[:n], C)
            oracle.negative_windows(s_h[:n], L, C, V, 7)
            dt = time.perf_counter() - t0
        cpu = {"value": 2 * W * n / dt, "unit": "windows/s", "cores": 1, "kind": "port",
               "sample": f"first {n} of {N} walks, {dt:.1f} s, oracle.context_windows + "
                         f"oracle.negative_windows (numpy), 1 thread pinned to one core",
               "host_cpu": model, "host_cores_available": cores, "pinned_core": pin.core}
        log(f"cpu baseline {cpu['value']:.3e} windows/s over {n} walks")
    line = {
        "metric": WIN_METRIC, "value": value, "unit": "windows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int64", "data": "synthetic",
        "config": {"workload": f"{args.config}: {desc}", "num_nodes": V, "num_walks": N,
                   "walk_length": L, "context_size": C, "windows_per_step": windows,
                   "positive_equals_torch_unfold": full_equal,
                   "negative_sample_bit_exact": bool(parity)},
        "roofline": roofline, "cpu_baseline": cpu,
    }
    if cpu:
        line["speedup_vs_cpu_baseline"] = value / cpu["value"]
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2",
                    choices=sorted(CONFIGS) + sorted(CSR_CONFIGS) + sorted(WIN_CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device-to-device copy (rocprof counter scale)")
    ap.add_argument("--gather-ceiling", action="store_true",
                    help="measure the random-read ceiling over tables of 32 MiB to 8 GiB")
    ap.add_argument("--gather-variant", default=None,
                    help="with --gather-ceiling: one variant 'dependent,chains,blocks_per_cu,"
                         "bytes' per size instead of the sweep")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the walks need no cross-GPU exchange, so k GPUs would "
              "each take N/k of the walks over a replicated CSR, and this build runs on a single "
              "MI355X. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import mlx_cluster_amd as mc
    from mlx_cluster_amd import synth

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        # A plain copy of known size: 1 GiB read + 1 GiB written per launch.
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_each_way": src.numel() * 4,
                          "launches": args.warmup + args.steps}), flush=True)
        return

    if args.gather_ceiling:
        v = tuple(int(x) for x in args.gather_variant.split(",")) if args.gather_variant else None
        print(json.dumps(gather_ceiling(torch, dev, v)), flush=True)
        return

    if args.config in CSR_CONFIGS:
        bench_csr(args, np, torch, mc, synth, dev)
        return
    if args.config in WIN_CONFIGS:
        bench_windows(args, np, torch, mc, synth, dev)
        return

    desc, kind, gargs, per_node, L, extra = CONFIGS[args.config]
    log(f"config {args.config}: {desc} on {torch.cuda.get_device_name(dev)}")
    if "cora" in gargs:
        rowptr, col = (torch.from_numpy(a).to(dev) for a in synth.cora_like(seed=0))
    elif "ba" in gargs:
        nodes, m, hubs, hub_degree = gargs["ba"]
        rowptr, col = synth.ba_hub_csr(nodes, m, hubs, hub_degree, seed=0, device=dev)
    else:
        rowptr, col = synth.rmat_csr(gargs["scale"], gargs["samples"], seed=0, device=dev,
                                     symmetrize=gargs["symmetrize"])
    V = rowptr.numel() - 1
    E = col.numel()
    N = extra.get("num_walks", per_node * V)
    start = torch.arange(N, device=dev, dtype=torch.int64) % V
    torch.cuda.synchronize()
    log(f"graph V={V} E={E}; walks N={N} L={L}")

    seeded = kind == "uniform_seeded"
    if seeded:
        # the walks of c2 without the rand tensor; rand is materialised only
        # for the parity sample and the CPU baseline, after timing
        kind = "uniform"
        rand = None
        step = lambda: mc.random_walk(rowptr, col, start, None, L, seed=2)
    elif kind == "uniform":
        rand = mc.philox_uniform((N, L), 2, device=dev)
        out_dtype = getattr(torch, extra.get("out_dtype", "int64"))
        step = lambda: mc.random_walk(rowptr, col, start, rand, L, out_dtype=out_dtype)
    else:
        rand = None
        step = lambda: mc.rejection_sampling(rowptr, col, start, L, extra["p"], extra["q"],
                                             seed=extra["seed"], rule=extra["rule"],
                                             symmetric=extra.get("symmetric", False))

    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)  # the walk kernels launch on this stream
    # Wall time of K calls back to back, with nothing else between them; then
    # K more calls bracketed by HIP events for the per-call GPU time (the
    # event records would otherwise add to the wall time of short calls).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    for ev0, ev1 in events:
        ev0.record(stream)
        out = step()
        ev1.record(stream)
    torch.cuda.synchronize()
    event_ms = [a.elapsed_time(b) for a, b in events]
    kernel_ms = float(np.mean(event_ms))
    kernel_ms_median = float(np.median(event_ms))
    walk_ms = walk_kernel_event_ms(torch, mc, stream, step, args.steps)
    ms_per_step = wall / args.steps * 1e3
    steps_per_launch = N * L
    value = steps_per_launch / (ms_per_step / 1e3)
    log(f"{ms_per_step:.3f} ms/step wall, {kernel_ms:.3f} ms/launch (events), "
        f"walk kernel {float(np.mean(walk_ms)):.3f} ms (events)")

    # One end-to-end call with allocation: the caching allocator is emptied
    # first, so the output and workspace come from fresh device allocations.
    del out
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    t0 = time.perf_counter()
    out = step()
    torch.cuda.synchronize()
    e2e_alloc_ms = (time.perf_counter() - t0) * 1e3
    log(f"{e2e_alloc_ms:.3f} ms end to end with fresh allocations")

    import oracle
    rowptr_h, col_h = rowptr.cpu().numpy(), col.cpu().numpy()
    g = torch.Generator().manual_seed(1)
    sample = torch.randint(0, N, (2000,), generator=g).to(dev)

    # Algorithmic bytes of one launch: one 64-B line per dependent random
    # read of the reference loop (rowptr pair and col, RandomWalk.cpp:45-54),
    # streams at their byte count.  M = steps from a node with deg > 0,
    # Z = walks that meet a deg-0 node (one rowptr read to find it).
    if kind == "uniform":
        M, Z = uniform_counts(torch, rowptr, out)
        rand_bytes = 0 if seeded else 4 * M  # generated uniforms are not read
        ob = out.element_size()  # output bytes per entry: 8, or 4 with int32 output
        roof_bytes = LINE * (M + Z) + LINE * M + rand_bytes + ob * N * (L + 1) + 8 * N
        useful_bytes = 16 * (M + Z) + 8 * M + rand_bytes + ob * N * (L + 1) + 8 * N
        units = dict(moving_steps=M, sink_walks=Z,
                     bytes_formula=(f"64*(M+Z) + 64*M + {'4*M + ' if not seeded else ''}"
                                    f"{ob}*N*(L+1) + 8*N"))
    else:
        # node2vec: the work depends on rejections, so it is counted by the
        # oracle on an evenly strided sample of walks and scaled to N.
        roof_bytes, useful_bytes, units = node2vec_bytes(np, oracle, rowptr_h, col_h, start.cpu().numpy(), L,
                                           extra)
    achieved = roof_bytes / (kernel_ms / 1e3) / 1e9 if roof_bytes else None
    traffic = traffic_from_profile(f"{kind}_walk_{args.config}")
    if "wide_bytes_per_launch" in units:
        units["frac_wide_formula"] = units["wide_bytes_per_launch"] / (kernel_ms / 1e3) / 1e9 / \
            PEAK_HBM_GBS
    # The walk kernel's own line rate (TCC_EA0_RDREQ per dispatch over its
    # average duration, from the committed profile of this source) against the
    # random-read ceiling at the call's random footprint.
    lines = line_roofline(mc, kind, args.config, V, E, N, L, extra)
    # the call's whole L2-to-fabric traffic (reads and writes of all its
    # kernels) against the ceiling's line traffic (128 bytes a line)
    lines["fabric_frac"] = (traffic / (kernel_ms / 1e3) / (lines["line_ceiling_per_s"] * 128)
                            if traffic and lines["line_ceiling_per_s"] else None)
    walk_kernel_ms = float(np.mean(walk_ms))
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": (achieved / PEAK_HBM_GBS) if achieved else None, "traffic": traffic,
                **lines,
                "algorithmic_bytes_per_launch": roof_bytes,
                "kernel_ms": kernel_ms, "kernel_ms_median": kernel_ms_median,
                "e2e_ms_with_allocation": e2e_alloc_ms,
                "kernel_ms_source": "HIP events around each call on its stream (mean; median beside it)",
                "walk_kernel_ms": walk_kernel_ms,
                "walk_kernel_ms_median": float(np.median(walk_ms)),
                "walk_kernel_ms_source": "HIP events the library records on the call's stream right "
                                         "before and after its walk kernel (mlxc_set_walk_events), "
                                         "mean over as many calls as timed (median beside it)",
                "frac_walk_kernel": (roof_bytes / (walk_kernel_ms / 1e3) / 1e9 / PEAK_HBM_GBS
                                     if roof_bytes else None),
                "useful_gbs": useful_bytes / (kernel_ms / 1e3) / 1e9,
                "useful_bytes_per_launch": useful_bytes,
                "fabric_gbs_measured": (traffic / (kernel_ms / 1e3) / 1e9) if traffic else None,
                "traffic_kind": TRAFFIC_KIND,
                **units}

    # Sampled bit-exact parity against the oracle, and the CPU baseline.
    if kind == "uniform" and rand is None:
        rand = mc.philox_uniform((N, L), 2, device=dev)
    if kind == "uniform":
        ref, _, st, _ = oracle.uniform_walk(rowptr_h, col_h, start[sample].cpu().numpy(),
                                            rand[sample].cpu().numpy(), L)
        got = out[sample].cpu().numpy()
    else:
        # walk ids index the Philox stream: check a contiguous block of
        # walks [s0, s0 + 2000) with the oracle told its first walk id
        s0 = int(sample[0].item()) % max(1, N - 2000)
        ref, _, st, _ = oracle.node2vec_walk(rowptr_h, col_h, start[s0:s0 + 2000].cpu().numpy(),
                                             L, extra["p"], extra["q"], extra["seed"],
                                             rule=RULE_ID[extra["rule"]], rows_sorted=True,
                                             first_walk=s0)
        got = out[s0:s0 + 2000].cpu().numpy()
    parity = bool(st == 0 and np.array_equal(got, ref))
    cpu = None
    model, cores = host_info()
    if not args.no_cpu_baseline and kind == "uniform":
        rand_h = rand.cpu().numpy()
        with one_core() as pin:
            rate, walks, dt, reps = cpu_baseline_uniform(np, oracle, rowptr_h, col_h,
                                                         start.cpu().numpy(), rand_h, L,
                                                         args.cpu_seconds)
        cpu = {"value": rate, "unit": "walk-steps/s", "cores": 1, "kind": "port",
               "sample": f"{walks} of {N} walks (evenly strided) x {L} steps, "
                         f"{runs_text(reps, dt)}, "
                         f"oracle/walk_oracle.c uniform walk writing nodes and edge ids "
                         f"(RandomWalk.cpp:57-58), 1 thread pinned to one core",
               "sample_fraction": walks / N}
        log(f"cpu baseline {rate:.3e} steps/s over {walks} walks")
    elif not args.no_cpu_baseline:
        with one_core() as pin:
            rate, walks, dt, reps = cpu_baseline_node2vec(np, oracle, rowptr_h, col_h,
                                                          start.cpu().numpy(), L, extra,
                                                          args.cpu_seconds)
        cpu = {"value": rate, "unit": "walk-steps/s", "cores": 1, "kind": "port",
               "sample": f"{walks} of {N} walks (evenly strided) x {L} steps, "
                         f"{runs_text(reps, dt)}, "
                         f"oracle/walk_oracle.c node2vec walk with libc rand() and linear "
                         f"is_neighbor scans as in the reference, 1 thread pinned to one core",
               "sample_fraction": walks / N}
        rand_h = None
        log(f"cpu baseline {rate:.3e} steps/s over {walks} walks")

    if cpu:
        cpu["host_cpu"] = model
        cpu["host_cores_available"] = cores
        cpu["pinned_core"] = pin.core
        threads = min(cores, 16)  # the GPU box's CPU share
        ctx = cpu_all_cores_context(np, torch, mc, kind, rowptr_h, col_h, start.cpu().numpy(),
                                    rand_h, L, extra, walks, threads)
        log(f"cpu all-cores context {ctx['value']:.3e} steps/s on {threads} threads")
    line = {
        "metric": METRIC, "value": value, "unit": "walk-steps/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int32" if out.dtype == torch.int32 else "int64",
        "data": "synthetic",
        "config": {"workload": f"{args.config}: {desc}", "num_nodes": V, "num_edges": E,
                   "num_walks": N, "walk_length": L, "walk_steps_per_launch": steps_per_launch,
                   "parity_sample_bit_exact": parity},
        "roofline": roofline, "cpu_baseline": cpu,
        # steps that leave a node of out-degree > 0, per second of wall time
        # (the rest are the stationary steps of walks absorbed by a sink)
        "moving_steps_per_s": units["moving_steps"] / (ms_per_step / 1e3),
    }
    if cpu:
        line["speedup_vs_cpu_baseline"] = value / cpu["value"]
        line["cpu_all_cores_context"] = ctx
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
