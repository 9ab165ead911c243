"""CPU baseline timing: the reference's generated-C backend on this host's cores.

TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg). The timed code is the reference's own
C kernels (mgc_kernels.c) driven by oracle/cbackend.py's restatement of its emitter, prebuilt
per workload and batch in oracle/_ref.

Method of the reference's latency benchmark (benchmarks/latency.py:105-191): every cell
(workload, batch, threads) runs in a fresh process with OMP_NUM_THREADS set, does its warmup
runs and then times ``repeat`` runs; the cells are interleaved over ``rounds`` rounds; a cell's
figure is the median of all its samples with a 2000-sample bootstrap 95% confidence interval.
The host is described by nproc and lscpu's model name.

    python -m oracle.cpu_bench --worker WORKLOAD BATCH THREADS --warmup W --repeat R
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def bootstrap_median_ci(samples: np.ndarray, n: int = 2000, seed: int = 0) -> tuple[float, float]:
    rng = np.random.default_rng(seed)
    medians = np.median(rng.choice(samples, (n, samples.size), replace=True), axis=1)
    return float(np.percentile(medians, 2.5)), float(np.percentile(medians, 97.5))


def host() -> dict:
    """nproc and the CPU model as lscpu reports it: the model name plus family / model /
    stepping, sockets and threads per core (a virtualized host may name only the vendor line)."""
    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, check=False).stdout
        for line in out.splitlines():
            key, _, value = line.partition(":")
            fields[key.strip()] = value.strip()
    except OSError:
        pass
    model = fields.get("Model name", "unknown")
    detail = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping", "Socket(s)",
                                                   "Core(s) per socket", "Thread(s) per core") if fields.get(k)]
    if detail:
        model += " (" + ", ".join(detail) + ")"
    try:
        nproc = int(subprocess.run(["nproc"], capture_output=True, text=True, check=False).stdout.strip())
    except (OSError, ValueError):
        nproc = os.cpu_count() or 1
    return {"nproc": nproc, "cpu_model": model}


def worker(workload: str, batch: int, threads: int, warmup: int, repeat: int) -> dict:
    from oracle import cbackend
    from oracle.interpreter import random_feeds

    model, graph, meta = cbackend.load_baseline(workload, batch)
    model.lib.mgc_set_num_threads(int(threads))
    feeds = random_feeds(graph, 0, int_high=30522 if workload in ("bert_base", "gpt2") else 100)
    for _ in range(warmup):
        model.run(feeds)
    times = []
    for _ in range(repeat):
        t0 = time.perf_counter()
        model.run(feeds)
        times.append(time.perf_counter() - t0)
    return {"workload": workload, "batch": batch, "threads": threads, "samples_ms": [1e3 * t for t in times]}


def run_cell(workload: str, batch: int, threads: int, warmup: int, repeat: int, timeout: float = 300) -> dict:
    """One cell in a fresh process (OMP_NUM_THREADS = threads)."""
    cmd = [sys.executable, "-m", "oracle.cpu_bench", "--worker", workload, str(batch), str(threads),
           "--warmup", str(warmup), "--repeat", str(repeat)]
    env = {**os.environ, "OMP_NUM_THREADS": str(threads)}
    out = subprocess.run(cmd, capture_output=True, text=True, env=env, cwd=ROOT, timeout=timeout, check=False)
    if out.returncode != 0:
        raise RuntimeError(f"cpu cell {workload} b{batch} t{threads} failed: {out.stderr[-1500:]}")
    return json.loads(out.stdout.strip().splitlines()[-1])


def measure(cells: list[tuple[str, int, int, int, int]], rounds: int = 3) -> list[dict]:
    """cells: (workload, batch, threads, warmup, repeat); rounds interleave the cells."""
    samples: dict[tuple[str, int, int], list[float]] = {}
    for _ in range(rounds):
        for workload, batch, threads, warmup, repeat in cells:
            got = run_cell(workload, batch, threads, warmup, repeat)
            samples.setdefault((workload, batch, threads), []).extend(got["samples_ms"])
    rows = []
    for (workload, batch, threads), ms in samples.items():
        arr = np.asarray(ms)
        lo, hi = bootstrap_median_ci(arr)
        rows.append({"workload": workload, "batch": batch, "threads": threads, "samples": int(arr.size),
                     "median_ms": float(np.median(arr)), "median_ci95_ms": [lo, hi]})
    return rows


def main() -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--worker", nargs=3, metavar=("WORKLOAD", "BATCH", "THREADS"))
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--repeat", type=int, default=30)
    args = p.parse_args()
    if args.worker:
        workload, batch, threads = args.worker
        print(json.dumps(worker(workload, int(batch), int(threads), args.warmup, args.repeat)))


if __name__ == "__main__":
    main()
