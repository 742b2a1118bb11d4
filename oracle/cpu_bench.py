"""ORACLE (test infrastructure only): time a CPU run of an ENNF model.

    python -m oracle.cpu_bench --kind reference|port --model m.ennf --batch B --seconds 10

kind=reference runs the reference's own runtime (oracle/_ref/libspinn_ref.so,
built from the reference sources by oracle/Makefile); kind=port runs the
restatement (oracle/liboracle.so). The protocol is the reference CLI's
(SPINN/run_time/main.c:42,83-108): 3 warm-up runs, then timed runs until the
time budget is spent; best and mean wall time per run include the input and
output copies. Thread count comes from OMP_NUM_THREADS, which the caller
sets in this process's environment before the libraries load. Prints one
JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _ref_runner(model: str, in_elems: int, out_elems: int):
    L = C.CDLL(str(HERE / "_ref" / "libspinn_ref.so"))
    L.spinn_load.restype = C.c_void_p
    L.spinn_load.argtypes = [C.c_char_p]
    L.spinn_plan.argtypes = [C.c_void_p, C.c_uint32]
    L.spinn_run.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
    L.spinn_free.argtypes = [C.c_void_p]
    ctx = L.spinn_load(model.encode())
    if not ctx or L.spinn_plan(ctx, 0) != 0:
        raise RuntimeError("reference runtime could not load/plan the model")
    x = np.random.default_rng(0).uniform(-1, 1, in_elems).astype(np.float32)
    y = np.empty(out_elems, np.float32)

    def run():
        L.spinn_run(ctx, x.ctypes.data, y.ctypes.data)

    return run, lambda: L.spinn_free(ctx)


def _port_runner(model: str, in_shape, out_shape):
    from oracle import oracle as O
    m = O.Model(model)
    x = np.random.default_rng(0).uniform(-1, 1, in_shape).astype(np.float32)

    def run():
        m.run(x, out_shape)

    return run, m.close


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--kind", choices=["reference", "port"], required=True)
    ap.add_argument("--model", required=True)
    ap.add_argument("--in-shape", required=True)
    ap.add_argument("--out-shape", required=True)
    ap.add_argument("--seconds", type=float, default=10.0)
    ap.add_argument("--max-runs", type=int, default=1000)
    a = ap.parse_args()
    in_shape = tuple(int(v) for v in a.in_shape.split(","))
    out_shape = tuple(int(v) for v in a.out_shape.split(","))
    if a.kind == "reference":
        run, close = _ref_runner(a.model, int(np.prod(in_shape)), int(np.prod(out_shape)))
    else:
        run, close = _port_runner(a.model, in_shape, out_shape)
    for _ in range(3):
        run()
    times = []
    t_end = time.perf_counter() + a.seconds
    while len(times) < a.max_runs and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    close()
    print(json.dumps({"kind": a.kind, "runs": len(times), "best_ms": 1e3 * min(times),
                      "avg_ms": 1e3 * float(np.mean(times)), "batch": in_shape[0],
                      "threads": int(os.environ.get("OMP_NUM_THREADS", "0") or 0)}))


if __name__ == "__main__":
    main()
