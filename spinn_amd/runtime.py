"""Python handle over the native host runtime (spinn_load / spinn_plan / spinn_run).

    with Session("model.ennf") as s:
        y = s.run(x)              # host in, host out (H2D + nodes + D2H + sync)
        s.upload_input(x)         # stage the input in HBM once ...
        s.run_resident()          # ... then each step copies it into the arena (device to
                                  # device) and runs the node loop, outputs left in HBM
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import native as N


class Session:
    def __init__(self, path, policy: int = N.POLICY_AUTO, graph: bool = False, max_arena: int = 0,
                 plan: bool = True):
        self.L = N.lib()
        self.path = os.fspath(path)
        self.ctx = self.L.spinn_load(self.path.encode())
        if not self.ctx:
            raise RuntimeError(f"spinn_load failed for {self.path}")
        if policy != N.POLICY_AUTO:
            N.check(self.L.spinn_set_conv_policy(self.ctx, policy), "spinn_set_conv_policy")
        self.planned = False
        if plan:
            rc = self.L.spinn_plan(self.ctx, max_arena)
            if rc != 0:
                self.close()
                raise RuntimeError(f"spinn_plan failed: {rc}")
            self.planned = True
            if graph:
                self.L.spinn_set_graph_mode(self.ctx, 1)

    # ---- model metadata ----
    @property
    def c(self) -> N.SpinnContext:
        return self.ctx.contents

    def tensor(self, tid: int) -> N.SpinnTensor:
        return self.c.tensors[tid]

    def dims(self, tid: int) -> tuple:
        t = self.tensor(tid)
        return tuple(t.dims[i] for i in range(t.ndim))

    @property
    def input_id(self) -> int:
        return self.c.input_ids[0]

    @property
    def output_id(self) -> int:
        return self.c.output_ids[0]

    def offsets(self) -> dict:
        """Arena offsets of every activation tensor with data (planner output)."""
        out = {}
        for i in range(self.c.num_tensors):
            t = self.c.tensors[i]
            if not t.is_weight and t.size > 0:
                out[i] = t.offset
        return out

    # ---- execution ----
    def run(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(self.dims(self.output_id), np.float32)
        rc = self.L.spinn_run(self.ctx, x.ctypes.data, y.ctypes.data)
        if rc != 0:
            raise N.SpinnError(rc, f"spinn_run (node {self.c.last_error_node})")
        return y

    def upload_input(self, x: np.ndarray) -> None:
        """Stage input 0 in the context's device staging buffer; every later
        run_resident() restores the arena's input region from it."""
        x = np.ascontiguousarray(x, np.float32)
        N.check(self.L.spinn_stage_input(self.ctx, x.ctypes.data, x.nbytes), "spinn_stage_input")

    _NP = {1: np.float32, 6: np.int32, 7: np.int64}

    def download(self, tid: int) -> np.ndarray:
        y = np.empty(self.dims(tid), self._NP.get(self.tensor(tid).dtype, np.float32))
        N.check(self.L.spinn_tensor_download(self.ctx, tid, y.ctypes.data, y.nbytes), "download")
        return y

    def run_resident(self) -> None:
        rc = self.L.spinn_run_resident(self.ctx)
        if rc != 0:
            raise N.SpinnError(rc, f"spinn_run_resident (node {self.c.last_error_node})")

    def node_times(self) -> np.ndarray:
        n = self.c.num_nodes
        buf = (C.c_float * n)()
        got = self.L.spinn_node_times(self.ctx, buf, n)
        return np.array(buf[:got], np.float64)

    def close(self) -> None:
        if getattr(self, "ctx", None):
            self.L.spinn_free(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
