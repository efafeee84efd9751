"""Load the MIRA golden fixtures (tests/golden/mira_w8a8_*.npz, written by
tests/golden/make_mira_fixtures.py from MIRA's own compiler) into harness graphs."""
from __future__ import annotations

import json
import os

import numpy as np

from harness.graph import Graph, TensorType

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = [f"{p}_{prec}" for p in ("mlp", "cnn") for prec in ("f32", "f16")]


class Fixture:
    def __init__(self, case: str):
        self.case = case
        self.z = np.load(os.path.join(HERE, "golden", f"mira_w8a8_{case}.npz"))
        self.doc = json.loads(str(self.z["graph"]))
        self.graph, self.values = self._build(self.doc)
        self.feeds = {v.name: self.z[f"feed:{v.name}"] for v in self.graph.inputs}

    def _attr(self, a):
        if isinstance(a, dict):
            if "array" in a:
                v = self.z[a["array"]]
                return v if v.ndim else v[()]
            if "tuple" in a:
                return tuple(self._attr(x) for x in a["tuple"])
            if "float" in a:
                return float(a["float"])
        if isinstance(a, list):
            return [self._attr(x) for x in a]
        return a

    def _build(self, doc: dict):
        g = Graph(self.case)
        by_id = {}
        for d in doc["inputs"]:
            by_id[d["id"]] = g.input(d["name"], d["shape"], d["dtype"])
        values = {}
        for d in doc["ops"]:
            r = d["result"]
            attrs = {k: self._attr(v) for k, v in d["attrs"].items()}
            v = g.emit(d["kind"], [by_id[i] for i in d["inputs"]], attrs, TensorType(r["dtype"], r["shape"]))
            by_id[r["id"]] = v
            key = f"value:{r['id']}"
            if key in self.z.files:
                values[v] = self.z[key]
        g.outputs = [by_id[i] for i in doc["outputs"]]
        g.check()
        return g, values

    def float_graph(self, which: str) -> dict:
        """MIRA's f32 float graph ("elaborated" or "optimized") as recorded: ops with kinds,
        input ids, attrs, and constants as {sha256, shape, dtype}."""
        return self.doc["float_graphs"][which]
