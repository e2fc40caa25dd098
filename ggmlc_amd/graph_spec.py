"""ggmlc's serialized execution graph (`ggmlc.graph_spec`, a JSON string in the GGUF
metadata) and its symbolic dimensions.

The JSON holds (`python/ggmlc/serialization/gguf.py:130-177` writes it,
`runtime/src/loader.cpp:218-445` reads it):

    {"name", "inputs": [tid], "outputs": [tid], "parameters": [tid],
     "symbol_table": [name], "metadata": {...},
     "tensors": {"<tid>": {"id", "name", "type", "ne": [dim x4], "storage",
                           "producer_id", "role"}},
     "nodes": [{"id", "opcode", "inputs": [tid], "outputs": [tid],
                "attributes": {...}, "name"}]}

A dim is {"type": "static", "val"} | {"type": "symbol", "name"} | {"type": op,
"left", "right"} with op in add, sub, mul, floordiv, ceildiv, evaluated in int64
like the runtime's DimExpr (`runtime/include/ggmlc/types.h:24-75`): division
truncates toward zero and ceildiv is (l + r - 1) / r. Opcodes are ggml's
`enum ggml_op` values (ggml 0.20.2); attribute values are read both as int64
(truncated) and as double, as the runtime does.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from typing import Any

# storage classes (types.h:77-84)
INPUT, PARAMETER, CONSTANT, ACTIVATION, STATE, OUTPUT = range(6)

# ggml 0.20.2 enum ggml_op, in order (third_party/ggml/include/ggml.h): the opcode of a
# graph node is the index of its name here
_OP_ORDER = [
    "NONE", "DUP", "ADD", "ADD_ID", "ADD1", "ACC", "SUB", "MUL", "DIV", "SQR", "SQRT", "LOG",
    "SIN", "COS", "SUM", "SUM_ROWS", "CUMSUM", "MEAN", "ARGMAX", "COUNT_EQUAL", "REPEAT",
    "REPEAT_BACK", "CONCAT", "SILU_BACK", "NORM", "RMS_NORM", "RMS_NORM_BACK", "GROUP_NORM",
    "L2_NORM", "MUL_MAT", "MUL_MAT_ID", "OUT_PROD", "SCALE", "SET", "CPY", "CONT", "RESHAPE",
    "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS", "GET_ROWS_BACK", "SET_ROWS", "DIAG",
    "DIAG_MASK_INF", "DIAG_MASK_ZERO", "SOFT_MAX", "SOFT_MAX_BACK", "ROPE", "ROPE_BACK", "CLAMP",
    "CONV_TRANSPOSE_1D", "IM2COL", "IM2COL_BACK", "IM2COL_3D", "COL2IM_1D", "CONV_2D", "CONV_3D",
    "CONV_2D_DW", "CONV_TRANSPOSE_2D", "POOL_1D", "POOL_2D", "POOL_2D_BACK", "UPSCALE", "PAD",
    "PAD_REFLECT_1D", "ROLL", "ARANGE", "TIMESTEP_EMBEDDING", "ARGSORT", "TOP_K", "LEAKY_RELU",
    "TRI", "FILL", "FLASH_ATTN_EXT", "FLASH_ATTN_BACK", "SSM_CONV", "SSM_SCAN", "WIN_PART",
    "WIN_UNPART", "GET_REL_POS", "ADD_REL_POS", "RWKV_WKV6", "GATED_LINEAR_ATTN", "RWKV_WKV7",
    "SOLVE_TRI", "GATED_DELTA_NET", "LIGHTNING_INDEXER", "DSV4_HC_COMB", "DSV4_HC_PRE",
    "DSV4_HC_POST", "UNARY", "MAP_CUSTOM1", "MAP_CUSTOM2", "MAP_CUSTOM3", "CUSTOM",
    "CROSS_ENTROPY_LOSS", "CROSS_ENTROPY_LOSS_BACK", "OPT_STEP_ADAMW", "OPT_STEP_SGD", "GLU",
]
OPS = {n: i for i, n in enumerate(_OP_ORDER)}
OP_NAMES = {v: k for k, v in OPS.items()}


def _tdiv(a: int, b: int) -> int:
    """int64 division truncating toward zero (C++ `/`)."""
    if b == 0:
        raise ZeroDivisionError("Division by zero in DimExpr")
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


@dataclass(frozen=True)
class Dim:
    """A symbolic dimension: kind in static | symbol | add | sub | mul | floordiv | ceildiv."""
    kind: str
    val: int = 1
    name: str = ""
    left: "Dim | None" = None
    right: "Dim | None" = None

    @staticmethod
    def static(v: int) -> "Dim":
        return Dim("static", int(v))

    @staticmethod
    def symbol(name: str) -> "Dim":
        return Dim("symbol", 0, name)

    def _bin(self, kind: str, other) -> "Dim":
        return Dim(kind, 0, "", self, other if isinstance(other, Dim) else Dim.static(other))

    def __add__(self, o):
        return self._bin("add", o)

    def __sub__(self, o):
        return self._bin("sub", o)

    def __mul__(self, o):
        return self._bin("mul", o)

    def __floordiv__(self, o):
        return self._bin("floordiv", o)

    def ceildiv(self, o) -> "Dim":
        return self._bin("ceildiv", o)

    def evaluate(self, env: dict[str, int]) -> int:
        k = self.kind
        if k == "static":
            return self.val
        if k == "symbol":
            if self.name not in env:
                raise KeyError(f"Symbol not found in environment: {self.name}")
            return int(env[self.name])
        a = self.left.evaluate(env)
        b = self.right.evaluate(env)
        if k == "add":
            return a + b
        if k == "sub":
            return a - b
        if k == "mul":
            return a * b
        if k == "floordiv":
            return _tdiv(a, b)
        if k == "ceildiv":
            return _tdiv(a + b - 1, b)
        return 1

    def free_symbols(self) -> set[str]:
        if self.kind == "symbol":
            return {self.name}
        if self.kind == "static":
            return set()
        return self.left.free_symbols() | self.right.free_symbols()

    def to_json(self) -> dict:
        if self.kind == "static":
            return {"type": "static", "val": self.val}
        if self.kind == "symbol":
            return {"type": "symbol", "name": self.name}
        return {"type": self.kind, "left": self.left.to_json(), "right": self.right.to_json()}

    @staticmethod
    def from_json(d: dict) -> "Dim":
        # unknown types read as static 1, like the runtime's parse_dim_expr (loader.cpp:218-250)
        t = d.get("type", "static")
        if t == "static":
            return Dim.static(int(d.get("val", 1)))
        if t == "symbol":
            return Dim.symbol(str(d.get("name", "")))
        if t in ("add", "sub", "mul", "floordiv", "ceildiv"):
            return Dim(t, 0, "", Dim.from_json(d["left"]), Dim.from_json(d["right"]))
        return Dim.static(1)


def _dim(x) -> Dim:
    return x if isinstance(x, Dim) else Dim.static(int(x))


@dataclass
class Tensor:
    id: int
    name: str
    type: int                   # ggml_type
    ne: tuple[Dim, Dim, Dim, Dim]
    storage: int = ACTIVATION
    producer_id: int | None = None
    role: str | None = None

    def shape(self, env: dict[str, int]) -> list[int]:
        return [d.evaluate(env) for d in self.ne]


@dataclass
class Node:
    id: int
    opcode: int
    inputs: list[int]
    outputs: list[int]
    attributes: dict[str, Any] = field(default_factory=dict)
    name: str = ""

    @property
    def op(self) -> str:
        return OP_NAMES.get(self.opcode, f"OP_{self.opcode}")

    def attr_int(self, key: str, default: int = 0) -> int:
        """The attribute as the runtime's int view: numbers truncated, bools 0/1,
        anything else the default."""
        v = self.attributes.get(key)
        if isinstance(v, bool):
            return int(v)
        if isinstance(v, (int, float)):
            return int(v)
        return default

    def attr_float(self, key: str, default: float = 0.0) -> float:
        v = self.attributes.get(key)
        if isinstance(v, bool):
            return float(v)
        if isinstance(v, (int, float)):
            return float(v)
        return default

    def has(self, key: str) -> bool:
        return key in self.attributes


@dataclass
class Graph:
    name: str = "main"
    inputs: list[int] = field(default_factory=list)
    outputs: list[int] = field(default_factory=list)
    parameters: list[int] = field(default_factory=list)
    symbol_table: list[str] = field(default_factory=list)
    metadata: dict[str, Any] = field(default_factory=dict)
    tensors: dict[int, Tensor] = field(default_factory=dict)
    nodes: list[Node] = field(default_factory=list)

    # -- building -----------------------------------------------------------------
    def add_tensor(self, name: str, ggml_type: int, ne, storage: int = ACTIVATION, role: str | None = None) -> int:
        tid = len(self.tensors)
        while tid in self.tensors:
            tid += 1
        ne = [_dim(d) for d in ne] + [Dim.static(1)] * (4 - len(ne))
        self.tensors[tid] = Tensor(tid, name, int(ggml_type), tuple(ne[:4]), storage, None, role)
        if storage == INPUT:
            self.inputs.append(tid)
        elif storage in (PARAMETER, CONSTANT):
            self.parameters.append(tid)
        return tid

    def add_node(self, opname: str | int, inputs: list[int], out: int, name: str = "", **attributes) -> int:
        nid = len(self.nodes)
        opcode = OPS[opname] if isinstance(opname, str) else int(opname)
        self.nodes.append(Node(nid, opcode, list(inputs), [out], dict(attributes), name))
        self.tensors[out].producer_id = nid
        return out

    # -- JSON -----------------------------------------------------------------------
    def to_json(self) -> str:
        tensors = {}
        for tid, t in self.tensors.items():
            tensors[str(tid)] = {"id": t.id, "name": t.name, "type": t.type, "ne": [d.to_json() for d in t.ne],
                                 "storage": t.storage, "producer_id": t.producer_id, "role": t.role}
        nodes = [{"id": n.id, "opcode": n.opcode, "inputs": n.inputs, "outputs": n.outputs,
                  "attributes": n.attributes, "name": n.name or ""} for n in self.nodes]
        spec = {"name": self.name, "inputs": self.inputs, "outputs": self.outputs, "parameters": self.parameters,
                "symbol_table": self.symbol_table, "metadata": self.metadata, "tensors": tensors, "nodes": nodes}
        return json.dumps(spec, separators=(",", ":"))

    @staticmethod
    def from_json(text: str) -> "Graph":
        spec = json.loads(text)
        g = Graph(name=spec.get("name", "main"), inputs=[int(i) for i in spec.get("inputs", [])],
                  outputs=[int(i) for i in spec.get("outputs", [])],
                  parameters=[int(i) for i in spec.get("parameters", [])],
                  symbol_table=[str(s) for s in spec.get("symbol_table", [])], metadata=spec.get("metadata", {}))
        for key, td in spec.get("tensors", {}).items():
            ne = [Dim.from_json(d) for d in td.get("ne", [])]
            ne = (ne + [Dim.static(1)] * 4)[:4]
            t = Tensor(int(td.get("id", key)), td.get("name", ""), int(td.get("type", 0)), tuple(ne),
                       int(td.get("storage", ACTIVATION)), td.get("producer_id"), td.get("role"))
            g.tensors[t.id] = t
        for nd in spec.get("nodes", []):
            g.nodes.append(Node(int(nd["id"]), int(nd["opcode"]), [int(i) for i in nd.get("inputs", [])],
                                [int(i) for i in nd.get("outputs", [])], dict(nd.get("attributes", {})),
                                nd.get("name") or ""))
        return g

    # -- symbols ------------------------------------------------------------------
    def shapes(self, env: dict[str, int]) -> dict[int, list[int]]:
        """Concrete ne of every tensor under `env` (the runtime's concrete_shapes_)."""
        return {tid: t.shape(env) for tid, t in self.tensors.items()}

    def free_symbols(self) -> set[str]:
        out: set[str] = set()
        for t in self.tensors.values():
            for d in t.ne:
                out |= d.free_symbols()
        return out
