"""The `rocm` target: MIRA's Target/Executable plugin protocol on MI355X.

Protocol (mira/backends/base.py:13-26):
    Target.name, Target.check(op) -> None | reason, Target.compile(graph) -> Executable
    Executable.run(feeds: {Value: ndarray}) -> {Value: ndarray}, Executable.report() -> str
An op check() rejects runs on the CPU through the partitioner
(mira/partition.py:70-93), exactly as for the reference's other targets.

compile() plans one device layout per value, packs and uploads every constant
once (int8 weights, f64 combined scales, epilogue operands), allocates every
activation buffer, and turns the segment into a list of launches of
libmira_rocm.so.  run() copies the inputs in, replays the launches on the
current HIP stream and copies the outputs out.  There is no other compute
path: without the library, compile() raises.

Device layouts.  Rank-4 values live in NHWC; every other value row-major
(C order, the last axis contiguous).  A value can exist as f32 and as one or
more int8 copies (one per x_scale its q-op consumers use); producers write the
f32 copy only if something reads it and fuse the first int8 copy into their
epilogue (requantization, mira/ops.py:602-603 applied to the result).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Callable, Optional

import numpy as np

from . import _lib as L
from . import pack


# Type annotations "Graph", "Op" and "Value" name MIRA's IR types (mira/ir.py:34-154); the
# target reads them by attribute only (kind, inputs, attrs, results, type.shape/dtype, producer,
# is_constant_like, is_control; graph inputs/ops/outputs/users()/compute_ops()), so any graph
# with those attributes compiles.

EPI_FNS = {"add", "sub", "mul", "div", "maximum", "minimum", "relu"}

_torch = None


def _t():
    global _torch
    if _torch is None:
        import torch
        _torch = torch
    return _torch


def conv_params(a: dict) -> tuple:
    """((sh, sw), (ph, pw), (dh, dw), groups) of a conv op's attrs (the names MIRA's conv2d
    and qconv2d ops carry; dilation and groups may be absent)."""
    return tuple(a["stride"]), tuple(a["padding"]), tuple(a.get("dilation", (1, 1))), a.get("groups", 1)


def conv_out(size: int, k: int, stride: int, pad: int, dilation: int = 1) -> int:
    """Output extent of a convolution or pooling window along one axis."""
    return (size + 2 * pad - dilation * (k - 1) - 1) // stride + 1


def _f32key(x: float) -> float:
    """x_scale as the quantizer sees it: rounded to f32 (mira/ops.py:603)."""
    return float(np.float32(x))


@dataclass
class DevValue:
    """Device copies of one IR value."""
    value: object
    nhwc: bool                                   # rank-4 values are stored NHWC
    f32: object = None                           # torch tensor (NHWC or row-major)
    i8: dict = field(default_factory=dict)       # f32 x_scale -> (torch int8 tensor, row stride)
    alias_of: Optional["DevValue"] = None
    half: bool = False                           # f32 holds an f16 value's IEEE halves (torch float16)

    @property
    def rows(self) -> int:
        s = self.value.type.shape
        if self.nhwc:
            return s[0] * s[2] * s[3]
        return int(np.prod(s[:-1], dtype=np.int64)) if len(s) > 1 else 1

    @property
    def cols(self) -> int:
        s = self.value.type.shape
        if self.nhwc:
            return s[1]
        return s[-1] if s else 1

    def i8_ld(self) -> int:
        return pack.c_pad_for(self.cols) if self.nhwc else pack.row_stride_for(self.cols)


# Result dtypes the kernels produce.  f16 values (the reference's default precision for
# accelerator targets, mira/passes.py:206-253): every op computes in f32 as the reference's
# ops do (mira/ops.py:43-44) and rounds its result to f16 where the reference casts it
# (.astype(float16)), so f16 results are bit-exact too.  They are stored as IEEE halves
# where the producer and every reader take halves (_plan_half_storage: the results of the
# int8 convolutions and the fused stem that only convolutions read, as their input's int8
# copy or as the residual), else as the f32 they equal exactly.
FLOAT_DTYPES = ("f32", "f16")

# ops whose rank-4 operands and results are images, stored NHWC
IMAGE_OPS = ("qconv2d", "conv2d", "maxpool2d", "pad", "reduce_mean")

W8_STREAM_ROWS = 64   # mr_w8_matmul_f32 streams the weights once per 8 rows when K % 4 != 0
F32IN_MAX_ROWS, F32IN_MAX_K = 8, 4096     # mr_qmatmul_f32in's decode shapes (k_pad <= 4096)
LNIN_MAX_K = 1024                          # mr_qmatmul_lnin's rows (k_pad <= 1024)


_UNARY_CODES = {L.EPI_FN[f] for f in L.EPI_UNARY}


def _contig(shape) -> tuple:
    """Element strides of a C-order tensor of this shape."""
    st, acc = [], 1
    for d in reversed(tuple(shape)):
        st.append(acc)
        acc *= int(d)
    return tuple(reversed(st))


def _is_contig(shape, strides) -> bool:
    """Does the strided view hold its elements in C order with no gaps (axes of extent 1,
    whose stride is never used, aside)?"""
    want = 1
    for d, s in zip(reversed(tuple(shape)), reversed(tuple(strides))):
        if d != 1:
            if s != want:
                return False
            want *= int(d)
    return True


def _ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def _truthy(t, v) -> bool:
    """A device loop's one-element condition, read back (an i32 value is held as its bits)."""
    x = t.reshape(-1)[:1]
    if v.type.dtype == "i32":
        x = x.view(_t().int32)
    return bool(x.item() != 0)


# Longest contraction whose int32 accumulator cannot overflow: K * 127 * 127 < 2^31
# (the library rejects longer ones).
MAX_EXACT_K = 133144


# a device loop (a while / if the target runs) carries values of these dtypes and of at
# most this rank; i32 values are held as their bits in the 4-byte buffers
LOOP_DTYPES = ("f32", "f16", "i32")
LOOP_MAX_RANK = 3


class RocmTarget:
    """MIRA Target for one MI355X (gfx950)."""
    name = "rocm"
    # while / if ops whose sub-graphs run here entirely run as device loops
    # (mira/partition.py:74-75); others stay with the host, their sub-graphs split as usual
    supports_control_flow = True

    def __init__(self, device: int = 0, debug_acc: bool = False, approx_f32: bool = False,
                 graph_loops: bool = True):
        """approx_f32: also run the float ops whose NumPy results depend on libm or on BLAS's
        summation order (softmax, f32 matmul of two float tensors, and gelu/sigmoid/tanh
        epilogue steps).  Their results then agree with the reference's to f32 rounding
        (relative ~1e-6), not bit for bit; every other op stays bit-exact.
        graph_loops: a while loop run on the device records its condition step and its body
        step as two HIP graphs after the first iteration and replays them, one launch each
        per iteration instead of one per kernel and copy (off: every iteration is queued
        kernel by kernel)."""
        self.device = device
        self.debug_acc = debug_acc
        self.approx_f32 = approx_f32
        self.graph_loops = graph_loops

    # ---------------------------------------------------------------- check

    def check(self, op: "Op") -> Optional[str]:
        """None if the rocm kernels run `op` with the golden model's exact arithmetic."""
        if op.is_control:
            return self._check_control(op)
        if any(r.type.dtype not in FLOAT_DTYPES for r in op.results):
            return "the rocm target computes f32 and f16 graphs only"
        k = op.kind
        if k == "cast":
            if op.inputs[0].type.dtype not in FLOAT_DTYPES:
                return "casts from integer types run on the host"
            return None
        if k in ("qmatmul", "qconv2d"):
            if k == "qconv2d" and op.attrs.get("groups", 1) != 1:
                return "grouped int8 convolution has no kernel"
            why = self._check_q_sizes(op)
            if why is not None:
                return why
            return self._check_epilogue(op, op.result.type.shape, k == "qconv2d")
        if k == "conv2d":
            x, w = op.inputs[0], op.inputs[1]
            (_, _, _, g) = conv_params(op.attrs)
            if w.producer is not None and w.producer.kind == "dequantize" and g == 1:
                return self._check_w8_conv2d(op)
            # depthwise (a dequantize weight of the weight-only mode is materialized in f32 at
            # compile time, exactly as mira/ops.py:581-586 does, so these stay bit-exact)
            if not (g == x.type.shape[1] == w.type.shape[0] and w.type.shape[1] == 1):
                return "only depthwise f32 convolution runs on rocm (dense f32 conv is not on the W8A8 path)"
            if w.producer is None or not w.producer.is_constant_like:
                return "depthwise weights must be constants"
            return self._check_epilogue(op, op.result.type.shape, True, first_operand=2)
        if k == "maxpool2d":
            return None
        if k == "pad":
            pads = tuple(tuple(p) for p in op.attrs["pads"])
            if op.inputs[0].type.rank != 4 or pads[0] != (0, 0) or pads[1] != (0, 0):
                return "pad runs on rocm only over H and W of an NCHW tensor"
            return None
        if k == "reduce_mean":
            axes = sorted(a % max(op.inputs[0].type.rank, 1) for a in op.attrs["axes"])
            if op.inputs[0].type.rank != 4 or axes != [2, 3]:
                return "reduce_mean runs on rocm only over H and W (global average pooling)"
            return None
        if k in ("reshape", "concat"):
            return None
        if k == "transpose":
            if not 1 <= op.inputs[0].type.rank <= 4:
                return "transpose runs on rocm for rank 1..4"
            return None
        if k == "layernorm":
            return None
        if k == "softmax":
            if not self.approx_f32:
                return "softmax calls exp (libm): not bit-reproducible on rocm (approx_f32 runs it)"
            r = op.inputs[0].type.rank
            if r == 0 or op.attrs["axis"] % r != r - 1:
                return "softmax runs on rocm over the last axis"
            return None
        if k == "matmul":
            w = op.inputs[1]
            if w.producer is not None and w.producer.kind == "dequantize":
                return self._check_w8_matmul(op)
            return self._check_f32_matmul(op)
        return f"'{k}' has no rocm kernel"

    @staticmethod
    def _check_q_sizes(op: "Op") -> Optional[str]:
        """The limits of the int8 contraction kernels, so an op past them stays on the CPU
        instead of failing at launch: their buffer loads take 32-bit byte offsets (int8
        activations and packed weights under 2 GiB) and they index pixels with int32."""
        q = op.attrs["q"]
        k_real = int(np.prod(q.shape, dtype=np.int64)) // q.shape[1 if op.kind == "qmatmul" else 0]
        if k_real > MAX_EXACT_K:
            return f"contraction length {k_real} > {MAX_EXACT_K}: the int32 accumulator could overflow"
        if op.kind == "qmatmul":
            K, N = q.shape
            rows = int(np.prod(op.inputs[0].type.shape[:-1], dtype=np.int64))
            if rows > 8 and rows * pack.row_stride_for(K) >= 2 ** 31:
                return "int8 matmul: an activation of 2 GiB or more"
            k_pad, n_pad = pack.roundup(K, pack.K_STEP), pack.roundup(N, pack.N_STEP)
        else:
            o, c, kh, kw = q.shape
            n, _, h, w = op.inputs[0].type.shape
            _, oh, ow = op.result.type.shape[1:]
            cp = pack.c_pad_for(c)
            if n * h * w >= 2 ** 31 or n * oh * ow >= 2 ** 31:
                return "int8 convolution: 2^31 pixels or more"
            if n * h * w * cp >= 2 ** 31:
                return "int8 convolution: an int8 input of 2 GiB or more"
            k = kh * (pack.conv_row_bytes(kw) if cp == 4 else kw * cp)
            k_pad, n_pad = pack.roundup(k, pack.K_STEP), pack.roundup(o, pack.N_STEP)
        if k_pad * n_pad >= 2 ** 31:
            return "int8 weights of 2 GiB or more"
        return None

    def _check_f32_matmul(self, op: "Op") -> Optional[str]:
        """matmul of two float tensors (attention scores and context): mr_bmm_f32 in the
        approximate mode only (BLAS's summation order is not reproducible)."""
        if not self.approx_f32:
            return ("f32 matmul stays on the CPU (its summation order is BLAS's, not reproducible bit for bit) "
                    "unless its weight is an int8 weight-only constant or approx_f32 is set")
        x, w = op.inputs[0], op.inputs[1]
        if x.type.dtype not in FLOAT_DTYPES or w.type.dtype not in FLOAT_DTYPES:
            return "f32 matmul needs float operands"
        if len(op.result.type.shape) - 2 > 4:
            return "f32 matmul runs on rocm for at most 4 batch dimensions"
        return self._check_epilogue(op, op.result.type.shape, False, first_operand=2)

    def _check_w8_matmul(self, op: "Op") -> Optional[str]:
        """Matmuls of the weight-only int8 mode (mira/quantize.py:45-68): an f32 activation
        against a `dequantize` [K, N] weight.  Decode shapes stream the weights once per 8
        rows; more rows run as f32-MFMA tiles when K % 4 == 0 (else at most W8_STREAM_ROWS
        rows).  These compute in f32 in another summation order than BLAS's, so they match
        the reference to f32 rounding (relative 1e-5), not bit for bit; every other f32
        matmul stays on the CPU."""
        x, w = op.inputs[0], op.inputs[1]
        p = w.producer
        if p is None or p.kind != "dequantize" or p.attrs["axis"] != 1 or w.type.rank != 2:
            return ("f32 matmul stays on the CPU (its summation order is BLAS's, not reproducible bit for bit) "
                    "unless its weight is an int8 weight-only constant")
        if x.type.rank not in (2, 3) or x.type.dtype not in FLOAT_DTYPES:
            return "weight-only int8 matmul runs on rocm for rank-2/3 float activations"
        rows = int(np.prod(x.type.shape[:-1], dtype=np.int64))
        K = int(x.type.shape[-1])
        if K % 4 != 0 and rows > W8_STREAM_ROWS:
            return (f"weight-only int8 matmul of {rows} rows runs on rocm only for K % 4 == 0 "
                    f"(or <= {W8_STREAM_ROWS} rows), K is {K}")
        if rows * K * 4 >= 2 ** 31:
            return "weight-only int8 matmul: an activation of 2 GiB or more"
        return self._check_epilogue(op, op.result.type.shape, False)

    def _check_w8_conv2d(self, op: "Op") -> Optional[str]:
        """Convolutions of the weight-only int8 mode: an f32 conv2d (groups 1) over a
        `dequantize` [O, C, KH, KW] weight, as an implicit GEMM on f32 MFMAs.  The kernel
        reads the NHWC image 4 channels at a time: a graph input whose channel count is not a
        multiple of 4 (a 3-channel stem) is copied to NHWC with its channels padded to 4, zero
        weights for the padding.  Like the weight-only matmul it matches the reference to f32
        rounding, not bit for bit."""
        x, w = op.inputs[0], op.inputs[1]
        p = w.producer
        (_, _, _, g) = conv_params(op.attrs)
        if p.attrs["axis"] != 0 or w.type.rank != 4 or g != 1:
            return "weight-only int8 convolution runs on rocm for dense (groups 1) convolutions"
        if x.type.rank != 4 or x.type.dtype not in FLOAT_DTYPES:
            return "weight-only int8 convolution needs an NCHW float input"
        n, c, h, wd = x.type.shape
        if c % 4 != 0 and x.producer is not None:
            return (f"weight-only int8 convolution of {c} channels (not a multiple of 4) runs on rocm only on a "
                    f"graph input, which the target copies to NHWC with the channels padded to 4")
        if n * h * wd * pack.roundup(c, 4) * 4 >= 2 ** 31:
            return "weight-only int8 convolution: an input of 2 GiB or more"
        return self._check_epilogue(op, op.result.type.shape, True, first_operand=2)

    def _check_epilogue(self, op: "Op", shape: tuple, is_conv: bool, first_operand: int = 1) -> Optional[str]:
        for fn, idx, _sw in op.attrs.get("epilogue", ()):
            if fn in L.EPI_APPROX and not self.approx_f32:
                return f"epilogue step '{fn}' calls libm: not bit-reproducible on rocm (approx_f32 runs it)"
            if fn not in EPI_FNS and fn not in L.EPI_APPROX:
                return f"epilogue step '{fn}' has no rocm implementation"
            if idx is None:
                continue
            v = op.inputs[idx]
            if v.type.dtype not in FLOAT_DTYPES:
                return "epilogue operands must be f32 or f16"
            if v.producer is not None and v.producer.is_constant_like:
                continue
            if _bcast_mode(v.type.shape, shape, is_conv) is None:
                return f"runtime epilogue operand {v.type} broadcasts onto {list(shape)} in a way rocm can't index"
        return None

    def _check_control(self, op: "Op") -> Optional[str]:
        """A while / if runs as a device loop when its values are f32 / f16 / i32 of rank <= 3
        and every op of its sub-graphs runs here (check_in_loop)."""
        for _, sg in op.subgraphs():
            for v in [*op.inputs, *op.results, *sg.inputs, *sg.outputs]:
                if v.type.dtype not in LOOP_DTYPES:
                    return f"control flow with {v.type.dtype} values runs on the host (its sub-graphs split for rocm)"
                if v.type.rank > LOOP_MAX_RANK:
                    return f"a device loop carries values of rank <= {LOOP_MAX_RANK}"
            for sop in sg.ops:
                if sop.is_constant_like:
                    continue
                why = self.check_in_loop(sop)
                if why is not None:
                    return f"control flow whose sub-graph holds {sop.kind} ({why}) runs on the host"
        return None

    def check_in_loop(self, op: "Op") -> Optional[str]:
        """check() for an op of a device loop's sub-graph, which may also hold what a loop's
        bookkeeping needs and elsewhere stays on the host: standalone elementwise ops (f32 /
        f16 / i32), casts to and from i32, gathers along axis 0, dynamic slices and updates,
        argmax over the last axis, where, static slices, and reshapes / concats of i32."""
        vals = [*op.inputs, *op.results]
        k = op.kind
        if any(v.type.dtype not in LOOP_DTYPES for v in vals):
            return "device loops hold f32, f16 and i32 values"
        if any(v.type.rank > 4 for v in vals):
            return "device loops hold values of rank <= 4"
        ints = any(v.type.dtype == "i32" for v in vals)
        if k in L.EW_FN:
            if len({v.type.dtype for v in op.inputs}) != 1 or (ints and k == "div"):
                return "elementwise operands of one dtype (no integer division)"
            return None
        if k == "cast":
            return None
        if k == "gather":
            return None if op.attrs["axis"] % op.inputs[0].type.rank == 0 else "gather runs on rocm along axis 0"
        if k in ("dynamic_slice", "dynamic_update_slice", "where", "slice"):
            return None
        if k == "argmax":
            x = op.inputs[0]
            return None if x.type.dtype in FLOAT_DTYPES and op.attrs["axis"] % x.type.rank == x.type.rank - 1 else \
                "argmax runs on rocm over the last axis of a float tensor"
        if k in ("reshape", "concat") and ints:
            return None
        return self.check(op)

    def compile(self, g: "Graph", compile_sub=None) -> "RocmExecutable":
        """compile_sub (MIRA's sub-graph compiler) is not needed: a device loop's sub-graphs are
        compiled here."""
        return RocmExecutable(g, self)


def _bcast_mode(oshape: tuple, rshape: tuple, is_conv: bool) -> Optional[int]:
    """How an operand of shape `oshape` broadcasts onto result `rshape` as device rows x cols."""
    r = len(rshape)
    o = (1,) * (r - len(oshape)) + tuple(oshape)
    if all(d == 1 for d in o):
        return L.BC_SCALAR
    if o == tuple(rshape):
        return L.BC_FULL
    ch = 1 if is_conv else r - 1                 # axis that becomes device columns
    if all(d == 1 for i, d in enumerate(o) if i != ch) and o[ch] == rshape[ch]:
        return L.BC_COL
    if o[ch] == 1 and all(d == rshape[i] for i, d in enumerate(o) if i != ch):
        return L.BC_ROW
    return None


class RocmExecutable:
    """A compiled rocm segment: device buffers, packed constants and a launch list."""

    def __init__(self, g: "Graph", target: RocmTarget, in_loop: bool = False, bind: Optional[dict] = None):
        """bind: graph input -> a contiguous f32 device tensor of its size that the launches read
        the input from in place of a staging buffer of their own (a device loop's state and
        captures); `bound` lists the inputs that took it."""
        torch = _t()
        self.g = g
        self.bind = bind or {}
        self.bound: set = set()
        self.target = target
        self.lib = L.load()
        if not torch.cuda.is_available():
            raise L.RocmError("the rocm target needs a ROCm GPU (torch.cuda.is_available() is False)")
        self.dev = torch.device("cuda", target.device)
        torch.cuda.set_device(self.dev)
        L.check(self.lib.mr_init(target.device), "mr_init")
        for op in g.ops:
            if not op.is_constant_like:
                reason = target.check_in_loop(op) if in_loop else target.check(op)
                if reason:
                    raise L.RocmError(f"rocm cannot run {op.kind}: {reason}")
        self.launches: list[tuple[str, Callable[[int], None]]] = []
        self.keep: list = []          # host objects (ctypes structs, tensors) the launches refer to
        self.dv: dict["Value", DevValue] = {}
        self.acc: dict["Value", object] = {}      # debug int32 accumulators per q-op result
        self.kernel_counts: dict[str, int] = {}
        self.launch_cost: list[tuple[str, int, int]] = []
        self.const_bytes = 0
        self._plan()

    # ---------------------------------------------------------------- planning

    def _plan(self) -> None:
        g = self.g
        users = g.users()
        self.users = users
        # producers inside this graph only: an input of a segment split from a larger graph
        # keeps its producer there, in another segment
        self.prod = {r: op for op in g.ops for r in op.results}
        self.consts = {op.result: op for op in g.ops if op.is_constant_like}
        # rank-4 values that an image op reads or writes live NHWC on the device; other
        # rank-4 values (attention heads [b, s, h, d], say) keep the graph's C order
        self.images: set = set()
        for op in g.ops:
            if op.kind in IMAGE_OPS:
                self.images.update(v for v in [*op.inputs, op.result] if v.type.rank == 4)
        # a cast's result shares its input's buffers, so their layouts agree: propagate along
        # chains of casts until nothing changes
        grew = True
        while grew:
            grew = False
            for op in g.ops:
                if op.kind == "cast" and (op.result in self.images) != (op.inputs[0] in self.images):
                    self.images.update((op.inputs[0], op.result))
                    grew = True
        # which forms each value needs
        self.need_f32: set = set(g.outputs)
        self.need_i8: dict["Value", list[float]] = {}
        self.folded_pads: set = set()
        self.fused_stem: dict = {}          # maxpool op -> (qconv2d op, pad op) run as one kernel
        self.skip: set = set()
        for op in g.ops:
            if op.is_constant_like:
                continue
            if op.kind in ("qmatmul", "qconv2d"):
                s = _f32key(op.attrs["x_scale"])
                lst = self.need_i8.setdefault(op.inputs[0], [])
                if s not in lst:
                    lst.append(s)
                for v in op.inputs[1:]:
                    self.need_f32.add(v)
            elif op.kind == "maxpool2d" and self._foldable_pad(op.inputs[0]):
                pad_op = self._producer(op.inputs[0])
                self.folded_pads.add(pad_op)
                conv = self._producer(pad_op.inputs[0])
                if self._stem_fusable(conv, pad_op, op):
                    self.fused_stem[op] = (conv, pad_op)
                    self.skip.add(conv)
                else:
                    self.need_f32.add(pad_op.inputs[0])
            else:
                for v in op.inputs:
                    if v is op.inputs[0] and self._padded_w8_input(op):
                        continue            # read through its own channel-padded NHWC copy
                    if v not in self.consts or op.kind not in ("conv2d", "matmul") or v is op.inputs[0]:
                        self.need_f32.add(v)
        # reshapes: the input must provide what the output's consumers read; a reshape
        # that keeps the int8 layout (same rows, columns and row stride) passes its
        # int8 copies through, so the producer writes them in its epilogue
        for op in reversed(g.ops):
            if op.kind == "reshape":
                r = op.result
                if r in self.need_f32 or r in self.need_i8:
                    self.need_f32.add(op.inputs[0])
                if r in self.need_i8 and self._i8_view(op.inputs[0], r):
                    lst = self.need_i8.setdefault(op.inputs[0], [])
                    lst += [s for s in self.need_i8[r] if s not in lst]
        # a cast to f16 that is a graph input's only use rounds the input buffer in place
        # before anything reads it; its result then shares the input's device copies
        self.input_casts: set = set()
        for op in g.ops:
            v = op.inputs[0] if op.kind == "cast" and op.inputs else None
            if v is not None and v in g.inputs and v not in g.outputs and len(users.get(v, [])) == 1 and \
                    v.type.dtype == "f32" and op.result.type.dtype == "f16":
                self.input_casts.add(op)
                r = op.result
                if r not in self.need_f32:
                    self.need_f32.discard(v)
                lst = self.need_i8.setdefault(v, [])
                lst += [s for s in self.need_i8.get(r, []) if s not in lst]
        # a fused stem that is its image input's only reader quantizes the rows it needs
        # from the f32 input itself: no int8 copy of the image is made
        self.stem_f32in: dict = {}          # maxpool op -> (graph input, quantize its f16 rounding)
        for pool, (conv, _) in self.fused_stem.items():
            src = self._stem_f32_source(conv)
            if src is None:
                continue
            self.stem_f32in[pool] = src
            xs = _f32key(conv.attrs["x_scale"])
            for v in {src[0], conv.inputs[0]}:
                self.need_i8[v] = [s for s in self.need_i8.get(v, []) if s != xs]
        self.staging: dict["Value", object] = {}
        self._pinned: dict["Value", object] = {}     # pinned host buffers of upload()
        self._upload_done = None                     # event after upload()'s last DMA
        self.canon: dict["Value", object] = {}     # C-order copies of NHWC values (_c_order)
        self.i8_preset: dict = {}      # value -> int8 copies an earlier kernel already wrote
        self._plan_attention()
        self._plan_views()
        self._plan_shared_input_matmuls()
        self._plan_f32in_matmuls()
        self._plan_lnin_matmuls()
        self._plan_half_storage()
        self._plan_expand_dw()
        for v in g.inputs:
            self._emit_input(v)
        for op in g.ops:
            if not self._device_op(op) or op in self.virtual:
                continue
            getattr(self, f"_emit_{op.kind}")(op)
        for v in g.outputs:
            if v in self.consts and v not in self.dv:
                self._const_dv(v)

    def _padded_w8_input(self, op: "Op") -> bool:
        """A weight-only convolution over a graph input whose channel count is not a multiple
        of 4: it reads its own channel-padded NHWC copy of the input (_emit_w8_conv2d)."""
        x = op.inputs[0]
        w = op.inputs[1] if len(op.inputs) > 1 else None
        return (op.kind == "conv2d" and w is not None and w in self.consts and
                self.consts[w].kind == "dequantize" and x in self.g.inputs and x.type.rank == 4 and
                x.type.shape[1] % 4 != 0)

    def _producer(self, v: "Value") -> Optional["Op"]:
        """The op of this graph that makes v (None for the graph's inputs)."""
        return self.prod.get(v)

    def _is_bmm(self, op: "Op") -> bool:
        w = op.inputs[1] if op.kind == "matmul" else None
        return w is not None and not (self._producer(w) is not None and self._producer(w).kind == "dequantize")

    def _view_chain(self, v: "Value") -> tuple:
        """(base, shape, strides, chain): v as a strided view of `base`, the first value up its
        chain of reshapes and transposes that has its own C-order buffer; `chain` lists the
        values passed on the way (v first).  A reshape of a view that is not contiguous stops
        the walk (that value is then the base)."""
        p = self._producer(v)
        shape = tuple(v.type.shape)
        if p is not None and v not in self.images and p.kind in ("transpose", "reshape") and \
                p.inputs[0] not in self.images and p.inputs[0] not in self.consts:
            base, s, st, chain = self._view_chain(p.inputs[0])
            if p.kind == "transpose":
                perm = tuple(p.attrs["perm"])
                return base, shape, tuple(st[i] for i in perm), [v] + chain
            if _is_contig(s, st):
                return base, shape, _contig(shape), [v] + chain
        return v, shape, _contig(shape), []

    def _only_feeds(self, v: "Value", op: "Op") -> bool:
        """Is every read of v, and of the reshapes/transposes made of it, an input of `op`?"""
        us = self.users.get(v, [])
        return bool(us) and v not in self.g.outputs and all(
            u is op or (u.kind in ("reshape", "transpose") and self._only_feeds(u.result, op)) for u in us)

    def _plan_attention(self) -> None:
        """Decode-step attention run as one mr_attention_decode_f32 launch (approx_f32 only): the
        chain matmul(q4, k4) with epilogue mul(scalar scale), add(mask over the keys) ->
        softmax(last axis) -> matmul(., v4), where q4 [B, H, 1, hd] is a head view of a [B, D]
        query, and k4 [B, H, hd, T+1] / v4 [B, H, T+1, hd] are head views of concat(cache
        [B, T, D], row [B, 1, D]) along axis 1.  The two matmuls, the softmax and both concats
        are not run; the kernel reads the caches and the step's rows in place."""
        self.attn: dict = {}
        if not self.target.approx_f32:
            return
        g, users = self.g, self.users
        for sm in g.ops:
            if sm.kind != "softmax" or not self._device_op(sm):
                continue
            sc = sm.inputs[0]
            A = self._producer(sc)
            if A is None or A.kind != "matmul" or not self._is_bmm(A) or users.get(sc) != [sm] or sc in g.outputs:
                continue
            r = sm.result.type.rank
            bus = users.get(sm.result, [])
            if r != 4 or sm.attrs["axis"] % r != 3 or len(bus) != 1 or sm.result in g.outputs:
                continue
            Bop = bus[0]
            if Bop.kind != "matmul" or not self._is_bmm(Bop) or Bop.inputs[0] is not sm.result:
                continue
            if any(v.type.dtype != "f32" for v in (*A.inputs[:2], A.result, Bop.inputs[1], Bop.result)):
                continue
            qb, qs, qst, _ = self._view_chain(A.inputs[0])
            kb, ks, kst, _ = self._view_chain(A.inputs[1])
            vb, vs, vst, _ = self._view_chain(Bop.inputs[1])
            if len(qs) != 4:
                continue
            Bn, H, one, hd = qs
            if one != 1 or hd not in (16, 32, 64):
                continue
            D = H * hd
            T1 = ks[3] if len(ks) == 4 else -1
            if ks != (Bn, H, hd, T1) or vs != (Bn, H, T1, hd) or T1 < 1 or T1 > 1024 or \
                    tuple(A.result.type.shape) != (Bn, H, 1, T1) or tuple(Bop.result.type.shape) != (Bn, H, 1, hd):
                continue
            if qb.type.shape != (Bn, D) or qst != (D, hd, qst[2], 1):
                continue
            if kst != (T1 * D, hd, 1, D) or vst != (T1 * D, hd, D, 1):
                continue
            cats = []
            for base, user in ((kb, A), (vb, Bop)):
                c = self._producer(base)
                if c is None or c.kind != "concat" or c.attrs["axis"] % 3 != 1 or len(c.inputs) != 2 or \
                        base.type.shape != (Bn, T1, D) or not self._only_feeds(base, user):
                    break
                cache, row = c.inputs
                rb, rs, rst, _ = self._view_chain(row)
                if cache.type.shape != (Bn, T1 - 1, D) or rb.type.shape != (Bn, D) or \
                        row.type.shape != (Bn, 1, D) or cache in self.images:
                    break
                cats.append((c, cache, rb))
            if len(cats) != 2:
                continue
            epi = A.attrs.get("epilogue", ())
            if len(epi) != 2 or epi[0][0] != "mul" or epi[1][0] != "add" or epi[0][2] or epi[1][2]:
                continue
            sv, mv = A.inputs[epi[0][1]], A.inputs[epi[1][1]]
            if sv not in self.consts or sv.type.numel != 1 or mv.type.numel != T1 or \
                    tuple(mv.type.shape)[-1] != T1 or mv.type.dtype != "f32":
                continue
            self.attn[Bop] = {"q": qb, "kc": cats[0][1], "kn": cats[0][2], "vc": cats[1][1], "vn": cats[1][2],
                              "mask": mv, "scale": float(np.asarray(self._const_value(sv)).reshape(())),
                              "B": Bn, "H": H, "hd": hd, "T": T1 - 1}
            self.skip.update((A, sm, cats[0][0], cats[1][0]))

    def _row_slice_ok(self, v: "Value") -> bool:
        """Can v's f32 copy be a column slice of a wider buffer (rows with a stride)?  Only when
        nothing reads it as a C-order buffer: it is a graph output (copied out by strides), or
        it feeds a fused attention (which takes row strides), views that are never run, ops
        that are not run, or reshapes of its rows that only such ops read."""
        for u in self.users.get(v, []):
            if u in self.skip or u in self.virtual:
                continue
            if u.kind == "reshape" and u.result not in self.g.outputs and self._row_slice_ok(u.result) and \
                    all(w in self.skip for w in self.users.get(u.result, [])):
                continue
            return False
        return True

    def _plan_shared_input_matmuls(self) -> None:
        """q-ops that read the same int8 activation at the same x_scale, without an epilogue and
        with f32 results only (a transformer's query/key/value projections) run as one
        mr_qmatmul over their weights side by side: each result is a column slice of one
        [rows, sum N] buffer.  Only results whose readers take row strides (see
        _row_slice_ok) join such a group."""
        self.row_group: dict = {}       # first op of a group -> the group's ops
        if self.target.debug_acc:
            return
        groups: dict = {}
        for op in self.g.ops:
            if op.kind != "qmatmul" or not self._device_op(op) or op.attrs.get("epilogue") or \
                    op.result.type.dtype != "f32" or op.result.type.rank != 2 or self.need_i8.get(op.result) or \
                    op.inputs[0] in self.images:
                continue
            if not self._row_slice_ok(op.result):
                continue
            groups.setdefault((op.inputs[0], _f32key(op.attrs["x_scale"])), []).append(op)
        for ops in groups.values():
            if len(ops) < 2:
                continue
            self.row_group[ops[0]] = ops
            self.skip.update(ops[1:])
            for op in ops:
                for u in self.users.get(op.result, []):
                    if u.kind == "reshape" and u not in self.virtual and u not in self.skip:
                        self.skip.add(u)          # read only by ops that are not run

    def _plan_f32in_matmuls(self) -> None:
        """A decode-shaped qmatmul (at most 8 rows, K <= 4096) that is the only reader of a
        segment input's int8 copy quantizes the input's f32 rows itself (mr_qmatmul_f32in):
        the first layer of an MLP step at batch 1 then needs no quantize launch."""
        self.f32in: dict = {}       # qmatmul op -> the segment input whose f32 rows it reads
        g = self.g
        for op in g.ops:
            if op.kind != "qmatmul" or not self._device_op(op) or op in self.row_group:
                continue
            v, xs = op.inputs[0], _f32key(op.attrs["x_scale"])
            K = int(np.shape(op.attrs["q"])[0])
            if v not in g.inputs or v in self.images or v in self.prealias or v.type.rank < 1 or \
                    pack.roundup(K, 64) > F32IN_MAX_K or not 1 <= DevValue(v, nhwc=False).rows <= F32IN_MAX_ROWS:
                continue
            if any(c.inputs[0] is v for c in self.input_casts):
                continue
            readers = [u for u in g.ops if u.kind in ("qmatmul", "qconv2d") and u.inputs[0] is v and
                       _f32key(u.attrs["x_scale"]) == xs]
            if readers != [op]:
                continue
            self.f32in[op] = v
            self.need_i8[v] = [t for t in self.need_i8.get(v, []) if t != xs]

    def _plan_lnin_matmuls(self) -> None:
        """A layernorm whose result only decode-shaped q-matmuls read, as their int8 input at
        one x_scale (a transformer decode step's projections after each layernorm), runs inside
        the launch of each of them, or of their group (mr_qmatmul_lnin): no layernorm launch,
        no int8 copy of its result."""
        self.lnin: dict = {}        # qmatmul op (a group's first op) -> the layernorm it runs
        g = self.g
        group_of = {o: head for head, ops in self.row_group.items() for o in ops}
        for ln in g.ops:
            if ln.kind != "layernorm" or not self._device_op(ln):
                continue
            r = ln.result
            d = r.type.shape[-1]
            rows = r.type.numel // d if d else 0
            if r in g.outputs or r in self.need_f32 or r in self.images or pack.roundup(d, 64) > LNIN_MAX_K or \
                    not 1 <= rows <= F32IN_MAX_ROWS:
                continue
            readers = self.users.get(r, [])
            if not readers or any(u.kind != "qmatmul" or u.inputs[0] is not r or r in u.inputs[1:] or
                                  (not self._device_op(u) and u not in group_of) for u in readers):
                continue
            if len({_f32key(u.attrs["x_scale"]) for u in readers}) != 1:
                continue
            # each reading launch (a q-op, or a group's first q-op) normalises the rows itself
            heads: dict = {}
            for u in readers:
                heads.setdefault(group_of.get(u, u), set()).add(u)
            if any(set(self.row_group.get(h, [h])) != us or h in self.f32in for h, us in heads.items()):
                continue
            for h in heads:
                self.lnin[h] = ln
            self.skip.add(ln)
            self.need_i8.pop(r, None)

    def _lnin_launch(self, ln: "Op", xs: float, b, kp: int, npad: int, M: int, N: int, K: int, e):
        """The launch of a q-matmul that runs the layernorm `ln` on its f32 rows first."""
        x = self._c_order(ln.inputs[0])
        gm, bt = self._c_order(ln.inputs[1]), self._c_order(ln.inputs[2])
        eps, f16, lib = float(ln.attrs["eps"]), int(ln.result.type.dtype == "f16"), self.lib
        return lambda s: L.check(lib.mr_qmatmul_lnin(x.data_ptr(), K, gm.data_ptr(), bt.data_ptr(), eps, f16, xs,
                                                     b.data_ptr(), kp, npad, M, N, K, C.byref(e), s),
                                 "mr_qmatmul_lnin")

    def _full_operand_reader(self, u: "Op", v: "Value") -> bool:
        """Does the q-op u read v only as its int8 input (inputs[0]: the copy v's producer
        writes) and/or as the one full-shape operand of its epilogue?"""
        if u.kind not in ("qconv2d", "qmatmul") or not self._device_op(u):
            return False
        is_conv = u.kind == "qconv2d"
        full = [idx for _, idx, _ in u.attrs.get("epilogue", ()) if idx is not None and
                u.inputs[idx] not in self.consts and
                _bcast_mode(u.inputs[idx].type.shape, u.result.type.shape, is_conv) == L.BC_FULL]
        steps = {idx for _, idx, _ in u.attrs.get("epilogue", ()) if idx is not None}
        for i, x in enumerate(u.inputs):
            if x is not v or i == 0:
                continue
            if i not in steps or i not in full or len(set(u.inputs[j] for j in full)) != 1:
                return False
        return True

    def _relu6_epilogue(self, op: "Op") -> bool:
        """The epilogue is add(per-channel constant) -> maximum(scalar constant) or relu ->
        minimum(scalar constant), none swapped: the form mr_qconv1x1_dw3x3 runs."""
        steps = tuple(op.attrs.get("epilogue", ()))
        if len(steps) != 3 or any(sw for _fn, _i, sw in steps):
            return False
        (f0, i0, _), (f1, i1, _), (f2, i2, _) = steps
        rshape = op.result.type.shape

        def mode(idx):
            v = op.inputs[idx]
            return _bcast_mode(np.shape(self._const_value(v)), rshape, True) if v in self.consts else None
        return (f0 == "add" and mode(i0) == L.BC_COL and f2 == "minimum" and mode(i2) == L.BC_SCALAR and
                (f1 == "relu" or (f1 == "maximum" and mode(i1) == L.BC_SCALAR)))

    def _plan_expand_dw(self) -> None:
        """A 1x1 q-convolution whose f32 result only a 3x3 depthwise convolution reads (a
        MobileNet block's expansion) runs inside that convolution's launch
        (mr_qconv1x1_dw3x3), and so does a 3x3 stem over an image of at most 4 channels
        (mr_qstem3x3_dw3x3): the expanded tensor is never stored.  Both epilogues bias ->
        ReLU6, f32 or f16 graphs (values not stored as halves), the depthwise result read as
        int8."""
        self.expand_dw: dict = {}           # depthwise op -> its expansion q-op
        if self.target.debug_acc:
            return
        g = self.g
        for op in g.ops:
            if op.kind != "conv2d" or not self._device_op(op) or len(op.inputs) < 2:
                continue
            v, w = op.inputs[0], op.inputs[1]
            e = self._producer(v)
            if w not in self.consts or self.consts[w].kind != "const" or e is None or e.kind != "qconv2d":
                continue
            if not self._device_op(e) or e in self.virtual or v in g.outputs or self.users.get(v, []) != [op]:
                continue
            (sh, sw), (ph, pw), (dh, dw), groups = conv_params(op.attrs)
            n, c, h, wd = v.type.shape
            if groups != c or np.shape(self._const_value(w)) != (c, 1, 3, 3) or sh != sw or sh not in (1, 2) or \
                    (ph, pw) != (1, 1) or (dh, dw) != (1, 1) or c % 4:
                continue
            q = np.asarray(e.attrs["q"])
            (esh, esw), (eph, epw), (edh, edw), eg = conv_params(e.attrs)
            cin = e.inputs[0].type.shape[1]
            expansion = q.shape[2:] == (1, 1) and (esh, esw, eph, epw, edh, edw, eg) == (1, 1, 0, 0, 1, 1, 1) and \
                4 < cin <= 192
            # a 3x3 stem over a 4-byte-per-pixel image (mr_qstem3x3_dw3x3)
            stem = q.shape[2:] == (3, 3) and esh == esw and esh in (1, 2) and (eph, epw, edh, edw, eg) == \
                (1, 1, 1, 1, 1) and cin <= 4
            if not (expansion or stem):
                continue
            if v.type.dtype != op.result.type.dtype or v.type.dtype not in FLOAT_DTYPES or v in self.half or \
                    op.result in self.half:
                continue
            if not self.need_i8.get(op.result) or not self._relu6_epilogue(e) or not self._relu6_epilogue(op):
                continue
            self.expand_dw[op] = e
            self.skip.add(e)
            self.need_f32.discard(v)

    def _plan_half_storage(self) -> None:
        """f16 values stored as IEEE halves (mr_epilogue's MR_EPI_OUT_H16 / MR_EPI_FULL_H16):
        an f16 result of an int8 convolution or of the fused stem that is not a segment
        output, whose producer writes at most one int8 copy, and that only q-ops read -- as
        their int8 input or as the residual of their epilogue.  The halves hold the same
        values as the f32 copies would, in half the bytes."""
        self.half: set = set()
        g = self.g
        stem_convs = {conv for conv, _ in self.fused_stem.values()}
        for op in g.ops:
            if not ((op.kind == "qconv2d" and self._device_op(op) and op not in stem_convs) or
                    (op.kind == "maxpool2d" and op in self.fused_stem)):
                continue
            v = op.result
            if v.type.dtype != "f16" or v in g.outputs or v not in self.need_f32 or len(self.need_i8.get(v, [])) > 1:
                continue
            if all(self._full_operand_reader(u, v) for u in self.users.get(v, [])):
                self.half.add(v)

    def _plan_views(self) -> None:
        """Two ways of not copying, decided before any buffer exists:
        * a transpose whose result is read only as a matmul operand (directly or through
          reshapes and transposes) is not run: the matmul reads its input as a strided view;
        * a segment input read only by one concat becomes a slice of the concat's result
          buffer, so the concat copies only its other operands (a key/value cache joined by
          the current step's row)."""
        torch = _t()
        g, users = self.g, self.users
        self.virtual: set = set()
        if self.target.approx_f32:
            through: dict = {}          # value -> number of matmul operand chains passing it
            for op in g.ops:
                if op.kind == "matmul" and self._is_bmm(op):
                    for v in op.inputs[:2]:
                        for c in self._view_chain(v)[3]:
                            through[c] = through.get(c, 0) + 1
            def only_views(r) -> bool:
                """Is every read of r, and of whatever reshapes/transposes make of it, a matmul
                operand chain?"""
                if r not in through or r in g.outputs:
                    return False
                return all((u.kind == "matmul" and self._is_bmm(u) and r in u.inputs[:2]) or
                           (u.kind in ("reshape", "transpose") and only_views(u.result))
                           for u in users.get(r, []))

            # a chain op is not run when nothing but the chains reads its result
            for op in g.ops:
                if op.kind in ("transpose", "reshape") and only_views(op.result):
                    self.virtual.add(op)
        self.concat_out: dict = {}     # concat op -> its preallocated C-order result buffer
        self.prealias: dict = {}       # segment input -> its slice of a concat result
        for op in g.ops:
            if op.kind != "concat" or op.result in self.images or not self._device_op(op):
                continue
            r = op.result
            axis = op.attrs["axis"] % r.type.rank
            buf, at = None, 0
            for v in op.inputs:
                n = v.type.shape[axis]
                if v in g.inputs and v not in g.outputs and v not in self.images and v not in self.prealias and \
                        op.inputs.count(v) == 1 and len(users.get(v, [])) == 1 and not self.need_i8.get(v):
                    if buf is None:
                        buf = torch.empty(r.type.shape, dtype=torch.float32, device=self.dev)
                    self.prealias[v] = buf.narrow(axis, at, n)
                at += n
            if buf is not None:
                self.concat_out[op] = buf

    def _device_op(self, op: "Op") -> bool:
        return not (op.is_constant_like or op in self.folded_pads or op in self.skip)

    def _i8_view(self, src: "Value", r: "Value") -> bool:
        """Is the int8 copy of `r` (a reshape of `src`) the same bytes as src's? Only for an
        [n, c, 1, 1] image <-> [n, c] (global average pooling into an fc layer): NHWC with
        1x1 pixels is row-major [n, c], and both strides round c up to 16."""
        if not ({src, r} & self.images):
            return False
        a, b = tuple(src.type.shape), tuple(r.type.shape)
        if len(a) == 4 and len(b) == 2:
            a, b = b, a
        return len(a) == 2 and len(b) == 4 and b[2] == b[3] == 1 and a == (b[0], b[1]) and \
            pack.c_pad_for(b[1]) == pack.row_stride_for(b[1])

    def _stem_fusable(self, conv: Optional["Op"], pad_op: "Op", pool: "Op") -> bool:
        """Can qconv2d -> pad -> maxpool2d run as mr_qconv2d_maxpool (the convolution is never stored)?
        The kernel pools the int32 accumulators, so the epilogue must commute with max."""
        if conv is None or conv.kind != "qconv2d" or self.target.debug_acc:
            return False
        r = conv.result
        if r in self.g.outputs or len(self.users.get(r, [])) != 1:
            return False
        n, c, h, w = conv.inputs[0].type.shape
        o, _, kh, kw = conv.attrs["q"].shape
        ow = r.type.shape[3]
        pads = tuple(tuple(x) for x in pad_op.attrs["pads"])
        pool_cfg = (pool.attrs["size"], pool.attrs["stride"], pads[2][0], pads[3][0])
        kernel_ok = (5 <= kh <= 8) if kw >= 5 else (kh <= 4)
        return (c <= 4 and o <= 64 and ow <= 128 and kw <= 8 and kernel_ok
                and pool_cfg in ((3, 2, 1, 1), (2, 2, 0, 0))
                and pool.result.type.shape[3] <= (60 if pool_cfg[0] == 3 else 64)
                and self._monotone_epilogue(conv))

    def _stem_f32_source(self, conv: "Op") -> Optional[tuple]:
        """(graph input, round to f16 first) when a fused stem can read its image straight from
        the f32 NCHW input with mr_qconv2d_maxpool_f32in: the convolution is the input's only
        reader (directly, or through the f16 cast of an f16 graph), the kernel has 7 rows of
        5-8 taps, no dilation, an even column stride, a row stride of at most 2, and input rows
        of at most 64 four-pixel groups."""
        x = conv.inputs[0]
        p = self._producer(x)
        f16 = p is not None and p in self.input_casts
        v = p.inputs[0] if f16 else x
        if v not in self.g.inputs or v in self.g.outputs or x in self.g.outputs:
            return None
        if len(self.users.get(v, [])) != 1 or len(self.users.get(x, [])) != 1:
            return None
        if v in self.need_f32 or x in self.need_f32 or v.type.dtype != "f32":
            return None
        _, c, kh, kw = conv.attrs["q"].shape
        (sh, sw), (_, pw), (dh, dw), _ = conv_params(conv.attrs)
        ow = conv.result.type.shape[3]
        groups = ((ow - 1) * sw + 8 - pw + (pw + 3) // 4 * 4 + 3) // 4     # 4-pixel column groups per input row
        if c > 4 or kh != 7 or not 5 <= kw <= 8 or (dh, dw) != (1, 1) or sw % 2 or sh > 2 or groups > 64:
            return None
        return v, f16

    def _monotone_epilogue(self, op: "Op") -> bool:
        """Every step non-decreasing in the value, with an operand that is the same across a
        pooling window (scalar or per-channel).  A mul qualifies when its operand is a
        constant that is finite and positive everywhere (a BatchNorm scale)."""
        rshape = op.result.type.shape
        for fn, idx, swapped in op.attrs.get("epilogue", ()):
            if fn == "relu":
                continue
            v = op.inputs[idx]
            if fn == "mul":
                if v not in self.consts:
                    return False
                m = np.asarray(self._const_value(v), np.float32)
                if not (np.isfinite(m).all() and (m > 0).all()):
                    return False
            elif fn not in ("add", "sub", "maximum", "minimum") or (fn == "sub" and swapped):
                return False
            shape = np.shape(self._const_value(v)) if v in self.consts else v.type.shape
            if _bcast_mode(shape, rshape, True) not in (L.BC_SCALAR, L.BC_COL):
                return False
        return True

    def _foldable_pad(self, v: "Value") -> bool:
        p = self._producer(v)
        if p is None or p.kind != "pad" or v in self.g.outputs or len(self.users.get(v, [])) != 1:
            return False
        pads = tuple(tuple(x) for x in p.attrs["pads"])
        return p.inputs[0].type.rank == 4 and pads[0] == (0, 0) and pads[1] == (0, 0)

    def _new_dv(self, v: "Value", with_i8: bool = False) -> DevValue:
        """Allocate v's f32 copy if anything reads it; int8 copies only for segment inputs
        (producers allocate the ones they write)."""
        torch = _t()
        d = DevValue(v, nhwc=v in self.images, half=v in self.half)
        if v in self.need_f32:
            s = v.type.shape
            shape = (s[0], s[2], s[3], s[1]) if d.nhwc else s
            d.f32 = torch.empty(shape, dtype=torch.float16 if d.half else torch.float32, device=self.dev)
        if with_i8:
            for xs in self.need_i8.get(v, []):
                d.i8[xs] = (torch.empty((d.rows, d.i8_ld()), dtype=torch.int8, device=self.dev), d.i8_ld())
        self.dv[v] = d
        return d

    def _emit_input(self, v: "Value") -> None:
        """A segment input lives on the device as f32 in the graph's own layout (NCHW for
        images); the launch list starts by building the copies the kernels read from it: the
        NHWC f32 copy and the int8 copies its q-op consumers need (their quantize_activation,
        mira/ops.py:602-603)."""
        torch = _t()
        lib = self.lib
        stage = self.prealias.get(v)
        bound = self.bind.get(v)
        if stage is None and bound is not None and bound.is_contiguous() and bound.numel() == v.type.numel and \
                not any(op.inputs[0] is v for op in self.input_casts):     # those round it in place
            stage = bound.view(v.type.shape)
            self.bound.add(v)
        if stage is None:
            stage = torch.empty(v.type.shape, dtype=torch.float32, device=self.dev)
        self.staging[v] = stage
        d = self._new_dv(v, with_i8=True)
        cast16 = any(op.inputs[0] is v for op in self.input_casts)
        # an image that only feeds q-ops is quantized straight from its f16 rounding
        fused16 = cast16 and d.nhwc and d.f32 is None
        if cast16 and not fused16:
            self._round_f16(stage, stage)
        quant_nchw = lib.mr_quantize_f16_nchw_nhwc if fused16 else lib.mr_quantize_nchw_nhwc
        if d.nhwc:
            n, c, h, w = v.type.shape
            if d.f32 is not None:
                dst = d.f32
                self._add("input", lambda s: L.check(lib.mr_nchw_to_nhwc_f32(stage.data_ptr(), n, c, h, w,
                                                                             dst.data_ptr(), s), "mr_nchw_to_nhwc_f32"),
                          nbytes=8 * n * c * h * w)
            for xs, (q, cp) in d.i8.items():
                self._add("input", lambda s, q=q, cp=cp, xs=xs: L.check(
                    quant_nchw(stage.data_ptr(), n, c, h, w, q.data_ptr(), cp, xs, s),
                    "mr_quantize_nchw_nhwc"), nbytes=4 * n * c * h * w + n * h * w * cp)
        else:
            if d.f32 is not None:
                d.f32 = stage.reshape(d.f32.shape)       # same layout: the kernels read the input itself
            rows, cols = d.rows, d.cols
            for xs, (q, ld) in d.i8.items():
                self._add("input", lambda s, q=q, ld=ld, xs=xs: L.check(
                    lib.mr_quantize_rows(stage.data_ptr(), rows, cols, cols, q.data_ptr(), ld, xs, s),
                    "mr_quantize_rows"), nbytes=4 * rows * cols + rows * ld)

    def _upload(self, arr: np.ndarray, dtype=None):
        torch = _t()
        a = np.ascontiguousarray(arr if dtype is None else arr.astype(dtype))
        if not a.flags.writeable:        # torch wraps only writable arrays (a read-only const attr)
            a = a.copy()
        t = torch.from_numpy(a).to(self.dev)
        self.const_bytes += a.nbytes
        self.keep.append(t)
        return t

    def _const_value(self, v: "Value") -> np.ndarray:
        op = self.consts[v]
        if op.kind == "const":
            return np.asarray(op.attrs["value"])
        # a `dequantize` constant (int8 weight-only mode), materialized once as
        # q * scale in f32, then in its dtype (mira/ops.py:581-586)
        a = op.attrs
        shape = [1] * a["q"].ndim
        shape[a["axis"]] = -1
        return (a["q"].astype(np.float32) * np.asarray(a["scale"], np.float32).reshape(shape)).astype(
            np.float16 if a["dtype"] == "f16" else np.float32)

    def _const_dv(self, v: "Value") -> DevValue:
        """A constant used as a data input: upload it in its device layout."""
        if v in self.dv:
            return self.dv[v]
        a = self._const_value(v)
        a = a.astype(np.int32).view(np.float32) if v.type.dtype == "i32" else a.astype(np.float32)
        d = DevValue(v, nhwc=v in self.images)
        d.f32 = self._upload(a.transpose(0, 2, 3, 1) if d.nhwc else a)
        self.dv[v] = d
        for xs in self.need_i8.get(v, []):
            d.i8[xs] = self._quantize_to(d, xs)
        return d

    def _src(self, v: "Value") -> DevValue:
        if v in self.consts:
            return self._const_dv(v)
        return self.dv[v]

    def _add(self, name: str, fn: Callable[[int], None], nbytes: int = 0, nops: int = 0) -> None:
        """Append a launch; nbytes/nops are its algorithmic HBM bytes and integer ops (each
        operand read once, each result written once; 2 ops per multiply-accumulate)."""
        self.launches.append((name, fn))
        self.launch_cost.append((name, int(nbytes), int(nops)))
        self.kernel_counts[name] = self.kernel_counts.get(name, 0) + 1

    @staticmethod
    def _epi_bytes(e, rows: int, cols: int) -> int:
        """Bytes the epilogue moves: full-shape operands read, f32/int8 results written."""
        n = 8 * cols if e.scale else 0
        full_b = 2 if e.flags & L.EPI_FULL_H16 else 4
        for i in range(e.n_steps):
            st = e.steps[i]
            if st.fn not in _UNARY_CODES:
                n += {L.BC_SCALAR: 4, L.BC_COL: 4 * cols, L.BC_ROW: 4 * rows, L.BC_FULL: full_b * rows * cols}[st.mode]
        if e.out_f32:
            n += (2 if e.flags & L.EPI_OUT_H16 else 4) * rows * cols
        if e.out_i8:
            n += rows * cols
        return n

    # ---------------------------------------------------------------- int8 copies

    def _quantize_to(self, d: DevValue, xs: float):
        """Schedule a standalone quantize of d's f32 copy (mira/ops.py:602-603)."""
        torch = _t()
        if d.half:
            raise L.RocmError("internal: a half-stored value has no standalone quantize")
        ld = d.i8_ld()
        q = torch.empty((d.rows, ld), dtype=torch.int8, device=self.dev)
        lib, src, rows, cols = self.lib, d.f32, d.rows, d.cols
        self._add("quantize", lambda s: L.check(lib.mr_quantize_rows(src.data_ptr(), rows, cols, cols, q.data_ptr(),
                                                                     ld, xs, s), "mr_quantize_rows"),
                  nbytes=4 * rows * cols + rows * ld)
        return q, ld

    def _finish_i8(self, d: DevValue, fused: Optional[float]) -> None:
        """int8 copies the producer did not write itself come from its f32 copy."""
        for xs in self.need_i8.get(d.value, []):
            if xs != fused and xs not in d.i8:
                d.i8[xs] = self._quantize_to(d, xs)

    # ---------------------------------------------------------------- epilogue descriptors

    def _epilogue(self, op: "Op", out: DevValue, is_conv: bool, first: int, scale) -> tuple:
        """Build the mr_epilogue for `op` writing into `out` (f32 and the first int8 copy)."""
        e = L.Epilogue()
        steps = op.attrs.get("epilogue", ())
        if len(steps) > L.MAX_EPI:
            raise L.RocmError(f"epilogue has {len(steps)} steps; the kernels take at most {L.MAX_EPI}")
        rshape = op.result.type.shape
        e.n_steps = len(steps)
        e.flags = L.EPI_OUT_F16 if op.result.type.dtype == "f16" else 0
        if out.half:
            e.flags |= L.EPI_OUT_H16
        for i, (fn, idx, sw) in enumerate(steps):
            st = e.steps[i]
            st.fn = L.EPI_FN[fn]
            st.swapped = int(bool(sw))
            if idx is None:
                continue
            v = op.inputs[idx]
            if v in self.consts:
                mode, t, ld = self._const_operand(v, rshape, is_conv)
            else:
                mode = _bcast_mode(v.type.shape, rshape, is_conv)
                t = self.dv[v].f32
                ld = out.cols if mode == L.BC_FULL else 1
                if self.dv[v].half:
                    if mode != L.BC_FULL:
                        raise L.RocmError(f"{op.kind}: a half-stored operand must be full-shape")
                    e.flags |= L.EPI_FULL_H16
            st.mode, st.ptr, st.ld = mode, t.data_ptr(), ld
        e.scale = _ptr(scale)
        e.out_f32 = _ptr(out.f32)
        e.ldo = out.cols
        fused = None
        wants = self.need_i8.get(out.value, [])
        if wants:
            fused = wants[0]
            q = _t().empty((out.rows, out.i8_ld()), dtype=_t().int8, device=self.dev)
            out.i8[fused] = (q, out.i8_ld())
            e.out_i8 = q.data_ptr()
            e.ldq = out.i8_ld()
            e.out_xs = fused
        if out.f32 is None and not wants:
            raise L.RocmError(f"{op.kind} result is never read")
        self.keep.append(e)
        return e, fused

    def _const_operand(self, v: "Value", rshape: tuple, is_conv: bool):
        a = self._const_value(v).astype(np.float32)
        mode = _bcast_mode(a.shape, rshape, is_conv)
        if mode is None:                     # partial broadcast: materialize the full operand
            a = np.broadcast_to(a, rshape)
            mode = L.BC_FULL
        if mode == L.BC_SCALAR:
            return mode, self._upload(a.reshape(1)), 0
        if mode in (L.BC_COL, L.BC_ROW):
            return mode, self._upload(a.reshape(-1)), 1
        full = np.broadcast_to(a, rshape)
        if is_conv:
            full = full.transpose(0, 2, 3, 1)
        cols = rshape[1] if is_conv else rshape[-1]
        return L.BC_FULL, self._upload(np.ascontiguousarray(full).reshape(-1, cols)), cols

    # ---------------------------------------------------------------- emitters

    def _acc_buffer(self, op: "Op", rows: int, cols: int):
        if not self.target.debug_acc:
            return None
        t = _t().empty((rows, cols), dtype=_t().int32, device=self.dev)
        self.acc[op.result] = t
        return t

    def _emit_qmatmul_group(self, ops: list) -> None:
        """One launch for q-ops sharing their int8 input (planned by _plan_shared_input_matmuls):
        the weights packed side by side, each result a column slice of the output rows."""
        torch = _t()
        xs = _f32key(ops[0].attrs["x_scale"])
        ln = self.lnin.get(ops[0])
        if ln is None:
            x = self._src(ops[0].inputs[0])
            xq, lda = x.i8[xs] if xs in x.i8 else self._quantize_to(x, xs)
        q = np.concatenate([np.asarray(op.attrs["q"], np.int8) for op in ops], axis=1)
        ws = np.concatenate([np.asarray(op.attrs["w_scale"], np.float32).reshape(-1) for op in ops])
        K, N = q.shape
        bl = pack.pack_matmul(q)
        b = self._upload(pack.device_weights(bl))
        scale = self._upload(pack.combined_scale(ops[0].attrs["x_scale"], ws))
        M = int(np.prod(ops[0].result.type.shape[:-1], dtype=np.int64))
        y = torch.empty((M, N), dtype=torch.float32, device=self.dev)
        at = 0
        for op in ops:
            n = op.result.type.shape[-1]
            self.dv[op.result] = DevValue(op.result, nhwc=False, f32=y[:, at:at + n])
            at += n
        e = L.Epilogue()
        e.scale, e.out_f32, e.ldo = scale.data_ptr(), y.data_ptr(), N
        self.keep.append(e)
        lib, kp, npad = self.lib, bl.shape[1], bl.shape[0]
        if ln is not None:
            self._add("qmatmul", self._lnin_launch(ln, xs, b, kp, npad, M, N, K, e),
                      nbytes=4 * M * K + 8 * K + K * N + 8 * N + 4 * M * N, nops=2 * M * N * K)
        else:
            self._add("qmatmul", lambda s: L.check(
                lib.mr_qmatmul(xq.data_ptr(), lda, b.data_ptr(), kp, npad, M, N, K, C.byref(e), s), "mr_qmatmul"),
                nbytes=M * K + K * N + 8 * N + 4 * M * N, nops=2 * M * N * K)

    def _emit_qmatmul(self, op: "Op") -> None:
        if op in self.row_group:
            return self._emit_qmatmul_group(self.row_group[op])
        a = op.attrs
        q = np.asarray(a["q"], np.int8)
        K, N = q.shape
        xs = _f32key(a["x_scale"])
        if op in self.f32in:
            return self._emit_qmatmul_f32in(op, self.staging[self.f32in[op]])
        ln = self.lnin.get(op)
        if ln is None:
            x = self._src(op.inputs[0])
            xq, lda = x.i8[xs] if xs in x.i8 else self._quantize_to(x, xs)
        bl = pack.pack_matmul(q)
        b = self._upload(pack.device_weights(bl))
        scale = self._upload(pack.combined_scale(a["x_scale"], a["w_scale"]))
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, False, 1, scale)
        acc = self._acc_buffer(op, out.rows, N)
        if acc is not None:
            e.out_acc, e.ldacc = acc.data_ptr(), N
        M = out.rows
        lib, kp, npad = self.lib, bl.shape[1], bl.shape[0]
        if ln is not None:
            self._add("qmatmul", self._lnin_launch(ln, xs, b, kp, npad, M, N, K, e),
                      nbytes=4 * M * K + 8 * K + K * N + self._epi_bytes(e, M, N), nops=2 * M * N * K)
        else:
            self._add("qmatmul", lambda s: L.check(
                lib.mr_qmatmul(xq.data_ptr(), lda, b.data_ptr(), kp, npad, M, N, K, C.byref(e), s), "mr_qmatmul"),
                nbytes=M * K + K * N + self._epi_bytes(e, M, N), nops=2 * M * N * K)
        self._finish_i8(out, fused)

    def _emit_qmatmul_f32in(self, op: "Op", x) -> None:
        """A qmatmul whose input is the f32 rows x (planned by _plan_f32in_matmuls)."""
        a = op.attrs
        q = np.asarray(a["q"], np.int8)
        K, N = q.shape
        bl = pack.pack_matmul(q)
        b = self._upload(pack.device_weights(bl))
        scale = self._upload(pack.combined_scale(a["x_scale"], a["w_scale"]))
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, False, 1, scale)
        acc = self._acc_buffer(op, out.rows, N)
        if acc is not None:
            e.out_acc, e.ldacc = acc.data_ptr(), N
        M = out.rows
        xs = _f32key(a["x_scale"])
        lib, kp, npad = self.lib, bl.shape[1], bl.shape[0]
        self._add("qmatmul", lambda s: L.check(
            lib.mr_qmatmul_f32in(x.data_ptr(), K, xs, b.data_ptr(), kp, npad, M, N, K, C.byref(e), s),
            "mr_qmatmul_f32in"), nbytes=4 * M * K + K * N + self._epi_bytes(e, M, N), nops=2 * M * N * K)
        self._finish_i8(out, fused)

    def _emit_matmul(self, op: "Op") -> None:
        w = op.inputs[1]
        if self._producer(w) is not None and self._producer(w).kind == "dequantize":
            return self._emit_w8_matmul(op)
        if op in self.attn:
            return self._emit_attention(op)
        return self._emit_bmm(op)

    def _emit_attention(self, op: "Op") -> None:
        """The fused decode attention planned by _plan_attention, at its context matmul.  When
        the context feeds an int8 consumer through a head-merging view ([B, H, 1, hd] ->
        [B, 1, H, hd] -> [B, D]), the kernel writes that int8 copy too."""
        torch = _t()
        a = self.attn[op]
        Bn, H, hd, T = a["B"], a["H"], a["hd"], a["T"]
        D = H * hd
        q, kc, vc = self._c_order(a["q"]), self._c_order(a["kc"]), self._c_order(a["vc"])
        kn, vn, mask = self._c_order(a["kn"]), self._c_order(a["vn"]), self._c_order(a["mask"])
        if kc.stride() != vc.stride() or kc.stride(2) != 1 or q.stride(1) != 1 or kn.stride(1) != 1 or \
                vn.stride(1) != 1 or not mask.is_contiguous():
            raise L.RocmError("attention operands are not row-major views")
        out = self._new_dv(op.result)
        if out.f32 is None:
            out.f32 = torch.empty(op.result.type.shape, dtype=torch.float32, device=self.dev)
        y = out.f32
        q8, ld8, xs = None, 0, 1.0
        t = self.users.get(op.result, [])
        if len(t) == 1 and t[0].kind == "transpose" and tuple(t[0].attrs["perm"]) == (0, 2, 1, 3):
            rs = self.users.get(t[0].result, [])
            if len(rs) == 1 and rs[0].kind == "reshape" and tuple(rs[0].result.type.shape) == (Bn, D):
                r = rs[0].result
                wants = self.need_i8.get(r, [])
                if wants:
                    xs, ld8 = wants[0], pack.row_stride_for(D)
                    q8 = torch.empty((Bn, ld8), dtype=torch.int8, device=self.dev)
                    self.i8_preset[r] = {xs: (q8, ld8)}
        lib, scale = self.lib, a["scale"]
        c_ld, c_bs = kc.stride(1), kc.stride(0)
        args = (q, q.stride(0), kc, vc, c_ld, c_bs, kn, kn.stride(0), vn, vn.stride(0), mask, scale, Bn, H, hd, T, y,
                D, q8, ld8, xs)
        self.keep.append(args)
        self._add("attention", lambda s: L.check(lib.mr_attention_decode_f32(
            args[0].data_ptr(), args[1], args[2].data_ptr(), args[3].data_ptr(), c_ld, c_bs, args[6].data_ptr(),
            args[7], args[8].data_ptr(), args[9], args[10].data_ptr(), scale, Bn, H, hd, T, y.data_ptr(), D,
            _ptr(q8), ld8, xs, s), "mr_attention_decode_f32"),
            nbytes=4 * (2 * Bn * (T + 1) * D + Bn * D + (T + 1)) + 4 * Bn * D + (Bn * ld8 if q8 is not None else 0),
            nops=4 * Bn * (T + 1) * D)
        self._finish_i8(out, None)

    def _emit_w8_matmul(self, op: "Op") -> None:
        """Weight-only int8 matmul (checked by _check_w8_matmul): the int8 weights are packed
        and uploaded once with their f32 scales; each run streams them through the
        mr_w8_matmul_f32 kernel."""
        x = self._src(op.inputs[0])
        w = self.consts[op.inputs[1]].attrs
        q = np.asarray(w["q"], np.int8)
        K, N = q.shape
        bl = pack.pack_matmul(q)
        b = self._upload(pack.device_weights(bl))
        ws = self._upload(np.asarray(w["scale"], np.float32).reshape(-1))
        w16 = int(w["dtype"] == "f16")        # mira/ops.py:584 casts the dequantized weight to its dtype
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, False, 2, None)
        M = out.rows
        lib, kp, npad, xf = self.lib, bl.shape[1], bl.shape[0], x.f32
        self._add("w8matmul", lambda s: L.check(
            lib.mr_w8_matmul_f32(xf.data_ptr(), K, b.data_ptr(), ws.data_ptr(), w16, kp, npad, M, N, K, C.byref(e),
                                 s),
            "mr_w8_matmul_f32"), nbytes=4 * M * K + K * N + 4 * N + self._epi_bytes(e, M, N))
        self._finish_i8(out, fused)

    def _emit_qconv2d(self, op: "Op") -> None:
        a = op.attrs
        xv = op.inputs[0]
        x = self._src(xv)
        q = np.asarray(a["q"], np.int8)
        n, c, h, w = xv.type.shape
        o, _, kh, kw = q.shape
        (sh, sw), (ph, pw), (dh, dw), _ = conv_params(a)
        oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(w, kw, sw, pw, dw)
        xs = _f32key(a["x_scale"])
        if xs in x.i8:
            xq, cp = x.i8[xs]
        else:
            xq, cp = self._quantize_to(x, xs)
        bl = pack.pack_conv(q, cp)
        b = self._upload(pack.device_weights(bl))
        scale = self._upload(pack.combined_scale(a["x_scale"], a["w_scale"]))
        geom = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=kh, kw=kw, sh=sh, sw=sw, ph=ph,
                          pw=pw, dh=dh, dw=dw)
        self.keep.append(geom)
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, True, 1, scale)
        acc = self._acc_buffer(op, out.rows, o)
        if acc is not None:
            e.out_acc, e.ldacc = acc.data_ptr(), o
        lib, kp, npad = self.lib, bl.shape[1], bl.shape[0]
        rows = n * oh * ow
        self._add("qconv2d", lambda s: L.check(
            lib.mr_qconv2d(xq.data_ptr(), C.byref(geom), b.data_ptr(), kp, npad, C.byref(e), s), "mr_qconv2d"),
            nbytes=n * h * w * c + o * c * kh * kw + self._epi_bytes(e, rows, o), nops=2 * rows * o * c * kh * kw)
        self._finish_i8(out, fused)

    def _emit_w8_conv2d(self, op: "Op") -> None:
        """Weight-only int8 convolution (checked by _check_w8_conv2d): the int8 weights are
        packed with a 16-channel-multiple tap stride and uploaded once with their f32 scales;
        each run is one mr_w8_conv2d_f32 implicit GEMM over the NHWC f32 image."""
        a = op.attrs
        xv = op.inputs[0]
        n, c, h, w = xv.type.shape
        wa = self.consts[op.inputs[1]].attrs
        q = np.asarray(wa["q"], np.int8)
        o, _, kh, kw = q.shape
        (sh, sw), (ph, pw), (dh, dw), _ = conv_params(a)
        _, _, oh, ow = op.result.type.shape
        lib = self.lib
        if c % 4:
            # a graph input of c channels (checked): an NHWC copy with the channels padded to
            # 4, and zero weights for them
            c4 = pack.roundup(c, 4)
            stage = self.staging[xv]
            xt = _t().empty((n, h, w, c4), dtype=_t().float32, device=self.dev)
            # c is rebound to c4 below: the launch takes the input's own count as a default
            self._add("input", lambda s, c=c: L.check(lib.mr_nchw_to_nhwc_pad_f32(stage.data_ptr(), n, c, h, w,
                                                                                   xt.data_ptr(), c4, s),
                                                      "mr_nchw_to_nhwc_pad_f32"), nbytes=4 * n * h * w * (c + c4))
            q = np.concatenate([q, np.zeros((o, c4 - c, kh, kw), np.int8)], axis=1)
            c = c4
        else:
            xt = self._src(xv).f32
        cp = pack.roundup(c, 16)                   # the packed taps' channel stride
        bl = pack.pack_conv(q, cp)
        b = self._upload(pack.device_weights(bl))
        ws = self._upload(np.asarray(wa["scale"], np.float32).reshape(-1))
        w16 = int(wa["dtype"] == "f16")
        geom = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=kh, kw=kw, sh=sh, sw=sw, ph=ph, pw=pw,
                          dh=dh, dw=dw)
        self.keep.append(geom)
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, True, 2, None)
        kp, npad = bl.shape[1], bl.shape[0]
        rows = n * oh * ow
        self._add("w8conv2d", lambda s: L.check(
            lib.mr_w8_conv2d_f32(xt.data_ptr(), C.byref(geom), b.data_ptr(), ws.data_ptr(), w16, kp, npad, C.byref(e),
                                 s), "mr_w8_conv2d_f32"),
            nbytes=4 * n * c * h * w + o * c * kh * kw + 4 * o + self._epi_bytes(e, rows, o),
            nops=2 * rows * o * c * kh * kw)
        self._finish_i8(out, fused)

    def _emit_conv2d(self, op: "Op") -> None:
        """Depthwise f32 convolution (groups == C, one filter per channel); a weight-only
        int8 convolution goes to _emit_w8_conv2d, and one fused with the 1x1 expansion
        before it (_plan_expand_dw) to _emit_expand_dw."""
        if op in self.expand_dw:
            return self._emit_expand_dw(op, self.expand_dw[op])
        wp = self._producer(op.inputs[1])
        if wp is not None and wp.kind == "dequantize" and conv_params(op.attrs)[3] == 1:
            return self._emit_w8_conv2d(op)
        a = op.attrs
        xv = op.inputs[0]
        x = self._src(xv)
        n, c, h, w = xv.type.shape
        wt = self._const_value(op.inputs[1]).astype(np.float32)        # [C, 1, KH, KW]
        _, _, kh, kw = wt.shape
        (sh, sw), (ph, pw), (dh, dw), _ = conv_params(a)
        oh, ow = conv_out(h, kh, sh, ph, dh), conv_out(w, kw, sw, pw, dw)
        wdev = self._upload(np.ascontiguousarray(wt[:, 0].transpose(1, 2, 0)))   # [KH, KW, C]
        geom = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=c, o=c, oh=oh, ow=ow, kh=kh, kw=kw, sh=sh, sw=sw, ph=ph, pw=pw,
                          dh=dh, dw=dw)
        self.keep.append(geom)
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, True, 2, None)
        lib, xt = self.lib, x.f32
        self._add("dwconv2d", lambda s: L.check(
            lib.mr_dwconv2d_f32(xt.data_ptr(), C.byref(geom), wdev.data_ptr(), C.byref(e), s), "mr_dwconv2d_f32"),
            nbytes=4 * n * c * h * w + 4 * c * kh * kw + self._epi_bytes(e, n * oh * ow, c))
        self._finish_i8(out, fused)

    def _emit_expand_dw(self, op: "Op", ex: "Op") -> None:
        """The expansion q-op `ex` and the depthwise convolution `op` as one mr_qconv1x1_dw3x3
        launch (mr_qstem3x3_dw3x3 when `ex` is a 3x3 stem): the expansion's epilogue has no
        outputs (its result is never stored), the depthwise one writes op's copies."""
        xv = ex.inputs[0]
        x = self._src(xv)
        xs = _f32key(ex.attrs["x_scale"])
        xq, cp = x.i8[xs] if xs in x.i8 else self._quantize_to(x, xs)
        q = np.asarray(ex.attrs["q"], np.int8)
        bl = pack.pack_conv(q, cp)
        b = self._upload(pack.device_weights(bl))
        scale = self._upload(pack.combined_scale(ex.attrs["x_scale"], ex.attrs["w_scale"]))
        ee = L.Epilogue()
        steps = ex.attrs["epilogue"]
        ee.n_steps = len(steps)
        ee.flags = L.EPI_OUT_F16 if ex.result.type.dtype == "f16" else 0
        for i, (fn, idx, _sw) in enumerate(steps):
            ee.steps[i].fn = L.EPI_FN[fn]
            if idx is not None:
                mode, t, ld = self._const_operand(ex.inputs[idx], ex.result.type.shape, True)
                ee.steps[i].mode, ee.steps[i].ptr, ee.steps[i].ld = mode, t.data_ptr(), ld
        ee.scale = scale.data_ptr()
        self.keep.append(ee)
        n, c, h, w = ex.result.type.shape
        _, _, oh, ow = op.result.type.shape
        (s, _), _, _, _ = conv_params(op.attrs)
        wt = self._const_value(op.inputs[1]).astype(np.float32)              # [C, 1, 3, 3]
        wdev = self._upload(np.ascontiguousarray(wt[:, 0].transpose(1, 2, 0)))   # [3, 3, C]
        geom = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=c, o=c, oh=oh, ow=ow, kh=3, kw=3, sh=s, sw=s, ph=1, pw=1, dh=1,
                          dw=1)
        self.keep.append(geom)
        out = self._new_dv(op.result)
        e, fused = self._epilogue(op, out, True, 2, None)
        lib, kp, npad, cin = self.lib, bl.shape[1], bl.shape[0], xv.type.shape[1]
        if q.shape[2:] == (3, 3):
            _, _, hi, wi = xv.type.shape
            (ss, _), _, _, _ = conv_params(ex.attrs)
            sg = L.ConvGeom(n=n, h=hi, w=wi, c=cin, c_pad=cp, o=c, oh=h, ow=w, kh=3, kw=3, sh=ss, sw=ss, ph=1, pw=1,
                            dh=1, dw=1)
            self.keep.append(sg)
            self._add("expand_dw", lambda st: L.check(
                lib.mr_qstem3x3_dw3x3(xq.data_ptr(), C.byref(sg), b.data_ptr(), kp, npad, C.byref(ee), C.byref(geom),
                                      wdev.data_ptr(), C.byref(e), st), "mr_qstem3x3_dw3x3"),
                nbytes=n * hi * wi * cp + c * cin * 9 + 36 * c + self._epi_bytes(e, n * oh * ow, c),
                nops=2 * n * h * w * c * cin * 9)
        else:
            self._add("expand_dw", lambda st: L.check(
                lib.mr_qconv1x1_dw3x3(xq.data_ptr(), cp, b.data_ptr(), kp, npad, cin, C.byref(ee), C.byref(geom),
                                      wdev.data_ptr(), C.byref(e), st), "mr_qconv1x1_dw3x3"),
                nbytes=n * h * w * cp + c * cin + 36 * c + self._epi_bytes(e, n * oh * ow, c),
                nops=2 * n * h * w * c * cin)
        self._finish_i8(out, fused)

    def _emit_fused_stem(self, op: "Op") -> None:
        conv, pad_op = self.fused_stem[op]
        a = conv.attrs
        f32in = self.stem_f32in.get(op)
        x = None if f32in else self._src(conv.inputs[0])
        q = np.asarray(a["q"], np.int8)
        n, c, h, w = conv.inputs[0].type.shape
        o, _, kh, kw = q.shape
        (sh, sw), (ph, pw), (dh, dw), _ = conv_params(a)
        _, _, oh, ow = conv.result.type.shape
        xs = _f32key(a["x_scale"])
        xq, cp = (None, 4) if f32in else x.i8[xs] if xs in x.i8 else self._quantize_to(x, xs)
        bl = pack.pack_conv(q, cp, min_rows=64)
        b = self._upload(pack.device_weights(bl))
        scale = self._upload(pack.combined_scale(a["x_scale"], a["w_scale"]))
        geom = L.ConvGeom(n=n, h=h, w=w, c=c, c_pad=cp, o=o, oh=oh, ow=ow, kh=kh, kw=kw, sh=sh, sw=sw, ph=ph,
                          pw=pw, dh=dh, dw=dw)
        self.keep.append(geom)
        out = self._new_dv(op.result)
        e, fused = self._epilogue(conv, out, True, 1, scale)
        pads = tuple(tuple(p) for p in pad_op.attrs["pads"])
        value = float(np.asarray(pad_op.attrs.get("value", 0)).astype(np.float32))
        size, stride = op.attrs["size"], op.attrs["stride"]
        _, _, poh, pw_ = op.result.type.shape
        lib, kp, npad = self.lib, bl.shape[1], bl.shape[0]
        pt, pl = pads[2][0], pads[3][0]
        out_bytes = o * c * kh * kw + self._epi_bytes(e, n * poh * pw_, o)
        if f32in:
            stage, rf16 = self.staging[f32in[0]], int(f32in[1])
            self._add("qconv2d_maxpool", lambda s: L.check(lib.mr_qconv2d_maxpool_f32in(
                stage.data_ptr(), xs, rf16, C.byref(geom), b.data_ptr(), kp, npad, C.byref(e), size, stride, pt, pl,
                value, poh, pw_, s), "mr_qconv2d_maxpool_f32in"), nbytes=4 * n * h * w * c + out_bytes,
                nops=2 * n * oh * ow * o * c * kh * kw)
        else:
            self._add("qconv2d_maxpool", lambda s: L.check(lib.mr_qconv2d_maxpool(
                xq.data_ptr(), C.byref(geom), b.data_ptr(), kp, npad, C.byref(e), size, stride, pt, pl, value, poh,
                pw_, s), "mr_qconv2d_maxpool"), nbytes=n * h * w * c + out_bytes, nops=2 * n * oh * ow * o * c * kh * kw)
        self._finish_i8(out, fused)

    def _emit_maxpool2d(self, op: "Op") -> None:
        if op in self.fused_stem:
            return self._emit_fused_stem(op)
        v = op.inputs[0]
        pt = pl = 0
        pad_value = 0.0
        if self._producer(v) is not None and self._producer(v) in self.folded_pads:
            p = self._producer(v)
            pads = tuple(tuple(x) for x in p.attrs["pads"])
            pt, pl = pads[2][0], pads[3][0]
            pad_value = float(np.asarray(p.attrs.get("value", 0)).astype(np.float32))
            v = p.inputs[0]
        x = self._src(v)
        n, c, h, w = v.type.shape
        _, _, oh, ow = op.result.type.shape
        k, st = op.attrs["size"], op.attrs["stride"]
        out = self._new_dv(op.result)
        wants = self.need_i8.get(op.result, [])
        fused = wants[0] if wants else None
        yq, cp = None, 0
        if fused is not None:
            cp = out.i8_ld()
            yq = _t().empty((out.rows, cp), dtype=_t().int8, device=self.dev)
            out.i8[fused] = (yq, cp)
        lib, xt, yt = self.lib, x.f32, out.f32
        xsv = fused if fused is not None else 1.0
        self._add("maxpool2d", lambda s: L.check(lib.mr_maxpool2d_f32(
            xt.data_ptr(), n, h, w, c, k, st, pt, pl, pad_value, oh, ow, _ptr(yt), _ptr(yq), cp, xsv, s),
            "mr_maxpool2d_f32"), nbytes=4 * n * h * w * c + (4 if yt is not None else 0) * n * oh * ow * c +
            (n * oh * ow * cp if yq is not None else 0))
        self._finish_i8(out, fused)

    def _emit_pad(self, op: "Op") -> None:
        x = self._src(op.inputs[0])
        n, c, h, w = op.inputs[0].type.shape
        pads = tuple(tuple(p) for p in op.attrs["pads"])
        (t, b), (l, r) = pads[2], pads[3]
        value = float(np.asarray(op.attrs.get("value", 0)).astype(np.float32))
        out = self._new_dv(op.result)
        if out.f32 is None:
            out.f32 = _t().empty((n, h + t + b, w + l + r, c), dtype=_t().float32, device=self.dev)
        lib, xt, yt = self.lib, x.f32, out.f32
        self._add("pad", lambda s: L.check(lib.mr_pad_hw_f32(xt.data_ptr(), n, h, w, c, t, b, l, r, value,
                                                             yt.data_ptr(), s), "mr_pad_hw_f32"),
                  nbytes=4 * n * c * (h * w + (h + t + b) * (w + l + r)))
        self._finish_i8(out, None)

    def _emit_reduce_mean(self, op: "Op") -> None:
        x = self._src(op.inputs[0])
        n, c, h, w = op.inputs[0].type.shape
        out = self._new_dv(op.result)
        f16 = int(op.result.type.dtype == "f16")      # the kernel rounds the mean to f16 first
        wants = self.need_i8.get(op.result, [])
        fused = wants[0] if wants else None
        yq, ld = None, 0
        if fused is not None:
            ld = out.i8_ld()
            yq = _t().empty((out.rows, ld), dtype=_t().int8, device=self.dev)
            out.i8[fused] = (yq, ld)
        lib, xt, yt = self.lib, x.f32, out.f32
        xsv = fused if fused is not None else 1.0
        self._add("mean_hw", lambda s: L.check(lib.mr_mean_hw_f32(
            xt.data_ptr(), n, h * w, c, _ptr(yt), _ptr(yq), ld, xsv, f16, s), "mr_mean_hw_f32"),
            nbytes=4 * n * h * w * c + (4 if yt is not None else 0) * n * c + (n * ld if yq is not None else 0))
        self._finish_i8(out, fused)

    def _round_f16(self, src, dst) -> None:
        """dst = f32(f16(src)) on the device (the reference's .astype(float16))."""
        lib, numel = self.lib, src.numel()
        self._add("round_f16", lambda s: L.check(lib.mr_round_f16_f32(src.data_ptr(), numel, dst.data_ptr(), s),
                                                 "mr_round_f16_f32"), nbytes=8 * numel)

    def _emit_cast(self, op: "Op") -> None:
        """mira/ops.py:405-406 between f32 and f16.  To f16: round (in place on the input
        buffer when the cast is a graph input's only use, see _plan); to f32: the f16
        values are already stored as f32, so the result shares the input's buffers."""
        x = self._src(op.inputs[0])
        r = op.result
        if "i32" in (r.type.dtype, op.inputs[0].type.dtype):     # device loops: through mr_cast_32
            if r.type.dtype == op.inputs[0].type.dtype:
                self.dv[r] = DevValue(r, nhwc=False, f32=x.f32)
                return
            xt = self._c_order(op.inputs[0])
            out, y = self._c_order_out(op)
            lib, n = self.lib, r.type.numel
            src, dst = L.DT[op.inputs[0].type.dtype], L.DT[r.type.dtype]
            self._add("cast", lambda s: L.check(lib.mr_cast_32(xt.data_ptr(), n, src, dst, y.data_ptr(), s),
                                                "mr_cast_32"), nbytes=8 * n)
            self._publish(out, y)
            return
        if op in self.input_casts or r.type.dtype == "f32" or op.inputs[0].type.dtype == "f16":
            self.dv[r] = DevValue(r, nhwc=x.nhwc, f32=x.f32, i8=x.i8)
            self._finish_i8(self.dv[r], None)
            return
        out = self._new_dv(r)
        if out.f32 is None:
            out.f32 = _t().empty_like(x.f32)
        self._round_f16(x.f32, out.f32)
        self._finish_i8(out, None)

    def _emit_reshape(self, op: "Op") -> None:
        torch = _t()
        src_v, r = op.inputs[0], op.result
        x = self._src(src_v)
        d = DevValue(r, nhwc=r in self.images)
        d.i8.update(self.i8_preset.get(r, {}))
        self.dv[r] = d
        if r not in self.need_f32 and r not in self.need_i8:
            return
        s_in = src_v.type.shape
        s_out = r.type.shape
        # NHWC of an [n, c, 1, 1] tensor is the same memory as C order of [n, c]
        same_order = (not x.nhwc and not d.nhwc) or (x.nhwc and s_in[2] * s_in[3] == 1 and not d.nhwc) or \
                     (not x.nhwc and d.nhwc and s_out[2] * s_out[3] == 1) or \
                     (x.nhwc and d.nhwc and s_in[1] == s_out[1] and s_in[2] * s_in[3] == 1)
        if same_order and x.f32 is not None:
            d.f32 = x.f32.view(-1)
        elif x.f32 is not None:
            # go through the canonical (NCHW / C-order) copy
            canon = x.f32
            if x.nhwc:
                n, c, h, w = s_in
                canon = torch.empty((n, c, h, w), dtype=torch.float32, device=self.dev)
                lib, xt, ct = self.lib, x.f32, canon
                self._add("nhwc_to_nchw", lambda s: L.check(lib.mr_nhwc_to_nchw_f32(
                    xt.data_ptr(), n, c, h, w, ct.data_ptr(), s), "mr_nhwc_to_nchw_f32"), nbytes=8 * n * c * h * w)
            if d.nhwc:
                n, c, h, w = r.type.shape
                d.f32 = torch.empty((n, h, w, c), dtype=torch.float32, device=self.dev)
                lib, ct, yt = self.lib, canon, d.f32
                self._add("nchw_to_nhwc", lambda s: L.check(lib.mr_nchw_to_nhwc_f32(
                    ct.data_ptr(), n, c, h, w, yt.data_ptr(), s), "mr_nchw_to_nhwc_f32"), nbytes=8 * n * c * h * w)
            else:
                d.f32 = canon
        else:
            raise L.RocmError("reshape input has no f32 copy")
        if self._i8_view(src_v, r):
            for xs in self.need_i8.get(r, []):
                if xs in x.i8:
                    d.i8[xs] = x.i8[xs]
        self._finish_i8(d, None)

    # ---------------------------------------------------------------- float ops of a decode step

    def _c_order(self, v: "Value"):
        """v's f32 values in the graph's C order (an NHWC image is converted once)."""
        torch = _t()
        d = self._src(v)
        if d.f32 is None:
            raise L.RocmError(f"{v} has no f32 copy on the device")
        if not d.nhwc:
            return d.f32
        if v not in self.canon:
            n, c, h, w = v.type.shape
            t = torch.empty((n, c, h, w), dtype=torch.float32, device=self.dev)
            lib, xt = self.lib, d.f32
            self._add("nhwc_to_nchw", lambda s: L.check(lib.mr_nhwc_to_nchw_f32(
                xt.data_ptr(), n, c, h, w, t.data_ptr(), s), "mr_nhwc_to_nchw_f32"), nbytes=8 * n * c * h * w)
            self.canon[v] = t
        return self.canon[v]

    def _c_order_out(self, op: "Op"):
        """Allocate op's result and return the buffer its kernel writes in C order: the f32
        copy itself, or a temporary that _publish converts when the result is stored NHWC."""
        torch = _t()
        out = self._new_dv(op.result)
        shape = op.result.type.shape
        if out.nhwc:
            return out, torch.empty(shape, dtype=torch.float32, device=self.dev)
        if out.f32 is None:
            out.f32 = torch.empty(shape, dtype=torch.float32, device=self.dev)
        return out, out.f32

    def _publish(self, out: DevValue, t) -> None:
        """Finish a result written in C order: the NHWC copy of an image, then the int8 copies."""
        if out.nhwc:
            torch = _t()
            n, c, h, w = out.value.type.shape
            if out.f32 is None:
                out.f32 = torch.empty((n, h, w, c), dtype=torch.float32, device=self.dev)
            lib, yt = self.lib, out.f32
            self._add("nchw_to_nhwc", lambda s: L.check(lib.mr_nchw_to_nhwc_f32(
                t.data_ptr(), n, c, h, w, yt.data_ptr(), s), "mr_nchw_to_nhwc_f32"), nbytes=8 * n * c * h * w)
        self._finish_i8(out, None)

    def _emit_layernorm(self, op: "Op") -> None:
        """mira/ops.py:356-360, bit-exact; the first int8 copy a q-op consumer needs is written
        by the same kernel."""
        torch = _t()
        xv = op.inputs[0]
        x = self._c_order(xv)
        gm, bt = self._c_order(op.inputs[1]), self._c_order(op.inputs[2])
        d = xv.type.shape[-1]
        rows = xv.type.numel // d
        out = self._new_dv(op.result)
        wants = self.need_i8.get(op.result, [])
        fused = wants[0] if wants and not out.nhwc else None
        yq, ld = None, 0
        if fused is not None:
            ld = out.i8_ld()
            yq = torch.empty((out.rows, ld), dtype=torch.int8, device=self.dev)
            out.i8[fused] = (yq, ld)
        if out.nhwc:
            y = torch.empty(op.result.type.shape, dtype=torch.float32, device=self.dev)
        else:
            if out.f32 is None and yq is None:
                out.f32 = torch.empty(op.result.type.shape, dtype=torch.float32, device=self.dev)
            y = out.f32
        eps, f16 = float(op.attrs["eps"]), int(op.result.type.dtype == "f16")
        lib, xs = self.lib, (fused if fused is not None else 1.0)
        self._add("layernorm", lambda s: L.check(lib.mr_layernorm_f32(
            x.data_ptr(), rows, d, gm.data_ptr(), bt.data_ptr(), eps, f16, _ptr(y), _ptr(yq), ld, xs, s),
            "mr_layernorm_f32"),
            nbytes=4 * rows * d + 8 * d + (4 * rows * d if y is not None else 0) + rows * ld)
        if out.nhwc:
            self._publish(out, y)
        else:
            self._finish_i8(out, fused)

    def _emit_softmax(self, op: "Op") -> None:
        """mira/ops.py:310-313 over the last axis (approx_f32 only)."""
        xv = op.inputs[0]
        x = self._c_order(xv)
        n = xv.type.shape[-1]
        rows = xv.type.numel // n
        out, y = self._c_order_out(op)
        lib, f16 = self.lib, int(op.result.type.dtype == "f16")
        self._add("softmax", lambda s: L.check(lib.mr_softmax_f32(x.data_ptr(), rows, n, f16, y.data_ptr(), s),
                                               "mr_softmax_f32"), nbytes=8 * rows * n)
        self._publish(out, y)

    def _emit_transpose(self, op: "Op") -> None:
        """mira/ops.py:375.  A permutation that keeps the order of the axes longer than 1 moves
        no data: the result shares the input's f32 buffer."""
        xv, r = op.inputs[0], op.result
        x = self._c_order(xv)
        shape, perm = tuple(xv.type.shape), tuple(op.attrs["perm"])
        moved = [p for p in perm if shape[p] != 1]
        if moved == sorted(moved) and r not in self.images:
            d = DevValue(r, nhwc=False, f32=x.view(r.type.shape))
            self.dv[r] = d
            self._finish_i8(d, None)
            return
        rank = len(shape)
        cs = (C.c_int64 * rank)(*shape)
        cp = (C.c_int32 * rank)(*perm)
        self.keep += [cs, cp]
        out, y = self._c_order_out(op)
        lib = self.lib
        self._add("transpose", lambda s: L.check(lib.mr_transpose_f32(x.data_ptr(), rank, cs, cp, y.data_ptr(), s),
                                                 "mr_transpose_f32"), nbytes=8 * xv.type.numel)
        self._publish(out, y)

    def _emit_concat(self, op: "Op") -> None:
        """mira/ops.py:403: each operand's [outer, inner] rows land at their column offset."""
        r = op.result
        rank = r.type.rank
        axis = op.attrs["axis"] % rank
        if op in self.concat_out:
            out = self._new_dv(r)
            out.f32 = y = self.concat_out[op]
        else:
            out, y = self._c_order_out(op)
        outer = int(np.prod(r.type.shape[:axis], dtype=np.int64))
        ld = int(np.prod(r.type.shape[axis:], dtype=np.int64))
        at = 0
        lib = self.lib
        # this op's own buffer has no other writer: its constant pieces (the fixed entries of a
        # window start such as [l, t, 0]) are copied once, here, and never again
        prefill = op not in self.concat_out
        filled = False
        for v in op.inputs:
            inner = int(np.prod(v.type.shape[axis:], dtype=np.int64))
            if outer * inner == 0 or v in self.prealias:      # empty, or already in place
                at += inner
                continue
            x = self._c_order(v)
            if prefill and v in self.consts:
                L.check(lib.mr_copy_rows_f32(x.data_ptr(), outer, inner, y.data_ptr(), ld, at,
                                             _t().cuda.current_stream(self.dev).cuda_stream), "mr_copy_rows_f32")
                filled = True
                at += inner
                continue
            self._add("concat", lambda s, x=x, inner=inner, at=at: L.check(lib.mr_copy_rows_f32(
                x.data_ptr(), outer, inner, y.data_ptr(), ld, at, s), "mr_copy_rows_f32"), nbytes=8 * outer * inner)
            at += inner
        if filled:          # done before any launch, whichever stream that is queued on
            _t().cuda.current_stream(self.dev).synchronize()
        self._publish(out, y)

    def _emit_elementwise(self, op: "Op") -> None:
        """A standalone elementwise op of a device loop (mira/ops.py:163-169): one
        mr_elementwise_f32 launch over the C-order result, operands broadcast by strides."""
        import ctypes as C
        fn = L.EW_FN[op.kind]
        shape = tuple(op.result.type.shape)
        full = (1,) * (4 - len(shape)) + shape

        def operand(v):
            """v's buffer as a view of v's shape and its element strides padded to rank 4
            (0 on broadcast axes); a strided view (a column slice of a shared-input q-op's
            result) is read through its own strides."""
            t = self._c_order(v)
            try:
                t = t.view(v.type.shape) if tuple(t.shape) != tuple(v.type.shape) else t
            except RuntimeError:
                raise L.RocmError(f"elementwise operand {v} is not addressable as {v.type}") from None
            vs = (1,) * (4 - v.type.rank) + tuple(v.type.shape)
            ts = (0,) * (4 - v.type.rank) + tuple(t.stride())
            return t, (C.c_int64 * 4)(*[0 if d == 1 else st for d, st in zip(vs, ts)])

        a, sa = operand(op.inputs[0])
        b, sb = operand(op.inputs[1]) if op.kind not in L.EW_UNARY else (None, (C.c_int64 * 4)(0, 0, 0, 0))
        sh = (C.c_int64 * 4)(*full)
        self.keep += [sa, sb, sh]
        out, y = self._c_order_out(op)
        lib, f16 = self.lib, int(op.result.type.dtype == "f16")
        n = op.result.type.numel
        nbytes = 4 * (a.numel() + (b.numel() if b is not None else 0) + n)
        if op.inputs[0].type.dtype == "i32":
            self._add("elementwise", lambda s: L.check(lib.mr_elementwise_i32(fn, a.data_ptr(), sa, _ptr(b), sb,
                                                                              y.data_ptr(), sh, s),
                                                       "mr_elementwise_i32"), nbytes=nbytes)
        else:
            self._add("elementwise", lambda s: L.check(lib.mr_elementwise_f32(fn, a.data_ptr(), sa, _ptr(b), sb,
                                                                              y.data_ptr(), sh, f16, s),
                                                       "mr_elementwise_f32"), nbytes=nbytes)
        self._publish(out, y)

    @staticmethod
    def _shape4(shape) -> object:
        import ctypes as C
        return (C.c_int64 * 4)(*((1,) * (4 - len(shape)) + tuple(shape)))

    def _bcast4(self, v, full) -> tuple:
        """v's C-order buffer and its element strides broadcast onto `full` (rank <= 4)."""
        import ctypes as C
        t = self._c_order(v)
        try:
            t = t.view(v.type.shape) if tuple(t.shape) != tuple(v.type.shape) else t
        except RuntimeError:
            raise L.RocmError(f"operand {v} is not addressable as {v.type}") from None
        vs = (1,) * (4 - v.type.rank) + tuple(v.type.shape)
        ts = (0,) * (4 - v.type.rank) + tuple(t.stride())
        st = (C.c_int64 * 4)(*[0 if d == 1 else x for d, x in zip(vs, ts)])
        self.keep.append(st)
        return t, st

    def _emit_gather(self, op: "Op") -> None:
        """mira/ops.py:479-484 along axis 0: rows of the table picked by i32 indices."""
        table, idx, r = op.inputs[0], op.inputs[1], op.result
        tt, it = self._c_order(table), self._c_order(idx)
        rows = table.type.shape[0]
        row = int(np.prod(table.type.shape[1:], dtype=np.int64))
        out, y = self._c_order_out(op)
        lib, n_idx = self.lib, idx.type.numel
        self._add("gather", lambda s: L.check(lib.mr_gather_rows_32(tt.data_ptr(), rows, row, it.data_ptr(), n_idx,
                                                                    y.data_ptr(), s), "mr_gather_rows_32"),
                  nbytes=4 * (n_idx + 2 * n_idx * row))
        self._publish(out, y)

    def _window_start(self, start_v) -> object:
        return self._c_order(start_v)

    def _emit_dynamic_slice(self, op: "Op") -> None:
        """mira/ops.py:551-554: the window at a runtime start (an i32 vector on the device)."""
        x, r = op.inputs[0], op.result
        xt, st = self._c_order(x), self._window_start(op.inputs[1])
        shape, size = self._shape4(x.type.shape), self._shape4(op.attrs["size"])
        self.keep += [shape, size]
        out, y = self._c_order_out(op)
        lib, rank = self.lib, x.type.rank
        self._add("dynamic_slice", lambda s: L.check(lib.mr_dynamic_slice_32(
            xt.data_ptr(), shape, st.data_ptr(), rank, size, y.data_ptr(), s), "mr_dynamic_slice_32"),
            nbytes=8 * r.type.numel)
        self._publish(out, y)

    def _emit_slice(self, op: "Op") -> None:
        """mira/ops.py:457-458: a static window, through the dynamic-slice kernel with a
        constant start."""
        x, r = op.inputs[0], op.result
        xt = self._c_order(x)
        begin, sz, full = list(op.attrs["begin"]), list(op.attrs["size"]), list(x.type.shape)
        # a window that is one contiguous run of x's C-order buffer (size-1 axes, then one
        # partial axis, then whole axes) is a view of it, as reshape is
        a = next((i for i, z in enumerate(sz) if z != 1), len(sz))
        if r not in self.images and xt.is_contiguous() and \
                all(begin[i] == 0 and sz[i] == full[i] for i in range(a + 1, len(sz))):
            off = sum(b * int(np.prod(full[i + 1:], dtype=np.int64)) for i, b in enumerate(begin))
            self.dv[r] = DevValue(r, nhwc=False, f32=xt.reshape(-1).narrow(0, off, r.type.numel).view(r.type.shape))
            self._finish_i8(self.dv[r], None)
            return
        st = self._upload(np.asarray(op.attrs["begin"], np.int32))
        shape, size = self._shape4(x.type.shape), self._shape4(op.attrs["size"])
        self.keep += [shape, size]
        out, y = self._c_order_out(op)
        lib, rank = self.lib, x.type.rank
        self._add("slice", lambda s: L.check(lib.mr_dynamic_slice_32(
            xt.data_ptr(), shape, st.data_ptr(), rank, size, y.data_ptr(), s), "mr_dynamic_slice_32"),
            nbytes=8 * r.type.numel)
        self._publish(out, y)

    def _emit_dynamic_update_slice(self, op: "Op") -> None:
        """mira/ops.py:567-572: a copy of x with the window at a runtime start replaced."""
        x, upd, r = op.inputs[0], op.inputs[1], op.result
        xt, ut, st = self._c_order(x), self._c_order(upd), self._window_start(op.inputs[2])
        shape, size = self._shape4(x.type.shape), self._shape4(upd.type.shape)
        self.keep += [shape, size]
        out, y = self._c_order_out(op)
        lib, rank = self.lib, x.type.rank
        self._add("dynamic_update_slice", lambda s: L.check(lib.mr_dynamic_update_slice_32(
            xt.data_ptr(), shape, ut.data_ptr(), size, st.data_ptr(), rank, y.data_ptr(), s),
            "mr_dynamic_update_slice_32"), nbytes=8 * r.type.numel)
        self._publish(out, y)

    def _emit_argmax(self, op: "Op") -> None:
        """mira/ops.py:527-528 over the last axis (first maximum, first NaN)."""
        x, r = op.inputs[0], op.result
        xt = self._c_order(x)
        n = x.type.shape[-1]
        rows = x.type.numel // n
        out, y = self._c_order_out(op)
        lib = self.lib
        self._add("argmax", lambda s: L.check(lib.mr_argmax_f32(xt.data_ptr(), rows, n, y.data_ptr(), s),
                                              "mr_argmax_f32"), nbytes=4 * (rows * n + rows))
        self._publish(out, y)

    def _emit_where(self, op: "Op") -> None:
        """mira/ops.py:432-433, the three operands broadcast by strides."""
        full = tuple(op.result.type.shape)
        (ct, cs), (at, as_), (bt, bs) = (self._bcast4(v, full) for v in op.inputs)
        sh = self._shape4(full)
        self.keep.append(sh)
        out, y = self._c_order_out(op)
        lib, cint = self.lib, int(op.inputs[0].type.dtype == "i32")
        self._add("where", lambda s: L.check(lib.mr_where_32(ct.data_ptr(), cint, cs, at.data_ptr(), as_,
                                                             bt.data_ptr(), bs, y.data_ptr(), sh, s), "mr_where_32"),
                  nbytes=16 * op.result.type.numel)
        self._publish(out, y)

    def _loop_results(self, op: "Op") -> list:
        torch = _t()
        outs = []
        for r in op.results:
            d = self._new_dv(r)
            if d.f32 is None:
                d.f32 = torch.empty(r.type.shape, dtype=torch.float32, device=self.dev)
            outs.append(d)
        return outs

    @staticmethod
    def _feed(sub: "RocmExecutable", values: list) -> None:
        for ph, t in zip(sub.g.inputs, values):
            if ph not in sub.bound:
                sub.device_input(ph).copy_(t.reshape(ph.type.shape))

    def _loop_body(self, body_g: "Graph", state: list, caps: list) -> "RocmExecutable":
        """The body sub-executable reading the loop state and captures in place.  Its outputs
        are copied into the state one after another, so an output stored in another slot's
        buffer would be read after that slot was overwritten: such a body gets staging
        buffers of its own instead."""
        body = RocmExecutable(body_g, self.target, in_loop=True, bind=dict(zip(body_g.inputs, state + caps)))
        for k, o in enumerate(body_g.outputs):
            p = body.device_output(o).untyped_storage().data_ptr()
            if any(j != k and t.untyped_storage().data_ptr() == p for j, t in enumerate(state)):
                return RocmExecutable(body_g, self.target, in_loop=True)
        return body

    def _emit_while(self, op: "Op") -> None:
        """A while op run on the device (mira/backends/cpu.py:44-51's semantics): the loop
        state lives in the op's result buffers, which the cond and body sub-executables read in
        place, as they read the captures; each iteration runs the cond, reads its one-element
        result back, and if it is non-zero runs the body and copies its outputs into the state.
        Nothing but that flag leaves the GPU; reading it synchronises the stream, so an
        executable holding a device loop is not captured into a HIP graph.  With the target's
        graph_loops, the two steps (copies and launches) are recorded as HIP graphs after the first iteration, which ran them eagerly,
        and replayed from then on; every buffer they touch is fixed at planning, so a replay
        does what the eager step does.  Sub-graphs that hold control ops of their own read
        flags on the host and stay eager."""
        torch = _t()
        ns, nc = op.attrs["n_state"], op.attrs["n_cond"]
        cond_g, body_g = op.attrs["cond"], op.attrs["body"]
        ins = [self._c_order(v) for v in op.inputs]
        init, cond_caps, body_caps = ins[:ns], ins[ns:ns + nc], ins[ns + nc:]
        outs = self._loop_results(op)
        state = [d.f32 for d in outs]
        # both steps read the state and the captures in place: only the body's outputs are
        # copied, into the state, once per iteration
        cond = RocmExecutable(cond_g, self.target, in_loop=True, bind=dict(zip(cond_g.inputs, state + cond_caps)))
        body = self._loop_body(body_g, state, body_caps)
        max_iters = int(op.attrs["max_iters"])
        feed = self._feed
        flag = cond.device_output(cond_g.outputs[0])
        dev = self.dev

        def cond_step() -> None:
            feed(cond, state + cond_caps)
            cond.launch()

        def body_step() -> None:
            feed(body, state + body_caps)
            body.launch()
            for t, o in zip(state, body_g.outputs):
                t.copy_(body.device_output(o).reshape(t.shape))

        steps = [cond_step, body_step]
        capture = self.target.graph_loops and not any(
            o.is_control for sg in (cond_g, body_g) for o in sg.ops)

        def record() -> None:
            graphs = []
            for fn in (cond_step, body_step):
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr):
                    fn()                            # recorded, not run
                graphs.append(gr)
            steps[:] = [gr.replay for gr in graphs]
            self.keep.extend(graphs)

        def run(_stream) -> None:
            for t, src in zip(state, init):
                t.copy_(src.reshape(t.shape))
            for it in range(max_iters):
                steps[0]()
                if not _truthy(flag, cond_g.outputs[0]):
                    return
                steps[1]()
                if it == 0 and capture and steps[0] is cond_step:
                    torch.cuda.current_stream(dev).synchronize()
                    record()
            raise L.RocmError(f"while loop exceeded {max_iters} iterations")

        self.keep += [cond, body]
        self._add("while", run)
        for d in outs:
            self._finish_i8(d, None)

    def _emit_if(self, op: "Op") -> None:
        """An if op run on the device (mira/backends/cpu.py:39-43's semantics): the condition's
        one element is read back, the taken branch's sub-executable runs on its captures and
        its outputs are copied into the op's results."""
        n = op.attrs["n_then"]
        then_g, else_g = op.attrs["then"], op.attrs["else"]
        branches = (RocmExecutable(then_g, self.target, in_loop=True),
                    RocmExecutable(else_g, self.target, in_loop=True))
        ins = [self._c_order(v) for v in op.inputs]
        cond, caps = ins[0], (ins[1:1 + n], ins[1 + n:])
        outs = self._loop_results(op)
        feed = self._feed

        def run(_stream) -> None:
            k = 0 if _truthy(cond, op.inputs[0]) else 1
            sub = branches[k]
            feed(sub, caps[k])
            sub.launch()
            for d, o in zip(outs, sub.g.outputs):
                d.f32.copy_(sub.device_output(o).reshape(d.f32.shape))

        self.keep += list(branches)
        self._add("if", run)
        for d in outs:
            self._finish_i8(d, None)

    def _emit_bmm(self, op: "Op") -> None:
        """f32 matmul of two float tensors with NumPy's batch broadcasting (mira/ops.py:217-219;
        approx_f32 only), the epilogue fused."""
        av, wv = op.inputs[0], op.inputs[1]
        rs = tuple(op.result.type.shape)
        nb = len(rs) - 2
        M, N, K = rs[-2], rs[-1], av.type.shape[-1]

        def operand(v):
            """(C-order base buffer, batch strides broadcast onto the result, last two strides)"""
            base, shape, st, _ = self._view_chain(v)
            t = self._c_order(base)
            pad = len(rs) - len(shape)
            full, fst = (1,) * pad + shape, (0,) * pad + st
            return t, [0 if full[i] == 1 else fst[i] for i in range(nb)], fst[-2], fst[-1]

        a, sa_, sam, sak = operand(av)
        w, sw_, swk, swn = operand(wv)
        bdim = (C.c_int64 * max(nb, 1))(*rs[:nb])
        sa = (C.c_int64 * max(nb, 1))(*sa_)
        sw = (C.c_int64 * max(nb, 1))(*sw_)
        mk = (C.c_int64 * 4)(sam, sak, swk, swn)
        self.keep += [bdim, sa, sw, mk]
        out = self._new_dv(op.result)
        if out.nhwc:
            raise L.RocmError("an f32 matmul result read as an image has no rocm layout")
        e, fused = self._epilogue(op, out, False, 2, None)
        batches = int(np.prod(rs[:nb], dtype=np.int64))
        lib = self.lib
        self._add("bmm_f32", lambda s: L.check(lib.mr_bmm_f32(
            a.data_ptr(), w.data_ptr(), nb, bdim, sa, sw, mk, M, N, K, C.byref(e), s), "mr_bmm_f32"),
            nbytes=4 * (av.type.numel + wv.type.numel) + self._epi_bytes(e, batches * M, N),
            nops=2 * batches * M * N * K)
        self._finish_i8(out, fused)

    # ---------------------------------------------------------------- run

    # bytes per host -> device chunk: the next chunk's copy into pinned memory overlaps the
    # previous chunk's DMA
    UPLOAD_CHUNK = 32 << 20

    def upload(self, feeds: dict) -> None:
        """Copy the segment inputs (host arrays, the graph's layout) into their device buffers,
        through pinned host buffers allocated on first use and kept with the executable: the
        arrays are copied into them in chunks by torch's multi-threaded CPU copy, and each
        chunk's DMA is queued on the current stream as soon as it is there."""
        torch = _t()
        stream = torch.cuda.current_stream(self.dev)
        if self._upload_done is not None:
            self._upload_done.synchronize()       # the pinned buffers are free again
        for v in self.g.inputs:
            if v.type.dtype == "i32":      # held as its bits (device loops)
                arr = np.ascontiguousarray(np.asarray(feeds[v], dtype=np.int32)).view(np.float32).reshape(-1)
            else:
                arr = np.ascontiguousarray(np.asarray(feeds[v], dtype=np.float32)).reshape(-1)
            if arr.size != v.type.numel:
                raise ValueError(f"input {v}: {arr.size} elements for {v.type}")
            pin = self._pinned.get(v)
            if pin is None:
                pin = self._pinned[v] = torch.empty(v.type.numel, dtype=torch.float32, pin_memory=True)
            src = torch.from_numpy(arr)
            stage = self.staging[v]
            if not stage.is_contiguous():     # a slice of a concat's buffer: one strided copy
                pin.copy_(src)
                stage.copy_(pin.view(v.type.shape), non_blocking=True)
                continue
            dst = stage.view(-1)
            step = max(self.UPLOAD_CHUNK // 4, 1)
            for a in range(0, arr.size, step):
                b = min(a + step, arr.size)
                pin[a:b].copy_(src[a:b])
                dst[a:b].copy_(pin[a:b], non_blocking=True)
        self._upload_done = torch.cuda.Event()
        self._upload_done.record(stream)

    def device_input(self, v: "Value"):
        """The device f32 buffer (graph layout) that `launch` reads segment input v from."""
        return self.staging[v]

    def device_output(self, v: "Value"):
        """The device f32 buffer (graph layout) that `launch` leaves output v in; it is rewritten
        by the next launch.  Only for values stored in C order (not NHWC images); the rows of a
        result computed beside others (_plan_shared_input_matmuls) are a strided view."""
        d = self._src(v)
        if d.nhwc or d.f32 is None:
            raise L.RocmError(f"{v} has no C-order f32 copy on the device")
        return d.f32.reshape(v.type.shape)

    def launch(self) -> None:
        """Queue every kernel of the segment on the current stream, starting from the f32 inputs
        already on the device (quantizing them is part of the work)."""
        stream = _t().cuda.current_stream(self.dev).cuda_stream
        for _name, fn in self.launches:
            fn(stream)

    def download(self) -> dict:
        torch = _t()
        out = {}
        for v in self.g.outputs:
            d = self._src(v)
            t = d.f32
            if d.nhwc:
                n, c, h, w = v.type.shape
                canon = torch.empty((n, c, h, w), dtype=torch.float32, device=self.dev)
                L.check(self.lib.mr_nhwc_to_nchw_f32(t.data_ptr(), n, c, h, w, canon.data_ptr(),
                                                     torch.cuda.current_stream(self.dev).cuda_stream),
                        "mr_nhwc_to_nchw_f32")
                t = canon
            host = t.reshape(v.type.shape).cpu().numpy()
            out[v] = host.view(np.int32) if v.type.dtype == "i32" else host.astype(v.type.np_dtype)
        return out

    def run(self, feeds: dict) -> dict:
        """mira/backends/base.py:13-14: host arrays in, finished host arrays out."""
        self.upload(feeds)
        self.launch()
        out = self.download()
        _t().cuda.synchronize(self.dev)
        return out

    def accumulators(self) -> dict:
        """int32 accumulators of every q-op from the last run (needs RocmTarget(debug_acc=True))."""
        return {v: t.cpu().numpy() for v, t in self.acc.items()}

    def device_of(self, v: "Value") -> Optional[str]:
        return "rocm" if v in self.dv else None

    def report(self) -> str:
        ks = ", ".join(f"{k} x{n}" for k, n in sorted(self.kernel_counts.items()))
        return (f"rocm (MI355X gfx950): {len(self.g.compute_ops())} ops -> {len(self.launches)} kernel launches "
                f"[{ks}]; {self.const_bytes / 2**20:.2f} MiB of packed constants on device")


for _kind in L.EW_FN:
    if not hasattr(RocmExecutable, f"_emit_{_kind}"):
        setattr(RocmExecutable, f"_emit_{_kind}", RocmExecutable._emit_elementwise)
