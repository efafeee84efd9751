"""A front end for MIRA's source language (.mira), the subset its CNN / MLP programs use:
the counterpart of mira/lexer.py, mira/parser.py and mira/elaborate.py for the W8A8 path,
producing this harness's graphs.

    program   := function*
    function  := "fn" NAME "(" [param ("," param)*] ")" "->" type "{" statement* "}"
    param     := ["const"] NAME ":" type
    type      := DTYPE ["[" dim ("," dim)* "]"]          DTYPE: f32 | f16
    dim       := integer arithmetic (+ - * /, parentheses) over literals and shape symbols
    statement := "let" NAME "=" expr  |  "return" expr
    expr      := the binary operators + - (loosest), * / @ (tighter), unary -, calls
                 f(arg, ..., name=value), names, numbers, true / false, [lists],
                 parentheses; "#" starts a comment

Elaboration inlines every call of a user function, binding the shape symbols of its
parameter types from the arguments (a symbol seen twice must agree) and checking the
result against the declared return type.  The entry function's plain parameters become
graph inputs; its `const` parameters are weights: given ones are used, the others are
drawn in declaration order from one seeded generator by MIRA's rule
(mira/elaborate.py:196-213, 1114-1123; harness.models.mira_random_weight).

Shape symbols bound in a function are plain numbers in its body, so `reshape(x, [B, C * H * W])`
works.  Builtins, with MIRA's parameter names and defaults (mira/elaborate.py:1081-1111):
relu sigmoid tanh gelu exp abs sqrt (x), maximum / minimum (a, b), matmul(a, b),
softmax(x, axis=-1), mean(x, axis=all, keepdims=false), transpose(x, perm=swap last two),
reshape(x, shape) with one -1 allowed, flatten(x, axis=1),
conv2d(x, w, stride=1, padding=0, dilation=1, groups=1),
maxpool2d / avgpool2d (x, size=2, stride=size, padding=0).
"""
from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Optional

import numpy as np

from harness.graph import Graph, Value
from harness.models import mira_random_weight


class MiraSyntaxError(ValueError):
    """A problem in the program text or its shapes, with its line."""


# ---------------------------------------------------------------- lexer

_TOKEN = re.compile(r"""
    (?P<ws>[ \t\r]+) | (?P<comment>\#[^\n]*) | (?P<nl>\n)
  | (?P<num>\d+\.\d*(?:[eE][+-]?\d+)?|\d+[eE][+-]?\d+|\.\d+(?:[eE][+-]?\d+)?|\d+)
  | (?P<name>[A-Za-z_][A-Za-z_0-9]*)
  | (?P<op>->|[-+*/@=(),:\[\]{}])
""", re.VERBOSE)

KEYWORDS = {"fn", "let", "return", "const"}


@dataclass
class Tok:
    kind: str      # num, name, kw, op, eof
    text: str
    line: int


def tokenize(src: str) -> list[Tok]:
    toks, line, i = [], 1, 0
    while i < len(src):
        m = _TOKEN.match(src, i)
        if not m:
            raise MiraSyntaxError(f"line {line}: unexpected character {src[i]!r}")
        kind = m.lastgroup
        text = m.group()
        if kind == "nl":
            line += 1
        elif kind == "name" and text in KEYWORDS:
            toks.append(Tok("kw", text, line))
        elif kind in ("num", "name", "op"):
            toks.append(Tok(kind, text, line))
        i = m.end()
    toks.append(Tok("eof", "", line))
    return toks


# ---------------------------------------------------------------- syntax tree

@dataclass
class TypeRef:
    dtype: str
    dims: list            # dim expressions (see _parse_dim): int, str, or (op, left, right)


@dataclass
class Param:
    name: str
    type: TypeRef
    const: bool


@dataclass
class Fn:
    name: str
    params: list[Param]
    ret: TypeRef
    body: list            # ("let", name, expr, line) | ("return", expr, line)
    line: int


# expressions: ("num", value) ("name", id) ("neg", e) ("bin", op, a, b) ("call", name, args, kwargs, line)


class _Parser:
    def __init__(self, toks: list[Tok]):
        self.t, self.i = toks, 0

    def peek(self, k: int = 0) -> Tok:
        return self.t[self.i + k]

    def take(self, text: Optional[str] = None, kind: Optional[str] = None) -> Tok:
        tok = self.t[self.i]
        if (text is not None and tok.text != text) or (kind is not None and tok.kind != kind):
            want = repr(text) if text is not None else kind
            raise MiraSyntaxError(f"line {tok.line}: expected {want}, found {tok.text or 'end of file'!r}")
        self.i += 1
        return tok

    def at(self, text: str) -> bool:
        return self.t[self.i].text == text and self.t[self.i].kind in ("op", "kw")

    def program(self) -> dict[str, Fn]:
        fns = {}
        while self.peek().kind != "eof":
            fn = self.function()
            if fn.name in fns:
                raise MiraSyntaxError(f"line {fn.line}: function '{fn.name}' defined twice")
            fns[fn.name] = fn
        return fns

    def function(self) -> Fn:
        line = self.take("fn").line
        name = self.take(kind="name").text
        self.take("(")
        params = []
        while not self.at(")"):
            const = self.peek().text == "const" and self.peek().kind == "kw"
            if const:
                self.take("const")
            pname = self.take(kind="name").text
            self.take(":")
            params.append(Param(pname, self.type_ref(), const))
            if not self.at(")"):
                self.take(",")
        self.take(")")
        self.take("->")
        ret = self.type_ref()
        self.take("{")
        body = []
        while not self.at("}"):
            tok = self.peek()
            if tok.text == "let" and tok.kind == "kw":
                self.take("let")
                lname = self.take(kind="name").text
                self.take("=")
                body.append(("let", lname, self.expr(), tok.line))
            elif tok.text == "return" and tok.kind == "kw":
                self.take("return")
                body.append(("return", self.expr(), tok.line))
            else:
                raise MiraSyntaxError(f"line {tok.line}: expected 'let' or 'return', found {tok.text!r}")
        self.take("}")
        return Fn(name, params, ret, body, line)

    def type_ref(self) -> TypeRef:
        dt = self.take(kind="name")
        if dt.text not in ("f32", "f16"):
            raise MiraSyntaxError(f"line {dt.line}: unsupported element type '{dt.text}' (f32, f16)")
        dims = []
        if self.at("["):
            self.take("[")
            while not self.at("]"):
                dims.append(self.dim_sum())
                if not self.at("]"):
                    self.take(",")
            self.take("]")
        return TypeRef(dt.text, dims)

    def dim_sum(self):
        d = self.dim_prod()
        while self.at("+") or self.at("-"):
            op = self.take().text
            d = (op, d, self.dim_prod())
        return d

    def dim_prod(self):
        d = self.dim_atom()
        while self.at("*") or self.at("/"):
            op = self.take().text
            d = (op, d, self.dim_atom())
        return d

    def dim_atom(self):
        tok = self.peek()
        if tok.kind == "num" and tok.text.isdigit():
            self.take()
            return int(tok.text)
        if tok.kind == "name":
            self.take()
            return tok.text
        if self.at("("):
            self.take("(")
            d = self.dim_sum()
            self.take(")")
            return d
        raise MiraSyntaxError(f"line {tok.line}: bad dimension {tok.text!r}")

    def expr(self):
        e = self.term()
        while self.at("+") or self.at("-"):
            op = self.take().text
            e = ("bin", op, e, self.term())
        return e

    def term(self):
        e = self.unary()
        while self.at("*") or self.at("/") or self.at("@"):
            op = self.take().text
            e = ("bin", op, e, self.unary())
        return e

    def unary(self):
        if self.at("-"):
            self.take("-")
            return ("neg", self.unary())
        return self.primary()

    def primary(self):
        tok = self.peek()
        if tok.kind == "num":
            self.take()
            return ("num", float(tok.text) if any(c in tok.text for c in ".eE") else int(tok.text))
        if self.at("("):
            self.take("(")
            e = self.expr()
            self.take(")")
            return e
        if self.at("["):       # a literal list (shapes, axes, permutations)
            self.take("[")
            items = []
            while not self.at("]"):
                items.append(self.expr())
                if not self.at("]"):
                    self.take(",")
            self.take("]")
            return ("list", items)
        if tok.kind == "name":
            self.take()
            if tok.text in ("true", "false"):
                return ("bool", tok.text == "true")
            if not self.at("("):
                return ("name", tok.text)
            self.take("(")
            args, kwargs = [], {}
            while not self.at(")"):
                if self.peek().kind == "name" and self.peek(1).text == "=":
                    key = self.take().text
                    self.take("=")
                    kwargs[key] = self.expr()
                else:
                    if kwargs:
                        raise MiraSyntaxError(f"line {tok.line}: positional argument after keyword arguments")
                    args.append(self.expr())
                if not self.at(")"):
                    self.take(",")
            self.take(")")
            return ("call", tok.text, args, kwargs, tok.line)
        raise MiraSyntaxError(f"line {tok.line}: unexpected {tok.text or 'end of file'!r}")


def parse(src: str) -> dict[str, Fn]:
    return _Parser(tokenize(src)).program()


# ---------------------------------------------------------------- elaboration

def _eval_dim(d, env: dict, line: int) -> int:
    if isinstance(d, int):
        return d
    if isinstance(d, str):
        if d not in env:
            raise MiraSyntaxError(f"line {line}: shape symbol '{d}' is not bound")
        return env[d]
    op, a, b = d
    x, y = _eval_dim(a, env, line), _eval_dim(b, env, line)
    if op == "/":
        if y == 0 or x % y:
            raise MiraSyntaxError(f"line {line}: dimension {x} / {y} is not a whole number")
        return x // y
    n = {"+": x + y, "-": x - y, "*": x * y}[op]
    if n < 0:
        raise MiraSyntaxError(f"line {line}: dimension evaluates to {n}")
    return n


def _show_dim(d) -> str:
    if isinstance(d, tuple):
        return f"{_show_dim(d[1])} {d[0]} {_show_dim(d[2])}"
    return str(d)


def _show(tref: TypeRef) -> str:
    return f"{tref.dtype}[{', '.join(_show_dim(d) for d in tref.dims)}]"


def _unify(tref: TypeRef, dtype: str, shape: tuple, env: dict, what: str, line: int, computed: bool) -> None:
    """Match a declared type with an actual one (mira/elaborate.py:255-277): plain shape symbols
    bind on first sight and must agree after; computed dims (H / 2) bind nothing and are
    checked only when `computed` is set, once every parameter has been unified."""
    def fail(reason: str) -> MiraSyntaxError:
        return MiraSyntaxError(f"line {line}: {what} has type {dtype}{list(shape)}, "
                               f"expected {_show(tref)} ({reason})")

    if tref.dtype != dtype:
        raise fail(f"{dtype} != {tref.dtype}")
    if len(tref.dims) != len(shape):
        raise fail(f"rank {len(shape)} != {len(tref.dims)}")
    for d, n in zip(tref.dims, shape):
        if isinstance(d, int):
            if d != n:
                raise fail(f"{n} != {d}")
        elif isinstance(d, str):
            if d in env and env[d] != n:
                raise fail(f"{d} is already {env[d]}, got {n}")
            env[d] = n
        elif computed and _eval_dim(d, env, line) != n:
            raise fail(f"{_show_dim(d)} = {_eval_dim(d, env, line)}, got {n}")


_UNARY = ("relu", "sigmoid", "tanh", "gelu", "exp", "abs", "sqrt")
_BINOP = {"+": "add", "-": "sub", "*": "mul", "/": "div"}
MAX_DEPTH = 64


def _num(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _describe(v) -> str:
    if isinstance(v, Value):
        return f"tensor {v.type}"
    return "list" if isinstance(v, list) else f"number {v}"


class Elaborator:
    """Inlines the entry function into one Graph (mira/elaborate.py:186-222 for the entry,
    :279-330 for calls)."""

    def __init__(self, fns: dict[str, Fn], name: str = "main"):
        self.fns = fns
        self.g = Graph(name)
        self.stack: list[str] = []

    # ---- values

    def tensor(self, v, line: int, dtype: str = "f32") -> Value:
        """Tensors pass through; numbers become scalar constants of `dtype`."""
        if isinstance(v, Value):
            return v
        if _num(v):
            return self.g.const(np.array(v, dtype=np.float16 if dtype == "f16" else np.float32))
        raise MiraSyntaxError(f"line {line}: expected a tensor, got {_describe(v)}")

    @staticmethod
    def int_(v, line: int, what: str) -> int:
        if isinstance(v, bool) or not (isinstance(v, int) or (isinstance(v, float) and v.is_integer())):
            raise MiraSyntaxError(f"line {line}: {what} must be a whole number, got {_describe(v)}")
        return int(v)

    def ints(self, v, line: int, what: str) -> list[int]:
        return [self.int_(x, line, what) for x in (v if isinstance(v, list) else [v])]

    def pair(self, v, line: int, what: str) -> tuple:
        xs = self.ints(v, line, what)
        if len(xs) == 1:
            return (xs[0], xs[0])
        if len(xs) != 2:
            raise MiraSyntaxError(f"line {line}: {what} takes one number or two, got {len(xs)}")
        return tuple(xs)

    # ---- functions

    def entry(self, fn_name: str, weights: dict, dims: dict, seed: Optional[int]) -> Graph:
        fn = self.fns.get(fn_name)
        if fn is None:
            raise MiraSyntaxError(f"no function named '{fn_name}' (the entry point)")
        env = dict(dims)
        rng = np.random.default_rng(seed) if seed is not None else None
        args = []
        for p in fn.params:
            for d in p.type.dims:
                if isinstance(d, str) and d not in env:
                    raise MiraSyntaxError(f"line {fn.line}: dimension '{d}' of the entry function needs a value "
                                          f"(dims={{'{d}': ...}})")
            shape = tuple(_eval_dim(d, env, fn.line) for d in p.type.dims)
            npdt = np.float16 if p.type.dtype == "f16" else np.float32
            if p.const:
                if p.name in weights:
                    arr = np.asarray(weights[p.name])
                    if tuple(arr.shape) != shape:
                        raise MiraSyntaxError(f"line {fn.line}: weight '{p.name}' has shape {list(arr.shape)}, "
                                              f"the parameter is {p.type.dtype}{list(shape)}")
                    arr = arr.astype(npdt)
                elif rng is not None:
                    arr = mira_random_weight(rng, shape).astype(npdt)
                else:
                    raise MiraSyntaxError(f"line {fn.line}: no value for const parameter '{p.name}' "
                                          "(pass weights, or a seed for random ones)")
                args.append(self.g.const(arr))
            else:
                args.append(self.g.input(p.name, shape, p.type.dtype))
        unknown = set(weights) - {p.name for p in fn.params if p.const}
        if unknown:
            raise MiraSyntaxError(f"weights given for unknown const parameters: {', '.join(sorted(unknown))}")
        out = self.call_function(fn, args, fn.line, preset=env)
        self.g.outputs = [out]
        return self.g

    def call_function(self, fn: Fn, args: list, line: int, preset: Optional[dict] = None) -> Value:
        if fn.name in self.stack:
            raise MiraSyntaxError(f"line {line}: recursive call to '{fn.name}'")
        if len(self.stack) >= MAX_DEPTH:
            raise MiraSyntaxError(f"line {line}: function calls nested too deeply")
        if len(args) != len(fn.params):
            raise MiraSyntaxError(f"line {line}: '{fn.name}' takes {len(fn.params)} arguments, got {len(args)}")
        env = dict(preset or {})
        scope: dict = {}
        for p, a in zip(fn.params, args):
            if p.const and self.stack:
                raise MiraSyntaxError(f"line {fn.line}: 'const' is only allowed on the entry function's parameters")
            scope[p.name] = a = self.tensor(a, line)
            _unify(p.type, a.type.dtype, a.type.shape, env, f"argument '{p.name}' of '{fn.name}'", line, False)
        for p in fn.params:
            a = scope[p.name]
            _unify(p.type, a.type.dtype, a.type.shape, env, f"argument '{p.name}' of '{fn.name}'", line, True)
        self.stack.append(fn.name)
        scope = {**env, **scope}            # shape symbols are plain numbers inside the body
        for st in fn.body:
            if st[0] == "let":
                scope[st[1]] = self.expr(st[2], scope, st[3])
                continue
            out = self.tensor(self.expr(st[1], scope, st[2]), st[2])
            _unify(fn.ret, out.type.dtype, out.type.shape, env, f"the result of '{fn.name}'", st[2], True)
            self.stack.pop()
            return out
        raise MiraSyntaxError(f"line {fn.line}: '{fn.name}' has no return")

    # ---- expressions

    def expr(self, e, scope: dict, line: int):
        kind = e[0]
        if kind in ("num", "bool"):
            return e[1]
        if kind == "list":
            return [self.expr(x, scope, line) for x in e[1]]
        if kind == "name":
            if e[1] not in scope:
                what = "a function; call it" if e[1] in self.fns or e[1] in BUILTINS else "undefined"
                raise MiraSyntaxError(f"line {line}: '{e[1]}' is {what}")
            return scope[e[1]]
        if kind == "neg":
            v = self.expr(e[1], scope, line)
            if isinstance(v, Value):
                return self.g.op("neg", [v])
            if _num(v):
                return -v
            raise MiraSyntaxError(f"line {line}: cannot negate a {_describe(v)}")
        if kind == "bin":
            return self.binary(e[1], self.expr(e[2], scope, line), self.expr(e[3], scope, line), line)
        _, name, args, kwargs, line = e
        vals = [self.expr(a, scope, line) for a in args]
        kw = {k: self.expr(v, scope, line) for k, v in kwargs.items()}
        if name in self.fns:
            if kw:
                raise MiraSyntaxError(f"line {line}: '{name}' takes no keyword arguments")
            return self.call_function(self.fns[name], vals, line)
        if name not in BUILTINS:
            raise MiraSyntaxError(f"line {line}: unknown function '{name}'")
        params, handler = BUILTINS[name]
        return handler(self, _bind_args(name, params, vals, kw, line), line)

    def binary(self, op: str, a, b, line: int):
        if _num(a) and _num(b):
            if op == "@":
                raise MiraSyntaxError(f"line {line}: '@' needs tensor operands")
            if op == "/":
                if b == 0:
                    raise MiraSyntaxError(f"line {line}: division by zero")
                return a // b if isinstance(a, int) and isinstance(b, int) and a % b == 0 else a / b
            return {"+": a + b, "-": a - b, "*": a * b}[op]
        if not isinstance(a, Value) and not isinstance(b, Value):
            raise MiraSyntaxError(f"line {line}: cannot apply '{op}' to {_describe(a)} and {_describe(b)}")
        dtype = a.type.dtype if isinstance(a, Value) else b.type.dtype
        a, b = self.tensor(a, line, dtype), self.tensor(b, line, dtype)
        try:
            return self.g.op("matmul" if op == "@" else _BINOP[op], [a, b])
        except ValueError as err:
            raise MiraSyntaxError(f"line {line}: {err}") from None

    def op(self, kind: str, ins: list, attrs: dict, line: int) -> Value:
        try:
            return self.g.op(kind, ins, attrs)
        except ValueError as err:
            raise MiraSyntaxError(f"line {line}: {kind}: {err}") from None


# ---------------------------------------------------------------- builtins
# (name, default) parameter lists and handlers, as MIRA's builtin table
# (mira/elaborate.py:1081-1111) declares them for these operators.

_REQUIRED = object()


def _bind_args(name: str, params: list, args: list, kw: dict, line: int) -> dict:
    if len(args) > len(params):
        raise MiraSyntaxError(f"line {line}: {name}() takes at most {len(params)} arguments, got {len(args)}")
    out = dict(zip((p for p, _ in params), args))
    for k, v in kw.items():
        if k not in (p for p, _ in params):
            raise MiraSyntaxError(f"line {line}: {name}() has no argument '{k}'")
        if k in out:
            raise MiraSyntaxError(f"line {line}: {name}() got '{k}' twice")
        out[k] = v
    for p, default in params:
        if p not in out:
            if default is _REQUIRED:
                raise MiraSyntaxError(f"line {line}: {name}() needs '{p}'")
            out[p] = default
    return out


def _unary(kind):
    return [("x", _REQUIRED)], lambda el, a, line: el.op(kind, [el.tensor(a["x"], line)], {}, line)


def _binary_fn(kind):
    def h(el, a, line):
        x, y = a["a"], a["b"]
        if not isinstance(x, Value) and not isinstance(y, Value):
            raise MiraSyntaxError(f"line {line}: {kind}() needs at least one tensor argument")
        dt = x.type.dtype if isinstance(x, Value) else y.type.dtype
        return el.op(kind, [el.tensor(x, line, dt), el.tensor(y, line, dt)], {}, line)
    return [("a", _REQUIRED), ("b", _REQUIRED)], h


def _mean(el, a, line):
    x = el.tensor(a["x"], line)
    axes = list(range(x.type.rank)) if a["axis"] is None else el.ints(a["axis"], line, "axis")
    if not isinstance(a["keepdims"], bool):
        raise MiraSyntaxError(f"line {line}: keepdims must be true or false")
    return el.op("reduce_mean", [x], {"axes": tuple(axes), "keepdims": a["keepdims"]}, line)


def _transpose(el, a, line):
    x = el.tensor(a["x"], line)
    if a["perm"] is None:
        if x.type.rank < 2:
            raise MiraSyntaxError(f"line {line}: transpose() of a rank-{x.type.rank} tensor needs a perm")
        perm = list(range(x.type.rank))
        perm[-2], perm[-1] = perm[-1], perm[-2]
    else:
        perm = el.ints(a["perm"], line, "perm")
    return el.op("transpose", [x], {"perm": tuple(perm)}, line)


def _reshape(el, a, line):
    x = el.tensor(a["x"], line)
    shape = el.ints(a["shape"], line, "shape")
    if shape.count(-1) > 1:
        raise MiraSyntaxError(f"line {line}: reshape: at most one dimension can be -1")
    if -1 in shape:
        known = int(np.prod([d for d in shape if d != -1], dtype=np.int64))
        if known == 0 or x.type.numel % known:
            raise MiraSyntaxError(f"line {line}: reshape: cannot infer -1 for {x.type} -> {shape}")
        shape[shape.index(-1)] = x.type.numel // known
    return el.op("reshape", [x], {"shape": tuple(shape)}, line)


def _flatten(el, a, line):
    x = el.tensor(a["x"], line)
    ax = el.int_(a["axis"], line, "axis")
    if not -(x.type.rank + 1) <= ax <= x.type.rank:
        raise MiraSyntaxError(f"line {line}: flatten axis {ax} out of range for {x.type}")
    ax %= x.type.rank + 1
    lead = int(np.prod(x.type.shape[:ax], dtype=np.int64))
    return el.op("reshape", [x], {"shape": (lead, x.type.numel // max(lead, 1))}, line)


def _conv2d(el, a, line):
    attrs = {"stride": el.pair(a["stride"], line, "stride"), "padding": el.pair(a["padding"], line, "padding")}
    if a["dilation"] != 1:
        attrs["dilation"] = el.pair(a["dilation"], line, "dilation")
    if a["groups"] != 1:
        attrs["groups"] = el.int_(a["groups"], line, "groups")
    return el.op("conv2d", [el.tensor(a["x"], line), el.tensor(a["w"], line)], attrs, line)


def _pool_input(el, a, line, fill: float) -> Value:
    """Padding for pooling is an explicit pad: -inf for max pooling so that it never wins."""
    x = el.tensor(a["x"], line)
    ph, pw = el.pair(a["padding"], line, "padding")
    if ph or pw:
        x = el.op("pad", [x], {"pads": ((0, 0), (0, 0), (ph, ph), (pw, pw)), "value": fill}, line)
    return x


def _maxpool(el, a, line):
    size = el.int_(a["size"], line, "size")
    stride = size if a["stride"] is None else el.int_(a["stride"], line, "stride")
    x = _pool_input(el, a, line, -np.inf)
    return el.op("maxpool2d", [x], {"size": size, "stride": stride}, line)


def _avgpool(el, a, line):
    """Average pooling as a depthwise convolution with a constant 1/(k*k) kernel."""
    size = el.int_(a["size"], line, "size")
    stride = size if a["stride"] is None else el.int_(a["stride"], line, "stride")
    x = _pool_input(el, a, line, 0.0)
    c = x.type.shape[1]
    w = el.g.const(np.full((c, 1, size, size), 1.0 / (size * size), dtype=x.type.np_dtype))
    return el.op("conv2d", [x, w], {"stride": (stride, stride), "padding": (0, 0), "groups": c}, line)


def _softmax(el, a, line):
    return el.op("softmax", [el.tensor(a["x"], line)], {"axis": el.int_(a["axis"], line, "axis")}, line)


def _matmul(el, a, line):
    return el.op("matmul", [el.tensor(a["a"], line), el.tensor(a["b"], line)], {}, line)


BUILTINS = {
    **{k: _unary(k) for k in _UNARY},
    "maximum": _binary_fn("maximum"),
    "minimum": _binary_fn("minimum"),
    "matmul": ([("a", _REQUIRED), ("b", _REQUIRED)], _matmul),
    "softmax": ([("x", _REQUIRED), ("axis", -1)], _softmax),
    "mean": ([("x", _REQUIRED), ("axis", None), ("keepdims", False)], _mean),
    "transpose": ([("x", _REQUIRED), ("perm", None)], _transpose),
    "reshape": ([("x", _REQUIRED), ("shape", _REQUIRED)], _reshape),
    "flatten": ([("x", _REQUIRED), ("axis", 1)], _flatten),
    "conv2d": ([("x", _REQUIRED), ("w", _REQUIRED), ("stride", 1), ("padding", 0), ("dilation", 1), ("groups", 1)],
               _conv2d),
    "maxpool2d": ([("x", _REQUIRED), ("size", 2), ("stride", None), ("padding", 0)], _maxpool),
    "avgpool2d": ([("x", _REQUIRED), ("size", 2), ("stride", None), ("padding", 0)], _avgpool),
}


def elaborate(src: str, entry: str = "main", weights: Optional[dict] = None, dims: Optional[dict] = None,
              seed: Optional[int] = 0, name: Optional[str] = None) -> Graph:
    """A .mira program as a harness Graph: the entry function inlined, its shape symbols from
    `dims`, its const parameters from `weights` or drawn from `seed` (None: all must be given)."""
    g = Elaborator(parse(src), name or entry).entry(entry, weights or {}, dims or {}, seed)
    g.check()
    return g
