"""A front end for MIRA's source language (.mira): the counterpart of mira/lexer.py,
mira/parser.py and mira/elaborate.py, producing this harness's graphs.

    program   := function*
    function  := "fn" NAME "(" [param ("," param)*] ")" "->" (type | "(" type ("," type)* ")") block
    param     := ["const"] NAME ":" type  |  NAME ":" "int"          (a compile-time integer)
    type      := DTYPE ["[" dim ("," dim)* "]"]          DTYPE: f32 | f16 | i32
    dim       := integer arithmetic (+ - * /, parentheses) over literals and shape symbols
    block     := "{" statement* "}"
    statement := "let" names [":" type] "=" expr  |  names "=" expr
               | NAME "[" item ("," item)* "]" "=" expr
               | "for" NAME "in" expr ".." expr block
               | "if" expr block ["else" (block | if-statement)]
               | "while" expr block
               | "return" expr ("," expr)*
    names     := NAME ("," NAME)*  |  "(" NAME ("," NAME)* ")"
    expr      := sum [("<" | "<=" | ">" | ">=" | "==" | "!=") sum]
    sum       := term (("+" | "-") term)*          term := unary (("*" | "/" | "@") unary)*
    unary     := "-" unary | power                 power := postfix ["**" unary]
    postfix   := primary ("[" item ("," item)* "]")*      item := expr | [expr] ":" [expr]
    primary   := number | true | false | DTYPE | NAME | NAME "(" args ")" | "(" expr ")"
               | "(" expr "," [expr ("," expr)*] ")" | "[" [expr ("," expr)*] "]"
    "#" starts a comment; a call's "(" and an index's "[" sit on the line of what they follow.

Elaboration inlines every call of a user function, binding the shape symbols of its
parameter types from the arguments (a symbol seen twice must agree), its `int` parameters
from compile-time numbers, and checks the results against the declared return types.
`for` loops are unrolled and `if` / `while` on compile-time conditions are decided while
elaborating; on a one-element runtime tensor they become `if` / `while` ops whose
sub-graphs capture the outer values they read (mira/elaborate.py:128-184, 428-519); indexed
assignment is a dynamic_update_slice.  `grad` (MIRA's autodiff) is reported as unsupported.
The entry
function's plain parameters become graph inputs, its `int` parameters take values from
`dims`; its `const` parameters are weights: given ones are used, the others are drawn in
declaration order from one seeded generator by MIRA's rule (mira/elaborate.py:196-213,
1114-1123; harness.models.mira_random_weight).

Shape symbols bound in a function are plain numbers in its body, so `reshape(x, [B, C * H * W])`
works.  Builtins, with MIRA's parameter names and defaults (mira/elaborate.py:1070-1111):
relu sigmoid tanh gelu exp log abs sign sqrt (x) -- on a number they compute at compile
time --, maximum / minimum (a, b), matmul(a, b), softmax(x, axis=-1),
sum / mean / max (x, axis=all, keepdims=false), layernorm(x, gamma, beta, eps=1e-5),
transpose(x, perm=swap last two), reshape(x, shape) with one -1 allowed, flatten(x, axis=1),
concat(xs, axis=0), cast(x, dtype), slice(x, begin, size), pad(x, pads, value=0),
broadcast(x, shape), gather(x, indices, axis=0), where(cond, a, b), size(x, axis),
dynamic_slice(x, start, size), dynamic_update_slice(x, update, start),
sort / cumprod (x, axis=-1), argmax / argmin (x, axis=-1, keepdims=false),
zeros / ones (shape, dtype=f32), full(shape, value, dtype=f32), arange(start, stop, dtype=i32),
conv2d(x, w, stride=1, padding=0, dilation=1, groups=1),
maxpool2d / avgpool2d (x, size=2, stride=size, padding=0).
Indexing follows mira/elaborate.py:617-675: the static subscripts of `x[...]` become one
slice, axes indexed by a single number are reshaped away, and i32 tensor subscripts become
gathers.  Comparisons of tensors give 1 / 0 in the operands' dtype: `a < b` is
greater(b, a), `a <= b` greater_equal(b, a), `a != b` 1 - equal(a, b) (mira/elaborate.py:566-597).
"""
from __future__ import annotations

import re
from dataclasses import dataclass
from typing import Optional

import numpy as np

from harness.graph import DTYPES, Graph, Value
from harness.models import mira_random_weight


class MiraSyntaxError(ValueError):
    """A problem in the program text or its shapes, with its line."""


# ---------------------------------------------------------------- lexer

_TOKEN = re.compile(r"""
    (?P<ws>[ \t\r]+) | (?P<comment>\#[^\n]*) | (?P<nl>\n)
  | (?P<num>\d+\.(?!\.)\d*(?:[eE][+-]?\d+)?|\d+[eE][+-]?\d+|\.\d+(?:[eE][+-]?\d+)?|\d+)
  | (?P<name>[A-Za-z_][A-Za-z_0-9]*)
  | (?P<op>->|\.\.|\*\*|<=|>=|==|!=|[-+*/@=(),:\[\]{}<>])
""", re.VERBOSE)

KEYWORDS = {"fn", "let", "return", "const", "for", "in", "while", "if", "else"}
COMPARE = ("<", "<=", ">", ">=", "==", "!=")
MAX_UNROLL = 10_000        # iterations of a `for` (or compile-time `while`) unrolled while elaborating
MAX_ITERS = 100_000        # iterations a runtime `while` may run


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
    dtype: str            # f32 / f16 / i32, or "int" for a compile-time integer parameter
    dims: list            # dim expressions: int, str, or (op, left, right)


@dataclass
class Param:
    name: str
    type: TypeRef
    const: bool


@dataclass
class Fn:
    name: str
    params: list[Param]
    rets: list[TypeRef]
    body: list
    line: int


# statements: ("let", names, TypeRef | None, expr, line)  ("assign", names, expr, line)
#             ("index_assign", name, items, expr, line)  ("for", var, start, stop, body, line)
#             ("if", cond, then_body, else_body | None, line)  ("while", cond, body, line)
#             ("return", [expr, ...], line)
# expressions: ("num", v) ("bool", v) ("dtype", name) ("name", id) ("neg", e) ("bin", op, a, b)
#              ("call", name, args, kwargs, line) ("list", items) ("tuple", items)
#              ("index", base, items, line) with items ("at", e) | ("range", lo | None, hi | None)


class _Parser:
    def __init__(self, toks: list[Tok]):
        self.t, self.i = toks, 0

    def peek(self, k: int = 0) -> Tok:
        return self.t[min(self.i + k, len(self.t) - 1)]

    def take(self, text: Optional[str] = None, kind: Optional[str] = None) -> Tok:
        tok = self.t[self.i]
        if (text is not None and tok.text != text) or (kind is not None and tok.kind != kind):
            want = repr(text) if text is not None else kind
            raise MiraSyntaxError(f"line {tok.line}: expected {want}, found {tok.text or 'end of file'!r}")
        self.i += 1
        return tok

    def at(self, text: str) -> bool:
        return self.t[self.i].text == text and self.t[self.i].kind in ("op", "kw")

    def same_line(self) -> bool:
        """The current token sits on the line of the one before it."""
        return self.i > 0 and self.t[self.i].line == self.t[self.i - 1].line

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
            const = self.at("const")
            if const:
                self.take("const")
            pname = self.take(kind="name").text
            self.take(":")
            tref = self.type_ref(allow_int=not const)
            params.append(Param(pname, tref, const))
            if not self.at(")"):
                self.take(",")
        self.take(")")
        self.take("->")
        if self.at("("):
            self.take("(")
            rets = [self.type_ref()]
            while self.at(","):
                self.take(",")
                rets.append(self.type_ref())
            self.take(")")
        else:
            rets = [self.type_ref()]
        return Fn(name, params, rets, self.block(), line)

    def block(self) -> list:
        self.take("{")
        body = []
        while not self.at("}"):
            if self.peek().kind == "eof":
                raise MiraSyntaxError(f"line {self.peek().line}: expected '}}', found end of file")
            body.append(self.statement())
        self.take("}")
        return body

    def names(self) -> list[str]:
        paren = self.at("(")
        if paren:
            self.take("(")
        out = [self.take(kind="name").text]
        while self.at(","):
            self.take(",")
            out.append(self.take(kind="name").text)
        if paren:
            self.take(")")
        if len(set(out)) != len(out):
            raise MiraSyntaxError(f"line {self.peek().line}: the same name appears twice")
        return out

    def statement(self):
        tok = self.peek()
        line = tok.line
        if tok.kind == "kw":
            if tok.text == "let":
                self.take("let")
                names = self.names()
                tref = None
                if self.at(":"):
                    self.take(":")
                    tref = self.type_ref()
                self.take("=")
                return ("let", names, tref, self.expr(), line)
            if tok.text == "return":
                self.take("return")
                vals = [self.expr()]
                while self.at(","):
                    self.take(",")
                    vals.append(self.expr())
                return ("return", vals, line)
            if tok.text == "for":
                self.take("for")
                var = self.take(kind="name").text
                self.take("in")
                start = self.expr()
                self.take("..")
                stop = self.expr()
                return ("for", var, start, stop, self.block(), line)
            if tok.text == "if":
                return self.if_statement()
            if tok.text == "while":
                self.take("while")
                cond = self.expr()
                return ("while", cond, self.block(), line)
        if tok.kind == "name" and self.peek(1).text == "[":
            name = self.take().text
            self.take("[")
            items = self.index_items()
            self.take("=")
            return ("index_assign", name, items, self.expr(), line)
        if tok.kind == "name" or (tok.kind == "op" and tok.text == "("):
            names = self.names()
            self.take("=")
            return ("assign", names, self.expr(), line)
        raise MiraSyntaxError(f"line {line}: expected 'let' or 'return', found {tok.text or 'end of file'!r}")

    def if_statement(self):
        line = self.take("if").line
        cond = self.expr()
        then = self.block()
        other = None
        if self.at("else"):
            self.take("else")
            other = [self.if_statement()] if self.at("if") else self.block()
        return ("if", cond, then, other, line)

    def type_ref(self, allow_int: bool = False) -> TypeRef:
        dt = self.take(kind="name")
        if dt.text == "int":
            if not allow_int:
                raise MiraSyntaxError(f"line {dt.line}: 'int' is only a parameter type (a compile-time integer)")
            return TypeRef("int", [])
        if dt.text not in DTYPES:
            raise MiraSyntaxError(f"line {dt.line}: unsupported element type '{dt.text}' ({', '.join(DTYPES)})")
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
        e = self.sum()
        if self.peek().kind == "op" and self.peek().text in COMPARE:
            op = self.take().text
            e = ("bin", op, e, self.sum())
            if self.peek().kind == "op" and self.peek().text in COMPARE:
                raise MiraSyntaxError(f"line {self.peek().line}: comparisons can't be chained; use parentheses")
        return e

    def sum(self):
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
        base = self.postfix()
        if self.at("**"):
            self.take("**")
            return ("bin", "**", base, self.unary())
        return base

    def postfix(self):
        e = self.primary()
        while self.at("[") and self.same_line():
            line = self.take("[").line
            e = ("index", e, self.index_items(), line)
        return e

    def index_items(self) -> list:
        """Subscripts up to and including the closing ']'."""
        items = []
        while True:
            lo = None if self.at(":") else self.expr()
            if self.at(":"):
                self.take(":")
                hi = None if (self.at(",") or self.at("]")) else self.expr()
                items.append(("range", lo, hi))
            else:
                items.append(("at", lo))
            if not self.at(","):
                break
            self.take(",")
        self.take("]")
        return items

    def primary(self):
        tok = self.peek()
        if tok.kind == "num":
            self.take()
            return ("num", float(tok.text) if any(c in tok.text for c in ".eE") else int(tok.text))
        if self.at("("):
            self.take("(")
            e = self.expr()
            if not self.at(","):
                self.take(")")
                return e
            items = [e]
            while self.at(","):
                self.take(",")
                if self.at(")"):
                    break
                items.append(self.expr())
            self.take(")")
            return ("tuple", items)
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
            if not (self.at("(") and self.same_line()):
                return ("dtype", tok.text) if tok.text in DTYPES else ("name", tok.text)
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


_UNARY = ("relu", "sigmoid", "tanh", "gelu", "exp", "log", "abs", "sign", "sqrt")
_BINOP = {"+": "add", "-": "sub", "*": "mul", "/": "div", "**": "pow"}
# MIRA builtins outside this front end (runtime indexing into loop state, autodiff, ...)
_UNSUPPORTED = ("grad", "scatter_add", "erf")
MAX_DEPTH = 64


class DType(str):
    """A dtype named in an expression (the `f32` of `cast(x, f32)`)."""


def _num(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


def _describe(v) -> str:
    if isinstance(v, Value):
        return f"tensor {v.type}"
    if isinstance(v, DType):
        return f"dtype {v}"
    if isinstance(v, tuple):
        return f"{len(v)} values"
    if isinstance(v, bool):
        return f"boolean {str(v).lower()}"
    return "list" if isinstance(v, list) else f"number {v}"


class Scope:
    """Names visible in a block; assignment rebinds a name where it was defined."""

    def __init__(self, parent: Optional["Scope"] = None):
        self.vars: dict = {}
        self.parent = parent

    def owner(self, name: str) -> Optional["Scope"]:
        s = self
        while s is not None and name not in s.vars:
            s = s.parent
        return s

    def lookup(self, name: str):
        s = self.owner(name)
        return None if s is None else s.vars[name]

    def snapshot(self) -> dict:
        """Every variable in sight: (scope id, name) -> (scope, value)."""
        out, s = {}, self
        while s is not None:
            for n, v in s.vars.items():
                out[(id(s), n)] = (s, v)
            s = s.parent
        return out

    def bindings(self) -> dict:
        """The whole-number names in sight (shape symbols, int parameters, loop counters)."""
        chain, s = [], self
        while s is not None:
            chain.append(s)
            s = s.parent
        out = {}
        for s in reversed(chain):
            out.update({k: v for k, v in s.vars.items() if isinstance(v, int) and not isinstance(v, bool)})
        return out


def _restore(snap: dict) -> dict:
    """Put the snapshotted variables back; returns those that had changed (key -> new value)."""
    changed = {}
    for key, (scope, old) in snap.items():
        new = scope.vars[key[1]]
        if new is not old:
            changed[key] = new
            scope.vars[key[1]] = old
    return changed


def _assigned(body: list) -> list:
    """Names a block assigns (plainly or by index), nested blocks included, first-seen order."""
    out: list = []
    for st in body:
        if st[0] == "assign":
            out += [n for n in st[1] if n not in out]
        elif st[0] == "index_assign" and st[1] not in out:
            out.append(st[1])
        subs = {"for": [st[4]] if st[0] == "for" else [], "while": [st[2]] if st[0] == "while" else [],
                "if": [st[2], st[3] or []] if st[0] == "if" else []}.get(st[0], [])
        for b in subs:
            out += [n for n in _assigned(b) if n not in out]
    return out


class _Ctx:
    """The graph being built and what it captured from the graphs around it."""

    def __init__(self, graph: Graph, parent: Optional["_Ctx"]):
        self.graph = graph
        self.parent = parent
        self.captures: dict = {}          # outer value -> its placeholder input here
        self.captured_outer: list = []    # the outer values, in input order
        self._owned: set = set()          # inputs and results of the ops seen so far
        self._synced = 0

    def owns(self, v: Value) -> bool:
        ops = self.graph.ops
        for op in ops[self._synced:]:
            self._owned.update(op.results)
        self._synced = len(ops)
        self._owned.update(self.graph.inputs)
        return v in self._owned


class Elaborator:
    """Inlines the entry function into one Graph (mira/elaborate.py:186-222 for the entry,
    :279-346 for calls, :348-528 for statements, :691-724 for indexed assignment)."""

    def __init__(self, fns: dict[str, Fn], name: str = "main"):
        self.fns = fns
        self.ctx = _Ctx(Graph(name), None)
        self.stack: list[str] = []
        self.counter = 0

    @property
    def g(self) -> Graph:
        return self.ctx.graph

    def local(self, v: Value, ctx: Optional[_Ctx] = None) -> Value:
        """`v` usable in ctx's graph: captured from an enclosing graph as a new input (a
        constant is copied instead)."""
        ctx = ctx or self.ctx
        if ctx.owns(v):
            return v
        if v in ctx.captures:
            return ctx.captures[v]
        if ctx.parent is None:
            raise AssertionError(f"{v!r} is not defined in any enclosing graph")
        if v.producer is not None and v.producer.kind == "const":
            c = ctx.graph.const(v.producer.attrs["value"])
        else:
            c = Value(v.type)
            ctx.graph.inputs.append(c)
            ctx.captured_outer.append(v)
        ctx.captures[v] = c
        return c

    def enter(self, label: str) -> _Ctx:
        self.ctx = _Ctx(Graph(f"{self.g.name}.{label}"), self.ctx)
        return self.ctx

    def exit(self, ctx: _Ctx) -> None:
        assert self.ctx is ctx
        self.ctx = ctx.parent

    # ---- values

    def tensor(self, v, line: int, dtype: str = "f32") -> Value:
        """Tensors pass through; numbers become scalar constants of `dtype`."""
        if isinstance(v, Value):
            return v
        if _num(v):
            if dtype == "i32" and float(v) != int(v):
                raise MiraSyntaxError(f"line {line}: the number {v} does not mix with an i32 tensor; "
                                      "cast the tensor to f32 first")
            return self.g.const(np.array(v, dtype=DTYPES[dtype]))
        raise MiraSyntaxError(f"line {line}: expected a tensor, got {_describe(v)}")

    def arg(self, v, line: int, dtype: str = "f32") -> Value:
        """A builtin's tensor argument, made local to the graph being built as it is read."""
        return self.local(self.tensor(v, line, dtype))

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

    @staticmethod
    def flag(v, line: int, what: str) -> bool:
        if not isinstance(v, bool):
            raise MiraSyntaxError(f"line {line}: {what} must be true or false")
        return v

    @staticmethod
    def dtype(v, line: int) -> str:
        if not isinstance(v, DType):
            raise MiraSyntaxError(f"line {line}: expected a dtype like f32 or i32, got {_describe(v)}")
        return str(v)

    # ---- functions

    def entry(self, fn_name: str, weights: dict, dims: dict, seed: Optional[int]) -> Graph:
        fn = self.fns.get(fn_name)
        if fn is None:
            raise MiraSyntaxError(f"no function named '{fn_name}' (the entry point)")
        env = dict(dims)
        rng = np.random.default_rng(seed) if seed is not None else None
        args = []
        for p in fn.params:
            if p.type.dtype == "int":
                if p.name not in env:
                    raise MiraSyntaxError(f"line {fn.line}: int parameter '{p.name}' of the entry function needs a "
                                          f"value (dims={{'{p.name}': ...}})")
                args.append(env[p.name])
                continue
            for d in p.type.dims:
                if isinstance(d, str) and d not in env:
                    raise MiraSyntaxError(f"line {fn.line}: dimension '{d}' of the entry function needs a value "
                                          f"(dims={{'{d}': ...}})")
            shape = tuple(_eval_dim(d, env, fn.line) for d in p.type.dims)
            npdt = DTYPES[p.type.dtype]
            if p.const:
                if p.name in weights:
                    arr = np.asarray(weights[p.name])
                    if tuple(arr.shape) != shape:
                        raise MiraSyntaxError(f"line {fn.line}: weight '{p.name}' has shape {list(arr.shape)}, "
                                              f"the parameter is {p.type.dtype}{list(shape)}")
                    arr = arr.astype(npdt)
                elif rng is not None:
                    arr = rng.integers(0, 8, shape).astype(npdt) if p.type.dtype == "i32" else \
                        mira_random_weight(rng, shape, npdt)
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
        self.g.outputs = list(out) if isinstance(out, tuple) else [out]
        return self.g

    def call_function(self, fn: Fn, args: list, line: int, preset: Optional[dict] = None):
        if fn.name in self.stack:
            raise MiraSyntaxError(f"line {line}: recursive call to '{fn.name}'")
        if len(self.stack) >= MAX_DEPTH:
            raise MiraSyntaxError(f"line {line}: function calls nested too deeply")
        if len(args) != len(fn.params):
            raise MiraSyntaxError(f"line {line}: '{fn.name}' takes {len(fn.params)} arguments, got {len(args)}")
        env = dict(preset or {})
        tensors: dict = {}
        for p, a in zip(fn.params, args):          # int parameters first: types may use them
            if p.type.dtype == "int":
                env[p.name] = self.int_(a, line, f"argument '{p.name}' of '{fn.name}'")
        for p, a in zip(fn.params, args):
            if p.type.dtype == "int":
                continue
            if p.const and self.stack:
                raise MiraSyntaxError(f"line {fn.line}: 'const' is only allowed on the entry function's parameters")
            tensors[p.name] = a = self.local(self.tensor(a, line, p.type.dtype))
            _unify(p.type, a.type.dtype, a.type.shape, env, f"argument '{p.name}' of '{fn.name}'", line, False)
        for p in fn.params:
            if p.name in tensors:
                a = tensors[p.name]
                _unify(p.type, a.type.dtype, a.type.shape, env, f"argument '{p.name}' of '{fn.name}'", line, True)
        scope = Scope()
        scope.vars.update(env)              # shape symbols are plain numbers inside the body
        for name, v in tensors.items():
            if name in env:
                raise MiraSyntaxError(f"line {fn.line}: parameter '{name}' has the name of a shape dimension")
            scope.vars[name] = v
        self.stack.append(fn.name)
        try:
            result = self.block(fn.body, scope, nested=False)
            if result is None:
                raise MiraSyntaxError(f"line {fn.line}: '{fn.name}' has no return")
            value, rline = result
            values = list(value) if isinstance(value, tuple) else [value]
            if len(values) != len(fn.rets):
                raise MiraSyntaxError(f"line {rline}: '{fn.name}' returns {len(values)} value(s), its signature "
                                      f"declares {len(fn.rets)}")
            out = []
            for v, tref in zip(values, fn.rets):
                v = self.local(self.tensor(v, rline, tref.dtype))
                _unify(tref, v.type.dtype, v.type.shape, env, f"the result of '{fn.name}'", rline, True)
                out.append(v)
            return tuple(out) if len(fn.rets) > 1 else out[0]
        finally:
            self.stack.pop()

    # ---- statements

    def block(self, body: list, scope: Scope, nested: bool) -> Optional[tuple]:
        for i, st in enumerate(body):
            kind, line = st[0], st[-1]
            if kind == "let":
                self.let(st, scope)
            elif kind == "assign":
                self.assign(st, scope)
            elif kind == "for":
                _, var, start, stop, inner, _ = st
                lo = self.int_(self.expr(start, scope, line), line, "loop bound")
                hi = self.int_(self.expr(stop, scope, line), line, "loop bound")
                if hi - lo > MAX_UNROLL:
                    raise MiraSyntaxError(f"line {line}: loop of {hi - lo} iterations; at most {MAX_UNROLL} unroll")
                for it in range(lo, hi):
                    s = Scope(scope)
                    s.vars[var] = it
                    self.block(inner, s, nested=True)
            elif kind == "if":
                self.if_stmt(st, scope)
            elif kind == "while":
                self.while_stmt(st, scope)
            elif kind == "index_assign":
                self.index_assign(st, scope)
            else:   # return
                if nested:
                    raise MiraSyntaxError(f"line {line}: 'return' must be the last statement of a function, "
                                          "not inside for / if")
                if i != len(body) - 1:
                    raise MiraSyntaxError(f"line {body[i + 1][-1]}: unreachable code after 'return'")
                vals = [self.expr(e, scope, line) for e in st[1]]
                return (vals[0] if len(vals) == 1 else tuple(vals)), line
        return None

    @staticmethod
    def destructure(names: list, v, line: int) -> list:
        if len(names) == 1:
            if isinstance(v, tuple):
                raise MiraSyntaxError(f"line {line}: this gives {len(v)} values; unpack them like 'let a, b = ...'")
            return [v]
        if not isinstance(v, tuple) or len(v) != len(names):
            raise MiraSyntaxError(f"line {line}: cannot unpack {_describe(v)} into {len(names)} names")
        return list(v)

    def let(self, st, scope: Scope) -> None:
        _, names, tref, e, line = st
        for n in names:
            if n in scope.vars:
                raise MiraSyntaxError(f"line {line}: '{n}' is already defined in this scope; "
                                      f"use '{n} = ...' to reassign")
        v = self.expr(e, scope, line)
        if tref is not None:
            v = self.tensor(v, line, tref.dtype)
            _unify(tref, v.type.dtype, v.type.shape, dict(scope.bindings()), f"'{names[0]}'", line, True)
        for n, x in zip(names, self.destructure(names, v, line)):
            scope.vars[n] = x

    def assign(self, st, scope: Scope) -> None:
        _, names, e, line = st
        values = self.destructure(names, self.expr(e, scope, line), line)
        for n, v in zip(names, values):
            owner = scope.owner(n)
            if owner is None:
                raise MiraSyntaxError(f"line {line}: assignment to undefined variable '{n}'; declare it with 'let'")
            old = owner.vars[n]
            if isinstance(old, Value):
                v = self.tensor(v, line, old.type.dtype)
                if v.type != old.type:
                    raise MiraSyntaxError(f"line {line}: '{n}' has type {old.type}; cannot assign a {v.type}")
            elif isinstance(v, (Value, tuple)):
                raise MiraSyntaxError(f"line {line}: '{n}' is a compile-time {_describe(old)}; "
                                      f"cannot assign a {_describe(v)}")
            owner.vars[n] = v

    @staticmethod
    def truthy(v, line: int) -> Optional[bool]:
        """A condition's compile-time truth, or None for a one-element runtime tensor."""
        if isinstance(v, Value):
            if v.type.numel != 1:
                raise MiraSyntaxError(f"line {line}: a condition must be a single value, got {v.type}; "
                                      "reduce it first (e.g. with max or sum)")
            return None
        if isinstance(v, bool) or _num(v):
            return bool(v)
        raise MiraSyntaxError(f"line {line}: a condition must be a boolean, a number or a one-element tensor; "
                              f"got {_describe(v)}")

    def if_stmt(self, st, scope: Scope) -> None:
        """A compile-time condition picks a branch now; a runtime one builds an `if` op whose
        branches output every variable either of them changes (mira/elaborate.py:428-465)."""
        _, cond_e, then, other, line = st
        cond = self.expr(cond_e, scope, line)
        static = self.truthy(cond, line)
        if static is not None:
            taken = then if static else other
            if taken:
                self.block(taken, Scope(scope), nested=True)
            return
        n, self.counter = self.counter, self.counter + 1
        branches = []
        for label, body in (("then", then), ("else", other or [])):
            snap = scope.snapshot()
            ctx = self.enter(f"if{n}.{label}")
            self.block(body, Scope(scope), nested=True)
            self.exit(ctx)
            branches.append((ctx, _restore(snap)))
        keys = list(dict.fromkeys(k for _, changed in branches for k in changed))
        snap = scope.snapshot()
        types = []
        for key in keys:
            orig = snap[key][1]
            if not isinstance(orig, Value):
                raise MiraSyntaxError(f"line {line}: '{key[1]}' is a compile-time value; it cannot change inside "
                                      "an 'if' whose condition is only known at runtime")
            types.append(orig.type)
        for ctx, changed in branches:
            ctx.graph.outputs = [self.local(changed.get(k, snap[k][1]), ctx) for k in keys]
        (then_ctx, _), (else_ctx, _) = branches
        ins = [self.local(cond)] + [self.local(v) for v in then_ctx.captured_outer] + \
              [self.local(v) for v in else_ctx.captured_outer]
        results = self.g.add_control("if", ins, {"then": then_ctx.graph, "else": else_ctx.graph,
                                                 "n_then": len(then_ctx.captured_outer)}, types)
        for key, r in zip(keys, results):
            snap[key][0].vars[key[1]] = r

    def while_stmt(self, st, scope: Scope) -> None:
        """A compile-time condition unrolls the loop now; a runtime one builds a `while` op whose
        state is every tensor variable the body assigns (mira/elaborate.py:467-519)."""
        _, cond_e, body, line = st
        cond = self.expr(cond_e, scope, line)
        if self.truthy(cond, line) is not None:
            for _ in range(MAX_UNROLL):
                if not self.truthy(self.expr(cond_e, scope, line), line):
                    return
                self.block(body, Scope(scope), nested=True)
            raise MiraSyntaxError(f"line {line}: compile-time while loop ran more than {MAX_UNROLL} iterations")
        names = []
        for name in _assigned(body):
            v = scope.lookup(name)
            if v is None:
                continue
            if not isinstance(v, Value):
                raise MiraSyntaxError(f"line {line}: '{name}' is a compile-time value; it cannot change inside a "
                                      "'while' whose condition is only known at runtime")
            names.append(name)
        init = [scope.lookup(nm) for nm in names]
        n, self.counter = self.counter, self.counter + 1

        def state_scope(ctx: _Ctx) -> Scope:
            s = Scope(scope)
            for nm, v in zip(names, init):
                ph = Value(v.type)
                ctx.graph.inputs.append(ph)
                s.vars[nm] = ph
            return s

        cond_ctx = self.enter(f"while{n}.cond")
        c = self.expr(cond_e, state_scope(cond_ctx), line)
        if not isinstance(c, Value) or c.type.numel != 1:
            raise MiraSyntaxError(f"line {line}: the loop condition must stay a one-element tensor")
        cond_ctx.graph.outputs = [self.local(c)]
        self.exit(cond_ctx)
        body_ctx = self.enter(f"while{n}.body")
        s = state_scope(body_ctx)
        snap = scope.snapshot()
        self.block(body, Scope(s), nested=True)
        if _restore(snap):
            raise MiraSyntaxError(f"line {line}: a compile-time value changed inside a runtime 'while' loop")
        body_ctx.graph.outputs = [self.local(s.vars[nm]) for nm in names]
        self.exit(body_ctx)
        ins = [self.local(v) for v in init] + [self.local(v) for v in cond_ctx.captured_outer] + \
              [self.local(v) for v in body_ctx.captured_outer]
        results = self.g.add_control("while", ins, {"cond": cond_ctx.graph, "body": body_ctx.graph,
                                                    "n_state": len(names), "n_cond": len(cond_ctx.captured_outer),
                                                    "max_iters": MAX_ITERS}, [v.type for v in init])
        for nm, r in zip(names, results):
            scope.owner(nm).vars[nm] = r

    def start_vector(self, parts: list, line: int) -> Value:
        """An i32[n] start position from compile-time ints and one-element i32 tensors."""
        if all(isinstance(p, int) for p in parts):
            return self.g.const(np.array(parts, dtype=np.int32))
        pieces = []
        for p in parts:
            if isinstance(p, int):
                pieces.append(self.g.const(np.array([p], dtype=np.int32)))
            else:
                if p.type.dtype != "i32" or p.type.numel != 1:
                    raise MiraSyntaxError(f"line {line}: a runtime position must be a one-element i32 tensor, "
                                          f"got {p.type}")
                pieces.append(self.op("reshape", [p], {"shape": (1,)}, line))
        return self.op("concat", pieces, {"axis": 0}, line)

    def index_assign(self, st, scope: Scope) -> None:
        """x[subscripts] = value as a dynamic_update_slice of the region (mira/elaborate.py:691-724)."""
        _, name, items, value, line = st
        owner = scope.owner(name)
        if owner is None:
            raise MiraSyntaxError(f"line {line}: assignment to undefined variable '{name}'; declare it with 'let'")
        x = owner.vars[name]
        if not isinstance(x, Value):
            raise MiraSyntaxError(f"line {line}: '{name}' is a compile-time {_describe(x)}; only tensors are indexed")
        x = self.local(x)
        starts, region, vshape = [], [], []
        for sub, d in zip(self.subscripts(items, x.type.shape, scope, line), x.type.shape):
            if sub[0] == "int":
                starts.append(sub[1])
                region.append(1)
            elif sub[0] == "range":
                starts.append(sub[1])
                region.append(sub[2] - sub[1])
                vshape.append(sub[2] - sub[1])
            else:
                if sub[1].type.numel != 1:
                    raise MiraSyntaxError(f"line {line}: indexed assignment takes one position per axis")
                starts.append(sub[1])
                region.append(1)
        v = self.tensor(self.expr(value, scope, line), line, x.type.dtype)
        if v.type.dtype != x.type.dtype:
            raise MiraSyntaxError(f"line {line}: cannot store a {v.type} into '{name}' ({x.type})")
        if v.type.shape != tuple(vshape):
            v = self.op("broadcast", [v], {"shape": tuple(vshape)}, line)
        v = self.op("reshape", [v], {"shape": tuple(region)}, line)
        start = self.start_vector(starts, line)
        owner.vars[name] = self.op("dynamic_update_slice", [x, v, start], {}, line)

    # ---- expressions

    def expr(self, e, scope: Scope, line: int):
        kind = e[0]
        if kind in ("num", "bool"):
            return e[1]
        if kind == "dtype":
            return DType(e[1])
        if kind == "list":
            return [self.expr(x, scope, line) for x in e[1]]
        if kind == "tuple":
            return tuple(self.expr(x, scope, line) for x in e[1])
        if kind == "name":
            v = scope.lookup(e[1])
            if v is None:
                what = "a function; call it" if e[1] in self.fns or e[1] in BUILTINS else "undefined"
                raise MiraSyntaxError(f"line {line}: '{e[1]}' is {what}")
            return v
        if kind == "neg":
            v = self.expr(e[1], scope, line)
            if isinstance(v, Value):
                return self.op("neg", [v], {}, line)
            if _num(v):
                return -v
            raise MiraSyntaxError(f"line {line}: cannot negate a {_describe(v)}")
        if kind == "bin":
            return self.binary(e[1], self.expr(e[2], scope, line), self.expr(e[3], scope, line), line)
        if kind == "index":
            return self.index(e, scope)
        _, name, args, kwargs, line = e
        vals = [self.expr(a, scope, line) for a in args]
        kw = {k: self.expr(v, scope, line) for k, v in kwargs.items()}
        if name in self.fns:
            fn = self.fns[name]
            if len(vals) > len(fn.params):
                raise MiraSyntaxError(f"line {line}: '{name}' takes {len(fn.params)} arguments, got {len(vals)}")
            args = vals + [None] * (len(fn.params) - len(vals))
            for k, v in kw.items():
                idx = next((i for i, p in enumerate(fn.params) if p.name == k), None)
                if idx is None:
                    raise MiraSyntaxError(f"line {line}: '{name}' has no parameter named '{k}'")
                if args[idx] is not None:
                    raise MiraSyntaxError(f"line {line}: argument '{k}' given twice")
                args[idx] = v
            missing = [p.name for p, a in zip(fn.params, args) if a is None]
            if missing:
                raise MiraSyntaxError(f"line {line}: call to '{name}' is missing argument(s): {', '.join(missing)}")
            return self.call_function(fn, args, line)
        if name in _UNSUPPORTED:
            raise MiraSyntaxError(f"line {line}: {name}() is not supported by this front end")
        if name not in BUILTINS:
            raise MiraSyntaxError(f"line {line}: unknown function '{name}'")
        params, handler = BUILTINS[name]
        return handler(self, _bind_args(name, params, vals, kw, line), line)

    def binary(self, op: str, a, b, line: int):
        if op in COMPARE and not isinstance(a, Value) and not isinstance(b, Value):
            if not all(_num(x) or isinstance(x, bool) for x in (a, b)):
                raise MiraSyntaxError(f"line {line}: cannot compare {_describe(a)} and {_describe(b)}")
            return {"<": a < b, "<=": a <= b, ">": a > b, ">=": a >= b, "==": a == b, "!=": a != b}[op]
        if _num(a) and _num(b):
            if op == "@":
                raise MiraSyntaxError(f"line {line}: '@' needs tensor operands")
            if op == "/":
                if b == 0:
                    raise MiraSyntaxError(f"line {line}: division by zero")
                return a // b if isinstance(a, int) and isinstance(b, int) and a % b == 0 else a / b
            return {"+": a + b, "-": a - b, "*": a * b, "**": a ** b}[op]
        if not isinstance(a, Value) and not isinstance(b, Value):
            raise MiraSyntaxError(f"line {line}: cannot apply '{op}' to {_describe(a)} and {_describe(b)}")
        dtype = a.type.dtype if isinstance(a, Value) else b.type.dtype
        a, b = self.tensor(a, line, dtype), self.tensor(b, line, dtype)
        if op == "@":
            return self.op("matmul", [a, b], {}, line)
        if op in COMPARE:
            if op == "!=":
                eq = self.op("equal", [a, b], {}, line)
                return self.op("sub", [self.tensor(1, line, dtype), eq], {}, line)
            kind = {"<": "greater", "<=": "greater_equal", ">": "greater", ">=": "greater_equal",
                    "==": "equal"}[op]
            return self.op(kind, [b, a] if op in ("<", "<=") else [a, b], {}, line)
        return self.op(_BINOP[op], [a, b], {}, line)

    def index(self, e, scope: Scope) -> Value:
        _, base, items, line = e
        x = self.expr(base, scope, line)
        if not isinstance(x, Value):
            raise MiraSyntaxError(f"line {line}: cannot index a {_describe(x)}")
        x = self.local(x)
        shape = x.type.shape
        subs = self.subscripts(items, shape, scope, line)
        begin = tuple(s[1] if s[0] != "tensor" else 0 for s in subs)
        size = tuple(1 if s[0] == "int" else s[2] - s[1] if s[0] == "range" else d for s, d in zip(subs, shape))
        if size != shape:
            x = self.op("slice", [x], {"begin": begin, "size": size}, line)
        kept = [i for i, s in enumerate(subs) if s[0] != "int"]
        if len(kept) != len(subs):
            x = self.op("reshape", [x], {"shape": tuple(size[i] for i in kept)}, line)
        shift = 0
        for axis, i in enumerate(kept):
            if subs[i][0] == "tensor":
                idx = subs[i][1]
                x = self.op("gather", [x, idx], {"axis": axis + shift}, line)
                shift += idx.type.rank - 1
        return x

    def subscripts(self, items: list, shape: tuple, scope: Scope, line: int) -> list:
        """Per axis ("int", k) | ("range", lo, hi) | ("tensor", i32 value); missing ones are whole
        ranges (mira/elaborate.py:617-650)."""
        if len(items) > len(shape):
            raise MiraSyntaxError(f"line {line}: {len(items)} subscripts for a rank-{len(shape)} tensor")
        subs = []         # per axis: ("int", k) | ("range", lo, hi) | ("tensor", value)
        for axis, d in enumerate(shape):
            it = items[axis] if axis < len(items) else ("range", None, None)
            if it[0] == "range":
                bounds = []
                for b, default in ((it[1], 0), (it[2], d)):
                    v = default if b is None else self.expr(b, scope, line)
                    if isinstance(v, Value):
                        raise MiraSyntaxError(f"line {line}: slice bounds must be compile-time numbers")
                    v = self.int_(v, line, "slice bound")
                    bounds.append(max(0, min(d, v + d if v < 0 else v)))
                if bounds[1] <= bounds[0]:
                    raise MiraSyntaxError(f"line {line}: empty slice {bounds[0]}:{bounds[1]} of an axis of size {d}")
                subs.append(("range", bounds[0], bounds[1]))
                continue
            v = self.expr(it[1], scope, line)
            if isinstance(v, Value):
                if v.type.dtype != "i32":
                    raise MiraSyntaxError(f"line {line}: tensor subscripts must be i32, got {v.type}")
                subs.append(("tensor", self.local(v)))
                continue
            k = self.int_(v, line, "index")
            if not -d <= k < d:
                raise MiraSyntaxError(f"line {line}: index {k} is out of range for an axis of size {d}")
            subs.append(("int", k % d))
        return subs

    def op(self, kind: str, ins: list, attrs: dict, line: int) -> Value:
        try:
            return self.g.op(kind, [self.local(v) for v in ins], attrs)
        except ValueError as err:
            raise MiraSyntaxError(f"line {line}: {kind}: {err}") from None


# ---------------------------------------------------------------- builtins
# (name, default) parameter lists and handlers, as MIRA's builtin table
# (mira/elaborate.py:1070-1111) declares them for these operators.

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
    def h(el, a, line):
        x = a["x"]
        if _num(x):         # compile-time arithmetic, as in / sqrt(D)
            from harness.hosteval import UNARY
            with np.errstate(all="raise"):
                try:
                    return float(UNARY[kind](np.float64(x)))
                except FloatingPointError:
                    raise MiraSyntaxError(f"line {line}: {kind}({x}) is undefined") from None
        return el.op(kind, [el.arg(x, line)], {}, line)
    return [("x", _REQUIRED)], h


def _binary_fn(kind):
    def h(el, a, line):
        x, y = a["a"], a["b"]
        if not isinstance(x, Value) and not isinstance(y, Value):
            raise MiraSyntaxError(f"line {line}: {kind}() needs at least one tensor argument")
        dt = x.type.dtype if isinstance(x, Value) else y.type.dtype
        return el.op(kind, [el.tensor(x, line, dt), el.tensor(y, line, dt)], {}, line)
    return [("a", _REQUIRED), ("b", _REQUIRED)], h


def _reduce(kind):
    def h(el, a, line):
        x = el.arg(a["x"], line)
        axes = list(range(x.type.rank)) if a["axis"] is None else el.ints(a["axis"], line, "axis")
        keep = el.flag(a["keepdims"], line, "keepdims")
        return el.op(kind, [x], {"axes": tuple(axes), "keepdims": keep}, line)
    return [("x", _REQUIRED), ("axis", None), ("keepdims", False)], h


def _transpose(el, a, line):
    x = el.arg(a["x"], line)
    if a["perm"] is None:
        if x.type.rank < 2:
            raise MiraSyntaxError(f"line {line}: transpose() of a rank-{x.type.rank} tensor needs a perm")
        perm = list(range(x.type.rank))
        perm[-2], perm[-1] = perm[-1], perm[-2]
    else:
        perm = el.ints(a["perm"], line, "perm")
    return el.op("transpose", [x], {"perm": tuple(perm)}, line)


def _reshape(el, a, line):
    x = el.arg(a["x"], line)
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
    x = el.arg(a["x"], line)
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
    return el.op("conv2d", [el.arg(a["x"], line), el.arg(a["w"], line)], attrs, line)


def _pool_input(el, a, line, fill: float) -> Value:
    """Padding for pooling is an explicit pad: -inf for max pooling so that it never wins."""
    x = el.arg(a["x"], line)
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
    return el.op("softmax", [el.arg(a["x"], line)], {"axis": el.int_(a["axis"], line, "axis")}, line)


def _matmul(el, a, line):
    return el.op("matmul", [el.arg(a["a"], line), el.arg(a["b"], line)], {}, line)


def _layernorm(el, a, line):
    eps = a["eps"]
    if not _num(eps):
        raise MiraSyntaxError(f"line {line}: layernorm eps must be a number")
    ins = [el.arg(a[k], line) for k in ("x", "gamma", "beta")]
    return el.op("layernorm", ins, {"eps": float(eps)}, line)


def _concat(el, a, line):
    xs = a["xs"]
    if not isinstance(xs, list) or not xs:
        raise MiraSyntaxError(f"line {line}: concat() takes a non-empty list of tensors")
    return el.op("concat", [el.arg(v, line) for v in xs], {"axis": el.int_(a["axis"], line, "axis")}, line)


def _cast(el, a, line):
    x = el.arg(a["x"], line)
    dt = el.dtype(a["dtype"], line)
    return x if x.type.dtype == dt else el.op("cast", [x], {"dtype": dt}, line)


def _slice(el, a, line):
    return el.op("slice", [el.arg(a["x"], line)], {"begin": tuple(el.ints(a["begin"], line, "begin")),
                                                     "size": tuple(el.ints(a["size"], line, "size"))}, line)


def _pad(el, a, line):
    pads = a["pads"]
    if not isinstance(pads, list) or not all(isinstance(p, list) and len(p) == 2 for p in pads):
        raise MiraSyntaxError(f"line {line}: pad() takes pads like [[1, 1], [0, 2]], one pair per axis")
    attrs = {"pads": tuple((el.int_(p[0], line, "pad"), el.int_(p[1], line, "pad")) for p in pads)}
    if a["value"] != 0:
        if not _num(a["value"]):
            raise MiraSyntaxError(f"line {line}: pad value must be a number")
        attrs["value"] = float(a["value"])
    return el.op("pad", [el.arg(a["x"], line)], attrs, line)


def _broadcast_fn(el, a, line):
    return el.op("broadcast", [el.arg(a["x"], line)], {"shape": tuple(el.ints(a["shape"], line, "shape"))}, line)


def _gather(el, a, line):
    return el.op("gather", [el.arg(a["x"], line), el.arg(a["indices"], line, "i32")],
                 {"axis": el.int_(a["axis"], line, "axis")}, line)


def _where(el, a, line):
    c, x, y = a["cond"], a["a"], a["b"]
    if not isinstance(c, Value):
        raise MiraSyntaxError(f"line {line}: where() needs a tensor condition; use if for compile-time choices")
    vals = [v for v in (x, y) if isinstance(v, Value)]
    dt = vals[0].type.dtype if vals else "f32"
    return el.op("where", [c, el.tensor(x, line, dt), el.tensor(y, line, dt)], {}, line)


def _size(el, a, line):
    x = el.arg(a["x"], line)
    ax = el.int_(a["axis"], line, "axis")
    if not -x.type.rank <= ax < x.type.rank:
        raise MiraSyntaxError(f"line {line}: axis {ax} out of range for {x.type}")
    return x.type.shape[ax]


def _axis_op(kind):
    return ([("x", _REQUIRED), ("axis", -1)],
            lambda el, a, line: el.op(kind, [el.arg(a["x"], line)], {"axis": el.int_(a["axis"], line, "axis")},
                                      line))


def _arg(kind):
    def h(el, a, line):
        attrs = {"axis": el.int_(a["axis"], line, "axis"), "keepdims": el.flag(a["keepdims"], line, "keepdims")}
        return el.op(kind, [el.arg(a["x"], line)], attrs, line)
    return [("x", _REQUIRED), ("axis", -1), ("keepdims", False)], h


def _start(el, v, line) -> Value:
    """A start position: an i32 tensor, or a list of ints and one-element i32 tensors."""
    if isinstance(v, Value):
        return el.local(v)
    if not isinstance(v, list):
        raise MiraSyntaxError(f"line {line}: a start position is a list like [t, 0] or an i32 tensor")
    return el.start_vector([el.local(p) if isinstance(p, Value) else el.int_(p, line, "start") for p in v], line)


def _dynamic_slice(el, a, line):
    return el.op("dynamic_slice", [el.arg(a["x"], line), _start(el, a["start"], line)],
                 {"size": tuple(el.ints(a["size"], line, "size"))}, line)


def _dynamic_update_slice(el, a, line):
    x = el.arg(a["x"], line)
    upd = el.tensor(a["update"], line, x.type.dtype)
    return el.op("dynamic_update_slice", [x, upd, _start(el, a["start"], line)], {}, line)


def _filled(value):
    def h(el, a, line):
        shape = el.ints(a["shape"], line, "shape")
        v = a["value"] if value is None else value
        if not _num(v):
            raise MiraSyntaxError(f"line {line}: the fill value must be a number")
        return el.g.const(np.full(shape, v, dtype=DTYPES[el.dtype(a["dtype"], line)]))
    return h


def _arange(el, a, line):
    start = el.int_(a["start"], line, "start")
    lo, hi = (0, start) if a["stop"] is None else (start, el.int_(a["stop"], line, "stop"))
    return el.g.const(np.arange(lo, hi, dtype=DTYPES[el.dtype(a["dtype"], line)]))


BUILTINS = {
    **{k: _unary(k) for k in _UNARY},
    "maximum": _binary_fn("maximum"),
    "minimum": _binary_fn("minimum"),
    "matmul": ([("a", _REQUIRED), ("b", _REQUIRED)], _matmul),
    "softmax": ([("x", _REQUIRED), ("axis", -1)], _softmax),
    "sum": _reduce("reduce_sum"),
    "mean": _reduce("reduce_mean"),
    "max": _reduce("reduce_max"),
    "transpose": ([("x", _REQUIRED), ("perm", None)], _transpose),
    "reshape": ([("x", _REQUIRED), ("shape", _REQUIRED)], _reshape),
    "flatten": ([("x", _REQUIRED), ("axis", 1)], _flatten),
    "conv2d": ([("x", _REQUIRED), ("w", _REQUIRED), ("stride", 1), ("padding", 0), ("dilation", 1), ("groups", 1)],
               _conv2d),
    "maxpool2d": ([("x", _REQUIRED), ("size", 2), ("stride", None), ("padding", 0)], _maxpool),
    "avgpool2d": ([("x", _REQUIRED), ("size", 2), ("stride", None), ("padding", 0)], _avgpool),
    "layernorm": ([("x", _REQUIRED), ("gamma", _REQUIRED), ("beta", _REQUIRED), ("eps", 1e-5)], _layernorm),
    "concat": ([("xs", _REQUIRED), ("axis", 0)], _concat),
    "cast": ([("x", _REQUIRED), ("dtype", _REQUIRED)], _cast),
    "slice": ([("x", _REQUIRED), ("begin", _REQUIRED), ("size", _REQUIRED)], _slice),
    "pad": ([("x", _REQUIRED), ("pads", _REQUIRED), ("value", 0)], _pad),
    "broadcast": ([("x", _REQUIRED), ("shape", _REQUIRED)], _broadcast_fn),
    "gather": ([("x", _REQUIRED), ("indices", _REQUIRED), ("axis", 0)], _gather),
    "where": ([("cond", _REQUIRED), ("a", _REQUIRED), ("b", _REQUIRED)], _where),
    "size": ([("x", _REQUIRED), ("axis", _REQUIRED)], _size),
    "zeros": ([("shape", _REQUIRED), ("dtype", DType("f32"))], _filled(0)),
    "ones": ([("shape", _REQUIRED), ("dtype", DType("f32"))], _filled(1)),
    "full": ([("shape", _REQUIRED), ("value", _REQUIRED), ("dtype", DType("f32"))], _filled(None)),
    "arange": ([("start", _REQUIRED), ("stop", None), ("dtype", DType("i32"))], _arange),
    "dynamic_slice": ([("x", _REQUIRED), ("start", _REQUIRED), ("size", _REQUIRED)], _dynamic_slice),
    "dynamic_update_slice": ([("x", _REQUIRED), ("update", _REQUIRED), ("start", _REQUIRED)],
                             _dynamic_update_slice),
    "sort": _axis_op("sort"),
    "cumprod": _axis_op("cumprod"),
    "argmax": _arg("argmax"),
    "argmin": _arg("argmin"),
}


def elaborate(src: str, entry: str = "main", weights: Optional[dict] = None, dims: Optional[dict] = None,
              seed: Optional[int] = 0, name: Optional[str] = None) -> Graph:
    """A .mira program as a harness Graph: the entry function inlined, its shape symbols and
    int parameters from `dims`, its const parameters from `weights` or drawn from `seed`
    (None: all must be given)."""
    g = Elaborator(parse(src), name or entry).entry(entry, weights or {}, dims or {}, seed)
    g.check()
    return g
