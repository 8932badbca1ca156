"""Textual MLIR reader for the StableHLO programs the lowering accepts.

The reference lowers a deserialized jaxlib module in-process through jaxlib's
MLIR bindings (python/pjrt_ocl/lowering.py:2976-3119, 3145-3157).  This build has
no hard dependency on jaxlib: the lowering reads MLIR *text*.  When jaxlib is
present the lowering service turns a VHLO portable artifact into text with
jaxlib's own deserializer and printer; without it, text is the program format.

Accepted syntax:
  * the generic operation form, which is what an MLIR printer emits with
    ``print_generic_op_form=True`` (every op, every attribute, regions);
  * the pretty forms that JAX's ``.as_text()`` prints for the module and
    function wrappers and for the common StableHLO ops (elementwise, constant,
    broadcast_in_dim, reshape, convert, transpose, dot_general, compare,
    select, iota, reduce with ``applies``, return, call).

The result is a small tree: ``Module`` -> ``Func`` -> ``Block`` -> ``Op`` with
``Value`` operands/results, attributes parsed into Python values (ints, floats,
lists, dicts) or the typed wrappers below.
"""
from __future__ import annotations

import dataclasses
import re

import numpy as np


class MlirSyntaxError(ValueError):
    pass


# ---- types ----------------------------------------------------------------------------

ELEM_TYPES = {"f32", "f64", "f16", "bf16", "i1", "i8", "i16", "i32", "i64", "ui8", "ui16", "ui32", "ui64",
              "si32", "si64", "complex<f32>", "complex<f64>", "f8E4M3FN", "f8E5M2"}


@dataclasses.dataclass(frozen=True)
class TensorType:
    shape: tuple
    elem: str

    @property
    def n(self) -> int:
        out = 1
        for d in self.shape:
            out *= d
        return out

    def __str__(self):
        return "tensor<" + "".join(f"{d}x" for d in self.shape) + self.elem + ">"


@dataclasses.dataclass(frozen=True)
class OtherType:
    text: str


@dataclasses.dataclass(frozen=True)
class FunctionType:
    inputs: tuple
    results: tuple


def parse_tensor_type(body: str) -> TensorType:
    """``4x8xf32`` / ``f32`` / ``?x4xf32`` (the text between ``tensor<`` and ``>``)."""
    body = body.split(",")[0].strip()          # drop an encoding (#stablehlo.bounds<...>)
    parts = body.split("x")
    dims = []
    k = 0
    while k < len(parts) - 1 and re.fullmatch(r"\d+|\?", parts[k]):
        if parts[k] == "?":
            raise MlirSyntaxError(f"dynamic shape unsupported: tensor<{body}>")
        dims.append(int(parts[k]))
        k += 1
    elem = "x".join(parts[k:])
    return TensorType(tuple(dims), elem)


# ---- attributes -------------------------------------------------------------------------

@dataclasses.dataclass
class DenseAttr:
    text: str             # the text between dense< and >
    type: object          # TensorType

    def array(self) -> np.ndarray:
        return dense_to_numpy(self.text, self.type)


@dataclasses.dataclass
class ArrayAttr:           # array<i64: 1, 2>
    elem: str
    values: list


@dataclasses.dataclass
class EnumAttr:            # #stablehlo<comparison_direction LT>
    dialect: str
    kind: str
    value: str


@dataclasses.dataclass
class StructAttr:          # #stablehlo.gather<offset_dims = [1], ...>
    name: str
    fields: dict


@dataclasses.dataclass
class TypedInt:            # 0 : i64
    value: int
    type: str


@dataclasses.dataclass
class SymbolRef:
    name: str


@dataclasses.dataclass
class RawAttr:
    text: str


def attr_ints(a) -> list:
    """An attribute holding a list of integers, in any of its spellings."""
    if isinstance(a, ArrayAttr):
        return [int(v) for v in a.values]
    if isinstance(a, DenseAttr):
        return [int(v) for v in a.array().reshape(-1)]
    if isinstance(a, list):
        return [int(v.value if isinstance(v, TypedInt) else v) for v in a]
    if isinstance(a, TypedInt):
        return [a.value]
    if isinstance(a, int):
        return [a]
    raise MlirSyntaxError(f"expected an integer list attribute, got {a!r}")


def attr_int(a) -> int:
    if isinstance(a, TypedInt):
        return a.value
    if isinstance(a, bool):
        return int(a)
    if isinstance(a, int):
        return a
    raise MlirSyntaxError(f"expected an integer attribute, got {a!r}")


def attr_enum(a) -> str:
    if isinstance(a, EnumAttr):
        return a.value
    if isinstance(a, str):
        return a
    if isinstance(a, RawAttr):
        return a.text.split()[-1].rstrip(">")
    raise MlirSyntaxError(f"expected an enum attribute, got {a!r}")


_FLOAT_NP = {"f32": np.float32, "f64": np.float64, "f16": np.float16}
_INT_NP = {"i1": np.bool_, "i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64,
           "ui8": np.uint8, "ui16": np.uint16, "ui32": np.uint32, "ui64": np.uint64,
           "si32": np.int32, "si64": np.int64}


def _np_dtype(elem: str):
    if elem in _FLOAT_NP:
        return _FLOAT_NP[elem]
    if elem == "bf16":
        return np.float32             # values widen to f32; the lowering rounds to bf16
    if elem in _INT_NP:
        return _INT_NP[elem]
    raise MlirSyntaxError(f"unsupported element type {elem}")


def _scalar(tok: str, elem: str):
    tok = tok.strip()
    if tok in ("true", "false"):
        return tok == "true"
    if elem in _INT_NP:
        return int(tok, 0)
    if tok.lower().startswith("0x"):              # a float as its bit pattern
        bits = int(tok, 16)
        if elem == "f64":
            return float(np.array([bits], np.uint64).view(np.float64)[0])
        if elem == "f16":
            return float(np.array([bits], np.uint16).view(np.float16)[0])
        if elem == "bf16":
            return float(np.array([bits << 16], np.uint32).view(np.float32)[0])
        return float(np.array([bits], np.uint32).view(np.float32)[0])
    return float(tok)


def dense_to_numpy(text: str, ttype: TensorType) -> np.ndarray:
    """The value of ``dense<text> : ttype``: a splat, a nested list or a hex blob."""
    text = text.strip()
    npdt = _np_dtype(ttype.elem)
    if text.startswith('"0x') or text.startswith('"0X'):
        raw = bytes.fromhex(text[3:-1])
        if ttype.elem == "bf16":
            arr = (np.frombuffer(raw, "<u2").astype(np.uint32) << 16).view(np.float32)
        elif ttype.elem == "i1":
            arr = np.frombuffer(raw, np.uint8).astype(np.bool_)
        else:
            arr = np.frombuffer(raw, np.dtype(npdt).newbyteorder("<"))
        if arr.size == 1:
            return np.full(ttype.shape, arr[0], npdt)
        return arr.reshape(ttype.shape).astype(npdt)
    if text.startswith("["):
        flat = [_scalar(t, ttype.elem) for t in re.split(r"[\[\],\s]+", text) if t]
        arr = np.array(flat, dtype=npdt)
        if arr.size == 1 and ttype.n != 1:
            return np.full(ttype.shape, arr[0], npdt)
        return arr.reshape(ttype.shape)
    if text.startswith("("):
        raise MlirSyntaxError("complex constants are unsupported")
    return np.full(ttype.shape, _scalar(text, ttype.elem), npdt)


# ---- IR tree ------------------------------------------------------------------------------

@dataclasses.dataclass(eq=False)
class Value:
    name: str
    type: object

    def __repr__(self):
        return f"%{self.name}:{self.type}"


@dataclasses.dataclass(eq=False)
class Block:
    args: list
    ops: list


@dataclasses.dataclass(eq=False)
class Op:
    name: str
    operands: list
    results: list
    attrs: dict
    regions: list            # list of regions, each a list of Blocks

    def attr(self, key, default=None):
        return self.attrs.get(key, default)


@dataclasses.dataclass(eq=False)
class Func:
    name: str
    args: list
    result_types: list
    body: Block
    visibility: str = "public"
    arg_attrs: list = dataclasses.field(default_factory=list)   # one dict per argument

    def arg_attr(self, i: int, key: str, default=None):
        return self.arg_attrs[i].get(key, default) if i < len(self.arg_attrs) else default


@dataclasses.dataclass(eq=False)
class Module:
    funcs: dict

    @property
    def main(self) -> Func:
        if "main" not in self.funcs:
            raise MlirSyntaxError("no func.func @main in module")
        return self.funcs["main"]


# ---- parser -------------------------------------------------------------------------------

_ID = re.compile(r"[A-Za-z_][A-Za-z0-9_$.\-]*")
_VAL = re.compile(r"%([A-Za-z0-9_$.\-]+)(?:#(\d+))?")
_NUM = re.compile(r"[-+]?(?:0x[0-9a-fA-F]+|\d+\.?\d*(?:[eE][-+]?\d+)?|inf|nan)")

# ops whose pretty form is "op %a, %b : type" (result type = the type)
_PRETTY_EW = {"add", "subtract", "multiply", "divide", "maximum", "minimum", "power", "atan2", "remainder", "and",
              "or", "xor", "shift_left", "shift_right_logical", "shift_right_arithmetic", "negate",
              "exponential", "log", "sqrt", "rsqrt", "tanh", "abs", "floor", "ceil", "sign", "log_plus_one",
              "exponential_minus_one", "cbrt", "sine", "cosine", "tan", "round_nearest_even",
              "round_nearest_afz", "not", "logistic", "is_finite", "popcnt", "count_leading_zeros"}


class _Parser:
    def __init__(self, text: str):
        # drop comments and location tails
        text = re.sub(r"//[^\n]*", "", text)
        self.s = text
        self.i = 0
        self.scopes = [{}]

    # -- lexical helpers --
    def ws(self):
        s, i = self.s, self.i
        while i < len(s):
            if s[i].isspace():
                i += 1
            elif s.startswith("loc(", i):
                i = self._balanced_end(i + 3, "(", ")")
            else:
                break
        self.i = i

    def peek(self, lit: str) -> bool:
        self.ws()
        return self.s.startswith(lit, self.i)

    def eat(self, lit: str) -> bool:
        if self.peek(lit):
            self.i += len(lit)
            return True
        return False

    def expect(self, lit: str):
        if not self.eat(lit):
            raise self.error(f"expected {lit!r}")

    def error(self, msg):
        line = self.s.count("\n", 0, self.i) + 1
        ctx = self.s[self.i:self.i + 60].replace("\n", " ")
        return MlirSyntaxError(f"line {line}: {msg} at {ctx!r}")

    def ident(self) -> str:
        self.ws()
        m = _ID.match(self.s, self.i)
        if not m:
            raise self.error("expected an identifier")
        self.i = m.end()
        return m.group(0)

    def string(self) -> str:
        self.ws()
        if self.s[self.i] != '"':
            raise self.error("expected a string")
        j = self.i + 1
        out = []
        while self.s[j] != '"':
            if self.s[j] == "\\":
                nxt = self.s[j + 1]
                if nxt in '"\\':
                    out.append(nxt)
                    j += 2
                    continue
                if nxt == "n":
                    out.append("\n")
                    j += 2
                    continue
                out.append(chr(int(self.s[j + 1:j + 3], 16)))
                j += 3
                continue
            out.append(self.s[j])
            j += 1
        self.i = j + 1
        return "".join(out)

    def _balanced_end(self, i: int, open_c: str, close_c: str) -> int:
        """Index just past the bracket that closes the one at s[i]."""
        depth = 0
        s = self.s
        while i < len(s):
            c = s[i]
            if c == '"':
                i += 1
                while s[i] != '"':
                    i += 2 if s[i] == "\\" else 1
            elif c == open_c:
                depth += 1
            elif c == close_c:
                depth -= 1
                if depth == 0:
                    return i + 1
            i += 1
        raise self.error("unbalanced brackets")

    def balanced(self, open_c="<", close_c=">") -> str:
        """Raw text inside the bracket pair starting at the cursor."""
        self.ws()
        if self.s[self.i] != open_c:
            raise self.error(f"expected {open_c!r}")
        end = self._angle_end(self.i) if open_c == "<" else self._balanced_end(self.i, open_c, close_c)
        body = self.s[self.i + 1:end - 1]
        self.i = end
        return body

    def _angle_end(self, i: int) -> int:
        # '<' ... '>' where '->' is not a closer
        depth = 0
        s = self.s
        while i < len(s):
            c = s[i]
            if c == '"':
                i += 1
                while s[i] != '"':
                    i += 2 if s[i] == "\\" else 1
            elif c == "<":
                depth += 1
            elif c == ">" and s[i - 1] != "-":
                depth -= 1
                if depth == 0:
                    return i + 1
            i += 1
        raise self.error("unbalanced <>")

    # -- values --
    def lookup(self, name: str, idx) -> Value:
        for sc in reversed(self.scopes):
            if name in sc:
                v = sc[name]
                if isinstance(v, list):
                    return v[int(idx or 0)]
                if idx not in (None, "0"):
                    raise self.error(f"%{name} has one result")
                return v
        raise self.error(f"undefined value %{name}")

    def value_ref(self) -> Value:
        self.ws()
        m = _VAL.match(self.s, self.i)
        if not m:
            raise self.error("expected an SSA value")
        self.i = m.end()
        return self.lookup(m.group(1), m.group(2))

    def value_list(self, close=")") -> list:
        vals = []
        if self.peek(close):
            return vals
        while True:
            vals.append(self.value_ref())
            if not self.eat(","):
                return vals

    # -- types --
    def type_(self):
        self.ws()
        if self.eat("tensor<"):
            self.i -= 1
            return parse_tensor_type(self.balanced("<", ">"))
        if self.peek("("):
            ins = self.type_list_paren()
            self.expect("->")
            if self.peek("("):
                outs = self.type_list_paren()
            else:
                outs = [self.type_()]
            return FunctionType(tuple(ins), tuple(outs))
        if self.peek("!"):
            self.i += 1
            name = self.ident()
            if self.peek("<"):
                name += "<" + self.balanced() + ">"
            return OtherType("!" + name)
        name = self.ident()
        if self.peek("<") and name in ("complex", "vector", "memref"):
            name += "<" + self.balanced() + ">"
        return OtherType(name)

    def type_list_paren(self) -> list:
        self.expect("(")
        out = []
        if self.eat(")"):
            return out
        while True:
            out.append(self.type_())
            if self.peek("{"):            # argument / result attributes
                self.attr_dict()
            if not self.eat(","):
                break
        self.expect(")")
        return out

    # -- attributes --
    def attr_dict(self) -> dict:
        self.expect("{")
        out = {}
        if self.eat("}"):
            return out
        while True:
            self.ws()
            key = self.string() if self.s[self.i] == '"' else self.ident()
            if self.eat("="):
                out[key] = self.attr()
            else:
                out[key] = True            # unit attribute
            if not self.eat(","):
                break
        self.expect("}")
        return out

    def attr(self):
        self.ws()
        s, i = self.s, self.i
        if s.startswith("dense<", i):
            self.i += 5
            body = self.balanced()
            ttype = None
            if self.eat(":"):
                ttype = self.type_()
            return DenseAttr(body, ttype)
        if s.startswith("array<", i):
            self.i += 5
            body = self.balanced()
            if ":" in body:
                elem, vals = body.split(":", 1)
                vs = [_scalar(v, elem.strip()) for v in vals.split(",") if v.strip()]
            else:
                elem, vs = body, []
            return ArrayAttr(elem.strip(), vs)
        if s.startswith("#", i):
            self.i += 1
            name = self.ident()
            body = self.balanced() if self.peek("<") else ""
            if "." in name:                        # #stablehlo.gather<...>
                return StructAttr(name, _struct_fields(body))
            toks = body.split()
            return EnumAttr(name, toks[0] if toks else "", toks[-1] if toks else "")
        if s.startswith('"', i):
            return self.string()
        if s.startswith("[", i):
            self.i += 1
            out = []
            if self.eat("]"):
                return out
            while True:
                out.append(self.attr())
                if not self.eat(","):
                    break
            self.expect("]")
            return out
        if s.startswith("{", i):
            return self.attr_dict()
        if s.startswith("@", i):
            self.i += 1
            return SymbolRef(self.ident())
        if s.startswith("(", i):
            return self.type_()                     # function_type
        m = _NUM.match(s, i)
        if m and (m.group(0)[0].isdigit() or m.group(0)[0] in "+-" or m.group(0) in ("inf", "nan")):
            self.i = m.end()
            tok = m.group(0)
            if self.eat(":"):
                ty = self.type_()
                tname = ty.text if isinstance(ty, OtherType) else str(ty)
                if tname.startswith(("f", "bf")):
                    return _scalar(tok, tname)
                return TypedInt(int(tok, 0), tname)
            return int(tok, 0) if re.fullmatch(r"[-+]?(0x[0-9a-fA-F]+|\d+)", tok) else float(tok)
        if s.startswith("true", i) or s.startswith("false", i):
            word = self.ident()
            return word == "true"
        if s.startswith("unit", i):
            self.ident()
            return True
        # a type used as an attribute (e.g. tensor<...>) or an unknown keyword
        ty = self.type_()
        return ty

    # -- operations --
    def op(self):
        """One operation; returns an Op, or None at a block terminator brace."""
        self.ws()
        results = []
        if self.s.startswith("%", self.i):
            while True:
                self.ws()
                m = re.compile(r"%([A-Za-z0-9_$.\-]+)(?::(\d+))?").match(self.s, self.i)
                if not m:
                    raise self.error("expected a result name")
                self.i = m.end()
                results.append((m.group(1), int(m.group(2) or 1)))
                if not self.eat(","):
                    break
            self.expect("=")
        self.ws()
        if self.s.startswith('"', self.i):
            op = self.generic_op()
        else:
            op = self.pretty_op(sum(c for _, c in results))
        # bind result names
        k = 0
        for name, cnt in results:
            vals = op.results[k:k + cnt]
            k += cnt
            self.scopes[-1][name] = vals if cnt > 1 else vals[0]
        return op

    def generic_op(self) -> Op:
        name = self.string()
        self.expect("(")
        operands = self.value_list()
        self.expect(")")
        attrs = {}
        if self.peek("<{"):
            self.i += 1
            attrs.update(self.attr_dict())
            self.expect(">")
        regions = []
        if self.peek("({"):
            self.expect("(")
            while True:
                regions.append(self.region())
                if not self.eat(","):
                    break
            self.expect(")")
        if self.peek("{"):
            attrs.update(self.attr_dict())
        self.expect(":")
        ft = self.type_()
        if not isinstance(ft, FunctionType):
            raise self.error("expected a function type after a generic op")
        results = [Value(f"r{id(ft)}_{k}", t) for k, t in enumerate(ft.results)]
        return Op(name, operands, results, attrs, regions)

    def region(self) -> list:
        self.expect("{")
        blocks = []
        self.scopes.append({})
        while not self.eat("}"):
            blocks.append(self.block())
        self.scopes.pop()
        return blocks

    def block(self) -> Block:
        args = []
        self.ws()
        if self.s.startswith("^", self.i):
            self.i += 1
            self.ident()
            if self.eat("("):
                while not self.eat(")"):
                    self.ws()
                    m = _VAL.match(self.s, self.i)
                    self.i = m.end()
                    self.expect(":")
                    v = Value(m.group(1), self.type_())
                    if self.peek("loc("):
                        self.ws()
                    self.scopes[-1][m.group(1)] = v
                    args.append(v)
                    self.eat(",")
            self.expect(":")
        ops = []
        while True:
            self.ws()
            if self.s.startswith("}", self.i) or self.s.startswith("^", self.i):
                break
            ops.append(self.op())
        return Block(args, ops)

    # -- pretty forms --
    def _typed_results(self, n_results: int):
        """': T' (result type T), ': (Ts) -> T' or ': (Ts) -> (Ts)'."""
        self.expect(":")
        ty = self.type_()
        if isinstance(ty, FunctionType):
            outs = list(ty.results)
        else:
            outs = [ty]
            while self.eat(","):
                outs.append(self.type_())
            if n_results > 1 and len(outs) == 2 * n_results:
                outs = outs[n_results:]
        return [Value(f"p{id(self)}_{self.i}_{k}", t) for k, t in enumerate(outs[-max(1, n_results):])]

    def _dims_list(self) -> list:
        self.expect("[")
        out = []
        while not self.eat("]"):
            self.ws()
            m = re.compile(r"-?\d+").match(self.s, self.i)
            out.append(int(m.group(0)))
            self.i = m.end()
            self.eat(",")
        return out

    def pretty_op(self, n_results: int) -> Op:
        name = self.ident()
        if "." not in name:
            name = {"return": "func.return", "call": "func.call"}.get(name, name)
        short = name.split(".", 1)[1] if name.startswith("stablehlo.") else None
        attrs = {}
        if name in ("func.return", "stablehlo.return"):
            operands = [] if self.peek("}") else self.value_list(close=":")
            if operands:
                self.expect(":")
                self.type_()
                while self.eat(","):
                    self.type_()
            return Op(name, operands, [], attrs, [])
        if name == "func.call":
            self.expect("@")
            callee = self.ident()
            self.expect("(")
            operands = self.value_list()
            self.expect(")")
            res = self._typed_results(n_results)
            return Op(name, operands, res, {"callee": SymbolRef(callee)}, [])
        if short == "constant":
            a = self.attr()
            if isinstance(a, DenseAttr) and a.type is None:
                self.expect(":")
                a.type = self.type_()
            return Op(name, [], [Value(f"c{self.i}", a.type)], {"value": a}, [])
        if short in _PRETTY_EW or short in ("convert", "reshape", "bitcast_convert", "select", "clamp",
                                            "optimization_barrier", "dynamic_update_slice"):
            operands = self.value_list(close=":")
            return Op(name, operands, self._typed_results(n_results), attrs, [])
        if short in ("dynamic_slice", "concatenate"):
            # %r = stablehlo.dynamic_slice %x, %i, %j, sizes = [1, 4] : ...
            # %r = stablehlo.concatenate %a, %b, dim = 0 : ...
            operands = []
            while True:
                self.ws()
                if self.s.startswith("%", self.i):
                    operands.append(self.value_ref())
                else:
                    key = self.ident()
                    self.expect("=")
                    if key == "sizes":
                        attrs["slice_sizes"] = ArrayAttr("i64", self._dims_list())
                    else:
                        attrs["dimension"] = TypedInt(int(self.ident_or_int()), "i64")
                if not self.eat(","):
                    break
            return Op(name, operands, self._typed_results(n_results), attrs, [])
        if short == "slice":
            # %r = stablehlo.slice %x [0:2, 1:3:1] : (T) -> T
            operands = [self.value_ref()]
            self.expect("[")
            starts, limits, strides = [], [], []
            while not self.eat("]"):
                self.ws()
                m = re.compile(r"(\d+):(\d+)(?::(\d+))?").match(self.s, self.i)
                if not m:
                    raise self.error("expected start:limit[:stride]")
                self.i = m.end()
                starts.append(int(m.group(1)))
                limits.append(int(m.group(2)))
                strides.append(int(m.group(3) or 1))
                self.eat(",")
            attrs.update(start_indices=ArrayAttr("i64", starts), limit_indices=ArrayAttr("i64", limits),
                         strides=ArrayAttr("i64", strides))
            return Op(name, operands, self._typed_results(n_results), attrs, [])
        if short in ("broadcast_in_dim", "transpose"):
            operands = [self.value_ref()]
            self.expect(",")
            self.ident()                       # dims
            self.expect("=")
            key = "broadcast_dimensions" if short == "broadcast_in_dim" else "permutation"
            attrs[key] = ArrayAttr("i64", self._dims_list())
            return Op(name, operands, self._typed_results(n_results), attrs, [])
        if short == "iota":
            self.ident()                       # dim
            self.expect("=")
            attrs["iota_dimension"] = TypedInt(int(self.ident_or_int()), "i64")
            return Op(name, [], self._typed_results(n_results), attrs, [])
        if short == "compare":
            direction = self.ident()
            self.expect(",")
            a = self.value_ref()
            self.expect(",")
            b = self.value_ref()
            attrs["comparison_direction"] = EnumAttr("stablehlo", "comparison_direction", direction)
            if self.eat(","):
                attrs["compare_type"] = EnumAttr("stablehlo", "comparison_type", self.ident())
            return Op(name, [a, b], self._typed_results(n_results), attrs, [])
        if short == "dot_general":
            a = self.value_ref()
            self.expect(",")
            b = self.value_ref()
            fields = {"lhs_batching_dimensions": [], "rhs_batching_dimensions": [],
                      "lhs_contracting_dimensions": [], "rhs_contracting_dimensions": []}
            while self.eat(","):
                key = self.ident()
                self.expect("=")
                if key in ("batching_dims", "contracting_dims"):
                    lhs = self._dims_list()
                    self.expect("x")
                    rhs = self._dims_list()
                    pre = "batching" if key == "batching_dims" else "contracting"
                    fields[f"lhs_{pre}_dimensions"] = lhs
                    fields[f"rhs_{pre}_dimensions"] = rhs
                else:
                    self.attr()                # precision / algorithm
            attrs["dot_dimension_numbers"] = StructAttr("stablehlo.dot", fields)
            return Op(name, [a, b], self._typed_results(n_results), attrs, [])
        if short == "reduce":
            # %r = stablehlo.reduce(%x init: %c) applies stablehlo.add across dimensions = [1] : ...
            self.expect("(")
            x = self.value_ref()
            self.ident()                       # init
            self.expect(":")
            init = self.value_ref()
            self.expect(")")
            if not self.eat("applies"):
                raise self.error("only the 'applies' form of a pretty reduce is supported; "
                                 "print with print_generic_op_form=True")
            body_op = self.ident()
            self.ident()                       # across
            self.ident()                       # dimensions
            self.expect("=")
            attrs["dimensions"] = ArrayAttr("i64", self._dims_list())
            res = self._typed_results(n_results)
            et = TensorType((), init.type.elem)
            p, q = Value("ra", et), Value("rb", et)
            r = Value("rr", et)
            body = Block([p, q], [Op(body_op, [p, q], [r], {}, []), Op("stablehlo.return", [r], [], {}, [])])
            return Op(name, [x, init], res, attrs, [[body]])
        raise self.error(f"pretty form of {name} is not supported; print the module with "
                         f"print_generic_op_form=True")

    def _at_attr_dict(self) -> bool:
        """'{key = ...' (an attribute dictionary) rather than '{ %0 = ...' (a body)."""
        self.ws()
        return re.compile(r'\{\s*(?:[A-Za-z_][\w.$\-]*|"[^"]*")\s*(?:=|\}|,)').match(self.s, self.i) is not None

    def ident_or_int(self) -> str:
        self.ws()
        m = re.compile(r"\d+").match(self.s, self.i)
        if m:
            self.i = m.end()
            return m.group(0)
        return self.ident()

    # -- module / functions --
    def module(self) -> Module:
        funcs = {}
        self.ws()
        if self.eat('"builtin.module"'):
            self.expect("(")
            self.expect(")")
            if self.peek("<{"):
                self.i += 1
                self.attr_dict()
                self.expect(">")
            self.expect("(")
            self.expect("{")
            self.ws()
            if self.s.startswith("^", self.i):
                self.ident()
                self.expect(":")
            while not self.eat("}"):
                f = self.func()
                funcs[f.name] = f
            self.expect(")")
            if self.peek("{"):
                self.attr_dict()
            self.expect(":")
            self.type_()
            return Module(funcs)
        wrapped = False
        if self.eat("module"):
            wrapped = True
            if self.peek("@"):
                self.i += 1
                self.ident()
            if self.eat("attributes"):
                self.attr_dict()
            self.expect("{")
        while True:
            self.ws()
            if self.i >= len(self.s) or self.s.startswith("}", self.i):
                break
            f = self.func()
            funcs[f.name] = f
        if wrapped:
            self.expect("}")
        return Module(funcs)

    def func(self) -> Func:
        self.ws()
        self.scopes = [{}]
        if self.s.startswith('"func.func"', self.i):
            op = self.generic_op_func()
            return op
        self.expect("func.func")
        vis = "public"
        if self.peek("public") or self.peek("private"):
            vis = self.ident()
        self.expect("@")
        name = self.ident()
        self.expect("(")
        args, arg_attrs = [], []
        while not self.eat(")"):
            self.ws()
            m = _VAL.match(self.s, self.i)
            self.i = m.end()
            self.expect(":")
            v = Value(m.group(1), self.type_())
            arg_attrs.append(self.attr_dict() if self.peek("{") else {})
            self.scopes[-1][m.group(1)] = v
            args.append(v)
            self.eat(",")
        rtypes = []
        if self.eat("->"):
            if self.peek("("):
                rtypes = self.type_list_paren()
            else:
                rtypes = [self.type_()]
                if self._at_attr_dict():
                    self.attr_dict()
        if self.eat("attributes"):
            self.attr_dict()
        self.expect("{")
        ops = []
        while not self.eat("}"):
            ops.append(self.op())
        return Func(name, args, rtypes, Block(args, ops), vis, arg_attrs)

    def generic_op_func(self) -> Func:
        self.string()                                   # "func.func"
        self.expect("(")
        self.expect(")")
        props = {}
        if self.peek("<{"):
            self.i += 1
            props.update(self.attr_dict())
            self.expect(">")
        self.expect("(")
        (blocks,) = [self.region()]
        self.expect(")")
        if self.peek("{"):
            props.update(self.attr_dict())
        self.expect(":")
        self.type_()
        ft = props.get("function_type")
        name = props.get("sym_name", "main")
        body = blocks[0]
        aa = props.get("arg_attrs")
        arg_attrs = [d if isinstance(d, dict) else {} for d in (aa.values if isinstance(aa, ArrayAttr) else aa or [])]
        return Func(name, body.args, list(ft.results) if isinstance(ft, FunctionType) else [], body,
                    props.get("sym_visibility", "public"), arg_attrs)


def _struct_fields(body: str) -> dict:
    """``offset_dims = [1], collapsed_slice_dims = [0], index_vector_dim = 1``."""
    out = {}
    for m in re.finditer(r"([A-Za-z_]+)\s*=\s*(\[[^\]]*\]|[-\w]+)", body):
        key, val = m.group(1), m.group(2)
        if val.startswith("["):
            out[key] = [int(v) for v in re.findall(r"-?\d+", val)]
        elif re.fullmatch(r"-?\d+", val):
            out[key] = int(val)
        else:
            out[key] = val
    return out


def parse_module(text: str) -> Module:
    """Parse MLIR text (a module, or bare func.func definitions) into a Module."""
    p = _Parser(text)
    mod = p.module()
    p.ws()
    if p.i != len(p.s):
        raise p.error("trailing text after the module")
    return mod
