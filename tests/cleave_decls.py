"""Reads the cleave-side drop-in declarations of the repository's integration
guide (its ```cleave blocks) and lowers each `extern(symbol) fn` the way the reference compiler
would, for tests/test_integration_decls.py (CPU) and tests/test_gpu_extern.py.

What is restated from the reference (read as text, not run):
  * the scalar types that have a C-ABI shape: i8 i16 i32 i64 f32 f64 bool
    (/root/reference/cleave/src/rust_bindings.rs:21-35);
  * an array parameter `[T; N]` lowers to two arguments, the aligned pointer
    and an i64 element count (/root/reference/cleave/src/mlir_lower.rs:1096-1114,
    :1720-1751);
  * an array result lowers to an i64 C result, the cleave-level value being
    the first array argument (mlir_lower.rs:1062-1075, :1123-1124); a `()`
    result lowers to no C result (:1076-1094);
  * a top-level `extern fn` may not be generic (ExternFnCannotBeGeneric,
    /root/reference/cleave/src/callgraph.rs:264-269);
  * the stdlib algebras an impl here may name, with their parameters and
    method signatures (/root/reference/stdlib/nn/nn.cleave:21-25, :97-109;
    stdlib/num/num.cleave:63-69; stdlib/linalg/matrix.cleave:22-24;
    stdlib/linalg/tensor.cleave:113-114; stdlib/io/io.cleave:12-14).
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

SCALARS = {"i8": "int8_t", "i16": "int16_t", "i32": "int32_t", "i64": "int64_t", "f32": "float",
           "f64": "double", "bool": "bool"}

# Reference algebras: name -> (parameters, {method: (param types, return type)}),
# types written over the algebra's own parameter names.
REFERENCE_ALGEBRAS = {
    "Activation": (["T"], {"relu": (["T"], "T"), "sigmoid": (["T"], "T"), "tanh": (["T"], "T")}),
    "Sum": (["Container", "T"], {"sum": (["Container"], "T")}),
    "Mean": (["Container", "T"], {"mean": (["Container"], "T")}),
    "Max": (["Container", "T"], {"max_of": (["Container"], "T")}),
    "Ring": (["T"], {"add": (["T", "T"], "T"), "sub": (["T", "T"], "T"), "mul": (["T", "T"], "T"),
                     "div": (["T", "T"], "T"), "neg": (["T"], "T"), "zero": ([], "T")}),
    "MatMul": (["A", "B", "C"], {"matmul": (["A", "B"], "C")}),
    "Index": (["Container", "Elem", "const K"], {"index": (["Container", "[i32; K]"], "Elem")}),
    "Print": (["T"], {"print": (["T"], "T")}),
}


@dataclass
class Algebra:
    name: str
    params: list[str]                      # "T", or "const K" for a const parameter
    methods: dict[str, tuple[list[str], str]]


@dataclass
class Extern:
    symbol: str
    name: str
    params: list[tuple[str, str]]          # (name, type)
    ret: str                               # "()" when absent
    impl_generics: list[str] = field(default_factory=list)   # "const N: i32" ...
    algebra: str | None = None
    algebra_args: list[str] = field(default_factory=list)
    top_level: bool = False
    fn_generics: list[str] = field(default_factory=list)


def split_top(s: str, sep: str = ",") -> list[str]:
    """Splits at `sep` outside brackets, parentheses and angle brackets."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "[(<":
            depth += 1
        elif ch in "])>":
            depth -= 1
        if ch == sep and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def cleave_blocks(text: str | None = None) -> list[str]:
    text = (ROOT / "INTEGRATION.md").read_text() if text is None else text
    blocks = re.findall(r"```cleave\n(.*?)```", text, re.S)
    return [re.sub(r"//[^\n]*", "", b) for b in blocks]


def _braced(src: str, open_at: int) -> tuple[str, int]:
    depth = 0
    for i in range(open_at, len(src)):
        if src[i] == "{":
            depth += 1
        elif src[i] == "}":
            depth -= 1
            if depth == 0:
                return src[open_at + 1:i], i + 1
    raise ValueError("unbalanced braces")


FN_RE = re.compile(r"(extern\((\w+)\)\s*)?fn\s+(\w+)\s*(<[^>]*>)?\s*\(([^)]*)\)\s*(->\s*(\[[^\]]*\]|\w+|\(\)))?\s*;",
                   re.S)


def _fn(m) -> tuple[str | None, str, list[str], list[tuple[str, str]], str]:
    symbol, name = m.group(2), m.group(3)
    gens = split_top(m.group(4)[1:-1]) if m.group(4) else []
    params = []
    for p in split_top(m.group(5)):
        pname, ptype = p.split(":", 1)
        params.append((pname.strip(), " ".join(ptype.split())))
    ret = " ".join(m.group(7).split()) if m.group(7) else "()"
    return symbol, name, gens, params, ret


def parse(blocks: list[str] | None = None) -> tuple[dict[str, Algebra], list[Extern]]:
    blocks = cleave_blocks() if blocks is None else blocks
    algebras: dict[str, Algebra] = {}
    externs: list[Extern] = []
    for src in blocks:
        pos = 0
        while pos < len(src):
            m = re.compile(r"\s*(algebra|impl|extern\(|fn\b)").match(src, pos)
            if not m:
                rest = src[pos:].strip()
                if rest:
                    raise ValueError(f"unparsed cleave text: {rest[:60]!r}")
                break
            kw = m.group(1)
            if kw == "algebra":
                h = re.compile(r"\s*algebra\s+(\w+)\s*<([^>]*)>\s*\{").match(src, pos)
                body, pos = _braced(src, h.end() - 1)
                methods = {}
                for fm in FN_RE.finditer(body):
                    _, name, _, params, ret = _fn(fm)
                    methods[name] = ([t for _, t in params], ret)
                params = [" ".join(p.split(":")[0].split()) for p in split_top(h.group(2))]
                algebras[h.group(1)] = Algebra(h.group(1), params, methods)
            elif kw == "impl":
                h = re.compile(r"\s*impl\s*(<[^{]*?>)?\s*(\w+)\s*<(.*?)>\s*\{", re.S).match(src, pos)
                gens = split_top(h.group(1)[1:-1]) if h.group(1) else []
                args = [" ".join(a.split()) for a in split_top(h.group(3))]
                body, pos = _braced(src, h.end() - 1)
                for fm in FN_RE.finditer(body):
                    symbol, name, fgens, params, ret = _fn(fm)
                    if symbol is None:
                        raise ValueError(f"impl method {name} is not extern")
                    externs.append(Extern(symbol, name, params, ret, gens, h.group(2), args, False, fgens))
            else:
                fm = FN_RE.match(src, pos)
                if not fm:
                    raise ValueError(f"unparsed fn near {src[pos:pos + 60]!r}")
                symbol, name, fgens, params, ret = _fn(fm)
                externs.append(Extern(symbol or name, name, params, ret, [], None, [], True, fgens))
                pos = fm.end()
    return algebras, externs


ARRAY_RE = re.compile(r"^\[\s*(\w+)\s*;\s*(\w+)\s*\]$")


def is_array(t: str) -> bool:
    return bool(ARRAY_RE.match(t))


def array_elem(t: str) -> str:
    return ARRAY_RE.match(t).group(1)


def type_errors(t: str, consts: set[str]) -> list[str]:
    """Why `t` is not a cleave type that can cross an extern (empty when it is)."""
    if t in SCALARS:
        return []
    m = ARRAY_RE.match(t)
    if not m:
        return [f"{t!r} is neither a cleave scalar nor an array of one"]
    errs = []
    if m.group(1) not in SCALARS:
        errs.append(f"array element {m.group(1)!r} of {t!r} is not a cleave scalar")
    if not (m.group(2).isdigit() or m.group(2) in consts):
        errs.append(f"array length {m.group(2)!r} of {t!r} is neither a literal nor a const generic in scope")
    return errs


def lower(e: Extern) -> tuple[str, list[tuple[str, bool]], int | None]:
    """The C prototype the reference's lowering gives `e`: (C return type,
    [(C parameter type, is_pointer)], index among e.params of the array the
    cleave result is, or None)."""
    cparams: list[tuple[str, bool]] = []
    identity = None
    for i, (_, t) in enumerate(e.params):
        if is_array(t):
            if identity is None:
                identity = i
            cparams.append((SCALARS[array_elem(t)], True))
            cparams.append(("int64_t", False))
        else:
            cparams.append((SCALARS[t], False))
    if is_array(e.ret):
        return "int64_t", cparams, identity
    if e.ret == "()":
        return "void", cparams, None
    return SCALARS[e.ret], cparams, None


def header_prototypes() -> dict[str, tuple[str, list[tuple[bool, str, bool]]]]:
    """include/cleave_hip.h: symbol -> (return type, [(const, base type, is_pointer)])."""
    src = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "cleave_hip.h").read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^CLEAVE_HIP_API\s+(.*?)\b(cleave_hip_\w+)\(([^)]*)\);", src, re.M | re.S):
        params = []
        text = " ".join(m.group(3).split())
        if text not in ("", "void"):
            for p in text.split(","):
                pm = re.match(r"(const\s+)?(\w+)\s*(\*?)\s*\w+$", p.strip())
                params.append((bool(pm.group(1)), pm.group(2), pm.group(3) == "*"))
        out[m.group(2)] = (" ".join(m.group(1).split()), params)
    return out
