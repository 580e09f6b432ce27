"""The cleave-side drop-in text of the integration guide, checked on the CPU against
what the reference's compiler accepts and emits (tests/cleave_decls.py holds
the restated rules):

  (i)   every impl names an algebra with the right number of parameters, and
        each extern method matches that algebra's signature under the impl's
        arguments;
  (ii)  every parameter and result type is a cleave type;
  (iii) lowering each declaration gives exactly include/cleave_hip.h's
        prototype for its symbol, and the array a cleave result hands back is
        the C function's first, writable pointer.
"""
from __future__ import annotations

import re

import pytest

import cleave_decls as cd


@pytest.fixture(scope="module")
def decls():
    return cd.parse()


def test_the_blocks_declare_the_drop_in(decls):
    algebras, externs = decls
    symbols = {e.symbol for e in externs}
    assert len(cd.cleave_blocks()) >= 2
    for must in ["cleave_hip_sum_f32_host", "cleave_hip_mean_f32_host", "cleave_hip_max_of_f32_host",
                 "cleave_hip_sum_i32_i64_host", "cleave_hip_index_f32_host", "cleave_hip_matmul_f32_into",
                 "cleave_hip_sigmoid_f32_into", "cleave_hip_escape_grid_i32"]:
        assert must in symbols, must


def _subst(t: str, env: dict[str, str]) -> str:
    t = t.strip()
    if t in env:
        return env[t]
    m = re.match(r"^\[\s*(\w+)\s*;\s*(\w+)\s*\]$", t)
    if m:
        return f"[{env.get(m.group(1), m.group(1))}; {env.get(m.group(2), m.group(2))}]"
    return t


def test_impls_match_their_algebras(decls):
    algebras, externs = decls
    table = {n: cd.Algebra(n, p, m) for n, (p, m) in cd.REFERENCE_ALGEBRAS.items()}
    for name in algebras:
        assert name not in table, f"{name} redeclares a reference algebra"
    table.update(algebras)
    seen: dict[tuple[str, tuple[str, ...]], set[str]] = {}
    for e in externs:
        if e.top_level:
            continue
        assert e.algebra in table, f"{e.symbol}: unknown algebra {e.algebra}"
        alg = table[e.algebra]
        assert len(e.algebra_args) == len(alg.params), (
            f"{e.symbol}: {e.algebra} takes {len(alg.params)} parameters, the impl gives {len(e.algebra_args)}")
        env = {p.replace("const ", "").strip(): a for p, a in zip(alg.params, e.algebra_args)}
        assert e.name in alg.methods, f"{e.symbol}: {e.algebra} has no method {e.name}"
        ptypes, ret = alg.methods[e.name]
        assert [_subst(t, env) for t in ptypes] == [t for _, t in e.params], (
            f"{e.symbol}: parameters {[t for _, t in e.params]} do not match {e.algebra}::{e.name}{ptypes}")
        assert _subst(ret, env) == e.ret, f"{e.symbol}: result {e.ret} does not match {e.algebra}::{e.name} -> {ret}"
        assert not e.fn_generics, f"{e.symbol}: method generics are not needed here"
        seen.setdefault((e.algebra, tuple(e.algebra_args)), set()).add(e.name)
    for (alg, args), methods in seen.items():
        assert methods == set(table[alg].methods), f"impl {alg}<{', '.join(args)}> misses {set(table[alg].methods) - methods}"


def test_every_type_is_a_cleave_type(decls):
    _, externs = decls
    for e in externs:
        assert not (e.top_level and e.fn_generics), f"{e.symbol}: a top-level extern fn cannot be generic"
        consts = set()
        for g in e.impl_generics:
            m = re.match(r"const\s+(\w+)\s*:\s*(\w+)$", g)
            assert m and m.group(2) == "i32", f"{e.symbol}: generic {g!r} is not a const i32"
            consts.add(m.group(1))
        errs = []
        for pname, t in e.params:
            errs += [f"{pname}: {x}" for x in cd.type_errors(t, consts)]
        if e.ret != "()":
            errs += [f"result: {x}" for x in cd.type_errors(e.ret, consts)]
        assert not errs, f"{e.symbol}: " + "; ".join(errs)
        assert "u32" not in str(e.params) and "u64" not in e.ret


def test_lowered_prototypes_match_the_header(decls):
    _, externs = decls
    protos = cd.header_prototypes()
    for e in externs:
        assert e.symbol in protos, f"{e.symbol} is not declared in include/cleave_hip.h"
        cret, cparams, identity = cd.lower(e)
        hret, hparams = protos[e.symbol]
        assert cret == hret, f"{e.symbol}: lowers to a {cret} result, the header returns {hret}"
        assert len(cparams) == len(hparams), f"{e.symbol}: lowers to {len(cparams)} C arguments, header has {len(hparams)}"
        for k, ((ct, cptr), (hconst, ht, hptr)) in enumerate(zip(cparams, hparams)):
            assert (ct, cptr) == (ht, hptr), f"{e.symbol} argument {k}: lowers to {ct}{'*' if cptr else ''}, header has {ht}{'*' if hptr else ''}"
        if identity is not None:
            # the cleave result is the first array: it must be the C function's
            # first argument and writable (the output the call fills)
            assert identity == 0, f"{e.symbol}: the first array parameter is not the first parameter"
            assert hparams[0][2] and not hparams[0][0], f"{e.symbol}: the identity array is not a writable pointer"


def test_the_checks_catch_the_mistakes_they_are_for():
    # planted on the CPU: one-parameter Sum, an unsigned grid, a non-identity
    # output order and a generic top-level extern must each be refused
    bad_sum = "impl<const N: i32> Sum<[f32; N]> { extern(cleave_hip_sum_f32_host) fn sum(c: [f32; N]) -> f32; }"
    _, ex = cd.parse([bad_sum])
    assert len(ex[0].algebra_args) != len(cd.REFERENCE_ALGEBRAS["Sum"][0])
    assert cd.type_errors("[u32; N]", {"N"})
    bad_order = ("algebra G<C> { fn g(x: C, out: C) -> C; }\n"
                 "impl<const N: i32> G<[f32; N]> { extern(cleave_hip_sigmoid_f32_host) fn g(x: [f32; N], out: [f32; N]) -> [f32; N]; }")
    _, ex = cd.parse([bad_order])
    cret, cparams, identity = cd.lower(ex[0])
    hret, hparams = cd.header_prototypes()["cleave_hip_sigmoid_f32_host"]
    assert cret != hret and hparams[0][0]  # i64 vs int32_t, and the first pointer is const
    _, ex = cd.parse(["extern(f) fn f<const N: i32>(x: [f32; N]) -> f32;"])
    assert ex[0].top_level and ex[0].fn_generics
