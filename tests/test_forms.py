"""The op-form table (include/nova_forms.h) that both carriers of the Nova ->
libnova_hip rewrite consult, the MLIR-free planner (libnova_run) and the
nova-hip-lower MLIR pass: the planner accepts exactly the forms the table
lists and declines the others with the table's reason; the pass routes every
op it lowers through the same table (it cannot be compiled in this image, so
that part is a check of its source)."""
import os
import re

import pytest

import nova_run
from conftest import REPO

HEADER = os.path.join(REPO, "include", "nova_forms.h")
PASS = os.path.join(REPO, "nova-compiler_amd", "mlir", "NovaHipLowering.cpp")
K_MAX_RANK = 8


def table():
    """kRankForms rows parsed from the header: {op: (nops, min, max)}."""
    text = open(HEADER).read()
    body = text[text.index("kRankForms[] = {"):]
    body = body[:body.index("};")]
    rows = {}
    for m in re.finditer(r'\{"([^"]+)",\s*(\d+),\s*\{([^}]*)\},\s*\{([^}]*)\}\}', body):
        def ints(s):
            s = s.replace("kMaxRank", str(K_MAX_RANK))
            return [eval(x) for x in s.split(",") if x.strip()]  # "kMaxRank - 1" etc.
        rows[m.group(1)] = (int(m.group(2)), ints(m.group(3)), ints(m.group(4)))
    return rows


def T(shape, dt="f32"):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def plan_one(args, op_line):
    """One function with `args` [(name, shape, dt)] and one op line; the
    planner's plan text, or the NovaRunError it raises."""
    sig = ", ".join(f"%{n}: {T(s, d)}" for n, s, d in args)
    text = f"func.func @f({sig}) {{\n  {op_line}\n  return\n}}\n"
    return nova_run.Program(text).plan("f")


def shp(fill, core, r):
    """A rank-r shape: the last min(r, len(core)) dims of `core` after
    leading dims of size `fill`."""
    k = min(r, len(core))
    return [fill] * (r - k) + core[len(core) - k:]


# Per op: a builder of (args, op line) for operand ranks `rk`, with shapes
# that satisfy the op's shape rules whenever the ranks do.
def build(op, rk):
    if op == "nova.matmul":
        ra, rb = rk
        nb = max(ra, rb) - 2
        ba = [2] * (ra - 2) if ra - 2 == nb else [1] * max(ra - 2, 0)
        bb = [2] * (rb - 2) if rb - 2 == nb else [1] * max(rb - 2, 0)
        a, b = ba + shp(2, [4, 8], min(ra, 2)), bb + shp(2, [8, 3], min(rb, 2))
        return [("a", a, "f32"), ("b", b, "f32")], \
            f"%r = nova.matmul %a, %b : {T(a)}, {T(b)}"
    if op == "nova.linear":
        ri, rw, rbias = rk
        x = shp(2, [4, 8], ri)
        w = shp(1, [8, 3], rw)
        b = shp(1, [3], rbias)
        return [("x", x, "f32"), ("w", w, "f32"), ("b", b, "f32")], \
            f"%r = nova.linear %x, %w, %b : {T(x)}, {T(w)}, {T(b)}"
    if op == "nova.layer_norm":
        rx, rg, rb = rk
        x = shp(2, [16], rx)
        g = shp(1, [16], rg)
        b = shp(1, [16], rb)
        return [("x", x, "f32"), ("g", g, "f32"), ("b", b, "f32")], \
            f"%y:3 = nova.layer_norm %x, %g, %b : {T(x)}, {T(g)}, {T(b)}"
    if op in ("nova.sce", "nova.sce_backward"):
        rx, rt = rk
        x = shp(2, [10], rx)
        t = [2] * rt
        res = "%s:2" if op == "nova.sce" else "%s"
        return [("x", x, "f32"), ("t", t, "i32")], f"{res} = {op} %x, %t : {T(x)}, {T(t, 'i32')}"
    if op == "nova.layer_norm_backward":
        rg, rx, rgam, rs, rr = rk
        gy = shp(2, [16], rg)
        x = shp(2, [16], rx)
        gam = shp(1, [16], rgam)
        nrows = 2 ** max(rx - 1, 0)
        def stats(r):
            return [] if r == 0 else [nrows] + [1] * (r - 1)
        s, r_ = stats(rs), stats(rr)
        return ([("gy", gy, "f32"), ("x", x, "f32"), ("g", gam, "f32"), ("s", s, "f32"),
                 ("r", r_, "f32")],
                f"%d:3 = nova.layer_norm_backward %gy, %x, %g, %s, %r : {T(gy)}, {T(x)}, "
                f"{T(gam)}, {T(s)}, {T(r_)}")
    if op in ("nova.linear_backward", "nova.matmul_backward"):
        rg, rx, rw = rk
        go = shp(2, [4, 3], rg)
        x = shp(2, [4, 8], rx)
        w = shp(1, [8, 3], rw)
        n = 3 if op == "nova.linear_backward" else 2
        return [("go", go, "f32"), ("x", x, "f32"), ("w", w, "f32")], \
            f"%g:{n} = {op} %go, %x, %w : {T(go)}, {T(x)}, {T(w)}"
    if op in ("nova.add", "nova.sub", "nova.mul", "nova.div"):
        ra, rb = rk
        a, b = [2] * ra, [2] * rb
        return [("a", a, "f32"), ("b", b, "f32")], f"%r = {op} %a, %b : {T(a)}, {T(b)}"
    if op == "nova.gelu":
        x = [2] * rk[0]
        return [("x", x, "f32")], f"%r = nova.gelu %x : {T(x)}"
    if op == "nova.gelu_backward":
        a, b = [2] * rk[0], [2] * rk[1]
        if rk[0] != rk[1]:
            return None
        return [("g", a, "f32"), ("x", b, "f32")], f"%r = nova.gelu_backward %g, %x : {T(a)}, {T(b)}"
    if op == "nova.gather":
        rt, ri = rk
        tab = shp(1, [6, 4], rt)
        idx = [2] * ri
        out = idx + tab[1:]
        return [("t", tab, "f32"), ("i", idx, "i32")], \
            f"%r = nova.gather %t [%i] : {T(tab)}, {T(idx, 'i32')} -> {T(out)}"
    if op == "nova.scatter_add":
        rb, ri, rs = rk
        base = shp(1, [6, 4], rb)
        idx = [2] * ri
        src = idx + [4] if rs == ri + 1 else None
        if src is None:
            return None
        return ([("b", base, "f32"), ("i", idx, "i32"), ("s", src, "f32")],
                f"%r = nova.scatter_add %b, %i, %s : {T(base)}, {T(idx, 'i32')}, {T(src)} -> {T(base)}")
    if op == "nova.reduce<sum>":
        x = [2] * rk[0]
        return [("x", x, "f32")], f"%r = nova.reduce<sum> %x dimension = [0] : {T(x)}"
    return None


RANK_OPS = [op for op in table() if op not in ("linalg.matmul", "linalg.batch_matmul",
                                               "nova.constant")]


# Operands whose rank is tied to another's by the shape rules:
# rank[follower] = rank[leader] + offset.
TIES = {
    "nova.sce": {1: (0, -1)}, "nova.sce_backward": {1: (0, -1)},
    "nova.layer_norm_backward": {1: (0, 0)}, "nova.linear_backward": {1: (0, 0)},
    "nova.matmul_backward": {1: (0, 0)}, "nova.gelu_backward": {1: (0, 0)},
    "nova.scatter_add": {2: (1, 1)},
}


def tie(op, rk, i):
    """rk with the ranks tied to operand i (or to their leader) adjusted."""
    rk = list(rk)
    for f, (l, off) in TIES.get(op, {}).items():
        if i == f:
            rk[l] = rk[f] - off
        else:
            rk[f] = rk[l] + off
    return rk


def rank_cases(op):
    """(ranks, in_form) around every operand's bounds: each operand at its
    minimum, one above it and at min(max, 5), with tied operands following;
    then each operand one below its minimum and one above its maximum (the
    rank check comes first, so the other operands need no adjustment)."""
    nops, lo, hi = table()[op]
    cases = []
    for i in range(nops):
        for r in sorted({lo[i], min(hi[i], lo[i] + 1), min(hi[i], 5)}):
            rk = list(lo)
            rk[i] = r
            rk = tie(op, rk, i)
            if all(lo[k] <= rk[k] <= hi[k] for k in range(nops)):
                cases.append((tuple(rk), True))
        for r in (lo[i] - 1, hi[i] + 1):
            if 0 <= r <= K_MAX_RANK and not lo[i] <= r <= hi[i]:
                rk = list(lo)
                rk[i] = r
                cases.append((tuple(rk), False))
    return cases


def test_table_parses_and_covers_the_pass_ops():
    t = table()
    for op in ("nova.matmul", "nova.linear", "nova.layer_norm", "nova.sce",
               "nova.sce_backward", "nova.layer_norm_backward", "nova.linear_backward",
               "nova.matmul_backward", "linalg.matmul", "linalg.batch_matmul"):
        assert op in t, op
    assert t["nova.matmul_backward"][2] == [2, 2, 2]       # rank 2 only
    assert t["nova.linear_backward"][2][0] == K_MAX_RANK   # rank-3 (GPT step) forms


@pytest.mark.parametrize("op", RANK_OPS)
def test_planner_accepts_exactly_the_rank_forms(op):
    seen = {True: 0, False: 0}
    for rk, in_form in rank_cases(op):
        b = build(op, rk)
        if b is None:
            continue
        args, line = b
        if in_form:
            plan_one(args, line)
        else:
            with pytest.raises(nova_run.NovaRunError, match="operand rank outside the form"):
                plan_one(args, line)
        seen[in_form] += 1
    nops, lo, hi = table()[op]
    bounded = any(lo[i] > 0 or hi[i] < K_MAX_RANK for i in range(nops))
    assert seen[True] > 0 and (seen[False] > 0 or not bounded), seen


def _mm(a, b, adt="f32", bdt="f32", cast=False, res=None):
    args = [("a", a, adt), ("b", b, bdt)]
    if not cast:
        r = f" -> {res}" if res else ""
        return args, f"%r = nova.matmul %a, %b : {T(a, adt)}, {T(b, bdt)}"
    lines = (f"%af = nova.cast %a : {T(a, adt)} -> {T(a)}\n  "
             f"%bf = nova.cast %b : {T(b, bdt)} -> {T(b)}\n  "
             f"%r = nova.matmul %af, %bf : {T(a)}, {T(b)}")
    return args, lines


@pytest.mark.parametrize("a,b,ok", [
    ([2, 3, 4, 8], [2, 3, 8, 5], True),     # equal batch dims
    ([2, 3, 4, 8], [8, 5], True),           # rank-2 operand broadcast
    ([2, 3, 4, 8], [1, 1, 8, 5], True),     # all-1 batch dims broadcast
    ([1, 4, 8], [6, 8, 5], True),
    ([2, 3, 4, 8], [3, 8, 5], False),       # partly broadcast
    ([2, 1, 4, 8], [1, 3, 8, 5], False),
    ([2, 4, 8], [3, 8, 5], False),          # does not broadcast
    ([2, 4, 8], [2, 7, 5], False),          # contraction dims differ
])
def test_matmul_batch_forms(a, b, ok):
    args, line = _mm(a, b)
    if ok:
        assert "_mlir_ciface_nova_hip_gemm" in plan_one(args, line)
    else:
        with pytest.raises(nova_run.NovaRunError, match="not on this path"):
            plan_one(args, line)


@pytest.mark.parametrize("adt,bdt,cast,ok", [
    ("f32", "f32", False, True),
    ("bf16", "bf16", True, True),     # f32 accumulate over bf16 data
    ("f16", "f16", True, True),
    ("f16", "f16", False, True),      # f16 x f16 -> f16, accumulated in f16
    ("bf16", "bf16", False, False),   # bf16 x bf16 -> f16 (NovaOps.cpp:1198): unpinned
    ("bf16", "f16", True, False),     # operands stored differently
])
def test_gemm_dtype_forms(adt, bdt, cast, ok):
    args, line = _mm([4, 8], [8, 3], adt, bdt, cast)
    if ok:
        assert "_mlir_ciface_nova_hip_gemm" in plan_one(args, line)
    else:
        with pytest.raises(nova_run.NovaRunError, match="not on this path"):
            plan_one(args, line)


@pytest.mark.parametrize("ins,outs,ok", [
    ("bf16", "f32", True), ("f16", "f32", True), ("f32", "f32", True),
    ("bf16", "bf16", True), ("f16", "f16", True), ("bf16", "f16", False), ("f32", "bf16", False),
])
def test_linalg_matmul_dtype_forms(ins, outs, ok):
    text = f"""func.func @f(%a: {T([4, 8], ins)}, %b: {T([8, 3], ins)}) {{
      %z = arith.constant 0.000000e+00 : {outs}
      %e = tensor.empty() : {T([4, 3], outs)}
      %c = linalg.fill ins(%z : {outs}) outs(%e : {T([4, 3], outs)}) -> {T([4, 3], outs)}
      %r = linalg.matmul ins(%a, %b : {T([4, 8], ins)}, {T([8, 3], ins)}) outs(%c : {T([4, 3], outs)}) -> {T([4, 3], outs)}
      return
    }}"""
    p = nova_run.Program(text)
    if ok:
        assert "_mlir_ciface_nova_hip_gemm" in p.plan("f")
    else:
        with pytest.raises(nova_run.NovaRunError, match="not on this path"):
            p.plan("f")


@pytest.mark.parametrize("ins,outs,ok", [
    ("f32", "f32", True), ("bf16", "bf16", True), ("f16", "f16", True),
    ("bf16", "f32", False), ("f16", "f32", False), ("bf16", "f16", False), ("f32", "bf16", False),
])
def test_linalg_matmul_into_data_holding_outs_dtype_forms(ins, outs, ok):
    """outs holding data (a function argument): the exact kernel sums from it,
    f32 or a 16-bit accumulator of the operands' own type; 16-bit operands
    into f32 data are declined (their zero-filled form is not)."""
    text = f"""func.func @f(%a: {T([4, 8], ins)}, %b: {T([8, 3], ins)}, %c: {T([4, 3], outs)}) {{
      %r = linalg.matmul ins(%a, %b : {T([4, 8], ins)}, {T([8, 3], ins)}) outs(%c : {T([4, 3], outs)}) -> {T([4, 3], outs)}
      return
    }}"""
    p = nova_run.Program(text)
    if ok:
        assert "accumulate-into=" in p.plan("f")
    else:
        with pytest.raises(nova_run.NovaRunError, match="not on this path"):
            p.plan("f")


@pytest.mark.parametrize("dt,cast,ok", [
    ("f32", False, True), ("bf16", True, True), ("bf16", False, False), ("f16", False, False),
])
def test_backward_gemm_dtype_forms(dt, cast, ok):
    """Backward GEMMs accumulate in f32: f32 operands, or 16-bit data read
    through widening casts (f32 grads).  With 16-bit results the reference
    accumulates in that type (linalg.generic over 16-bit outs): declined."""
    go, x, w = [2, 4, 3], [2, 4, 8], [8, 3]
    args = [("go", go, dt), ("x", x, dt), ("w", w, dt)]
    if cast:
        line = (f"%gf = nova.cast %go : {T(go, dt)} -> {T(go)}\n  "
                f"%xf = nova.cast %x : {T(x, dt)} -> {T(x)}\n  "
                f"%wf = nova.cast %w : {T(w, dt)} -> {T(w)}\n  "
                f"%g:3 = nova.linear_backward %gf, %xf, %wf : {T(go)}, {T(x)}, {T(w)}")
    else:
        line = f"%g:3 = nova.linear_backward %go, %x, %w : {T(go, dt)}, {T(x, dt)}, {T(w, dt)}"
    if ok:
        assert "_mlir_ciface_nova_hip_linear_backward" in plan_one(args, line)
    else:
        with pytest.raises(nova_run.NovaRunError, match="not on this path"):
            plan_one(args, line)


def test_gpt_step_backward_forms_are_rank3():
    """The reference GPT step's own backward GEMMs (ltest/test.mlir:40, 42):
    rank-3 nova.linear_backward, in the table and planned."""
    go, x, w = [8, 16, 12], [8, 16, 20], [20, 12]
    plan = plan_one([("go", go, "f32"), ("x", x, "f32"), ("w", w, "f32")],
                    f"%g:3 = nova.linear_backward %go, %x, %w : {T(go)}, {T(x)}, {T(w)}")
    assert "_mlir_ciface_nova_hip_linear_backward(b0[8,16,12]f32" in plan


def test_pass_routes_every_lowering_through_the_table():
    """NovaHipLowering.cpp (not compilable here: no MLIR) asks
    nova_forms::check() for every op it lowers, before it creates any op, and
    has no rank or dtype refusals of its own."""
    src = open(PASS).read()
    assert '#include "nova_forms.h"' in src
    assert "nova_forms::check(" in src
    for fn in re.findall(r"LogicalResult (lower\w+)\(", src):
        body = src[src.index(f"LogicalResult {fn}("):]
        body = body[:body.index("\n  }\n")]
        assert "declined(" in body, fn
        first_create = body.find("rewriter.create")
        first_check = body.find("declined(")
        assert first_create == -1 or first_check < first_create, fn
    assert "getRank() > 3" not in src and "getRank() != 2" not in src
    # every row of the table is named (as the form the op is checked under)
    named = set(re.findall(r'"((?:nova|linalg)\.[a-z_<>]+)"', src))
    assert set(table()) <= named, set(table()) - named
