"""CPU check of the Julia binding a maintainer adds (the ```julia block of the
integration guide at the repository root, DOC) against the C header.

Every ``ccall((:moe_..., LIB), Ret, (ArgTypes...), args...)`` in the Julia
block must name a function include/moe_mi355x.h declares, with the same
return type, the same number of parameters, a Julia type that matches each C
parameter type, and as many arguments as its type tuple lists.  Every
function the header declares must have at least one ccall, and the Julia
mirrors of the two structs must list the C structs' fields in order with
matching types."""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_mi355x.h")
DOC = os.path.join(REPO, "INTEGRATION.md")

# Julia type -> the C types (whitespace removed) it may stand for
JULIA_TO_C = {
    "Cint": {"int"},
    "Cstring": {"constchar*"},
    "Int32": {"int32_t", "int"},
    "Int64": {"int64_t"},
    "UInt64": {"uint64_t"},
    "Float32": {"float"},
    "Ptr{Float32}": {"float*", "constfloat*"},
    "Ref{Float32}": {"float*"},
    "Ptr{Int32}": {"int32_t*", "constint32_t*"},
    "Ref{Int64}": {"int64_t*"},
    "Ref{MoeConfigC}": {"constmoe_config*"},
    "Ref{Ptr{Cvoid}}": {"moe_handle**"},
    "Ref{MoeForwardAux}": {"moe_forward_aux*"},
    # untyped pointers: data of either dtype, the handle, a stream, a NULL aux
    "Ptr{Cvoid}": {"void*", "constvoid*", "moe_handle*", "constmoe_handle*", "moe_forward_aux*"},
}
STRUCT_FIELDS = {"Int32": "int32_t", "Float32": "float", "Ptr{Float32}": "float*", "Ptr{Int32}": "int32_t*",
                 "NTuple{5,Int32}": "int32_t[5]"}


def _split_top(s):
    """Split on commas outside (), {} and []."""
    out, depth, cur = [], 0, []
    for ch in s:
        if ch in "({[":
            depth += 1
        elif ch in ")}]":
            depth -= 1
        if ch == "," and depth == 0:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    out.append("".join(cur).strip())
    return [x for x in out if x]


def _match(s, i):
    """Index of the bracket closing the one at s[i]."""
    pairs = {"(": ")", "{": "}", "[": "]"}
    stack = []
    for j in range(i, len(s)):
        if s[j] in pairs:
            stack.append(pairs[s[j]])
        elif stack and s[j] == stack[-1]:
            stack.pop()
            if not stack:
                return j
    raise ValueError("unbalanced brackets at %d" % i)


def julia_block():
    text = open(DOC).read()
    m = re.search(r"```julia\n(.*?)```", text, flags=re.S)
    assert m, "no Julia block in the integration guide"
    return m.group(1)


def julia_ccalls():
    """[(name, return type, [arg types], number of arguments passed)]"""
    src = julia_block()
    calls = []
    for m in re.finditer(r"ccall\(\(:(moe_\w+),\s*LIB\)", src):
        open_paren = src.index("(", m.start())
        end = _match(src, open_paren)
        body = src[open_paren + 1:end]
        parts = _split_top(body)
        ret, tup = parts[1], parts[2]
        assert tup.startswith("(") and tup.endswith(")"), (m.group(1), tup)
        types = _split_top(tup[1:-1])
        calls.append((m.group(1), ret, types, len(parts) - 3))
    return calls


def header_decls():
    """{name: (return type, [param types])}, types with whitespace removed."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*((?:const\s+)?\w+\s*\**)\s*(moe_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        types = []
        for p in _split_top(" ".join(params.split())):
            if p == "void":
                continue
            # drop the parameter name (the last identifier)
            t = re.sub(r"\b\w+\s*$", "", p)
            types.append(t.replace(" ", ""))
        decls[name] = (ret.replace(" ", ""), types)
    return decls


def header_struct(name):
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    m = re.search(r"typedef struct \{([^{}]*)\}\s*" + name + r"\s*;", text)
    assert m, name
    fields = []
    for line in m.group(1).split(";"):
        line = " ".join(line.split())
        if not line:
            continue
        fm = re.match(r"(\w+)\s*(\**)\s*(\w+)\s*(\[\d+\])?$", line)
        assert fm, line
        fields.append((fm.group(3), fm.group(1) + fm.group(2) + (fm.group(4) or "")))
    return fields


def julia_struct(name):
    src = julia_block()
    m = re.search(r"struct " + name + r"\b[^\n]*\n(.*?)\nend", src, flags=re.S)
    assert m, name
    body = re.sub(r"#[^\n]*", "", m.group(1))
    return [(f, t) for f, t in re.findall(r"(\w+)::([\w{},]+)", body)]


def test_parsers_find_the_boundary():
    decls = header_decls()
    assert "moe_forward" in decls and decls["moe_abi_version"] == ("int", [])
    assert decls["moe_create"] == ("int", ["constmoe_config*", "moe_handle**"])
    assert len(julia_ccalls()) >= len(decls)


@pytest.mark.parametrize("call", julia_ccalls(), ids=lambda c: c[0])
def test_ccall_matches_header(call):
    name, ret, types, nargs = call
    decls = header_decls()
    assert name in decls, f"{name} is not declared in include/moe_mi355x.h"
    cret, ctypes_ = decls[name]
    assert cret in JULIA_TO_C[ret], (name, ret, cret)
    assert len(types) == len(ctypes_), f"{name}: {len(types)} Julia argument types, {len(ctypes_)} C parameters"
    for i, (jt, ct) in enumerate(zip(types, ctypes_)):
        assert jt in JULIA_TO_C, f"{name} argument {i}: unknown Julia type {jt}"
        assert ct in JULIA_TO_C[jt], f"{name} argument {i}: Julia {jt} for C {ct}"
    assert nargs == len(types), f"{name}: {nargs} arguments passed for {len(types)} types"


def test_every_entry_point_has_a_binding():
    bound = {c[0] for c in julia_ccalls()}
    missing = sorted(set(header_decls()) - bound)
    assert not missing, f"no ccall in the integration guide for {missing}"


@pytest.mark.parametrize("jname,cname", [("MoeConfigC", "moe_config"), ("MoeForwardAux", "moe_forward_aux")])
def test_struct_mirrors(jname, cname):
    jf = julia_struct(jname)
    cf = header_struct(cname)
    assert [f for f, _ in jf] == [f for f, _ in cf]
    for (f, jt), (_, ct) in zip(jf, cf):
        assert STRUCT_FIELDS[jt] == ct, (f, jt, ct)
