"""The Free Pascal / Delphi binding (mormot2-qwen-tts_amd/pascal/
mormot.ai.tts.qwen.hip.pas) against include/q3h.h, on the CPU: no Pascal
compiler exists in this image, so the unit is checked by reading it.

- every C entry point has one `cdecl; external` declaration of the same name,
  the same number of parameters, and per parameter the same class (pointer,
  32-bit integer, 64-bit integer, float): an `out` / `var` parameter or a
  pointer type stands for a C pointer, and no structure is passed as a
  `const` record (FPC may pass those by value under cdecl);
- every C structure has a Pascal record with the same fields in the same
  order, at the same offsets and of the same size under C packing: the C side
  from gcc (offsetof / sizeof of include/q3h.h), the Pascal side laid out from
  the record declarations with {$packrecords C} rules.
"""
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q3h.h")
UNIT = os.path.join(ROOT, "mormot2-qwen-tts_amd", "pascal", "mormot.ai.tts.qwen.hip.pas")


def strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def strip_pas_comments(s):
    s = re.sub(r"\{[^}]*\}", " ", s)  # {...} (directives included)
    return re.sub(r"//[^\n]*", " ", s)


def c_class(decl):
    decl = decl.strip()
    if "*" in decl:
        return "ptr"
    t = decl.rsplit(None, 1)[0] if len(decl.split()) > 1 else decl
    t = t.replace("const", "").strip()
    return {"int": "i32", "int32_t": "i32", "int64_t": "i64", "float": "f32",
            "uint64_t": "u64", "void": "void"}[t]


def c_functions():
    s = strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"(int64_t|int|const\s+char\s*\*)\s*(q3h_\w+)\s*\(([^)]*)\)\s*;", s):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        ret = "ptr" if "*" in ret else c_class(ret + " x")
        args = [] if params in ("", "void") else [c_class(p) for p in params.split(",")]
        out[name] = (ret, args)
    return out


PAS_PTR_TYPES = {"pointer", "psingle", "ppsingle", "pinteger", "pansichar"}


def pas_class(t, mod):
    t = t.strip().lower()
    if mod in ("out", "var", "constref"):
        return "ptr"
    if t in PAS_PTR_TYPES or t.startswith("pq3h_") or t.startswith("q3h_"):
        return "ptr"
    return {"integer": "i32", "int64": "i64", "single": "f32", "uint64": "u64"}[t]


def pas_functions():
    s = strip_pas_comments(open(UNIT).read())
    s = s.split("implementation")[0]
    out = {}
    for m in re.finditer(r"function\s+(q3h_\w+)\s*(\(([^)]*)\))?\s*:\s*(\w+)\s*;\s*cdecl\s*;"
                         r"\s*external\s+LIBQ3H\s*;", s, flags=re.I):
        name, params, ret = m.group(1), m.group(3) or "", m.group(4)
        args = []
        for group in [g for g in params.split(";") if g.strip()]:
            names, typ = group.split(":")
            words = names.split()
            mod = words[0].lower() if words[0].lower() in ("out", "var", "const",
                                                           "constref") else ""
            if mod == "const":
                assert not typ.strip().lower().startswith("q3h_"), \
                    f"{name}: a const record parameter may be passed by value"
            n = len([w for w in names.replace(mod, "", 1 if mod else 0).split(",") if w.strip()])
            args += [pas_class(typ, mod)] * n
        out[name] = (pas_class(ret, ""), args)
    return out


def test_every_entry_point_is_declared_alike():
    c, p = c_functions(), pas_functions()
    assert len(c) >= 36
    assert set(c) == set(p), (set(c) ^ set(p))
    for name in c:
        assert c[name] == p[name], (name, c[name], p[name])


# ---- structure layouts

def c_structs():
    s = strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(q3h_\w+)\s*;", s, flags=re.S):
        body, name = m.group(1), m.group(2)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            # "const void *wq, *wk" / "int32_t a, b" / "q3h_codec_res res[3]"
            head = re.match(r"((?:const\s+)?\w+)\s*(.*)", decl)
            for part in head.group(2).split(","):
                nm = re.sub(r"[\s*]", "", re.sub(r"\[.*\]", "", part))
                fields.append(nm)
        out[name] = fields
    return out


def c_layout(structs):
    """{struct: (size, [(field, offset)])} from gcc"""
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "q3h.h"', "int main(void) {"]
    for st, fields in structs.items():
        lines.append(f'printf("{st} %zu\\n", sizeof({st}));')
        for f in fields:
            lines.append(f'printf("{st}.{f} %zu\\n", offsetof({st}, {f}));')
    lines.append("return 0; }")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-I", os.path.dirname(HEADER), src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    lay = {}
    for row in out.strip().splitlines():
        key, val = row.split()
        if "." in key:
            st, f = key.split(".")
            lay.setdefault(st, [None, []])[1].append((f, int(val)))
        else:
            lay.setdefault(key, [None, []])[0] = int(val)
    return lay


PAS_SCALARS = {"integer": (4, 4), "single": (4, 4), "uint64": (8, 8), "int64": (8, 8)}


def pas_records():
    s = strip_pas_comments(open(UNIT).read()).split("implementation")[0]
    recs = {}
    for m in re.finditer(r"(q3h_\w+)\s*=\s*record(.*?)end\s*;", s, flags=re.S | re.I):
        name, body = m.group(1), m.group(2)
        fields = []
        for decl in [d for d in body.split(";") if d.strip()]:
            names, typ = decl.split(":", 1)
            for nm in names.split(","):
                fields.append((nm.strip(), typ.strip()))
        recs[name] = fields
    return recs


def pas_type_layout(t, recs):
    """(size, align) of a Pascal type under C packing"""
    t = t.strip()
    m = re.match(r"array\s*\[\s*(\d+)\s*\.\.\s*(\d+)\s*\]\s*of\s+(\w+)", t, flags=re.I)
    if m:
        size, align = pas_type_layout(m.group(3), recs)
        return size * (int(m.group(2)) - int(m.group(1)) + 1), align
    tl = t.lower()
    if tl in PAS_SCALARS:
        return PAS_SCALARS[tl]
    if tl in PAS_PTR_TYPES or tl.startswith("pq3h_"):
        return 8, 8
    if t in recs:
        size, align, _ = pas_record_layout(t, recs)
        return size, align
    raise KeyError(t)


def pas_record_layout(name, recs):
    off, align, offs = 0, 1, []
    for f, t in recs[name]:
        size, a = pas_type_layout(t, recs)
        off = (off + a - 1) // a * a
        offs.append((f, off))
        off += size
        align = max(align, a)
    return (off + align - 1) // align * align, align, offs


def test_every_structure_has_the_same_layout():
    cs = c_structs()
    lay = c_layout(cs)
    recs = pas_records()
    assert len(cs) >= 10
    for st in cs:
        assert st in recs, f"no Pascal record {st}"
        size, _, offs = pas_record_layout(st, recs)
        csize, coffs = lay[st]
        assert [f for f, _ in offs] == [f for f, _ in coffs], (st, offs, coffs)
        assert offs == coffs, (st, offs, coffs)
        assert size == csize, (st, size, csize)


def test_unit_sets_c_packing_and_declares_its_pointer_types():
    s = open(UNIT).read()
    assert re.search(r"\{\$packrecords\s+C\}", s, flags=re.I)
    assert re.search(r"PPSingle\s*=\s*\^PSingle", s)
