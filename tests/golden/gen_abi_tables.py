#!/usr/bin/env python3
"""Writes exl3_abi_tables.json: the reference's op schemas (parameter specs, operand lists, doc strings) and operand positions, read
AS TEXT from /root/reference/include/exl3_abi.h (lines 286-355 positions, 366-627 schemas). Nothing of the reference is
compiled or imported; the JSON is data the plugin tests compare libexl3c4.so's exports with.

The header's tables use a few C macros (EXL3_GEMM_PARAMS, EXL3_MOD4_SHAPE, EXL3_GU_CLASS(q) ...); this script expands
the object-like ones by text substitution and the class ones by replacing `#q` with the argument, as the C
preprocessor would, then reads every `{ "name", KIND, FLAG, ... }` entry of each array in order."""
import json
import os
import re
import sys

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/include/exl3_abi.h"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "exl3_abi_tables.json")
text = open(SRC).read()


def macros(t):
    """#define NAME body (with backslash continuations), object-like and one-argument function-like."""
    out = {}
    for m in re.finditer(r"#define\s+(\w+)(\((\w+)\))?\s+((?:[^\n]*\\\n)*[^\n]*)", t):
        name, arg, body = m.group(1), m.group(3), m.group(4).replace("\\\n", " ")
        out[name] = (arg, body)
    return out


M = macros(text)


def expand(body):
    for _ in range(4):
        for name, (arg, mb) in M.items():
            if arg is None:
                body = re.sub(r"\b%s\b" % name, lambda _m, mb=mb: mb, body)
            else:   # NAME(v): the body with `"text" #arg` pasted as "textv"
                body = re.sub(r"\b%s\((\w+)\)" % name,
                              lambda m, mb=mb, arg=arg: re.sub(r'"\s*#\s*%s\b' % arg, m.group(1) + '"', mb), body)
    return body


def braced(t, start):
    """The text inside the braces opening at or after `start` (nesting counted)."""
    i = t.index("{", start)
    depth = 0
    for j in range(i, len(t)):
        depth += t[j] == "{"
        depth -= t[j] == "}"
        if depth == 0:
            return t[i + 1:j]
    raise SystemExit("unbalanced")


def array(kind, name):
    m = re.search(r"static const %s %s\[\d*\]\s*=" % (kind, name), text)
    if not m:
        raise SystemExit(f"{kind} {name} not found")
    body = expand(braced(text, m.end()))
    return re.findall(r'\{\s*"([^"]+)"\s*,\s*(RAD_\w+)\s*,\s*(\w+)', body)


params = {n: array("RadParamSpec", n) for n in ("p_gu", "p_dn", "p_pg", "p_gd", "p_gu4", "p_dn4", "p_pg4", "p_gd4")}
opds = {n: array("RadOperandSpec", n) for n in ("gate_up", "down", "prep_gu", "gate_up_down", "gate_up4", "down4",
                                                   "prep_gu4", "gate_up_down4")}
order = [("moe_exl3_gate_up", "p_gu", "gate_up"), ("moe_exl3_down", "p_dn", "down"),
         ("moe_exl3_prep_gu", "p_pg", "prep_gu"), ("moe_exl3_gate_up_down", "p_gd", "gate_up_down"),
         ("moe_exl3_gate_up_mod4", "p_gu4", "gate_up4"), ("moe_exl3_down_mod4", "p_dn4", "down4"),
         ("moe_exl3_prep_gu_mod4", "p_pg4", "prep_gu4"), ("moe_exl3_gate_up_down_mod4", "p_gd4", "gate_up_down4")]
# the schema table's op order, as the header's s[8] lists them
s_body = braced(text, re.search(r"static const RadOpSchema s\[8\]\s*=", text).end())
listed = re.findall(r"\{\s*(EXL3_OP_\w+)\s*,", s_body)
names = {m.group(1): m.group(2) for m in re.finditer(r'#define\s+(EXL3_OP_\w+)\s+"([^"]+)"', text)}
schema_ops = [names[x] for x in listed]
assert schema_ops == [o for o, _, _ in order], schema_ops

# each schema's doc string: the adjacent string literals of its entry, joined as the C compiler joins them
docs = []
depth, start = 0, None
for j, ch in enumerate(s_body):
    if ch == "{":
        depth += 1
        if depth == 1:
            start = j
    elif ch == "}":
        depth -= 1
        if depth == 0:
            docs.append("".join(re.findall(r'"((?:[^"\\]|\\.)*)"', s_body[start:j + 1])))
assert len(docs) == len(order), len(docs)

schemas = []
for (op, p, o), doc in zip(order, docs):
    schemas.append({"op": op,
                    "params": [[k, kind.replace("RAD_P_", ""), req.replace("RAD_", "")] for k, kind, req in params[p]],
                    "operands": [[n, d.replace("RAD_OPD_", ""), int(opt)] for n, d, opt in opds[o]],
                    "doc": doc})

pos = {}
for var, op in (("gu", "moe_exl3_gate_up"), ("dn", "moe_exl3_down"), ("pg", "moe_exl3_prep_gu"),
                ("gd", "moe_exl3_gate_up_down"), ("gu4", "moe_exl3_gate_up_mod4"), ("dn4", "moe_exl3_down_mod4"),
                ("pg4", "moe_exl3_prep_gu_mod4"), ("gd4", "moe_exl3_gate_up_down_mod4")):
    m = re.search(r"static const Exl3Positions %s\s*=" % var, text)
    body = braced(text, m.end()).replace("EXL3_NO_CLASS", "{ -1, -1, -1, -1, -1, -1, -1 }")
    nums = [int(v) for v in re.findall(r"-?\d+", body)]
    x, srt, off, y, n_opd, n_cls = nums[:6]
    planes = [nums[6 + 7 * c: 13 + 7 * c] for c in range(4)]
    pos[op] = {"x": x, "sorted": srt, "offset": off, "y": y, "n_opd": n_opd, "n_cls": n_cls, "plane": planes,
               "ids": nums[34]}

json.dump({"source": "include/exl3_abi.h (read as text)", "planes": ["codes", "suh", "suh1", "svh", "dn_suh",
                                                                        "dn_codes", "dn_svh"],
           "schemas": schemas, "positions": pos}, open(OUT, "w"), indent=1)
print("wrote", OUT, [(s["op"], len(s["params"]), len(s["operands"])) for s in schemas])
