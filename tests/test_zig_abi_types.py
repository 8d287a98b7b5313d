"""The Zig binding (mobile-moe.zig_amd/zig/hip_backend.zig) against the C ABI
(include/mmhip.h), type by type, without a Zig compiler (the image has none).

- Every `extern fn` has the header's parameter and return types: Zig types are
  mapped to C (u32 -> uint32_t, c_int -> int, ?*const anyopaque -> const
  void*, [*:0]const u8 -> const char*, *?*Ctx -> mmhip_ctx**, ...), pointer
  depth and the constness of every pointee included; optional (`?`) is
  nullability, not a type difference.
- Every `extern struct` has the header struct's fields in the same order with
  the same types.
- A C program built with gcc prints sizeof / offsetof of every struct field,
  and they equal the layout that C's rules (natural alignment, x86-64) give
  the Zig field list: an extern struct is laid out by those rules, so the
  engine and the library agree on every byte of mmhip_moe_weights,
  mmhip_route_params, mmhip_gguf_tensor, mmhip_op_schedule and the others.
The reference binds its C bridge the same way (metal_backend.zig:7-26)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mmhip.h")
ZIG = os.path.join(ROOT, "mobile-moe.zig_amd", "zig", "hip_backend.zig")

# Zig name of each C type the binding mirrors.
C_TO_ZIG = {
    "mmhip_ctx": "Ctx", "mmhip_weight": "Weight", "mmhip_moe_layer": "MoeLayerHandle", "mmhip_gguf": "GgufHandle",
    "mmhip_moe_weights": "MoeWeights", "mmhip_route_params": "RouteParams", "mmhip_shape": "Shape",
    "mmhip_op_schedule": "OpSchedule", "mmhip_plan_hparams": "PlanHyperParams", "mmhip_perf_entry": "PerfEntry",
    "mmhip_gguf_info": "GgufInfo", "mmhip_gguf_tensor": "GgufTensor", "mmhip_gemv_group": "GemvGroup",
}
C_SCALARS = {"uint8_t": "u8", "char": "u8", "uint32_t": "u32", "int32_t": "i32", "uint64_t": "u64",
             "int64_t": "i64", "float": "f32", "double": "f64", "size_t": "usize", "int": "c_int", "void": "void"}
ZIG_SCALARS = {"u8": "u8", "u32": "u32", "i32": "i32", "u64": "u64", "i64": "i64", "f32": "f32", "f64": "f64",
               "usize": "usize", "c_int": "c_int", "void": "void", "anyopaque": "void"}
# size / alignment on x86-64 (System V): the host side of the ABI.
SIZES = {"u8": 1, "u32": 4, "i32": 4, "u64": 8, "i64": 8, "f32": 4, "f64": 8, "usize": 8, "c_int": 4}


# ---------------------------------------------------------------- C side

def _strip_c(src):
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    return "\n".join(line for line in src.splitlines() if not line.strip().startswith("#"))


def _c_type(tokens):
    """tokens of one declaration without its name -> canonical type string."""
    base, base_const, i = None, False, 0
    while i < len(tokens) and tokens[i] != "*":
        if tokens[i] == "const":
            base_const = True
        elif tokens[i] not in ("struct", "extern", '"C"', "{"):
            base = tokens[i]
        i += 1
    name = C_SCALARS.get(base, C_TO_ZIG.get(base, base))
    t = ("const " if base_const else "") + name
    while i < len(tokens):
        if tokens[i] == "*":
            t = f"ptr({t})"
        elif tokens[i] == "const":
            t = "const " + t
        i += 1
    return t


def _split_decl(decl):
    """'const char* const* names' -> (canonical type, 'names', array_len or None)."""
    decl = decl.strip()
    arr = None
    m = re.match(r"^(.*?)\[(\d+)\]$", decl)
    if m:
        decl, arr = m.group(1).strip(), int(m.group(2))
    tokens = re.findall(r"[A-Za-z_][A-Za-z_0-9]*|\*", decl)
    name = tokens[-1]
    return _c_type(tokens[:-1]), name, arr


def _top(t):
    return t[len("const "):] if t.startswith("const ") else t


def c_functions():
    src = _strip_c(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(mmhip_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", src):
        ret = _c_type(re.findall(r"[A-Za-z_][A-Za-z_0-9]*|\*", m.group(1)))
        params = m.group(3).strip()
        plist = [] if params in ("", "void") else [_top(_split_decl(p)[0]) for p in params.split(",")]
        out[m.group(2)] = (_top(ret), plist)
    return out


def c_structs():
    src = _strip_c(open(HEADER).read())
    out = {}
    for m in re.finditer(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", src, flags=re.S):
        fields = []
        for stmt in m.group(1).split(";"):
            stmt = " ".join(stmt.split())
            if not stmt:
                continue
            first, *rest = stmt.split(",")
            t, name, arr = _split_decl(first)
            fields.append((name, _top(t), arr))
            base = first.strip()[: first.strip().rfind(name)]
            for r in rest:
                t2, n2, a2 = _split_decl(base + " " + r.strip())
                fields.append((n2, _top(t2), a2))
        out[C_TO_ZIG.get(m.group(2), m.group(2))] = (m.group(2), fields)
    return out


# ---------------------------------------------------------------- Zig side

def _zig_type(s):
    """'?*const anyopaque' -> 'ptr(const void)', '[4]u64' -> ('u64', 4)."""
    s = s.strip()
    m = re.match(r"^\[(\d+)\](.*)$", s)
    if m:
        return _zig_type(m.group(2))[0], int(m.group(1))
    if s.startswith("?"):
        return _zig_type(s[1:])
    m = re.match(r"^(\*|\[\*\]|\[\*:0\])\s*(const\s+)?(.*)$", s)
    if m:
        inner, _ = _zig_type(m.group(3))
        return f"ptr({'const ' if m.group(2) else ''}{inner})", None
    return ZIG_SCALARS.get(s, s), None


def zig_functions():
    src = open(ZIG).read()
    out = {}
    for m in re.finditer(r"^extern fn (mmhip_[a-z0-9_]+)\((.*?)\)\s*([^;]+);", src, flags=re.M):
        params = []
        if m.group(2).strip():
            for p in re.split(r",\s*(?=[a-z_][a-z_0-9]*\s*:)", m.group(2)):
                params.append(_zig_type(p.split(":", 1)[1])[0])
        out[m.group(1)] = (_zig_type(m.group(3))[0], params)
    return out


def zig_structs():
    src = open(ZIG).read()
    out = {}
    for m in re.finditer(r"pub const (\w+) = extern struct \{(.*?)\};", src, flags=re.S):
        body = re.sub(r"//[^\n]*", "", m.group(2))
        fields = []
        for f in re.split(r",\s*(?=[a-z_][a-z_0-9]*\s*:)|,\s*$", body.strip()):
            f = f.strip().rstrip(",")
            if not f:
                continue
            name, rest = f.split(":", 1)
            rest = rest.split("=", 1)[0]
            t, arr = _zig_type(rest)
            fields.append((name.strip().rstrip("_"), t, arr))
        out[m.group(1)] = fields
    return out


# ---------------------------------------------------------------- tests

def test_extern_fn_types_match_header():
    c, z = c_functions(), zig_functions()
    assert sorted(c) == sorted(z)
    bad = [(n, c[n], z[n]) for n in c if c[n] != z[n]]
    assert not bad, "type mismatches (C vs Zig):\n" + "\n".join(f"{n}: {a} vs {b}" for n, a, b in bad)


def test_a_wrong_zig_type_is_caught():
    """The comparison is not vacuous: a u32 where the header has uint64_t,
    a dropped const and a missing pointer level all show up."""
    assert _zig_type("u32")[0] != _c_type(["uint64_t"])
    assert _zig_type("*anyopaque")[0] != _top(_split_decl("const void* p")[0])
    assert _zig_type("*Ctx")[0] != _top(_split_decl("mmhip_ctx** out_ctx")[0])
    assert _zig_type("[*]const [*:0]const u8")[0] == _top(_split_decl("const char* const* names")[0])
    assert _zig_type("[*]const [*:0]u8")[0] != _top(_split_decl("const char* const* names")[0])


def test_extern_struct_fields_match_header():
    c, z = c_structs(), zig_structs()
    for zname, (cname, cfields) in c.items():
        assert zname in z, f"{cname} has no extern struct {zname} in the Zig binding"
        assert z[zname] == cfields, f"{cname}: C {cfields}\n   vs Zig {z[zname]}"
    for must in ("MoeWeights", "RouteParams", "GgufTensor", "OpSchedule", "Shape", "PerfEntry", "PlanHyperParams",
                 "GgufInfo"):
        assert must in c


def _layout(fields, structs):
    """(size, align, {field: offset}) by C's rules for a Zig field list."""
    off, align, offs = 0, 1, {}
    for name, t, arr in fields:
        if t.startswith("ptr("):
            sz = al = 8
        elif t in SIZES:
            sz = al = SIZES[t]
        else:
            sz, al, _ = _layout(structs[t], structs)
        n = arr or 1
        off = (off + al - 1) // al * al
        offs[name] = off
        off += sz * n
        align = max(align, al)
    return (off + align - 1) // align * align, align, offs


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_c(tmp_path):
    c, z = c_structs(), zig_structs()
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "mmhip.h"', "int main(void) {"]
    for zname, (cname, cfields) in c.items():
        lines.append(f'printf("{zname} size %zu\\n", sizeof({cname}));')
        for fname, _, _ in cfields:
            lines.append(f'printf("{zname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        parts = line.split()
        got[(parts[0], parts[1])] = int(parts[2])
    for zname in c:
        size, _, offs = _layout(z[zname], z)
        assert got[(zname, "size")] == size, zname
        for fname, off in offs.items():
            assert got[(zname, fname)] == off, (zname, fname)
    # the structs the engine fills field by field
    assert got[("MoeWeights", "size")] == 88 and got[("MoeWeights", "router_host")] == 32
    assert got[("RouteParams", "size")] == 16 and got[("RouteParams", "deferral_bias_host")] == 8
    assert got[("GgufTensor", "size")] == 88 and got[("GgufTensor", "data")] == 80
    assert got[("OpSchedule", "size")] == 40 and got[("OpSchedule", "estimated_us")] == 32
