"""The Rust FFI module (rust-gpu_amd/ffi/t0_gemm.rs) against the C header it
binds (include/t0_gemm.h), on the CPU (no Rust toolchain here):

- every function of the header is declared once in the module's extern
  block, with the same name, argument count and argument types under the
  C -> Rust type map below, and the same return type; nothing extra;
- every struct of the header is a #[repr(C)] struct with the same fields in
  the same order and mapped types, and its layout (each field's offset and
  the size) computed by repr(C)'s rules from the Rust types equals the one
  gcc reports for the C struct; opaque handles are opaque structs;
- every enum constant and #define of the header is a Rust const with the
  value gcc computes.

The reference surface these bind (src/prelude.rs:11-19, src/t0/mod.rs:76-83)
includes the tile_ir dispatch calls its callers make
(tests/precision_vs_torch.rs:149-172, src/t0/tile_ir.rs:5064-5082)."""
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "t0_gemm.h")
RUST = os.path.join(ROOT, "rust-gpu_amd", "ffi", "t0_gemm.rs")

SCALARS = {"uint8_t": "u8", "uint16_t": "u16", "uint32_t": "u32", "uint64_t": "u64", "int32_t": "i32",
           "int": "c_int", "char": "c_char", "float": "f32", "double": "f64", "size_t": "usize", "void": "c_void"}
SIZES = {"u8": 1, "u16": 2, "u32": 4, "u64": 8, "i32": 4, "c_int": 4, "f32": 4, "f64": 8, "usize": 8}


# ---------------------------------------------------------------- C side
def _strip_c(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return text


def _c_decl(decl, field=False):
    """'const uint32_t grid[3]' -> (name, rust type, alternative rust type):
    an array argument is a pointer to the array (or to its first element),
    an array field is the array itself."""
    decl = " ".join(decl.split())
    m = re.match(r"^(.*?)(\w+)\s*(\[(\d+)\])?$", decl)
    assert m, decl
    base, name, arr = m.group(1).strip(), m.group(2), m.group(4)
    stars = base.count("*")
    base_const = base.startswith("const ")
    core = base.replace("const", " ").replace("*", " ").strip()
    assert " " not in core, decl
    t = SCALARS.get(core, core)
    if arr is not None and field:
        assert stars == 0, decl
        return name, f"[{t}; {arr}]", None
    if arr is not None:
        ptr = "*const" if base_const else "*mut"
        return name, f"{ptr} [{t}; {arr}]", f"{ptr} {t}"
    for i in range(stars):
        t = ("*const " if (i == 0 and base_const) else "*mut ") + t
    return name, t, None


def _c_type(ret):
    """A return type like 'const char*' -> Rust."""
    _, t, _ = _c_decl(ret.strip() + " x")
    return t


def parse_header():
    text = _strip_c(open(HEADER).read())
    text = "\n".join(l for l in text.splitlines() if not l.strip().startswith("#"))
    text = text.replace('extern "C" {', "")
    structs, opaque, funcs, enums = {}, set(), {}, []
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S):
        assert m.group(1) == m.group(3)
        fields = []
        for stmt in m.group(2).split(";"):
            stmt = " ".join(stmt.split())
            if not stmt:
                continue
            first, *rest = [s.strip() for s in stmt.split(",")]
            name, t, _ = _c_decl(first, field=True)
            fields.append((name, t))
            base = first[: first.rfind(name)].strip()
            for r in rest:
                name2, t2, _ = _c_decl(base + " " + r, field=True)
                fields.append((name2, t2))
        structs[m.group(1)] = fields
    text_ns = re.sub(r"typedef\s+struct\s+(\w+)\s*\{.*?\}\s*\w+\s*;", " ", text, flags=re.S)
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s+(\w+)\s*;", text_ns):
        assert m.group(1) == m.group(2)
        opaque.add(m.group(1))
    for m in re.finditer(r"(?:typedef\s+)?enum\s*\w*\s*\{(.*?)\}\s*\w*\s*;", text_ns, flags=re.S):
        for item in m.group(1).split(","):
            item = item.strip()
            if item:
                enums.append(item.split("=")[0].strip())
    text_nt = re.sub(r"typedef[^;]*;", " ", re.sub(r"(?:typedef\s+)?enum\s*\w*\s*\{.*?\}\s*\w*\s*;", " ",
                                                   text_ns, flags=re.S))
    for stmt in text_nt.split(";"):
        stmt = " ".join(stmt.split())
        m = re.match(r"^(.*?)\b(t0_\w+)\s*\((.*)\)$", stmt)
        if not m:
            assert not stmt.strip("} "), f"unparsed header statement: {stmt!r}"
            continue
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [_c_decl(p) for p in params.split(",")]
        assert name not in funcs, name
        funcs[name] = (_c_type(ret) if ret != "void" else None, plist)
    defines = re.findall(r"^#define\s+(T0_\w+)\s", open(HEADER).read(), flags=re.M)
    defines = [d for d in defines if d != "T0_GEMM_H"]
    return structs, opaque, funcs, enums, defines


# ------------------------------------------------------------- Rust side
def _norm(t):
    return " ".join(t.replace("*", " *").split()).replace("* ", "*").replace("*const", "*const ") \
        .replace("*mut", "*mut ").replace("  ", " ").strip()


def _split_top(s, sep=","):
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "([":
            depth += 1
        elif ch in ")]":
            depth -= 1
        if ch == sep and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [x.strip() for x in out if x.strip()]


def parse_rust():
    src = open(RUST).read()
    code = re.sub(r"//[^\n]*", "", src)
    for a, b in ("()", "[]", "{}"):
        assert code.count(a) == code.count(b), f"unbalanced {a}{b}"
    structs, opaque = {}, set()
    for m in re.finditer(r"((?:#\[[^\]]*\]\s*)*)pub struct (\w+)\s*\{(.*?)\n\}", code, flags=re.S):
        attrs, name, body = m.group(1), m.group(2), m.group(3)
        assert "#[repr(C)]" in attrs, f"{name} is not #[repr(C)]"
        fields = []
        for f in _split_top(body):
            fm = re.match(r"^(pub\s+)?(\w+)\s*:\s*(.+)$", " ".join(f.split()))
            assert fm, f
            fields.append((bool(fm.group(1)), fm.group(2), _norm(fm.group(3))))
        if all(not pub for pub, _, _ in fields):
            opaque.add(name)
        else:
            assert all(pub for pub, _, _ in fields), name
            structs[name] = [(n, t) for _, n, t in fields]
    blocks = re.findall(r'unsafe extern "C"\s*\{(.*?)\n\}', code, flags=re.S)
    assert len(blocks) == 1
    funcs = {}
    for stmt in _split_top(blocks[0], ";"):
        stmt = " ".join(stmt.split())
        m = re.match(r"^pub fn (\w+)\((.*)\)\s*(->\s*(.+))?$", stmt)
        assert m, f"unparsed extern item: {stmt!r}"
        params = []
        for p in _split_top(m.group(2)):
            pn, pt = p.split(":", 1)
            params.append((pn.strip(), _norm(pt)))
        assert m.group(1) not in funcs, m.group(1)
        funcs[m.group(1)] = (_norm(m.group(4)) if m.group(4) else None, params)
    consts = {}
    for m in re.finditer(r"pub const (\w+)\s*:\s*\w+\s*=\s*([^;]+);", code):
        expr = m.group(2).strip()
        assert re.fullmatch(r"[-\d\s<()]+", expr), expr
        consts[m.group(1)] = eval(expr)   # digits, minus, shifts and parentheses only
    return structs, opaque, funcs, consts


@pytest.fixture(scope="module")
def parsed():
    return parse_header(), parse_rust()


def test_every_function_is_bound_with_its_signature(parsed):
    (_, _, cfuncs, _, _), (_, _, rfuncs, _) = parsed
    assert set(rfuncs) == set(cfuncs), (sorted(set(cfuncs) - set(rfuncs)), sorted(set(rfuncs) - set(cfuncs)))
    for name, (cret, cparams) in cfuncs.items():
        rret, rparams = rfuncs[name]
        assert rret == (_norm(cret) if cret else None), (name, cret, rret)
        assert len(rparams) == len(cparams), name
        for (cn, ct, alt), (rn, rt) in zip(cparams, rparams):
            assert rt in (_norm(ct), _norm(alt) if alt else None), (name, cn, ct, rt)


def test_every_struct_matches_field_by_field(parsed):
    (cstructs, copaque, _, _, _), (rstructs, ropaque, _, _) = parsed
    assert set(rstructs) == set(cstructs)
    assert ropaque == copaque
    for name, cfields in cstructs.items():
        rf = rstructs[name]
        assert [n for n, _ in rf] == [n for n, _ in cfields], name
        for (n, ct), (_, rt) in zip(cfields, rf):
            assert rt == _norm(ct), (name, n, ct, rt)


def _rust_layout(structs, name, memo={}):
    """(size, align, {field: offset}) by repr(C): fields in order, each at
    the next multiple of its alignment, the size rounded up to the largest."""
    if name in memo:
        return memo[name]
    off, align, offs = 0, 1, {}
    for f, t in structs[name]:
        if t.startswith("*"):
            s = a = 8
        elif t.startswith("["):
            et, n = re.fullmatch(r"\[(\w+); (\d+)\]", t).groups()
            a = SIZES[et]
            s = a * int(n)
        elif t in SIZES:
            s = a = SIZES[t]
        else:
            s, a, _ = _rust_layout(structs, t)
        off = (off + a - 1) // a * a
        offs[f] = off
        off += s
        align = max(align, a)
    res = ((off + align - 1) // align * align, align, offs)
    memo[name] = res
    return res


def _gcc_facts(cstructs, consts):
    prog = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for name, fields in cstructs.items():
        prog.append(f'printf("S {name} %zu %zu\\n", sizeof({name}), _Alignof({name}));')
        for f, _ in fields:
            prog.append(f'printf("F {name} {f} %zu\\n", offsetof({name}, {f}));')
    for c in consts:
        prog.append(f'printf("C {c} %lld\\n", (long long)({c}));')
    prog.append("return 0; }")
    with tempfile.TemporaryDirectory() as td:
        c_path, exe = os.path.join(td, "facts.c"), os.path.join(td, "facts")
        open(c_path, "w").write("\n".join(prog))
        subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-o", exe, c_path], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    sizes, offs, vals = {}, {}, {}
    for line in out.splitlines():
        kind, *rest = line.split()
        if kind == "S":
            sizes[rest[0]] = (int(rest[1]), int(rest[2]))
        elif kind == "F":
            offs[(rest[0], rest[1])] = int(rest[2])
        else:
            vals[rest[0]] = int(rest[1])
    return sizes, offs, vals


def test_struct_layouts_and_constants_agree_with_gcc(parsed):
    (cstructs, _, _, enums, defines), (rstructs, _, _, rconsts) = parsed
    sizes, offs, vals = _gcc_facts(cstructs, enums + defines)
    for name in cstructs:
        size, align, roffs = _rust_layout(rstructs, name)
        assert (size, align) == sizes[name], (name, (size, align), sizes[name])
        for f, o in roffs.items():
            assert o == offs[(name, f)], (name, f, o, offs[(name, f)])
    assert set(enums + defines) <= set(rconsts), sorted(set(enums + defines) - set(rconsts))
    for c in enums + defines:
        assert rconsts[c] == vals[c], (c, rconsts[c], vals[c])


def test_tile_ir_dispatch_calls_are_bound(parsed):
    """The calls the reference's tile_ir callers make, by name."""
    _, (rstructs, _, rfuncs, _) = parsed
    for t in ("t0_tile_gemm", "t0_gemm_desc", "t0_rmsnorm_desc", "t0_gemm_config", "t0_w4a16_desc"):
        assert t in rstructs
    for f in ("t0_gemm", "t0_gemm_select", "t0_ensure_tile_kernel", "t0_tile_build_kernargs_m",
              "t0_tile_compute_grid", "t0_tile_auto_select", "t0_tile_name", "t0_dispatch"):
        assert f in rfuncs


def test_the_parser_catches_a_wrong_binding(parsed, tmp_path, monkeypatch):
    """A transposed pair of fields or a narrowed argument must fail the checks."""
    src = open(RUST).read()
    bad = src.replace("pub lda: u32,\n    pub ldb: u32,", "pub ldb: u32,\n    pub lda: u32,", 1)
    assert bad != src
    p = tmp_path / "bad.rs"
    p.write_text(bad)
    monkeypatch.setattr(__import__(__name__), "RUST", str(p))
    with pytest.raises(AssertionError):
        test_every_struct_matches_field_by_field((parse_header(), parse_rust()))
    bad2 = src.replace("pub fn t0_tile_compute_grid(spec: *const t0_tile_gemm, m: u32, n: u32,",
                       "pub fn t0_tile_compute_grid(spec: *const t0_tile_gemm, m: u16, n: u32,", 1)
    assert bad2 != src
    p.write_text(bad2)
    with pytest.raises(AssertionError):
        test_every_function_is_bound_with_its_signature((parse_header(), parse_rust()))
