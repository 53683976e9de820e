"""The Rust crate's FFI layer (rusticide-hip/src/sys.rs) against the C header
(include/rusticide_hip.h) it binds.

There is no Rust toolchain in this image, so the crate is not compiled here;
this test parses both files and requires that every non-hook entry point of
the header is declared in the crate's `extern "C"` blocks with the same name,
argument count, argument types and return type (C types mapped to their
Rust FFI spellings), that the crate declares nothing the header lacks, and
that the #[repr(C)] structs and the status enum match field for field.
Entry points whose header comment calls them a test, bench or tuning hook
are for this repository's tests and bench only; nothing in rusticide binds
them, so the crate leaves them out.
"""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rusticide_hip.h")
SYS_RS = os.path.join(ROOT, "rusticide-hip", "src", "sys.rs")

C_BASE = {
    "float": "f32", "double": "f64", "int": "c_int", "size_t": "usize", "uint32_t": "u32", "uint64_t": "u64",
    "int8_t": "i8", "int32_t": "i32", "uint8_t": "u8", "char": "c_char", "void": "c_void",
}


def rust_of_c(ctype: str) -> str:
    """A C type (no declarator name) in Rust FFI spelling: `const T *const *`
    is `*const *const T`, `T **` is `*mut *mut T`, `T x[N]` a `*mut T`."""
    toks = re.findall(r"\*|\[\d*\]|const|[A-Za-z_]\w*", ctype)
    lead_const, base, rest = False, None, []
    for t in toks:
        if base is None:
            if t == "const":
                lead_const = True
            else:
                base = t
        else:
            rest.append(t)
    assert base is not None, ctype
    cur = C_BASE.get(base, base)
    cur_const = lead_const
    i = 0
    while i < len(rest):
        t = rest[i]
        if t == "*" or t.startswith("["):
            cur = ("*const " if cur_const else "*mut ") + cur
            cur_const = i + 1 < len(rest) and rest[i + 1] == "const"
            if cur_const:
                i += 1
        i += 1
    return "()" if cur == "c_void" else cur


def split_decl(param: str):
    """('type', 'name') of one C parameter or field declarator."""
    param = param.strip()
    m = re.match(r"^(.*?)([A-Za-z_]\w*)\s*(\[\d*\])?$", param, re.S)
    assert m, param
    return m.group(1) + (" " + m.group(3) if m.group(3) else ""), m.group(2)


def header_text():
    return open(HEADER).read()


def header_functions():
    """{name: (return type, [param types], is_hook)} of the header's functions."""
    raw = header_text()
    comments = [(m.start(), m.end(), m.group(0)) for m in re.finditer(r"/\*.*?\*/", raw, re.S)]
    text = re.sub(r"/\*.*?\*/", lambda m: " " * len(m.group(0)), raw, flags=re.S)
    text = re.sub(r"^\s*#.*$", lambda m: " " * len(m.group(0)), text, flags=re.M)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(rh_\w+)\s*\(([^;{}()]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        before = [c for c in comments if c[1] <= m.start(2)]
        doc = before[-1][2] if before else ""
        hook = re.search(r"\b(test|bench|tuning) hooks?\b", doc, re.I) is not None
        plist = [] if params in ("", "void") else [rust_of_c(split_decl(p)[0]) for p in params.split(",")]
        out[name] = (rust_of_c(ret.strip()), plist, hook)
    return out


def rust_type(t: str) -> str:
    t = re.sub(r"\s+", " ", t.strip())
    return re.sub(r"\*(const|mut) ", r"*\1 ", t)


def rust_functions():
    """{name: (return type, [param types])} of the crate's extern "C" blocks."""
    text = re.sub(r"//[^\n]*", "", open(SYS_RS).read())
    out = {}
    for block in re.finditer(r'extern\s+"C"\s*\{(.*?)\n\}', text, re.S):
        for m in re.finditer(r"pub\s+fn\s+(\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block.group(1), re.S):
            name, params, ret = m.group(1), m.group(2).strip().rstrip(","), m.group(4)
            plist = [] if not params else [rust_type(p.split(":", 1)[1]) for p in params.split(",") if p.strip()]
            out[name] = (rust_type(ret) if ret else "()", plist)
    return out


def test_every_boundary_entry_point_is_bound_with_the_same_signature():
    c, r = header_functions(), rust_functions()
    bound = {n for n, (_, _, hook) in c.items() if not hook}
    assert len(bound) >= 40, sorted(bound)
    assert bound == set(r), f"header only: {sorted(bound - set(r))}; crate only: {sorted(set(r) - bound)}"
    for name in sorted(bound):
        want = c[name][:2]
        assert r[name] == want, f"{name}: crate {r[name]}, header {want}"


def test_the_hooks_left_out_are_the_headers_test_bench_and_tuning_hooks():
    hooks = {n for n, (_, _, hook) in header_functions().items() if hook}
    assert hooks == {
        "rh_quantize", "rh_ternary_dot_i32", "rh_expf_host", "rh_sqrt_host", "rh_math_device",
        "rh_stream_read_device", "rh_hold_device", "rh_matmul_batch_device_repeat", "rh_reload_tuning",
        "rh_ordered_sum_device", "rh_greedy_pick_device", "rh_ordered_sum4_device", "rh_rope_table_host",
    }, sorted(hooks)


def c_structs():
    """{name: [(field, rust type)]} of the header's typedef structs."""
    text = re.sub(r"/\*.*?\*/", "", header_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef\s+struct\s+(\w+)\s*\{(.*?)\}\s*(\w+)\s*;", text, re.S):
        fields = []
        for decl in m.group(2).split(";"):
            decl = decl.strip()
            if not decl:
                continue
            first, *more = decl.split(",")
            ftype, fname = split_decl(first)
            base = re.sub(r"\*|\[\d*\]", "", ftype).strip()
            for part, (t, n) in [(first, (ftype, fname))] + [(p, split_decl(base + " " + p.strip())) for p in more]:
                arr = re.search(r"\[(\d+)\]", part)
                if arr:
                    fields.append((n, f"[{C_BASE.get(base, base)}; {arr.group(1)}]"))
                else:
                    fields.append((n, rust_of_c(t)))
        out[m.group(1)] = fields
    return out


def rust_structs():
    text = re.sub(r"//[^\n]*", "", open(SYS_RS).read())
    out = {}
    for m in re.finditer(r"#\[repr\(C\)\][^{;]*?pub struct (\w+)\s*\{(.*?)\}", text, re.S):
        fields = []
        for f in m.group(2).split(","):
            f = f.strip()
            if f.startswith("pub "):
                n, t = f[4:].split(":", 1)
                fields.append((n.strip(), rust_type(t)))
        if fields:
            out[m.group(1)] = fields
    return out


def test_repr_c_structs_match_the_header_field_for_field():
    c, r = c_structs(), rust_structs()
    assert set(c) == {"rh_job", "rh_decoder_config", "rh_decoder_block", "rh_decoder_weights", "rh_gguf_error"}
    for name, fields in c.items():
        assert r.get(name) == fields, f"{name}: crate {r.get(name)}, header {fields}"


def test_status_enum_matches_the_header():
    text = re.sub(r"/\*.*?\*/", "", header_text(), flags=re.S)
    body = re.search(r"typedef enum rh_status \{(.*?)\}", text, re.S).group(1)
    c = {int(v) for v in re.findall(r"RH_\w+\s*=\s*(\d+)", body)}
    rs = re.search(r"pub enum rh_status \{(.*?)\}", open(SYS_RS).read(), re.S).group(1)
    r = {int(v) for v in re.findall(r"\w+\s*=\s*(\d+)", rs)}
    assert c == r == set(range(16))


def test_the_c_type_mapping_itself():
    # the mapping the checks above rely on, on the shapes the header uses
    assert rust_of_c("const float *") == "*const f32"
    assert rust_of_c("rh_ctx **") == "*mut *mut rh_ctx"
    assert rust_of_c("const char **") == "*mut *const c_char"
    assert rust_of_c("const void *const *") == "*const *const c_void"
    assert rust_of_c("const rh_matrix *const *") == "*const *const rh_matrix"
    assert rust_of_c("uint64_t [4]") == "*mut u64"
    assert rust_of_c("void") == "()"
    assert split_decl("uint64_t shape[4]") == ("uint64_t  [4]", "shape")
