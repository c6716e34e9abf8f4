"""The Rust FFI crate (rust/ssdq-sys) binds exactly the C ABI of include/ssdq.h.

There is no Rust toolchain in this image, so the crate is checked as text:
every function the header declares is declared in the crate's extern block,
with the same argument count and names and the Rust type the C type maps to
(int -> c_int, size_t -> usize, float -> f32, const T* -> *const T, T* ->
*mut T, void* -> c_void pointers), and the same return type; the constants
(status codes, GgmlType ids, layer regions) carry the header's values; the
layer config struct has the header's fields in order.  The safe crate
(rust/ssdq) only calls functions the raw crate declares.
"""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ssdq.h"
SYS = ROOT / "rust" / "ssdq-sys" / "src" / "lib.rs"
SAFE = ROOT / "rust" / "ssdq" / "src" / "lib.rs"

SCALAR = {"int": "c_int", "size_t": "usize", "float": "f32", "void": "c_void", "char": "c_char",
          "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "int32_t": "i32", "uint32_t": "u32",
          "uint64_t": "u64", "ssdq_stream_t": "ssdq_stream_t", "ssdq_ctx": "ssdq_ctx",
          "ssdq_weights": "ssdq_weights", "ssdq_layer_config": "ssdq_layer_config"}


def strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def c_type_to_rust(t):
    """'const float*' -> '*const f32'; 'const void* const*' -> '*const *const c_void'."""
    t = t.strip()
    # split off pointer levels from the right, each with its own constness
    m = re.match(r"^(const\s+)?(\w+)\s*(.*)$", t)
    assert m, t
    base_const, base, rest = m.group(1) is not None, m.group(2), m.group(3).replace(" ", "")
    levels = re.findall(r"\*(const)?", rest)  # '*', '*const' ... from the base outwards
    if not levels:
        return SCALAR[base]
    # C: 'const T* const* p' = p is a pointer (non-const) to a const pointer to const T
    consts = [base_const] + [lv == "const" for lv in levels[:-1]]
    out = SCALAR[base]
    for c in consts:
        out = ("*const " if c else "*mut ") + out
    return out


def header_functions():
    src = strip_c_comments(HEADER.read_text())
    src = "\n".join(l for l in src.splitlines() if not l.lstrip().startswith("#"))
    src = re.sub(r"\s+", " ", src)
    funcs = {}
    order = []
    for m in re.finditer(r"([\w\s\*]+?)\b(ssdq_\w+)\s*\(([^()]*)\)\s*;", src):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        if ret.startswith("typedef") or "struct" in ret:
            continue
        args = []
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                pm = re.match(r"^(.*?)(\w+)$", p)
                args.append((pm.group(2), c_type_to_rust(pm.group(1))))
        funcs[name] = (None if ret == "void" else c_type_to_rust(ret), args)
        order.append(name)
    return funcs, order


def rust_functions():
    src = re.sub(r"//[^\n]*", " ", SYS.read_text())
    block = src[src.index('extern "C" {'):]
    block = re.sub(r"\s+", " ", block)
    funcs = {}
    order = []
    for m in re.finditer(r"pub fn (\w+)\(([^()]*)\)\s*(->\s*([^;]+))?;", block):
        name, params, ret = m.group(1), m.group(2).strip(), m.group(4)
        args = []
        if params:
            for p in params.split(","):
                p = p.strip()
                if not p:
                    continue
                an, at = p.split(":", 1)
                args.append((an.strip().replace("r#", ""), re.sub(r"\s+", " ", at.strip())))
        funcs[name] = (ret.strip() if ret else None, args)
        order.append(name)
    return funcs, order


def test_every_header_function_is_bound_with_matching_types():
    hf, horder = header_functions()
    rf, rorder = rust_functions()
    assert len(hf) >= 40, sorted(hf)
    assert set(hf) == set(rf), (sorted(set(hf) - set(rf)), sorted(set(rf) - set(hf)))
    assert horder == rorder  # same order as the header, so a reviewer can read them side by side
    for name, (hret, hargs) in hf.items():
        rret, rargs = rf[name]
        assert hret == rret, (name, hret, rret)
        assert [a for a, _ in hargs] == [a for a, _ in rargs], name
        assert [t for _, t in hargs] == [t for _, t in rargs], (name, hargs, rargs)


def test_constants_and_layer_config_match_the_header():
    h = strip_c_comments(HEADER.read_text())
    hdefs = {m.group(1): int(m.group(2).strip("()")) for m in
             re.finditer(r"#define (SSDQ_\w+) \(?(-?\d+)\)?", h)}
    r = SYS.read_text()
    rdefs = {m.group(1): int(m.group(2)) for m in re.finditer(r"pub const (SSDQ_\w+): \w+ = (-?\d+);", r)}
    assert len(hdefs) >= 35
    assert hdefs == rdefs, (set(hdefs) ^ set(rdefs), {k: (hdefs[k], rdefs.get(k)) for k in hdefs if hdefs[k] != rdefs.get(k)})
    hcfg = re.search(r"typedef struct ssdq_layer_config \{(.*?)\}", h, re.S).group(1)
    hfields = [(m.group(2), SCALAR[m.group(1)]) for m in re.finditer(r"(\w+) (\w+);", hcfg)]
    rcfg = re.search(r"pub struct ssdq_layer_config \{(.*?)\}", r, re.S).group(1)
    rfields = [(m.group(1), m.group(2)) for m in re.finditer(r"pub (\w+): (\w+),", rcfg)]
    assert hfields == rfields


def test_safe_crate_calls_only_declared_functions():
    rf, _ = rust_functions()
    called = set(re.findall(r"ffi::(ssdq_\w+)\(", SAFE.read_text()))
    assert called and called <= set(rf), called - set(rf)


def test_c_type_mapping():
    assert c_type_to_rust("const float*") == "*const f32"
    assert c_type_to_rust("float* const*") == "*const *mut f32"
    assert c_type_to_rust("const void* const*") == "*const *const c_void"
    assert c_type_to_rust("ssdq_ctx**") == "*mut *mut ssdq_ctx"
    assert c_type_to_rust("size_t") == "usize"
