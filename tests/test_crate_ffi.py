"""The Rust binding (crates/strata-backend-hip) against include/strata_hip.h,
as text (no Rust toolchain is needed): every declared entry point is bound
with the same parameter and return types, every status code, type id, flag
and mode has the same value, every struct the same fields in the same order
and types, and the trait implementation passes the configured flags instead
of hard-coded zeros."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "strata_hip.h")
CRATE = os.path.join(ROOT, "crates", "strata-backend-hip")

STRUCTS = {"sh_context": "ShContext", "sh_quant_tensor": "ShQuantTensor", "sh_expert_view": "ShExpertView",
           "sh_rope_cfg": "ShRopeCfg", "sh_gguf": "ShGguf", "sh_gguf_tensor_info": "ShGgufTensorInfo",
           "sh_expert_dev": "ShExpertDev", "sh_gguf_model": "ShGgufModel"}
SCALARS = {"int": "c_int", "char": "c_char", "uint32_t": "u32", "uint64_t": "u64", "int64_t": "i64",
           "int32_t": "i32", "int8_t": "i8", "uint8_t": "u8", "double": "f64", "float": "f32", "void": "c_void"}


def c_to_rust(ctype):
    """C parameter / field type -> the Rust FFI type it must be bound as
    (`const T*` -> `*const T`, `T*` -> `*mut T`, outer pointers mutable)."""
    t = ctype.strip()
    const = t.startswith("const ")
    if const:
        t = t[len("const "):]
    stars = t.count("*")
    base = t.replace("*", "").strip()
    r = STRUCTS.get(base) or SCALARS[base]
    if stars == 0:
        return r
    r = ("*const " if const else "*mut ") + r
    for _ in range(stars - 1):
        r = "*mut " + r
    return r


def norm(s):
    return " ".join(s.split())


def header_text():
    return re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)


def header_functions():
    out = {}
    for ret, name, params in re.findall(r"\n(int|const char\*)\s+(sh_\w+)\((.*?)\);", header_text(), flags=re.S):
        ps = [p.strip() for p in norm(params).split(",")]
        types = [] if ps == ["void"] else [re.match(r"(.*?)(\w+)$", p).group(1) for p in ps]
        out[name] = ([c_to_rust(t) for t in types], "c_int" if ret == "int" else "*const c_char")
    return out


def rust_functions():
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    block = text[text.index('extern "C" {'):]
    out = {}
    for name, params, ret in re.findall(r"pub fn (sh_\w+)\((.*?)\)\s*->\s*(.*?);", block, flags=re.S):
        ps = [p for p in norm(params).split(", ") if p]
        out[name] = ([p.split(": ", 1)[1] for p in ps], norm(ret))
    return out


def test_every_entry_point_is_bound_with_the_header_types():
    h, r = header_functions(), rust_functions()
    assert h, "no declarations parsed from the header"
    assert sorted(h) == sorted(r), f"missing: {sorted(set(h) - set(r))}, extra: {sorted(set(r) - set(h))}"
    for name in h:
        assert r[name] == h[name], f"{name}: header {h[name]}, ffi.rs {r[name]}"


def test_the_python_mirror_and_the_crate_bind_the_same_symbols():
    import strata_hip as H
    assert sorted(H.EXPORTS) == sorted(rust_functions())


def test_constants_match():
    defines = dict(re.findall(r"#define (SH_\w+) \(?(-?\d+)u?\)?", header_text()))
    defines.pop("STRATA_HIP_H", None)
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    consts = dict(re.findall(r"pub const (SH_\w+): \w+ = (-?\d+);", text))
    assert defines and sorted(defines) == sorted(consts)
    for k, v in defines.items():
        assert int(consts[k]) == int(v), k


def struct_fields_c(name):
    m = re.search(r"typedef struct " + name + r" \{(.*?)\} " + name + ";", header_text(), flags=re.S)
    fields = []
    for decl in m.group(1).split(";"):
        decl = norm(decl)
        if not decl:
            continue
        fm = re.match(r"(.*?)(\w+)(\[(\d+)\])?$", decl)
        ty, nm, arr = fm.group(1), fm.group(2), fm.group(4)
        rt = c_to_rust(ty)
        fields.append((nm, f"[{rt}; {arr}]" if arr else rt))
    return fields


def struct_fields_rust(name):
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    m = re.search(r"pub struct " + name + r" \{(.*?)\n\}", text, flags=re.S)
    return [(f.split(": ")[0].replace("pub ", "").strip(), f.split(": ")[1].strip().rstrip(","))
            for f in m.group(1).strip().splitlines() if f.strip().startswith("pub ")]


@pytest.mark.parametrize("c_name", ["sh_quant_tensor", "sh_expert_view", "sh_rope_cfg", "sh_gguf_tensor_info",
                                    "sh_expert_dev"])
def test_struct_layouts_match(c_name):
    c = [(("type_" if n == "type" else n), t) for n, t in struct_fields_c(c_name)]
    assert c == struct_fields_rust(STRUCTS[c_name])


def test_opaque_handles_are_declared():
    text = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    for name in ("ShContext", "ShGguf", "ShGgufModel"):
        assert re.search(r"#\[repr\(C\)\]\s*pub struct " + name + r" \{\s*_opaque: \[u8; 0\],\s*\}", text), name


def test_lib_passes_the_configured_flags():
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    assert "flags: 0" not in lib
    assert "flags: self.opts.tensor_flags(w.quant)" in lib
    assert "flags: self.opts.expert_flags(w.quant)" in lib
    for trait_method in ("fn name(", "fn gemv(", "fn expert_gemv(", "fn rms_norm(", "fn rope_neox(",
                         "fn softmax(", "fn l2_norm(", "fn add("):
        assert trait_method in lib, trait_method


def test_build_script_links_the_library():
    b = open(os.path.join(CRATE, "build.rs")).read()
    assert "cargo:rustc-link-lib=dylib=strata_hip" in b
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "strata-backend-hip"' in cargo and 'links = "strata_hip"' in cargo


def test_device_errors_propagate_and_only_unsupported_or_caller_errors_go_to_the_cpu():
    """The status mapping of the trait methods (the wgpu backend returns its
    device errors, crates/strata-backend-wgpu/src/gpu.rs:331-365): every
    trait method goes through `route`, whose CPU arm names exactly the
    unsupported-type/shape and caller-argument codes, and whose catch-all is
    `Error::Backend`; no trait method retries a device failure on the CPU."""
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    m = re.search(r"fn route\(rc: c_int, what: &str\) -> Result<Route> \{(.*?)\n\}", lib, flags=re.S)
    assert m, "route() not found"
    body = m.group(1)
    cpu_arm = re.search(r"\n\s*((?:ffi::SH_ERR_\w+\s*\|?\s*)+)=> \{", body)
    assert cpu_arm, body
    codes = sorted(c.strip() for c in cpu_arm.group(1).split("|"))
    assert codes == ["ffi::SH_ERR_SHAPE", "ffi::SH_ERR_TRUNCATED", "ffi::SH_ERR_UNSUPPORTED_QUANT",
                     "ffi::SH_ERR_UNSUPPORTED_SHAPE"], codes
    assert "ffi::SH_OK => Ok(Route::Done)" in body
    assert re.search(r"_ => Err\(Error::Backend", body)
    impl = lib[lib.index("impl ComputeBackend for HipBackend"):lib.index("#[cfg(test)]")]
    # no status check that swallows an error into a CPU retry
    assert "check(rc)" not in impl and "tracing::warn!" not in impl
    for method in ("gemv", "expert_gemv", "rms_norm", "rope_neox", "softmax", "l2_norm", "add"):
        assert f'route(rc, "{method}")?' in impl, method
