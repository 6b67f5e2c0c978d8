"""The Rust drop-in written out in INTEGRATION.md against the C ABI it binds.

Every `extern "C"` declaration in the document's Rust blocks must name a function that
`include/camelid_hip.h` / `include/camelid_gguf.h` declare, with the same arity, argument
types and return type (C types mapped to their Rust FFI equivalents, pointer constness
included); `HipDims` must lay out `camelid_hip_dims` field for field; and the wrapper must
define every `CudaResidentDecode` method the seam calls (cuda_resident.rs:5601-8857).
Runs without a GPU.
"""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent

# C scalar / struct spellings -> the Rust FFI type the binding must use
_BASE = {
    "uint8_t": "u8", "int8_t": "i8", "uint16_t": "u16", "int16_t": "i16", "uint32_t": "u32",
    "int32_t": "i32", "uint64_t": "u64", "int64_t": "i64", "size_t": "usize", "int": "i32",
    "float": "f32", "double": "f64", "char": "i8", "void": "c_void",
    # opaque handles are void pointers on the Rust side
    "camelid_hip_engine": "c_void", "camelid_gguf": "c_void",
    "camelid_hip_dims": "HipDims", "camelid_gguf_tensor": "GgufTensor", "camelid_gguf_rope": "GgufRope",
}
_RUST_ALIAS = {"c_int": "i32", "c_float": "f32", "c_char": "i8", "c_uint": "u32", "c_double": "f64"}

ENGINE_FUNCTIONS = [
    "camelid_hip_engine_new", "camelid_hip_check_model", "camelid_hip_engine_free", "camelid_hip_last_error",
    "camelid_hip_set_layer", "camelid_hip_set_output", "camelid_hip_weights_ready", "camelid_hip_filled",
    "camelid_hip_set_filled", "camelid_hip_max_pos", "camelid_hip_n_layers", "camelid_hip_uses_kquant",
    "camelid_hip_seed_layer", "camelid_hip_read_kv_layer", "camelid_hip_forward_token", "camelid_hip_prefill",
    "camelid_hip_verify", "camelid_hip_set_embedding", "camelid_hip_set_rope_table", "camelid_hip_generate",
    "camelid_gguf_open", "camelid_gguf_close", "camelid_hip_load_gguf",
]
# CudaResidentDecode's methods that the seam calls (cuda_resident.rs:5601-8857)
WRAPPER_METHODS = [
    "new", "set_layer_located", "set_output", "uses_kquant", "weights_ready", "filled", "set_filled",
    "is_offloaded", "max_pos", "n_layers", "seed_layer", "read_kv_layer", "forward_token",
    "forward_token_logits", "prefill", "prefill_batched", "verify_batch", "set_device_decode_tables",
    "device_decode_ready", "read_out_tokens",
]


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def c_type_to_rust(ctype, array=False):
    """'const uint8_t* const' (+ array) -> '*const *const u8'.  Pointer levels read inside
    out: the qualifier written before each '*' is the constness of what that pointer points
    to; an array parameter decays to one more pointer level."""
    t = " ".join(ctype.replace("*", " * ").split())
    if array:
        t += " *"
    segs = t.split("*")
    base_words = segs[0].split()
    base = [w for w in base_words if w not in ("const", "struct")]
    assert len(base) == 1, f"unparsed C type {ctype!r}"
    rust = _BASE[base[0]]
    for k in range(1, len(segs)):
        const = "const" in segs[k - 1].split()
        rust = ("*const " if const else "*mut ") + rust
    return rust


def _c_param(p):
    p = " ".join(p.split())
    m = re.fullmatch(r"(.*?)\b(\w+)\s*(\[\s*\w*\s*\])?", p)
    assert m, f"unparsed C parameter {p!r}"
    return c_type_to_rust(m.group(1), array=bool(m.group(3)))


def c_prototypes():
    protos = {}
    for h in ("include/camelid_hip.h", "include/camelid_gguf.h"):
        text = _strip_c_comments((ROOT / h).read_text())
        for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(camelid_\w+)\s*\(([^)]*)\)\s*;", text):
            ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
            ret = ret.split("\n")[-1].strip()
            args = [] if params in ("", "void") else [_c_param(p) for p in params.split(",")]
            protos[name] = (None if ret == "void" else c_type_to_rust(ret), args)
    return protos


def _norm_rust(t):
    t = " ".join(t.replace("*const", "*const ").replace("*mut", "*mut ").split())
    for a, b in _RUST_ALIAS.items():
        t = re.sub(rf"\b{a}\b", b, t)
    return t


def rust_blocks():
    doc = (ROOT / "INTEGRATION.md").read_text()
    return re.findall(r"```rust\n(.*?)```", doc, flags=re.S)


def rust_externs():
    decls = {}
    for block in rust_blocks():
        for ext in re.finditer(r'extern "C"\s*\{(.*?)\n\}', block, flags=re.S):
            for m in re.finditer(r"fn\s+(\w+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", ext.group(1), flags=re.S):
                name, params, ret = m.group(1), m.group(2).strip(), m.group(4)
                args = []
                for p in filter(None, (x.strip() for x in params.split(","))):
                    _, ty = p.split(":", 1)
                    args.append(_norm_rust(ty))
                assert name not in decls or decls[name] == (ret and _norm_rust(ret), args), name
                decls[name] = (_norm_rust(ret) if ret else None, args)
    return decls


def test_c_type_mapping_examples():
    assert c_type_to_rust("const uint8_t* const", array=True) == "*const *const u8"
    assert c_type_to_rust("const size_t", array=True) == "*const usize"
    assert c_type_to_rust("camelid_hip_engine**") == "*mut *mut c_void"
    assert c_type_to_rust("const camelid_hip_engine*") == "*const c_void"
    assert c_type_to_rust("const char*") == "*const i8"
    assert c_type_to_rust("float*") == "*mut f32"


def test_every_rust_extern_matches_the_c_header():
    protos = c_prototypes()
    decls = rust_externs()
    assert len(protos) > 40 and len(decls) >= len(ENGINE_FUNCTIONS)
    for name, (ret, args) in decls.items():
        assert name in protos, f"{name} is declared in INTEGRATION.md but not in include/"
        cret, cargs = protos[name]
        assert len(args) == len(cargs), f"{name}: {len(args)} Rust arguments vs {len(cargs)} in C"
        for i, (r, c) in enumerate(zip(args, cargs)):
            assert r == c, f"{name} argument {i}: Rust {r!r} vs C {c!r}"
        assert ret == cret, f"{name} return: Rust {ret!r} vs C {cret!r}"


def test_rust_binding_declares_the_whole_engine_method_set():
    decls = rust_externs()
    missing = [f for f in ENGINE_FUNCTIONS if f not in decls]
    assert not missing, f"INTEGRATION.md binds no {missing}"


def test_rust_wrapper_defines_every_resident_method():
    src = "\n".join(rust_blocks())
    missing = [m for m in WRAPPER_METHODS if not re.search(rf"\bpub fn {m}\s*\(", src)]
    assert not missing, f"HipResidentDecode lacks {missing}"
    assert "same pattern" not in src and "..." not in src.replace("..=", "")


def test_hip_dims_matches_the_c_struct():
    text = _strip_c_comments((ROOT / "include/camelid_hip.h").read_text())
    body = re.search(r"typedef struct camelid_hip_dims\s*\{(.*?)\}", text, flags=re.S).group(1)
    c_fields = [(f.split()[-1], c_type_to_rust(" ".join(f.split()[:-1]))) for f in body.split(";") if f.strip()]
    src = "\n".join(rust_blocks())
    rbody = re.search(r"pub struct HipDims\s*\{(.*?)\n\}", src, flags=re.S).group(1)
    r_fields = [(n.strip().removeprefix("pub ").strip(), _norm_rust(t.strip()))
                for n, t in (f.split(":") for f in rbody.split(",") if ":" in f)]
    assert "#[repr(C)]" in src.split("pub struct HipDims")[0][-200:]
    assert r_fields == c_fields
