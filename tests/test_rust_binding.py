"""The Rust host module (nebula_amd/rust/qgemm.rs, for crates/nebula-hydrogen) against the C
header it binds (include/hq_qgemm.h): every declared function is in its extern block with the
same name, arity, parameter and return types (by the C -> Rust type mapping below), every
#[repr(C)] struct mirrors its C struct field by field, and the size asserts agree with the
struct sizes the Python binding computes. No Rust toolchain exists in this image, so this is
the check that keeps the module in step with the ABI.
"""
import ctypes
import re
from pathlib import Path

from nebula_amd import gguf as G
from nebula_amd import hq

ROOT = Path(__file__).resolve().parent.parent
HEADER = (ROOT / "include" / "hq_qgemm.h").read_text()
RUST = (ROOT / "nebula_amd" / "rust" / "qgemm.rs").read_text()

C_TO_RUST = {
    "void": "()", "const char*": "*const c_char", "char*": "*mut c_char", "size_t": "usize", "size_t*": "*mut usize",
    "uint32_t": "u32", "uint32_t*": "*mut u32", "const uint32_t*": "*const u32", "int64_t": "i64",
    "int64_t*": "*mut i64", "uint64_t": "u64", "uint64_t*": "*mut u64", "double*": "*mut f64", "int": "c_int",
    "uint16_t*": "*mut u16", "const uint16_t*": "*const u16", "float*": "*mut f32", "const float*": "*const f32",
    "const void*": "*const c_void", "void*": "*mut c_void", "hq_status": "Status", "hq_format": "Format",
    "hq_dtype": "Dtype", "hq_stream": "Stream", "const hq_segment*": "*const Segment", "hq_gguf**": "*mut *mut Gguf",
    "hq_gguf*": "*mut Gguf", "const hq_gguf*": "*const Gguf", "hq_gguf_header_info*": "*mut GgufHeaderInfo",
    "hq_gguf_tensor_info*": "*mut GgufTensorInfo", "uint64_t[4]": "[u64; 4]", "const int8_t*": "*const i8",
    "int8_t*": "*mut i8", "int64_t": "i64",
}
STRUCTS = {"hq_segment": "Segment", "hq_gguf_header_info": "GgufHeaderInfo", "hq_gguf_tensor_info": "GgufTensorInfo"}


def c_decls():
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    out = {}
    for m in re.finditer(r"((?:const\s+)?\w+\s*\**)\s*\b(hq_\w+)\s*\(([^)]*)\)\s*;", text):
        ret, name, params = m.group(1).replace(" ", ""), m.group(2), m.group(3).strip()
        ps = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                t = p.rsplit(" ", 1)[0] if " " in p else p
                t = t.replace(" *", "*")
                ps.append(t)
        out[name] = (ret.replace("constchar", "const char"), ps)
    return out


def rust_decls():
    block = RUST[RUST.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    out = {}
    for m in re.finditer(r"pub fn (hq_\w+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        types = [" ".join(p.split(":", 1)[1].split()) for p in params]
        out[m.group(1)] = ((m.group(3) or "()").strip(), types)
    return out


def test_every_function_is_bound_with_the_same_signature():
    c, r = c_decls(), rust_decls()
    assert set(c) == set(hq.EXPORTS) == set(r), (set(c) ^ set(r))
    for name, (cret, cps) in c.items():
        rret, rps = r[name]
        assert C_TO_RUST[cret] == rret, (name, cret, rret)
        assert len(cps) == len(rps), (name, cps, rps)
        for i, (ct, rt) in enumerate(zip(cps, rps)):
            assert C_TO_RUST[ct] == rt, (name, i, ct, rt)


def c_struct_fields(cname):
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), text, flags=re.S).group(1)
    fields = []
    for line in body.split(";"):
        line = " ".join(line.split())
        if not line:
            continue
        m = re.match(r"((?:const )?\w+\**)\s*(.*)", line)
        base, names = m.group(1), m.group(2)
        for nm in names.split(","):
            nm = nm.strip()
            stars = len(nm) - len(nm.lstrip("*"))
            nm = nm.lstrip("*")
            t = base + "*" * stars
            arr = re.match(r"(\w+)\[(\d+)\]", nm)
            if arr:
                nm, t = arr.group(1), f"{t}[{arr.group(2)}]"
            fields.append((nm, t))
    return fields


def rust_struct_fields(rname):
    body = re.search(r"pub struct %s \{(.*?)\n\}" % rname, RUST, flags=re.S).group(1)
    return [(f.split(":", 1)[0].replace("pub ", "").replace("r#", "").strip(), " ".join(f.split(":", 1)[1].split()))
            for f in body.split(",") if ":" in f]


def test_structs_mirror_the_header():
    for cname, rname in STRUCTS.items():
        cf, rf = c_struct_fields(cname), rust_struct_fields(rname)
        assert len(cf) == len(rf), (cname, cf, rf)
        for (cn, ct), (rn, rt) in zip(cf, rf):
            assert cn.lower() == rn, (cname, cn, rn)
            mapped = C_TO_RUST.get(ct, {"void*": "*mut c_void"}.get(ct))
            if ct == "const char*":
                mapped = "*const c_char"
            assert mapped == rt, (cname, cn, ct, rt)


def test_size_asserts_match_the_abi():
    sizes = dict(re.findall(r"size_of::<(\w+)>\(\) == (\d+)", RUST))
    assert int(sizes["Segment"]) == ctypes.sizeof(hq.Segment)
    assert int(sizes["GgufHeaderInfo"]) == ctypes.sizeof(G.HeaderInfo)
    assert int(sizes["GgufTensorInfo"]) == ctypes.sizeof(G.TensorInfo)
    assert "NOALLOC_SCRATCH_BYTES: usize = 16 << 20" in RUST and hq.NOALLOC_SCRATCH_BYTES == 16 << 20
    assert re.search(r"HQ_NOALLOC_SCRATCH_BYTES \(\(size_t\)16 << 20\)", HEADER)
